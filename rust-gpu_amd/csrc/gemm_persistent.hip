// gemm_persistent.hip — launches of the persistent GEMM kernels (gemm_persistent.h) for
// the persistent TileGemm presets (src/t0/tile_ir.rs:540-604).
#include <string.h>

#include <algorithm>

#include "gemm_persistent.h"
#include "t0mi_ctx.h"

namespace t0mi {

namespace {

// Workgroups of `kernel` one CU holds at once (at least 1); asked once per kernel.
template <typename F>
uint32_t wgs_per_cu(F kernel, int threads) {
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, threads, 0) != hipSuccess || n < 1) n = 1;
  return (uint32_t)n;
}

// Grid of a persistent launch: the work items, or as many workgroups as the GPU holds at
// once if that is fewer, rounded down to a multiple of the 8 XCDs (the kernels keep each
// workgroup's items on its XCD).
uint32_t persistent_grid(const t0mi_ctx* ctx, uint32_t per_cu, uint32_t items) {
  uint32_t g = std::min<uint32_t>(items, per_cu * (uint32_t)std::max(1, ctx->cu_count));
  if (g >= 8) g -= g % 8;
  return std::max<uint32_t>(g, 1);
}

template <bool NN>
void launch_decode(const t0mi_ctx* ctx, hipStream_t s, const GemmParams& p) {
  static const uint32_t per_cu = wgs_per_cu(gemm_persistent_decode_kernel<NN>, PD_WAVES * 64);
  const uint32_t g = persistent_grid(ctx, per_cu, p.tiles_m * p.tiles_n);
  hipLaunchKernelGGL((gemm_persistent_decode_kernel<NN>), dim3(g), dim3(PD_WAVES * 64), 0, s, p);
}

template <int BM, int BN, int BK, int WM, int WN, int S, bool NN>
void launch_tiles(const t0mi_ctx* ctx, hipStream_t s, const GemmParams& p) {
  static const uint32_t per_cu = wgs_per_cu(gemm_bf16_persistent_kernel<BM, BN, BK, WM, WN, S, NN>, WM * WN * 64);
  const uint32_t g = persistent_grid(ctx, per_cu, p.tiles_m * p.tiles_n * p.split_k);
  hipLaunchKernelGGL((gemm_bf16_persistent_kernel<BM, BN, BK, WM, WN, S, NN>), dim3(g), dim3(WM * WN * 64), 0, s,
                     p);
}

struct PersistentTiles {
  int bm, bn, bk, wm, wn, stages, nn;
  void (*fn)(const t0mi_ctx*, hipStream_t, const GemmParams&);
};
// The kernels the three persistent presets lower to (32x64 k16, 128x64 k32, 256x128 k32),
// both B layouts.
const PersistentTiles kTiles[] = {
    {32, 64, 16, 1, 1, 2, 0, launch_tiles<32, 64, 16, 1, 1, 2, false>},
    {32, 64, 16, 1, 1, 2, 1, launch_tiles<32, 64, 16, 1, 1, 2, true>},
    {128, 64, 32, 2, 1, 2, 0, launch_tiles<128, 64, 32, 2, 1, 2, false>},
    {128, 64, 32, 2, 1, 2, 1, launch_tiles<128, 64, 32, 2, 1, 2, true>},
    {256, 128, 32, 2, 2, 2, 0, launch_tiles<256, 128, 32, 2, 2, 2, false>},
    {256, 128, 32, 2, 2, 2, 1, launch_tiles<256, 128, 32, 2, 2, 2, true>},
};

const PersistentTiles* find_tiles(const t0mi_gemm_config& cfg) {
  const int nn = cfg.transpose == T0MI_NN;
  const int stages = cfg.stages ? (int)cfg.stages : 2;
  for (const PersistentTiles& t : kTiles)
    if (t.bm == (int)cfg.tile_m && t.bn == (int)cfg.tile_n && t.bk == (int)cfg.tile_k && t.wm == (int)cfg.wave_m &&
        t.wn == (int)cfg.wave_n && t.stages == stages && t.nn == nn)
      return &t;
  return nullptr;
}

}  // namespace

const char* persistent_route(const t0mi_gemm_config& cfg, uint32_t m, uint32_t n, uint32_t k) {
  // The decode kernel takes whole 32-K blocks and 32-bit lane offsets into A and (NT) B.
  const bool offsets32 = (uint64_t)m * k * 2 < (1ull << 32) &&
                         (cfg.transpose == T0MI_NN || (uint64_t)n * k * 2 < (1ull << 32));
  if ((m <= kPersistentDecodeRows && k % 32 == 0 && offsets32) || k == 0) return "decode";
  return find_tiles(cfg) ? "tiles" : "one-shot";
}

int run_gemm_persistent(t0mi_ctx* ctx, const t0mi_gemm_config& cfg, const GemmLaunchEntry* e, uint64_t x,
                        uint64_t b, uint64_t y, uint64_t bias, uint32_t m, uint32_t n, uint32_t k,
                        const EpiChain& epi) {
  if (m == 0 || n == 0) return T0MI_OK;
  if (k % 8) return set_error(T0MI_ERR_INVALID, "K=%u must be a multiple of 8", k);
  if (n % 8) return set_error(T0MI_ERR_INVALID, "N=%u must be a multiple of 8", n);
  if ((x | b | y) & 15) return set_error(T0MI_ERR_INVALID, "X, B and Y must be 16-byte aligned");
  if (chain_uses(epi, EOP_BIAS) && !bias) return set_error(T0MI_ERR_INVALID, "bias epilogue with null bias");
  if (bias & 3) return set_error(T0MI_ERR_INVALID, "bias must be 4-byte aligned");
  const int nn = cfg.transpose == T0MI_NN;
  const char* route = persistent_route(cfg, m, n, k);
  if (route[0] == 'd' && k > 0 && (nn || m > 16 || (uint64_t)n > 16ull * (uint64_t)ctx->cu_count)) {
    // Decode-sized calls where the one-shot schedule auto_select picks for the
    // same call is faster (MI355X, K = 4096, f32 out, direct launches: NN 1 / 16
    // rows x 4096 13.2 / 13.6 us against 15.9 / 18.7; NT 32 / 64 rows x 4096
    // 13.9 / 15.3 against 16.4 / 27.7; NT 16 x 11008, more 16-column units than
    // CUs, 23.2 against 30.2 in a graph replay): that schedule runs, under the
    // spec's name, kernargs and grid.  NT up to 16 rows and one round of units
    // keeps the one-launch decode kernel (1 / 16 x 4096: 8.9 / 11.8 against
    // 13.7 / 13.2 us).
    return run_gemm_auto(ctx, cfg.transpose, x, b, y, m, n, k, cfg.out_dtype, bias, &epi);
  }
  if (route[0] == 'o') {
    // A persistent spec of the caller's own whose tile has no persistent instantiation:
    // the same tile's one-shot kernel, one plane (split-K is not part of a persistent run).
    t0mi_gemm_config c = cfg;
    c.split_k = 0;
    return run_gemm(ctx, c, e, x, b, y, bias, m, n, k, epi);
  }
  GemmParams p;
  memset(&p, 0, sizeof p);
  p.a = (const uint16_t*)x;
  p.b = (const uint16_t*)b;
  p.y = (void*)y;
  p.bias = (const float*)bias;
  p.M = m;
  p.N = n;
  p.K = k;
  p.lda = k;
  p.ldb = nn ? n : k;
  p.ldy = n;
  p.split_k = 1;
  p.k_per_split = k;
  p.out_bf16 = cfg.out_dtype == T0MI_OUT_BF16;
  p.epi = epi;
  p.xcd_remap = 1;
  if (ctx->null_backend) return T0MI_OK;
  if (route[0] == 'd') {
    p.tiles_m = (m + PD_ROWS - 1) / PD_ROWS;
    p.tiles_n = (n + PD_COLS - 1) / PD_COLS;
    if (nn)
      launch_decode<true>(ctx, ctx->stream, p);
    else
      launch_decode<false>(ctx, ctx->stream, p);
  } else {
    p.tiles_m = (m + cfg.tile_m - 1) / cfg.tile_m;
    p.tiles_n = (n + cfg.tile_n - 1) / cfg.tile_n;
    find_tiles(cfg)->fn(ctx, ctx->stream, p);
  }
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return set_error(T0MI_ERR_HIP, "persistent GEMM launch: %s", hipGetErrorString(err));
  return T0MI_OK;
}

int run_gemm_decode_nt(t0mi_ctx* ctx, uint64_t x, uint64_t b, uint64_t y, uint32_t m, uint32_t n, uint32_t k,
                       uint32_t out_dtype, uint64_t bias, const EpiChain& epi) {
  if (m == 0 || m > 16 || k == 0 || k % 32 || n % 8 || (uint64_t)n > 16ull * (uint64_t)ctx->cu_count) return 1;
  if ((uint64_t)m * k * 2 >= (1ull << 32) || (uint64_t)n * k * 2 >= (1ull << 32)) return 1;
  // Argument errors are left to the caller's general route, which reports them.
  if ((x | b | y) & 15 || bias & 3 || (chain_uses(epi, EOP_BIAS) && !bias)) return 1;
  GemmParams p;
  memset(&p, 0, sizeof p);
  p.a = (const uint16_t*)x;
  p.b = (const uint16_t*)b;
  p.y = (void*)y;
  p.bias = (const float*)bias;
  p.M = m;
  p.N = n;
  p.K = k;
  p.lda = k;
  p.ldb = k;
  p.ldy = n;
  p.split_k = 1;
  p.k_per_split = k;
  p.out_bf16 = out_dtype == T0MI_OUT_BF16;
  p.epi = epi;
  p.xcd_remap = 1;
  p.tiles_m = (m + PD_ROWS - 1) / PD_ROWS;
  p.tiles_n = (n + PD_COLS - 1) / PD_COLS;
  if (ctx->null_backend) return T0MI_OK;
  launch_decode<false>(ctx, ctx->stream, p);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return set_error(T0MI_ERR_HIP, "decode GEMM launch: %s", hipGetErrorString(err));
  return T0MI_OK;
}

}  // namespace t0mi
