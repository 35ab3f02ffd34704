// gemm_xk.hip — split-K GEMMs with the partials combined inside the launch
// through one XCD's L2 (gemm_bf16_xk_kernel, gemm_bf16_kernel.h), for the tiles
// the cost model picks with split-K: 128x128x64 (2x2 waves, 3 LDS stages; the
// skinny and decode-sized shapes), 64x128x64 and 128x256x64
// (2x2 waves, 2 stages; wider N), both B layouts.  Without it a split-K GEMM
// writes split_k fp32 planes to HBM and a second launch sums them.
#include <string.h>

#include <mutex>

#include "t0mi_ctx.h"

namespace t0mi {
namespace {

struct XkEntry {
  int bm, bn, bk, wm, wn, stages, nn;
  const void* kernel;  // for the occupancy query
  void (*launch)(dim3 grid, hipStream_t stream, const GemmParams& p);
  int per_cu;  // workgroups a CU holds at once (queried once; 0: not yet)
};

template <int BM, int BN, int BK, int WM, int WN, int S, bool NN>
void launch_xk(dim3 grid, hipStream_t stream, const GemmParams& p) {
  hipLaunchKernelGGL((gemm_bf16_xk_kernel<BM, BN, BK, WM, WN, S, NN>), grid, dim3(WM * WN * 64), 0, stream, p);
}

#define T0MI_XKE(BM, BN, BK, WM, WN, S, NN)                                                            \
  {BM, BN, BK, WM, WN, S, NN, (const void*)&gemm_bf16_xk_kernel<BM, BN, BK, WM, WN, S, (bool)NN>, \
   &launch_xk<BM, BN, BK, WM, WN, S, (bool)NN>, 0}
XkEntry kXk[] = {
    T0MI_XKE(128, 128, 64, 2, 2, 3, 1), T0MI_XKE(128, 128, 64, 2, 2, 3, 0), T0MI_XKE(64, 128, 64, 2, 2, 2, 1),
    T0MI_XKE(64, 128, 64, 2, 2, 2, 0),  T0MI_XKE(128, 256, 64, 2, 2, 2, 1), T0MI_XKE(128, 256, 64, 2, 2, 2, 0),
};
#undef T0MI_XKE
std::mutex g_xk_mu;

}  // namespace

// The exchange's wait bound: 20 ms of the 100 MHz s_memrealtime clock.  Every
// piece of a tile is resident from the start (the grid fits the GPU in one
// round), so a piece waits at most for the slowest piece's K loop.
constexpr uint64_t kXkWaitTicks = 2000000;

int launch_gemm_xk(t0mi_ctx* ctx, const t0mi_gemm_config& cfg, GemmParams p, bool* launched) {
  *launched = false;
  if (ctx->null_backend || ctx->xk_nx == 0) return T0MI_OK;
  uint32_t wm = 0, wn = 0;
  if (!wave_layout(cfg, &wm, &wn)) return T0MI_OK;
  XkEntry* e = nullptr;
  for (XkEntry& x : kXk)
    if (x.bm == (int)cfg.tile_m && x.bn == (int)cfg.tile_n && x.bk == (int)cfg.tile_k && x.wm == (int)wm &&
        x.wn == (int)wn && x.stages == (int)stages_of(cfg) && x.nn == (cfg.transpose == T0MI_NN ? 1 : 0))
      e = &x;
  const uint32_t sk = p.split_k;
  if (!e || sk < 2 || sk > 16) return T0MI_OK;
  {
    std::lock_guard<std::mutex> lk(g_xk_mu);
    if (e->per_cu == 0) {
      int n = 0;
      hipError_t err = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, e->kernel, e->wm * e->wn * 64, 0);
      e->per_cu = err == hipSuccess && n > 0 ? n : -1;
    }
  }
  if (e->per_cu < 1) return T0MI_OK;
  // Every piece of a tile waits for the others: the whole grid, and each XCD's
  // share of it, must be resident at once.
  const uint32_t nx = ctx->xk_nx, tiles = p.tiles_m * p.tiles_n;
  const uint64_t grid = (uint64_t)(tiles + nx - 1) / nx * nx * sk;
  if (grid > (uint64_t)ctx->cu_count * (uint64_t)e->per_cu) return T0MI_OK;
  XcdExchange x;
  bool ok = false;
  int rc = xk_prepare(ctx, tiles, (size_t)tiles * sk * e->bm * e->bn * 4, &x, &ok);
  if (rc || !ok) return rc;
  p.xk = x;
  p.xk_wait_ticks = kXkWaitTicks;
  p.swap_grid = cfg.swap_grid;
  e->launch(dim3((uint32_t)grid), ctx->stream, p);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return set_error(T0MI_ERR_HIP, "xk gemm launch: %s", hipGetErrorString(err));
  *launched = true;
  return T0MI_OK;
}

}  // namespace t0mi
