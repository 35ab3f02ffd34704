// t0mi_config.cpp — GemmConfig, presets, naming, grids, kernargs and selection.
//
// Host-only logic of the GEMM path, restated from the reference's Rust:
//   GemmConfig + presets + derived sizes + name  src/t0/gemm_gen.rs:55-235
//   compute_grid / _split_k / _auto               src/t0/gemm_gen.rs:308-329, 430-437
//   build_kernargs / _with_bias                   src/t0/gemm_gen.rs:439-484
//   auto_select / auto_select_legacy              src/t0/gemm_gen.rs:340-404
//   cached_auto_select                            src/t0/prefill_spec_cache.rs:42-76
// The RDNA cost model (src/t0/cost_model.rs: 256 VGPRs, wave32, 64 KB LDS) is
// replaced by a gfx950 model: 64-wide waves, 512 VGPR+AGPR per lane, 160 KB
// LDS per CU, 256 CUs, v_mfma_f32_32x32x16_bf16 at 32 cycles.
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <tuple>

#include "t0mi_internal.h"

namespace t0mi {

static thread_local std::string g_last_error;

int set_error(int code, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

uint32_t split_k_of(const t0mi_gemm_config& c) { return c.split_k > 1 ? c.split_k : 1; }

static bool is_pow2(uint32_t v) { return v && !(v & (v - 1)); }

bool wave_layout(const t0mi_gemm_config& c, uint32_t* wm, uint32_t* wn) {
  if (c.wg_size == 0 || c.wg_size % 64) return false;
  const uint32_t nw = c.wg_size / 64;
  if (c.wave_m || c.wave_n) {
    if (c.wave_m * c.wave_n != nw) return false;
    *wm = c.wave_m;
    *wn = c.wave_n;
    return true;
  }
  // Derived: as many waves along M as the tile has 32-row blocks, rest along N.
  uint32_t best_m = 0;
  for (uint32_t m = 1; m <= nw; ++m)
    if (nw % m == 0 && c.tile_m % (32 * m) == 0 && c.tile_n % (32 * (nw / m)) == 0) best_m = m;
  if (!best_m) return false;
  *wm = best_m;
  *wn = nw / best_m;
  return true;
}

uint32_t stages_of(const t0mi_gemm_config& c) { return c.stages ? c.stages : 2u; }

static uint32_t lds_total(const t0mi_gemm_config& c) {
  // `stages` copies of the A and B tiles, bf16, no padding (XOR swizzle instead).
  return stages_of(c) * (c.tile_m + c.tile_n) * c.tile_k * 2u;
}

static uint32_t est_regs(const t0mi_gemm_config& c) {
  uint32_t wm = 1, wn = 1;
  if (!wave_layout(c, &wm, &wn)) return 0xFFFFFFFFu;
  const uint32_t nthr = c.wg_size;
  const uint32_t acc = (c.tile_m / wm) * (c.tile_n / wn) / 64;                // fp32 per lane
  const uint32_t frags = ((c.tile_m / wm) / 32 + (c.tile_n / wn) / 32) * 4;  // one k-step
  const uint32_t stage = ((c.tile_m + c.tile_n) * c.tile_k * 2 + nthr * 16 - 1) / (nthr * 16) * 4;
  return acc + frags + stage + 40;
}

bool config_feasible(const t0mi_gemm_config& c, std::string* why) {
  auto fail = [&](const char* m) {
    if (why) *why = m;
    return false;
  };
  if (c.wg_size < 64 || c.wg_size > 1024 || c.wg_size % 64)
    return fail("wg_size must be a multiple of 64 in [64, 1024] (gfx950 waves are 64 wide)");
  if (c.tile_m < 32 || c.tile_m % 32 || c.tile_n < 32 || c.tile_n % 32)
    return fail("tile_m and tile_n must be multiples of 32 (32x32 MFMA blocks)");
  if (c.tile_k != 16 && c.tile_k != 32 && c.tile_k != 64) return fail("tile_k must be 16, 32 or 64");
  uint32_t wm, wn;
  if (!wave_layout(c, &wm, &wn)) return fail("no wave layout splits the tile into 32x32 multiples");
  if (c.tile_m % (32 * wm) || c.tile_n % (32 * wn)) return fail("wave tile is not a multiple of 32x32");
  if (stages_of(c) < 2 || stages_of(c) > 5) return fail("stages must be 2..5");
  if (lds_total(c) > 160u * 1024u) return fail("LDS over 160 KB");
  if (est_regs(c) > 512) return fail("estimated registers over 512 (VGPR+AGPR)");
  const uint32_t sk = split_k_of(c);
  if (!is_pow2(sk) || sk > 16) return fail("split_k must be a power of two <= 16");
  if (c.transpose > T0MI_NN) return fail("bad transpose");
  if (c.epilogue > T0MI_EPI_BIAS_ADD_RELU_STORE_F32) return fail("bad epilogue");
  if (c.out_dtype > T0MI_OUT_BF16) return fail("bad out_dtype");
  return true;
}

std::string config_name(const t0mi_gemm_config& c) {
  // GemmConfig::name, src/t0/gemm_gen.rs:215-235.
  char buf[256];
  const char* lds_tag = c.use_lds ? (c.double_buffer ? "_ldsdb" : "_lds") : "_direct";
  char sk_tag[16] = "";
  if (c.split_k > 1) snprintf(sk_tag, sizeof sk_tag, "_sk%u", c.split_k);
  char pass_tag[16] = "";
  if (c.n_col_passes > 1) snprintf(pass_tag, sizeof pass_tag, "_%up", c.n_col_passes);
  const char* grid_tag = c.swap_grid ? "" : "_mg";
  const char* wgp_tag = c.wgp_mode ? "_wgp" : "";
  const char* trans_tag = c.transpose == T0MI_NN ? "_nn" : "";
  const char* epi_tag = c.epilogue == T0MI_EPI_BIAS_ADD_STORE_F32        ? "_bias"
                        : c.epilogue == T0MI_EPI_BIAS_ADD_RELU_STORE_F32 ? "_bias_relu"
                                                                         : "";
  // gfx950 extensions: only present when they differ from the defaults, so
  // every reference config keeps its reference name.
  const char* out_tag = c.out_dtype == T0MI_OUT_BF16 ? "_bf16o" : "";
  char wave_tag[24] = "";
  if (c.wave_m || c.wave_n) {
    t0mi_gemm_config d = c;
    d.wave_m = d.wave_n = 0;
    uint32_t dm = 0, dn = 0;
    if (!wave_layout(d, &dm, &dn) || dm != c.wave_m || dn != c.wave_n)
      snprintf(wave_tag, sizeof wave_tag, "_w%ux%u", c.wave_m, c.wave_n);
  }
  char stage_tag[16] = "";
  if (stages_of(c) != 2) snprintf(stage_tag, sizeof stage_tag, "_s%u", stages_of(c));
  snprintf(buf, sizeof buf, "t0_gemm_%ux%u_k%u%s%s%s%s%s%s%s%s%s%s", c.tile_m, c.tile_n, c.tile_k, lds_tag,
           sk_tag, pass_tag, grid_tag, wgp_tag, trans_tag, epi_tag, out_tag, wave_tag, stage_tag);
  return buf;
}

// ---------------------------------------------------------------- variants --

const std::vector<GemmVariant>& gemm_variants() {
  static const std::vector<GemmVariant> v = [] {
    std::vector<GemmVariant> out;
    for (int nn = 0; nn < 2; ++nn) {
#define T0MI_V(BM, BN, BK, WM, WN, S) out.push_back(GemmVariant{BM, BN, BK, WM, WN, S, nn});
#define T0MI_V_NT(BM, BN, BK, WM, WN, S) \
  if (!nn) out.push_back(GemmVariant{BM, BN, BK, WM, WN, S, nn});
#include "gemm_variants.def"
#undef T0MI_V
#undef T0MI_V_NT
    }
    return out;
  }();
  return v;
}

bool has_variant(const t0mi_gemm_config& c) {
  uint32_t wm, wn;
  if (!wave_layout(c, &wm, &wn)) return false;
  for (const auto& v : gemm_variants())
    if ((uint32_t)v.bm == c.tile_m && (uint32_t)v.bn == c.tile_n && (uint32_t)v.bk == c.tile_k &&
        (uint32_t)v.wm == wm && (uint32_t)v.wn == wn && (uint32_t)v.stages == stages_of(c) &&
        (uint32_t)v.nn == (c.transpose == T0MI_NN))
      return true;
  return false;
}

static uint32_t round_up(uint32_t v, uint32_t m) { return (v + m - 1) / m * m; }

const GemmVariant* physical_variant(uint32_t tile_m, uint32_t tile_n, uint32_t tile_k, uint32_t wg_size,
                                    uint32_t stages, int nn, uint32_t* bk_out) {
  // Rows and columns round up to whole 32x32 MFMA blocks (NN B tiles to 64
  // columns, the transpose-read width); K steps of 16, 32 or 64 divide any
  // logical tile_k that is a multiple of 16.  Among matching kernels: the
  // logical stage count and workgroup size if one has them, else the first.
  const uint32_t bm = round_up(tile_m, 32);
  const uint32_t bn = nn ? std::max(64u, round_up(tile_n, 32)) : round_up(tile_n, 32);
  const uint32_t bk = tile_k % 64 == 0 ? 64 : tile_k % 32 == 0 ? 32 : 16;
  const GemmVariant* best = nullptr;
  int best_score = -1;
  for (const auto& v : gemm_variants()) {
    if ((uint32_t)v.bm != bm || (uint32_t)v.bn != bn || (uint32_t)v.bk != bk || v.nn != nn) continue;
    const int score = 2 * ((uint32_t)v.stages == stages) + ((uint32_t)(64 * v.wm * v.wn) == round_up(wg_size, 64));
    if (score > best_score) best = &v, best_score = score;
  }
  if (best && bk_out) *bk_out = bk;
  return best;
}

bool config_physical(const t0mi_gemm_config& c, t0mi_gemm_config* phys, std::string* why) {
  auto fail = [&](const std::string& m) {
    if (why) *why = m;
    return false;
  };
  // A gfx950-native config runs its own kernel.
  std::string native_why;
  if (config_feasible(c, &native_why) && has_variant(c)) {
    *phys = c;
    return true;
  }
  // Reference shapes with no kernel of their own on 64-wide waves (the wave32
  // tile_16x64_k16 preset, gemm_gen.rs:88-90, that bf16_matmul.rs:140-149
  // selects for m <= 16; rows or columns that are not whole 32x32 blocks; a
  // tile_k of 48) run on the prebuilt kernel covering the same tile.  Results
  // do not depend on the tile, and the logical config keeps its name, grid,
  // kernarg layout and attributes.
  if (c.wave_m || c.wave_n) return fail(native_why.empty() ? "no prebuilt kernel for this wave layout" : native_why);
  if (c.wg_size < 32 || c.wg_size > 1024 || c.wg_size % 32)
    return fail("wg_size must be a multiple of 32 in [32, 1024]");
  if (!c.tile_m || !c.tile_n || c.tile_m % 16 || c.tile_n % 16 || c.tile_m > 256 || c.tile_n > 256)
    return fail("tile_m and tile_n must be multiples of 16 up to 256");
  if (!c.tile_k || c.tile_k % 16 || c.tile_k > 256) return fail("tile_k must be a multiple of 16 up to 256");
  const uint32_t sk = split_k_of(c);
  if (!is_pow2(sk) || sk > 16) return fail("split_k must be a power of two <= 16");
  if (c.transpose > T0MI_NN || c.epilogue > T0MI_EPI_BIAS_ADD_RELU_STORE_F32 || c.out_dtype > T0MI_OUT_BF16)
    return fail("bad transpose, epilogue or out_dtype");
  if (stages_of(c) < 2 || stages_of(c) > 5) return fail("stages must be 2..5");
  uint32_t bk = 0;
  const GemmVariant* v = physical_variant(c.tile_m, c.tile_n, c.tile_k, c.wg_size, stages_of(c),
                                          c.transpose == T0MI_NN, &bk);
  if (!v) return fail(native_why.empty() ? "no prebuilt gfx950 kernel covers this tile" : native_why);
  t0mi_gemm_config p = c;
  p.tile_m = v->bm;
  p.tile_n = v->bn;
  p.tile_k = bk;
  p.wg_size = 64u * v->wm * v->wn;
  p.wave_m = v->wm;
  p.wave_n = v->wn;
  p.stages = v->stages == 2 ? 0 : v->stages;
  if (!config_feasible(p, why)) return false;
  *phys = p;
  return true;
}

// ------------------------------------------------------------- cost model --
// Analytic time estimate (microseconds) on MI355X for one config.
// Workgroups of config c one CU holds at once, limited by LDS (160 KB) and by
// registers (512 per lane, 4 SIMDs); at most 8.
static double wg_per_cu_of(const t0mi_gemm_config& c) {
  uint32_t wm = 1, wn = 1;
  wave_layout(c, &wm, &wn);
  const double W = wm * wn;
  const double regs = std::max(64u, est_regs(c));
  const double waves_per_simd = std::max(1.0, floor(512.0 / regs));
  const double wg = std::min(floor(160.0 * 1024.0 / lds_total(c)), floor(4.0 * waves_per_simd / W));
  return std::max(1.0, std::min(wg, 8.0));
}

static const double kCUs = 256;

static double estimate_us(const t0mi_gemm_config& c, uint32_t m, uint32_t n, uint32_t k) {
  const double CUS = kCUs, CLK = 2.4e9, FLOP_PER_CLK_CU = 4096.0;
  const double HBM = 6.0e12, L2 = 30.0e12;
  uint32_t wm = 1, wn = 1;
  wave_layout(c, &wm, &wn);
  const double W = wm * wn;
  const double FM = (c.tile_m / wm) / 32.0, FN = (c.tile_n / wn) / 32.0;
  // MFMA issue efficiency of one wave: 32-cycle MFMAs against the LDS reads
  // and address work of each 16-deep k-step, plus a per-K-tile barrier and
  // global->LDS staging cost (~200 cycles) that deeper tiles amortise.
  const double KS = c.tile_k / 16.0;
  const double mf = FM * FN * 32.0 * KS;
  const double eff = mf / (mf + (16.0 * (FM + FN) + 24.0) * KS + 200.0);
  const uint32_t sk = split_k_of(c);
  const double tm = ceil((double)m / c.tile_m), tn = ceil((double)n / c.tile_n);
  const double tiles = tm * tn * sk;
  const double wg_per_cu = wg_per_cu_of(c);
  const double kp = ceil((double)k / sk / c.tile_k) * c.tile_k;
  const double flops_tile = 2.0 * c.tile_m * c.tile_n * kp;
  const double busy = std::min(1.0, W * wg_per_cu / 4.0);
  // A single wave per SIMD has nothing to issue while it waits on its own LDS
  // reads and barriers (measured: 256x256 with 4 waves runs ~10% slower than
  // with 8 at 4096^3, despite the larger per-wave MFMA blocks).
  const double hide = W * wg_per_cu / 4.0 < 2.0 ? 0.8 : 1.0;
  // A last, partly filled round of tiles runs on a lightly loaded GPU (the power
  // limit no longer sets the clock): 0.6 of a full round when nearly empty
  // (1536 x 11008 x 4096 with 256 x 256 tiles, 258 tiles on 256 CUs: 158 us,
  // against ~94 us per full round at 4096^3).
  const double slots = CUS * wg_per_cu;
  const double full_rounds = floor(tiles / slots), rest = tiles - full_rounds * slots;
  const double rounds_c = full_rounds + (rest > 0 ? 0.6 + 0.4 * rest / slots : 0.0);
  const double t_comp = rounds_c * wg_per_cu * flops_tile / (FLOP_PER_CLK_CU * CLK * eff * busy * hide);
  const double out_b = c.out_dtype == T0MI_OUT_BF16 ? 2.0 : 4.0;
  double hbm_bytes = 2.0 * m * k + 2.0 * k * n + (sk > 1 ? 0.0 : out_b) * m * n;
  const double l2_bytes = tiles * (c.tile_m + c.tile_n) * kp * 2.0;
  // What one CU streams: its share of the workgroups, each its A and B panels
  // over its K range and its split-K plane.  The rate a CU sustains through the
  // LDS DMA of these kernels is set by the bytes it keeps in flight -- the
  // workgroups resident on it at once, each with its LDS stages of a K tile --
  // and saturates at ~50 GB/s: 5 + 0.4 GB/s per KB in flight.  Fitted to the
  // times of every prebuilt candidate on 82 shapes (m = 1 .. 4096, N and K of
  // 4096 .. 14336, both B layouts; B rotated over copies that exceed the
  // Infinity Cache): with a fixed 55 GB/s per CU the model's pick came within
  // 3 % of the fastest candidate on 31 of them, with this rate on 68.  It is
  // what makes 128 x 128 tiles with four LDS stages and the many small
  // workgroups of 64 x 64 / 64 x 128 tiles beat 128 x 256 tiles at 1-128 rows.
  // Fewer resident waves than SIMDs issue the loads more slowly (single-wave
  // 64 x 64 workgroups against four-wave ones of the same tile): the rate
  // scales with the resident waves up to four (checked on 80 further shapes,
  // N and K of 5120 .. 13824: picks within 3 % of the fastest on 55 of them
  // against 38 for the fixed rate).
  const double per_wg = (c.tile_m + c.tile_n) * kp * 2.0 + (sk > 1 ? c.tile_m * c.tile_n * 4.0 : 0.0);
  const double wg_on_cu = std::min(wg_per_cu, ceil(tiles / CUS));
  const double stages = std::max<uint32_t>(2u, c.stages);
  const double in_flight_kb = wg_on_cu * stages * (c.tile_m + c.tile_n) * c.tile_k * 2.0 / 1024.0;
  const double R_CU = std::min(50.0, 5.0 + 0.4 * in_flight_kb) * 1e9 * std::min(1.0, wg_on_cu * W / 4.0);
  const double cu_bytes = ceil(tiles / CUS) * per_wg;
  const double t_mem = std::max({hbm_bytes / HBM, l2_bytes / L2, cu_bytes / R_CU});
  double t = std::max(t_comp, t_mem) * 1e6 + 3.0;
  // The split-K reduce pass is a separate launch: it reads every fp32 partial
  // plane, just written and mostly served by the Infinity Cache (~12 TB/s),
  // and writes the output once.
  if (sk > 1) t += (sk * 4.0 * m * n / 12.0e12 + out_b * m * n / HBM) * 1e6 + 2.0;
  // The split-K planes are stored after the K loops, all workgroups at once, so
  // their write does not overlap the streaming of the operands; fitted with the
  // rate above at three times the plane bytes over the HBM rate (the write-back
  // after the kernel and the reduce's first reads wait on it).
  if (sk > 1) t += 3.0 * sk * 4.0 * m * n / HBM * 1e6;
  return t;
}

static t0mi_gemm_config make_cfg(int bm, int bn, int bk, int wm, int wn, uint32_t sk, uint32_t transpose,
                                 uint32_t out_dtype, uint32_t stages = 2) {
  t0mi_gemm_config c;
  memset(&c, 0, sizeof c);
  c.stages = stages == 2 ? 0 : stages;
  c.tile_m = bm;
  c.tile_n = bn;
  c.tile_k = bk;
  c.wg_size = 64 * wm * wn;
  c.use_lds = 1;
  c.double_buffer = 1;
  c.split_k = sk > 1 ? sk : 0;
  c.n_col_passes = 1;
  c.swap_grid = 1;
  c.transpose = transpose;
  c.out_dtype = out_dtype;
  c.wave_m = wm;
  c.wave_n = wn;
  // Keep the reference-preset names when the wave layout is the derived one.
  t0mi_gemm_config d = c;
  d.wave_m = d.wave_n = 0;
  uint32_t dm, dn;
  if (wave_layout(d, &dm, &dn) && dm == (uint32_t)wm && dn == (uint32_t)wn) c.wave_m = c.wave_n = 0;
  return c;
}

std::vector<t0mi_gemm_config> rank_candidates(uint32_t m, uint32_t n, uint32_t k, uint32_t transpose,
                                              uint32_t out_dtype, std::vector<double>* est_us) {
  std::vector<std::pair<double, t0mi_gemm_config>> scored;
  const int want_nn = transpose == T0MI_NN;
  for (const auto& v : gemm_variants()) {
    if (v.nn != want_nn) continue;
    for (uint32_t sk = 1; sk <= 16; sk *= 2) {
      // Each partition keeps at least eight K tiles: with fewer, the per-workgroup
      // prologue, plane store and the reduce launch outweigh the shorter K loop
      // (1024^3 with 128 x 128 tiles: 12.5 us unsplit, 18.2 us at split-K 4).
      if (sk > 1 && (uint64_t)k < (uint64_t)sk * v.bk * 8) break;
      t0mi_gemm_config c = make_cfg(v.bm, v.bn, v.bk, v.wm, v.wn, sk, transpose, out_dtype, v.stages);
      if (!config_feasible(c, nullptr)) continue;
      scored.push_back({estimate_us(c, m, n, k), c});
    }
  }
  std::stable_sort(scored.begin(), scored.end(),
                   [](const std::pair<double, t0mi_gemm_config>& a, const std::pair<double, t0mi_gemm_config>& b) {
                     return a.first < b.first;
                   });
  std::vector<t0mi_gemm_config> out;
  if (est_us) est_us->clear();
  for (auto& s : scored) {
    out.push_back(s.second);
    if (est_us) est_us->push_back(s.first);
  }
  return out;
}

bool plan_column_split(const t0mi_gemm_config& head, uint32_t m, uint32_t n, uint32_t k, uint32_t transpose,
                       uint32_t out_dtype, uint32_t* n_main, t0mi_gemm_config* tail, uint32_t cus) {
  if (split_k_of(head) > 1 || m == 0 || n == 0 || k == 0 || cus == 0) return false;
  const uint64_t slots = (uint64_t)(cus * wg_per_cu_of(head));
  const uint64_t tm = (m + head.tile_m - 1) / head.tile_m, tn = (n + head.tile_n - 1) / head.tile_n;
  const uint64_t full_rounds = tm * tn / slots;
  if (full_rounds == 0 || tm * tn % slots == 0) return false;
  // Whole columns of tiles that fill whole rounds (at most that many tiles).
  const uint64_t main_tn = full_rounds * slots / tm;
  if (main_tn == 0 || main_tn >= tn) return false;
  const uint32_t n1 = (uint32_t)(main_tn * head.tile_n), n2 = n - n1;
  std::vector<double> est;
  const std::vector<t0mi_gemm_config> cands = rank_candidates(m, n2, k, transpose, out_dtype, &est);
  for (size_t i = 0; i < cands.size(); ++i) {
    if (!has_variant(cands[i])) continue;
    // Kept only when the model expects the pair to beat the single launch by more
    // than a launch's worth.
    if (estimate_us(head, m, n1, k) + est[i] + 1.0 >= estimate_us(head, m, n, k)) return false;
    *n_main = n1;
    *tail = cands[i];
    return true;
  }
  return false;
}

}  // namespace t0mi

using namespace t0mi;

// ===================================================================== C ABI ==

extern "C" const char* t0mi_last_error(void) { return g_last_error.c_str(); }
extern "C" int t0mi_abi_version(void) { return T0MI_ABI_VERSION; }
extern "C" const char* t0mi_build_target(void) { return "gfx950"; }

namespace {
struct Preset {
  const char* name;
  uint32_t tm, tn, tk, wg, use_lds, np;
};
// src/t0/gemm_gen.rs:87-145 (reference presets; wgp_mode=true, swap_grid=true there),
// followed by the gfx950 presets.
const Preset kPresets[] = {
    {"tile_16x64_k16", 16, 64, 16, 32, 1, 1},     {"tile_32x64_direct", 32, 64, 16, 64, 0, 1},
    {"tile_32x64_k16", 32, 64, 16, 64, 1, 1},     {"tile_32x64_k32", 32, 64, 32, 64, 1, 1},
    {"tile_32x128_k16", 32, 128, 16, 64, 1, 1},   {"tile_64x64_k16", 64, 64, 16, 64, 1, 1},
    {"tile_64x64_k32", 64, 64, 32, 64, 1, 1},     {"tile_128x64_k16", 128, 64, 16, 128, 1, 1},
    {"tile_64x128_k16", 64, 128, 16, 64, 1, 1},   {"tile_128x64_k32", 128, 64, 32, 128, 1, 1},
    {"tile_128x128_k16", 128, 128, 16, 128, 1, 1}, {"tile_64x64_k64", 64, 64, 64, 64, 1, 1},
    {"tile_128x128_2pass", 128, 64, 16, 128, 1, 2}, {"tile_64x128_2pass", 64, 64, 16, 64, 1, 2},
};
struct Preset950 {
  const char* name;
  int bm, bn, bk, wm, wn, stages;
};
const Preset950 kPresets950[] = {
    {"gfx950_256x256_k64_w2x4", 256, 256, 64, 2, 4, 2},    {"gfx950_256x256_k32_w2x4_s3", 256, 256, 32, 2, 4, 3},
    {"gfx950_256x256_k32_w2x4_s4", 256, 256, 32, 2, 4, 4}, {"gfx950_256x256_k64_w2x2", 256, 256, 64, 2, 2, 2},
    {"gfx950_256x128_k64_w2x4_s3", 256, 128, 64, 2, 4, 3}, {"gfx950_256x128_k64_w2x2", 256, 128, 64, 2, 2, 2},
    {"gfx950_128x256_k64_w2x2", 128, 256, 64, 2, 2, 2},    {"gfx950_128x128_k64_w2x2", 128, 128, 64, 2, 2, 2},
    {"gfx950_128x128_k64_w2x2_s3", 128, 128, 64, 2, 2, 3}, {"gfx950_128x64_k64_w2x2", 128, 64, 64, 2, 2, 2},
    {"gfx950_64x128_k64_w2x2", 64, 128, 64, 2, 2, 2},      {"gfx950_64x64_k64_w2x2", 64, 64, 64, 2, 2, 2},
    {"gfx950_128x128_k32_w2x2", 128, 128, 32, 2, 2, 2},
};
}  // namespace

extern "C" int t0mi_config_preset(const char* name, t0mi_gemm_config* out) {
  if (!name || !out) return set_error(T0MI_ERR_INVALID, "null argument");
  for (const auto& p : kPresets) {
    if (strcmp(p.name, name) == 0) {
      memset(out, 0, sizeof *out);
      out->tile_m = p.tm;
      out->tile_n = p.tn;
      out->tile_k = p.tk;
      out->wg_size = p.wg;
      out->use_lds = p.use_lds;
      out->double_buffer = p.use_lds;
      out->n_col_passes = p.np;
      out->swap_grid = 1;
      out->wgp_mode = 1;
      return T0MI_OK;
    }
  }
  for (const auto& p : kPresets950) {
    if (strcmp(p.name, name) == 0) {
      *out = make_cfg(p.bm, p.bn, p.bk, p.wm, p.wn, 1, T0MI_NT, T0MI_OUT_F32, p.stages);
      return T0MI_OK;
    }
  }
  return set_error(T0MI_ERR_NOT_FOUND, "unknown preset '%s'", name);
}

extern "C" int t0mi_config_preset_names(char* buf, size_t len) {
  std::string s;
  for (const auto& p : kPresets) s += std::string(s.empty() ? "" : ",") + p.name;
  for (const auto& p : kPresets950) s += std::string(",") + p.name;
  if (buf && len) {
    strncpy(buf, s.c_str(), len - 1);
    buf[len - 1] = 0;
  }
  return (int)s.size();
}

extern "C" int t0mi_gemm_variants(char* buf, size_t len) {
  std::string s;
  for (const auto& v : gemm_variants()) {
    char e[64];
    snprintf(e, sizeof e, "%s%dx%dx%d_w%dx%d_s%d%s", s.empty() ? "" : ",", v.bm, v.bn, v.bk, v.wm, v.wn, v.stages,
             v.nn ? "_nn" : "");
    s += e;
  }
  if (buf && len) {
    strncpy(buf, s.c_str(), len - 1);
    buf[len - 1] = 0;
  }
  return (int)s.size();
}

extern "C" uint32_t t0mi_config_n_waves(const t0mi_gemm_config* cfg) { return cfg ? cfg->wg_size / 64 : 0; }
extern "C" uint32_t t0mi_config_lds_total(const t0mi_gemm_config* cfg) { return cfg ? lds_total(*cfg) : 0; }
extern "C" uint32_t t0mi_config_estimated_regs(const t0mi_gemm_config* cfg) { return cfg ? est_regs(*cfg) : 0; }

extern "C" int t0mi_config_is_feasible(const t0mi_gemm_config* cfg) {
  t0mi_gemm_config phys;
  return cfg && (config_feasible(*cfg, nullptr) || config_physical(*cfg, &phys, nullptr)) ? 1 : 0;
}

extern "C" int t0mi_config_name(const t0mi_gemm_config* cfg, char* buf, size_t len) {
  if (!cfg) return set_error(T0MI_ERR_INVALID, "null config");
  std::string s = config_name(*cfg);
  if (buf && len) {
    strncpy(buf, s.c_str(), len - 1);
    buf[len - 1] = 0;
  }
  return (int)s.size();
}

extern "C" int t0mi_compute_grid(const t0mi_gemm_config* cfg, uint32_t m, uint32_t n, uint32_t grid[2]) {
  // src/t0/gemm_gen.rs:308-318.
  if (!cfg || !grid || !cfg->tile_m || !cfg->tile_n) return set_error(T0MI_ERR_INVALID, "bad argument");
  const uint32_t tiles_m = (m + cfg->tile_m - 1) / cfg->tile_m;
  const uint32_t tiles_n = (n + cfg->tile_n - 1) / cfg->tile_n;
  if (cfg->swap_grid) {
    grid[0] = tiles_n * cfg->wg_size;
    grid[1] = tiles_m;
  } else {
    grid[0] = tiles_m * cfg->wg_size;
    grid[1] = tiles_n;
  }
  return T0MI_OK;
}

extern "C" int t0mi_compute_grid_split_k(const t0mi_gemm_config* cfg, uint32_t m, uint32_t n, uint32_t split_k,
                                         uint32_t grid[2]) {
  // src/t0/gemm_gen.rs:321-329 (the reference asserts a power of two).
  if (!is_pow2(split_k)) return set_error(T0MI_ERR_INVALID, "split_k=%u must be power of 2", split_k);
  int rc = t0mi_compute_grid(cfg, m, n, grid);
  if (rc) return rc;
  grid[1] *= split_k;
  return T0MI_OK;
}

extern "C" int t0mi_compute_grid_auto(const t0mi_gemm_config* cfg, uint32_t m, uint32_t n, uint32_t grid[2]) {
  // src/t0/gemm_gen.rs:430-437.
  if (!cfg) return set_error(T0MI_ERR_INVALID, "null config");
  const uint32_t sk = split_k_of(*cfg);
  return sk > 1 ? t0mi_compute_grid_split_k(cfg, m, n, sk, grid) : t0mi_compute_grid(cfg, m, n, grid);
}

static void put_u64(uint8_t* p, uint64_t v) {
  for (int i = 0; i < 8; ++i) p[i] = (uint8_t)(v >> (8 * i));
}
static void put_u32(uint8_t* p, uint32_t v) {
  for (int i = 0; i < 4; ++i) p[i] = (uint8_t)(v >> (8 * i));
}

extern "C" int t0mi_build_kernargs(uint64_t x, uint64_t wt, uint64_t y, uint32_t k, uint32_t n, uint32_t m,
                                   const t0mi_gemm_config* cfg, uint8_t out[40]) {
  // src/t0/gemm_gen.rs:439-458.
  if (!cfg || !out) return set_error(T0MI_ERR_INVALID, "null argument");
  const uint32_t sk = split_k_of(*cfg);
  const uint32_t y_stride = sk > 1 ? m * n * 4u : 0u;
  put_u64(out + 0, x);
  put_u64(out + 8, wt);
  put_u64(out + 16, y);
  put_u32(out + 24, k);
  put_u32(out + 28, n);
  put_u32(out + 32, 0u);
  put_u32(out + 36, y_stride);
  return T0MI_OK;
}

extern "C" int t0mi_build_kernargs_with_bias(uint64_t x, uint64_t wt, uint64_t y, uint32_t k, uint32_t n,
                                             uint32_t m, const t0mi_gemm_config* cfg, uint64_t bias,
                                             uint8_t out[48]) {
  // src/t0/gemm_gen.rs:460-484.
  int rc = t0mi_build_kernargs(x, wt, y, k, n, m, cfg, out);
  if (rc) return rc;
  put_u64(out + 40, bias);
  return T0MI_OK;
}

extern "C" int t0mi_auto_select(uint32_t m, uint32_t k, uint32_t n, t0mi_gemm_config* out) {
  // auto_select -> cost_model::predict_best (src/t0/gemm_gen.rs:340, cost_model.rs:660-668);
  // falls back to the legacy heuristic when the model finds nothing.
  if (!out) return set_error(T0MI_ERR_INVALID, "null config");
  if (!m || !n || !k) return set_error(T0MI_ERR_INVALID, "zero dimension");
  auto c = rank_candidates(m, n, k, T0MI_NT, T0MI_OUT_F32, nullptr);
  if (c.empty()) return t0mi_auto_select_legacy(m, k, n, out);
  *out = c[0];
  return T0MI_OK;
}

extern "C" int t0mi_auto_select_layout(uint32_t m, uint32_t k, uint32_t n, uint32_t transpose, uint32_t out_dtype,
                                       t0mi_gemm_config* out) {
  // auto_select for a given B layout and output type: the same cost-model
  // ranking, restricted to prebuilt kernels of that layout (NN needs tile_n >= 64).
  if (!out) return set_error(T0MI_ERR_INVALID, "null config");
  if (!m || !n || !k) return set_error(T0MI_ERR_INVALID, "zero dimension");
  if (transpose > T0MI_NN || out_dtype > T0MI_OUT_BF16) return set_error(T0MI_ERR_INVALID, "bad layout or out_dtype");
  auto c = rank_candidates(m, n, k, transpose, out_dtype, nullptr);
  if (c.empty()) return set_error(T0MI_ERR_NO_KERNEL, "no prebuilt kernel for %ux%ux%u", m, n, k);
  *out = c[0];
  return T0MI_OK;
}

extern "C" int t0mi_auto_schedule_gemm(uint32_t m, uint32_t n, uint32_t k, uint32_t transpose, uint32_t out_dtype,
                                       t0mi_gemm_config* out, double* est_us, uint32_t cap, uint32_t* count) {
  // cost_model::auto_schedule_gemm (src/t0/cost_model.rs:464-534): every feasible
  // prebuilt configuration of the layout, best first, with its estimate.
  if (!count || (cap && !out)) return set_error(T0MI_ERR_INVALID, "null output");
  if (!m || !n || !k) return set_error(T0MI_ERR_INVALID, "zero dimension");
  if (transpose > T0MI_NN || out_dtype > T0MI_OUT_BF16) return set_error(T0MI_ERR_INVALID, "bad layout or out_dtype");
  std::vector<double> est;
  auto c = rank_candidates(m, n, k, transpose, out_dtype, &est);
  *count = (uint32_t)c.size();
  for (uint32_t i = 0; i < cap && i < c.size(); ++i) {
    out[i] = c[i];
    if (est_us) est_us[i] = est[i];
  }
  return T0MI_OK;
}

extern "C" int t0mi_auto_select_legacy(uint32_t m, uint32_t k, uint32_t n, t0mi_gemm_config* out) {
  // The shape buckets of auto_select_legacy (src/t0/gemm_gen.rs:351-404), with
  // gfx950 tiles: large squares take the 256x256 8-wave tile, thin/small
  // problems take smaller tiles plus split-K so that >= 256 CUs get work.
  if (!out) return set_error(T0MI_ERR_INVALID, "null config");
  if (!m || !n || !k) return set_error(T0MI_ERR_INVALID, "zero dimension");
  auto clamp_sk = [&](uint32_t tile_k, uint32_t want) -> uint32_t {
    uint32_t sk = std::min(want, k / tile_k);
    while (sk > 1 && k % (tile_k * sk) != 0) sk /= 2;
    return sk > 1 ? sk : 1;
  };
  const uint64_t mn = (uint64_t)m * n;
  if (m >= 2048 && n >= 2048) {
    *out = make_cfg(256, 256, 64, 2, 4, 1, T0MI_NT, T0MI_OUT_F32);
  } else if (mn >= 1024ull * 1024ull) {
    *out = make_cfg(128, 128, 64, 2, 2, 1, T0MI_NT, T0MI_OUT_F32);
  } else if (m <= 256 && k >= 512 && n >= 1024) {
    // Thin: few output tiles, long K -> split K.
    const uint32_t tiles = ((m + 127) / 128) * ((n + 63) / 64);
    const uint32_t want = tiles >= 256 ? 1 : std::min(16u, 256u / std::max(1u, tiles));
    *out = make_cfg(128, 64, 64, 2, 2, clamp_sk(64, want), T0MI_NT, T0MI_OUT_F32);
  } else {
    const uint32_t tiles = ((m + 63) / 64) * ((n + 63) / 64);
    const uint32_t want = tiles >= 128 ? 1 : std::min(8u, 256u / std::max(1u, tiles));
    *out = make_cfg(64, 64, 64, 2, 2, k >= 256 ? clamp_sk(64, want) : 1, T0MI_NT, T0MI_OUT_F32);
  }
  return T0MI_OK;
}

namespace {
std::mutex g_spec_mu;
std::map<std::tuple<uint32_t, uint32_t, uint32_t>, t0mi_gemm_config> g_spec_cache;
}  // namespace

extern "C" int t0mi_cached_auto_select(uint32_t m, uint32_t k, uint32_t n, t0mi_gemm_config* out) {
  // src/t0/prefill_spec_cache.rs:42-76: process-wide (m,k,n) -> config map.
  if (!out) return set_error(T0MI_ERR_INVALID, "null config");
  std::lock_guard<std::mutex> lk(g_spec_mu);
  auto key = std::make_tuple(m, k, n);
  auto it = g_spec_cache.find(key);
  if (it != g_spec_cache.end()) {
    *out = it->second;
    return T0MI_OK;
  }
  int rc = t0mi_auto_select(m, k, n, out);
  if (rc) return rc;
  g_spec_cache[key] = *out;
  return T0MI_OK;
}

extern "C" void t0mi_clear_spec_cache(void) {
  std::lock_guard<std::mutex> lk(g_spec_mu);
  g_spec_cache.clear();
}

extern "C" size_t t0mi_spec_cache_len(void) {
  std::lock_guard<std::mutex> lk(g_spec_mu);
  return g_spec_cache.size();
}
