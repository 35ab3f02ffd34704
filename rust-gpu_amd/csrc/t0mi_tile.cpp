// t0mi_tile.cpp — the tile_ir surface: TileGemm specs, presets, names, LDS and
// grid arithmetic, kernarg layouts and tile_auto_select.
//
// Host-only logic restated from the reference's Rust:
//   TileGemm + EpilogueOp + TileTranspose        src/t0/tile_ir.rs:20-152
//   presets tile_*                               src/t0/tile_ir.rs:156-604
//   n_waves / wg_size / lds_total / name          src/t0/tile_ir.rs:607-701
//   tile_auto_select                             src/t0/tile_ir.rs:740-870
//   build_kernargs / _m / _m_with_counter        src/t0/tile_ir.rs:4570-4637
//   compute_grid                                 src/t0/tile_ir.rs:4645-4666
//   kernarg allocator (8-aligned pointers)       src/t0/compile.rs:120-180
// The lowering (lower_gemm, tile_ir.rs:887) becomes a lookup of the prebuilt
// gfx950 kernel with the spec's tile shape (tile_lower below).
#include <string.h>

#include <string>

#include "t0mi_internal.h"

namespace t0mi {

namespace {

struct TilePreset {
  const char* name;
  uint32_t m, n, k, wgp, db, swap_grid, acc_swap, persistent;
};

// Field values of each TileGemm::tile_* constructor (all: split_k 1, NT,
// triple_buffer false, waves_per_wg None, BF16_F32, no epilogue).
const TilePreset kTilePresets[] = {
    {"tile_128x64_k16", 128, 64, 16, 0, 1, 1, 0, 0},
    {"tile_64x64_k16", 64, 64, 16, 0, 1, 1, 0, 0},
    {"tile_64x64_k32", 64, 64, 32, 0, 1, 1, 0, 0},
    {"tile_64x64_k64", 64, 64, 64, 0, 1, 1, 0, 0},
    {"tile_32x64_k16", 32, 64, 16, 0, 1, 1, 0, 0},
    {"tile_128x64_k32", 128, 64, 32, 0, 1, 1, 0, 0},
    {"tile_64x128_k32", 64, 128, 32, 0, 1, 1, 1, 0},
    {"tile_64x128_k16", 64, 128, 16, 0, 1, 1, 0, 0},
    {"tile_128x128_k16", 128, 128, 16, 0, 1, 1, 0, 0},
    {"tile_128x128_k32", 128, 128, 32, 1, 0, 1, 1, 0},
    {"tile_128x128_k48", 128, 128, 48, 0, 1, 1, 0, 0},
    {"tile_128x128_k16_swap", 128, 128, 16, 0, 1, 1, 1, 0},
    {"tile_128x128_k32_swap", 128, 128, 32, 0, 1, 1, 1, 0},
    {"tile_256x64_k32_wgp", 256, 64, 32, 1, 1, 1, 0, 0},
    {"tile_256x64_k64_wgp", 256, 64, 64, 1, 1, 1, 0, 0},
    {"tile_128x128_k64", 128, 128, 64, 0, 1, 1, 1, 0},
    {"tile_128x64_k64", 128, 64, 64, 0, 1, 1, 0, 0},
    {"tile_32x32_k16", 32, 32, 16, 0, 1, 1, 0, 0},
    {"tile_32x128_k16", 32, 128, 16, 0, 1, 1, 0, 0},
    {"tile_128x32_k16", 128, 32, 16, 0, 1, 1, 0, 0},
    {"tile_64x256_k32", 64, 256, 32, 0, 1, 1, 0, 0},
    {"tile_128x256_k32", 128, 256, 32, 0, 1, 1, 0, 0},
    {"tile_256x128_k32", 256, 128, 32, 0, 1, 1, 0, 0},
    {"tile_persistent_decode", 32, 64, 16, 0, 1, 0, 0, 1},
    {"tile_persistent_128x64_k32", 128, 64, 32, 0, 1, 1, 0, 1},
    {"tile_persistent_256x128_k32", 256, 128, 32, 0, 1, 1, 1, 1},
};

t0mi_tile_spec make_tile(const TilePreset& p) {
  t0mi_tile_spec s;
  memset(&s, 0, sizeof s);
  s.tile_m = p.m;
  s.tile_n = p.n;
  s.tile_k = p.k;
  s.wgp_mode = p.wgp;
  s.double_buffer = p.db;
  s.split_k = 1;
  s.swap_grid = p.swap_grid;
  s.transpose = T0MI_NT;
  s.acc_swap = p.acc_swap;
  s.persistent = p.persistent;
  return s;
}

bool preset_by_name(const char* name, t0mi_tile_spec* out) {
  for (const auto& p : kTilePresets)
    if (!strcmp(p.name, name)) {
      *out = make_tile(p);
      return true;
    }
  return false;
}

t0mi_tile_spec preset(const char* name) {
  t0mi_tile_spec s;
  preset_by_name(name, &s);
  return s;
}

bool has_op(const t0mi_tile_spec& s, uint32_t op) {
  const uint32_t n = s.n_epilogue < T0MI_TILE_MAX_EPILOGUE ? s.n_epilogue : T0MI_TILE_MAX_EPILOGUE;
  for (uint32_t i = 0; i < n; ++i)
    if (s.epilogue[i] == op) return true;
  return false;
}

uint32_t lds_per_buffer(const t0mi_tile_spec& s) { return (s.tile_m + s.tile_n) * s.tile_k * 2u; }

uint32_t acc_swap_region(const t0mi_tile_spec& s) {
  // Every wave keeps all of its row blocks: n_col_tiles x 8 VGPRs x 32 lanes x 4 B each.
  const uint32_t nw = tile_n_waves(s);
  const uint32_t rows_per_wave = nw ? s.tile_m / nw : 0;
  const uint32_t n_row_blocks = rows_per_wave / 16;
  const uint32_t n_col_tiles = s.tile_n / 16;
  return n_row_blocks * (n_col_tiles * 8u) * 32u * 4u * nw;
}

}  // namespace

uint32_t tile_n_waves(const t0mi_tile_spec& s) { return s.waves_per_wg ? s.waves_per_wg : s.tile_m / 32; }
uint32_t tile_wg_size(const t0mi_tile_spec& s) { return tile_n_waves(s) * 32u; }
uint32_t tile_split_k(const t0mi_tile_spec& s) { return s.split_k > 1 ? s.split_k : 1u; }

static uint32_t tile_lds_total(const t0mi_tile_spec& s) {
  const uint32_t per = lds_per_buffer(s);
  const uint32_t gemm_lds = s.triple_buffer ? per * 3 : s.double_buffer ? per * 2 : per;
  const uint32_t base = s.acc_swap ? gemm_lds + acc_swap_region(s) : gemm_lds;
  return s.persistent ? base + 16u : base;
}

std::string tile_name(const t0mi_tile_spec& s) {
  static const char* kOp[] = {"bias", "scale", "relu", "silu", "gelu", "abs", "neg", "clamp"};
  std::string r = "tile_gemm_" + std::to_string(s.tile_m) + "x" + std::to_string(s.tile_n) + "_k" +
                  std::to_string(s.tile_k);
  if (s.double_buffer) r += "_db";
  if (s.split_k > 1) r += "_sk" + std::to_string(s.split_k);
  if (!s.swap_grid) r += "_mg";
  if (s.wgp_mode) r += "_wgp";
  if (s.transpose == T0MI_NN) r += "_nn";
  if (s.acc_swap) r += "_swap";
  if (s.persistent) r += "_persistent";
  const uint32_t n = s.n_epilogue < T0MI_TILE_MAX_EPILOGUE ? s.n_epilogue : T0MI_TILE_MAX_EPILOGUE;
  if (n) {
    r += "_";
    for (uint32_t i = 0; i < n; ++i) {
      if (i) r += "_";
      r += s.epilogue[i] < 8 ? kOp[s.epilogue[i]] : "?";
    }
  }
  // gfx950 extension, absent for every reference spec.
  if (s.out_dtype == T0MI_OUT_BF16) r += "_bf16o";
  return r;
}

bool tile_valid(const t0mi_tile_spec& s, EpiChain* chain, std::string* why) {
  auto fail = [&](const std::string& m) {
    if (why) *why = m;
    return false;
  };
  if (!s.tile_m || !s.tile_n || s.tile_m % 16 || s.tile_n % 16)
    return fail("tile_m and tile_n must be non-zero multiples of 16");
  if (!s.tile_k || s.tile_k % 16) return fail("tile_k must be a non-zero multiple of 16");
  const uint32_t sk = tile_split_k(s);
  if (sk & (sk - 1) || sk > 16) return fail("split_k must be 1, 2, 4, 8 or 16");
  if (s.transpose > T0MI_NN) return fail("bad transpose");
  if (s.wmma_format != 0) return fail("only wmma_format BF16_F32 (0) is on the gfx950 path");
  if (s.out_dtype > T0MI_OUT_BF16) return fail("bad out_dtype");
  if (s.n_epilogue > T0MI_TILE_MAX_EPILOGUE) return fail("more than 8 epilogue ops");
  if (s.waves_per_wg && s.tile_m % s.waves_per_wg) return fail("waves_per_wg must divide tile_m");
  EpiChain c;
  memset(&c, 0, sizeof c);
  for (uint32_t i = 0; i < s.n_epilogue; ++i) {
    if (s.epilogue[i] > T0MI_TEPI_CLAMP) return fail("unknown epilogue op " + std::to_string(s.epilogue[i]));
    c.ops |= s.epilogue[i] << (4 * i);
  }
  c.n = s.n_epilogue;
  if (chain) *chain = c;
  return true;
}

TileArgLayout tile_arg_layout(const t0mi_tile_spec& s) {
  TileArgLayout l;
  memset(&l, 0, sizeof l);
  uint32_t off = s.persistent ? 64u : 44u;
  if (has_op(s, T0MI_TEPI_BIAS_ADD)) {
    off = (off + 7u) & ~7u;
    l.bias = off;
    off += 8;
  }
  if (has_op(s, T0MI_TEPI_SCALE)) {
    l.scale = off;
    off += 4;
  }
  if (has_op(s, T0MI_TEPI_CLAMP)) {
    l.clamp_min = off;
    l.clamp_max = off + 4;
    off += 8;
  }
  l.size = off;
  return l;
}

bool tile_lower(const t0mi_tile_spec& s, t0mi_gemm_config* cfg, std::string* why) {
  if (!tile_valid(s, nullptr, why)) return false;
  const int nn = s.transpose == T0MI_NN;
  const int want_stages = s.triple_buffer ? 3 : 2;
  // The kernel with the spec's tile, or the one covering it (a k48 tile runs
  // as three 16-K steps; NN tiles narrower than 64 columns on the 64-column
  // NN kernel); the result does not depend on the tile.
  uint32_t bk = 0;
  const GemmVariant* pick =
      physical_variant(s.tile_m, s.tile_n, s.tile_k, 0, want_stages, nn, &bk);
  if (!pick) {
    if (why)
      *why = "no gfx950 kernel covers a " + std::to_string(s.tile_m) + "x" + std::to_string(s.tile_n) + " k" +
             std::to_string(s.tile_k) + (nn ? " NN" : " NT") + " tile";
    return false;
  }
  t0mi_gemm_config c;
  memset(&c, 0, sizeof c);
  c.tile_m = pick->bm;
  c.tile_n = pick->bn;
  c.tile_k = bk;
  c.wg_size = 64u * pick->wm * pick->wn;
  c.wave_m = pick->wm;
  c.wave_n = pick->wn;
  c.stages = pick->stages == 2 ? 0 : pick->stages;
  c.use_lds = 1;
  c.double_buffer = 1;
  c.split_k = tile_split_k(s) > 1 ? tile_split_k(s) : 0;
  c.n_col_passes = 1;
  c.swap_grid = s.swap_grid;
  c.wgp_mode = s.wgp_mode;
  c.transpose = s.transpose;
  c.epilogue = T0MI_EPI_STORE_F32;
  c.out_dtype = s.out_dtype;
  std::string w;
  if (!config_feasible(c, &w)) {
    if (why) *why = "lowered config infeasible: " + w;
    return false;
  }
  *cfg = c;
  return true;
}

}  // namespace t0mi

using namespace t0mi;

// ===================================================================== C ABI ==

extern "C" int t0mi_tile_preset(const char* name, t0mi_tile_spec* out) {
  if (!name || !out) return set_error(T0MI_ERR_INVALID, "null argument");
  if (!preset_by_name(name, out)) return set_error(T0MI_ERR_NOT_FOUND, "unknown TileGemm preset '%s'", name);
  return T0MI_OK;
}

extern "C" const char* t0mi_tile_preset_names(void) {
  static const std::string names = [] {
    std::string r;
    for (const auto& p : kTilePresets) {
      if (!r.empty()) r += ",";
      r += p.name;
    }
    return r;
  }();
  return names.c_str();
}

extern "C" int t0mi_tile_name(const t0mi_tile_spec* s, char* buf, size_t len) {
  if (!s) return set_error(T0MI_ERR_INVALID, "null spec");
  const std::string n = tile_name(*s);
  if (buf && len) {
    strncpy(buf, n.c_str(), len - 1);
    buf[len - 1] = 0;
  }
  return (int)n.size();
}

extern "C" uint32_t t0mi_tile_n_waves(const t0mi_tile_spec* s) { return s ? tile_n_waves(*s) : 0; }
extern "C" uint32_t t0mi_tile_wg_size(const t0mi_tile_spec* s) { return s ? tile_wg_size(*s) : 0; }
extern "C" uint32_t t0mi_tile_lds_total(const t0mi_tile_spec* s) { return s ? tile_lds_total(*s) : 0; }
extern "C" uint32_t t0mi_tile_kernarg_size(const t0mi_tile_spec* s) { return s ? tile_arg_layout(*s).size : 0; }

extern "C" int t0mi_tile_auto_select(uint32_t m, uint32_t k, uint32_t n, uint32_t transpose, t0mi_tile_spec* out) {
  if (!out) return set_error(T0MI_ERR_INVALID, "null output");
  if (transpose > T0MI_NN) return set_error(T0MI_ERR_INVALID, "bad transpose");
  const uint32_t min_dim = m < n ? m : n, max_dim = m > n ? m : n;
  const bool k32 = k >= 32 && k % 32 == 0, k64 = k >= 64 && k % 64 == 0;
  const char* pick;
  if (min_dim >= 128 && max_dim >= 4096)
    pick = k64 ? "tile_128x128_k64" : k32 ? "tile_128x128_k32" : "tile_128x128_k16";
  else if (min_dim >= 64 && max_dim >= 2048)
    pick = (m >= 256 && k32) ? "tile_256x64_k32_wgp" : k32 ? "tile_64x64_k32" : "tile_64x64_k16";
  else if (min_dim >= 64)
    pick = k32 ? "tile_64x64_k32" : "tile_64x64_k16";  // the reference keeps its k64 branch disabled
  else if (n >= 256 && k32)
    pick = m >= 128 ? "tile_128x256_k32" : "tile_64x256_k32";
  else if (m >= 256 && n >= 128 && k32)
    pick = "tile_256x128_k32";
  else if (n >= 128 && k32)
    pick = "tile_64x64_k32";
  else if (m >= 128 && n < 32)
    pick = "tile_128x32_k16";
  else if (m < 32 && n >= 128)
    pick = "tile_32x128_k16";
  else if (m < 32 && n < 32)
    pick = "tile_32x32_k16";
  else if (k32)
    pick = "tile_64x64_k32";
  else
    pick = "tile_32x64_k16";
  t0mi_tile_spec s = preset(pick);
  // The reference's 64 KB single-WG LDS guard (an RDNA4 limit) falls back to
  // 64x128 k32; kept so the selected spec, and its name, match.
  if (tile_lds_total(s) > 65536) s = preset("tile_64x128_k32");
  s.transpose = transpose;
  // Automatic split-K stays disabled as in the reference (split_k = 1).
  *out = s;
  return T0MI_OK;
}

static uint32_t sk_shift_of(const t0mi_tile_spec& s) {
  switch (s.split_k) {
    case 2: return 1;
    case 4: return 2;
    case 8: return 3;
    case 16: return 4;
    default: return 0;
  }
}

static void put_u32(uint8_t* p, uint32_t v) {
  for (int i = 0; i < 4; ++i) p[i] = (uint8_t)(v >> (8 * i));
}
static void put_u64(uint8_t* p, uint64_t v) {
  for (int i = 0; i < 8; ++i) p[i] = (uint8_t)(v >> (8 * i));
}

static int tile_ka(uint64_t x, uint64_t wt, uint64_t y, uint32_t k, uint32_t n, uint32_t m, const t0mi_tile_spec* s,
                   bool with_tail, uint64_t counter, uint32_t shift, uint32_t per_wg, uint8_t* out, size_t cap) {
  if (!s) return set_error(T0MI_ERR_INVALID, "null spec");
  const size_t len = (with_tail && s->persistent) ? 64 : 44;
  if (!out || cap < len) return (int)len;
  memset(out, 0, len);
  put_u64(out + 0, x);
  put_u64(out + 8, wt);
  put_u64(out + 16, y);
  put_u32(out + 24, k);
  put_u32(out + 28, n);
  put_u32(out + 32, sk_shift_of(*s));
  put_u32(out + 36, 0);  // y_split_stride: the reference always passes 0
  put_u32(out + 40, m);
  if (len == 64) {
    put_u64(out + 48, counter);
    put_u32(out + 56, shift);
    put_u32(out + 60, per_wg);
  }
  return (int)len;
}

extern "C" int t0mi_tile_build_kernargs(uint64_t x, uint64_t wt, uint64_t y, uint32_t k, uint32_t n,
                                        const t0mi_tile_spec* s, uint8_t* out, size_t cap) {
  return tile_ka(x, wt, y, k, n, 0, s, false, 0, 0, 0, out, cap);
}

extern "C" int t0mi_tile_build_kernargs_m(uint64_t x, uint64_t wt, uint64_t y, uint32_t k, uint32_t n, uint32_t m,
                                          const t0mi_tile_spec* s, uint8_t* out, size_t cap) {
  return tile_ka(x, wt, y, k, n, m, s, true, 0, 0, 0, out, cap);
}

extern "C" int t0mi_tile_build_kernargs_m_with_counter(uint64_t x, uint64_t wt, uint64_t y, uint32_t k, uint32_t n,
                                                       uint32_t m, const t0mi_tile_spec* s, uint64_t counter,
                                                       uint32_t n_tiles_n_shift, uint32_t tiles_per_wg, uint8_t* out,
                                                       size_t cap) {
  return tile_ka(x, wt, y, k, n, m, s, true, counter, n_tiles_n_shift, tiles_per_wg, out, cap);
}

extern "C" int t0mi_tile_append_epilogue_args(const t0mi_tile_spec* s, uint64_t bias, float scale, float clamp_min,
                                              float clamp_max, uint8_t* buf, size_t cap, size_t* len) {
  if (!s || !buf || !len) return set_error(T0MI_ERR_INVALID, "null argument");
  const TileArgLayout l = tile_arg_layout(*s);
  const size_t base = s->persistent ? 64 : 44;
  if (*len != base)
    return set_error(T0MI_ERR_KERNARG, "epilogue arguments follow the %zu-byte GEMM kernarg, got %zu bytes", base,
                     *len);
  if (cap < l.size) return set_error(T0MI_ERR_INVALID, "buffer too small: need %u bytes", l.size);
  memset(buf + base, 0, l.size - base);
  if (l.bias) put_u64(buf + l.bias, bias);
  uint32_t u;
  if (l.scale) {
    memcpy(&u, &scale, 4);
    put_u32(buf + l.scale, u);
  }
  if (l.clamp_min) {
    memcpy(&u, &clamp_min, 4);
    put_u32(buf + l.clamp_min, u);
    memcpy(&u, &clamp_max, 4);
    put_u32(buf + l.clamp_max, u);
  }
  *len = l.size;
  return T0MI_OK;
}

extern "C" int t0mi_tile_compute_grid(const t0mi_tile_spec* s, uint32_t m, uint32_t n, uint32_t grid[3]) {
  if (!s || !grid) return set_error(T0MI_ERR_INVALID, "null argument");
  if (!s->tile_m || !s->tile_n) return set_error(T0MI_ERR_INVALID, "zero tile size");
  const uint32_t wg = tile_wg_size(*s);
  if (s->persistent) {
    grid[0] = wg;
    grid[1] = 1;
    grid[2] = 1;
    return T0MI_OK;
  }
  const uint32_t wn = (n + s->tile_n - 1) / s->tile_n, wm = (m + s->tile_m - 1) / s->tile_m;
  const uint32_t sk = tile_split_k(*s);
  grid[0] = (s->swap_grid ? wn : wm) * wg;
  grid[1] = (s->swap_grid ? wm : wn) * sk;
  grid[2] = 1;
  return T0MI_OK;
}
