// t0mi_internal.h — shared declarations of the libt0mi implementation files.
#pragma once
#include <stdint.h>
#include <stddef.h>
#include <string>
#include <vector>

#include "../../include/t0mi.h"
#include "epi_chain.h"

namespace t0mi {

// Thread-local error string behind t0mi_last_error().
int set_error(int code, const char* fmt, ...);

// Wave layout actually used for a config (explicit or derived).
bool wave_layout(const t0mi_gemm_config& c, uint32_t* wm, uint32_t* wn);
std::string config_name(const t0mi_gemm_config& c);
bool config_feasible(const t0mi_gemm_config& c, std::string* why);
uint32_t split_k_of(const t0mi_gemm_config& c);

// Prebuilt gfx950 GEMM variants (template instantiations).
struct GemmVariant {
  int bm, bn, bk, wm, wn, stages, nn;
};
// LDS pipeline stages of a config (0 means the default, 2).
uint32_t stages_of(const t0mi_gemm_config& c);
// All prebuilt variants (both layouts).
const std::vector<GemmVariant>& gemm_variants();
bool has_variant(const t0mi_gemm_config& c);
// The prebuilt kernel that covers a logical tile: rows and columns rounded up
// to 32 (NN columns to at least 64), a K step of 64, 32 or 16 dividing tile_k;
// the matching variant with the given stage count and workgroup size if there
// is one.  *bk_out = the K step.  Null if none covers it.
const GemmVariant* physical_variant(uint32_t tile_m, uint32_t tile_n, uint32_t tile_k, uint32_t wg_size,
                                    uint32_t stages, int nn, uint32_t* bk_out);
// The config whose prebuilt kernel runs `c`: `c` itself when it is feasible
// on gfx950 and prebuilt, else the covering variant (reference shapes such as
// the wave32 tile_16x64_k16 preset).  False with the reason if none.
bool config_physical(const t0mi_gemm_config& c, t0mi_gemm_config* phys, std::string* why);

// Cost-model candidates for (m, n, k), best first: configs whose kernels are
// prebuilt, with split-K options.  Used by auto_select and the tuner.
std::vector<t0mi_gemm_config> rank_candidates(uint32_t m, uint32_t n, uint32_t k, uint32_t transpose,
                                              uint32_t out_dtype, std::vector<double>* est_us);
// Column split of an auto-scheduled GEMM whose head candidate (unsplit K) fills
// some whole rounds of the GPU's workgroup slots and then part of one more: the
// columns [0, *n_main) of the whole rounds run on `head`, the columns
// [*n_main, n) as a GEMM of their own on *tail (the ranking's head for that
// shape, split-K included).  A partly filled last round of large tiles takes
// nearly a full round's time on a few CUs; the tail's own tile and split spread
// those columns over the GPU.  True only when the cost model expects the pair
// of launches to be faster than the single one.  `cus`: the GPU's compute
// units (the workgroup slots of a round).
bool plan_column_split(const t0mi_gemm_config& head, uint32_t m, uint32_t n, uint32_t k, uint32_t transpose,
                       uint32_t out_dtype, uint32_t* n_main, t0mi_gemm_config* tail, uint32_t cus = 256);

// ---- tile_ir surface (t0mi_tile.cpp) ----
// Byte offsets of the epilogue arguments in a TileGemm kernarg (0 = absent)
// and the total size the lowered kernel declares.
struct TileArgLayout {
  uint32_t bias, scale, clamp_min, clamp_max, size;
};
TileArgLayout tile_arg_layout(const t0mi_tile_spec& s);
// Checks a spec; fills the epilogue chain it encodes.
bool tile_valid(const t0mi_tile_spec& s, EpiChain* chain, std::string* why);
// The GemmConfig of the prebuilt gfx950 kernel that implements a spec
// (same tile_m x tile_n x tile_k and layout), or false with the reason.
bool tile_lower(const t0mi_tile_spec& s, t0mi_gemm_config* cfg, std::string* why);
std::string tile_name(const t0mi_tile_spec& s);
uint32_t tile_n_waves(const t0mi_tile_spec& s);
uint32_t tile_wg_size(const t0mi_tile_spec& s);
uint32_t tile_split_k(const t0mi_tile_spec& s);

}  // namespace t0mi
