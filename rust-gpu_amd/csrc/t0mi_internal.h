// t0mi_internal.h — shared declarations of the libt0mi implementation files.
#pragma once
#include <stdint.h>
#include <stddef.h>
#include <string>
#include <vector>

#include "../../include/t0mi.h"

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

// Cost-model candidates for (m, n, k), best first: configs whose kernels are
// prebuilt, with split-K options.  Used by auto_select and the tuner.
std::vector<t0mi_gemm_config> rank_candidates(uint32_t m, uint32_t n, uint32_t k, uint32_t transpose,
                                              uint32_t out_dtype, std::vector<double>* est_us);

}  // namespace t0mi
