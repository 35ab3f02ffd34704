// gemm_inst.hip — instantiates one block of gemm_variants.def for one B layout.
// Compiled eight times by the build (T0MI_PART = 0..3, T0MI_INST_NN = 0/1, with
// T0MI_TABLE_FN naming the table accessor) so the variants build in parallel.
#include "gemm_pingpong.h"
#include "t0mi_ctx.h"

#ifndef T0MI_PART
#error "T0MI_PART must be defined"
#endif
#ifndef T0MI_INST_NN
#error "T0MI_INST_NN must be defined"
#endif

namespace t0mi {

// The 256x256x64 2x4-wave configuration runs the ping-pong kernel (same
// results, bit for bit) whenever its K-granularity precondition holds.
template <int BM, int BN, int BK, int WM, int WN, int S, bool NN>
static void launch_variant(dim3 g, hipStream_t s, const GemmParams& p) {
  if constexpr (BM == 256 && BN == 256 && BK == 64 && WM == 2 && WN == 4 && S == 2) {
    if (pingpong_ok(p)) {
      hipLaunchKernelGGL((gemm_bf16_pingpong_kernel<NN, true>), g, dim3(512), 0, s, p);
      return;
    }
  }
  hipLaunchKernelGGL((gemm_bf16_kernel<BM, BN, BK, WM, WN, S, NN>), g, dim3(WM * WN * 64), 0, s, p);
}

#define T0MI_V(BM, BN, BK, WM, WN, S)                                                                  \
  static void launch_##BM##_##BN##_##BK##_##WM##_##WN##_##S(dim3 g, hipStream_t s, const GemmParams& p) { \
    launch_variant<BM, BN, BK, WM, WN, S, (T0MI_INST_NN != 0)>(g, s, p);                              \
  }
#if T0MI_INST_NN
#define T0MI_V_NT(BM, BN, BK, WM, WN, S)
#else
#define T0MI_V_NT(BM, BN, BK, WM, WN, S) T0MI_V(BM, BN, BK, WM, WN, S)
#endif
#include "gemm_variants.def"
#undef T0MI_V

static const GemmLaunchEntry kTable[] = {
#define T0MI_V(BM, BN, BK, WM, WN, S) \
  {BM, BN, BK, WM, WN, S, T0MI_INST_NN, launch_##BM##_##BN##_##BK##_##WM##_##WN##_##S},
#include "gemm_variants.def"
#undef T0MI_V
#undef T0MI_V_NT
};

const GemmLaunchEntry* T0MI_TABLE_FN(size_t* n) {
  *n = sizeof kTable / sizeof kTable[0];
  return kTable;
}

}  // namespace t0mi
