// epi_chain.h — the fused GEMM epilogue chain, shared by host and device code.
#pragma once
#include <stdint.h>

namespace t0mi {

// Fused epilogue: a chain of up to 8 element-wise ops applied in order to each
// fp32 result before the store (tile_ir EpilogueOp, src/t0/tile_ir.rs:40-58,
// lowered at :3400-3540).  gemm_gen's BiasAddStoreF32 / BiasAddReluStoreF32
// (src/t0/gemm_gen.rs:41-49) are the chains {BIAS} and {BIAS, RELU}.
enum : uint32_t {
  EOP_BIAS = 0,   // v += bias[col]            (bias: [N] f32)
  EOP_SCALE = 1,  // v *= scale
  EOP_RELU = 2,   // v = max(v, 0)
  EOP_SILU = 3,   // v = v * rcp(1 + exp2(-v * log2 e))
  EOP_GELU = 4,   // v = v * rcp(1 + exp2(-1.702 v * log2 e))  (sigmoid form, as lowered)
  EOP_ABS = 5,    // v = |v|
  EOP_NEG = 6,    // v = -v
  EOP_CLAMP = 7,  // v = min(max(v, lo), hi)
};
constexpr int EPI_MAX_OPS = 8;

struct EpiChain {
  uint32_t n;    // ops in the chain (0 = plain store)
  uint32_t ops;  // op i in bits [4i, 4i+4)
  float scale, lo, hi;
};

}  // namespace t0mi
