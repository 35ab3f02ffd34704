// w4a16.hip — INT4-weight / bf16-activation GEMM and the standalone INT4 dequant.
//
// Semantics follow the reference's INT4 definition (src/t0/quant_kernels.rs:1-25,
// 74-100): element 2i of a byte is its low nibble, w = (q - zp) * scale with
// one scale / zero-point per group of `group` consecutive K elements.  The
// reference has no fused W4A16 GEMM (only a standalone dequant kernel whose GPU
// code is defective); this file is the fused gfx950 path.
//
// Weight layout (qweight): u32 [K/8][N]; word (kk, n) holds q[8kk+e][n] in bits
// 4e..4e+3.  One word is exactly the 8 K-values one MFMA lane feeds for one
// column, so the weights cross HBM once, at 4 bits, with 16-byte loads
// (4 adjacent columns per lane).
//
// Dequant inside the K loop, exactly:
//   (0x43004300 | (w >> 4j) & 0x000F000F) is the bf16 pair (128+q_j, 128+q_{j+4}),
//   exact integers.  The MFMA multiplies them with bf16 activations in fp32
//   (exact products), so per group and column
//       P = sum_k a_k * (128 + q_k),   S = sum_k a_k   (S from an MFMA with ones)
//       y += s * (P - (128 + z) * S)                      == sum_k a_k * (q_k - z) * s
//   The activation operand is permuted to the same k order as the nibble pairs.
#include <string.h>

#include "t0mi_ctx.h"
#include "w4a16_decode.h"
#include "w4a16_pingpong.h"
#include "w4a16_prefill.h"

using namespace t0mi;

namespace t0mi {

// Decode kernel: M <= 16 rows per slab.  One workgroup = WAVES waves on one
// 64-column strip; wave v takes k-blocks [kb0 + v*KBW, +KBW) of this grid.y
// partition.  Each lane issues all its 16-byte weight and activation loads up
// front (KBW of each), then runs 4 MFMAs per k-block (one per column word).
// Waves are reduced through LDS in wave order; with gridDim.y > 1 each
// partition writes an f32 plane that t0mi_splitk_reduce sums.
template <int WAVES, int KBW>
__global__ __launch_bounds__(WAVES * 64) void w4a16_decode_kernel(W4Params p) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c = lane & 15, g = lane >> 4;  // column quad, k sub-row (packed row within a k-block)
  const int n0 = blockIdx.x * 64;
  const int ncol = n0 + 4 * c;
  const int kb_tot = (int)(p.K / 32);
  const int kb_part0 = (int)(blockIdx.y * p.kb_per_split);
  int kb_part1 = kb_part0 + (int)p.kb_per_split;
  kb_part1 = kb_part1 < kb_tot ? kb_part1 : kb_tot;
  const int kb0 = kb_part0 + wave * KBW;
  const int kbpg = (int)(p.group / 32);
  const bool col_ok = ncol < (int)p.N;
  const int arow = c;  // activation row fed by this lane (A operand row = lane % 16)
  const bool row_ok = arow < (int)p.M;

  u32x4 wv[KBW], av[KBW];
#pragma unroll
  for (int b = 0; b < KBW; ++b) {
    const int kb = kb0 + b;
    u32x4 w = {0u, 0u, 0u, 0u}, a = {0u, 0u, 0u, 0u};
    if (kb < kb_part1) {
      if (col_ok) w = __builtin_nontemporal_load((const u32x4*)(p.w + (size_t)(kb * 4 + g) * p.N + ncol));
      if (row_ok) a = *(const u32x4*)(p.a + (size_t)arow * p.K + kb * 32 + g * 8);
    }
    wv[b] = w;
    av[b] = a;
  }

  const bf16x8_t ones = __builtin_bit_cast(bf16x8_t, (u32x4){0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u});
  f32x4 acc[4], P[4], S;
#pragma unroll
  for (int j = 0; j < 4; ++j) acc[j] = (f32x4){0.f, 0.f, 0.f, 0.f};

  // Output rows held by this lane: 4*g + r; columns ncol + j.
#pragma unroll
  for (int b = 0; b < KBW; ++b) {
    const int kb = kb0 + b;
    if (kb >= kb_part1) break;
    if (b == 0 || (kb % kbpg) == 0) {
#pragma unroll
      for (int j = 0; j < 4; ++j) P[j] = (f32x4){0.f, 0.f, 0.f, 0.f};
      S = (f32x4){0.f, 0.f, 0.f, 0.f};
    }
    const bf16x8_t A = perm_act(av[b]);
    S = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, ones, S, 0, 0, 0);
    P[0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, nib_pairs(wv[b].x), P[0], 0, 0, 0);
    P[1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, nib_pairs(wv[b].y), P[1], 0, 0, 0);
    P[2] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, nib_pairs(wv[b].z), P[2], 0, 0, 0);
    P[3] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, nib_pairs(wv[b].w), P[3], 0, 0, 0);
    if (((kb + 1) % kbpg) == 0 || kb + 1 == kb_part1 || b + 1 == KBW) {
      // Group (or wave range) ends: y += s * (P - (128 + z) * S).
      // Output column of P[j] for this lane is ncol' = n0 + 4*(lane & 15) + j,
      // the same four columns this lane loaded.
      const int grp = kb / kbpg;
      float s[4], z[4];
      if (col_ok) {
        const u32x2 sv = *(const u32x2*)(p.scales + (size_t)grp * p.N + ncol);
        s[0] = bf16f(sv.x & 0xFFFFu);
        s[1] = bf16f(sv.x >> 16);
        s[2] = bf16f(sv.y & 0xFFFFu);
        s[3] = bf16f(sv.y >> 16);
        if (p.zeros) {
          const uint32_t zw = p.zeros[(size_t)grp * (p.N / 8) + ncol / 8] >> (4 * (ncol & 7));
#pragma unroll
          for (int j = 0; j < 4; ++j) z[j] = 128.0f + (float)((zw >> (4 * j)) & 0xFu);
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j) z[j] = 128.0f + (float)p.zp_const;
        }
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) s[j] = 0.f, z[j] = 0.f;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc[j].x += s[j] * (P[j].x - z[j] * S.x);
        acc[j].y += s[j] * (P[j].y - z[j] * S.y);
        acc[j].z += s[j] * (P[j].z - z[j] * S.z);
        acc[j].w += s[j] * (P[j].w - z[j] * S.w);
      }
    }
  }

  // Cross-wave reduction in wave order.  red[wave][lane][16].
  __shared__ float red[WAVES * 64 * 16];
  float* mine = red + (wave * 64 + lane) * 16;
#pragma unroll
  for (int j = 0; j < 4; ++j) *(f32x4*)(mine + 4 * j) = acc[j];
  __syncthreads();
  // Thread t < 64*16/4: handles lane L = t / 4 and word j = t % 4 (4 rows).
  for (int t = threadIdx.x; t < 64 * 4; t += WAVES * 64) {
    const int L = t >> 2, j = t & 3;
    f32x4 s4 = *(const f32x4*)(red + (0 * 64 + L) * 16 + 4 * j);
    for (int v = 1; v < WAVES; ++v) {
      const f32x4 t4 = *(const f32x4*)(red + (v * 64 + L) * 16 + 4 * j);
      s4.x += t4.x;
      s4.y += t4.y;
      s4.z += t4.z;
      s4.w += t4.w;
    }
    const int col = n0 + 4 * (L & 15) + j;
    const int row0 = 4 * (L >> 4);
    if (col >= (int)p.N) continue;
    const float vals[4] = {s4.x, s4.y, s4.z, s4.w};
    if (gridDim.y > 1) {
      float* yp = (float*)((char*)p.y + (size_t)blockIdx.y * p.y_split_stride);
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (row0 + r < (int)p.M) yp[(size_t)(row0 + r) * p.N + col] = vals[r];
    } else if (p.out_bf16) {
      uint16_t* yp = (uint16_t*)p.y;
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (row0 + r < (int)p.M) yp[(size_t)(row0 + r) * p.N + col] = f32_to_bf16_rne(vals[r]);
    } else {
      float* yp = (float*)p.y;
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (row0 + r < (int)p.M) yp[(size_t)(row0 + r) * p.N + col] = vals[r];
    }
  }
}

// Decode kernel for group sizes of KBPG k-blocks (32 K values each) with
// KBPG | KBW: every wave covers whole groups, so group boundaries are static.
// Same decomposition as w4a16_decode_kernel (one 64-column strip per
// workgroup, waves split the K range, LDS reduction in wave order), but the
// weights, activations, scales and zero points of the wave are all requested
// up front, out-of-range k-blocks are zero-filled instead of branched around,
// and the loop over groups is fully static.
template <int WAVES, int KBW, int KBPG, bool ZEROS>
__global__ __launch_bounds__(WAVES * 64) void w4a16_decode_grouped(W4Params p) {
  static_assert(KBW % KBPG == 0, "whole groups per wave");
  constexpr int NG = KBW / KBPG;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * 64;
  const int ncol = n0 + 4 * c;
  const int kb_tot = (int)(p.K / 32);
  const int kb0 = (int)(blockIdx.y * p.kb_per_split) + wave * KBW;
  const bool col_ok = ncol < (int)p.N;
  const int ncol_c = col_ok ? ncol : 0;
  const bool row_ok = c < (int)p.M;
  const int ngroups = kb_tot / KBPG;

  u32x4 wv[KBW], av[KBW];
#pragma unroll
  for (int b = 0; b < KBW; ++b) {
    const int kb = kb0 + b;
    const bool ok = kb < kb_tot;
    const int kbc = ok ? kb : 0;
    u32x4 w = __builtin_nontemporal_load((const u32x4*)(p.w + (size_t)(kbc * 4 + g) * p.N + ncol_c));
    u32x4 a = *(const u32x4*)(p.a + (size_t)(row_ok ? c : 0) * p.K + kbc * 32 + g * 8);
    wv[b] = (ok && col_ok) ? w : (u32x4){0u, 0u, 0u, 0u};
    av[b] = (ok && row_ok) ? a : (u32x4){0u, 0u, 0u, 0u};
  }
  u32x2 sv[NG];
  uint32_t zv[NG];
#pragma unroll
  for (int q = 0; q < NG; ++q) {
    int grp = kb0 / KBPG + q;
    grp = grp < ngroups ? grp : ngroups - 1;
    sv[q] = *(const u32x2*)(p.scales + (size_t)grp * p.N + ncol_c);
    zv[q] = ZEROS ? p.zeros[(size_t)grp * (p.N / 8) + ncol_c / 8] >> (4 * (ncol_c & 7)) : 0u;
  }

  const bf16x8_t ones = __builtin_bit_cast(bf16x8_t, (u32x4){0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u});
  f32x4 acc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) acc[j] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int q = 0; q < NG; ++q) {
    f32x4 P[4], S = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j) P[j] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < KBPG; ++i) {
      const int b = q * KBPG + i;
      const bf16x8_t A = perm_act(av[b]);
      S = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, ones, S, 0, 0, 0);
      P[0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, nib_pairs(wv[b].x), P[0], 0, 0, 0);
      P[1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, nib_pairs(wv[b].y), P[1], 0, 0, 0);
      P[2] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, nib_pairs(wv[b].z), P[2], 0, 0, 0);
      P[3] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, nib_pairs(wv[b].w), P[3], 0, 0, 0);
    }
    // y += s * (P - (128 + z) * S) for the four columns ncol + j of this lane.
    const float s4[4] = {bf16f(sv[q].x & 0xFFFFu), bf16f(sv[q].x >> 16), bf16f(sv[q].y & 0xFFFFu),
                         bf16f(sv[q].y >> 16)};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float z = 128.0f + (float)(ZEROS ? ((zv[q] >> (4 * j)) & 0xFu) : p.zp_const);
      acc[j].x = fmaf(s4[j], fmaf(-z, S.x, P[j].x), acc[j].x);
      acc[j].y = fmaf(s4[j], fmaf(-z, S.y, P[j].y), acc[j].y);
      acc[j].z = fmaf(s4[j], fmaf(-z, S.z, P[j].z), acc[j].z);
      acc[j].w = fmaf(s4[j], fmaf(-z, S.w, P[j].w), acc[j].w);
    }
  }

  // Cross-wave reduction in wave order, then store (or an f32 partial plane).
  __shared__ float red[WAVES * 64 * 16];
  float* mine = red + (wave * 64 + lane) * 16;
#pragma unroll
  for (int j = 0; j < 4; ++j) *(f32x4*)(mine + 4 * j) = acc[j];
  __syncthreads();
  for (int t = threadIdx.x; t < 64 * 4; t += WAVES * 64) {
    const int L = t >> 2, j = t & 3;
    f32x4 s4 = *(const f32x4*)(red + L * 16 + 4 * j);
    for (int v = 1; v < WAVES; ++v) {
      const f32x4 t4 = *(const f32x4*)(red + (v * 64 + L) * 16 + 4 * j);
      s4.x += t4.x;
      s4.y += t4.y;
      s4.z += t4.z;
      s4.w += t4.w;
    }
    const int col = n0 + 4 * (L & 15) + j;
    const int row0 = 4 * (L >> 4);
    if (col >= (int)p.N) continue;
    const float vals[4] = {s4.x, s4.y, s4.z, s4.w};
    if (gridDim.y > 1) {
      float* yp = (float*)((char*)p.y + (size_t)blockIdx.y * p.y_split_stride);
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (row0 + r < (int)p.M) yp[(size_t)(row0 + r) * p.N + col] = vals[r];
    } else if (p.out_bf16) {
      uint16_t* yp = (uint16_t*)p.y;
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (row0 + r < (int)p.M) yp[(size_t)(row0 + r) * p.N + col] = f32_to_bf16_rne(vals[r]);
    } else {
      float* yp = (float*)p.y;
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (row0 + r < (int)p.M) yp[(size_t)(row0 + r) * p.N + col] = vals[r];
    }
  }
}

// Standalone INT4 dequant to [K][N] (replaces build_dequant_int4_{f32,bf16},
// quant_kernels.rs:53-171, whose addressing is defective): thread (x, y) owns
// k-octet kk = y and columns n .. n+3 (n = 4x): one 16-byte qweight load, its
// four bf16 scales and zero points, and eight output rows written as 8-byte
// (bf16) or 16-byte (f32) row segments, coalesced along N.
// v = (q - z) * s is exact in fp32; round_mode 0 stores it, 1 truncates to
// bf16 (the reference's store_bf16), 2 rounds to nearest even.
__global__ __launch_bounds__(256) void dequant_int4_kernel(const uint32_t* __restrict__ w,
                                                           const uint16_t* __restrict__ scales,
                                                           const uint32_t* __restrict__ zeros, uint32_t zp_const,
                                                           void* __restrict__ out, uint32_t K, uint32_t N,
                                                           uint32_t group, uint32_t round_mode) {
  const uint32_t n = (blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (n >= N) return;  // N % 8 == 0: a thread's four columns are all in range or all out
  for (uint32_t kk = blockIdx.y; kk < K / 8; kk += gridDim.y) {
    const u32x4 wq = __builtin_nontemporal_load((const u32x4*)(w + (size_t)kk * N + n));
    const uint32_t wv[4] = {wq.x, wq.y, wq.z, wq.w};
    uint32_t gk = kk * 8 / group;
    u32x2 sv = *(const u32x2*)(scales + (size_t)gk * N + n);
    uint32_t zw = zeros ? zeros[(size_t)gk * (N / 8) + n / 8] >> (4 * (n & 7)) : 0u;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t k = kk * 8 + e;
      if (group % 8 != 0 && k / group != gk) {  // a group boundary inside the octet
        gk = k / group;
        sv = *(const u32x2*)(scales + (size_t)gk * N + n);
        zw = zeros ? zeros[(size_t)gk * (N / 8) + n / 8] >> (4 * (n & 7)) : 0u;
      }
      float v[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int q = (int)((wv[j] >> (4 * e)) & 0xFu);
        const int z = zeros ? (int)((zw >> (4 * j)) & 0xFu) : (int)zp_const;
        const uint32_t sb = j < 2 ? sv.x : sv.y;
        const float sc = __builtin_bit_cast(float, (j & 1) ? (sb & 0xFFFF0000u) : (sb << 16));
        v[j] = (float)(q - z) * sc;
      }
      const size_t o = (size_t)k * N + n;
      if (round_mode == 0) {
        *(f32x4*)((float*)out + o) = f32x4{v[0], v[1], v[2], v[3]};
      } else {
        uint32_t h[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          h[j] = round_mode == 1 ? __builtin_bit_cast(uint32_t, v[j]) >> 16 : (uint32_t)f32_to_bf16_rne(v[j]);
        *(u32x2*)((uint16_t*)out + o) = u32x2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
      }
    }
  }
}

}  // namespace t0mi

static int hip_fail(hipError_t e, const char* what) {
  return set_error(T0MI_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

// Routes by row count (measured at K = 4096, N = 11008 and 14336):
//  - the decode kernel over 16-row slabs, several per launch sharing one pass
//    over the weights, for groups 32..256 up to kDecodeMaxLaunches launches
//    (group 128: 191 rows; 16 / 32 / 48 / 64 rows in one launch: about 8.4 /
//    10.3 / 12.9 / 15.6 us at N = 11008), for other groups up to kDecodeMaxRows
//    rows (a fused kernel's dequant work per workgroup does not shrink with M);
//  - then the 128x128 fused prefill kernel (w4a16_prefill.h) up to
//    kPingPongRows - 1 (128 rows: 34 us);
//  - then, when K and the group are multiples of 64, the fused ping-pong kernel
//    (w4a16_pingpong.h) below kTwoPassRows (512 rows: 81 us; the other routes
//    98-101 us);
//  - from kTwoPassRows rows on (and for groups the fused kernels do not take)
//    the weights are dequantized once to bf16 and the dense NN GEMM runs: the
//    dequant pass (0.5 B read + 2 B written per weight, at HBM speed) then costs
//    less than dequantizing inside every M tile's K-loop, which is VALU work
//    (N = 14336: 2048 rows 193 us two-pass against 208 us fused; 4096 rows 357
//    against 420);
//    and from kSplitRouteRows + 1 rows on when the fused kernel's tiles overflow
//    one round and the dense GEMM's plan splits the columns.
static constexpr uint32_t kDecodeMaxRows = 80;    // groups the one-slab decode kernels take
// Groups 32..256: up to kDecodeMaxLaunches multi-slab launches (N = 11008: three
// launches of four slabs, 191 rows, 47 us against 47 for the 128x128 kernel; two
// launches, 96..128 rows, 26..31 us against 32..34).
static constexpr uint32_t kDecodeMaxLaunches = 3;
// Slabs per launch of the decode kernel: two for group 256 (whose larger chunks
// need twice the LDS per slab), four for group 128 (the one group whose four-slab
// registers fit without spilling), three otherwise.
static uint32_t decode_max_slabs(uint32_t group) { return group == 256 ? 2 : group == 128 ? 4 : 3; }
static constexpr uint32_t kPingPongRows = 192;
static constexpr uint32_t kTwoPassRows = 1536;
static constexpr uint32_t kSplitRouteRows = 1024;
static constexpr uint32_t kPrefillTwoPassRows = 768;  // groups or K the ping-pong kernel does not take
static constexpr uint32_t kXkMaxPieces = 16;          // pieces per strip the decode kernel's sum takes

static int launch_dequant(t0mi_ctx* ctx, uint64_t qweight, uint64_t scales, uint64_t qzeros, uint32_t zp_const,
                          uint64_t out, uint32_t k, uint32_t n, uint32_t group, uint32_t round_mode) {
  const dim3 grid((n / 4 + 255) / 256, std::min<uint32_t>(k / 8, 65535u));
  hipLaunchKernelGGL(dequant_int4_kernel, grid, dim3(256), 0, ctx->stream, (const uint32_t*)qweight,
                     (const uint16_t*)scales, (const uint32_t*)qzeros, zp_const, (void*)out, k, n, group, round_mode);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? T0MI_OK : hip_fail(e, "dequant launch");
}

// The fused ping-pong kernel (w4a16_pingpong.h): 256x256 tiles, K split so
// that the workgroups cover the CUs when the tiles do not (the split t0mi_gemm
// would use with the same power-of-two split_k); partial planes are summed in
// partition order by the split-K reduce.  Callers check
// w4_pingpong_ok(k, group, ...) for whole 64-K tiles and groups.
static int launch_w4_pingpong(t0mi_ctx* ctx, uint64_t a, uint64_t qweight, uint64_t scales, uint64_t qzeros,
                              uint32_t zp_const, uint64_t y, uint32_t m, uint32_t k, uint32_t n, uint32_t group,
                              bool out_bf16) {
  W4PPParams q;
  memset(&q, 0, sizeof q);
  GemmParams& g = q.g;
  g.a = (const uint16_t*)a;
  g.y = (void*)y;
  g.M = m;
  g.N = n;
  g.K = k;
  g.lda = k;
  g.ldy = n;
  g.tiles_m = (m + 255) / 256;
  g.tiles_n = (n + 255) / 256;
  g.xcd_remap = 1;
  g.out_bf16 = out_bf16;
  // A power of two (as the GEMM configs use) up to 8 and the CUs' share of
  // tiles, halved while a partition of whole 64-K tiles would be empty.
  const uint32_t tiles = g.tiles_m * g.tiles_n, nk_all = k / 64;
  const uint32_t want = std::min(8u, (uint32_t)ctx->cu_count / std::max(1u, tiles));
  uint32_t sk = 1;
  while (sk * 2 <= want && sk * 2 <= nk_all) sk *= 2;
  while (sk > 1 && ((nk_all + sk - 1) / sk) * (sk - 1) >= nk_all) sk /= 2;
  const uint32_t kt = (nk_all + sk - 1) / sk;
  g.split_k = sk;
  g.k_per_split = kt * 64;
  q.w = (const uint32_t*)qweight;
  q.scales = (const uint16_t*)scales;
  q.zeros = (const uint32_t*)qzeros;
  q.zp_const = zp_const;
  q.group = group;
  const size_t plane = (size_t)m * n * 4;
  if (sk > 1) {
    int rc = ensure_workspace(ctx, plane * sk);
    if (rc) return rc;
    g.y = ctx->ws;
    g.y_split_stride = plane;
  }
  const dim3 grid(g.tiles_n, g.tiles_m * sk);
  if (qzeros)
    hipLaunchKernelGGL(w4a16_pingpong_kernel<true>, grid, dim3(512), 0, ctx->stream, q);
  else
    hipLaunchKernelGGL(w4a16_pingpong_kernel<false>, grid, dim3(512), 0, ctx->stream, q);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "w4a16 ping-pong launch");
  if (sk > 1) return launch_splitk_reduce(ctx, (const float*)ctx->ws, (void*)y, nullptr, m, n, n, sk, out_bf16, EpiChain{});
  return T0MI_OK;
}

// One slab (m <= 16), groups 32..256, when N has too few 64-column strips to
// give every CU one (strips * 2 <= CUs): the decode kernel with its K range
// split over workgroups inside one launch (w4a16_decode_v2 with XK).  The
// pieces of a strip, numbered onto the strip's XCD, are combined by the last
// piece to arrive through device-coherent partial slots (xcd_exchange.h).  The
// largest power-of-two piece count up to 8 that keeps strips * pieces <= CUs;
// a piece is nw waves of kbw k-blocks (whole groups).
// Measured at K = 4096, group 128 (per call, against one workgroup per strip):
// N = 1376 (the column-parallel shard of config 4 over 8 GPUs): 8 pieces of
// 4 waves x 4 k-blocks, 5.10 against 7.36 us (graph replay); with the slots
// kept in L2 (not coherent across XCDs) N = 2752: 4 pieces of 8 x 4, 5.55
// against 7.25 us; N = 5504: 2 pieces of 8 x 8, 6.88 against 7.36 us; N = 11008
// (config 4): every split measured slower (9.3-10.8 us against 8.1: the
// exchange's store, ticket and slot reads cost ~2 us under full HBM load), so
// wide N keeps one workgroup per strip.  Returns 1 when the split does not
// apply (the caller takes the strip-per-workgroup route).
static int launch_decode_xk(t0mi_ctx* ctx, W4Params p, uint32_t m, uint32_t k, uint32_t n, uint32_t group,
                            uint64_t y, bool zeros) {
  const uint32_t kbpg = group / 32, kb_tot = k / 32, strips = (n + 63) / 64, unit = std::max(4u, kbpg);
  const uint32_t cus = (uint32_t)ctx->cu_count;
  uint32_t pieces = 8;
  while (pieces > 1 && strips * pieces > cus) pieces /= 2;
  if (pieces == 1 || kb_tot < 2 * unit) return 1;
  // k-blocks of a piece, then 4 waves for up to 16 of them, else 8, each wave
  // a whole number of groups (at most 16 k-blocks: the registers of 16 loads).
  const uint32_t kbr = (kb_tot + pieces - 1) / pieces;
  const uint32_t nw = kbr <= 16 ? 4 : 8;
  const uint32_t kbw = ((kbr + nw - 1) / nw + unit - 1) / unit * unit;
  if (kbw > 16) return 1;
  pieces = (kb_tot + nw * kbw - 1) / (nw * kbw);
  if (pieces < 2 || pieces > kXkMaxPieces) return 1;
  XcdExchange x;
  bool ok = false;
  int rc = xk_prepare(ctx, strips, (size_t)strips * pieces * 1024 * 4, &x, &ok);
  if (rc) return rc;
  if (!ok) return 1;
  p.M = m;
  p.y = (void*)y;
  p.strips = strips;
  p.pieces = pieces;
  p.xk = x;
  const uint32_t grid = (strips + x.nx - 1) / x.nx * x.nx * pieces;
  // CH: chunks of 4 k-blocks (whole groups for group 256).
#define T0MI_XK(NW, KBW, G)                                                                                        \
  if (zeros)                                                                                                      \
    hipLaunchKernelGGL((w4a16_decode_v2<NW, KBW, G / 32, true, KBW / (G / 32 > 4 ? G / 32 : 4), 1, true>),      \
                       dim3(grid), dim3(NW * 64), 0, ctx->stream, p);                                             \
  else                                                                                                            \
    hipLaunchKernelGGL((w4a16_decode_v2<NW, KBW, G / 32, false, KBW / (G / 32 > 4 ? G / 32 : 4), 1, true>),     \
                       dim3(grid), dim3(NW * 64), 0, ctx->stream, p);
#define T0MI_XK_W(NW, G)              \
  if (kbw == 4) {                     \
    T0MI_XK(NW, (G == 256 ? 8 : 4), G) \
  } else if (kbw == 8) {              \
    T0MI_XK(NW, 8, G)                 \
  } else {                            \
    T0MI_XK(NW, 16, G)                \
  }
#define T0MI_XK_G(NW)                   \
  switch (group) {                      \
    case 32: T0MI_XK_W(NW, 32) break;   \
    case 64: T0MI_XK_W(NW, 64) break;   \
    case 128: T0MI_XK_W(NW, 128) break; \
    default: T0MI_XK_W(NW, 256) break;  \
  }
  if (nw == 4) {
    T0MI_XK_G(4)
  } else {
    T0MI_XK_G(8)
  }
#undef T0MI_XK_G
#undef T0MI_XK_W
#undef T0MI_XK
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? T0MI_OK : hip_fail(e, "w4a16 decode launch");
}

extern "C" int t0mi_set_w4a16_workspace_limit(t0mi_ctx* ctx, uint64_t bytes) {
  int rc = check_ctx(ctx);
  if (rc) return rc;
  T0MI_SUBMIT_GUARD(ctx);
  ctx->w4_cvt_limit = bytes;
  return T0MI_OK;
}

extern "C" int t0mi_w4a16_gemm(t0mi_ctx* ctx, uint64_t a, uint64_t qweight, uint64_t scales, uint64_t qzeros,
                               uint32_t zp_const, uint64_t y, uint32_t m, uint32_t k, uint32_t n, uint32_t group,
                               uint32_t out_dtype) {
  int rc = check_ctx(ctx);
  if (rc) return rc;
  T0MI_SUBMIT_GUARD(ctx);
  if (!a || !qweight || !scales || !y) return set_error(T0MI_ERR_INVALID, "null pointer");
  if (group == 0 || group % 32) return set_error(T0MI_ERR_INVALID, "group=%u must be a positive multiple of 32", group);
  if (k % group) return set_error(T0MI_ERR_INVALID, "K=%u must be a multiple of group=%u", k, group);
  if (n % 8) return set_error(T0MI_ERR_INVALID, "N=%u must be a multiple of 8", n);
  if (zp_const > 15) return set_error(T0MI_ERR_INVALID, "zp_const=%u outside 0..15", zp_const);
  if (out_dtype > T0MI_OUT_BF16) return set_error(T0MI_ERR_INVALID, "bad out_dtype");
  // The prefill routes store whole 16-byte vectors (split-K reduce, staged
  // tiles, the dense GEMM of the two-pass route), so Y is 16-byte aligned for
  // every route; qzeros words are read as u32.
  if ((a | qweight | y) & 15) return set_error(T0MI_ERR_INVALID, "A, qweight and Y must be 16-byte aligned");
  if (scales & 7) return set_error(T0MI_ERR_INVALID, "scales must be 8-byte aligned");
  if (qzeros & 3) return set_error(T0MI_ERR_INVALID, "qzeros must be 4-byte aligned");
  if (m == 0 || n == 0) return T0MI_OK;
  if (ctx->null_backend) return T0MI_OK;
  // An empty contraction (K = 0, which every group divides): Y = 0.
  if (k == 0) return fill_async(ctx, (void*)y, 0, (size_t)m * n * (out_dtype == T0MI_OUT_BF16 ? 2 : 4));
  W4Params p;
  memset(&p, 0, sizeof p);
  p.a = (const uint16_t*)a;
  p.w = (const uint32_t*)qweight;
  p.scales = (const uint16_t*)scales;
  p.zeros = (const uint32_t*)qzeros;
  p.K = k;
  p.N = n;
  p.group = group;
  p.zp_const = zp_const;
  p.out_bf16 = out_dtype == T0MI_OUT_BF16;
  p.nib_mask = 0x000F000Fu;
  p.nib_magic = 0x43004300u;
  const bool pow2_group = (group & (group - 1)) == 0;
  const bool v2_group = group == 32 || group == 64 || group == 128 || group == 256;
  const uint32_t decode_max = v2_group ? 16 * decode_max_slabs(group) * kDecodeMaxLaunches : kDecodeMaxRows;
  const bool pingpong = w4_pingpong_ok(k, group, 1, k);
  bool two_pass = m >= (pingpong ? kTwoPassRows : kPrefillTwoPassRows) || (m > decode_max && !pow2_group);
  // The dense GEMM's schedule, planned once (with this GPU's CU count) and run
  // by the dequant-once route below when it is taken.
  AutoPlan plan;
  bool planned = false;
  if (!two_pass && pingpong && m > kSplitRouteRows) {
    // The fused ping-pong kernel's 256 x 256 tiles overflow one round of the
    // GPU: where the dense GEMM's plan splits the columns instead (whole rounds
    // on 256 x 256, the rest on their own tile), dequant-once runs that plan
    // (1280 x 14336 x 4096: 179 us against 208.5 fused).  Below kSplitRouteRows
    // rows the dequant pass costs more than the split saves (768 x 28672:
    // 215 against 204 us).
    const uint64_t tiles = (uint64_t)((m + 255) / 256) * ((n + 255) / 256);
    if (tiles > (uint64_t)ctx->cu_count) {
      planned = auto_plan(m, n, k, T0MI_NN, out_dtype, (uint32_t)ctx->cu_count, &plan);
      if (planned && plan.n1 < n) two_pass = true;
    }
  }
  bool fused_only = false;  // the caller's limit turned the dequant-once route off
  if (two_pass && (uint64_t)k * n * 2 > ctx->w4_cvt_limit) {
    // The caller's limit on the conversion buffer: dequantize inside the K loop instead.
    if (!pingpong && !pow2_group)
      return set_error(T0MI_ERR_INVALID,
                       "%u rows with group %u need the %llu-byte dequantized weight buffer, above the limit "
                       "of %llu bytes (no fused kernel takes this group)",
                       m, group, (unsigned long long)k * n * 2, (unsigned long long)ctx->w4_cvt_limit);
    two_pass = false;
    fused_only = true;
  }
  // The ping-pong kernel takes any group that is a multiple of 64 and any M
  // (rows past M load zeros); below kPingPongRows it runs only for groups the
  // 128x128 fused kernel cannot index (not a power of two) once the limit has
  // ruled out dequant-once.
  if (pingpong && !two_pass && (m >= kPingPongRows || (fused_only && !pow2_group && m > decode_max)))
    return launch_w4_pingpong(ctx, a, qweight, scales, qzeros, zp_const, y, m, k, n, group, p.out_bf16);
  if (two_pass) {
    // W -> bf16 [K][N] (RNE of the exact (q - z) * s: the value the fused
    // kernels round to as well) in the library's conversion buffer, then the
    // NN GEMM with the cost model's config for this shape.
    rc = ensure_cvt_buffer(ctx, (size_t)k * n * 2);
    if (rc) return rc;
    rc = launch_dequant(ctx, qweight, scales, qzeros, zp_const, (uint64_t)ctx->cvt, k, n, group, 2);
    if (rc) return rc;
    if (planned) return run_gemm_planned(ctx, plan, T0MI_NN, a, (uint64_t)ctx->cvt, y, m, n, k, out_dtype);
    return run_gemm_auto(ctx, T0MI_NN, a, (uint64_t)ctx->cvt, y, m, n, k, out_dtype);
  }
  if (m > decode_max) {
    // The 128x128 fused kernel indexes scales and zero points by k >> log2(group).
    if (!pow2_group)
      return set_error(T0MI_ERR_INVALID, "internal: %u rows with group %u reached the power-of-two fused kernel", m,
                       group);
    // Many rows: dequant fused into the MFMA K-loop, weights read once per tile column.
    W4PrefillParams q;
    memset(&q, 0, sizeof q);
    q.a = (const uint16_t*)a;
    q.w = (const uint32_t*)qweight;
    q.scales = (const uint16_t*)scales;
    q.zeros = (const uint32_t*)qzeros;
    q.y = (void*)y;
    q.M = m;
    q.N = n;
    q.K = k;
    q.group_shift = (uint32_t)__builtin_ctz(group);
    q.zp_const = zp_const;
    q.out_bf16 = p.out_bf16;
    q.xcd_remap = 1;
    // 128x128 tiles, 8 waves (two per SIMD, so that one wave's dequant runs
    // beside the other's MFMAs), 4 tiles in flight.
    // With fewer tiles than CUs, K is split so that every CU dequantizes a
    // share of the weights; the partitions' f32 planes are then summed in
    // partition order (deterministic) by the split-K reduce.
    q.tiles_m = (m + 127) / 128;
    q.tiles_n = (n + 127) / 128;
    const uint32_t tiles = q.tiles_m * q.tiles_n, nk_all = (k + 63) / 64;
    uint32_t sk = std::max(1u, std::min(4u, (uint32_t)ctx->cu_count / std::max(1u, tiles)));
    sk = std::min(sk, nk_all);
    q.kt_per_split = (nk_all + sk - 1) / sk;
    sk = (nk_all + q.kt_per_split - 1) / q.kt_per_split;  // no empty partition
    const size_t plane = (size_t)m * n * 4;
    if (sk > 1) {
      rc = ensure_workspace(ctx, plane * sk);
      if (rc) return rc;
      q.y = ctx->ws;
      q.y_split_stride = plane;
    }
    const dim3 grid(q.tiles_n, q.tiles_m * sk);
    if (qzeros)
      hipLaunchKernelGGL((w4a16_prefill_kernel<128, 128, 64, 2, 4, 4, true>), grid, dim3(512), 0, ctx->stream, q);
    else
      hipLaunchKernelGGL((w4a16_prefill_kernel<128, 128, 64, 2, 4, 4, false>), grid, dim3(512), 0, ctx->stream, q);
    if (sk > 1) {
      hipError_t le = hipGetLastError();
      if (le != hipSuccess) return hip_fail(le, "w4a16 prefill launch");
      return launch_splitk_reduce(ctx, (const float*)ctx->ws, (void*)y, nullptr, m, n, n, sk, p.out_bf16, EpiChain{});
    }
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? T0MI_OK : hip_fail(e, "w4a16 prefill launch");
  }
  // Decode: 64-column strips; groups of 32..256 K run the v2 kernel (8-wave
  // workgroups of 16 k-blocks per wave, issued and computed in chunks of one
  // group or 4 blocks), other groups the generic kernel.
  const bool v2 = group == 32 || group == 64 || group == 128 || group == 256;
  if (v2 && m <= 16) {
    rc = launch_decode_xk(ctx, p, m, k, n, group, y, qzeros != 0);
    if (rc <= 0) return rc;  // launched, or failed; 1: the exchange is off, take the planes route
  }
  constexpr int KBW2 = 16;
  constexpr int WAVES = 8, KBW = 16;  // generic kernel
  const uint32_t kb_tot = k / 32;
  uint32_t nw2 = 8;
  if (v2) {
    const uint32_t waves_needed = (kb_tot + KBW2 - 1) / KBW2;
    nw2 = waves_needed <= 4 ? 4 : 8;
  }
  const uint32_t per_part = v2 ? nw2 * KBW2 : WAVES * KBW;
  const uint32_t ky = (kb_tot + per_part - 1) / per_part;
  p.kb_per_split = per_part;
  const uint32_t strips = (n + 63) / 64;
  // Row slabs of 16: the v2 kernel takes up to decode_max_slabs(group) slabs per
  // launch (one pass over the weights feeds them all), spread evenly over the
  // fewest launches (5 slabs as 3 + 2, not 4 + 1); the other kernels one.
  const uint32_t slabs = (m + 15) / 16;
  const uint32_t launches = v2 ? (slabs + decode_max_slabs(group) - 1) / decode_max_slabs(group) : slabs;
  for (uint32_t r0 = 0, done = 0, l = 0, rs = 1; r0 < m; r0 += 16 * rs, done += rs, ++l) {
    rs = (slabs - done + (launches - l) - 1) / (launches - l);
    const uint32_t mr = std::min(16u * rs, m - r0);
    p.a = (const uint16_t*)a + (size_t)r0 * k;
    p.M = mr;
    const size_t ob = out_dtype == T0MI_OUT_BF16 ? 2 : 4;
    if (ky > 1) {
      const size_t plane = (size_t)mr * n * 4;
      rc = ensure_workspace(ctx, plane * ky);
      if (rc) return rc;
      p.y = ctx->ws;
      p.y_split_stride = plane;
    } else {
      p.y = (char*)y + (size_t)r0 * n * ob;
    }
    const bool z = qzeros != 0;
    if (v2) {
      const dim3 grid(strips, ky), block(nw2 * 64);
#define T0MI_W4_V2_RS(NW, G, RS)                                                                               \
  if (z)                                                                                                       \
    hipLaunchKernelGGL((w4a16_decode_v2<NW, KBW2, G / 32, true, G <= 128 ? 4 : 2, RS>), grid, block, 0,        \
                       ctx->stream, p);                                                                        \
  else                                                                                                         \
    hipLaunchKernelGGL((w4a16_decode_v2<NW, KBW2, G / 32, false, G <= 128 ? 4 : 2, RS>), grid, block, 0,       \
                       ctx->stream, p);
#define T0MI_W4_V2(NW, G)                                                                                      \
  switch (rs) {                                                                                                \
    case 4: T0MI_W4_V2_RS(NW, G, (G == 128 ? 4 : G == 256 ? 2 : 3)) break; /* 4 only for group 128 */         \
    case 3: T0MI_W4_V2_RS(NW, G, (G == 256 ? 2 : 3)) break; /* never 3 for group 256 */                        \
    case 2: T0MI_W4_V2_RS(NW, G, 2) break;                                                                     \
    default: T0MI_W4_V2_RS(NW, G, 1) break;                                                                    \
  }
      // The switch below holds the instantiated slab counts (four only for
      // group 128, two for group 256): a launch of more slabs than the group's
      // kernel takes would leave rows unwritten.
      if (rs > decode_max_slabs(group))
        return set_error(T0MI_ERR_INVALID, "internal: %u row slabs per launch for group %u (at most %u)", rs, group,
                         decode_max_slabs(group));
#define T0MI_W4_V2_G(NW)                                                                                       \
  switch (group) {                                                                                             \
    case 32: T0MI_W4_V2(NW, 32) break;                                                                         \
    case 64: T0MI_W4_V2(NW, 64) break;                                                                         \
    case 128: T0MI_W4_V2(NW, 128) break;                                                                       \
    default: T0MI_W4_V2(NW, 256) break;                                                                        \
  }
      if (nw2 == 4) {
        T0MI_W4_V2_G(4)
      } else {
        T0MI_W4_V2_G(8)
      }
#undef T0MI_W4_V2_G
#undef T0MI_W4_V2
#undef T0MI_W4_V2_RS
    } else {
      const dim3 grid(strips, ky), block(WAVES * 64);
      if (group == 512) {
        if (z)
          hipLaunchKernelGGL((w4a16_decode_grouped<WAVES, KBW, 16, true>), grid, block, 0, ctx->stream, p);
        else
          hipLaunchKernelGGL((w4a16_decode_grouped<WAVES, KBW, 16, false>), grid, block, 0, ctx->stream, p);
      } else {  // groups spanning several waves' K ranges
        hipLaunchKernelGGL((w4a16_decode_kernel<WAVES, KBW>), grid, block, 0, ctx->stream, p);
      }
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, "w4a16 launch");
    if (ky > 1) {
      rc = launch_splitk_reduce(ctx, (const float*)ctx->ws, (char*)y + (size_t)r0 * n * ob, nullptr, mr, n, n, ky,
                                p.out_bf16, EpiChain{});
      if (rc) return rc;
    }
  }
  return T0MI_OK;
}

extern "C" int t0mi_dequant_int4(t0mi_ctx* ctx, uint64_t qweight, uint64_t scales, uint64_t qzeros, uint32_t zp_const,
                                 uint64_t out, uint32_t k, uint32_t n, uint32_t group, uint32_t round_mode) {
  int rc = check_ctx(ctx);
  if (rc) return rc;
  T0MI_SUBMIT_GUARD(ctx);
  if (!qweight || !scales || !out) return set_error(T0MI_ERR_INVALID, "null pointer");
  if (group == 0 || k % group || k % 8) return set_error(T0MI_ERR_INVALID, "K=%u must be a multiple of group=%u and 8", k, group);
  if (n % 8) return set_error(T0MI_ERR_INVALID, "N=%u must be a multiple of 8", n);
  if (round_mode > 2) return set_error(T0MI_ERR_INVALID, "round_mode=%u (0 f32, 1 bf16 trunc, 2 bf16 rne)", round_mode);
  if (zp_const > 15) return set_error(T0MI_ERR_INVALID, "zp_const=%u outside 0..15", zp_const);
  if (ctx->null_backend || k == 0 || n == 0) return T0MI_OK;
  if ((qweight & 15) || (scales & 7) || (out & (round_mode == 0 ? 15 : 7)))
    return set_error(T0MI_ERR_INVALID, "qweight and an f32 out must be 16-byte aligned, scales and a bf16 out 8-byte");
  return launch_dequant(ctx, qweight, scales, qzeros, zp_const, out, k, n, group, round_mode);
}
