// w4a16_prefill.h — gfx950 W4A16 GEMM for many rows (prefill): int4 dequant fused
// into the MFMA K-loop of the bf16 GEMM.
//
// Y[M,N] = A[M,K] . W,  W[k][n] = (q[k][n] - z[k/g][n]) * s[k/g][n]
//   A       bf16 [M][K] (row-major)
//   qweight u32  [K/8][N]: nibble e of word (k/8, n) is q[8(k/8)+e][n] (the
//           reference's low-nibble-first order, src/t0/quant_kernels.rs:3-10)
//   scales  bf16 [K/g][N]; zeros u32 [K/g][N/8] (nibble e = column 8j+e) or a constant.
//
// Weights cross HBM once, at 4 bits.  Per K tile:
//   * A goes global -> LDS by DMA exactly as in gemm_bf16_kernel (swizzled
//     K-contiguous rows);
//   * B arrives one tile ahead as packed words in registers: thread t owns one
//     k-octet r and four consecutive columns, i.e. one 16-byte load per tile
//     (a wave reads one 1 KB row of qweight: coalesced along N);
//   * during the MFMAs of tile it, each thread dequantises its four words of
//     tile it+1 — (q - z) * s exactly in fp32, rounded once to bf16 (RNE) —
//     and writes them as the swizzled K-contiguous [BN][BK] LDS tile that the
//     NT fragment reads use.
// Prefill takes power-of-two group sizes (group index = k >> log2 g).
// The bf16 rounding of the dequantised weight is the only difference from an
// exact-dequant GEMM; it is the same value t0mi_dequant_int4 produces with
// round_mode 2.
#pragma once
#include "gemm_bf16_kernel.h"

namespace t0mi {

struct W4PrefillParams {
  const uint16_t* a;       // [M, K] bf16
  const uint32_t* w;       // [K/8, N]
  const uint16_t* scales;  // [K/g, N] bf16
  const uint32_t* zeros;   // [K/g, N/8] or null (zp_const)
  void* y;                 // [M, N] f32 or bf16
  uint32_t M, N, K, group_shift, zp_const, out_bf16;  // group = 1 << group_shift
  uint32_t tiles_m, tiles_n, xcd_remap;
};

// Packed B of one thread for one K tile: four columns' words plus their scales
// and zero points.
struct W4Regs {
  u32x4 w;      // words of columns n..n+3 for k-octet r
  u32x2 s;      // bf16 scales of columns n..n+3
  uint32_t z;   // qzeros word holding the four columns' zero points
};

template <int BM, int BN, int BK, int WM, int WN, bool ZEROS>
__global__ __launch_bounds__(WM * WN * 64) void w4a16_prefill_kernel(W4PrefillParams p) {
  constexpr int NWAVES = WM * WN, NTHR = NWAVES * 64;
  constexpr int TM = BM / WM, TN = BN / WN, FM = TM / 32, FN = TN / 32;
  constexpr int KC = BK / 8, KS = BK / 16;
  constexpr int A_ELEMS = BM * BK, B_ELEMS = BN * BK, BUF = A_ELEMS + B_ELEMS;
  constexpr int A_BLOCKS = A_ELEMS * 2 / 1024;
  constexpr int COLQ = BN / 4;  // 4-column groups per tile row
  static_assert(TM % 32 == 0 && TN % 32 == 0, "wave tile must be a multiple of 32x32");
  static_assert(BK == 32 || BK == 64, "tile_k 32 or 64");
  static_assert(NTHR == COLQ * KC, "one 16-byte word group per thread per K tile");
  static_assert(KS >= 2 && KS <= 4, "the four words of a thread are spread over the k-steps");

  __shared__ __attribute__((aligned(1024))) uint16_t smem[2 * BUF];

  int tm, tn, part;
  tile_coords_of(p.tiles_m, p.tiles_n, p.xcd_remap, tm, tn, part);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int m0 = tm * BM, n0 = tn * BN;
  const int K = (int)p.K;
  const int nk = (K + BK - 1) / BK;

  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
  const uint32_t smem_base = lds_addr(smem);
  auto load_a = [&](int k0, int stage) {
    const uint32_t a_lds = smem_base + (uint32_t)(stage * BUF * 2);
#pragma unroll
    for (int j = 0; j < (A_BLOCKS + NWAVES - 1) / NWAVES; ++j) {
      const int blk = wave_s + j * NWAVES;
      if (A_BLOCKS % NWAVES != 0 && blk >= A_BLOCKS) break;
      const int q = blk * 64 + lane;
      const int row = q / KC, pc = q % KC;
      const int lc = pc ^ swz<KC>(row);
      int gr = m0 + row;
      gr = gr < (int)p.M ? gr : (int)p.M - 1;
      const int gk = k0 + lc * 8;
      const void* src = gk < K ? (const void*)(p.a + (size_t)gr * K + gk) : (const void*)g_zero16;
      lds_dma16(src, a_lds + blk * 1024);
    }
  };

  // This thread's slot in the packed B tile.
  const int br = tid / COLQ;           // k-octet within the tile (= logical 16-byte chunk)
  const int bc = (tid % COLQ) * 4;     // first of four columns within the tile
  // Columns past N and k-octets past K are clamped onto real data: the
  // columns are never stored and the A operand is zero past K, so the loads
  // need no predicate.
  const int gn = min(n0 + bc, (int)p.N - 4);  // N % 8 == 0
  const int ko_last = K / 8 - 1;
  auto load_b = [&](int k0, W4Regs& r) {
    const int ko = min(k0 / 8 + br, ko_last);  // qweight row
    r.w = *(const u32x4*)(p.w + (size_t)ko * p.N + gn);
    const uint32_t g = (uint32_t)(ko * 8) >> p.group_shift;
    r.s = *(const u32x2*)(p.scales + (size_t)g * p.N + gn);
    // Used only when the tile is dequantised, so the load stays in flight
    // across the MFMAs of the current tile.
    if constexpr (ZEROS) r.z = p.zeros[(size_t)g * (p.N / 8) + (uint32_t)gn / 8];
  };
  // Dequantise column j of r into its 16-byte LDS chunk of stage `stage`.
  // A nibble pair becomes the bf16 pair (128 + q) with one and/or (exact),
  // each half widens to fp32 with one shift or mask, and
  //   fma(128 + q, s, -(128 + z) * s) = (q - z) * s
  // is exact: both products have at most 16 significant bits and the result
  // at most 12.  It is then rounded once to bf16.
  auto put_b = [&](const W4Regs& r, int j, int stage) {
    const uint32_t wj = j == 0 ? r.w.x : j == 1 ? r.w.y : j == 2 ? r.w.z : r.w.w;
    const uint32_t sb = j < 2 ? r.s.x : r.s.y;
    const float s = __builtin_bit_cast(float, (j & 1) ? (sb & 0xFFFF0000u) : (sb << 16));
    const float zb = (float)((ZEROS ? (r.z >> (4 * ((gn & 7) + j))) & 0xFu : p.zp_const) + 128u);
    const float c = -zb * s;
    float v[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      // low half: q_e, high half: q_{e+4}
      const uint32_t pr = ((wj >> (4 * e)) & 0x000F000Fu) | 0x43004300u;
      v[e] = __builtin_fmaf(__builtin_bit_cast(float, pr << 16), s, c);
      v[e + 4] = __builtin_fmaf(__builtin_bit_cast(float, pr & 0xFFFF0000u), s, c);
    }
    u32x4 o;
    o.x = pack_bf16x2(v[0], v[1]);
    o.y = pack_bf16x2(v[2], v[3]);
    o.z = pack_bf16x2(v[4], v[5]);
    o.w = pack_bf16x2(v[6], v[7]);
    const int n = bc + j;
    uint16_t* Bs = smem + stage * BUF + A_ELEMS;
    *(u32x4*)(Bs + n * BK + ((br ^ swz<KC>(n)) * 8)) = o;
  };

  // Fragment reads: both operands K-contiguous (the NT path of gemm_bf16_kernel).
  const int lrow = lane & 31, lhalf = lane >> 5;
  int a_off[KS], b_off[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const int c = ks * 2 + lhalf;
    a_off[ks] = (wm * TM + lrow) * BK + ((c ^ swz<KC>(lrow)) * 8);
    b_off[ks] = (wn * TN + lrow) * BK + ((c ^ swz<KC>(lrow)) * 8);
  }
  auto read_frags = [&](const uint16_t* As, int ks, bf16x8* xa, bf16x8* xb) {
    const uint16_t* Bs = As + A_ELEMS;
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) xa[fm] = *(const bf16x8*)(As + a_off[ks] + fm * 32 * BK);
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) xb[fn] = *(const bf16x8*)(Bs + b_off[ks] + fn * 32 * BK);
  };

  f32x16 acc[FN][FM];
#pragma unroll
  for (int fn = 0; fn < FN; ++fn)
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[fn][fm][e] = 0.0f;

  // Prologue: tile 0 in stage 0 (A by DMA, B dequantised from registers), the
  // packed words of tile 1 requested.
  W4Regs cur, nxt;
  if (nk > 0) {
    load_a(0, 0);
    load_b(0, cur);
    wait_vmcnt<0>();
#pragma unroll
    for (int j = 0; j < 4; ++j) put_b(cur, j, 0);
    if (nk > 1) load_b(BK, cur);
  }
  for (int it = 0; it < nk; ++it) {
    const int c = it & 1;
    // Tile it's A DMA and tile it+1's packed words have landed; the barrier
    // publishes tile it (every wave's DMA and dequant writes) and frees stage
    // c^1, computed in iteration it-1.
    wait_vmcnt<0>();
    __syncthreads();
    const bool more = it + 1 < nk;
    if (more) load_a((it + 1) * BK, c ^ 1);
    if (it + 2 < nk) load_b((it + 2) * BK, nxt);
    const uint16_t* As = smem + c * BUF;
    bf16x8 xa[2][FM], xb[2][FN];
    read_frags(As, 0, xa[0], xb[0]);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int cc = ks & 1;
      if (ks + 1 < KS) read_frags(As, ks + 1, xa[cc ^ 1], xb[cc ^ 1]);
#pragma unroll
      for (int fn = 0; fn < FN; ++fn)
#pragma unroll
        for (int fm = 0; fm < FM; ++fm)
          acc[fn][fm] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xb[cc][fn], xa[cc][fm], acc[fn][fm], 0, 0, 0);
      // Tile it+1's B: 4 / KS columns per k-step, between this k-step's MFMAs.
      if (more) {
#pragma unroll
        for (int j = ks * (4 / KS); j < (ks + 1) * (4 / KS); ++j) put_b(cur, j, c ^ 1);
      }
    }
    cur = nxt;
  }

  // Epilogue (as gemm_bf16_kernel): four consecutive columns per (lane, g).
#pragma unroll
  for (int fm = 0; fm < FM; ++fm) {
    const int m = m0 + wm * TM + fm * 32 + lrow;
    if (m >= (int)p.M) continue;
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int n = n0 + wn * TN + fn * 32 + g * 8 + lhalf * 4;
        if (n >= (int)p.N) continue;
        const float v0 = acc[fn][fm][g * 4 + 0], v1 = acc[fn][fm][g * 4 + 1];
        const float v2 = acc[fn][fm][g * 4 + 2], v3 = acc[fn][fm][g * 4 + 3];
        if (p.out_bf16) {
          u32x2 o;
          o.x = (uint32_t)f32_to_bf16_rne(v0) | ((uint32_t)f32_to_bf16_rne(v1) << 16);
          o.y = (uint32_t)f32_to_bf16_rne(v2) | ((uint32_t)f32_to_bf16_rne(v3) << 16);
          *(u32x2*)((uint16_t*)p.y + (size_t)m * p.N + n) = o;
        } else {
          *(f32x4*)((float*)p.y + (size_t)m * p.N + n) = f32x4{v0, v1, v2, v3};
        }
      }
    }
  }
}

}  // namespace t0mi
