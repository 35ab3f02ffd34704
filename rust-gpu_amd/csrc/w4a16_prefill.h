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
//   * A arrives in registers (16-byte loads, the same swizzled K-contiguous
//     1 KB LDS blocks the GEMM's DMA fills) and B as packed words: thread t
//     owns one k-octet r and CPT (2 or 4) consecutive columns, i.e. one 8- or
//     16-byte load per tile (coalesced along N);
//   * both are requested S-1 tiles ahead into a ring of S register sets, so
//     S-1 tiles are in flight while one is computed.  At small M a tile's
//     MFMA work is far shorter than the memory latency, and the latency, not
//     the bandwidth, sets the speed; every load is compiler-tracked, so each
//     register set is waited for exactly when it is consumed;
//   * during the MFMAs of tile it, each thread writes tile it+1's A into the
//     other LDS stage and dequantises its CPT words of tile it+1 — (q - z) * s
//     exactly in fp32, rounded once to bf16 (RNE) — into the swizzled
//     K-contiguous [BN][BK] B tile that the NT fragment reads use.
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
  uint32_t kt_per_split;    // K tiles per partition (grid = tiles x partitions)
  uint64_t y_split_stride;  // > 0: partition p stores raw f32 sums at y + p * stride
};

// Packed B of one thread for one K tile: CPT (2 or 4) consecutive columns'
// words for one k-octet, their bf16 scales (two per word) and the qzeros word
// holding their zero points.
template <int CPT>
struct W4Regs {
  uint32_t w[CPT];
  uint32_t s[CPT / 2];
  uint32_t z;
};

template <int BM, int BN, int BK, int WM, int WN, int S, bool ZEROS>
__global__ __launch_bounds__(WM * WN * 64) void w4a16_prefill_kernel(W4PrefillParams p) {
  constexpr int NWAVES = WM * WN, NTHR = NWAVES * 64;
  constexpr int TM = BM / WM, TN = BN / WN, FM = TM / 32, FN = TN / 32;
  constexpr int KC = BK / 8, KS = BK / 16;
  constexpr int A_ELEMS = BM * BK, B_ELEMS = BN * BK, BUF = A_ELEMS + B_ELEMS;
  constexpr int A_BLOCKS = A_ELEMS * 2 / 1024;
  constexpr int APT = A_BLOCKS / NWAVES;  // 16-byte A loads per thread per tile
  constexpr int CPT = BN * KC / NTHR;     // columns (packed words) per thread per K tile
  constexpr int COLQ = BN / CPT;          // CPT-column groups per tile row
  static_assert(TM % 32 == 0 && TN % 32 == 0, "wave tile must be a multiple of 32x32");
  static_assert(BK == 32 || BK == 64, "tile_k 32 or 64");
  static_assert((CPT == 2 || CPT == 4) && NTHR * CPT == BN * KC, "2 or 4 packed words per thread per K tile");
  static_assert(A_BLOCKS % NWAVES == 0, "every thread loads the same number of A chunks");
  static_assert(S >= 2 && S <= 6, "2..6 tiles in the register ring");

  __shared__ __attribute__((aligned(1024))) uint16_t smem[2 * BUF];

  int tm, tn, part;
  tile_coords_of(p.tiles_m, p.tiles_n, p.xcd_remap, tm, tn, part);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int m0 = tm * BM, n0 = tn * BN;
  const int K = (int)p.K;
  // This partition's K tiles: [kt0, kt0 + nk).
  const int nk_all = (K + BK - 1) / BK;
  const int kt0 = part * (int)p.kt_per_split;
  const int nk = min(nk_all - kt0, (int)p.kt_per_split);

  // One tile's registers: this thread's A chunks and packed B words.
  struct TileRegs {
    u32x4 a[APT];
    W4Regs<CPT> b;
  };
  // A chunk j of this thread: LDS block blk = wave + j * NWAVES, slot `lane`,
  // holding row `row`, 16-byte chunk `lc` (swizzled) of the K-contiguous tile.
  int a_row[APT], a_lc[APT];
#pragma unroll
  for (int j = 0; j < APT; ++j) {
    const int q = (wave + j * NWAVES) * 64 + lane;
    const int row = q / KC, pc = q % KC;
    a_lc[j] = pc ^ swz<KC>(row);
    const int gr = m0 + row;
    a_row[j] = gr < (int)p.M ? gr : (int)p.M - 1;
  }

  // This thread's slot in the packed B tile.
  const int br = tid / COLQ;           // k-octet within the tile (= logical 16-byte chunk)
  const int bc = (tid % COLQ) * CPT;   // first of CPT columns within the tile
  // Columns past N and k-octets past K are clamped onto real data: the
  // columns are never stored and the A operand is zero past K, so the loads
  // need no predicate.
  const int gn = min(n0 + bc, (int)p.N - CPT);  // N % 8 == 0
  const int ko_last = K / 8 - 1;
  auto load_b = [&](int k0, W4Regs<CPT>& r) {
    const int ko = min(k0 / 8 + br, ko_last);  // qweight row
    const uint32_t g = (uint32_t)(ko * 8) >> p.group_shift;
    if constexpr (CPT == 4) {
      const u32x4 w = __builtin_nontemporal_load((const u32x4*)(p.w + (size_t)ko * p.N + gn));
      const u32x2 sc = *(const u32x2*)(p.scales + (size_t)g * p.N + gn);
      r.w[0] = w.x, r.w[1] = w.y, r.w[2] = w.z, r.w[3] = w.w;
      r.s[0] = sc.x, r.s[1] = sc.y;
    } else {
      const u32x2 w = __builtin_nontemporal_load((const u32x2*)(p.w + (size_t)ko * p.N + gn));
      r.w[0] = w.x, r.w[1] = w.y;
      r.s[0] = *(const uint32_t*)(p.scales + (size_t)g * p.N + gn);
    }
    if constexpr (ZEROS) r.z = p.zeros[(size_t)g * (p.N / 8) + (uint32_t)gn / 8];
  };
  auto load_tile = [&](int t, TileRegs& r) {
    const int k0 = (kt0 + t) * BK;
#pragma unroll
    for (int j = 0; j < APT; ++j) {
      // Chunks past K read column 0 of the row instead (a global address either
      // way: a select between A and another buffer would make the pointer
      // generic, and flat loads are waited for all together); put_a zeroes them.
      const int gk = k0 + a_lc[j] * 8;
      r.a[j] = *(const u32x4*)(p.a + (size_t)a_row[j] * K + (gk < K ? gk : 0));
    }
    load_b(k0, r.b);
  };
  auto put_a = [&](const TileRegs& r, int t, int stage) {
    uint16_t* As = smem + stage * BUF;
#pragma unroll
    for (int j = 0; j < APT; ++j) {
      // The empty asm pins the zeroing here: without it the compiler moves the
      // select next to the load (the same condition), which then has to wait
      // for the load as soon as it is issued.
      u32x4 v = r.a[j];
      asm volatile("" : "+v"(v));
      if ((kt0 + t) * BK + a_lc[j] * 8 >= K) v = (u32x4){0u, 0u, 0u, 0u};
      *(u32x4*)(As + (wave + j * NWAVES) * 512 + lane * 8) = v;
    }
  };
  // Dequantise column j of r into its 16-byte LDS chunk of stage `stage`.
  // A nibble pair becomes the bf16 pair (128 + q) with one and/or (exact),
  // each half widens to fp32 with one shift or mask, and
  //   fma(128 + q, s, -(128 + z) * s) = (q - z) * s
  // is exact: both products have at most 16 significant bits and the result
  // at most 12.  It is then rounded once to bf16.
  auto put_b = [&](const W4Regs<CPT>& r, int j, int stage) {
    const uint32_t wj = r.w[j];
    const uint32_t sb = r.s[j / 2];
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

  // Ring slot u holds tile it0 + u (it0 a multiple of S): the loop below is
  // unrolled S times so that every slot index is a compile-time constant.
  // Every iteration requests one tile (past the last tile, the last one again,
  // never used): the number of loads in flight is then the same on every path
  // and the compiler waits for each register set exactly, not for all loads.
  TileRegs ring[S];
  if (nk <= 0) return;  // the host sizes partitions so that none is empty (K == 0 never launches)
  // Prologue: tiles 0 .. S-2 requested; tile 0 written to stage 0.
#pragma unroll
  for (int t = 0; t < S - 1; ++t) load_tile(min(t, nk - 1), ring[t]);
  put_a(ring[0], 0, 0);
#pragma unroll
  for (int j = 0; j < CPT; ++j) put_b(ring[0].b, j, 0);
  // FULL: a main-loop iteration, where tile it+1 always exists (no branch).
  auto iteration = [&](auto uc, auto full_c, int it) {
    constexpr int u = decltype(uc)::value;
    constexpr bool FULL = decltype(full_c)::value;
    const int c = it & 1;
    // Publishes stage c (written during iteration it-1 or the prologue) and
    // proves every wave is done reading stage c^1 (iteration it-1).  The
    // scheduling barriers keep each iteration's work inside it: hoisted into
    // an earlier iteration, the dequant of a tile waits for loads that are
    // meant to be still in flight.
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    load_tile(min(it + S - 1, nk - 1), ring[(u + S - 1) % S]);
    __builtin_amdgcn_sched_barrier(0);
    const bool more = FULL || it + 1 < nk;
    const TileRegs& nx = ring[(u + 1) % S];
    if (more) put_a(nx, it + 1, c ^ 1);
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
      // Tile it+1's B: column j during k-step j * KS / CPT, between this
      // k-step's MFMAs.
      if (more) {
#pragma unroll
        for (int j = 0; j < CPT; ++j)
          if (j * KS / CPT == ks) put_b(nx.b, j, c ^ 1);
      }
    }
  };
  int it0 = 0;
  for (; it0 + S < nk; it0 += S)
    static_for<S>([&](auto uc) { iteration(uc, std::true_type{}, it0 + decltype(uc)::value); });
  // The last 1 .. S tiles.
  static_for<S>([&](auto uc) {
    if (it0 + decltype(uc)::value < nk) iteration(uc, std::false_type{}, it0 + decltype(uc)::value);
  });

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
        if (p.y_split_stride) {  // partition plane: raw f32 sums, summed by the reduce pass
          float* yp = (float*)((char*)p.y + (size_t)part * p.y_split_stride);
          *(f32x4*)(yp + (size_t)m * p.N + n) = f32x4{v0, v1, v2, v3};
        } else if (p.out_bf16) {
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
