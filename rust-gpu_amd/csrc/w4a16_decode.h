// w4a16_decode.h — gfx950 W4A16 decode GEMM (M <= 16 rows per launch slab).
//
// Y[M,N] = A[M,K] . W[K,N] with W stored as INT4 nibbles (u32 [K/8][N]; word
// (kk, n) holds q[8kk+e][n] in bits 4e..4e+3, the reference's low-nibble-first
// order, src/t0/quant_kernels.rs:3-10), one bf16 scale per `group` K values and
// column, and a zero point per group and column (packed u32 [K/g][N/8]) or a
// constant.  w = (q - z) * s exactly as the reference defines it
// (quant_kernels.rs:24, 95-100); the reference itself has no fused kernel.
//
// Exact dequant inside the MFMA: (0x43004300 | (w >> 4j) & 0x000F000F) is the
// bf16 pair (128 + q_j, 128 + q_{j+4}), exact integers, so per group and column
//     P = sum_k a_k (128 + q_k),   S = sum_k a_k   (an MFMA against ones)
//     y += s * (P - (128 + z) * S)                  == sum_k a_k (q_k - z) s
// with the activation operand permuted into the same k order as the pairs.
//
// Memory plan (HBM-bound: 0.5 B per weight): a workgroup owns a 64-column
// strip; each of its NW waves owns KBW consecutive 32-K blocks, taken in CH
// chunks: a chunk's activation, scale/zero and 16-byte weight loads
// (non-temporal, one 1 KB row segment per instruction) are issued, then its
// blocks are dequantized and multiplied in arrival order while later chunks'
// loads of the other waves are in flight.  A CU accepts load instructions far
// more slowly than its waves can issue them and serves the oldest waves first;
// chunking keeps every wave's compute close behind its own data instead of
// leaving the youngest waves all their work at the end.  The waves' [16 x 64]
// fp32 partials are summed through LDS in wave order (deterministic) and stored
// as 8-byte bf16 (16-byte f32) row segments.
#pragma once
#include "gemm_bf16_kernel.h"
#include "xcd_exchange.h"

namespace t0mi {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

struct W4Params {
  const uint16_t* a;       // [M, K] bf16
  const uint32_t* w;       // [K/8, N] packed int4
  const uint16_t* scales;  // [K/g, N] bf16
  const uint32_t* zeros;   // [K/g, N/8] packed int4, or null -> zp_const
  void* y;                 // [M, N] out (or f32 partial planes)
  uint32_t M, K, N, group; // group % 32 == 0
  uint32_t zp_const;
  uint32_t out_bf16;
  uint32_t kb_per_split;   // k-blocks (of 32) per grid.y partition
  uint64_t y_split_stride; // bytes between partial planes when gridDim.y > 1
  uint32_t nib_mask;       // 0x000F000F (see nib_pairs_ao)
  uint32_t nib_magic;      // 0x43004300
  // In-launch K split (w4a16_decode_v2 with XK): 64-column strips, K pieces per
  // strip (pieces * NW * KBW k-blocks cover K), and the XCD exchange.
  uint32_t strips, pieces;
  XcdExchange xk;
};

__device__ __forceinline__ bf16x8_t nib_pairs(uint32_t w) {
  // 8 nibbles -> bf16 (128+q) in element order q0,q4,q1,q5,q2,q6,q3,q7.
  u32x4 d;
  d.x = (w & 0x000F000Fu) | 0x43004300u;
  d.y = ((w >> 4) & 0x000F000Fu) | 0x43004300u;
  d.z = ((w >> 8) & 0x000F000Fu) | 0x43004300u;
  d.w = ((w >> 12) & 0x000F000Fu) | 0x43004300u;
  return __builtin_bit_cast(bf16x8_t, d);
}

// nib_pairs in 7 VALU instructions (3 shifts, 4 v_bfi_b32): with mask =
// 0x000F000F and magic = 0x43004300 (disjoint bits), (mask & x) | (~mask & magic)
// is (x & mask) | magic, the bit-field-insert form.  Both arrive as kernel
// arguments so that they stay in registers instead of folding into literals
// (a gfx9 VOP3 instruction takes no literal operand).
__device__ __forceinline__ uint32_t bfi(uint32_t mask, uint32_t x, uint32_t y) { return (mask & x) | (~mask & y); }
__device__ __forceinline__ bf16x8_t nib_pairs_ao(uint32_t w, uint32_t mask, uint32_t magic) {
  u32x4 d;
  d.x = bfi(mask, w, magic);
  d.y = bfi(mask, w >> 4, magic);
  d.z = bfi(mask, w >> 8, magic);
  d.w = bfi(mask, w >> 12, magic);
  return __builtin_bit_cast(bf16x8_t, d);
}

__device__ __forceinline__ bf16x8_t perm_act(u32x4 a) {
  // a = (a0,a1)(a2,a3)(a4,a5)(a6,a7) -> (a0,a4)(a1,a5)(a2,a6)(a3,a7)
  u32x4 o;
  o.x = __builtin_amdgcn_perm(a.z, a.x, 0x05040100u);
  o.y = __builtin_amdgcn_perm(a.z, a.x, 0x07060302u);
  o.z = __builtin_amdgcn_perm(a.w, a.y, 0x05040100u);
  o.w = __builtin_amdgcn_perm(a.w, a.y, 0x07060302u);
  return __builtin_bit_cast(bf16x8_t, o);
}

__device__ __forceinline__ float bf16f(uint32_t h) { return __builtin_bit_cast(float, h << 16); }

// One workgroup = NW waves on one 64-column strip; wave v of partition
// blockIdx.y owns k-blocks [kb0, kb0 + KBW), kb0 = (blockIdx.y * NW + v) * KBW.
// Groups are KBPG k-blocks (KBPG | KBW), so every wave covers whole groups and
// K % group == 0 makes every group either complete or absent: absent groups
// (the ragged end of K) are skipped by a wave-uniform branch and their loads
// read a clamped, valid address.  Lane (c, g) = (lane % 16, lane / 16) loads
// the 4 words of columns n0 + 4c .. +3 for K sub-row g of each block and
// activation row c (rows >= M read row 0 and are never stored).
//
// RS row slabs of 16 (1..4) share one pass over the weights: each dequantized
// weight fragment feeds every slab's MFMAs, and every row goes through exactly
// the operations of a 16-row launch on its own slab (bit-identical results).
//
// XK (one slab): a 1-D grid of strips x p.pieces workgroups numbered for the
// XCD exchange (xcd_exchange.h); piece c of a strip covers k-blocks
// [c * NW * KBW, (c + 1) * NW * KBW).  With one piece the strip is stored
// directly; otherwise the pieces store their [16 x 64] fp32 partials with the
// device-scope policy (normally all on the strip's XCD) and the last piece sums
// them in piece order and stores Y, all in this launch: every CU gets several
// workgroups however few strips N has.
template <int NW, int KBW, int KBPG, bool ZEROS, int CH = 1, int RS = 1, bool XK = false>
__global__ __launch_bounds__(NW * 64) void w4a16_decode_v2(W4Params p) {
  static_assert(KBW % KBPG == 0, "whole groups per wave");
  static_assert(RS >= 1 && RS <= 4, "one to four row slabs");
  static_assert(!XK || RS == 1, "the in-launch K split runs one slab");
  // CH chunks per wave: chunk c's loads are issued, then its blocks computed,
  // before chunk c+1's loads (CB blocks, whole groups and pairs per chunk).
  constexpr int CB = KBW / CH;
  static_assert(KBW % CH == 0 && CB % KBPG == 0 && CB % 2 == 0, "chunks of whole groups and pairs");
  // The wave index is wave-uniform: in an SGPR, the LDS slice and K-range
  // addresses are scalar arithmetic (3 % faster than as a per-lane value).
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int c = lane & 15, g = lane >> 4;
  uint32_t strip = blockIdx.x, part = blockIdx.y;
  if (XK) {
    xk_unpack(blockIdx.x, p.xk.nx, p.pieces, &strip, &part);
    if (strip >= p.strips) return;  // the numbering's padding (whole workgroup)
    xk_check_placement(p.xk);
  }
  const int n0 = (int)strip * 64;
  const int ncol = n0 + 4 * c;
  const bool col_ok = ncol < (int)p.N;  // N % 8 == 0, so the whole quad is in range
  const int ncol_c = col_ok ? ncol : 0;
  const int kb_tot = (int)(p.K / 32);
  const int kb0 = __builtin_amdgcn_readfirstlane(((int)part * NW + wave) * KBW);
  int nkb = kb_tot - kb0;  // valid k-blocks of this wave (wave-uniform)
  nkb = nkb < 0 ? 0 : (nkb > KBW ? KBW : nkb);

  const int ngroups = kb_tot / KBPG;
  const uint32_t mask = p.nib_mask, magic = p.nib_magic;
  const bf16x8_t ones = __builtin_bit_cast(bf16x8_t, (u32x4){0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u});
  f32x4 acc[RS][4];
#pragma unroll
  for (int s = 0; s < RS; ++s)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[s][j] = (f32x4){0.f, 0.f, 0.f, 0.f};

  // Activation slices are loaded 1 KB (8 rows x one 128-byte line of 64 K
  // values) per instruction, stored to LDS and read back in the MFMA layout
  // with ds_read_b128.  Piece (row 8h + r, 16-byte chunk x) of the block
  // (pair p, half h) sits in slot
  //   dec_slot(h, r, x) = 16 * (x >> 1) + ((8h + r) ^ (8 * (x & 1) + (x >> 1))),
  // so for a fixed chunk the 16 rows fall in 16 distinct 16-byte bank groups
  // and the fragment reads (16 rows x one chunk per 16 lanes) are free of bank
  // conflicts.
  // With one slab a wave's slice keeps all its KBW blocks; with more it holds
  // the current chunk of every slab (a chunk's LDS writes come after the
  // previous chunk's reads have been consumed, and the slice is the wave's own).
  static_assert(KBW % 2 == 0, "k-blocks are moved in pairs");
  constexpr int SMEM_KB = RS == 1 ? (KBW > 4 ? KBW : 4) : (CB > 4 ? RS * CB : RS * 4);  // KB per wave
  static_assert(NW * SMEM_KB <= 160, "the workgroup's LDS fits a CU (160 KB)");
  __shared__ __attribute__((aligned(1024))) float smem[NW * SMEM_KB * 256];
  const uint32_t lds_wave = lds_addr(smem) + (uint32_t)(wave * SMEM_KB * 1024);
  // Byte offset of the 2 KB pair holding block `blk` of the chunk starting at B0, slab s.
  auto pair_off = [](int s, int B0, int blk) {
    return (uint32_t)((RS == 1 ? (B0 + blk) >> 1 : s * (CB / 2) + (blk >> 1)) * 2048);
  };
  // Loads: the 16 lanes of quarter k read rows k and k+4 (two whole lines) of
  // the 8-row half; the two rows' slot sets are disjoint, so the stores are
  // conflict-free too.
  const int ld_r = (lane >> 4) + 4 * ((lane >> 3) & 1), ld_x = lane & 7;
  const int st_off[2] = {16 * dec_slot(0, ld_r, ld_x), 1024 + 16 * dec_slot(1, ld_r, ld_x)};
  int rd_off[2];  // fragment byte offset for k-block parity 0 / 1
#pragma unroll
  for (int beta = 0; beta < 2; ++beta) {
    const int h = c >> 3, r = c & 7, x = 4 * beta + g;
    rd_off[beta] = h * 1024 + 16 * dec_slot(h, r, x);
  }

  // FULL: all KBW blocks of the wave exist (every wave but those at the ragged
  // end of K); then nothing is clamped or skipped and no branch separates the
  // loads from their uses.
  auto body = [&](auto full_c, auto chunk_c) {
    constexpr bool FULL = decltype(full_c)::value;
    constexpr int B0 = decltype(chunk_c)::value * CB;  // first block of this chunk
    constexpr int G0 = B0 / KBPG, NGC = CB / KBPG;      // its groups
    u32x4 wv[CB], at[RS * CB];
    u32x2 sv[NGC];
    uint32_t zv[NGC];
    // Activation loads (L2-resident) first, then scales, weights last: loads
    // complete in issue order, so block b's dequant waits only for weight row b.
#pragma unroll
    for (int sl = 0; sl < RS; ++sl) {
#pragma unroll
      for (int pp = 0; pp < CB / 2; ++pp) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          int row = 16 * sl + 8 * h + ld_r;
          row = row < (int)p.M ? row : 0;
          int kofs = (kb0 + B0 + 2 * pp) * 32 + 8 * ld_x;
          if (!FULL) kofs = kofs + 8 <= (int)p.K ? kofs : 0;
          at[sl * CB + 2 * pp + h] = *(const u32x4*)(p.a + (size_t)row * p.K + kofs);
        }
      }
    }
#pragma unroll
    for (int q = 0; q < NGC; ++q) {
      int grp = kb0 / KBPG + G0 + q;
      if (!FULL) grp = grp < ngroups ? grp : ngroups - 1;
      sv[q] = *(const u32x2*)(p.scales + (size_t)grp * p.N + ncol_c);
      zv[q] = ZEROS ? p.zeros[(size_t)grp * (p.N / 8) + ncol_c / 8] : 0u;  // shifted at use
    }
#pragma unroll
    for (int b = 0; b < CB; ++b) {
      int kb = kb0 + B0 + b;
      if (!FULL) kb = kb < kb_tot ? kb : kb_tot - 1;
      wv[b] = __builtin_nontemporal_load((const u32x4*)(p.w + (size_t)(kb * 4 + g) * p.N + ncol_c));
    }
    // Every load is issued before the first dequant: nothing may move across.
    __builtin_amdgcn_sched_barrier(0);
    // Activation pieces -> this wave's LDS slice (slot = lane), read back below
    // in the MFMA layout; LDS operations of one wave complete in order.
#pragma unroll
    for (int sl = 0; sl < RS; ++sl)
#pragma unroll
      for (int i = 0; i < CB; ++i)
        *(__attribute__((address_space(3))) u32x4*)(size_t)(lds_wave + pair_off(sl, B0, i) + (uint32_t)st_off[i & 1]) =
            at[sl * CB + i];
#pragma unroll
    for (int q = 0; q < NGC; ++q) {
      if (!FULL && (G0 + q) * KBPG >= nkb) break;  // wave-uniform: the ragged end of K
      f32x4 P[RS][4], S[RS];
#pragma unroll
      for (int sl = 0; sl < RS; ++sl) {
        S[sl] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; ++j) P[sl][j] = (f32x4){0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int i = 0; i < KBPG; ++i) {
        const int b = q * KBPG + i;  // block within the chunk
        const bf16x8_t W[4] = {nib_pairs_ao(wv[b].x, mask, magic), nib_pairs_ao(wv[b].y, mask, magic),
                               nib_pairs_ao(wv[b].z, mask, magic), nib_pairs_ao(wv[b].w, mask, magic)};
#pragma unroll
        for (int sl = 0; sl < RS; ++sl) {
          const u32x4 av = *(const __attribute__((address_space(3))) u32x4*)(size_t)(
              lds_wave + pair_off(sl, B0, b) + (uint32_t)rd_off[b & 1]);
          const bf16x8_t A = perm_act(av);
          S[sl] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, ones, S[sl], 0, 0, 0);
#pragma unroll
          for (int j = 0; j < 4; ++j) P[sl][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, W[j], P[sl][j], 0, 0, 0);
        }
      }
      // y += s * (P - (128 + z) * S) for the four columns ncol + j of this lane.
      const float s4[4] = {bf16f(sv[q].x & 0xFFFFu), bf16f(sv[q].x >> 16), bf16f(sv[q].y & 0xFFFFu),
                           bf16f(sv[q].y >> 16)};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float z = 128.0f + (float)(ZEROS ? ((zv[q] >> (4 * ((ncol_c & 7) + j))) & 0xFu) : p.zp_const);
#pragma unroll
        for (int sl = 0; sl < RS; ++sl) {
          acc[sl][j].x = fmaf(s4[j], fmaf(-z, S[sl].x, P[sl][j].x), acc[sl][j].x);
          acc[sl][j].y = fmaf(s4[j], fmaf(-z, S[sl].y, P[sl][j].y), acc[sl][j].y);
          acc[sl][j].z = fmaf(s4[j], fmaf(-z, S[sl].z, P[sl][j].z), acc[sl][j].z);
          acc[sl][j].w = fmaf(s4[j], fmaf(-z, S[sl].w, P[sl][j].w), acc[sl][j].w);
        }
      }
    }
  };
  if (nkb == KBW)
    static_for<CH>([&](auto cc) { body(std::integral_constant<bool, true>{}, cc); });
  else
    static_for<CH>([&](auto cc) { body(std::integral_constant<bool, false>{}, cc); });

  // Lane (c, g) holds rows 4g + r, columns 4c + j as acc[j][r].  Each wave
  // stages its [16 x 64] partial (row-major) at the start of its own
  // activation slice — its reads of the slice precede these writes in program
  // order and a wave's LDS operations complete in order — so one barrier
  // separates the writes from the sum, in which each of 256 threads adds one
  // row segment of 4 columns over the waves (in wave order) and stores it with
  // one vector store.
  static_assert(SMEM_KB * 256 >= RS * 16 * 64, "a wave's slice holds its [16 x 64] partials");
  float* red = smem;
  float* mine = red + wave * SMEM_KB * 256;
#pragma unroll
  for (int sl = 0; sl < RS; ++sl)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      *(f32x4*)(mine + sl * 1024 + (4 * g + r) * 64 + 4 * c) =
          (f32x4){acc[sl][0][r], acc[sl][1][r], acc[sl][2][r], acc[sl][3][r]};
  __syncthreads();
  auto wave_sum = [&](int so) {
    f32x4 s4 = *(const f32x4*)(red + so);
#pragma unroll
    for (int v = 1; v < NW; ++v) {
      const f32x4 t4 = *(const f32x4*)(red + v * SMEM_KB * 256 + so);
      s4.x += t4.x;
      s4.y += t4.y;
      s4.z += t4.z;
      s4.w += t4.w;
    }
    return s4;
  };
  if (XK && p.pieces > 1) {
    // This piece's [16 x 64] partial -> its slot; the last piece of the strip
    // sums the slots in piece order (its own from registers) and stores Y.
    constexpr int SEG = (256 + NW * 64 - 1) / (NW * 64);  // row segments per thread
    const auto slots = xk_slots(p.xk.part + (size_t)strip * p.pieces * 1024, p.pieces * 4096u);
    f32x4 own[SEG];
#pragma unroll
    for (int i = 0; i < SEG; ++i) {
      const int t = (int)threadIdx.x + i * NW * 64;
      if (t < 256) {
        own[i] = wave_sum((t >> 4) * 64 + 4 * (t & 15));
        xk_store(slots, (part * 1024u + (t >> 4) * 64u + 4u * (t & 15)) * 4u, own[i]);
      }
    }
    if (!xk_arrive(p.xk, strip, p.pieces)) return;
    // Every slot load is issued before the first add: loads under a branch
    // would each wait at the branch join (the first XK build read 7 slots one
    // after another, 10 us at config 4).  Slot indices past the piece count are
    // clamped to the last slot and their values not added.
    auto sum_slots = [&](auto pmax_c, int so, const f32x4& mine) {
      constexpr int PMAX = decltype(pmax_c)::value;
      f32x4 v[PMAX];
#pragma unroll
      for (int q = 0; q < PMAX; ++q) {
        const int qq = q < (int)p.pieces ? q : (int)p.pieces - 1;
        v[q] = xk_load(slots, (uint32_t)(qq * 1024 + so) * 4u);
      }
      f32x4 s4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int q = 0; q < PMAX; ++q) {
        const f32x4 t4 = q == (int)part ? mine : v[q];
        if (q < (int)p.pieces) {
          s4.x += t4.x;
          s4.y += t4.y;
          s4.z += t4.z;
          s4.w += t4.w;
        }
      }
      return s4;
    };
#pragma unroll
    for (int i = 0; i < SEG; ++i) {
      const int t = (int)threadIdx.x + i * NW * 64;
      if (t >= 256) continue;
      const int C = t & 15, R = t >> 4, so = R * 64 + 4 * C;
      // pieces <= 16 (kXkMaxPieces on the host)
      const f32x4 s4 = p.pieces <= 8 ? sum_slots(std::integral_constant<int, 8>{}, so, own[i])
                                     : sum_slots(std::integral_constant<int, 16>{}, so, own[i]);
      const int col = n0 + 4 * C;
      if (R >= (int)p.M || col >= (int)p.N) continue;
      if (p.out_bf16) {
        *(u32x2*)((uint16_t*)p.y + (size_t)R * p.N + col) = u32x2{pack_bf16x2(s4.x, s4.y), pack_bf16x2(s4.z, s4.w)};
      } else {
        f32x2_t* o = (f32x2_t*)((float*)p.y + (size_t)R * p.N + col);
        o[0] = f32x2_t{s4.x, s4.y};
        o[1] = f32x2_t{s4.z, s4.w};
      }
    }
    xk_reset(p.xk, strip);
    return;
  }
  for (int t = threadIdx.x; t < 256 * RS; t += NW * 64) {
    const int C = t & 15, R = t >> 4;  // R: output row of this launch (slab R / 16)
    const int so = (R >> 4) * 1024 + (R & 15) * 64 + 4 * C;
    const f32x4 s4 = wave_sum(so);
    const int col = n0 + 4 * C;
    if (R >= (int)p.M || col >= (int)p.N) continue;
    if (p.out_bf16 && gridDim.y == 1) {
      u32x2 o;
      o.x = pack_bf16x2(s4.x, s4.y);
      o.y = pack_bf16x2(s4.z, s4.w);
      *(u32x2*)((uint16_t*)p.y + (size_t)R * p.N + col) = o;
    } else {
      // f32 output or partial plane; Y is only guaranteed 8-byte aligned.
      float* yp = (float*)((char*)p.y + (gridDim.y > 1 ? (size_t)blockIdx.y * p.y_split_stride : 0));
      f32x2_t* o = (f32x2_t*)(yp + (size_t)R * p.N + col);
      o[0] = f32x2_t{s4.x, s4.y};
      o[1] = f32x2_t{s4.z, s4.w};
    }
  }
}

}  // namespace t0mi
