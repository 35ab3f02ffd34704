// w4a16_pingpong.h — gfx950 W4A16 GEMM with the dequant fused into the K loop,
// on the ping-pong schedule of gemm_pingpong.h (256x256x64 tiles, 8 waves in
// two groups alternating LDS-read and MFMA phases).
//
//   Y[M,N] = A[M,K] . W[K,N],  w[k][n] = bf16_rne((q[k][n] - z[k/g][n]) * s[k/g][n])
//
// W is packed int4 u32 [K/8][N] (word (kk, n) holds q[8kk+e][n] in bits
// 4e..4e+3, the reference's low-nibble-first order, src/t0/quant_kernels.rs:3-10),
// scales bf16 [K/g][N], zero points packed int4 u32 [K/g][N/8] or a constant.
// The weight is rounded once to bf16, exactly as dequant_int4_kernel does for
// the dequant-then-GEMM route, and the MFMA order per accumulator is that of
// gemm_bf16_pingpong_kernel<NN, true> (v_mfma_f32_16x16x32_bf16, 8 x 4 blocks
// per wave): for the same problem the two routes give bit-identical results.
//
// What differs from the bf16 GEMM: the B tile is DMA'd as packed words (8 rows
// of 256 words = 8 KB per 64-K tile instead of 32 KB of bf16).  In the NN MFMA
// operand layout a lane's 8 consecutive k values of one column are exactly one
// packed word, so each B fragment is one ds_read_b32 plus ~23 VALU
// instructions in the read phase: nibbles spread to bytes (2 AND/shift),
// v_cvt_f32_ubyte0..3, one fma q*s + (-z*s) (exact: |q - z| < 16 and s has 8
// significant bits) and v_cvt_pk_bf16_f32 (RNE).  The read phase has the slack
// for it and for the DMA (the MFMA phase is the longer of the two).  Each
// tile's 256 scales and 32 zero words travel with its packed words (DMA into
// the same LDS slot).
//
// Preconditions (w4_pingpong_ok): K and the split-K partition length are
// multiples of 64 and the group a multiple of 64, so every 64-K tile lies in
// one group.  Ragged M: A through buffer resources (rows past M load zeros);
// ragged N: packed words, scales and zero words are read through buffer
// resources (past the end of the tensor they load zeros; inside it, columns
// past N read the next row's values, whose products land in columns that are
// not stored).
#pragma once
#include "gemm_pingpong.h"

namespace t0mi {

struct W4PPParams {
  GemmParams g;            // A, Y, M, N, K, lda (= K), ldy, tiles, split-K, output; b / ldb unused
  const uint32_t* w;       // [K/8, N] packed int4
  const uint16_t* scales;  // [K/g, N] bf16
  const uint32_t* zeros;   // [K/g, N/8] packed int4, or null -> zp_const
  uint32_t zp_const, group;
};

inline bool w4_pingpong_ok(uint32_t K, uint32_t group, uint32_t split_k, uint32_t k_per_split) {
  if (K == 0 || K % 64 != 0 || group == 0 || group % 64 != 0) return false;
  if (split_k > 1 && k_per_split % 64 != 0) return false;
  return true;
}

// Byte n of x as a float: v_cvt_f32_ubyte<n>, one instruction (written out
// because the compiler, knowing the byte holds a nibble, otherwise extracts it
// with v_bfe_u32 first).
template <int B>
__device__ __forceinline__ float ubyte_f32(uint32_t x) {
  float f;
  if constexpr (B == 0) asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(f) : "v"(x));
  else if constexpr (B == 1) asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(f) : "v"(x));
  else if constexpr (B == 2) asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(f) : "v"(x));
  else asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(f) : "v"(x));
  return f;
}

// 8 nibbles (k order) of one packed word -> 8 bf16 weights (q - z) * s, RNE;
// cz = -z * s.  22 VALU instructions.
__device__ __forceinline__ bf16x8 dequant_word(uint32_t w, float s, float cz) {
  const uint32_t lo = w & 0x0F0F0F0Fu;         // nibbles 0, 2, 4, 6 in bytes 0..3
  const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;  // nibbles 1, 3, 5, 7
  u32x4 o;
  o.x = pack_bf16x2(__builtin_fmaf(ubyte_f32<0>(lo), s, cz), __builtin_fmaf(ubyte_f32<0>(hi), s, cz));
  o.y = pack_bf16x2(__builtin_fmaf(ubyte_f32<1>(lo), s, cz), __builtin_fmaf(ubyte_f32<1>(hi), s, cz));
  o.z = pack_bf16x2(__builtin_fmaf(ubyte_f32<2>(lo), s, cz), __builtin_fmaf(ubyte_f32<2>(hi), s, cz));
  o.w = pack_bf16x2(__builtin_fmaf(ubyte_f32<3>(lo), s, cz), __builtin_fmaf(ubyte_f32<3>(hi), s, cz));
  return __builtin_bit_cast(bf16x8, o);
}

template <bool ZEROS>
__global__ __launch_bounds__(512) void w4a16_pingpong_kernel(W4PPParams q) {
  const GemmParams& p = q.g;
  constexpr int BK = 64, TN = 64;
  constexpr int FM = 8, FN = 4, KC = 8, KS = 2;  // 16x16 blocks per wave, k-steps of 32
  constexpr int AH_BYTES = 128 * BK * 2;         // half A tile, bf16
  // Packed-word B tile: 8 k-octet rows of 256 words, rows BROW bytes apart; a
  // fragment read takes 16 consecutive words of each of 4 consecutive rows
  // (lane l: row 4 ks + l / 16), and a pitch of 272 words (16 mod 64 banks)
  // puts those four runs on disjoint banks.  Then the tile's 256 bf16 scales
  // (at +0 of the SZ area) and 32 zero words (at +1024); the rest of the SZ
  // area takes the zeros that the out-of-range lanes of those two DMAs write.
  constexpr int BROW = 1088, SZ = 8 * BROW, BSLOT = SZ + 2048;
  constexpr int A_AREA = 4 * AH_BYTES;  // two groups x two slots
  constexpr int LDS_BYTES = A_AREA + 3 * BSLOT > 8 * 16384 ? A_AREA + 3 * BSLOT : 8 * 16384;  // staged store reuses it
  __shared__ __attribute__((aligned(1024))) uint8_t smem[LDS_BYTES];

  int tm, tn, part;
  tile_coords(p, tm, tn, part);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int g = wave >> 2, w4 = wave & 3;
  const bool g0 = g == 0;
  const int wn = wave & 3;
  const int m0 = tm * 256, n0 = tn * 256;
  const int kbeg = part * (int)p.k_per_split;
  int kend = kbeg + (int)p.k_per_split;
  if (kend > (int)p.K) kend = (int)p.K;
  const int nk = kend > kbeg ? (kend - kbeg) / BK : 0;
  const uint32_t N = p.N;
  const uint32_t smem_base = lds_addr(smem);
  const uint32_t a_lds0 = smem_base + (uint32_t)(g * 2 * AH_BYTES) + w4 * 1024;
  const uint32_t b_lds0 = smem_base + (uint32_t)A_AREA + (uint32_t)((4 * g + w4) * BROW);

  // ---- DMA -----------------------------------------------------------------
  // A: as in gemm_bf16_pingpong_kernel<., true> (four row-block resources per
  // group, the 16x16x32 row layout).
  uint32_t a_voff;
  {
    int row, lc;
    kc_dma_chunk<KC, true>(w4 * 64 + lane, &row, &lc);
    a_voff = (uint32_t)(row * (int)p.lda + lc * 8) * 2u;
  }
  const uint64_t a_row_bytes = (uint64_t)p.lda * 2u;
  u32x4 a_rs[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r0 = m0 + g * 128 + j * 32, left_rows = (int)p.M - r0;
    const uint64_t left = left_rows <= 0 ? 0u : (uint64_t)left_rows * a_row_bytes;
    a_rs[j] = make_rsrc((const char*)p.a + (uint64_t)r0 * a_row_bytes, left > 0x7fffffffu ? 0x7fffffffu : (uint32_t)left);
  }
  // B: wave w4 of group g loads packed-word row kk = 4g + w4 of each tile: the
  // 256 words of columns n0 .. n0+255 (1 KB, 16 bytes per lane).
  const uint64_t w_bytes = (uint64_t)(p.K / 8) * N * 4u;
  auto dma = [&](int t, auto jc) {
    constexpr int j = decltype(jc)::value;
    if constexpr (j < 4) {
      lds_dma16_rsrc(a_rs[j], a_voff, (uint32_t)(kbeg + t * BK) * 2u,
                     a_lds0 + (uint32_t)((t & 1) * AH_BYTES) + 4 * j * 1024);
    } else {
      const uint64_t off = ((uint64_t)((kbeg + t * BK) / 8 + 4 * g + w4) * N + (uint64_t)n0) * 4u;
      const uint64_t left = w_bytes - off;  // off < w_bytes: the row exists
      const u32x4 rs = make_rsrc((const char*)q.w + off, left > 0x7fffffffu ? 0x7fffffffu : (uint32_t)left);
      lds_dma16_rsrc(rs, (uint32_t)lane * 16u, 0u, b_lds0 + (uint32_t)((t % 3) * BSLOT));
    }
  };
  // Scales (and zero words) of tile t: 512 (128) bytes from column n0 of the
  // tile's group row, issued by wave 0; lanes past them are out of range.
  constexpr int NSZ = ZEROS ? 2 : 1;  // wave 0's extra loads per tile
  auto dma_sz = [&](int t) {
    const uint32_t gk = (uint32_t)(kbeg + t * BK) / q.group;
    const uint32_t slot = smem_base + (uint32_t)A_AREA + (uint32_t)((t % 3) * BSLOT) + SZ;
    const uint64_t s_bytes = (uint64_t)(p.K / q.group) * N * 2u, s_off = ((uint64_t)gk * N + n0) * 2u;
    const uint64_t s_left = s_bytes - s_off;
    lds_dma16_rsrc(make_rsrc((const char*)q.scales + s_off, s_left > 512u ? 512u : (uint32_t)s_left), (uint32_t)lane * 16u,
                   0u, slot);
    if constexpr (ZEROS) {
      const uint64_t z_bytes = (uint64_t)(p.K / q.group) * (N / 8) * 4u, z_off = ((uint64_t)gk * (N / 8) + n0 / 8) * 4u;
      const uint64_t z_left = z_bytes - z_off;
      lds_dma16_rsrc(make_rsrc((const char*)q.zeros + z_off, z_left > 128u ? 128u : (uint32_t)z_left),
                     (uint32_t)lane * 16u, 0u, slot + 1024u);
    }
  };
  // s_waitcnt vmcnt(N) with N = n for waves 1-7 and n + extra for wave 0.
  auto wait_loads = [&](auto n_c, auto extra_c) {
    constexpr int n = decltype(n_c)::value, extra = decltype(extra_c)::value;
    if (wave == 0)
      wait_vmcnt<n + extra>();
    else
      wait_vmcnt<n>();
  };

  const int lr = lane & 15, lq = lane >> 4;
  // ---- LDS -> fragments --------------------------------------------------------
  int a_off[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) a_off[ks] = kc_slot<KC, true>(lr, ks * 4 + lq) * 8;
  bf16x8 xa[KS][FM], xb[KS][FN];
  uint32_t bw[KS][FN];
  // A fragment i (k-step i / FM, row block i % FM); B word i (k-step i / FN,
  // column block i % FN): k-octet row 4 ks + l / 16, column 16 fn + l % 16 of
  // the wave's 64.
  auto read_a = [&](const uint16_t* As, auto ic) {
    constexpr int i = decltype(ic)::value;
    xa[i / FM][i % FM] = *(const bf16x8*)(As + a_off[i / FM] + (i % FM) * 16 * BK);
  };
  const int b_lane = lq * (BROW / 4) + wn * TN + lr;  // in words
  auto read_b = [&](const uint32_t* Bw, auto ic) {
    constexpr int i = decltype(ic)::value;
    constexpr int ks = i / FN, fn = i % FN;
    bw[ks][fn] = Bw[b_lane + ks * 4 * (BROW / 4) + fn * 16];
  };

  f32x4 acc[FN][FM];
#pragma unroll
  for (int fn = 0; fn < FN; ++fn)
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[fn][fm][r] = 0.0f;

  const uint16_t* a_slots = (const uint16_t*)(smem + g * 2 * AH_BYTES);
  // R(u): tile u's 8 packed B words and its scales / zero points, then its 16
  // A fragments with one word dequantized after every second A read, so the
  // VALU work overlaps the A reads in flight and each word dies early.  The
  // DMA of this wave (A of tile u+1 when DA; B, and for wave 0 the scales and
  // zero points, of tile u+2 when DB) is issued between the A reads; at the end
  // every load issued before R(u) is waited for (B of tile u+1, which the other
  // group reads after the next barrier).
  auto read_phase = [&](int u, auto da_c, auto db_c) {
    constexpr bool DA = decltype(da_c)::value, DB = decltype(db_c)::value;
    const uint16_t* As = a_slots + (u & 1) * (AH_BYTES / 2);
    const uint8_t* Bslot = smem + A_AREA + (u % 3) * BSLOT;
    const uint32_t* Bw = (const uint32_t*)Bslot;
    static_for<KS * FN>([&](auto ic) {
      read_b(Bw, ic);
      __builtin_amdgcn_sched_barrier(0);
    });
    float s_t[FN], cz_t[FN];
    uint32_t sraw[FN], zraw[FN];
#pragma unroll
    for (int f = 0; f < FN; ++f) {
      sraw[f] = ((const uint16_t*)(Bslot + SZ))[wn * TN + f * 16 + lr];
      if constexpr (ZEROS) zraw[f] = ((const uint32_t*)(Bslot + SZ + 1024))[(wn * TN + f * 16 + lr) / 8];
    }
    __builtin_amdgcn_sched_barrier(0);
    wait_lgkmcnt0();
#pragma unroll
    for (int f = 0; f < FN; ++f) {
      s_t[f] = __builtin_bit_cast(float, sraw[f] << 16);
      const float z = ZEROS ? (float)((zraw[f] >> (4 * (lr & 7))) & 0xFu) : (float)q.zp_const;
      cz_t[f] = -z * s_t[f];  // exact: z < 16, s has 8 significant bits
    }
    static_for<KS * FM>([&](auto ic) {
      constexpr int i = decltype(ic)::value;
      read_a(As, ic);
      if constexpr (i % 2 == 1) {
        constexpr int wi = i / 2, ks = wi / FN, fn = wi % FN;
        xb[ks][fn] = dequant_word(bw[ks][fn], s_t[fn], cz_t[fn]);
      }
      if constexpr (DA && i % 2 == 1 && i / 2 < 4) dma(u + 1, std::integral_constant<int, i / 2>{});
      if constexpr (DB && i == 9) dma(u + 2, std::integral_constant<int, 4>{});
      if constexpr (DB && i == 11)
        if (wave == 0) dma_sz(u + 2);
      __builtin_amdgcn_sched_barrier(0);
    });
    wait_lgkmcnt0();
    wait_loads(std::integral_constant<int, (DA ? 4 : 0) + (DB ? 1 : 0)>{},
               std::integral_constant<int, DB ? NSZ : 0>{});
  };
  // M(u): the tile's MFMAs in k-step order, then this wave's A of tile u+1 is
  // waited for (its B, scales and zero points of tile u+2 may stay in flight).
  auto mfma_phase = [&](auto db_c) {
    constexpr bool DB = decltype(db_c)::value;
    static_for<KS * FN * FM>([&](auto ic) {
      constexpr int i = decltype(ic)::value;
      constexpr int ks = i / (FN * FM), fn = (i / FM) % FN, fm = i % FM;
      acc[fn][fm] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xb[ks][fn], xa[ks][fm], acc[fn][fm], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    });
    wait_loads(std::integral_constant<int, DB ? 1 : 0>{}, std::integral_constant<int, DB ? NSZ : 0>{});
  };
  auto bar = []() {
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
  };
  using True = std::integral_constant<bool, true>;
  using False = std::integral_constant<bool, false>;

  // The schedule of gemm_bf16_pingpong_kernel: R(u) bar M(u) bar per tile,
  // group 1 one barrier behind; the prologue loads tile 0 and the B (with
  // scales and zero points) of tile 1 and waits for tile 0.
  if (nk > 0) {
    static_for<5>([&](auto jc) { dma(0, jc); });
    if (wave == 0) dma_sz(0);
  }
  if (nk > 1) {
    dma(1, std::integral_constant<int, 4>{});
    if (wave == 0) dma_sz(1);
    wait_loads(std::integral_constant<int, 1>{}, std::integral_constant<int, NSZ>{});
  } else {
    wait_vmcnt<0>();
  }
  bar();
  if (!g0) bar();
  int u = 0;
  for (; u + 2 < nk; ++u) {
    read_phase(u, True{}, True{});
    bar();
    mfma_phase(True{});
    bar();
  }
  if (u + 1 < nk) {
    read_phase(u, True{}, False{});
    bar();
    mfma_phase(False{});
    bar();
    ++u;
  }
  if (u < nk) {
    read_phase(u, False{}, False{});
    bar();
    mfma_phase(False{});
  }
  if (g0) bar();

  // ---- epilogue (as gemm_bf16_pingpong_kernel<., true>) ------------------------
  const bool partial_plane = p.split_k > 1;
  char* ybase = (char*)p.y + (partial_plane ? (size_t)part * p.y_split_stride : 0);
  const int row0 = m0 + g * 128;
  const int col0 = n0 + wn * TN;
  if (!partial_plane && p.out_bf16 && m0 + 256 <= (int)p.M && n0 + 256 <= (int)p.N && ((uintptr_t)p.y & 15) == 0) {
    store_tile_bf16_staged16<FM>(p, acc, (char*)smem + wave * 16384, ybase, row0, col0, lane);
  } else {
    static_for<FM>([&](auto fmc) {
      constexpr int fm = decltype(fmc)::value;
      const int m = row0 + fm * 16 + lr;
      if (m < (int)p.M) {
        static_for<FN>([&](auto fnc) {
          constexpr int fn = decltype(fnc)::value;
          store_block16(p, acc[fn][fm], ybase, m, col0 + fn * 16 + lq * 4, partial_plane);
        });
      }
    });
  }
}

}  // namespace t0mi
