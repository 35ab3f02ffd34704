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
// the dequant-then-GEMM route, and each accumulator sums its products in the
// same k order as gemm_bf16_pingpong_kernel<NN, true>: for the same problem the
// two routes give bit-identical results (that kernel issues
// v_mfma_f32_16x16x32_bf16, this one v_mfma_f32_32x32x16_bf16, which on gfx950
// give identical sums for the same k order; the GPU tests check it).  This
// kernel stays on 32x32x16: with 16x16x32 blocks its read phase (8 packed words,
// the scales and zero points of 4 column blocks and the dequant temporaries)
// no longer fits beside the 128 accumulators and 96 operand registers of the
// 256 a wave has, and spills.
//
// What differs from the bf16 GEMM: the B tile is DMA'd as packed words (8 rows
// of 256 words = 8 KB per 64-K tile instead of 32 KB of bf16).  In the NN MFMA
// operand layout a lane's 8 consecutive k values of one column are exactly one
// packed word, so a B fragment is one ds_read_b32 plus ~23 VALU instructions:
// nibbles spread to bytes (2 AND/shift), v_cvt_f32_ubyte0..3, one fma
// q*s + (-z*s) (exact: |q - z| < 16 and s has 8 significant bits) and
// v_cvt_pk_bf16_f32 (RNE).  Both groups multiply the same B tile (by their own
// 128 rows of A), so each word is dequantized once per workgroup, half of each
// tile by either group in its read phase, and the other group reads those
// fragments back from LDS as bf16.  Each tile's 256 scales and 32 zero words
// travel with its packed words (DMA into the same LDS slot).
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
  constexpr int FM = 4, FN = 2, KC = 8, KS = 4;
  constexpr int AH_BYTES = 128 * BK * 2;  // half A tile, bf16
  // Packed-word B tile: 8 k-octet rows of 256 words, rows 1152 bytes apart so
  // that the two half-waves of a fragment read (rows kk, kk+1) hit disjoint
  // banks; then the tile's 256 bf16 scales (at +0 of the SZ area) and 32 zero
  // words (at +1024); the rest of the SZ area takes the zeros that the
  // out-of-range lanes of those two DMAs write.
  constexpr int BROW = 1152, SZ = 8 * BROW, BSLOT = SZ + 2048;
  constexpr int A_AREA = 4 * AH_BYTES;  // two groups x two slots
  constexpr int XB_OFF = A_AREA + 3 * BSLOT;  // dequantized fragments: F (16 KB), then S (16 KB)
  constexpr int LDS_BYTES = XB_OFF + 32768 > 8 * 16384 ? XB_OFF + 32768 : 8 * 16384;  // staged store reuses it
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
  // A: four row-block resources per group, as in gemm_bf16_pingpong_kernel.
  uint32_t a_voff;
  {
    const int row = w4 * 8 + (lane >> 3), pc = lane & 7;
    a_voff = (uint32_t)(row * (int)p.lda + ((pc ^ swz<KC>(row)) * 8)) * 2u;
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
  constexpr int NDMA = 5;

  const int lrow = lane & 31, lhalf = lane >> 5;
  // ---- LDS -> fragments --------------------------------------------------------
  int a_off[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) a_off[ks] = lrow * BK + (((ks * 2 + lhalf) ^ swz<KC>(lrow)) * 8);
  bf16x8 xa[KS][FM], xb[KS][FN];
  uint32_t bw[KS][FN];
  // A fragment i (k-step i / FM, row block i % FM).
  auto read_a = [&](const uint16_t* As, auto ic) {
    constexpr int i = decltype(ic)::value;
    xa[i / FM][i % FM] = *(const bf16x8*)(As + a_off[i / FM] + (i % FM) * 32 * BK);
  };
  // Packed B word i of k-steps K0.. (k-step K0 + i / FN, column block i % FN):
  // a lane base plus an immediate.
  const int b_lane = lhalf * (BROW / 4) + wn * TN + lrow;  // in words
  auto read_b = [&](const uint32_t* Bw, auto k0c, auto ic) {
    constexpr int i = decltype(ic)::value;
    constexpr int ks = decltype(k0c)::value + i / FN, fn = i % FN;
    bw[ks][fn] = Bw[b_lane + ks * 2 * (BROW / 4) + fn * 32];
  };

  f32x16 acc[FN][FM];
#pragma unroll
  for (int fn = 0; fn < FN; ++fn)
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[fn][fm][r] = 0.0f;

  const uint16_t* a_slots = (const uint16_t*)(smem + g * 2 * AH_BYTES);
  // Dequantized B fragments shared by the two groups, so that each packed word
  // is dequantized once per workgroup: region F holds k-steps 0-1 of a tile,
  // dequantized by group 1 in its read phase of the previous tile (their packed
  // rows 0-3 are group 0's DMA, landed a phase earlier), region S k-steps 2-3,
  // dequantized by group 0 in its read phase of the tile and read by group 1 in
  // the next phase.  Fragment (ks, fn) of column block wn lies at
  // XB_OFF + wn * 4 KB + ((ks % 2) * 2 + fn) KB (+ 16 KB for S), 16 bytes per
  // lane; only the waves of column block wn touch it, and one barrier separates
  // every write from its reads and every read from the next write.
  uint8_t* const xf = smem + XB_OFF + wn * 4096 + lane * 16;
  uint8_t* const xs = xf + 16384;
  auto frag = [](uint8_t* base, int ks, int fn) -> bf16x8* { return (bf16x8*)(base + ((ks & 1) * 2 + fn) * 1024); };
  // The lane's two columns' scales and zero points of a tile (issue, then after
  // the wait -z * s, exact: z < 16 and s has 8 significant bits).
  uint32_t sraw[2], zraw[2];
  float s_t[2], cz_t[2];
  auto sz_read = [&](const uint8_t* Bslot) {
#pragma unroll
    for (int f = 0; f < 2; ++f) {
      sraw[f] = ((const uint16_t*)(Bslot + SZ))[wn * TN + f * 32 + lrow];
      if constexpr (ZEROS) zraw[f] = ((const uint32_t*)(Bslot + SZ + 1024))[(wn * TN + f * 32 + lrow) / 8];
    }
  };
  auto sz_math = [&]() {
#pragma unroll
    for (int f = 0; f < 2; ++f) {
      s_t[f] = __builtin_bit_cast(float, sraw[f] << 16);
      const float z = ZEROS ? (float)((zraw[f] >> (4 * (lrow & 7))) & 0xFu) : (float)q.zp_const;
      cz_t[f] = -z * s_t[f];
    }
  };
  // Ring slots as wave-uniform scalars: each LDS address is then one add of a
  // loop-invariant lane offset and the slot (u % 3 left to the compiler is
  // strength-reduced across iterations into two per-iteration terms).
  auto a_slot = [&](int u) { return a_slots + __builtin_amdgcn_readfirstlane((int)(u & 1)) * (AH_BYTES / 2); };
  auto b_slot = [&](int u) { return smem + A_AREA + __builtin_amdgcn_readfirstlane((int)(u % 3)) * BSLOT; };
  // R(u), group 0: the packed words of k-steps 2-3 and the F fragments of
  // k-steps 0-1, then tile u's 16 A fragments with one word dequantized (into
  // xb and S) after every fourth A read, so the VALU work overlaps the A reads
  // in flight.
  auto read_phase_g0 = [&](int u) {
    const uint16_t* As = a_slot(u);
    const uint8_t* Bslot = b_slot(u);
    const uint32_t* Bw = (const uint32_t*)Bslot;
    static_for<4>([&](auto ic) {
      read_b(Bw, std::integral_constant<int, 2>{}, ic);
      __builtin_amdgcn_sched_barrier(0);
    });
    static_for<4>([&](auto ic) {
      constexpr int i = decltype(ic)::value, ks = i / FN, fn = i % FN;
      xb[ks][fn] = *frag(xf, ks, fn);
      __builtin_amdgcn_sched_barrier(0);
    });
    sz_read(Bslot);
    __builtin_amdgcn_sched_barrier(0);
    wait_lgkmcnt0();
    sz_math();
    static_for<KS * FM>([&](auto ic) {
      constexpr int i = decltype(ic)::value;
      read_a(As, ic);
      if constexpr (i % 4 == 1) {
        constexpr int wi = i / 4, ks = 2 + wi / FN, fn = wi % FN;
        xb[ks][fn] = dequant_word(bw[ks][fn], s_t[fn], cz_t[fn]);
        *frag(xs, ks, fn) = xb[ks][fn];
      }
      __builtin_amdgcn_sched_barrier(0);
    });
    wait_lgkmcnt0();
  };
  // R(u), group 1: tile u's 8 fragments from F and S and, when tile u+1
  // exists (NX), its packed words of k-steps 0-1 and its scales; after the
  // wait (which also lets the F reads return before F is rewritten) tile u's
  // 16 A fragments with one of tile u+1's words dequantized into F after every
  // fourth A read.
  auto read_phase_g1 = [&](int u, auto nx_c) {
    constexpr bool NX = decltype(nx_c)::value;
    const uint16_t* As = a_slot(u);
    static_for<KS * FN>([&](auto ic) {
      constexpr int i = decltype(ic)::value, ks = i / FN, fn = i % FN;
      xb[ks][fn] = *frag(ks < 2 ? xf : xs, ks, fn);
      __builtin_amdgcn_sched_barrier(0);
    });
    if constexpr (NX) {
      const uint8_t* Bslot = b_slot(u + 1);
      const uint32_t* Bw = (const uint32_t*)Bslot;
      static_for<4>([&](auto ic) {
        read_b(Bw, std::integral_constant<int, 0>{}, ic);
        __builtin_amdgcn_sched_barrier(0);
      });
      sz_read(Bslot);
    }
    __builtin_amdgcn_sched_barrier(0);
    wait_lgkmcnt0();
    if constexpr (NX) sz_math();
    static_for<KS * FM>([&](auto ic) {
      constexpr int i = decltype(ic)::value;
      read_a(As, ic);
      if constexpr (NX && i % 4 == 1) {
        constexpr int wi = i / 4, ks = wi / FN, fn = wi % FN;
        *frag(xf, ks, fn) = dequant_word(bw[ks][fn], s_t[fn], cz_t[fn]);
      }
      __builtin_amdgcn_sched_barrier(0);
    });
    wait_lgkmcnt0();
  };
  auto mfma_phase = [&](auto dma_c, int td) {
    constexpr bool D = decltype(dma_c)::value;
    static_for<KS * FN * FM>([&](auto ic) {
      constexpr int i = decltype(ic)::value;
      constexpr int ks = i / (FN * FM), fn = (i / FM) % FN, fm = i % FM;
      acc[fn][fm] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xb[ks][fn], xa[ks][fm], acc[fn][fm], 0, 0, 0);
      if constexpr (D && i >= 16 && (i - 16) % 3 == 0 && (i - 16) / 3 < NDMA)
        dma(td, std::integral_constant<int, (i - 16) / 3>{});
      if constexpr (D && i == 31)
        if (wave == 0) dma_sz(td);
      __builtin_amdgcn_sched_barrier(0);
    });
  };
  auto bar = []() {
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
  };
  using True = std::integral_constant<bool, true>;
  using False = std::integral_constant<bool, false>;

  // The ping-pong schedule (R(u) bar M(u) bar per tile, group 1 one barrier
  // behind), with the DMA of tile u+2 (with its scales and zero points) inside
  // M(u) -- between 32-cycle MFMAs a DMA issue does not stall the MFMA stream,
  // and the read phase carries the dequant -- each wave waiting for its DMA at
  // the end of its next read phase.  Before group 0's first read phase group 1
  // dequantizes tile 0's k-steps 0-1 into F (one extra barrier for both groups).
  if (nk > 0) {
    static_for<NDMA>([&](auto jc) { dma(0, jc); });
    if (wave == 0) dma_sz(0);
  }
  if (nk > 1) {
    static_for<NDMA>([&](auto jc) { dma(1, jc); });
    if (wave == 0) dma_sz(1);
  }
  wait_vmcnt<0>();
  bar();
  if (!g0 && nk > 0) {
    const uint8_t* Bslot = b_slot(0);
    const uint32_t* Bw = (const uint32_t*)Bslot;
    static_for<4>([&](auto ic) { read_b(Bw, std::integral_constant<int, 0>{}, ic); });
    sz_read(Bslot);
    wait_lgkmcnt0();
    sz_math();
    static_for<4>([&](auto ic) {
      constexpr int i = decltype(ic)::value, ks = i / FN, fn = i % FN;
      *frag(xf, ks, fn) = dequant_word(bw[ks][fn], s_t[fn], cz_t[fn]);
    });
    wait_lgkmcnt0();
  }
  bar();
  if (!g0) bar();
  // Each group runs its own copy of the loops (a wave-uniform branch taken once
  // instead of once per read phase); both execute the same barriers.
  auto run = [&](auto g0_c) {
    constexpr bool G0 = decltype(g0_c)::value;
    int u = 0;
    for (; u + 2 < nk; ++u) {
      if constexpr (G0) read_phase_g0(u);
      else read_phase_g1(u, True{});
      wait_vmcnt<0>();
      bar();
      mfma_phase(True{}, u + 2);
      bar();
    }
    for (; u < nk; ++u) {
      if constexpr (G0) read_phase_g0(u);
      else if (u + 1 < nk) read_phase_g1(u, True{});
      else read_phase_g1(u, False{});
      wait_vmcnt<0>();
      bar();
      mfma_phase(False{}, 0);
      if (u + 1 < nk) bar();
    }
  };
  if (g0) run(True{});
  else run(False{});
  if (g0) bar();

  // ---- epilogue --------------------------------------------------------------
  const bool partial_plane = p.split_k > 1;
  char* ybase = (char*)p.y + (partial_plane ? (size_t)part * p.y_split_stride : 0);
  const int row0 = m0 + g * 128;
  const int col0 = n0 + wn * TN;
  if (!partial_plane && p.out_bf16 && m0 + 256 <= (int)p.M && n0 + 256 <= (int)p.N && ((uintptr_t)p.y & 15) == 0) {
    store_tile_bf16_staged<FM, FN>(p, acc, (char*)smem + wave * 16384, ybase, row0, col0, lane);
  } else {
    static_for<FM>([&](auto fmc) {
      constexpr int fm = decltype(fmc)::value;
      const int m = row0 + fm * 32 + lrow;
      if (m < (int)p.M) {
        static_for<FN>([&](auto fnc) {
          constexpr int fn = decltype(fnc)::value;
          store_block(p, acc[fn][fm], ybase, m, col0 + fn * 32 + lhalf * 4, partial_plane);
        });
      }
    });
  }
}

}  // namespace t0mi
