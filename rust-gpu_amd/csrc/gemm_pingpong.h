// gemm_pingpong.h — gfx950 bf16 GEMM, 256x256x64 tiles (NN and NT), 8 waves in
// two groups that alternate between LDS reads and MFMA bursts ("ping-pong").
//
// Same math and the same per-accumulator MFMA order as gemm_bf16_kernel
// <256, 256, 64, 2, 4, 2, NN> (so results are bit-identical to it); it replaces
// that instantiation where its preconditions hold (pingpong_ok below):
//   src/t0/gemm_gen.rs:668-1438 (generate_lds_db): NT is the reference's
//   layout, NN the one BASELINE.json names.
//
// Schedule.  Waves 0-3 (group 0) own rows 0-127 of the tile and waves 4-7
// (group 1) rows 128-255; wave w and wave w+4 run on the same SIMD.  Every
// wave runs, per 64-K tile u, a read phase R(u) (all 32 fragments of the tile
// from LDS into registers) and an MFMA phase M(u) (the tile's 32 MFMAs, back
// to back), separated by workgroup barriers.  Group 1 starts one barrier
// later, so in every barrier interval one wave of each SIMD issues MFMAs while
// its partner reads LDS: the MFMA pipe is fed by one wave at a time without
// gaps.  With both waves of a SIMD interleaving reads and MFMAs (the generic
// kernel) the older wave finishes its tile early and waits at the barrier
// while the younger one runs alone and cannot keep the pipe busy.
//
// LDS (160 KB): B tile ring of 3 slots (32 KB each) and, per group, a ring of
// 2 slots for its own half of the A tile (16 KB each; each group reads only its
// own rows).  All global -> LDS DMA is issued inside the read phases, between
// the LDS reads, so the MFMA phases are MFMAs only (a DMA instruction issued
// between 16-cycle MFMAs stalls the MFMA stream; the read phase has the slack):
//   group g, R(u): its A rows of tile u+1 and its half of B of tile u+2
//   (group 0: A rows 0-127, NN B k-rows 8-15 of each 16, NT B rows 0-127;
//    group 1: A rows 128-255, the other B k-rows / rows).
// A(u+1) goes to the A slot the group read in R(u-1); B(u+2) to the B slot
// both groups read in R(u-1), which the other group finished one interval
// before.  Waits (vmcnt counts a wave's DMA in issue order): at the end of
// R(u), for everything issued before R(u) -- B(u+1), which the other group
// reads after the next barrier; at the end of M(u), for A(u+1), which the
// group reads in R(u+1).  Each B half has two intervals to land, each A
// tile the rest of its read phase and one MFMA phase.
//
// Ragged edges: A (and NT's B) is read through buffer resources whose record
// count ends at row M (N), so rows past it load as zeros; NN's B columns past N
// are clamped (their products land in columns that are not stored).  K (per
// split-K partition) must be a multiple of 64 — pingpong_ok() checks it on the
// host.
//
// Output: full tiles with bf16 output (16-byte aligned Y) are staged through
// LDS by store_tile_bf16_staged (each wave's 128 x 64 block, written as whole
// 128-byte rows, 8 rows per store instruction); partial tiles, f32 output and
// split-K partial planes use store_block.
#pragma once
#include "gemm_bf16_kernel.h"

namespace t0mi {

// 16-byte buffer -> LDS DMA with range checking: lane i's 16 bytes at
// rsrc.base + soff + voff land at LDS byte address m0 + 16*i; lanes whose
// offset is at or beyond the record count write zeros.  Same tracking rules as
// lds_dma16.
__device__ __forceinline__ void lds_dma16_rsrc(u32x4 rsrc, uint32_t voff, uint32_t soff, uint32_t lds_byte_addr) {
  const uint32_t m0v = __builtin_amdgcn_readfirstlane(lds_byte_addr);
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %4\n\t"
      "buffer_load_dwordx4 %1, %2, %3 offen lds\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(voff), "s"(rsrc), "s"(soff), "s"(m0v)
      :);
}

// 16-byte global -> LDS DMA, address = uniform base (SGPR pair) + 32-bit lane offset.
__device__ __forceinline__ void lds_dma16_sv(const void* sbase, uint32_t voff, uint32_t lds_byte_addr) {
  const uint32_t m0v = __builtin_amdgcn_readfirstlane(lds_byte_addr);
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %3\n\t"
      "global_load_lds_dwordx4 %1, %2\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(voff), "s"(sbase), "s"(m0v)
      :);
}

// Raw buffer resource: 48-bit base, record count in bytes, gfx9 default flags.
__device__ __forceinline__ u32x4 make_rsrc(const void* base, uint32_t nbytes) {
  const uint64_t b = (uint64_t)base;
  u32x4 r;
  r.x = __builtin_amdgcn_readfirstlane((uint32_t)b);
  r.y = __builtin_amdgcn_readfirstlane((uint32_t)(b >> 32) & 0xffffu);
  r.z = __builtin_amdgcn_readfirstlane(nbytes);
  r.w = __builtin_amdgcn_readfirstlane(0x00020000u);
  return r;
}

// Host-side check of the ping-pong kernel's preconditions (the 256x256x64
// 2x4-wave configuration is assumed by the caller).
inline bool pingpong_ok(const GemmParams& p) {
  if (p.K == 0 || p.K % 64 != 0) return false;
  if (p.split_k > 1 && p.k_per_split % 64 != 0) return false;
  if (p.N < 8) return false;
  return true;
}

// NN: B = B[K,N] (ldb = N), LDS tile [64 k][256 n], K-contiguous operand by
// transpose reads.  NT: B = WT[N,K] (ldb = K), LDS tile [256 n][64 k] laid out
// and loaded like A (rows past N read zeros), fragments by ds_read_b128.
// X16: v_mfma_f32_16x16x32_bf16 (each wave 8 x 4 blocks of 16 x 16, 2 k-steps
// of 32 per tile) instead of v_mfma_f32_32x32x16_bf16 (4 x 2 blocks of 32 x 32,
// 4 k-steps of 16).  Same FLOPs, LDS bytes and DMA per tile and the same
// schedule; the 16x16x32 instruction reads and writes half the accumulator
// bytes per FLOP and draws less power, so the clock the power limit allows on
// this kernel is higher.
template <bool NN, bool X16>
__global__ __launch_bounds__(512) void gemm_bf16_pingpong_kernel(GemmParams p) {
  constexpr int BK = 64, BN = 256, TN = 64;
  constexpr int MB = X16 ? 16 : 32;            // MFMA block edge
  constexpr int FM = 128 / MB, FN = TN / MB;   // blocks per wave
  constexpr int KS = X16 ? 2 : 4;              // k-steps per 64-K tile
  constexpr int KG = 64 / MB;                  // lane groups = 16-byte k-chunks per k-step
  constexpr int KC = 8, NC = 32;
  constexpr int B_ELEMS = BN * BK, AH_ELEMS = 128 * BK;  // B tile, half A tile
  constexpr int NR = FM + (NN ? 2 * FN : FN);            // LDS reads per k-step
  constexpr int NMF = KS * FN * FM;                      // MFMAs per tile
  typedef float accv __attribute__((ext_vector_type(MB * MB / 64)));  // accumulators per lane
  __shared__ __attribute__((aligned(1024))) uint16_t smem[3 * B_ELEMS + 4 * AH_ELEMS];

  int tm, tn, part;
  tile_coords(p, tm, tn, part);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int g = wave >> 2, w4 = wave & 3;  // group, wave within the group
  const bool g0 = g == 0;
  const int wn = wave & 3;                 // 64-column slice of the tile
  const int m0 = tm * 256, n0 = tn * BN;
  const int kbeg = part * (int)p.k_per_split;
  int kend = kbeg + (int)p.k_per_split;
  if (kend > (int)p.K) kend = (int)p.K;
  const int nk = kend > kbeg ? (kend - kbeg) / BK : 0;
  const uint32_t smem_base = lds_addr(smem);
  const uint32_t a_slot0 = smem_base + (uint32_t)(3 * B_ELEMS * 2 + g * 2 * AH_ELEMS * 2);

  // ---- DMA addressing ------------------------------------------------------
  // Wave w4 of group g fills, per tile, 1 KB blocks w4 + 4j (j = 0..3) of its
  // half of the A tile (8 rows x 64 K each) and 4 blocks of the B tile: NT
  // blocks 16g + w4 + 4j (8 n-rows x 64 K), NN blocks 4g + w4 + 8j (2 k-rows x
  // 256 columns: k-rows 8g + 2w4 + 16j and the next).  The swizzles depend on
  // the row modulo 32 (swz) or 8 (rot16) (A, NT B) or on bits 0, 1 and 3 of
  // the k-row (NN B),
  // which j does not change, so one lane offset serves all four loads of a
  // kind; j and the tile move the uniform base.
  uint32_t a_voff, b_voff;
  {
    int row, lc;  // block w4 of the group's half tile: rows 8 w4 .. 8 w4 + 7
    kc_dma_chunk<KC, X16>(w4 * 64 + lane, &row, &lc);
    a_voff = (uint32_t)(row * (int)p.lda + lc * 8) * 2u;
    if constexpr (NN) {
      int brow, blc;  // block 4g + w4: k-rows 2 (4g + w4) and the next
      nn_dma_chunk<NC, X16>((4 * g + w4) * 64 + lane, &brow, &blc);
      int gn = n0 + blc * 8;
      gn = gn < (int)p.N ? gn : (int)p.N - 8;
      b_voff = (uint32_t)(brow * (int)p.ldb + gn) * 2u;
    } else {
      b_voff = (uint32_t)(row * (int)p.ldb + lc * 8) * 2u;
    }
  }
  // A through four buffer resources, one per 32-row block j of this group's
  // half, fixed for the whole K loop: base = row block start, record count =
  // bytes up to the end of row M-1 (0 for blocks past M), so lanes on rows >= M
  // read zeros.  The tile's K position goes in the scalar offset operand; valid
  // rows stay in range and rows past M out of range whether or not the range
  // check counts that operand (k0 + 64 <= K <= lda).
  const uint64_t a_row_bytes = (uint64_t)p.lda * 2u;
  const uint64_t b_row_bytes = (uint64_t)p.ldb * 2u;
  // Resource based at row r0 of a row-major [rows][ld] operand whose record
  // count ends with row rows-1 (0 when r0 >= rows; the base is then never
  // dereferenced).
  auto block_rsrc = [](const uint16_t* base, int rows, int r0, uint64_t row_bytes) {
    const int left_rows = rows - r0;
    const uint64_t left = left_rows <= 0 ? 0u : (uint64_t)left_rows * row_bytes;
    return make_rsrc((const char*)base + (uint64_t)r0 * row_bytes, left > 0x7fffffffu ? 0x7fffffffu : (uint32_t)left);
  };
  u32x4 a_rs[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) a_rs[j] = block_rsrc(p.a, (int)p.M, m0 + g * 128 + j * 32, a_row_bytes);
  // NT: B rows (n) the same way, so rows past N read zeros.
  u32x4 b_rs[NN ? 1 : 4];
  if constexpr (!NN) {
#pragma unroll
    for (int j = 0; j < 4; ++j) b_rs[j] = block_rsrc(p.b, (int)p.N, n0 + g * 128 + j * 32, b_row_bytes);
  }
  const uint32_t b_lds0 = smem_base + (NN ? 4 * g + w4 : 16 * g + w4) * 1024;
  const uint32_t a_lds0 = a_slot0 + w4 * 1024;
  // DMA j of tile t: j < 4 from A row block j; else NN: the wave's B block
  // 4g + w4 + 8(j-4), i.e. k-rows 8g + 2w4 + 16(j-4) and the next; NT: B row
  // block j-4.
  auto dma = [&](int t, const char* b_tile, auto jc) {
    constexpr int j = decltype(jc)::value;
    if constexpr (j < 4) {
      lds_dma16_rsrc(a_rs[j], a_voff, (uint32_t)(kbeg + t * BK) * 2u,
                     a_lds0 + (uint32_t)((t & 1) * AH_ELEMS * 2) + 4 * j * 1024);
    } else if constexpr (NN) {
      lds_dma16_sv(b_tile + (uint64_t)(j - 4) * 16u * b_row_bytes, b_voff,
                   b_lds0 + (uint32_t)((t % 3) * B_ELEMS * 2) + 8 * (j - 4) * 1024);
    } else {
      lds_dma16_rsrc(b_rs[j - 4], b_voff, (uint32_t)(kbeg + t * BK) * 2u,
                     b_lds0 + (uint32_t)((t % 3) * B_ELEMS * 2) + 4 * (j - 4) * 1024);
    }
  };
  auto b_tile_of = [&](int t) { return NN ? (const char*)p.b + (uint64_t)(kbeg + t * BK) * b_row_bytes : nullptr; };

  // ---- LDS -> fragments ------------------------------------------------------
  // K-contiguous operands: lane l reads row l % MB of the block, k-chunk
  // KG ks + l / MB.  The blocks of a wave are MB rows apart and the swizzle
  // repeats every 32 (swz) or 8 (rot16) rows, so one offset per k-step serves
  // every block.
  const int lrow = lane % MB, lgrp = lane / MB;
  int a_off[KS], b_off[NN ? 1 : KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    a_off[ks] = kc_slot<KC, X16>(lrow, ks * KG + lgrp) * 8;
    if constexpr (!NN) b_off[ks] = kc_slot<KC, X16>(wn * TN + lrow, ks * KG + lgrp) * 8;
  }
  // NN transpose reads: lane l addresses k-row nn_krow0 + 4h (+ the k-step's
  // base) and 4 columns at nn_col0 (+ the block's base).
  const int tg = lane >> 4, ti = lane & 15;
  const int nn_krow0 = X16 ? x16_krow(lane, 0) : 8 * (tg >> 1) + (ti >> 2);
  const int nn_col0 = wn * TN + (X16 ? x16_col(lane) : 16 * (tg & 1) + 4 * (ti & 3));
  const int nn_sw = swz_nn<NC, X16>(nn_krow0);
  // Loop-invariant element offset of each block's transpose reads (k-row
  // nn_krow0 of the tile, the block's columns): the k-step and half then go in
  // the instruction's offset field, so a block's four reads share one address.
  int nn_fo[FN];
#pragma unroll
  for (int fn = 0; fn < FN; ++fn) nn_fo[fn] = nn_krow0 * BN + nn_col_off(nn_col0 + fn * MB, nn_sw);

  bf16x8 xa[KS][FM], xb[KS][FN];
  i16x4 tr[KS][FN][2];
  auto read_one = [&](const uint16_t* As, const uint16_t* Bs, auto ic) {
    constexpr int i = decltype(ic)::value;
    constexpr int ks = i / NR, r = i % NR;
    if constexpr (r < FM) {
      xa[ks][r] = *(const bf16x8*)(As + a_off[ks] + r * MB * BK);
    } else if constexpr (!NN) {
      xb[ks][r - FM] = *(const bf16x8*)(Bs + b_off[ks] + (r - FM) * MB * BK);
    } else {
      constexpr int fn = (r - FM) / 2, h = (r - FM) % 2;
      tr[ks][fn][h] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) i16x4*)(Bs + nn_fo[fn] + (ks * (X16 ? 32 : 16) + 4 * h) * BN));
      if constexpr (h == 1)
        xb[ks][fn] = __builtin_bit_cast(bf16x8, __builtin_shufflevector(tr[ks][fn][0], tr[ks][fn][1], 0, 1, 2, 3,
                                                                        4, 5, 6, 7));
    }
  };

  accv acc[FN][FM];
#pragma unroll
  for (int fn = 0; fn < FN; ++fn)
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int r = 0; r < MB * MB / 64; ++r) acc[fn][fm][r] = 0.0f;

  const uint16_t* a_slots = smem + 3 * B_ELEMS + g * 2 * AH_ELEMS;
  // R(u): the tile's fragments, with DMA j (A of tile u+1 for j < 4 when DA,
  // B of tile u+2 for 4 <= j < 8 - BMM when DB) issued after read RD * j + 1;
  // then the reads are waited for, and this wave's DMA issued before R(u)
  // (its B half of tile u+1): vmcnt may keep only the loads issued here.
  // BMM: B loads issued from the MFMA phase instead.  Each stalls the MFMA
  // stream for ~26 cycles; with one add per fragment address every read phase
  // ends well inside the other group's MFMA phase (NN ~800 of ~1080 cycles), so
  // all loads stay in the read phases (one NN load in the MFMA phase measured
  // 0.8 % slower at 4096^3).  Kept as a parameter for read phases that grow.
  constexpr int BMM = 0;
  constexpr int NRD = KS * NR, RD = NRD / 8;
  auto read_phase = [&](int u, auto da_c, auto db_c) {
    constexpr bool DA = decltype(da_c)::value, DB = decltype(db_c)::value;
    // The ring slots as wave-uniform scalars: every fragment address is then
    // one add of a loop-invariant lane offset and the slot, with the rest in
    // the instruction's offset field.  (Left to the compiler, u % 3 is strength-
    // reduced across iterations into two per-iteration terms, and the 16
    // transpose reads took two VALU instructions each: 35 per read phase
    // against 6, 2.7 % of the 4096^3 NN time.)
    const uint16_t* As = a_slots + __builtin_amdgcn_readfirstlane((int)(u & 1)) * AH_ELEMS;
    const uint16_t* Bs = smem + __builtin_amdgcn_readfirstlane((int)(u % 3)) * B_ELEMS;
    const char* b_tile = DB ? b_tile_of(u + 2) : nullptr;
    static_for<NRD>([&](auto ic) {
      constexpr int i = decltype(ic)::value;
      read_one(As, Bs, ic);
      if constexpr (i % RD == 1) {
        constexpr int j = i / RD;
        if constexpr (j < 4 && DA) dma(u + 1, nullptr, std::integral_constant<int, j>{});
        if constexpr (j >= 4 && j < 8 - BMM && DB) dma(u + 2, b_tile, std::integral_constant<int, j>{});
      }
      __builtin_amdgcn_sched_barrier(0);
    });
    wait_lgkmcnt0();
    wait_vmcnt<(DA ? 4 : 0) + (DB ? 4 - BMM : 0)>();
  };
  // M(u): the tile's MFMAs in k-step order (the generic kernel's accumulation
  // order), with the last BMM B loads of tile u+2 in the middle; then this
  // wave's A of tile u+1 is waited for (its B of tile u+2 may stay in flight).
  auto mfma_phase = [&](int u, auto db_c) {
    constexpr bool DB = decltype(db_c)::value;
    const char* b_tile = DB && BMM > 0 ? b_tile_of(u + 2) : nullptr;
    static_for<NMF>([&](auto ic) {
      constexpr int i = decltype(ic)::value;
      constexpr int ks = i / (FN * FM), fn = (i / FM) % FN, fm = i % FM;
      if constexpr (X16)
        acc[fn][fm] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xb[ks][fn], xa[ks][fm], acc[fn][fm], 0, 0, 0);
      else
        acc[fn][fm] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xb[ks][fn], xa[ks][fm], acc[fn][fm], 0, 0, 0);
      if constexpr (BMM > 0 && DB && i % (NMF / BMM) == NMF / BMM / 2)
        dma(u + 2, b_tile, std::integral_constant<int, 8 - BMM + i / (NMF / BMM)>{});
      __builtin_amdgcn_sched_barrier(0);
    });
    wait_vmcnt<DB ? 4 : 0>();
  };
  auto bar = []() {
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
  };
  using True = std::integral_constant<bool, true>;
  using False = std::integral_constant<bool, false>;

  // Prologue: A and B of tile 0 and B of tile 1; tile 0 waited for.  Every
  // wave then runs R(u) bar M(u) bar; group 1 starts one barrier later and
  // group 0 ends with one extra, so both pass 2*nk + 1 barriers.
  if (nk > 0) static_for<8>([&](auto jc) { dma(0, b_tile_of(0), jc); });
  if (nk > 1) {
    const char* b1 = b_tile_of(1);
    static_for<4>([&](auto jc) { dma(1, b1, std::integral_constant<int, 4 + decltype(jc)::value>{}); });
    wait_vmcnt<4>();  // tile 0 landed; B of tile 1 is waited for at the end of R(0)
  } else {
    wait_vmcnt<0>();
  }
  bar();
  if (!g0) bar();
  int u = 0;
  for (; u + 2 < nk; ++u) {
    read_phase(u, True{}, True{});
    bar();
    mfma_phase(u, True{});
    bar();
  }
  if (u + 1 < nk) {
    read_phase(u, True{}, False{});
    bar();
    mfma_phase(u, False{});
    bar();
    ++u;
  }
  if (u < nk) {
    read_phase(u, False{}, False{});
    bar();
    mfma_phase(u, False{});
  }
  if (g0) bar();
  // Here every wave has finished its LDS reads and DMA (group 0 met group 1
  // at the barrier after group 1's last read phase).

  // ---- epilogue ------------------------------------------------------------
  const bool partial_plane = p.split_k > 1;
  char* ybase = (char*)p.y + (partial_plane ? (size_t)part * p.y_split_stride : 0);
  const int row0 = m0 + g * 128;
  const int col0 = n0 + wn * TN;
  if (!partial_plane && p.out_bf16 && m0 + 256 <= (int)p.M && n0 + 256 <= (int)p.N && ((uintptr_t)p.y & 15) == 0) {
    if constexpr (X16)
      store_tile_bf16_staged16<FM>(p, acc, (char*)smem + wave * 16384, ybase, row0, col0, lane);
    else
      store_tile_bf16_staged<FM, FN>(p, acc, (char*)smem + wave * 16384, ybase, row0, col0, lane);
  } else {
    static_for<FM>([&](auto fmc) {
      constexpr int fm = decltype(fmc)::value;
      const int m = row0 + fm * MB + lrow;
      if (m < (int)p.M) {
        static_for<FN>([&](auto fnc) {
          constexpr int fn = decltype(fnc)::value;
          if constexpr (X16)
            store_block16(p, acc[fn][fm], ybase, m, col0 + fn * 16 + lgrp * 4, partial_plane);
          else
            store_block(p, acc[fn][fm], ybase, m, col0 + fn * 32 + lgrp * 4, partial_plane);
        });
      }
    });
  }
}

}  // namespace t0mi
