// gemm_bf16_kernel.h — gfx950 bf16 GEMM kernel template (MFMA 32x32x16, fp32 accumulate).
//
// Replaces the RDNA WMMA kernels that the reference generates at run time:
//   src/t0/gemm_gen.rs:668-1438   (generate_lds_db)
//   src/t0/tile_ir.rs:887-4250    (lower_gemm)
// Same math — Y[M,N] = X[M,K] . B, bf16 inputs, fp32 accumulation — laid out
// for CDNA4:
//   * global -> LDS with global_load_lds_dwordx4 (no VGPR staging, no ds_write):
//     each wave instruction fills one contiguous 1 KB LDS block, so the LDS
//     swizzle is applied on the global side (each lane fetches the chunk that
//     belongs at its LDS slot);
//   * a ring of S = 2..5 LDS stages, one barrier per K tile; waits count
//     outstanding DMA instructions (vmcnt) so up to S-1 tiles are in flight,
//     and with S >= 3 each tile's loads are spread over the previous tile's
//     k-steps; the first fragments of tile it+1 are read during tile it's last
//     k-step;
//   * v_mfma_f32_32x32x16_bf16 with the A and B fragments of the next k-step
//     read from LDS while the current k-step's MFMAs run.
//
// Layouts:
//   A  = X[M,K] row-major (lda = K); LDS tile [BM][BK], 16-byte chunks XOR-swizzled
//        per row, fragments read with ds_read_b128.
//   NT: B = WT[N,K] row-major (ldb = K) — the reference's only implemented layout;
//        LDS tile [BN][BK] like A.
//   NN: B = B[K,N] row-major (ldb = N) — BASELINE.json's layout.  The LDS tile is
//        stored as loaded, [BK][BN], and the K-contiguous MFMA operand is formed
//        by ds_read_b64_tr_b16 (gfx950 transpose read): within a 16-lane group,
//        lane l receives element (l % 4) of the 8-byte chunks addressed by lanes
//        4e + l/4, e = 0..3.
// Output: f32 or bf16 (round to nearest even), after an optional fused epilogue chain.
// Split-K: partition p covers K range [p*Kp, (p+1)*Kp) and writes its own f32
// plane at Y + p*y_split_stride (src/t0/gemm_gen.rs:760-793).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <utility>

#include "epi_chain.h"
#include "index_maps.h"

namespace t0mi {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef short i16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float epi_apply(float v, float bias, const EpiChain& e) {
#pragma unroll 1
  for (uint32_t i = 0; i < e.n; ++i) {
    switch ((e.ops >> (4 * i)) & 0xFu) {
      case EOP_BIAS: v += bias; break;
      case EOP_SCALE: v *= e.scale; break;
      case EOP_RELU: v = fmaxf(v, 0.0f); break;
      case EOP_SILU: v = v * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-v * 1.44269504f)); break;
      case EOP_GELU: v = v * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-(1.702f * v) * 1.44269504f)); break;
      case EOP_ABS: v = fabsf(v); break;
      case EOP_NEG: v = -v; break;
      default: v = fminf(fmaxf(v, e.lo), e.hi); break;
    }
  }
  return v;
}

struct GemmParams {
  const uint16_t* a;      // X [M,K] bf16
  const uint16_t* b;      // WT [N,K] (NT) or B [K,N] (NN) bf16
  void* y;                // output
  const float* bias;      // [N] f32 or null
  uint32_t M, N, K;
  uint32_t lda, ldb, ldy; // element strides
  uint32_t tiles_m, tiles_n;
  uint32_t split_k;       // partitions (power of two)
  uint32_t k_per_split;   // K range per partition (multiple of 8)
  uint64_t y_split_stride;// bytes between partial planes (split_k > 1)
  uint32_t out_bf16;      // 1: bf16 RNE store, 0: f32 store
  EpiChain epi;           // fused epilogue (final planes only)
  uint32_t swap_grid;     // reference grid axis convention (informational)
  uint32_t xcd_remap;     // 1: make tiles that share an XCD (L2) contiguous
  uint32_t stream_out;    // 1: staged bf16 stores are non-temporal (set when all
                          // workgroups run at once, so every store comes at the end)
};

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  // v_cvt_pk_bf16_f32 rounds to nearest even (gfx950).
  __bf16 h = (__bf16)f;
  return __builtin_bit_cast(uint16_t, h);
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
// Two floats -> packed bf16 pair (lo in bits 0..15), RNE: one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t));
}

// Calls f(std::integral_constant<int, 0>) .. f(std::integral_constant<int, N-1>):
// a loop the compiler cannot leave rolled, for register arrays that must only
// be indexed by constants.
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// Stores one 32x32 accumulator block.  Lane l holds rows m (one per lane) and
// columns n + 8*g + {0..3}, g = 0..3 (n already includes 4*(l >> 5)).  Columns
// at or beyond N are skipped (the tile's N tail).
__device__ __forceinline__ void store_block(const GemmParams& p, const f32x16& a, char* ybase, int m, int n,
                                            bool partial_plane) {
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int nc = n + g * 8;
    if (nc >= (int)p.N) continue;
    float v0 = a[g * 4 + 0], v1 = a[g * 4 + 1], v2 = a[g * 4 + 2], v3 = a[g * 4 + 3];
    if (!partial_plane && p.epi.n) {
      f32x4 bv = {0.0f, 0.0f, 0.0f, 0.0f};
      if (p.bias) bv = f32x4{p.bias[nc], p.bias[nc + 1], p.bias[nc + 2], p.bias[nc + 3]};
      v0 = epi_apply(v0, bv.x, p.epi);
      v1 = epi_apply(v1, bv.y, p.epi);
      v2 = epi_apply(v2, bv.z, p.epi);
      v3 = epi_apply(v3, bv.w, p.epi);
    }
    if (!partial_plane && p.out_bf16) {
      u32x2 o;
      o.x = pack_bf16x2(v0, v1);
      o.y = pack_bf16x2(v2, v3);
      *(u32x2*)((uint16_t*)ybase + (size_t)m * p.ldy + nc) = o;
    } else {
      f32x4 o = {v0, v1, v2, v3};
      *(f32x4*)((float*)ybase + (size_t)m * p.ldy + nc) = o;
    }
  }
}

// swz / swz_nn (the LDS swizzles) and the DMA chunk maps: index_maps.h.

// Linear work item `lin` of `nwg` -> (tile_m, tile_n, partition).
// Workgroups are dispatched round-robin over the 8 XCDs; with xcd_remap the
// items that run on the same XCD (same L2) are made contiguous, then tiles are
// walked in groups of GROUP_M tile rows so each XCD works on a compact block
// of output tiles (shared A rows / B columns stay L2-resident).  A persistent
// kernel whose grid is a multiple of 8 keeps every item of a workgroup on that
// workgroup's XCD, so the same numbering applies to its loop.
__device__ __forceinline__ void tile_coords_lin(uint32_t lin, uint32_t nwg, uint32_t tiles_m, uint32_t tiles_n,
                                                uint32_t xcd_remap, int& tm, int& tn, int& part) {
  if (xcd_remap && (nwg % 8u) == 0u) lin = (lin % 8u) * (nwg / 8u) + lin / 8u;
  uint32_t tiles = tiles_m * tiles_n;
  part = (int)(lin / tiles);
  uint32_t t = lin % tiles;
  const uint32_t GROUP_M = 4;
  uint32_t group_size = GROUP_M * tiles_n;
  uint32_t g = t / group_size;
  uint32_t first_m = g * GROUP_M;
  uint32_t gm = tiles_m - first_m < GROUP_M ? tiles_m - first_m : GROUP_M;
  uint32_t r = t % group_size;
  tm = (int)(first_m + r % gm);
  tn = (int)(r / gm);
}

// The one-shot kernels: item = linear workgroup id.
__device__ __forceinline__ void tile_coords_of(uint32_t tiles_m, uint32_t tiles_n, uint32_t xcd_remap, int& tm,
                                               int& tn, int& part) {
  tile_coords_lin(blockIdx.x + blockIdx.y * gridDim.x, gridDim.x * gridDim.y, tiles_m, tiles_n, xcd_remap, tm, tn,
                  part);
}

__device__ __forceinline__ void tile_coords(const GemmParams& p, int& tm, int& tn, int& part) {
  tile_coords_of(p.tiles_m, p.tiles_n, p.xcd_remap, tm, tn, part);
}

// 16-byte global -> LDS DMA: lane i's 16 bytes land at LDS byte address
// m0 + 16*i.  Issued through inline asm so the compiler does not track it; the
// kernel waits for it explicitly (vmcnt + barrier) before the stage is read.
// No "memory" clobber: the DMA always targets a stage that no instruction
// between two barriers reads, so LDS reads may be scheduled across it; being
// volatile, it keeps its order against the barrier and waitcnt builtins.
__device__ __forceinline__ void lds_dma16(const void* g, uint32_t lds_byte_addr) {
  const uint32_t m0v = __builtin_amdgcn_readfirstlane(lds_byte_addr);
  uint32_t saved;
  // m0 is a compiler-reserved register: keep its value across the statement.
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "global_load_lds_dwordx4 %1, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(g), "s"(m0v)
      :);
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(size_t)(const __attribute__((address_space(3))) void*)p;
}

// s_waitcnt vmcnt(N) (gfx9 encoding: vmcnt low bits [3:0], high bits [15:14];
// expcnt and lgkmcnt left at their maxima).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N <= 63, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// s_waitcnt lgkmcnt(0) (vmcnt and expcnt left at their maxima).
__device__ __forceinline__ void wait_lgkmcnt0() { __builtin_amdgcn_s_waitcnt(0xF | (0x7 << 4) | (0x3 << 14)); }

// 16 zero bytes: the DMA source of K-tail chunks, so every K tile issues the
// same number of DMA loads (the vmcnt arithmetic below relies on it).
static __device__ __attribute__((aligned(16))) const uint32_t g_zero16[4] = {0u, 0u, 0u, 0u};

// Stores a wave's FM*32 x FN*32 accumulator block as bf16 through a private
// LDS block `st` (FM*32 * FN*32 * 2 bytes): each lane writes its 8-byte row
// pieces with the 16-byte chunks of every row XOR-swizzled by the row index,
// then the block is read back so that each 16-byte-per-lane store instruction
// writes 512 / (FN*32) whole rows of FN*64 contiguous bytes (the direct stores
// of store_block write 16 bytes into each of 32 rows).  The epilogue chain is
// applied before the conversion.  Caller's contract: a full tile (all rows and
// columns in range), bf16 output, not a partial plane, 16-byte aligned Y, and
// no pending LDS reads or DMA into `st`.
template <int FM, int FN>
__device__ __forceinline__ void store_tile_bf16_staged(const GemmParams& p, const f32x16 (&acc)[FN][FM], char* st,
                                                       char* ybase, int row0, int col0, int lane) {
  constexpr int TN = FN * 32, CH = TN / 8, RPI = 64 / CH;  // 16-byte chunks per row, rows per store
  const int lrow = lane & 31, lhalf = lane >> 5;
  static_for<FM>([&](auto fmc) {
    constexpr int fm = decltype(fmc)::value;
    static_for<FN>([&](auto fnc) {
      constexpr int fn = decltype(fnc)::value;
      const int r = fm * 32 + lrow;
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        float v0 = acc[fn][fm][gq * 4 + 0], v1 = acc[fn][fm][gq * 4 + 1];
        float v2 = acc[fn][fm][gq * 4 + 2], v3 = acc[fn][fm][gq * 4 + 3];
        if (p.epi.n) {
          const int nc = col0 + fn * 32 + gq * 8 + lhalf * 4;
          f32x4 bv = {0.0f, 0.0f, 0.0f, 0.0f};
          if (p.bias) bv = f32x4{p.bias[nc], p.bias[nc + 1], p.bias[nc + 2], p.bias[nc + 3]};
          v0 = epi_apply(v0, bv.x, p.epi);
          v1 = epi_apply(v1, bv.y, p.epi);
          v2 = epi_apply(v2, bv.z, p.epi);
          v3 = epi_apply(v3, bv.w, p.epi);
        }
        const int c = fn * 4 + gq;  // 16-byte chunk of the row
        u32x2 o;
        o.x = pack_bf16x2(v0, v1);
        o.y = pack_bf16x2(v2, v3);
        *(u32x2*)(st + r * TN * 2 + ((c ^ (r & (CH - 1))) * 16) + lhalf * 8) = o;
      }
    });
  });
  wait_lgkmcnt0();  // the block is read back only by the wave that wrote it
  const int rr = lane / CH, cc = lane % CH;
  char* yrow = ybase + ((size_t)(row0 + rr) * p.ldy + col0 + cc * 8) * 2;
#pragma unroll
  for (int i = 0; i < FM * 32 / RPI; ++i) {
    const int r = i * RPI + rr;
    const u32x4 v = *(const u32x4*)(st + r * TN * 2 + ((cc ^ (r & (CH - 1))) * 16));
    u32x4* dst = (u32x4*)(yrow + (size_t)i * RPI * p.ldy * 2);
    if (p.stream_out)
      __builtin_nontemporal_store(v, dst);
    else
      *dst = v;
  }
}

// Stores one 16x16 accumulator block of v_mfma_f32_16x16x32_bf16: lane l holds
// row m (= block row l % 16) and columns n .. n+3 (n already includes
// 4*(l >> 4)).  Columns at or beyond N are skipped (the tile's N tail).
__device__ __forceinline__ void store_block16(const GemmParams& p, const f32x4& a, char* ybase, int m, int n,
                                              bool partial_plane) {
  if (n >= (int)p.N) return;
  float v0 = a[0], v1 = a[1], v2 = a[2], v3 = a[3];
  if (!partial_plane && p.epi.n) {
    f32x4 bv = {0.0f, 0.0f, 0.0f, 0.0f};
    if (p.bias) bv = f32x4{p.bias[n], p.bias[n + 1], p.bias[n + 2], p.bias[n + 3]};
    v0 = epi_apply(v0, bv.x, p.epi);
    v1 = epi_apply(v1, bv.y, p.epi);
    v2 = epi_apply(v2, bv.z, p.epi);
    v3 = epi_apply(v3, bv.w, p.epi);
  }
  if (!partial_plane && p.out_bf16) {
    u32x2 o;
    o.x = pack_bf16x2(v0, v1);
    o.y = pack_bf16x2(v2, v3);
    *(u32x2*)((uint16_t*)ybase + (size_t)m * p.ldy + n) = o;
  } else {
    f32x4 o = {v0, v1, v2, v3};
    *(f32x4*)((float*)ybase + (size_t)m * p.ldy + n) = o;
  }
}

// store_tile_bf16_staged for a wave's FM*16 x 64 block of 16x16 accumulators
// (FN = 4): each lane's 8-byte row pieces go to a private LDS block `st`
// (FM*16 rows of 128 bytes, chunks swizzled by stage_swz16), which is read back
// as 8 whole rows per 16-byte-per-lane store instruction.  Same contract.
template <int FM>
__device__ __forceinline__ void store_tile_bf16_staged16(const GemmParams& p, const f32x4 (&acc)[4][FM], char* st,
                                                         char* ybase, int row0, int col0, int lane) {
  constexpr int TN = 64, CH = 8, RPI = 8;  // 16-byte chunks per row, rows per store instruction
  const int lr = lane & 15, lq = lane >> 4;
  static_for<FM>([&](auto fmc) {
    constexpr int fm = decltype(fmc)::value;
    const int r = fm * 16 + lr;
    static_for<4>([&](auto fnc) {
      constexpr int fn = decltype(fnc)::value;
      float v0 = acc[fn][fm][0], v1 = acc[fn][fm][1], v2 = acc[fn][fm][2], v3 = acc[fn][fm][3];
      if (p.epi.n) {
        const int nc = col0 + fn * 16 + lq * 4;
        f32x4 bv = {0.0f, 0.0f, 0.0f, 0.0f};
        if (p.bias) bv = f32x4{p.bias[nc], p.bias[nc + 1], p.bias[nc + 2], p.bias[nc + 3]};
        v0 = epi_apply(v0, bv.x, p.epi);
        v1 = epi_apply(v1, bv.y, p.epi);
        v2 = epi_apply(v2, bv.z, p.epi);
        v3 = epi_apply(v3, bv.w, p.epi);
      }
      const int c = fn * 2 + (lq >> 1);  // 16-byte chunk of the row
      u32x2 o;
      o.x = pack_bf16x2(v0, v1);
      o.y = pack_bf16x2(v2, v3);
      *(u32x2*)(st + r * TN * 2 + ((c ^ stage_swz16(r)) * 16) + (lq & 1) * 8) = o;
    });
  });
  wait_lgkmcnt0();  // the block is read back only by the wave that wrote it
  const int rr = lane / CH, cc = lane % CH;
  char* yrow = ybase + ((size_t)(row0 + rr) * p.ldy + col0 + cc * 8) * 2;
#pragma unroll
  for (int i = 0; i < FM * 16 / RPI; ++i) {
    const int r = i * RPI + rr;
    const u32x4 v = *(const u32x4*)(st + r * TN * 2 + ((cc ^ stage_swz16(r)) * 16));
    u32x4* dst = (u32x4*)(yrow + (size_t)i * RPI * p.ldy * 2);
    if (p.stream_out)
      __builtin_nontemporal_store(v, dst);
    else
      *dst = v;
  }
}

template <int BM, int BN, int BK, int WM, int WN, int S, bool NN>
struct GemmTile {
  static constexpr int NWAVES = WM * WN;
  static constexpr int NTHR = NWAVES * 64;
  static constexpr int TM = BM / WM, TN = BN / WN;  // per-wave tile
  static constexpr int FM = TM / 32, FN = TN / 32;  // 32x32 MFMA blocks per wave
  static constexpr int KC = BK / 8;                 // 16-byte chunks per K-contiguous row
  static constexpr int KS = BK / 16;                // MFMA k-steps per tile
  static constexpr int NC = BN / 8;                 // NN: 16-byte chunks per B row
  static constexpr int A_ELEMS = BM * BK, B_ELEMS = BN * BK;
  static constexpr int A_BLOCKS = A_ELEMS * 2 / 1024;  // 1 KB LDS blocks per A tile
  static constexpr int B_BLOCKS = B_ELEMS * 2 / 1024;
  static_assert(TM % 32 == 0 && TN % 32 == 0, "wave tile must be a multiple of 32x32");
  static_assert(BK == 16 || BK == 32 || BK == 64, "tile_k must be 16, 32 or 64");
  static_assert((A_ELEMS * 2) % 1024 == 0 && (B_ELEMS * 2) % 1024 == 0, "tiles must be whole 1 KB blocks");
  static_assert(!NN || NC >= 8, "NN tiles need tile_n >= 64");
  static_assert(S >= 2 && S <= 5, "2..5 LDS stages");
  // Waiting for one tile by count (vmcnt) needs every wave to issue the same
  // number of DMA loads per tile; other splits wait for all loads.
  static constexpr bool EVEN = A_BLOCKS % NWAVES == 0 && B_BLOCKS % NWAVES == 0;
  static constexpr int LPT = A_BLOCKS / NWAVES + B_BLOCKS / NWAVES;  // DMA loads per wave per tile
  static_assert(S == 2 || EVEN, "more than two stages need an even DMA split");
  static_assert(!EVEN || LPT * (S - 1) <= 63, "vmcnt range");
};

// One output tile (tm, tn) of K partition `part`: the whole kernel body, called
// once by gemm_bf16_kernel and in a loop by the persistent kernel.
template <int BM, int BN, int BK, int WM, int WN, int S, bool NN>
__device__ __forceinline__ void gemm_bf16_tile(const GemmParams& p, int tm, int tn, int part) {
  using T = GemmTile<BM, BN, BK, WM, WN, S, NN>;
  constexpr int FM = T::FM, FN = T::FN, KC = T::KC, KS = T::KS, NC = T::NC;
  constexpr int TM = T::TM, TN = T::TN;
  constexpr int A_ELEMS = T::A_ELEMS, B_ELEMS = T::B_ELEMS;

  constexpr int BUF = A_ELEMS + B_ELEMS;  // elements per LDS stage (A tile then B tile)
  __shared__ __attribute__((aligned(1024))) uint16_t smem[S * BUF];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int m0 = tm * BM, n0 = tn * BN;
  const int kbeg = part * (int)p.k_per_split;
  int kend = kbeg + (int)p.k_per_split;
  if (kend > (int)p.K) kend = (int)p.K;
  const int nk = kend > kbeg ? (kend - kbeg + BK - 1) / BK : 0;

  // ---- global -> LDS ------------------------------------------------------
  // Wave w fills 1 KB blocks w, w + NWAVES, ...; lane l writes chunk l of its
  // block, fetching the global chunk that the swizzle assigns to that slot.
  // Source pointers are formed once for tile 0 and stepped by a constant per
  // tile; chunks past the end of the K range (last tile only, checked only
  // when that tile is loaded) read 16 zero bytes instead, so every tile issues
  // the same number of DMA loads.
  constexpr int NA = (T::A_BLOCKS + T::NWAVES - 1) / T::NWAVES;
  constexpr int NB = (T::B_BLOCKS + T::NWAVES - 1) / T::NWAVES;
  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
  const uint32_t smem_base = lds_addr(smem);
  const int kspan = kend - kbeg;
  const uint16_t* a_src[NA];
  const uint16_t* b_src[NB];
  int a_kofs[NA], b_kofs[NB];  // K offset of the lane's chunk inside a tile
#pragma unroll
  for (int j = 0; j < NA; ++j) {
    int row, lc;
    kc_dma_chunk<KC>((wave_s + j * T::NWAVES) * 64 + lane, &row, &lc);
    int gr = m0 + row;
    gr = gr < (int)p.M ? gr : (int)p.M - 1;
    a_src[j] = p.a + (size_t)gr * p.lda + kbeg + lc * 8;
    a_kofs[j] = lc * 8;
  }
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    const int q = (wave_s + j * T::NWAVES) * 64 + lane;
    if constexpr (!NN) {
      int row, lc;
      kc_dma_chunk<KC>(q, &row, &lc);
      int gr = n0 + row;
      gr = gr < (int)p.N ? gr : (int)p.N - 1;
      b_src[j] = p.b + (size_t)gr * p.ldb + kbeg + lc * 8;
      b_kofs[j] = lc * 8;
    } else {
      int row, lc;  // row = k within the tile
      nn_dma_chunk<NC>(q, &row, &lc);
      int gn = n0 + lc * 8;
      gn = gn < (int)p.N ? gn : (int)p.N - 8;
      b_src[j] = p.b + (size_t)(kbeg + row) * p.ldb + gn;
      b_kofs[j] = row;
    }
  }
  const size_t b_step = NN ? (size_t)BK * p.ldb : (size_t)BK;
  // DMA load j of tile t (j < NA: A block, else B block) into `stage`.
  // CHECK: the tile may end past the K range (only the last tile can).
  auto dma_one = [&](int t, int stage, auto jc, auto check_c) {
    constexpr int j = decltype(jc)::value;
    constexpr bool CHECK = decltype(check_c)::value;
    const uint32_t a_lds = smem_base + (uint32_t)(stage * BUF * 2);
    const int krem = kspan - t * BK;
    if constexpr (j < NA) {
      const int blk = wave_s + j * T::NWAVES;
      if (T::A_BLOCKS % T::NWAVES != 0 && blk >= T::A_BLOCKS) return;
      const void* src = a_src[j] + (size_t)t * BK;
      if (CHECK && a_kofs[j] >= krem) src = g_zero16;
      lds_dma16(src, a_lds + blk * 1024);
    } else {
      const int blk = wave_s + (j - NA) * T::NWAVES;
      if (T::B_BLOCKS % T::NWAVES != 0 && blk >= T::B_BLOCKS) return;
      const void* src = b_src[j - NA] + (size_t)t * b_step;
      if (CHECK && b_kofs[j - NA] >= krem) src = g_zero16;
      lds_dma16(src, a_lds + (uint32_t)(A_ELEMS * 2) + blk * 1024);
    }
  };
  auto load_tile = [&](int t, int stage) {
    const uint32_t a_lds = smem_base + (uint32_t)(stage * BUF * 2);
    const uint32_t b_lds = a_lds + (uint32_t)(A_ELEMS * 2);
    const int krem = kspan - t * BK;  // chunks at K offset >= krem are past the end
#pragma unroll
    for (int j = 0; j < NA; ++j) {
      const int blk = wave_s + j * T::NWAVES;
      if (T::A_BLOCKS % T::NWAVES != 0 && blk >= T::A_BLOCKS) break;
      const void* src = a_kofs[j] < krem ? (const void*)(a_src[j] + (size_t)t * BK) : (const void*)g_zero16;
      lds_dma16(src, a_lds + blk * 1024);
    }
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int blk = wave_s + j * T::NWAVES;
      if (T::B_BLOCKS % T::NWAVES != 0 && blk >= T::B_BLOCKS) break;
      const void* src = b_kofs[j] < krem ? (const void*)(b_src[j] + (size_t)t * b_step) : (const void*)g_zero16;
      lds_dma16(src, b_lds + blk * 1024);
    }
  };

  // ---- LDS -> fragments ---------------------------------------------------
  // K-contiguous tiles: the swizzle depends only on the low 5 row bits, so a
  // fragment's address is a lane constant per k-step plus an immediate
  // fm*32*BK (or fn*32*BK) offset.
  const int lrow = lane & 31;
  const int lhalf = lane >> 5;
  int a_off[KS], b_off[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const int c = ks * 2 + lhalf;
    a_off[ks] = kc_slot<KC>(wm * TM + lrow, c) * 8;
    b_off[ks] = kc_slot<KC>(wn * TN + lrow, c) * 8;
  }
  // NN transpose read: 16-lane group g, lane i addresses row
  // k = ks*16 + 8*(g>>1) + 4*r + (i>>2), columns col0 + 16*(g&1) + 4*(i&3) .. +3.
  const int tg = lane >> 4, ti = lane & 15;
  const int nn_krow0 = 8 * (tg >> 1) + (ti >> 2);       // + ks*16 + 4*r
  const int nn_col0 = wn * TN + 16 * (tg & 1) + 4 * (ti & 3);  // + fn*32
  const int nn_sw = swz_nn<NC>(nn_krow0);                   // (k & 3) is the same for every ks, r

  // LDS read r of k-step ks (r < FM: A fragment r; then B: fragment r - FM
  // (NT), or transpose half (r - FM) % 2 of fragment (r - FM) / 2 (NN)).
  i16x4 trh[FN][2];
  auto read_one = [&](const uint16_t* As, int ks, auto rc, bf16x8* xa, bf16x8* xb) {
    constexpr int r = decltype(rc)::value;
    const uint16_t* Bs = As + A_ELEMS;
    if constexpr (r < FM) {
      xa[r] = *(const bf16x8*)(As + a_off[ks] + r * 32 * BK);
    } else if constexpr (!NN) {
      xb[r - FM] = *(const bf16x8*)(Bs + b_off[ks] + (r - FM) * 32 * BK);
    } else {
      constexpr int fn = (r - FM) / 2, h = (r - FM) % 2;
      const int col = nn_col0 + fn * 32;
      const int eoff = nn_col_off(col, nn_sw);
      const int krow = ks * 16 + 4 * h + nn_krow0;
      trh[fn][h] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) i16x4*)(Bs + krow * BN + eoff));
      if constexpr (h == 1) {
        u32x4 u;
        u.x = (uint32_t)(uint16_t)trh[fn][0].x | ((uint32_t)(uint16_t)trh[fn][0].y << 16);
        u.y = (uint32_t)(uint16_t)trh[fn][0].z | ((uint32_t)(uint16_t)trh[fn][0].w << 16);
        u.z = (uint32_t)(uint16_t)trh[fn][1].x | ((uint32_t)(uint16_t)trh[fn][1].y << 16);
        u.w = (uint32_t)(uint16_t)trh[fn][1].z | ((uint32_t)(uint16_t)trh[fn][1].w << 16);
        xb[fn] = __builtin_bit_cast(bf16x8, u);
      }
    }
  };
  auto read_frags = [&](const uint16_t* As, int ks, bf16x8* xa, bf16x8* xb) {
    const uint16_t* Bs = As + A_ELEMS;
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) xa[fm] = *(const bf16x8*)(As + a_off[ks] + fm * 32 * BK);
    if constexpr (!NN) {
#pragma unroll
      for (int fn = 0; fn < FN; ++fn) xb[fn] = *(const bf16x8*)(Bs + b_off[ks] + fn * 32 * BK);
    } else {
#pragma unroll
      for (int fn = 0; fn < FN; ++fn) {
        const int col = nn_col0 + fn * 32;
        const int eoff = nn_col_off(col, nn_sw);
        i16x4 v[2];
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          const int krow = ks * 16 + 4 * r + nn_krow0;
          v[r] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) i16x4*)(Bs + krow * BN + eoff));
        }
        u32x4 u;
        u.x = (uint32_t)(uint16_t)v[0].x | ((uint32_t)(uint16_t)v[0].y << 16);
        u.y = (uint32_t)(uint16_t)v[0].z | ((uint32_t)(uint16_t)v[0].w << 16);
        u.z = (uint32_t)(uint16_t)v[1].x | ((uint32_t)(uint16_t)v[1].y << 16);
        u.w = (uint32_t)(uint16_t)v[1].z | ((uint32_t)(uint16_t)v[1].w << 16);
        xb[fn] = __builtin_bit_cast(bf16x8, u);
      }
    }
  };

  f32x16 acc[FN][FM];
#pragma unroll
  for (int fn = 0; fn < FN; ++fn)
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[fn][fm][r] = 0.0f;

  // LDS instructions per k-step: FM b128 reads of A, FN b128 (NT) or 2*FN
  // transpose reads (NN) of B.
  constexpr int NREAD = FM + (NN ? 2 * FN : FN);
  constexpr int NMFMA = FM * FN;
  constexpr int NDMA = NA + NB;  // DMA loads per wave per tile (some may be idle)
  auto mfma_step = [&](const bf16x8* xa, const bf16x8* xb) {
#pragma unroll
    for (int fn = 0; fn < FN; ++fn)
#pragma unroll
      for (int fm = 0; fm < FM; ++fm)
        acc[fn][fm] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xb[fn], xa[fm], acc[fn][fm], 0, 0, 0);
  };
  // Scheduler hint for one k-step: its MFMAs with the LDS reads of the next
  // k-step slotted between them, so each fragment is requested a full k-step
  // (NMFMA x 32 cycles) before use.
  auto interleave_hint = [&]() {
#pragma unroll
    for (int i = 0; i < NMFMA; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if (i < NREAD) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    if (NREAD > NMFMA) __builtin_amdgcn_sched_group_barrier(0x100, NREAD - NMFMA, 0);
  };

  // Ring of S stages; tile t lives in stage t % S.  In iteration `it` the wave
  // runs k-steps 0 .. KS-2 of tile `it`, then waits for its own DMA of tile
  // it+1 and meets the other waves at the barrier, which (a) publishes tile
  // it+1 and (b) proves every wave has read all of stage it % S (the fragments
  // of the last k-step are already in registers).  The first fragments of tile
  // it+1 are read while the last k-step's MFMAs run, so the MFMA stream does not
  // drain at tile boundaries.  Where the DMA goes:
  //   S = 2 (or an uneven DMA split): the prologue requests tiles 0 .. S-1 and
  //   stage it % S receives tile it+S after the barrier, during the last
  //   k-step;
  //   S >= 3 with an even split ("spread"): the prologue requests tiles
  //   0 .. S-2 and iteration `it` loads tile it+S-1 into stage (it-1) % S,
  //   free since the previous barrier, with the loads spread one per MFMA
  //   slot over all KS k-steps (load j in k-step j*KS/LPT).  A CU accepts a
  //   1 KB load only every ~22 cycles, so a whole tile's DMA squeezed into one
  //   k-step stalls the issuing wave; spread, the same loads cost 1.5-3.5 %
  //   less time (bit-identical results).
  // vmcnt arithmetic: with an even DMA split every wave issues LPT loads per
  // tile, so "tile it+1 landed" is vmcnt <= the number of loads issued after
  // it (S = 2: LPT * (S-2); spread: LPT * (S-3) + the loads of tile it+S-1
  // issued before the barrier); otherwise, and near the end of K, the wave
  // waits for all loads.
  constexpr int LPT = T::LPT;
  constexpr bool EVEN = T::EVEN;
  bf16x8 xa[2][FM], xb[2][FN];
  constexpr bool SPREAD = EVEN && S >= 3;
  constexpr int PRO = SPREAD ? S - 1 : S;  // tiles loaded by the prologue
  if (nk > 0) {
#pragma unroll
    for (int t = 0; t < PRO; ++t)
      if (t < nk) load_tile(t, t);
    if (EVEN && nk >= PRO)
      wait_vmcnt<EVEN ? LPT * (PRO - 1) : 0>();
    else
      wait_vmcnt<0>();
    __syncthreads();
    read_frags(smem, 0, xa[0], xb[0]);
  }
  constexpr int CL = (KS - 1) & 1;  // fragment buffer of the last k-step
  // One iteration; BARRIER: not the last tile; LOAD: tile it+S exists.  The
  // three loop copies below keep each body free of branches, so the compiler's
  // LDS wait counts never merge the next tile's reads into the current ones.
  // Spread DMA: tile it+S-1 goes into stage (it-1) % S (free since the previous
  // barrier); load j is issued in k-step j*KS/LPT, one per MFMA slot.
  constexpr int PRE = SPREAD ? (LPT * (KS - 1) + KS - 1) / KS : 0;  // loads j with j*KS/LPT < KS-1
  auto iteration = [&](int it, auto barrier_c, auto load_c, auto check_c) {
    constexpr bool BARRIER = decltype(barrier_c)::value, LOAD = decltype(load_c)::value;
    // Stages as wave-uniform scalars, so that each LDS address is one add of a
    // loop-invariant lane offset and the stage (it % S left to the compiler is
    // strength-reduced across iterations into several per-iteration terms).
    const int cs = __builtin_amdgcn_readfirstlane(it % S);
    const uint16_t* cur = smem + cs * BUF;
    const int lt = SPREAD ? it + S - 1 : it + S;          // tile loaded by this iteration
    const int ls = __builtin_amdgcn_readfirstlane(SPREAD ? (it + S - 1) % S : it % S);  // its stage
    static_for<KS - 1>([&](auto ksc) {
      constexpr int ks = decltype(ksc)::value;
      constexpr int c = ks & 1;
      if constexpr (SPREAD && LOAD) {
        // reads of k-step ks+1, this k-step's MFMAs, and its DMA loads, one per slot
        constexpr int J0 = (ks * LPT + KS - 1) / KS, J1 = ((ks + 1) * LPT + KS - 1) / KS;  // j in [J0, J1)
        constexpr int NJ = J1 - J0;
        constexpr int NMEM2 = NJ > NREAD ? NJ : NREAD;
        constexpr int NSL = NMFMA > NMEM2 ? NMFMA : NMEM2;
        static_for<NSL>([&](auto ic) {
          constexpr int i = decltype(ic)::value;
          if constexpr (i < NMFMA) {
            constexpr int fn = i / FM, fm = i % FM;
            acc[fn][fm] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xb[c][fn], xa[c][fm], acc[fn][fm], 0, 0, 0);
          }
          if constexpr (i < NJ) dma_one(lt, ls, std::integral_constant<int, J0 + i>{}, check_c);
          if constexpr (i < NREAD) read_one(cur, ks + 1, std::integral_constant<int, i>{}, xa[c ^ 1], xb[c ^ 1]);
          __builtin_amdgcn_sched_barrier(0);
        });
      } else {
        read_frags(cur, ks + 1, xa[c ^ 1], xb[c ^ 1]);
        mfma_step(xa[c], xb[c]);
        interleave_hint();
      }
    });
    if constexpr (BARRIER) {
      if constexpr (SPREAD && LOAD)
        wait_vmcnt<SPREAD ? LPT * (S - 3) + PRE : 0>();  // tile it+1 landed
      else if constexpr (!SPREAD && LOAD && EVEN)
        wait_vmcnt<EVEN ? LPT * (S - 2) : 0>();  // tile it+1 landed, it+2 .. it+S-1 may fly
      else
        wait_vmcnt<0>();
      wait_lgkmcnt0();
      __syncthreads();
      const uint16_t* nxt = smem + __builtin_amdgcn_readfirstlane((it + 1) % S) * BUF;
      constexpr int JL = SPREAD ? PRE : 0;
      constexpr int NDL = NDMA - JL;  // loads left for the last k-step
      constexpr int NMEM = NDL > NREAD ? NDL : NREAD;
      constexpr int NSLOT = NMFMA > NMEM ? NMFMA : NMEM;
      static_for<NSLOT>([&](auto ic) {
        constexpr int i = decltype(ic)::value;
        if constexpr (i < NMFMA) {
          constexpr int fn = i / FM, fm = i % FM;
          acc[fn][fm] =
              __builtin_amdgcn_mfma_f32_32x32x16_bf16(xb[CL][fn], xa[CL][fm], acc[fn][fm], 0, 0, 0);
        }
        if constexpr (LOAD && i < NDL) dma_one(lt, ls, std::integral_constant<int, JL + i>{}, check_c);
        if constexpr (i < NREAD) read_one(nxt, 0, std::integral_constant<int, i>{}, xa[CL ^ 1], xb[CL ^ 1]);
        __builtin_amdgcn_sched_barrier(0);
      });
    } else {
      mfma_step(xa[CL], xb[CL]);
    }
    if constexpr (CL == 0) {
#pragma unroll
      for (int f = 0; f < FM; ++f) xa[0][f] = xa[1][f];
#pragma unroll
      for (int f = 0; f < FN; ++f) xb[0][f] = xb[1][f];
    }
  };
  using True = std::integral_constant<bool, true>;
  using False = std::integral_constant<bool, false>;
  const int nfull = kspan / BK;  // tiles that end inside the K range
  int it = 0;
  constexpr int AHEAD = SPREAD ? S - 1 : S;  // iteration it loads tile it + AHEAD
  for (; it + AHEAD < nfull; ++it) iteration(it, True{}, True{}, False{});  // steady state
  for (; it + AHEAD < nk; ++it) iteration(it, True{}, True{}, True{});      // loads the partial last tile
  for (; it + 1 < nk; ++it) iteration(it, True{}, False{}, False{});
  if (it < nk) iteration(it, False{}, False{}, False{});

  // Epilogue.  Lane l of block (fn, fm) holds C[m][n] for
  //   m = fm*32 + (l & 31),  n = fn*32 + 8*g + 4*(l >> 5) + {0..3},  g = 0..3,
  // i.e. four consecutive columns per (lane, g): one 16-byte (f32) or
  // 8-byte (bf16) store.  The (fm, fn) loops are expanded at compile time so
  // acc is only ever indexed by constants and stays in registers.
  const bool partial_plane = p.split_k > 1;
  char* ybase = (char*)p.y + (partial_plane ? (size_t)part * p.y_split_stride : 0);
  // Full tiles with bf16 output: stage each wave's block through the (now
  // idle) LDS ring and store whole rows, when the blocks fit in it.
  if constexpr (BM * BN <= S * BUF) {
    if (!partial_plane && p.out_bf16 && m0 + BM <= (int)p.M && n0 + BN <= (int)p.N && ((uintptr_t)p.y & 15) == 0) {
      __syncthreads();  // every wave has read its last fragments (no DMA is pending)
      store_tile_bf16_staged<FM, FN>(p, acc, (char*)smem + wave * TM * TN * 2, ybase, m0 + wm * TM,
                                     n0 + wn * TN, lane);
      return;
    }
  }
  static_for<FM>([&](auto fmc) {
    constexpr int fm = decltype(fmc)::value;
    const int m = m0 + wm * TM + fm * 32 + lrow;
    if (m < (int)p.M) {
      static_for<FN>([&](auto fnc) {
        constexpr int fn = decltype(fnc)::value;
        store_block(p, acc[fn][fm], ybase, m, n0 + wn * TN + fn * 32 + lhalf * 4, partial_plane);
      });
    }
  });
}

template <int BM, int BN, int BK, int WM, int WN, int S, bool NN>
__global__ __launch_bounds__(WM * WN * 64) void gemm_bf16_kernel(GemmParams p) {
  int tm, tn, part;
  tile_coords(p, tm, tn, part);
  gemm_bf16_tile<BM, BN, BK, WM, WN, S, NN>(p, tm, tn, part);
}

}  // namespace t0mi
