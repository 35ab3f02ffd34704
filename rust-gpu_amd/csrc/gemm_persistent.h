// gemm_persistent.h — persistent bf16 GEMM kernels (gfx950) for the reference's
// persistent TileGemm presets.
//
// The reference's persistent presets (tile_persistent_decode, src/t0/tile_ir.rs:540-561;
// tile_persistent_128x64_k32 / _256x128_k32, :563-604) lower to one workgroup that loops
// over the output tiles (the static slice tile_idx = iter, tile_ir.rs:1062-1120), so that a
// decode-sized GEMM is one dispatch.  On gfx950 one workgroup is one of 256 CUs, so here a
// persistent launch is a grid sized to what the GPU holds at once, each workgroup looping
// over work units with a stride of the grid: every workgroup stays resident until the
// units run out, and the schedule is static (no counter), so results do not depend on
// timing.
//
// gemm_persistent_decode_kernel — M small (decode: M = 1 .. 64), N and K large.
//   Unit: 32 rows x 16 columns of Y over the whole K range.  With one 16-column strip per
//   unit, N = 4096 gives 256 units (one per CU) without splitting K across workgroups, so
//   the sum needs no second launch.  The 16 waves of a workgroup split the unit's K range
//   into 16 contiguous pieces; each wave loads its operands straight into registers (8
//   k-blocks of 32 in flight, 16 bytes per lane per load, all issued before the first
//   MFMA) and accumulates with v_mfma_f32_16x16x32_bf16 (rows 16..31 only when the unit
//   has them).  The 16 wave partials meet in LDS and are summed in wave order (a fixed
//   order: results are deterministic), then the epilogue chain runs once and each row
//   segment is one 16-byte store.
//   Operand fragments (16x16x32 layout): lane l holds row / column l % 16, K elements
//   8 * (l / 16) .. +7 of the k-block.  NT: B's rows are K-contiguous, so the fragment is
//   one 16-byte load.  NN: B is [K, N]; each lane loads 8 columns of one K row, the wave
//   writes the 32 x 16 block to its own 1 KB of LDS and reads the fragment back with two
//   ds_read_b64_tr_b16 (the transpose read).  The block's 4-row groups are stored in the
//   order k = 0-3, 8-11, 16-19, 24-27, 4-7, ... so that each half-wave's transpose read
//   covers 256 contiguous bytes (no bank conflict).
//   Bounds: rows >= M and columns >= N read a clamped (valid) row / column whose results
//   are never stored.  K must be a multiple of 32 (whole k-blocks) and the lane offsets
//   32-bit (A and an NT B under 4 GiB); the host routes other shapes to the tile kernel.
//
// gemm_bf16_persistent_kernel (gemm_bf16_kernel.h's tile body in a loop) — larger M: the
//   spec's own tile shape, tiles walked with the grid stride; consecutive tiles of one XCD
//   stay contiguous as in the one-shot kernel.
#pragma once
#include <type_traits>

#include "gemm_bf16_kernel.h"

namespace t0mi {

constexpr int PD_WAVES = 16;  // waves per workgroup; each owns 1/16 of the unit's K range
constexpr int PD_CH = 8;      // k-blocks (32 K each) a wave has in flight
constexpr int PD_ROWS = 32;   // unit rows (two 16-row MFMA blocks)
constexpr int PD_COLS = 16;   // unit columns (one 16-column MFMA block)

// NN block layout in a wave's LDS (nn_pd_krow, nn_pd_tr_off): index_maps.h.

// 16-byte load through the global address space (a generic pointer would become a flat
// load, which the compiler can only wait for with vmcnt(0) lgkmcnt(0)).
__device__ __forceinline__ bf16x8 gload16(const char* base, uint32_t off) {
  return *(const __attribute__((address_space(1))) bf16x8*)(base + off);
}

// Grid-stride position -> unit: workgroups are dispatched round-robin over the 8 XCDs;
// with G a multiple of 8, workgroup b runs on XCD b % 8, so b is renumbered to make the
// workgroups of one XCD take neighbouring column strips (they share 128-byte lines of an
// NN B row and the rows of A).
__device__ __forceinline__ uint32_t pd_logical_wg() {
  const uint32_t g = gridDim.x, b = blockIdx.x;
  return (g % 8u) == 0u ? (b % 8u) * (g / 8u) + b / 8u : b;
}

template <bool NN>
__global__ __launch_bounds__(PD_WAVES * 64) void gemm_persistent_decode_kernel(GemmParams p) {
  __shared__ __attribute__((aligned(16))) f32x4 red[PD_WAVES][2][64];                 // wave partials
  __shared__ __attribute__((aligned(1024))) uint16_t bst[NN ? PD_WAVES * 512 : 8];  // NN: 1 KB per wave
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const uint32_t units = p.tiles_m * p.tiles_n;
  const int K = (int)p.K, M = (int)p.M, N = (int)p.N;
  const int nkb = (K + 31) >> 5;
  const int kb0 = wave * nkb / PD_WAVES, kb1 = (wave + 1) * nkb / PD_WAVES;
  const int kq = 8 * (lane >> 4);  // the lane's K chunk inside a k-block (NT B and A)
  uint16_t* my_bst = bst + (NN ? wave * 512 : 0);

  // One unit's K loop for this wave; TWO: the unit has rows 16..31.
  auto k_loop = [&](int m0, int n0, auto two_c, f32x4& acc0, f32x4& acc1) {
    constexpr bool TWO = decltype(two_c)::value;
    // Byte offsets of the lane's 16 bytes from the k-block's base address (which is
    // wave-uniform), so every load is an SGPR base plus one 32-bit VGPR offset.
    const uint32_t r0 = (uint32_t)min(m0 + (lane & 15), M - 1);
    const uint32_t r1 = (uint32_t)min(m0 + 16 + (lane & 15), M - 1);
    const uint32_t a_off0 = (r0 * p.lda + kq) * 2u, a_off1 = (r1 * p.lda + kq) * 2u;
    uint32_t b_off;
    size_t b_step;  // bytes between consecutive k-blocks of B
    if constexpr (NN) {
      const uint32_t c = (uint32_t)min(n0 + 8 * (lane & 1), N - 8);
      b_off = ((uint32_t)nn_pd_krow(lane) * p.ldb + c) * 2u;
      b_step = (size_t)64 * p.ldb;
    } else {
      const uint32_t c = (uint32_t)min(n0 + (lane & 15), N - 1);
      b_off = (c * p.ldb + kq) * 2u;
      b_step = 64;
    }
    for (int c0 = kb0; c0 < kb1; c0 += PD_CH) {
      bf16x8 xb[PD_CH], xa0[PD_CH], xa1[PD_CH];
#pragma unroll
      for (int j = 0; j < PD_CH; ++j) {
        // Slots past the wave's range (last chunk only) reload its last k-block; their
        // MFMAs are skipped.
        const int kb = min(c0 + j, kb1 - 1);
        const char* bb = (const char*)p.b + (size_t)kb * b_step;
        const char* ab = (const char*)p.a + (size_t)kb * 64;
        xb[j] = gload16(bb, b_off);
        xa0[j] = gload16(ab, a_off0);
        if constexpr (TWO) xa1[j] = gload16(ab, a_off1);
      }
      // Every load of the chunk is issued before the first MFMA waits for one.
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 0; j < PD_CH; ++j) {
        if (c0 + j >= kb1) break;
        bf16x8 fb;
        if constexpr (NN) {
          *(bf16x8*)(my_bst + 8 * lane) = xb[j];
          i16x4 v[2];
#pragma unroll
          for (int h = 0; h < 2; ++h)
            v[h] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) i16x4*)((char*)my_bst + nn_pd_tr_off(lane, h)));
          u32x4 u;
          u.x = (uint32_t)(uint16_t)v[0].x | ((uint32_t)(uint16_t)v[0].y << 16);
          u.y = (uint32_t)(uint16_t)v[0].z | ((uint32_t)(uint16_t)v[0].w << 16);
          u.z = (uint32_t)(uint16_t)v[1].x | ((uint32_t)(uint16_t)v[1].y << 16);
          u.w = (uint32_t)(uint16_t)v[1].z | ((uint32_t)(uint16_t)v[1].w << 16);
          fb = __builtin_bit_cast(bf16x8, u);
        } else {
          fb = xb[j];
        }
        acc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fb, xa0[j], acc0, 0, 0, 0);
        if constexpr (TWO) acc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fb, xa1[j], acc1, 0, 0, 0);
      }
    }
  };

  const uint32_t start = pd_logical_wg();
  for (uint32_t u = start; u < units; u += gridDim.x) {
    const int m0 = (int)(u / p.tiles_n) * PD_ROWS, n0 = (int)(u % p.tiles_n) * PD_COLS;
    const bool two = m0 + 16 < M;
    f32x4 acc0 = {0.0f, 0.0f, 0.0f, 0.0f}, acc1 = {0.0f, 0.0f, 0.0f, 0.0f};
    if (two)
      k_loop(m0, n0, std::true_type{}, acc0, acc1);
    else
      k_loop(m0, n0, std::false_type{}, acc0, acc1);
    // Lane l of block h holds Y[m0 + 16h + l % 16][n0 + 4 (l / 16) + 0..3].
    red[wave][0][lane] = acc0;
    if (two) red[wave][1][lane] = acc1;
    __syncthreads();
    const int t = threadIdx.x;
    if (t < 2 * 64) {
      const int row = t >> 2, cg = t & 3;  // unit row, 4-column group
      const int h = row >> 4;
      const int m = m0 + row, n = n0 + 4 * cg;
      if ((h == 0 || two) && m < M && n < N) {
        const int src = cg * 16 + (row & 15);
        f32x4 s = red[0][h][src];
#pragma unroll
        for (int w = 1; w < PD_WAVES; ++w) s += red[w][h][src];
        float v0 = s.x, v1 = s.y, v2 = s.z, v3 = s.w;
        if (p.epi.n) {
          f32x4 bv = {0.0f, 0.0f, 0.0f, 0.0f};
          if (p.bias) bv = f32x4{p.bias[n], p.bias[n + 1], p.bias[n + 2], p.bias[n + 3]};
          v0 = epi_apply(v0, bv.x, p.epi);
          v1 = epi_apply(v1, bv.y, p.epi);
          v2 = epi_apply(v2, bv.z, p.epi);
          v3 = epi_apply(v3, bv.w, p.epi);
        }
        if (p.out_bf16) {
          u32x2 o;
          o.x = pack_bf16x2(v0, v1);
          o.y = pack_bf16x2(v2, v3);
          *(u32x2*)((uint16_t*)p.y + (size_t)m * p.ldy + n) = o;
        } else {
          *(f32x4*)((float*)p.y + (size_t)m * p.ldy + n) = f32x4{v0, v1, v2, v3};
        }
      }
    }
    __syncthreads();  // red is rewritten by the next unit
  }
}

// The generic tile kernel, persistent: work item u (tile, K partition) for u = blockIdx.x,
// blockIdx.x + gridDim.x, ...; the barrier between items keeps the next item's prologue
// DMA out of the LDS ring until every wave is done with the previous one.
template <int BM, int BN, int BK, int WM, int WN, int S, bool NN>
__global__ __launch_bounds__(WM * WN * 64) void gemm_bf16_persistent_kernel(GemmParams p) {
  const uint32_t items = p.tiles_m * p.tiles_n * p.split_k;
  for (uint32_t u = blockIdx.x; u < items; u += gridDim.x) {
    int tm, tn, part;
    tile_coords_lin(u, items, p.tiles_m, p.tiles_n, p.xcd_remap, tm, tn, part);
    gemm_bf16_tile<BM, BN, BK, WM, WN, S, NN>(p, tm, tn, part);
    __syncthreads();
  }
}

}  // namespace t0mi
