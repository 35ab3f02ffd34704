// index_maps.h — the index maps of the gfx950 kernels: LDS swizzles, the
// chunk each DMA lane fetches, and the activation slot map of the W4A16
// decode kernel.  Plain constexpr integer functions, compiled into the kernels
// and, without HIP, into the host-side simulation that checks them (coverage
// exactly once, LDS bijections, bank-conflict freedom; tests/index_maps_sim.cpp).
#pragma once

#if defined(__HIPCC__)
#define T0MI_HD __host__ __device__ __forceinline__
#else
#define T0MI_HD inline
#endif

namespace t0mi {

// XOR swizzle of 16-byte chunks inside a K-contiguous LDS row of KC chunks.
// Any 8 consecutive rows (aligned to 8) reading the same logical chunk land in
// 8 distinct 16-byte slots of a 128-byte bank line.
// Only the low 5 row bits are used, so rows 32 apart share the swizzle.
template <int KC>
T0MI_HD constexpr int swz(int r) {
  return ((r / (8 / KC)) ^ ((r >> 3) & 3)) & (KC - 1);
}

// Swizzle of the 16-byte chunks of an NN B row (row = k, NC chunks per row).
// A transpose read is served 32 lanes at a time: two 16-lane groups that read
// the same 4 consecutive rows, 32 bytes each, in adjacent 32-byte column slots
// (2j, 2j+1).  XOR of the chunk index with 4*(k % 4) moves row k to slot
// offset 2*(k % 4), so the 4 rows x 2 slots cover 8 distinct 32-byte slots:
// all 64 banks, no conflict.  Rows of 8 chunks (tile_n = 64) have only 4
// slots; there 2*(k % 4) keeps each 16-lane group conflict-free.
template <int NC>
T0MI_HD constexpr int swz_nn(int k) {
  return NC >= 16 ? (k & 3) << 2 : (k & 3) << 1;
}

// K-contiguous tile [rows][KC chunks] (A, and NT's B): LDS chunk slot q (the
// DMA's 1 KB block q / 64, lane q % 64) receives logical chunk *lc of row *row.
template <int KC>
T0MI_HD void kc_dma_chunk(int q, int* row, int* lc) {
  *row = q / KC;
  *lc = (q % KC) ^ swz<KC>(*row);
}
// The LDS chunk slot holding logical chunk c of row `row` (the fragment reads).
template <int KC>
T0MI_HD constexpr int kc_slot(int row, int c) {
  return row * KC + (c ^ swz<KC>(row));
}

// NN B tile [k rows][NC chunks of 8 columns]: LDS chunk slot q receives the
// 8 columns starting at 8 * *lc of k-row *krow.
template <int NC>
T0MI_HD void nn_dma_chunk(int q, int* krow, int* lc) {
  *krow = q / NC;
  *lc = (q % NC) ^ swz_nn<NC>(*krow);
}
// Element offset of column `col` (a multiple of 4) within an NN k-row whose
// swizzle is `sw` (= swz_nn(k); kernels compute it once, since every k-row a
// lane reads has the same k % 4).
T0MI_HD constexpr int nn_col_off(int col, int sw) { return (((col >> 3) ^ sw) << 3) + (col & 4); }
// LDS element offset of column `col` of k-row k: the address of a
// ds_read_b64_tr_b16 lane, which reads 4 columns.
template <int NC>
T0MI_HD constexpr int nn_elem(int k, int col) {
  return k * NC * 8 + nn_col_off(col, swz_nn<NC>(k));
}

// W4A16 decode: 16-byte slot (0..63, within one 1 KB half of a 2 KB pair of
// k-blocks) of piece (row 8h + r, 16-byte chunk x) of the activation block.
// For a fixed chunk the 16 rows fall in 16 distinct 16-byte bank groups.
T0MI_HD constexpr int dec_slot(int h, int r, int x) {
  return 16 * (x >> 1) + ((8 * h + r) ^ (8 * (x & 1) + (x >> 1)));
}

}  // namespace t0mi
