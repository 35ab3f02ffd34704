// index_maps.h — the index maps of the gfx950 kernels: LDS swizzles, the
// chunk each DMA lane fetches, the activation slot map of the W4A16 decode
// kernel, and the workgroup numbering of its in-launch K split.  Plain constexpr integer functions, compiled into the kernels
// and, without HIP, into the host-side simulation that checks them (coverage
// exactly once, LDS bijections, bank-conflict freedom; tests/index_maps_sim.cpp).
#pragma once
#include <stdint.h>

#if defined(__HIPCC__)
#define T0MI_HD __host__ __device__ __forceinline__
#else
#define T0MI_HD inline
#endif

namespace t0mi {

// LDS bank conflicts (gfx950; 64 banks of 4 bytes), as measured with
// SQ_LDS_BANK_CONFLICT on lane -> address tables (t0mi_probe_lds): a
// ds_read_b128 takes 4 cycles when conflict-free, each half-wave (lanes 0-31,
// 32-63) in 2 cycles of 16 lanes.  The split of a half-wave into its two
// cycles is not lanes 0-15 / 16-31: lanes whose indices differ in bits 0-3 and
// address the same bank at different addresses conflict, lanes differing in
// bit 4 do not, yet 16 lanes reading 16 distinct slots modulo 256 bytes can
// still conflict with the other 16 of their half-wave.  The measurements fit
// a split by the parity of lane bits 3 and 4 combined with other lane or
// address bits (48 such rules fit all of them); a cycle is conflict-free when
// its 16 lanes read 16 distinct 16-byte slots modulo 256 bytes.  The layouts
// below are conflict-free under every one of those rules.  ds_read_b64 and
// ds_read_b64_tr_b16 half-waves are served in one cycle of 32 lanes (32
// distinct 8-byte slots modulo 256 bytes).

// XOR swizzle of 16-byte chunks inside a K-contiguous LDS row of KC chunks,
// for the 32x32x16 operand layout (lane l reads row l % 32, chunk c + l / 32):
// a half-wave reads 32 consecutive rows at one logical chunk.  For 64-byte
// rows (KC = 4) bits 2-3 of the row (the rows 4 apart that share bank
// columns); the formula of the other widths gives them two-way conflicts
// (measured).  Only the low 5 row bits are used, so rows 32 apart share the
// swizzle.
template <int KC>
T0MI_HD constexpr int swz(int r) {
  return KC == 4 ? (r >> 2) & 3 : ((r / (8 / KC)) ^ ((r >> 3) & 3)) & (KC - 1);
}

// Rotation of 64-K (KC = 8) rows for the 16x16x32 operand layout (lane l reads
// row l % 16, chunk c + l / 16, c a multiple of 4): logical chunk c of row r
// sits at position (c + r) % 8.  With XOR swizzles this layout conflicts two
// ways (a half-wave reads each of its 16 rows at chunks a and a ^ 1, and the
// XOR keeps those pairs together); the rotation is conflict-free.  Rows 8
// apart share it.
T0MI_HD constexpr int rot16(int r, int c) { return (c + r) & 7; }

// Swizzle of the 16-byte chunks of an NN B row (row = k, NC chunks per row).
// A transpose read is served 32 lanes at a time.  With the 32x32x16 operand
// (X16 = false) its two 16-lane groups read the same 4 consecutive rows, 32
// bytes each, in adjacent 32-byte column slots (2j, 2j+1).  XOR of the chunk
// index with 4*(k % 4) moves row k to slot offset 2*(k % 4), so the 4 rows x 2
// slots cover 8 distinct 32-byte slots: all 64 banks, no conflict.  Rows of 8
// chunks (tile_n = 64) have only 4 slots; there 2*(k % 4) keeps each 16-lane
// group conflict-free.  With the 16x16x32 operand (X16 = true) the two groups
// read the same 32 bytes of columns in rows 8 apart; bit 3 of k then also flips
// bit 1 of the chunk index, moving the second group to the other 32 bytes of
// each 64-byte slot pair.
template <int NC, bool X16 = false>
T0MI_HD constexpr int swz_nn(int k) {
  return NC >= 16 ? ((k & 3) << 2) ^ (X16 ? ((k >> 3) & 1) << 1 : 0) : (k & 3) << 1;
}

// K-contiguous tile [rows][KC chunks] (A, and NT's B): LDS chunk slot q (the
// DMA's 1 KB block q / 64, lane q % 64) receives logical chunk *lc of row *row.
// X16: the swizzle of the 16x16x32 layout (KC = 8 only).
template <int KC, bool X16 = false>
T0MI_HD void kc_dma_chunk(int q, int* row, int* lc) {
  static_assert(!X16 || KC == 8, "the 16x16x32 layout is for 64-K rows");
  *row = q / KC;
  *lc = X16 ? (q % KC - *row) & 7 : (q % KC) ^ swz<KC>(*row);
}
// The LDS chunk slot holding logical chunk c of row `row` (the fragment reads).
template <int KC, bool X16 = false>
T0MI_HD constexpr int kc_slot(int row, int c) {
  return row * KC + (X16 ? rot16(row, c) : c ^ swz<KC>(row));
}

// NN B tile [k rows][NC chunks of 8 columns]: LDS chunk slot q receives the
// 8 columns starting at 8 * *lc of k-row *krow.
template <int NC, bool X16 = false>
T0MI_HD void nn_dma_chunk(int q, int* krow, int* lc) {
  *krow = q / NC;
  *lc = (q % NC) ^ swz_nn<NC, X16>(*krow);
}
// Element offset of column `col` (a multiple of 4) within an NN k-row whose
// swizzle is `sw` (= swz_nn(k); kernels compute it once, since every k-row a
// lane reads has the same k % 4, and with X16 the same bit 3).
T0MI_HD constexpr int nn_col_off(int col, int sw) { return (((col >> 3) ^ sw) << 3) + (col & 4); }
// LDS element offset of column `col` of k-row k: the address of a
// ds_read_b64_tr_b16 lane, which reads 4 columns.
template <int NC, bool X16 = false>
T0MI_HD constexpr int nn_elem(int k, int col) {
  return k * NC * 8 + nn_col_off(col, swz_nn<NC, X16>(k));
}

// Operand maps of v_mfma_f32_16x16x32_bf16 as the X16 kernels use them (lane l,
// 8 bf16 per lane): the K-contiguous operand (A rows; NT's B rows) takes row
// l % 16 of its 16-row block, k-chunk l / 16 (8 of K) of the 32-K step; the NN
// B operand (column l % 16, k 8 (l / 16) + 0..7) is two transpose reads h = 0,
// 1, lane l addressing k-row 8 (l / 16) + 4 h + (l % 16) / 4 of the step and
// the 4 columns starting at 4 (l % 4) of the block.  Output: lane l holds
// rows 4 (l / 16) + 0..3 of the instruction's first operand, column l % 16
// of its second -- the kernels pass B first, so lane l holds row l % 16 of the
// block and its 4 consecutive columns 4 (l / 16) + 0..3.
T0MI_HD constexpr int x16_krow(int lane, int h) { return 8 * (lane >> 4) + 4 * h + ((lane & 15) >> 2); }
T0MI_HD constexpr int x16_col(int lane) { return 4 * (lane & 3); }

// Swizzle of the 16-byte chunks of a 128-byte row of the bf16 output staging
// block of the X16 ping-pong kernel.  A ds_write_b64 pass (32 lanes) writes
// rows r0 .. r0+15 (16-row block), two 8-byte halves of one chunk each; rows
// with equal r % 2 share 128-byte bank lines, and (r ^ (r >> 3)) % 8 gives the
// 8 rows of each parity 8 distinct chunk positions.
T0MI_HD constexpr int stage_swz16(int r) { return (r ^ (r >> 3)) & 7; }

// W4A16 decode: 16-byte slot (0..63, within one 1 KB half of a 2 KB pair of
// k-blocks) of piece (row 8h + r, 16-byte chunk x) of the activation block.
// For a fixed chunk the 16 rows fall in 16 distinct 16-byte bank groups.
T0MI_HD constexpr int dec_slot(int h, int r, int x) {
  return 16 * (x >> 1) + ((8 * h + r) ^ (8 * (x & 1) + (x >> 1)));
}

// Persistent decode kernel, NN: a wave turns a 32 (K) x 16 (column) bf16 block
// into the 16x16x32 B operand through 1 KB of its own LDS.  Lane l loads 8
// columns (8 * (l & 1) .. +7) of K row nn_pd_krow(l) and stores the 16 bytes at
// byte 16 l; the 4-row groups land in the order k = 0-3, 8-11, 16-19, 24-27,
// 4-7, ..., so that the transpose read h of lane l (K rows 8 (l / 16) + 4 h +
// 0..3 of column l % 16) starts at nn_pd_tr_off(l, h) and each half-wave's read
// covers 256 contiguous bytes.
T0MI_HD constexpr int nn_pd_krow(int l) { return 8 * ((l >> 3) & 3) + 4 * (l >> 5) + ((l & 7) >> 1); }
T0MI_HD constexpr int nn_pd_tr_off(int l, int h) {
  return h * 512 + (l >> 4) * 128 + ((l & 15) >> 2) * 32 + (l & 3) * 8;
}

// ---- in-launch split-K numbering (xcd_exchange.h) ------------------------------

// Workgroup `id` of a launch whose tiles are each split over `pieces`
// workgroups, numbered id = ((tile / nx) * pieces + piece) * nx + tile % nx so
// that all pieces of a tile share id % nx (the XCD under round-robin dispatch):
// (tile, piece) of `id`.  Tiles past the caller's count are the numbering's
// padding to a multiple of nx.
T0MI_HD void xk_unpack(uint32_t id, uint32_t nx, uint32_t pieces, uint32_t* tile, uint32_t* piece) {
  const uint32_t xs = id % nx, r = id / nx;
  *piece = r % pieces;
  *tile = (r / pieces) * nx + xs;
}

}  // namespace t0mi
