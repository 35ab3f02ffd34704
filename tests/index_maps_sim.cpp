// index_maps_sim.cpp — host-side simulation of the gfx950 kernels' index maps
// (rust-gpu_amd/csrc/index_maps.h, compiled here without HIP), in the way the
// kernels decompose their work: which LDS slot every DMA lane fills with which
// global chunk, which slot every fragment read takes, and which LDS banks a
// read or write instruction touches.  Checks, for every tile shape built:
//   - every (row, chunk) of a tile is fetched exactly once and each LDS slot
//     written once (a bijection), with no source outside the tile;
//   - every fragment read finds the chunk the MFMA operand expects there;
//   - the per-lane constants the kernels hoist out of their loops (swizzles of
//     rows 32 or 4 apart, the ping-pong kernel's per-wave offsets) are valid
//     for every load they serve;
//   - the bank-conflict freedom the swizzles are designed for.
// The counterpart of the reference's CPU-side locks (tests/gemm_memory_safety.rs).
// Prints each failure; exit status 1 if any.
#include <stdio.h>

#include <set>
#include <vector>

#include "../rust-gpu_amd/csrc/index_maps.h"

using namespace t0mi;

static int g_fail = 0, g_checks = 0;
#define CHECK(cond, ...)                                   \
  do {                                                     \
    ++g_checks;                                            \
    if (!(cond)) {                                         \
      if (g_fail++ < 30) {                                 \
        printf("FAIL line %d: ", __LINE__);                \
        printf(__VA_ARGS__);                               \
        printf("\n");                                      \
      }                                                    \
    }                                                      \
  } while (0)

// ---- K-contiguous tiles (A, NT's B) of the generic kernel -------------------
// Wave w issues loads j = 0..ceil(blocks / nwaves) - 1 of block w + j * nwaves
// (blocks past the tile are skipped); lane l of a block fills chunk slot
// block * 64 + l.  Fragment reads take kc_slot(row, c).
template <int KC>
static void kc_tile(int rows, int nwaves) {
  const int chunks = rows * KC, blocks = chunks / 64;
  CHECK(chunks % 64 == 0, "KC=%d rows=%d: tile is not whole 1 KB blocks", KC, rows);
  std::vector<int> fetched(chunks, 0), slot_holds(chunks, -1);
  const int nloads = (blocks + nwaves - 1) / nwaves;
  for (int w = 0; w < nwaves; ++w)
    for (int j = 0; j < nloads; ++j) {
      const int blk = w + j * nwaves;
      if (blk >= blocks) continue;
      for (int lane = 0; lane < 64; ++lane) {
        const int q = blk * 64 + lane;
        int row, lc;
        kc_dma_chunk<KC>(q, &row, &lc);
        CHECK(row >= 0 && row < rows && lc >= 0 && lc < KC, "KC=%d q=%d -> (%d,%d) outside the tile", KC, q, row, lc);
        if (row < 0 || row >= rows || lc < 0 || lc >= KC) continue;
        fetched[row * KC + lc]++;
        CHECK(slot_holds[q] < 0, "KC=%d slot %d written twice", KC, q);
        slot_holds[q] = row * KC + lc;
      }
    }
  for (int i = 0; i < chunks; ++i) CHECK(fetched[i] == 1, "KC=%d rows=%d chunk %d fetched %d times", KC, rows, i, fetched[i]);
  for (int row = 0; row < rows; ++row)
    for (int c = 0; c < KC; ++c) {
      const int s = kc_slot<KC>(row, c);
      CHECK(s >= 0 && s < chunks && slot_holds[s] == row * KC + c, "KC=%d read (%d,%d) at slot %d finds %d", KC, row,
            c, s, s >= 0 && s < chunks ? slot_holds[s] : -1);
    }
  for (int row = 0; row < rows; ++row)
    CHECK(swz<KC>(row) == swz<KC>(row % 32), "KC=%d swz(%d) != swz(%d)", KC, row, row % 32);
  // ds_read_b128: 32 lanes read rows 32i .. 32i+31 at one logical chunk; each
  // aligned group of 8 rows lands in 8 distinct 16-byte slots of a 128-byte line.
  for (int r0 = 0; r0 < rows; r0 += 8)
    for (int c = 0; c < KC; ++c) {
      std::set<int> slots;
      for (int r = r0; r < r0 + 8; ++r) slots.insert(kc_slot<KC>(r, c) % 8);
      CHECK(slots.size() == 8, "KC=%d rows %d..%d chunk %d: %zu distinct slots in a 128-byte line", KC, r0, r0 + 7, c,
            slots.size());
    }
}

// ---- NN B tiles [BK k-rows][NC chunks] of the generic kernel ------------------
template <int NC>
static void nn_tile(int krows, int nwaves) {
  const int chunks = krows * NC, blocks = chunks / 64;
  std::vector<int> fetched(chunks, 0), slot_holds(chunks, -1);
  const int nloads = (blocks + nwaves - 1) / nwaves;
  for (int w = 0; w < nwaves; ++w)
    for (int j = 0; j < nloads; ++j) {
      const int blk = w + j * nwaves;
      if (blk >= blocks) continue;
      for (int lane = 0; lane < 64; ++lane) {
        const int q = blk * 64 + lane;
        int k, lc;
        nn_dma_chunk<NC>(q, &k, &lc);
        CHECK(k >= 0 && k < krows && lc >= 0 && lc < NC, "NC=%d q=%d -> (%d,%d) outside", NC, q, k, lc);
        if (k < 0 || k >= krows || lc < 0 || lc >= NC) continue;
        fetched[k * NC + lc]++;
        slot_holds[q] = k * NC + lc;
      }
    }
  for (int i = 0; i < chunks; ++i) CHECK(fetched[i] == 1, "NC=%d chunk %d fetched %d times", NC, i, fetched[i]);
  // Transpose reads: lane (tg, ti) of k-step ks, half h reads 4 columns at
  // k-row ks*16 + 4h + 8(tg>>1) + (ti>>2), column col0 + 16(tg&1) + 4(ti&3)
  // (+ 32 fn + a wave's column base); the element found must be that column.
  const int BN = NC * 8;
  for (int k = 0; k < krows; ++k)
    for (int col = 0; col < BN; col += 4) {
      const int e = nn_elem<NC>(k, col);
      const int slot = e / 8, within = e % 8;
      CHECK(slot >= 0 && slot < chunks, "NC=%d (%d,%d) -> element %d outside", NC, k, col, e);
      if (slot < 0 || slot >= chunks) continue;
      const int held = slot_holds[slot];
      CHECK(held / NC == k && (held % NC) * 8 + within == col, "NC=%d read (%d,%d) finds k-row %d column %d", NC, k,
            col, held / NC, (held % NC) * 8 + within);
      // the swizzle the kernels hoist: k-rows of one lane differ by multiples of 4
      CHECK(swz_nn<NC>(k) == swz_nn<NC>(k & 3), "NC=%d swz_nn(%d)", NC, k);
    }
  // Bank conflicts of one ds_read_b64_tr_b16 pass (lanes 0-31 or 32-63): 64 banks of 4 bytes.
  for (int ks = 0; ks * 16 < krows; ++ks)
    for (int h = 0; h < 2; ++h)
      for (int cb = 0; cb + 32 <= BN; cb += 32)
        for (int pass = 0; pass < 2; ++pass) {
          std::vector<int> bank_use(64, 0);
          for (int lane = 32 * pass; lane < 32 * pass + 32; ++lane) {
            const int tg = lane >> 4, ti = lane & 15;
            const int k = ks * 16 + 4 * h + 8 * (tg >> 1) + (ti >> 2);
            const int col = cb + 16 * (tg & 1) + 4 * (ti & 3);
            if (NC == 8 && (tg & 1)) continue;  // 64-column rows: checked per 16-lane group below
            const int byte = nn_elem<NC>(k, col) * 2;
            bank_use[(byte / 4) % 64]++;
            bank_use[(byte / 4 + 1) % 64]++;
          }
          for (int b = 0; b < 64; ++b)
            CHECK(bank_use[b] <= 1, "NC=%d ks=%d h=%d cols %d pass %d: bank %d used %d times", NC, ks, h, cb, pass, b,
                  bank_use[b]);
        }
}

// ---- ping-pong kernel (256 x 256 x 64, 8 waves in two groups) ---------------
// Wave w4 of group g: A loads j = 0..3 fill blocks w4 + 4j of the group's
// 128-row half (buffer resource at row g*128 + 32 j, one lane offset from
// block w4); B loads j = 0..3 fill blocks 16g + w4 + 4j of the B tile (NN: base
// address moved by 8 k-rows per j; NT: resource at row g*128 + 32 j).
static void pingpong() {
  constexpr int KC = 8, NC = 32;
  std::vector<int> a_fetch(256 * KC, 0), bnn_fetch(64 * NC, 0), bnt_fetch(256 * KC, 0);
  std::vector<int> a_half_holds[2] = {std::vector<int>(128 * KC, -1), std::vector<int>(128 * KC, -1)};
  for (int g = 0; g < 2; ++g)
    for (int w4 = 0; w4 < 4; ++w4)
      for (int lane = 0; lane < 64; ++lane) {
        int row, lc, brow, blc;
        kc_dma_chunk<KC>(w4 * 64 + lane, &row, &lc);           // the kernel's a_voff / NT b_voff
        nn_dma_chunk<NC>((16 * g + w4) * 64 + lane, &brow, &blc);  // the kernel's NN b_voff
        CHECK(row < 32, "ping-pong A lane offset row %d leaves its 32-row block", row);
        for (int j = 0; j < 4; ++j) {
          // A: LDS slot (4j + w4) * 64 + lane of the half; source row 32 j + row of the half
          const int q = (4 * j + w4) * 64 + lane;
          int r2, l2;
          kc_dma_chunk<KC>(q, &r2, &l2);
          CHECK(r2 == 32 * j + row && l2 == lc, "ping-pong A j=%d w4=%d lane=%d: slot wants (%d,%d), load gives (%d,%d)",
                j, w4, lane, r2, l2, 32 * j + row, lc);
          a_fetch[(g * 128 + 32 * j + row) * KC + lc]++;
          a_half_holds[g][q] = (32 * j + row) * KC + lc;
          // NN B: block 16g + w4 + 4j
          int k3, l3;
          nn_dma_chunk<NC>((16 * g + w4 + 4 * j) * 64 + lane, &k3, &l3);
          CHECK(k3 == brow + 8 * j && l3 == blc, "ping-pong NN B j=%d: slot wants (%d,%d), load gives (%d,%d)", j, k3,
                l3, brow + 8 * j, blc);
          if (brow + 8 * j < 64) bnn_fetch[(brow + 8 * j) * NC + blc]++;
          // NT B: block 16g + w4 + 4j of [256 n][8 chunks]
          int r4, l4;
          kc_dma_chunk<KC>((16 * g + w4 + 4 * j) * 64 + lane, &r4, &l4);
          CHECK(r4 == g * 128 + 32 * j + row && l4 == lc, "ping-pong NT B j=%d: (%d,%d) vs (%d,%d)", j, r4, l4,
                g * 128 + 32 * j + row, lc);
          bnt_fetch[(g * 128 + 32 * j + row) * KC + lc]++;
        }
      }
  for (int i = 0; i < 256 * KC; ++i) CHECK(a_fetch[i] == 1 && bnt_fetch[i] == 1, "ping-pong A/NT-B chunk %d", i);
  for (int i = 0; i < 64 * NC; ++i) CHECK(bnn_fetch[i] == 1, "ping-pong NN-B chunk %d fetched %d times", i, bnn_fetch[i]);
  // A fragment reads of a group: row 32 fm + lrow of its half, chunk 2 ks + lhalf
  for (int g = 0; g < 2; ++g)
    for (int fm = 0; fm < 4; ++fm)
      for (int lrow = 0; lrow < 32; ++lrow)
        for (int c = 0; c < KC; ++c) {
          const int s = kc_slot<KC>(lrow, c) + fm * 32 * KC;  // a_off + fm * 32 * BK, in chunks
          CHECK(a_half_holds[g][s] == (32 * fm + lrow) * KC + c, "ping-pong A read g=%d fm=%d row %d chunk %d", g, fm,
                lrow, c);
        }
}

// ---- W4A16 decode activation slots ---------------------------------------------
// Load lane l holds (row 8h + ld_r, chunk ld_x) of block half h, ld_r = (l >> 4) +
// 4((l >> 3) & 1), ld_x = l & 7, and stores it at h*1024 + 16 dec_slot(h, ld_r, ld_x);
// MFMA lane (c, g) = (l % 16, l / 16) of block parity beta reads (row c, chunk 4 beta + g)
// at (c >> 3)*1024 + 16 dec_slot(c >> 3, c & 7, 4 beta + g).
static void decode_slots() {
  std::vector<int> holds(128, -1);  // 16-byte slots of a 2 KB pair
  for (int h = 0; h < 2; ++h) {
    std::set<int> s;
    for (int r = 0; r < 8; ++r)
      for (int x = 0; x < 8; ++x) {
        const int v = dec_slot(h, r, x);
        CHECK(v >= 0 && v < 64, "dec_slot(%d,%d,%d) = %d outside a 1 KB half", h, r, x, v);
        s.insert(v);
      }
    CHECK(s.size() == 64, "dec_slot(%d, ., .) is not a bijection (%zu slots)", h, s.size());
    for (int quarter = 0; quarter < 4; ++quarter) {
      std::set<int> banks;
      for (int l = 16 * quarter; l < 16 * quarter + 16; ++l) {
        const int ld_r = (l >> 4) + 4 * ((l >> 3) & 1), ld_x = l & 7;
        const int slot = h * 64 + dec_slot(h, ld_r, ld_x);
        CHECK(holds[slot] < 0, "decode slot %d stored twice", slot);
        holds[slot] = (8 * h + ld_r) * 8 + ld_x;
        banks.insert(slot % 16);
      }
      CHECK(banks.size() == 16, "decode store quarter %d of half %d: %zu bank groups", quarter, h, banks.size());
    }
  }
  for (int beta = 0; beta < 2; ++beta)
    for (int g = 0; g < 4; ++g) {
      std::set<int> banks;
      for (int c = 0; c < 16; ++c) {
        const int slot = (c >> 3) * 64 + dec_slot(c >> 3, c & 7, 4 * beta + g);
        CHECK(holds[slot] == c * 8 + 4 * beta + g, "decode read beta=%d lane (%d,%d) finds row %d chunk %d", beta, c, g,
              holds[slot] / 8, holds[slot] % 8);
        banks.insert(slot % 16);
      }
      CHECK(banks.size() == 16, "decode read beta=%d g=%d: %zu bank groups", beta, g, banks.size());
    }
}

int main() {
  // Tile shapes of the prebuilt variants: rows 32..256, BK 16 / 32 / 64 (KC 2 / 4 / 8),
  // NN tile_n 64 / 128 / 256 (NC 8 / 16 / 32) with BK k-rows; 2 to 8 waves.
  for (int rows : {32, 64, 128, 256})
    for (int nw : {2, 4, 8}) {
      if (rows * 2 >= 64) kc_tile<2>(rows, nw);
      kc_tile<4>(rows, nw);
      kc_tile<8>(rows, nw);
    }
  for (int krows : {16, 32, 64})
    for (int nw : {2, 4, 8}) {
      nn_tile<8>(krows, nw);
      nn_tile<16>(krows, nw);
      nn_tile<32>(krows, nw);
    }
  pingpong();
  decode_slots();
  printf("%d checks, %d failures\n", g_checks, g_fail);
  return g_fail ? 1 : 0;
}
