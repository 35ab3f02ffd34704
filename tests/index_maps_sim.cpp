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
//   - the bank-conflict freedom the swizzles are designed for, under the LDS
//     rule measured on gfx950 (see lds_rules below).
// The counterpart of the reference's CPU-side locks (tests/gemm_memory_safety.rs).
// Prints each failure; exit status 1 if any.
#include <stdio.h>

#include <algorithm>
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

// ---- LDS bank rule of ds_read_b128 (gfx950) ----------------------------------
// Measured with SQ_LDS_IDX_ACTIVE / SQ_INSTS_LDS on one-pattern launches
// (t0mi_probe_lds): LDS cycles per ds_read_b128 of each lane -> address table,
// 4 when conflict-free.  The 31 observations below are the patterns of
// bench.py --only lds (lds_patterns), with the cycles measured for each.  A rule
// here: each half-wave (32 lanes) is served in two cycles, a lane going to
// cycle parity(lane & ML) ^ parity(addr & MA); a cycle costs the largest number
// of distinct addresses that share one 16-byte slot modulo 256 bytes (64 banks
// of 4 bytes).  lds_rules() keeps every (ML, MA) that reproduces all the
// measurements; layouts are checked under all of them.
static int parity(unsigned v) { return __builtin_popcount(v) & 1; }
static int b128_cycles(const int* addr, unsigned ml, unsigned ma) {
  int total = 0;
  for (int h = 0; h < 2; ++h)
    for (int cyc = 0; cyc < 2; ++cyc) {
      std::set<int> seen;
      std::vector<std::set<int>> slot(16);
      for (int l = 32 * h; l < 32 * h + 32; ++l)
        if ((parity(l & ml) ^ parity(addr[l] & ma)) == cyc) slot[(addr[l] % 256) / 16].insert(addr[l]);
      size_t worst = 0;
      for (auto& v : slot) worst = v.size() > worst ? v.size() : worst;
      total += (int)worst;
    }
  return total;
}
struct LdsRule { unsigned ml, ma; };
static std::vector<LdsRule> g_rules;
static void lds_rules() {
  struct Obs { int addr[64]; int cycles; };
  std::vector<Obs> obs;
  auto add = [&](int cycles, auto f) { Obs o; for (int l = 0; l < 64; ++l) o.addr[l] = f(l); o.cycles = cycles; obs.push_back(o); };
  auto swz8 = [](int r) { return swz<8>(r); };
  const int FAR = 16384;
  add(4, [](int l) { return 16 * l; });
  add(4, [&](int l) { return (l % 32) * 128 + ((l / 32) ^ swz8(l % 32)) * 16; });
  add(8, [&](int l) { return (l % 16) * 128 + ((l / 16) ^ swz8(l % 16)) * 16; });
  add(4, [&](int l) { return (l % 16) * 128 + ((l / 16 + l % 16) % 8) * 16; });
  add(16, [&](int l) { return (l % 16) * 128 + (l / 16) * 16; });
  add(6, [&](int l) { return l < 16 ? (l % 16) * 128 + ((l / 16) ^ swz8(l % 16)) * 16 : FAR + 16 * l; });
  add(6, [&](int l) { return l >= 16 && l < 32 ? (l % 16) * 128 + ((l / 16) ^ swz8(l % 16)) * 16 : FAR + 16 * l; });
  add(8, [&](int l) { return (l & 31) < 16 ? (l % 16) * 128 + ((l / 16) ^ swz8(l % 16)) * 16 : FAR + 16 * l; });
  add(4, [&](int l) { return l < 32 ? (l % 32) * 128 + ((l / 32) ^ swz8(l % 32)) * 16 : FAR + 16 * l; });
  add(4, [&](int l) { return (l / 16) * 256 + (l % 16) * 16; });
  // rows of 32 K (64 bytes) under the former swizzle of swz<4>, then the current one
  auto swz4_old = [](int r) { return ((r / 2) ^ ((r >> 3) & 3)) & 3; };
  add(8, [&](int l) { return ((l % 32) * 4 + ((l / 32) ^ swz4_old(l % 32))) * 16; });
  add(8, [&](int l) { return ((l % 32) * 4 + ((2 + l / 32) ^ swz4_old(l % 32))) * 16; });
  add(4, [&](int l) { return ((l % 32) * 4 + ((l / 32) ^ ((l % 32 >> 2) & 3))) * 16; });
  add(4, [&](int l) { return ((l % 32) * 4 + ((2 + l / 32) ^ ((l % 32 >> 2) & 3))) * 16; });
  add(6, [&](int l) { return l < 16 ? 32 * l : FAR + 16 * l; });
  add(4, [&](int l) { return l < 16 ? 32 * l : l < 32 ? (l - 16) * 32 + 16 : FAR + 16 * l; });
  add(4, [&](int l) { return l < 16 ? 16 * l : l < 32 ? (l - 16) * 16 + 4096 : FAR + 16 * l; });
  for (int b = 0; b < 6; ++b)
    for (int d : {256, 512, 1024}) {
      if (d != 1024 && (b == 1 || b == 2)) continue;  // not measured
      add(b <= 3 ? 8 : 4, [&](int l) { return (l & ~(1 << b)) * 16 + ((l >> b) & 1) * d; });
    }
  for (unsigned ml = 0; ml < 32; ++ml)
    for (unsigned ma = 0; ma < 4096; ma += 16) {
      bool ok = true;
      for (auto& o : obs)
        if (b128_cycles(o.addr, ml, ma) != o.cycles) { ok = false; break; }
      if (ok) g_rules.push_back({ml, ma});
    }
  CHECK(!g_rules.empty(), "no LDS rule reproduces the measurements");
}
// The most cycles one ds_read_b128 of this lane -> address table takes under
// any rule that fits the measurements.
static int b128_worst(const int* addr) {
  int w = 0;
  for (auto& r : g_rules) { const int c = b128_cycles(addr, r.ml, r.ma); w = c > w ? c : w; }
  return w;
}

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
  // ds_read_b128 of the 32x32x16 operand: lane l reads row r0 + l % 32 at
  // logical chunk c + l / 32 (KC >= 2) -- conflict-free under the measured rule.
  for (int r0 = 0; r0 + 32 <= rows; r0 += 32)
    for (int c = 0; c + 1 < KC; c += 2) {
      int addr[64];
      for (int l = 0; l < 64; ++l) addr[l] = kc_slot<KC>(r0 + l % 32, c + l / 32) * 16;
      const int cyc = b128_worst(addr);
      CHECK(cyc == 4, "KC=%d rows %d.. chunk %d: %d LDS cycles per read", KC, r0, c, cyc);
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
// block w4); B loads j = 0..3 fill, NN: blocks 4g + w4 + 8j of the B tile
// (base address moved by 16 k-rows per j, one lane offset from block 4g + w4);
// NT: blocks 16g + w4 + 4j (resource at row g*128 + 32 j).  X16: the 16x16x32
// operand maps (rot16 rows, swz_nn<32, true>, x16_krow / x16_col).
template <bool X16>
static void pingpong() {
  constexpr int KC = 8, NC = 32;
  std::vector<int> a_fetch(256 * KC, 0), bnn_fetch(64 * NC, 0), bnt_fetch(256 * KC, 0);
  std::vector<int> a_half_holds[2] = {std::vector<int>(128 * KC, -1), std::vector<int>(128 * KC, -1)};
  std::vector<int> bnt_holds(256 * KC, -1), bnn_holds(64 * NC, -1);
  for (int g = 0; g < 2; ++g)
    for (int w4 = 0; w4 < 4; ++w4)
      for (int lane = 0; lane < 64; ++lane) {
        int row, lc, brow, blc;
        kc_dma_chunk<KC, X16>(w4 * 64 + lane, &row, &lc);                // the kernel's a_voff / NT b_voff
        nn_dma_chunk<NC, X16>((4 * g + w4) * 64 + lane, &brow, &blc);    // the kernel's NN b_voff
        CHECK(row < 32, "ping-pong A lane offset row %d leaves its 32-row block", row);
        for (int j = 0; j < 4; ++j) {
          // A: LDS slot (4j + w4) * 64 + lane of the half; source row 32 j + row of the half
          const int q = (4 * j + w4) * 64 + lane;
          int r2, l2;
          kc_dma_chunk<KC, X16>(q, &r2, &l2);
          CHECK(r2 == 32 * j + row && l2 == lc, "ping-pong A j=%d w4=%d lane=%d: slot wants (%d,%d), load gives (%d,%d)",
                j, w4, lane, r2, l2, 32 * j + row, lc);
          a_fetch[(g * 128 + 32 * j + row) * KC + lc]++;
          a_half_holds[g][q] = (32 * j + row) * KC + lc;
          // NN B: block 4g + w4 + 8j, k-rows 16 j further
          const int qb = (4 * g + w4 + 8 * j) * 64 + lane;
          int k3, l3;
          nn_dma_chunk<NC, X16>(qb, &k3, &l3);
          CHECK(k3 == brow + 16 * j && l3 == blc, "ping-pong NN B j=%d: slot wants (%d,%d), load gives (%d,%d)", j, k3,
                l3, brow + 16 * j, blc);
          if (brow + 16 * j < 64) {
            bnn_fetch[(brow + 16 * j) * NC + blc]++;
            bnn_holds[qb] = (brow + 16 * j) * NC + blc;
          }
          // NT B: block 16g + w4 + 4j of [256 n][8 chunks]
          const int qt = (16 * g + w4 + 4 * j) * 64 + lane;
          int r4, l4;
          kc_dma_chunk<KC, X16>(qt, &r4, &l4);
          CHECK(r4 == g * 128 + 32 * j + row && l4 == lc, "ping-pong NT B j=%d: (%d,%d) vs (%d,%d)", j, r4, l4,
                g * 128 + 32 * j + row, lc);
          bnt_fetch[(g * 128 + 32 * j + row) * KC + lc]++;
          bnt_holds[qt] = (g * 128 + 32 * j + row) * KC + lc;
        }
      }
  for (int i = 0; i < 256 * KC; ++i) CHECK(a_fetch[i] == 1 && bnt_fetch[i] == 1, "ping-pong A/NT-B chunk %d", i);
  for (int i = 0; i < 64 * NC; ++i) CHECK(bnn_fetch[i] == 1, "ping-pong NN-B chunk %d fetched %d times", i, bnn_fetch[i]);
  // K-contiguous fragment reads: lane l of block fm reads row MB fm + l % MB of
  // the group's half at chunk KG ks + l / MB, through the kernel's a_off[ks]
  // (computed for block 0) plus MB fm rows.
  constexpr int MB = X16 ? 16 : 32, KG = 64 / MB, KS = X16 ? 2 : 4, FM = 128 / MB;
  for (int g = 0; g < 2; ++g)
    for (int ks = 0; ks < KS; ++ks)
      for (int fm = 0; fm < FM; ++fm) {
        int addr[64];
        for (int lane = 0; lane < 64; ++lane) {
          const int r = fm * MB + lane % MB, c = ks * KG + lane / MB;
          const int s = kc_slot<KC, X16>(lane % MB, c) + fm * MB * KC;
          CHECK(a_half_holds[g][s] == r * KC + c, "ping-pong A read g=%d ks=%d fm=%d lane %d", g, ks, fm, lane);
          addr[lane] = s * 16;
          // NT B fragments read the same way from rows wn*64 + ... of the B tile
          for (int wn = 0; wn < 4 && fm < 64 / MB; ++wn) {
            const int sb = kc_slot<KC, X16>(wn * 64 + lane % MB, c) + fm * MB * KC;
            CHECK(bnt_holds[sb] == (wn * 64 + fm * MB + lane % MB) * KC + c, "ping-pong NT B read wn=%d fm=%d", wn, fm);
          }
        }
        const int cyc = b128_worst(addr);
        CHECK(cyc == 4, "ping-pong%s A read ks=%d fm=%d: %d LDS cycles", X16 ? " X16" : "", ks, fm, cyc);
      }
  // NN transpose reads: lane l of k-step ks, half h, block fn addresses k-row
  // ks*KK + 4h + krow0(l) and the 4 columns at wn*64 + fn*MB + col0(l); the
  // hoisted swizzle of krow0 must serve every k-row the lane reads.
  constexpr int KK = X16 ? 32 : 16, FN = 64 / MB;
  for (int wn = 0; wn < 4; ++wn)
    for (int ks = 0; ks < KS; ++ks)
      for (int h = 0; h < 2; ++h)
        for (int fn = 0; fn < FN; ++fn) {
          std::vector<int> bank_use(64, 0);
          for (int lane = 0; lane < 64; ++lane) {
            const int tg = lane >> 4, ti = lane & 15;
            const int krow0 = X16 ? x16_krow(lane, 0) : 8 * (tg >> 1) + (ti >> 2);
            const int col0 = wn * 64 + (X16 ? x16_col(lane) : 16 * (tg & 1) + 4 * (ti & 3));
            const int k = ks * KK + 4 * h + krow0, col = col0 + fn * MB;
            CHECK((swz_nn<NC, X16>(k)) == (swz_nn<NC, X16>(krow0)), "ping-pong NN swizzle of k-row %d", k);
            const int e = k * NC * 8 + nn_col_off(col, swz_nn<NC, X16>(krow0));
            const int held = bnn_holds[e / 8];
            CHECK(held / NC == k && (held % NC) * 8 + e % 8 == col, "ping-pong NN read (%d,%d) finds (%d,%d)", k, col,
                  held / NC, (held % NC) * 8 + e % 8);
            if (lane == 32) {
              for (int b = 0; b < 64; ++b)
                CHECK(bank_use[b] <= 1, "ping-pong NN tr ks=%d h=%d fn=%d lanes 0-31: bank %d used %d times", ks, h, fn,
                      b, bank_use[b]);
              std::fill(bank_use.begin(), bank_use.end(), 0);
            }
            bank_use[(e * 2 / 4) % 64]++;
            bank_use[(e * 2 / 4 + 1) % 64]++;
          }
          for (int b = 0; b < 64; ++b)
            CHECK(bank_use[b] <= 1, "ping-pong NN tr ks=%d h=%d fn=%d lanes 32-63: bank %d used %d times", ks, h, fn, b,
                  bank_use[b]);
        }
  if (X16) {
    // the transpose-read lane map gives the 16x16x32 B operand: within each
    // 16-lane group, lane L receives element (L % 4) of the chunks addressed by
    // lanes 4e + L / 4 (e = 0..3), i.e. k-row x16_krow(4e + L/4) at column
    // x16_col(4e + L/4) + L % 4; it must be k-row 8 (l / 16) + 4 h + e, column l % 16
    for (int lane = 0; lane < 64; ++lane)
      for (int h = 0; h < 2; ++h)
        for (int e = 0; e < 4; ++e) {
          const int src = (lane & ~15) + 4 * e + (lane & 15) / 4;
          CHECK(x16_krow(src, h) == 8 * (lane >> 4) + 4 * h + e && x16_col(src) + (lane & 3) == (lane & 15),
                "x16 transpose map lane %d h %d e %d", lane, h, e);
        }
    // output staging: each (row, 16-byte chunk) of a wave's 128 x 64 bf16 block
    // has its own slot
    std::set<int> slots;
    for (int r = 0; r < 128; ++r)
      for (int c = 0; c < 8; ++c) slots.insert(r * 8 + (c ^ stage_swz16(r)));
    CHECK(slots.size() == 1024, "X16 output staging is not a bijection");
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

// ---- persistent decode kernel, NN block ------------------------------------------
// Lane l stores 8 columns 8 (l & 1) .. +7 of K row nn_pd_krow(l) at byte 16 l of a 1 KB
// block.  ds_read_b64_tr_b16 at byte offset o: within each 16-lane group, lane L receives
// element L % 4 of the 8-byte chunks addressed by lanes 4e + L / 4 (e = 0..3).  The 16x16x32
// B operand needs, in read h, K rows 8 (L / 16) + 4 h + e of column L % 16.
static void persistent_nn_block() {
  std::vector<int> krow_of(1024, -1), col_of(1024, -1);  // per byte pair: K row, column
  std::set<int> pieces;
  for (int l = 0; l < 64; ++l) {
    const int k = nn_pd_krow(l), c0 = 8 * (l & 1);
    CHECK(k >= 0 && k < 32, "nn_pd_krow(%d) = %d", l, k);
    pieces.insert(k * 2 + (l & 1));
    for (int j = 0; j < 8; ++j) {
      krow_of[16 * l + 2 * j] = k;
      col_of[16 * l + 2 * j] = c0 + j;
    }
  }
  CHECK(pieces.size() == 64, "NN persistent block stores are not a bijection (%zu pieces)", pieces.size());
  for (int h = 0; h < 2; ++h) {
    for (int half = 0; half < 2; ++half) {  // a transpose read is served 32 lanes at a time
      std::set<int> chunks;
      int lo = 1 << 30, hi = -1;
      for (int l = 32 * half; l < 32 * half + 32; ++l) {
        const int o = nn_pd_tr_off(l, h);
        CHECK(o >= 0 && o + 8 <= 1024 && o % 8 == 0, "nn_pd_tr_off(%d,%d) = %d", l, h, o);
        chunks.insert(o / 8);
        lo = std::min(lo, o);
        hi = std::max(hi, o + 8);
      }
      CHECK(chunks.size() == 32 && hi - lo == 256, "NN persistent tr read h=%d lanes %d-%d: %zu chunks over %d bytes", h,
            32 * half, 32 * half + 31, chunks.size(), hi - lo);
    }
    for (int L = 0; L < 64; ++L)
      for (int e = 0; e < 4; ++e) {
        const int src = (L & ~15) + 4 * e + (L & 15) / 4;
        const int byte = nn_pd_tr_off(src, h) + 2 * (L % 4);
        CHECK(krow_of[byte] == 8 * (L >> 4) + 4 * h + e && col_of[byte] == (L & 15),
              "NN persistent read h=%d lane %d element %d finds (k %d, col %d)", h, L, e, krow_of[byte], col_of[byte]);
      }
  }
}

// ---- in-launch split-K numbering (xk_unpack) -----------------------------------
// Over the launch's grid (tiles rounded up to a multiple of nx, times pieces): every
// (tile, piece) of the real tiles appears exactly once, padding ids name tiles past the
// count, and every piece of a tile has the id modulo nx of the others (one XCD).
static void xk_numbering(uint32_t tiles, uint32_t pieces, uint32_t nx) {
  const uint32_t grid = (tiles + nx - 1) / nx * nx * pieces;
  std::vector<int> seen((size_t)tiles * pieces, 0);
  std::vector<int> xcd(tiles, -1);
  for (uint32_t id = 0; id < grid; ++id) {
    uint32_t t, pc;
    xk_unpack(id, nx, pieces, &t, &pc);
    CHECK(pc < pieces, "xk %u x%u nx %u: id %u -> piece %u", tiles, pieces, nx, id, pc);
    if (t >= tiles) continue;  // padding
    ++seen[(size_t)t * pieces + pc];
    if (xcd[t] < 0) xcd[t] = (int)(id % nx);
    CHECK(xcd[t] == (int)(id % nx), "xk %u x%u: tile %u on ids of residues %d and %u", tiles, pieces, t, xcd[t],
          id % nx);
  }
  for (size_t i = 0; i < seen.size(); ++i)
    CHECK(seen[i] == 1, "xk %u x%u nx %u: (tile %zu, piece %zu) taken %d times", tiles, pieces, nx, i / pieces,
          i % pieces, seen[i]);
}

int main() {
  lds_rules();
  printf("%zu LDS rules fit the measurements\n", g_rules.size());
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
  persistent_nn_block();
  pingpong<false>();
  pingpong<true>();
  decode_slots();
  for (uint32_t tiles : {1u, 7u, 22u, 90u, 171u, 256u})
    for (uint32_t pieces : {1u, 2u, 3u, 8u, 16u})
      for (uint32_t nx : {1u, 8u}) xk_numbering(tiles, pieces, nx);
  printf("%d checks, %d failures\n", g_checks, g_fail);
  return g_fail ? 1 : 0;
}
