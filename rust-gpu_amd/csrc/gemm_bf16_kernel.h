// gemm_bf16_kernel.h — gfx950 bf16 GEMM kernel template (MFMA 32x32x16, fp32 accumulate).
//
// Replaces the RDNA WMMA kernels that the reference generates at run time:
//   src/t0/gemm_gen.rs:668-1438   (generate_lds_db)
//   src/t0/tile_ir.rs:887-4250    (lower_gemm)
// Same math — Y[M,N] = X[M,K] . B, bf16 inputs, fp32 accumulation — but laid
// out for CDNA4: 64-wide waves, v_mfma_f32_32x32x16_bf16, a double-buffered
// LDS tile with an XOR swizzle, 128-bit global loads and a K loop that issues
// the next tile's global loads before the current tile's MFMAs.
//
// Layouts:
//   A  = X[M,K] row-major (lda = K).
//   NT: B = WT[N,K] row-major (ldb = K)  — the reference's only implemented layout.
//   NN: B = B[K,N] row-major (ldb = N)   — BASELINE.json's layout.  8x8 blocks are
//       transposed in registers (v_perm_b32) on their way into LDS, so both
//       layouts reach the MFMA loop as K-contiguous LDS rows.
// Output: f32 or bf16 (round to nearest even), optional bias / bias+ReLU.
// Split-K: partition p covers K range [p*Kp, (p+1)*Kp) and writes its own f32
// plane at Y + p*y_split_stride (src/t0/gemm_gen.rs:760-793), or, with
// reduce_ws != 0, an f32 plane in a workspace that a reduce kernel sums.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace t0mi {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

enum : uint32_t { EPI_NONE = 0, EPI_BIAS = 1, EPI_BIAS_RELU = 2 };

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
  uint32_t epilogue;      // EPI_*
  uint32_t swap_grid;     // reference grid axis convention (informational)
  uint32_t xcd_remap;     // 1: make tiles that share an XCD (L2) contiguous
};

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  // v_cvt_pk_bf16_f32 rounds to nearest even (gfx950).
  __bf16 h = (__bf16)f;
  return __builtin_bit_cast(uint16_t, h);
}

// XOR swizzle of 16-byte chunks inside an LDS row of KC chunks.  Any 8
// consecutive rows (aligned to 8) reading the same logical chunk land in 8
// distinct 16-byte slots of a 128-byte bank line, and the 8x8-transposed NN
// stores (rows 8*nb + i, i fixed) also spread over the slots.
template <int KC>
__device__ __forceinline__ int swz(int r) {
  constexpr int RPL = 8 / KC;  // rows per 128-byte line
  return ((r / RPL) ^ (r >> 3)) & (KC - 1);
}

// Linear workgroup id -> (tile_m, tile_n, partition).
// Workgroups are dispatched round-robin over the 8 XCDs; with xcd_remap the
// ids that run on the same XCD (same L2) are made contiguous, then tiles are
// walked in groups of GROUP_M tile rows so each XCD works on a compact block
// of output tiles (shared A rows / B columns stay L2-resident).
__device__ __forceinline__ void tile_coords(const GemmParams& p, int& tm, int& tn, int& part) {
  uint32_t nwg = gridDim.x * gridDim.y;
  uint32_t lin = blockIdx.x + blockIdx.y * gridDim.x;
  if (p.xcd_remap && (nwg % 8u) == 0u) lin = (lin % 8u) * (nwg / 8u) + lin / 8u;
  uint32_t tiles = p.tiles_m * p.tiles_n;
  part = (int)(lin / tiles);
  uint32_t t = lin % tiles;
  const uint32_t GROUP_M = 4;
  uint32_t group_size = GROUP_M * p.tiles_n;
  uint32_t g = t / group_size;
  uint32_t first_m = g * GROUP_M;
  uint32_t gm = p.tiles_m - first_m < GROUP_M ? p.tiles_m - first_m : GROUP_M;
  uint32_t r = t % group_size;
  tm = (int)(first_m + r % gm);
  tn = (int)(r / gm);
}

template <int BM, int BN, int BK, int WM, int WN, bool NN>
__global__ __launch_bounds__(WM * WN * 64) void gemm_bf16_kernel(GemmParams p) {
  constexpr int NTHR = WM * WN * 64;
  constexpr int TM = BM / WM, TN = BN / WN;  // per-wave tile
  constexpr int FM = TM / 32, FN = TN / 32;  // 32x32 MFMA blocks per wave
  constexpr int KC = BK / 8;                 // 16-byte chunks per LDS row
  constexpr int KS = BK / 16;                // MFMA k-steps per tile
  static_assert(TM % 32 == 0 && TN % 32 == 0, "wave tile must be a multiple of 32x32");
  static_assert(BK == 16 || BK == 32 || BK == 64, "tile_k must be 16, 32 or 64");
  constexpr int A_CH = BM * KC;                    // 16-byte chunks of the A tile
  constexpr int A_LD = (A_CH + NTHR - 1) / NTHR;   // per thread
  constexpr int B_CH = BN * KC;                    // NT: chunks of the B tile
  constexpr int B_LD = (B_CH + NTHR - 1) / NTHR;
  constexpr int B_BLK = (BK / 8) * (BN / 8);       // NN: 8x8 blocks of the B tile
  constexpr int B_BL = (B_BLK + NTHR - 1) / NTHR;
  constexpr int A_ELEMS = BM * BK, B_ELEMS = BN * BK;

  __shared__ __attribute__((aligned(16))) uint16_t smem[2 * (A_ELEMS + B_ELEMS)];
  uint16_t* const As0 = smem;
  uint16_t* const Bs0 = smem + 2 * A_ELEMS;

  int tm, tn, part;
  tile_coords(p, tm, tn, part);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int m0 = tm * BM, n0 = tn * BN;
  const int kbeg = part * (int)p.k_per_split;
  int kend = kbeg + (int)p.k_per_split;
  if (kend > (int)p.K) kend = (int)p.K;
  const int nk = kend > kbeg ? (kend - kbeg + BK - 1) / BK : 0;

  u32x4 ra[A_LD];
  u32x4 rb[NN ? B_BL * 8 : B_LD];

  auto gload = [&](int k0) {
#pragma unroll
    for (int j = 0; j < A_LD; ++j) {
      const int i = tid + j * NTHR;
      const int row = i / KC, c = i % KC;
      int gr = m0 + row;
      gr = gr < (int)p.M ? gr : (int)p.M - 1;
      const int gk = k0 + c * 8;
      u32x4 v = {0u, 0u, 0u, 0u};
      if ((A_CH % NTHR == 0 || i < A_CH) && gk < kend)
        v = *(const u32x4*)(p.a + (size_t)gr * p.lda + gk);
      ra[j] = v;
    }
    if constexpr (!NN) {
#pragma unroll
      for (int j = 0; j < B_LD; ++j) {
        const int i = tid + j * NTHR;
        const int row = i / KC, c = i % KC;
        int gr = n0 + row;
        gr = gr < (int)p.N ? gr : (int)p.N - 1;
        const int gk = k0 + c * 8;
        u32x4 v = {0u, 0u, 0u, 0u};
        if ((B_CH % NTHR == 0 || i < B_CH) && gk < kend)
          v = *(const u32x4*)(p.b + (size_t)gr * p.ldb + gk);
        rb[j] = v;
      }
    } else {
#pragma unroll
      for (int j = 0; j < B_BL; ++j) {
        const int bi = tid + j * NTHR;
        const int kb = bi / (BN / 8), nb = bi % (BN / 8);
        const int gn = n0 + nb * 8;
        const bool ok = (B_BLK % NTHR == 0 || bi < B_BLK) && gn < (int)p.N;
#pragma unroll
        for (int r = 0; r < 8; ++r) {
          const int gk = k0 + kb * 8 + r;
          u32x4 v = {0u, 0u, 0u, 0u};
          if (ok && gk < kend) v = *(const u32x4*)(p.b + (size_t)gk * p.ldb + gn);
          rb[j * 8 + r] = v;
        }
      }
    }
  };

  auto sstore = [&](int buf) {
    uint16_t* As = As0 + buf * A_ELEMS;
    uint16_t* Bs = Bs0 + buf * B_ELEMS;
#pragma unroll
    for (int j = 0; j < A_LD; ++j) {
      const int i = tid + j * NTHR;
      if (A_CH % NTHR == 0 || i < A_CH) {
        const int row = i / KC, c = i % KC;
        *(u32x4*)(As + row * BK + ((c ^ swz<KC>(row)) * 8)) = ra[j];
      }
    }
    if constexpr (!NN) {
#pragma unroll
      for (int j = 0; j < B_LD; ++j) {
        const int i = tid + j * NTHR;
        if (B_CH % NTHR == 0 || i < B_CH) {
          const int row = i / KC, c = i % KC;
          *(u32x4*)(Bs + row * BK + ((c ^ swz<KC>(row)) * 8)) = rb[j];
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < B_BL; ++j) {
        const int bi = tid + j * NTHR;
        if (B_BLK % NTHR == 0 || bi < B_BLK) {
          const int kb = bi / (BN / 8), nb = bi % (BN / 8);
          const u32x4* in = &rb[j * 8];
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            // column i of the 8x8 block: k = 0..7 from rows 0..7, packed in pairs.
            const int d = i >> 1;
            const uint32_t sel = (i & 1) ? 0x07060302u : 0x05040100u;
            u32x4 o;
            o.x = __builtin_amdgcn_perm(in[1][d], in[0][d], sel);
            o.y = __builtin_amdgcn_perm(in[3][d], in[2][d], sel);
            o.z = __builtin_amdgcn_perm(in[5][d], in[4][d], sel);
            o.w = __builtin_amdgcn_perm(in[7][d], in[6][d], sel);
            const int row = nb * 8 + i;
            *(u32x4*)(Bs + row * BK + ((kb ^ swz<KC>(row)) * 8)) = o;
          }
        }
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

  const int lrow = lane & 31;
  const int lhalf = lane >> 5;

  if (nk > 0) {
    gload(kbeg);
    sstore(0);
    __syncthreads();
  }
  for (int it = 0; it < nk; ++it) {
    const int cur = it & 1;
    if (it + 1 < nk) gload(kbeg + (it + 1) * BK);
    const uint16_t* As = As0 + cur * A_ELEMS;
    const uint16_t* Bs = Bs0 + cur * B_ELEMS;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int c = ks * 2 + lhalf;
      bf16x8 xa[FM], xb[FN];
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) {
        const int row = wm * TM + fm * 32 + lrow;
        xa[fm] = *(const bf16x8*)(As + row * BK + ((c ^ swz<KC>(row)) * 8));
      }
#pragma unroll
      for (int fn = 0; fn < FN; ++fn) {
        const int row = wn * TN + fn * 32 + lrow;
        xb[fn] = *(const bf16x8*)(Bs + row * BK + ((c ^ swz<KC>(row)) * 8));
      }
#pragma unroll
      for (int fn = 0; fn < FN; ++fn)
#pragma unroll
        for (int fm = 0; fm < FM; ++fm)
          acc[fn][fm] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xb[fn], xa[fm], acc[fn][fm], 0, 0, 0);
    }
    if (it + 1 < nk) sstore(cur ^ 1);
    __syncthreads();
  }

  // Epilogue.  Lane l of block (fn, fm) holds C[m][n] for
  //   m = fm*32 + (l & 31),  n = fn*32 + 8*g + 4*(l >> 5) + {0..3},  g = 0..3,
  // i.e. four consecutive columns per (lane, g): one 16-byte (f32) or
  // 8-byte (bf16) store.
  const bool partial_plane = p.split_k > 1;
  char* ybase = (char*)p.y + (partial_plane ? (size_t)part * p.y_split_stride : 0);
#pragma unroll
  for (int fm = 0; fm < FM; ++fm) {
    const int m = m0 + wm * TM + fm * 32 + lrow;
    if (m >= (int)p.M) continue;
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int n = n0 + wn * TN + fn * 32 + g * 8 + lhalf * 4;
        if (n >= (int)p.N) continue;
        float v0 = acc[fn][fm][g * 4 + 0], v1 = acc[fn][fm][g * 4 + 1];
        float v2 = acc[fn][fm][g * 4 + 2], v3 = acc[fn][fm][g * 4 + 3];
        if (!partial_plane && p.epilogue != EPI_NONE) {
          v0 += p.bias[n]; v1 += p.bias[n + 1]; v2 += p.bias[n + 2]; v3 += p.bias[n + 3];
          if (p.epilogue == EPI_BIAS_RELU) {
            v0 = fmaxf(v0, 0.0f); v1 = fmaxf(v1, 0.0f); v2 = fmaxf(v2, 0.0f); v3 = fmaxf(v3, 0.0f);
          }
        }
        if (!partial_plane && p.out_bf16) {
          u32x2 o;
          o.x = (uint32_t)f32_to_bf16_rne(v0) | ((uint32_t)f32_to_bf16_rne(v1) << 16);
          o.y = (uint32_t)f32_to_bf16_rne(v2) | ((uint32_t)f32_to_bf16_rne(v3) << 16);
          *(u32x2*)((uint16_t*)ybase + (size_t)m * p.ldy + n) = o;
        } else {
          f32x4 o = {v0, v1, v2, v3};
          *(f32x4*)((float*)ybase + (size_t)m * p.ldy + n) = o;
        }
      }
    }
  }
}

}  // namespace t0mi
