// t0mi_probes.hip — measurement kernels behind the floors the GEMM and W4A16
// kernels are judged against (built as libt0mi_probes.so, apart from the
// product library; driven by bench.py --only stream / mfma):
//   - a streaming read of a buffer with 16-byte loads, normal or non-temporal
//     (the W4A16 decode's weight loads): the best any kernel reading those
//     bytes once can do, and the calibration of rocprofv3 FETCH_SIZE for that
//     load type;
//   - an empty kernel: the per-launch cost of back-to-back dispatches;
//   - MFMA loops (32x32x16 or 16x16x32 bf16, with the register set of a GEMM
//     wave tile of 128 x 64 or 128 x 128, operands in registers or re-read from
//     LDS) on random or zero operands, with s_memtime / s_memrealtime stamps:
//     the FLOP rate and the shader clock the power limit allows with no HBM
//     traffic, and what the LDS reads of each wave tile cost in clock.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Each thread reads UNROLL 16-byte elements per step, `stride` elements apart,
// and folds them with XOR; a workgroup stores its fold only if it equals a
// value the host never passes, so every load stays live and nothing is written.
template <bool NT, int UNROLL>
__global__ __launch_bounds__(256) void probe_stream(const u32x4* __restrict__ src, size_t n16, uint32_t never,
                                                    uint32_t* __restrict__ sink) {
  const size_t stride = (size_t)gridDim.x * 256;
  u32x4 acc = {0u, 0u, 0u, 0u};
  size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  for (; i + (UNROLL - 1) * stride < n16; i += UNROLL * stride) {
    u32x4 v[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) v[u] = NT ? __builtin_nontemporal_load(src + i + u * stride) : src[i + u * stride];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) acc ^= v[u];
  }
  for (; i < n16; i += stride) acc ^= NT ? __builtin_nontemporal_load(src + i) : src[i];
  const uint32_t f = acc.x ^ acc.y ^ acc.z ^ acc.w;
  if (f == never) sink[blockIdx.x] = f;
}

// 2-D block read: the matrix is `rows` rows of `pitch` bytes; workgroup (cb, rb)
// reads rows [rb * R, rb * R + R) x bytes [cb * L, cb * L + L) with 16-byte loads
// (non-temporal), lanes walking the block row-major, UNROLL loads in flight per
// thread.  The access shape of a GEMM or decode workgroup's operand block.
__global__ __launch_bounds__(256) void probe_block(const char* __restrict__ src, uint32_t pitch, uint32_t L,
                                                  uint32_t R, uint32_t cblocks, uint32_t never,
                                                  uint32_t* __restrict__ sink) {
  const uint32_t cb = blockIdx.x % cblocks, rb = blockIdx.x / cblocks;
  const uint32_t chunks = L / 16, total = chunks * R;
  const char* base = src + (size_t)rb * R * pitch + (size_t)cb * L;
  u32x4 acc = {0u, 0u, 0u, 0u};
  uint32_t i = threadIdx.x;
  for (; i + 7 * 256 < total; i += 8 * 256) {
    u32x4 v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const uint32_t q = i + u * 256;
      v[u] = __builtin_nontemporal_load((const u32x4*)(base + (size_t)(q / chunks) * pitch + (q % chunks) * 16));
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) acc ^= v[u];
  }
  for (; i < total; i += 256)
    acc ^= __builtin_nontemporal_load((const u32x4*)(base + (size_t)(i / chunks) * pitch + (i % chunks) * 16));
  const uint32_t f = acc.x ^ acc.y ^ acc.z ^ acc.w;
  if (f == never) sink[blockIdx.x] = f;
}

__global__ __launch_bounds__(256) void probe_empty(uint32_t never, uint32_t* sink) {
  if (threadIdx.x == never) sink[0] = never;
}

// MFMA loop with a GEMM wave's register set.  WAVES waves per workgroup (8: two
// per SIMD, 4: one), each owning FM x FN accumulator blocks and running, per
// iteration (64 of K), the blocks' MFMAs in k-step order:
//   X16 = false: v_mfma_f32_32x32x16_bf16, 4 k-steps of 16, blocks 32 x 32;
//   X16 = true:  v_mfma_f32_16x16x32_bf16, 2 k-steps of 32, blocks 16 x 16.
// LDS = false: the fragments stay in registers (loaded once); LDS = true: every
// k-step's fragments are read from LDS (64 KB of src copied in at the start,
// ds_read_b128 of whole 1 KB blocks, conflict-free), one k-step ahead, one read
// after each of the step's first FM + FN MFMAs, waited for at the start of the
// next step -- the LDS traffic of a GEMM with that wave tile.  Wave 0 of each workgroup records (s_memtime,
// s_memrealtime) before and after its loop.
template <int WAVES, int FM, int FN, bool X16, bool LDS>
__global__ __launch_bounds__(WAVES * 64) void probe_mfma(const bf16x8* __restrict__ src, uint32_t n_frag,
                                                         uint32_t iters, float* __restrict__ out,
                                                         uint64_t* __restrict__ stamps) {
  constexpr int KS = X16 ? 2 : 4, NF = FM + FN;
  typedef float accv __attribute__((ext_vector_type(X16 ? 4 : 16)));
  __shared__ __attribute__((aligned(1024))) bf16x8 lds[LDS ? 4096 : 1];
  const uint32_t t = blockIdx.x * (WAVES * 64) + threadIdx.x;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  if constexpr (LDS) {
    for (uint32_t c = threadIdx.x; c < 4096; c += WAVES * 64) lds[c] = src[(blockIdx.x * 4096u + c) % n_frag];
  }
  // registers: without LDS all KS steps' fragments; with LDS two steps' (current, next)
  constexpr int RS = LDS ? 2 : KS;
  bf16x8 x[RS][NF];
  // block of fragment (ks, f) in iteration it: a per-iteration base below 32
  // plus ks * NF + f (< 32), so each read is one ds_read_b128 with a constant offset
  auto lds_frag = [&](uint32_t it, int ks, int f) {
    const int base = (int)((it * 5u + (uint32_t)wave * 7u) & 31u);
    return lds[(base + ks * NF + f) * 64 + lane];
  };
  if constexpr (!LDS) {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int f = 0; f < NF; ++f) x[ks][f] = src[(t * (KS * NF) + ks * NF + f) % n_frag];
  }
  accv acc[FN][FM];
#pragma unroll
  for (int fn = 0; fn < FN; ++fn)
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int r = 0; r < (X16 ? 4 : 16); ++r) acc[fn][fm][r] = 0.0f;
  __syncthreads();
  if constexpr (LDS) {
#pragma unroll
    for (int f = 0; f < NF; ++f) x[0][f] = lds_frag(0, 0, f);
  }
  const uint64_t c0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  for (uint32_t it = 0; it < iters; ++it) {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int cur = LDS ? (ks & 1) : ks, nxt = (ks + 1) & 1;
      const uint32_t nit = ks + 1 < KS ? it : it + 1;
      const int nks = ks + 1 < KS ? ks + 1 : 0;
      // this step's fragments (read during the previous step) have landed; the
      // next step's reads all follow
      if constexpr (LDS) __builtin_amdgcn_s_waitcnt(0xF | (0x7 << 4) | (0x3 << 14));
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < FN * FM; ++i) {
        const int fn = i / FM, fm = i % FM;
        if constexpr (X16)
          acc[fn][fm] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x[cur][FM + fn], x[cur][fm], acc[fn][fm], 0, 0, 0);
        else
          acc[fn][fm] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(x[cur][FM + fn], x[cur][fm], acc[fn][fm], 0, 0, 0);
        if constexpr (LDS) {
          if (i < NF) x[nxt][i] = lds_frag(nit, nks, i);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      // Keep this step's fragments live to the end of the step, so the next
      // step's reads cannot be given the registers of fragments that MFMAs
      // still in flight are reading.
      if constexpr (LDS) {
#pragma unroll
        for (int f = 0; f < NF; ++f) asm volatile("" ::"v"(x[cur][f]));
      }
    }
  }
  float s = 0.0f;
#pragma unroll
  for (int fn = 0; fn < FN; ++fn)
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int r = 0; r < (X16 ? 4 : 16); ++r) s += acc[fn][fm][r];
  const uint64_t c1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
  out[t] = s;
  if (threadIdx.x == 0) {
    stamps[4 * blockIdx.x + 0] = c0;
    stamps[4 * blockIdx.x + 1] = c1;
    stamps[4 * blockIdx.x + 2] = r0;
    stamps[4 * blockIdx.x + 3] = r1;
  }
}

// LDS read pattern: every wave of the workgroup reads, iters times, 16 bytes
// (ds_read_b128) or 8 bytes (ds_read_b64) per lane at byte offset table[lane]
// of a 64 KB LDS buffer, one read in flight per wave.  Run under rocprofv3
// with SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE, a table tells how many LDS
// cycles one read of that lane -> address pattern takes.
template <int BYTES>
__global__ __launch_bounds__(512) void probe_lds(const uint32_t* __restrict__ table, uint32_t iters,
                                                 uint32_t* __restrict__ out) {
  __shared__ __attribute__((aligned(1024))) u32x4 lds[4096];
  for (uint32_t c = threadIdx.x; c < 4096; c += 512) lds[c] = u32x4{c, c + 1u, c + 2u, c + 3u};
  __syncthreads();
  const uint32_t off = table[threadIdx.x & 63] & 0xFFF8u;
  const uint32_t addr = (uint32_t)(size_t)(const __attribute__((address_space(3))) void*)lds + off;
  u32x4 acc = {0u, 0u, 0u, 0u};
  for (uint32_t it = 0; it < iters; ++it) {
    u32x4 v = {0u, 0u, 0u, 0u};
    if constexpr (BYTES == 16) {
      asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(addr));
    } else {
      u32x2 w;
      asm volatile("ds_read_b64 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(w) : "v"(addr));
      v.x = w.x;
      v.y = w.y;
    }
    acc ^= v;
  }
  out[blockIdx.x * 512 + threadIdx.x] = acc.x ^ acc.y ^ acc.z ^ acc.w;
}

int launched() { return hipGetLastError() == hipSuccess ? 0 : -3; }

}  // namespace

extern "C" {

// Reads `bytes` (a multiple of 16) at src once with `grid` workgroups of 256
// threads; nt != 0: non-temporal loads.  sink: `grid` u32 (never written).
int t0mi_probe_stream(void* stream, const void* src, size_t bytes, int nt, uint32_t grid, uint32_t* sink) {
  if (!src || !sink || (bytes & 15) || ((uintptr_t)src & 15) || grid == 0) return -1;
  const size_t n16 = bytes / 16;
  if (nt)
    hipLaunchKernelGGL((probe_stream<true, 8>), dim3(grid), dim3(256), 0, (hipStream_t)stream, (const u32x4*)src, n16,
                       0xFFFFFFFFu, sink);
  else
    hipLaunchKernelGGL((probe_stream<false, 8>), dim3(grid), dim3(256), 0, (hipStream_t)stream, (const u32x4*)src,
                       n16, 0xFFFFFFFFu, sink);
  return launched();
}

// Reads a matrix of `rows` x `pitch` bytes once, as blocks of R rows x L bytes
// (one workgroup of 256 threads per block; L a multiple of 16 dividing pitch,
// R dividing rows).  sink: one u32 per workgroup (never written).
int t0mi_probe_block(void* stream, const void* src, uint32_t rows, uint32_t pitch, uint32_t L, uint32_t R,
                     uint32_t* sink) {
  if (!src || !sink || L == 0 || R == 0 || (L & 15) || pitch % L || rows % R || ((uintptr_t)src & 15) ||
      (pitch & 15))
    return -1;
  const uint32_t cblocks = pitch / L, grid = cblocks * (rows / R);
  hipLaunchKernelGGL(probe_block, dim3(grid), dim3(256), 0, (hipStream_t)stream, (const char*)src, pitch, L, R,
                     cblocks, 0xFFFFFFFFu, sink);
  return launched();
}

// An empty kernel of `grid` workgroups of 256 threads.
int t0mi_probe_empty(void* stream, uint32_t grid, uint32_t* sink) {
  if (!sink || grid == 0) return -1;
  hipLaunchKernelGGL(probe_empty, dim3(grid), dim3(256), 0, (hipStream_t)stream, 0xFFFFFFFFu, sink);
  return launched();
}

// `grid` workgroups running the MFMA loop `variant` for `iters` iterations
// (64 of K each) on fragments taken from src (n_frag 16-byte fragments):
//   0: 8 waves x (4 x 2 blocks 32x32x16), registers only (the ping-pong
//      GEMM's wave tile, 128 x 64);   1: the same, fragments read from LDS;
//   2: 4 waves x (4 x 4 blocks 32x32x16) (wave tile 128 x 128);  3: + LDS;
//   4: 4 waves x (8 x 8 blocks 16x16x32) (wave tile 128 x 128);  5: + LDS;
//   6: 8 waves x (8 x 4 blocks 16x16x32) (wave tile 128 x 64);   7: + LDS.
// Each SIMD runs 2^21 FLOP per iteration in every variant (a workgroup's
// count: t0mi_probe_mfma_flop).  out: grid * 512 floats; stamps: grid * 4 u64.
int t0mi_probe_mfma(void* stream, const void* src, uint32_t n_frag, uint32_t iters, uint32_t grid, float* out,
                    uint64_t* stamps, int variant) {
  if (!src || !out || !stamps || n_frag == 0 || grid == 0 || ((uintptr_t)src & 15)) return -1;
  const hipStream_t st = (hipStream_t)stream;
  const bf16x8* s = (const bf16x8*)src;
  switch (variant) {
    case 0: hipLaunchKernelGGL((probe_mfma<8, 4, 2, false, false>), dim3(grid), dim3(512), 0, st, s, n_frag, iters, out, stamps); break;
    case 1: hipLaunchKernelGGL((probe_mfma<8, 4, 2, false, true>), dim3(grid), dim3(512), 0, st, s, n_frag, iters, out, stamps); break;
    case 2: hipLaunchKernelGGL((probe_mfma<4, 4, 4, false, false>), dim3(grid), dim3(256), 0, st, s, n_frag, iters, out, stamps); break;
    case 3: hipLaunchKernelGGL((probe_mfma<4, 4, 4, false, true>), dim3(grid), dim3(256), 0, st, s, n_frag, iters, out, stamps); break;
    case 4: hipLaunchKernelGGL((probe_mfma<4, 8, 8, true, false>), dim3(grid), dim3(256), 0, st, s, n_frag, iters, out, stamps); break;
    case 5: hipLaunchKernelGGL((probe_mfma<4, 8, 8, true, true>), dim3(grid), dim3(256), 0, st, s, n_frag, iters, out, stamps); break;
    case 6: hipLaunchKernelGGL((probe_mfma<8, 8, 4, true, false>), dim3(grid), dim3(512), 0, st, s, n_frag, iters, out, stamps); break;
    case 7: hipLaunchKernelGGL((probe_mfma<8, 8, 4, true, true>), dim3(grid), dim3(512), 0, st, s, n_frag, iters, out, stamps); break;
    default: return -1;
  }
  return launched();
}

// `grid` workgroups of 8 waves reading LDS with the lane -> byte offset
// pattern table[0..63] (device memory; offsets below 64 KB, multiples of the read size),
// `iters` reads per wave of `bytes` (16 or 8) per lane.  out: grid * 512 u32.
int t0mi_probe_lds(void* stream, const uint32_t* table, uint32_t bytes, uint32_t iters, uint32_t grid,
                   uint32_t* out) {
  if (!table || !out || grid == 0 || (bytes != 16 && bytes != 8)) return -1;
  if (bytes == 16)
    hipLaunchKernelGGL(probe_lds<16>, dim3(grid), dim3(512), 0, (hipStream_t)stream, table, iters, out);
  else
    hipLaunchKernelGGL(probe_lds<8>, dim3(grid), dim3(512), 0, (hipStream_t)stream, table, iters, out);
  return launched();
}

// FLOP one workgroup of MFMA-loop `variant` runs per iteration (0 for an unknown variant).
uint64_t t0mi_probe_mfma_flop(int variant) {
  switch (variant) {
    case 0: case 1: return 8ull * 8 * 4 * (2 * 32 * 32 * 16);
    case 2: case 3: return 4ull * 16 * 4 * (2 * 32 * 32 * 16);
    case 4: case 5: return 4ull * 64 * 2 * (2 * 16 * 16 * 32);
    case 6: case 7: return 8ull * 32 * 2 * (2 * 16 * 16 * 32);
    default: return 0;
  }
}

}  // extern "C"
