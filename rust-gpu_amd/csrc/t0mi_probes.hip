// t0mi_probes.hip — measurement kernels behind the floors the GEMM and W4A16
// kernels are judged against (built as libt0mi_probes.so, apart from the
// product library; driven by bench.py --only stream / mfma):
//   - a streaming read of a buffer with 16-byte loads, normal or non-temporal
//     (the W4A16 decode's weight loads): the best any kernel reading those
//     bytes once can do, and the calibration of rocprofv3 FETCH_SIZE for that
//     load type;
//   - an empty kernel: the per-launch cost of back-to-back dispatches;
//   - a pure MFMA loop (v_mfma_f32_32x32x16_bf16, the GEMM's instruction, in
//     the ping-pong kernel's per-phase pattern) on random or zero operands,
//     with s_memtime / s_memrealtime stamps: the FLOP rate and the shader clock
//     the power limit allows with no memory traffic at all.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

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

// 8 waves (two per SIMD), each with the ping-pong kernel's register set: 16 A
// and 8 B fragments (4 k-steps of 4 x 2 fragments) and 8 accumulators of
// 32x32; one iteration = the 32 MFMAs of a 64-K tile.  Wave 0 of each
// workgroup records (s_memtime, s_memrealtime) before and after its loop.
__global__ __launch_bounds__(512) void probe_mfma(const bf16x8* __restrict__ src, uint32_t n_frag, uint32_t iters,
                                                  float* __restrict__ out, uint64_t* __restrict__ stamps) {
  bf16x8 xa[4][4], xb[4][2];
  const uint32_t t = blockIdx.x * 512 + threadIdx.x;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
    for (int f = 0; f < 4; ++f) xa[ks][f] = src[(t * 24 + ks * 6 + f) % n_frag];
#pragma unroll
    for (int f = 0; f < 2; ++f) xb[ks][f] = src[(t * 24 + ks * 6 + 4 + f) % n_frag];
  }
  f32x16 acc[2][4];
#pragma unroll
  for (int fn = 0; fn < 2; ++fn)
#pragma unroll
    for (int fm = 0; fm < 4; ++fm)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[fn][fm][r] = 0.0f;
  __syncthreads();
  const uint64_t c0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  for (uint32_t it = 0; it < iters; ++it) {
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int fn = 0; fn < 2; ++fn)
#pragma unroll
        for (int fm = 0; fm < 4; ++fm)
          acc[fn][fm] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xb[ks][fn], xa[ks][fm], acc[fn][fm], 0, 0, 0);
  }
  float s = 0.0f;
#pragma unroll
  for (int fn = 0; fn < 2; ++fn)
#pragma unroll
    for (int fm = 0; fm < 4; ++fm)
#pragma unroll
      for (int r = 0; r < 16; ++r) s += acc[fn][fm][r];
  const uint64_t c1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
  out[t] = s;
  if (threadIdx.x == 0) {
    stamps[4 * blockIdx.x + 0] = c0;
    stamps[4 * blockIdx.x + 1] = c1;
    stamps[4 * blockIdx.x + 2] = r0;
    stamps[4 * blockIdx.x + 3] = r1;
  }
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

// `grid` workgroups of 8 waves, each wave running iters x 32 MFMAs 32x32x16
// (2 * 32 * 32 * 16 * 32 FLOP per iteration) on fragments taken from src
// (n_frag 16-byte fragments).  out: grid * 512 floats; stamps: grid * 4 u64.
int t0mi_probe_mfma(void* stream, const void* src, uint32_t n_frag, uint32_t iters, uint32_t grid, float* out,
                    uint64_t* stamps) {
  if (!src || !out || !stamps || n_frag == 0 || grid == 0 || ((uintptr_t)src & 15)) return -1;
  hipLaunchKernelGGL(probe_mfma, dim3(grid), dim3(512), 0, (hipStream_t)stream, (const bf16x8*)src, n_frag, iters,
                     out, stamps);
  return launched();
}

}  // extern "C"
