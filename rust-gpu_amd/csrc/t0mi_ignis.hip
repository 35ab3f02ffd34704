// t0mi_ignis.hip — the callers around the GEMM path: Ignis matmul
// (src/ignis/ops/bf16_matmul.rs:33-423) and the GPTQ container conversion
// (src/t0/quant_kernels.rs:177-294), with their data movement on the GPU.
//
// The reference reads its f32 operands back to the host, converts them to bf16
// (round to nearest even, bf16_matmul.rs:372), transposes W, pads every
// dimension to the tile size, uploads, runs the NT kernel and unpads the f32
// result with a second kernel.  Here one HBM-bound kernel converts (and, for
// the weight gradient's X^T operand, transposes through LDS) into a
// library-owned bf16 buffer; the GEMM takes NN or NT natively and masks ragged
// tiles, so padding is needed only to give K and N the 8-element (16-byte)
// row granularity of the GEMM's loads, and only then is the result unpadded.
#include <string.h>

#include <algorithm>

#include "t0mi_ctx.h"

using namespace t0mi;

namespace t0mi {

// dst[r][c] = RNE(src[r][c]) for r < src_rows and c < cols, 0 elsewhere in
// [rows][ld] (ld % 8 == 0): 8 outputs (one 16-byte store) per thread.
__global__ __launch_bounds__(256) void cvt_bf16_kernel(const float* __restrict__ src, uint16_t* __restrict__ dst,
                                                       uint32_t rows, uint32_t src_rows, uint32_t cols, uint32_t ld) {
  const uint32_t chunks = ld / 8;
  const size_t total = (size_t)rows * chunks;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
    const uint32_t r = (uint32_t)(i / chunks), c0 = (uint32_t)(i % chunks) * 8;
    const float* s = src + (size_t)r * cols + c0;
    float v[8];
    if (r >= src_rows) {
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = 0.0f;
    } else if (c0 + 8 <= cols && (cols % 4) == 0) {
      const f32x4 a = *(const f32x4*)s, b = *(const f32x4*)(s + 4);
      v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = c0 + j < cols ? s[j] : 0.0f;
    }
    u32x4 o;
    o.x = pack_bf16x2(v[0], v[1]);
    o.y = pack_bf16x2(v[2], v[3]);
    o.z = pack_bf16x2(v[4], v[5]);
    o.w = pack_bf16x2(v[6], v[7]);
    *(u32x4*)(dst + (size_t)r * ld + c0) = o;
  }
}

// dst[i] = RNE(src[i]) for i < count: 8 per thread (16-byte load/store pairs
// where a whole chunk is in range, element stores for the tail).
__global__ __launch_bounds__(256) void cvt_bf16_flat_kernel(const float* __restrict__ src, uint16_t* __restrict__ dst,
                                                            uint64_t count) {
  const uint64_t chunks = (count + 7) / 8;
  for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < chunks; i += (uint64_t)gridDim.x * blockDim.x) {
    const uint64_t e0 = i * 8;
    if (e0 + 8 <= count) {
      const f32x4 a = *(const f32x4*)(src + e0), b = *(const f32x4*)(src + e0 + 4);
      u32x4 o;
      o.x = pack_bf16x2(a.x, a.y);
      o.y = pack_bf16x2(a.z, a.w);
      o.z = pack_bf16x2(b.x, b.y);
      o.w = pack_bf16x2(b.z, b.w);
      *(u32x4*)(dst + e0) = o;
    } else {
      for (uint64_t e = e0; e < count; ++e) dst[e] = f32_to_bf16_rne(src[e]);
    }
  }
}

// dst[c][r] = RNE(src[r][c]) for r < rows, 0 for rows <= r < ld (dst has `cols`
// rows of ld elements).  64x64 tiles through LDS: reads are row segments of
// src, writes row segments of dst.
__global__ __launch_bounds__(256) void cvt_bf16_transpose_kernel(const float* __restrict__ src,
                                                                 uint16_t* __restrict__ dst, uint32_t rows,
                                                                 uint32_t cols, uint32_t ld) {
  __shared__ float tile[64][65];
  const uint32_t r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const uint32_t r = r0 + ty + 4 * i, c = c0 + tx;
    tile[ty + 4 * i][tx] = (r < rows && c < cols) ? src[(size_t)r * cols + c] : 0.0f;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const uint32_t c = c0 + ty + 4 * i, r = r0 + tx;  // output row c, column r
    if (c < cols && r < ld) dst[(size_t)c * ld + r] = f32_to_bf16_rne(tile[tx][ty + 4 * i]);
  }
}

// dst[r][c] = src[r][c] for c < n (src row stride ld).
__global__ __launch_bounds__(256) void unpad_f32_kernel(const float* __restrict__ src, float* __restrict__ dst,
                                                        uint32_t m, uint32_t n, uint32_t ld) {
  const size_t total = (size_t)m * n;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
    const uint32_t r = (uint32_t)(i / n), c = (uint32_t)(i % n);
    dst[i] = src[(size_t)r * ld + c];
  }
}

// GPTQ packed [N][K/2] bytes viewed as u32 [N][K/8] -> qweight u32 [K/8][N]:
// the little-endian word of GPTQ bytes 4kk..4kk+3 of row n holds elements
// 8kk..8kk+7 of that row at bits 4e (element 2i = low nibble of byte i), which
// is word (kk, n) of the W4A16 layout.  64x64 tiles through LDS.
__global__ __launch_bounds__(256) void gptq_qweight_kernel(const uint32_t* __restrict__ packed,
                                                           uint32_t* __restrict__ qweight, uint32_t N, uint32_t K8) {
  __shared__ uint32_t tile[64][65];
  const uint32_t n0 = blockIdx.y * 64, k0 = blockIdx.x * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const uint32_t n = n0 + ty + 4 * i, kk = k0 + tx;
    if (n < N && kk < K8) tile[ty + 4 * i][tx] = packed[(size_t)n * K8 + kk];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const uint32_t kk = k0 + ty + 4 * i, n = n0 + tx;
    if (n < N && kk < K8) qweight[(size_t)kk * N + n] = tile[tx][ty + 4 * i];
  }
}

// scales f32 [N][G] -> bf16 [G][N] (RNE); zeros i32 [N][G] -> u32 [G][N/8]
// (nibble e of word j = zero of column 8j + e).  One thread per output word
// of zeros, i.e. 8 columns of one group.
__global__ __launch_bounds__(256) void gptq_params_kernel(const float* __restrict__ s, const int32_t* __restrict__ z,
                                                          uint16_t* __restrict__ s_out, uint32_t* __restrict__ z_out,
                                                          uint32_t N, uint32_t G) {
  const uint32_t words = N / 8;
  const size_t total = (size_t)G * words;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
    const uint32_t g = (uint32_t)(i / words), j = (uint32_t)(i % words);
    uint32_t zw = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t n = 8 * j + e;
      s_out[(size_t)g * N + n] = f32_to_bf16_rne(s[(size_t)n * G + g]);
      zw |= ((uint32_t)z[(size_t)n * G + g] & 0xFu) << (4 * e);
    }
    z_out[i] = zw;
  }
}

}  // namespace t0mi

namespace {

int hip_fail(hipError_t e, const char* what) { return set_error(T0MI_ERR_HIP, "%s: %s", what, hipGetErrorString(e)); }

uint32_t grid_for(t0mi_ctx* ctx, size_t items) {
  return (uint32_t)std::max<size_t>(1, std::min<size_t>((items + 255) / 256, (size_t)ctx->cu_count * 8));
}

uint32_t up8(uint32_t v) { return (v + 7) & ~7u; }

// bf16 copy of f32 [src_rows][cols] into [rows][ld] (rows >= src_rows,
// ld >= cols, zero-filled beyond the source).
int cvt(t0mi_ctx* ctx, uint64_t src, uint16_t* dst, uint32_t rows, uint32_t src_rows, uint32_t cols, uint32_t ld) {
  if (rows == 0 || ld == 0) return T0MI_OK;
  hipLaunchKernelGGL(cvt_bf16_kernel, dim3(grid_for(ctx, (size_t)rows * (ld / 8))), dim3(256), 0, ctx->stream,
                     (const float*)src, dst, rows, src_rows, cols, ld);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? T0MI_OK : hip_fail(e, "bf16 conversion launch");
}

// bf16 transpose of f32 [rows][cols] into [cols][ld] (ld >= rows, zero-filled tail).
int cvt_t(t0mi_ctx* ctx, uint64_t src, uint16_t* dst, uint32_t rows, uint32_t cols, uint32_t ld) {
  if (rows == 0 || cols == 0) return T0MI_OK;
  const dim3 grid((cols + 63) / 64, (ld + 63) / 64);
  hipLaunchKernelGGL(cvt_bf16_transpose_kernel, grid, dim3(256), 0, ctx->stream, (const float*)src, dst, rows, cols,
                     ld);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? T0MI_OK : hip_fail(e, "bf16 transpose launch");
}

int common_checks(t0mi_ctx* ctx, uint64_t a, uint64_t b, uint64_t c) {
  int rc = check_ctx(ctx);
  if (rc) return rc;
  if (!a || !b || !c) return set_error(T0MI_ERR_INVALID, "null pointer");
  if ((a | b | c) & 15) return set_error(T0MI_ERR_INVALID, "buffers must be 16-byte aligned");
  return T0MI_OK;
}

// Y[m,n] = A[m,kc] . B with bf16 operands already in ctx->cvt (A at offset 0
// with row stride kp, B at b_off), f32 out.  Pads n to np when needed: the GEMM
// writes [m, np] into the tail of the buffer and the valid columns are copied.
int gemm_into(t0mi_ctx* ctx, uint32_t transpose, size_t b_off, uint64_t y, uint32_t m, uint32_t n, uint32_t np,
              uint32_t kp, size_t pad_off) {
  uint8_t* base = (uint8_t*)ctx->cvt;
  const uint64_t a = (uint64_t)base, b = (uint64_t)(base + b_off);
  if (np == n) return run_gemm_auto(ctx, transpose, a, b, y, m, n, kp);
  float* tmp = (float*)(base + pad_off);
  int rc = run_gemm_auto(ctx, transpose, a, b, (uint64_t)tmp, m, np, kp);
  if (rc) return rc;
  hipLaunchKernelGGL(unpad_f32_kernel, dim3(grid_for(ctx, (size_t)m * n)), dim3(256), 0, ctx->stream, tmp,
                     (float*)y, m, n, np);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? T0MI_OK : hip_fail(e, "unpad launch");
}

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

}  // namespace

extern "C" int t0mi_f32_to_bf16(t0mi_ctx* ctx, uint64_t src_f32, uint64_t dst_bf16, uint64_t count) {
  int rc = check_ctx(ctx);
  if (rc) return rc;
  T0MI_SUBMIT_GUARD(ctx);
  if (count == 0) return T0MI_OK;
  if (!src_f32 || !dst_bf16) return set_error(T0MI_ERR_INVALID, "null pointer");
  if ((src_f32 & 15) || (dst_bf16 & 15)) return set_error(T0MI_ERR_INVALID, "buffers must be 16-byte aligned");
  if (ctx->null_backend) return T0MI_OK;
  hipLaunchKernelGGL(cvt_bf16_flat_kernel, dim3(grid_for(ctx, (size_t)((count + 7) / 8))), dim3(256), 0, ctx->stream,
                     (const float*)src_f32, (uint16_t*)dst_bf16, count);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? T0MI_OK : hip_fail(e, "bf16 conversion launch");
}

// matmul forward: Y = bf16(X) . bf16(W) (bf16_matmul.rs:33-96, 159-209), NN.
extern "C" int t0mi_matmul_f32(t0mi_ctx* ctx, uint64_t x, uint64_t w, uint64_t y, uint32_t m, uint32_t k,
                               uint32_t n) {
  int rc = common_checks(ctx, x, w, y);
  if (rc) return rc;
  T0MI_SUBMIT_GUARD(ctx);
  if (m == 0 || n == 0) return T0MI_OK;
  const uint32_t kp = up8(k), np = up8(n);
  const size_t xa = align256((size_t)m * kp * 2), wb = align256((size_t)kp * np * 2);
  const size_t pad = np != n ? (size_t)m * np * 4 : 0;
  rc = ensure_cvt_buffer(ctx, xa + wb + pad);
  if (rc) return rc;
  if (ctx->null_backend) return T0MI_OK;
  uint8_t* base = (uint8_t*)ctx->cvt;
  if ((rc = cvt(ctx, x, (uint16_t*)base, m, m, k, kp))) return rc;
  if ((rc = cvt(ctx, w, (uint16_t*)(base + xa), kp, k, n, np))) return rc;  // rows k..kp-1 zero
  return gemm_into(ctx, T0MI_NN, xa, y, m, n, np, kp, xa + wb);
}

// matmul_with_wt_bf16 (bf16_matmul.rs:99-134): WT bf16 [n, k] used in place, NT.
extern "C" int t0mi_matmul_wt_bf16(t0mi_ctx* ctx, uint64_t x, uint64_t wt_bf16, uint64_t y, uint32_t m,
                                   uint32_t k, uint32_t n) {
  int rc = common_checks(ctx, x, wt_bf16, y);
  if (rc) return rc;
  T0MI_SUBMIT_GUARD(ctx);
  if (k % 8 || n % 8) return set_error(T0MI_ERR_INVALID, "K=%u and N=%u must be multiples of 8 (WT is used in place)", k, n);
  if (wt_bf16 & 15) return set_error(T0MI_ERR_INVALID, "WT must be 16-byte aligned");
  if (m == 0 || n == 0) return T0MI_OK;
  rc = ensure_cvt_buffer(ctx, align256((size_t)m * k * 2));
  if (rc) return rc;
  if (ctx->null_backend) return T0MI_OK;
  if ((rc = cvt(ctx, x, (uint16_t*)ctx->cvt, m, m, k, k))) return rc;
  return run_gemm_auto(ctx, T0MI_NT, (uint64_t)ctx->cvt, wt_bf16, y, m, n, k);
}

// gemm_backward_data (bf16_matmul.rs:216-262): dX[m,k] = dY[m,n] . W[k,n]^T.
// As an NT GEMM: A = dY (contraction n), B = W read as [k rows][n] (NT "WT").
extern "C" int t0mi_matmul_backward_data(t0mi_ctx* ctx, uint64_t dy, uint64_t w, uint64_t dx, uint32_t m,
                                         uint32_t k, uint32_t n) {
  int rc = common_checks(ctx, dy, w, dx);
  if (rc) return rc;
  T0MI_SUBMIT_GUARD(ctx);
  if (m == 0 || k == 0) return T0MI_OK;
  const uint32_t cp = up8(n), op = up8(k);  // contraction n, output columns k
  const size_t da = align256((size_t)m * cp * 2), wb = align256((size_t)op * cp * 2);
  const size_t pad = op != k ? (size_t)m * op * 4 : 0;
  rc = ensure_cvt_buffer(ctx, da + wb + pad);
  if (rc) return rc;
  if (ctx->null_backend) return T0MI_OK;
  uint8_t* base = (uint8_t*)ctx->cvt;
  if ((rc = cvt(ctx, dy, (uint16_t*)base, m, m, n, cp))) return rc;
  if ((rc = cvt(ctx, w, (uint16_t*)(base + da), op, k, n, cp))) return rc;  // rows k..op-1 zero
  return gemm_into(ctx, T0MI_NT, da, dx, m, k, op, cp, da + wb);
}

// gemm_backward_weight (bf16_matmul.rs:268-316): dW[k,n] = X[m,k]^T . dY[m,n].
// A = X^T (converted and transposed on the GPU, contraction m), B = dY (NN).
extern "C" int t0mi_matmul_backward_weight(t0mi_ctx* ctx, uint64_t x, uint64_t dy, uint64_t dw, uint32_t m,
                                           uint32_t k, uint32_t n) {
  int rc = common_checks(ctx, x, dy, dw);
  if (rc) return rc;
  T0MI_SUBMIT_GUARD(ctx);
  if (k == 0 || n == 0) return T0MI_OK;
  const uint32_t cp = up8(m), np = up8(n);  // contraction m, output columns n
  const size_t xa = align256((size_t)k * cp * 2), db = align256((size_t)cp * np * 2);
  const size_t pad = np != n ? (size_t)k * np * 4 : 0;
  rc = ensure_cvt_buffer(ctx, xa + db + pad);
  if (rc) return rc;
  if (ctx->null_backend) return T0MI_OK;
  uint8_t* base = (uint8_t*)ctx->cvt;
  if ((rc = cvt_t(ctx, x, (uint16_t*)base, m, k, cp))) return rc;
  if ((rc = cvt(ctx, dy, (uint16_t*)(base + xa), cp, m, n, np))) return rc;  // rows m..cp-1 zero
  return gemm_into(ctx, T0MI_NN, xa, dw, k, n, np, cp, xa + db);
}

extern "C" int t0mi_gptq_convert(t0mi_ctx* ctx, uint64_t packed, uint64_t scales_f32, uint64_t zeros_i32,
                                 uint32_t rows, uint32_t cols, uint32_t group, uint64_t qweight,
                                 uint64_t scales_bf16, uint64_t qzeros) {
  int rc = check_ctx(ctx);
  if (rc) return rc;
  T0MI_SUBMIT_GUARD(ctx);
  if (!packed || !scales_f32 || !zeros_i32 || !qweight || !scales_bf16 || !qzeros)
    return set_error(T0MI_ERR_INVALID, "null pointer");
  if (group == 0 || cols % group) return set_error(T0MI_ERR_INVALID, "K=%u must be a multiple of group=%u", cols, group);
  if (cols % 8 || rows % 8) return set_error(T0MI_ERR_INVALID, "K=%u and N=%u must be multiples of 8", cols, rows);
  if ((packed | scales_f32 | zeros_i32 | qweight | qzeros) & 3 || (scales_bf16 & 1))
    return set_error(T0MI_ERR_INVALID, "misaligned buffer (4-byte sections, 2-byte bf16 scales)");
  if (rows == 0 || cols == 0 || ctx->null_backend) return T0MI_OK;
  const uint32_t K8 = cols / 8, G = cols / group;
  hipLaunchKernelGGL(gptq_qweight_kernel, dim3((K8 + 63) / 64, (rows + 63) / 64), dim3(256), 0, ctx->stream,
                     (const uint32_t*)packed, (uint32_t*)qweight, rows, K8);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "gptq qweight launch");
  hipLaunchKernelGGL(gptq_params_kernel, dim3(grid_for(ctx, (size_t)G * (rows / 8))), dim3(256), 0, ctx->stream,
                     (const float*)scales_f32, (const int32_t*)zeros_i32, (uint16_t*)scales_bf16, (uint32_t*)qzeros,
                     rows, G);
  e = hipGetLastError();
  return e == hipSuccess ? T0MI_OK : hip_fail(e, "gptq params launch");
}
