/*
 * oracle.c — CPU restatement of the reference's GEMM-path arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (libt0mi) links, loads or
 * calls this file.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg use it, and only as the checker / the timed CPU baseline.
 *
 * Build: oracle/Makefile (gcc -O3 -ffp-contract=off -fopenmp, no fast-math).
 * -ffp-contract=off matters: the reference is Rust, which never contracts
 * a*b+c into an FMA, so the per-output fp32 sum must be one rounded multiply
 * followed by one rounded add, k ascending.
 *
 * Parity pins (each function says which check pins it; see tests/test_oracle.py):
 *   - bf16 conversions: known answers of tests/tile_gemm_contract.rs:137-154
 *     and the RNE closed form;
 *   - GEMM: the reference's committed torch fixtures (benchmarks/torch_ref),
 *     the integer-pattern known answers of src/t0/auto_gemm.rs:235-269,
 *     brute force against float64 on tiny shapes;
 *   - INT4: the host unit tests of src/t0/quant_kernels.rs:342-490;
 *   - epilogue chain: closed forms per op (relu/abs/neg/clamp/scale/bias exact,
 *     silu(0) = 0, silu(x) -> x and -> 0 in the tails, sigmoid-gelu at known
 *     points) and order-of-application checks.
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <math.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------ */
/* bf16 conversions                                                          */
/* ------------------------------------------------------------------------ */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* src/t0/tile_ir.rs:4681-4683 (bf16_to_f32: bits << 16). */
float orc_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

/* src/t0/tile_ir.rs:4677-4679 (f32_to_bf16: truncation, high 16 bits). */
uint16_t orc_bf16_trunc(float f) { return (uint16_t)(f2u(f) >> 16); }

/* src/ignis/ops/bf16_matmul.rs:372 and examples/test_gemm_correctness.rs:15-20:
 * round to nearest even, ((bits + 0x7FFF + ((bits>>16)&1)) >> 16).  The
 * reference formula turns a NaN with a low-only payload into Inf; NaN handling
 * is added here (quiet the NaN, keep sign and high payload), matching what
 * the GPU's v_cvt_pk_bf16_f32 produces for NaN inputs. */
uint16_t orc_bf16_rne(float f) {
  uint32_t b = f2u(f);
  if ((b & 0x7F800000u) == 0x7F800000u && (b & 0x007FFFFFu) != 0)
    return (uint16_t)((b >> 16) | 0x0040u);
  uint32_t r = ((b >> 16) & 1u) + 0x7FFFu;
  return (uint16_t)((b + r) >> 16);
}

void orc_f32_to_bf16_rne_array(const float* x, uint16_t* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = orc_bf16_rne(x[i]);
}
void orc_f32_to_bf16_trunc_array(const float* x, uint16_t* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = orc_bf16_trunc(x[i]);
}

/* ------------------------------------------------------------------------ */
/* Seeded generators (examples/test_gemm_correctness.rs:45-58)               */
/* ------------------------------------------------------------------------ */
/* xorshift64 with state = seed ^ 0xDEADBEEFCAFEBABE; each draw applies
 * <<13, >>7, <<17 and uses the high 32 bits.  u = (float)(state>>32) /
 * (float)u32::MAX, in f32 as the reference computes it (u32::MAX rounds to
 * 2^32 in f32).  U(a,b) = a + (b-a)*u in f32.  N(mu,sigma) by Box-Muller from
 * two consecutive draws, computed in double.  Nibbles are (state>>60)&0xF. */

typedef struct { uint64_t s; } orc_rng;

static inline uint64_t rng_next(orc_rng* r) {
  uint64_t s = r->s;
  s ^= s << 13;
  s ^= s >> 7;
  s ^= s << 17;
  r->s = s;
  return s;
}

static inline void rng_init(orc_rng* r, uint64_t seed) { r->s = seed ^ 0xDEADBEEFCAFEBABEull; }

/* The reference's own generator, verbatim semantics: U(-1,1) then RNE bf16. */
void orc_rand_bf16_ref(uint16_t* out, int64_t n, uint64_t seed) {
  orc_rng r; rng_init(&r, seed);
  const float umax = (float)4294967295u;
  for (int64_t i = 0; i < n; ++i) {
    uint64_t s = rng_next(&r);
    float f = ((float)(uint32_t)(s >> 32) / umax) * 2.0f - 1.0f;
    out[i] = orc_bf16_rne(f);
  }
}

void orc_gen_uniform_bf16(uint16_t* out, int64_t n, uint64_t seed, float lo, float hi) {
  orc_rng r; rng_init(&r, seed);
  const float umax = (float)4294967295u;
  const float w = hi - lo;
  for (int64_t i = 0; i < n; ++i) {
    uint64_t s = rng_next(&r);
    float u = (float)(uint32_t)(s >> 32) / umax;
    float p = w * u;
    out[i] = orc_bf16_rne(lo + p);
  }
}

void orc_gen_normal_bf16(uint16_t* out, int64_t n, uint64_t seed, float mu, float sigma) {
  orc_rng r; rng_init(&r, seed);
  const double two_pi = 6.283185307179586476925286766559;
  for (int64_t i = 0; i < n; ++i) {
    uint64_t s1 = rng_next(&r), s2 = rng_next(&r);
    /* (x+1)/(2^32+1) keeps u1 strictly inside (0,1) so log(u1) is finite. */
    double u1 = ((double)(uint32_t)(s1 >> 32) + 1.0) / 4294967297.0;
    double u2 = (double)(uint32_t)(s2 >> 32) / 4294967296.0;
    double z = sqrt(-2.0 * log(u1)) * cos(two_pi * u2);
    float v = (float)((double)mu + (double)sigma * z);
    out[i] = orc_bf16_rne(v);
  }
}

void orc_gen_nibbles(uint8_t* out, int64_t n, uint64_t seed) {
  orc_rng r; rng_init(&r, seed);
  for (int64_t i = 0; i < n; ++i) out[i] = (uint8_t)((rng_next(&r) >> 60) & 0xF);
}

/* ------------------------------------------------------------------------ */
/* GEMM: cpu_gemm_nt_bf16 (src/t0/tile_ir.rs:5021-5038)                      */
/* ------------------------------------------------------------------------ */
/* y[i,j] = sum_k f32(x[i,k]) * f32(w[.,.]) with ONE fp32 accumulator per
 * output, starting at 0.0f, k ascending, each product rounded to fp32 then
 * added.  The loops below run i-k-j (an accumulator row per i) so that the
 * j loop vectorises; each y[i,j] still sees exactly the reference's sequence
 * of roundings (0 + p0) + p1 + ... + p_{K-1}, so the result is bit-identical
 * to the reference's i-j-k order.  Rows are split across OpenMP threads;
 * summation order per output does not depend on the thread count.
 *
 * b_nn = 0: NT, B is WT[N,K] (reference layout).
 * b_nn = 1: NN, B is B[K,N] row-major (BASELINE.json layout); identical
 *           values to NT on the transposed matrix. */
static void gemm_rows_kn(const uint16_t* a, const float* bkn, float* y,
                         int64_t i0, int64_t i1, int64_t N, int64_t K) {
  for (int64_t i = i0; i < i1; ++i) {
    float* yr = y + i * N;
    for (int64_t j = 0; j < N; ++j) yr[j] = 0.0f;
    const uint16_t* ar = a + i * K;
    for (int64_t k = 0; k < K; ++k) {
      const float av = orc_bf16_to_f32(ar[k]);
      const float* br = bkn + k * N;
      for (int64_t j = 0; j < N; ++j) {
        float p = av * br[j];
        yr[j] = yr[j] + p;
      }
    }
  }
}

/* Returns 0 on success, -1 on allocation failure. nthreads <= 0: all cores. */
int orc_gemm_bf16(const uint16_t* a, const uint16_t* b, float* y,
                  int64_t M, int64_t N, int64_t K, int b_nn, int nthreads) {
  float* bkn = (float*)malloc((size_t)K * (size_t)N * sizeof(float));
  if (!bkn) return -1;
  for (int64_t k = 0; k < K; ++k)
    for (int64_t j = 0; j < N; ++j)
      bkn[k * N + j] = orc_bf16_to_f32(b_nn ? b[k * N + j] : b[j * K + k]);
#ifdef _OPENMP
  int nt = nthreads > 0 ? nthreads : omp_get_max_threads();
  #pragma omp parallel for schedule(dynamic, 1) num_threads(nt)
  for (int64_t i = 0; i < M; ++i) gemm_rows_kn(a, bkn, y, i, i + 1, N, K);
#else
  (void)nthreads;
  gemm_rows_kn(a, bkn, y, 0, M, N, K);
#endif
  free(bkn);
  return 0;
}

/* Literal i-j-k restatement of src/t0/tile_ir.rs:5021-5038 (NT only), kept
 * single-threaded and unvectorised so tests can check that the fast loop
 * above reproduces it bit for bit. */
void orc_gemm_nt_bf16_literal(const uint16_t* x, const uint16_t* wt, float* y,
                              int64_t M, int64_t N, int64_t K) {
  for (int64_t i = 0; i < M; ++i)
    for (int64_t j = 0; j < N; ++j) {
      float sum = 0.0f;
      for (int64_t k = 0; k < K; ++k) {
        float a = orc_bf16_to_f32(x[i * K + k]);
        float b = orc_bf16_to_f32(wt[j * K + k]);
        float p = a * b;
        sum = sum + p;
      }
      y[i * N + j] = sum;
    }
}

/* ------------------------------------------------------------------------ */
/* INT4 (src/t0/quant_kernels.rs)                                            */
/* ------------------------------------------------------------------------ */
/* Logical weight W[k][n], k in [0,K), n in [0,N), nibble q in 0..15.
 *
 * qweight layout: u32 word[kk][n] = sum_e q[8kk+e][n] << 4e,
 *   i.e. 8 nibbles along K per word, nibble e at bits 4e..4e+3 (the same
 *   "element 2i = low nibble" order as the reference's little-endian bytes).
 * GPTQ container layout (quant_kernels.rs:188-294): rows = N output features,
 *   cols = K; bytes packed[n][k/2], low nibble = element 2i, high = 2i+1
 *   (quant_kernels.rs:3-10, 197-199); scales f32 [n][k/g]; zp i32 [n][k/g].
 * qzeros layout (prefill, GPTQ-style): u32 zword[g][nn] = sum_e z[g][8nn+e] << 4e.
 * Dequant (quant_kernels.rs:24, 95-100): w = (float)(q - zp) * scale. */

void orc_pack_qweight(const uint8_t* q, uint32_t* w, int64_t K, int64_t N) {
  for (int64_t kk = 0; kk < K / 8; ++kk)
    for (int64_t n = 0; n < N; ++n) {
      uint32_t v = 0;
      for (int e = 0; e < 8; ++e) v |= (uint32_t)(q[(kk * 8 + e) * N + n] & 0xF) << (4 * e);
      w[kk * N + n] = v;
    }
}

void orc_unpack_qweight(const uint32_t* w, uint8_t* q, int64_t K, int64_t N) {
  for (int64_t kk = 0; kk < K / 8; ++kk)
    for (int64_t n = 0; n < N; ++n)
      for (int e = 0; e < 8; ++e) q[(kk * 8 + e) * N + n] = (uint8_t)((w[kk * N + n] >> (4 * e)) & 0xF);
}

/* q[k][n] -> GPTQ bytes packed[n][k/2]. */
void orc_pack_gptq_bytes(const uint8_t* q, uint8_t* packed, int64_t K, int64_t N) {
  for (int64_t n = 0; n < N; ++n)
    for (int64_t i = 0; i < K / 2; ++i)
      packed[n * (K / 2) + i] = (uint8_t)((q[(2 * i) * N + n] & 0xF) | ((q[(2 * i + 1) * N + n] & 0xF) << 4));
}

/* GPTQ bytes packed[n][k/2] -> q[k][n].  quant_kernels.rs:346-382: byte 0xAB
 * gives element 2i = 0xB (low), element 2i+1 = 0xA (high). */
void orc_unpack_gptq_bytes(const uint8_t* packed, uint8_t* q, int64_t K, int64_t N) {
  for (int64_t n = 0; n < N; ++n)
    for (int64_t i = 0; i < K / 2; ++i) {
      uint8_t b = packed[n * (K / 2) + i];
      q[(2 * i) * N + n] = b & 0x0F;
      q[(2 * i + 1) * N + n] = (b >> 4) & 0x0F;
    }
}

void orc_pack_qzeros(const uint8_t* z, uint32_t* zw, int64_t G, int64_t N) {
  for (int64_t g = 0; g < G; ++g)
    for (int64_t nn = 0; nn < N / 8; ++nn) {
      uint32_t v = 0;
      for (int e = 0; e < 8; ++e) v |= (uint32_t)(z[g * N + nn * 8 + e] & 0xF) << (4 * e);
      zw[g * (N / 8) + nn] = v;
    }
}

/* Exact fp32 dequant of the whole matrix into wf[k][n].
 * scales: bf16 [K/g][N]; zeros: either qzeros u32 [K/g][N/8] (zw != NULL) or
 * the constant zp_const.  (q - z) is an exact small integer and s a bf16, so
 * (float)(q - z) * s is exact in fp32. */
void orc_dequant_qweight_f32(const uint32_t* w, const uint16_t* scales, const uint32_t* zw,
                             int zp_const, float* wf, int64_t K, int64_t N, int64_t g) {
  for (int64_t k = 0; k < K; ++k) {
    int64_t gi = k / g;
    for (int64_t n = 0; n < N; ++n) {
      int q = (int)((w[(k / 8) * N + n] >> (4 * (k % 8))) & 0xF);
      int z = zw ? (int)((zw[gi * (N / 8) + n / 8] >> (4 * (n % 8))) & 0xF) : zp_const;
      float s = orc_bf16_to_f32(scales[gi * N + n]);
      wf[k * N + n] = (float)(q - z) * s;
    }
  }
}

/* The reference's GptqWeight dequant, row-major over its own [rows=N][cols=K]
 * element order: out[n*K + k] = (float)(q - zp[n][k/g]) * scale[n][k/g]
 * (quant_kernels.rs:74-100; round_mode 0 = f32 output). */
void orc_dequant_gptq_f32(const uint8_t* packed, const float* scales, const int32_t* zp,
                          float* out, int64_t rows, int64_t cols, int64_t g) {
  int64_t ng = cols / g;
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t c = 0; c < cols; ++c) {
      int64_t e = r * cols + c;
      uint8_t b = packed[e >> 1];
      int q = (e & 1) ? ((b >> 4) & 0xF) : (b & 0xF);
      int64_t gi = r * ng + c / g;
      int32_t v = (int32_t)q - zp[gi];
      out[e] = (float)v * scales[gi];
    }
}

/* W4A16 GEMM oracle: exact fp32 dequant followed by the cpu_gemm_nt_bf16 loop
 * (k ascending, one fp32 accumulator, no FMA).  y is f32 [M][N]. */
int orc_w4a16_gemm(const uint16_t* a, const uint32_t* w, const uint16_t* scales, const uint32_t* zw,
                   int zp_const, float* y, int64_t M, int64_t N, int64_t K, int64_t g, int nthreads) {
  float* wf = (float*)malloc((size_t)K * (size_t)N * sizeof(float));
  if (!wf) return -1;
  orc_dequant_qweight_f32(w, scales, zw, zp_const, wf, K, N, g);
#ifdef _OPENMP
  int nt = nthreads > 0 ? nthreads : omp_get_max_threads();
  #pragma omp parallel for schedule(dynamic, 1) num_threads(nt)
  for (int64_t i = 0; i < M; ++i) gemm_rows_kn(a, wf, y, i, i + 1, N, K);
#else
  (void)nthreads;
  gemm_rows_kn(a, wf, y, 0, M, N, K);
#endif
  free(wf);
  return 0;
}

/* ------------------------------------------------------------------------ */
/* Epilogue chain (EpilogueOp, src/t0/tile_ir.rs:40-58, lowered at 3400-3540) */
/* ------------------------------------------------------------------------ */
/* ops[i] in 0..7 = BiasAdd, Scale, ReLU, SiLU, GELU, Abs, Neg, Clamp, applied
 * in order to every y[m][n] (fp32).  SiLU is x * 1/(1 + e^-x); GELU is the
 * sigmoid form the reference lowers (tile_ir.rs:3470-3500): x * 1/(1 + e^-1.702x).
 * Exact libm exp and division here; the GPU uses the hardware exp2 / rcp, as
 * the reference's v_exp_f32 / v_rcp_f32 do. */
void orc_epilogue(float* y, int64_t M, int64_t N, const uint32_t* ops, int n_ops, const float* bias,
                  float scale, float lo, float hi) {
  for (int64_t m = 0; m < M; ++m)
    for (int64_t n = 0; n < N; ++n) {
      float v = y[m * N + n];
      for (int i = 0; i < n_ops; ++i) {
        switch (ops[i]) {
          case 0: v = v + bias[n]; break;
          case 1: v = v * scale; break;
          case 2: v = v > 0.0f ? v : 0.0f; break;
          case 3: v = v / (1.0f + expf(-v)); break;
          case 4: v = v / (1.0f + expf(-1.702f * v)); break;
          case 5: v = fabsf(v); break;
          case 6: v = -v; break;
          default: v = v < lo ? lo : v; v = v > hi ? hi : v; break;
        }
      }
      y[m * N + n] = v;
    }
}

int orc_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
