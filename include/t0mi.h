/*
 * t0mi.h — C ABI of the MI355X (gfx950) GEMM hot path.
 *
 * Drop-in replacement for the GEMM path of T0-GPU (clearnature/rust-gpu):
 * the GemmConfig -> gemm_gen / tile_ir kernels, the auto-select and autotune
 * entries, GpuKernel load/dispatch, and an INT4-dequant (W4A16) GEMM.  Every
 * entry point below names the reference item it replaces (file:line in the
 * reference tree).  Plain C types only: pointers, sizes and POD structs.
 *
 * Conventions
 *  - Every function returning int returns T0MI_OK (0) or a negative T0MI_ERR_*.
 *    The reference returns Result<_, String>; the string is available through
 *    t0mi_last_error() (thread-local, valid until the thread's next failing
 *    call).  Reference panics (infeasible config, kernarg-length mismatch,
 *    LDS over budget) become T0MI_ERR_INVALID / T0MI_ERR_KERNARG here.
 *  - Device pointers are uint64_t GPU virtual addresses, as in the reference's
 *    kernarg builders (GpuBuffer::gpu_addr()).
 *  - Argument order follows the reference function being replaced, including
 *    its quirks: build_kernargs takes (x, wt, y, k, n, m), auto_select takes
 *    (m, k, n), GemmTuner::tune takes (m, n, k).
 *  - Grids are HSA work-item grids, as in the reference (grid_x = tiles * wg);
 *    the HIP shim converts them to workgroup counts at launch.
 *  - Threads: a runtime (t0mi_ctx) may be shared, like the reference's
 *    Arc<GpuRuntime>.  Its kernel cache and allocation table are locked, and
 *    every call that launches work or uses the runtime's workspace holds a
 *    per-runtime lock, so launches reach its stream in call order; waits run
 *    outside the lock.  A capture (t0mi_capture_begin .. _end) records what
 *    any thread launches on the runtime meanwhile: capture from one thread.
 */
#ifndef T0MI_H
#define T0MI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define T0MI_ABI_VERSION 1

/* ---- status codes ---------------------------------------------------- */
#define T0MI_OK 0
#define T0MI_ERR_INVALID (-1)   /* bad argument / infeasible config (reference: panic) */
#define T0MI_ERR_NO_KERNEL (-2) /* no prebuilt gfx950 code object for this config */
#define T0MI_ERR_HIP (-3)       /* HIP runtime failure (alloc, copy, launch) */
#define T0MI_ERR_POISONED (-4)  /* runtime poisoned by an earlier failed wait */
#define T0MI_ERR_KERNARG (-5)   /* kernarg length differs from the kernel's declaration */
#define T0MI_ERR_TIMEOUT (-6)   /* dispatch did not complete in time; runtime poisoned */
#define T0MI_ERR_NOT_FOUND (-7) /* cache miss / unknown preset */
#define T0MI_ERR_NO_DEVICE (-8) /* no gfx950 device visible */
#define T0MI_ERR_CAPTURE (-9)   /* call cannot run while the runtime's stream is captured */

/* Thread-local description of the last error on this thread. */
const char* t0mi_last_error(void);
/* ABI version and the gfx target the kernels were built for ("gfx950"). */
int t0mi_abi_version(void);
const char* t0mi_build_target(void);

/* ---- GemmConfig (src/t0/gemm_gen.rs:22-84) ----------------------------- */
typedef enum { T0MI_NT = 0, T0MI_NN = 1 } t0mi_transpose;            /* gemm_gen.rs:22-29 */
typedef enum {                                                        /* gemm_gen.rs:41-49 */
  T0MI_EPI_STORE_F32 = 0,
  T0MI_EPI_BIAS_ADD_STORE_F32 = 1,
  T0MI_EPI_BIAS_ADD_RELU_STORE_F32 = 2
} t0mi_epilogue;
typedef enum { T0MI_OUT_F32 = 0, T0MI_OUT_BF16 = 1 } t0mi_out_dtype; /* new: bf16 store, RNE */

/* Field-for-field mirror of GemmConfig (gemm_gen.rs:55-84).  Booleans are
 * uint32_t 0/1; split_k 0 or 1 means None.  The last four fields are gfx950
 * extensions with no reference counterpart; zero keeps reference behaviour
 * (f32 output, wave layout derived from wg_size, two LDS stages).
 * wg_size is the workgroup size the config's work-item grid is counted in.
 * A config with no gfx950 kernel of its own shape — the wave32 preset
 * tile_16x64_k16 (wg_size 32, 16 rows), tiles that are not whole 32x32 MFMA
 * blocks, a tile_k of 48 — runs on the prebuilt kernel covering its tile
 * (rows and columns rounded up to 32, K steps of 16/32/64 dividing tile_k);
 * it keeps its name, kernargs, grid and attributes, and the results do not
 * depend on the tile. */
typedef struct t0mi_gemm_config {
  uint32_t tile_m, tile_n, tile_k, wg_size;
  uint32_t use_lds, double_buffer;
  uint32_t split_k;
  uint32_t lds_pad, n_col_passes;
  uint32_t swap_grid, wgp_mode;
  uint32_t transpose; /* t0mi_transpose */
  uint32_t epilogue;  /* t0mi_epilogue */
  uint32_t out_dtype; /* t0mi_out_dtype (gfx950 extension) */
  uint32_t wave_m, wave_n; /* waves along M and N; 0,0 = derive (gfx950 extension) */
  uint32_t stages;    /* LDS pipeline stages 2..5; 0 = 2 (double_buffer) (gfx950 extension) */
} t0mi_gemm_config;

/* Presets by reference name, e.g. "tile_128x64_k16" (gemm_gen.rs:87-145), plus
 * the gfx950 presets listed by t0mi_config_preset_names().  Returns
 * T0MI_ERR_NOT_FOUND for an unknown name. */
int t0mi_config_preset(const char* name, t0mi_gemm_config* out);
/* Comma-separated preset names; writes at most len bytes (NUL-terminated). */
int t0mi_config_preset_names(char* buf, size_t len);
/* The prebuilt gfx950 kernels (the set a config must hit for t0mi_kernel_get):
 * comma-separated "tile_m x tile_n x tile_k _w wave_m x wave_n _s stages [_nn]"
 * entries, e.g. "256x256x64_w2x4_s2_nn".  No reference counterpart (the reference
 * generates any config at run time); used by tuners and sweeps. */
int t0mi_gemm_variants(char* buf, size_t len);
/* Derived quantities (gemm_gen.rs:147-201). */
uint32_t t0mi_config_n_waves(const t0mi_gemm_config* cfg);
uint32_t t0mi_config_lds_total(const t0mi_gemm_config* cfg);
uint32_t t0mi_config_estimated_regs(const t0mi_gemm_config* cfg);
/* gemm_gen.rs:203-213, re-derived for gfx950: 1 if a prebuilt kernel runs the
 * config (its own shape within the wave64 / 512 VGPR+AGPR / 160 KB LDS limits,
 * or the kernel covering a reference tile, see above), 0 otherwise. */
int t0mi_config_is_feasible(const t0mi_gemm_config* cfg);
/* GemmConfig::name (gemm_gen.rs:215-235): same tags, plus "_bf16o" for bf16
 * output and "_w{M}x{N}" for a non-default wave layout.  It is the kernel
 * cache key.  Returns the full length (like snprintf). */
int t0mi_config_name(const t0mi_gemm_config* cfg, char* buf, size_t len);

/* ---- grids and kernargs (byte-identical to the Rust builders) ----------- */
/* compute_grid / compute_grid_split_k / compute_grid_auto (gemm_gen.rs:308-329, 430-437). */
int t0mi_compute_grid(const t0mi_gemm_config* cfg, uint32_t m, uint32_t n, uint32_t grid[2]);
int t0mi_compute_grid_split_k(const t0mi_gemm_config* cfg, uint32_t m, uint32_t n, uint32_t split_k,
                              uint32_t grid[2]);
int t0mi_compute_grid_auto(const t0mi_gemm_config* cfg, uint32_t m, uint32_t n, uint32_t grid[2]);
/* build_kernargs (gemm_gen.rs:439-458): 40 bytes
 *   [X u64 @0, WT u64 @8, Y u64 @16, K u32 @24, N u32 @28, split_k_shift u32 @32 (=0),
 *    y_split_stride u32 @36 (= m*n*4 if split_k > 1)]. */
int t0mi_build_kernargs(uint64_t x, uint64_t wt, uint64_t y, uint32_t k, uint32_t n, uint32_t m,
                        const t0mi_gemm_config* cfg, uint8_t out[40]);
/* build_kernargs_with_bias (gemm_gen.rs:460-484): 48 bytes, bias u64 @40. */
int t0mi_build_kernargs_with_bias(uint64_t x, uint64_t wt, uint64_t y, uint32_t k, uint32_t n,
                                  uint32_t m, const t0mi_gemm_config* cfg, uint64_t bias,
                                  uint8_t out[48]);

/* ---- selection and tuning ---------------------------------------------- */
/* auto_select(m, k, n) (gemm_gen.rs:340 -> cost_model::predict_best): a gfx950
 * cost model over the prebuilt kernels.  transpose / out_dtype of the result
 * are T0MI_NT / T0MI_OUT_F32 like the reference; callers set them after. */
int t0mi_auto_select(uint32_t m, uint32_t k, uint32_t n, t0mi_gemm_config* out);
/* cost_model::auto_schedule_gemm (src/t0/cost_model.rs:464-534; note its
 * (m, n, k) order): the ranking behind t0mi_auto_select_layout -- every
 * prebuilt configuration of the layout, best first, with the model's estimate
 * in microseconds.  Writes up to cap entries; *count = the full list length. */
int t0mi_auto_schedule_gemm(uint32_t m, uint32_t n, uint32_t k, uint32_t transpose, uint32_t out_dtype,
                            t0mi_gemm_config* out, double* est_us, uint32_t cap, uint32_t* count);
/* The schedule of the library's own auto-scheduled GEMMs (the dequant-once
 * route of t0mi_w4a16_gemm and the t0mi_matmul_* calls): *head, the ranking's
 * first prebuilt configuration, over columns [0, *n_main) and, when
 * *n_main < n, *tail over [*n_main, n) as a second launch.  The split is
 * planned when head's tiles fill some whole rounds of the GPU and part of one
 * more and the model expects the pair to be faster (e.g. 4096 x 14336 x 4096 NN:
 * 256x256 tiles over 12288 columns, the last 2048 on their own tile).  NT
 * calls of 1..16 rows with K a multiple of 32 and N at most 16 x the CU count
 * run the one-launch persistent decode kernel instead (faster there than any
 * split-K schedule).  No reference counterpart (cost_model.rs:464-534 ranks one
 * configuration per shape); for callers and tests that need to know what runs.
 * Host only. */
int t0mi_auto_gemm_plan(uint32_t m, uint32_t n, uint32_t k, uint32_t transpose, uint32_t out_dtype,
                        t0mi_gemm_config* head, uint32_t* n_main, t0mi_gemm_config* tail);
/* auto_select_legacy (gemm_gen.rs:351-404), re-derived for gfx950. */
int t0mi_auto_select_legacy(uint32_t m, uint32_t k, uint32_t n, t0mi_gemm_config* out);
/* gfx950 extension of auto_select (gemm_gen.rs:340), which only knows the NT
 * layout and f32 output: the same ranking for a given layout (t0mi_transpose)
 * and out_dtype, over the kernels prebuilt for that layout. */
int t0mi_auto_select_layout(uint32_t m, uint32_t k, uint32_t n, uint32_t transpose, uint32_t out_dtype,
                            t0mi_gemm_config* out);
/* cached_auto_select (src/t0/prefill_spec_cache.rs:42-76): process-wide cache. */
int t0mi_cached_auto_select(uint32_t m, uint32_t k, uint32_t n, t0mi_gemm_config* out);
void t0mi_clear_spec_cache(void);
size_t t0mi_spec_cache_len(void);

/* ---- runtime: GpuRuntime / GpuKernel (src/ignis/gpu_context.rs, src/kfd/) - */
typedef struct t0mi_ctx t0mi_ctx;       /* GpuRuntime (gpu_context.rs:99-120) */
typedef struct t0mi_kernel t0mi_kernel; /* GpuKernel (src/kfd/kernel.rs) */

/* GpuRuntime::new (gpu_context.rs:151): opens a HIP device (the first gfx950
 * one when device < 0) and creates its own stream (default priority). */
int t0mi_ctx_create(int device, t0mi_ctx** out);
/* Same, but launches go to an existing hipStream_t owned by the caller
 * (for example torch.cuda.current_stream().cuda_stream); NULL means the
 * device's null (default) stream, not a new one. */
int t0mi_ctx_create_on_stream(int device, void* hip_stream, t0mi_ctx** out);
/* A runtime with no device: dispatches are validated (kernarg length,
 * poisoning) and recorded but compute nothing.  For control-path tests. */
int t0mi_ctx_create_null(t0mi_ctx** out);
void t0mi_ctx_destroy(t0mi_ctx* ctx);
void* t0mi_ctx_stream(t0mi_ctx* ctx);
/* GpuRuntime::is_poisoned / mark_poisoned (gpu_context.rs:190-197). */
int t0mi_is_poisoned(t0mi_ctx* ctx);
void t0mi_mark_poisoned(t0mi_ctx* ctx);
/* Timeout of a synchronous dispatch / wait (aql.rs:481-545 uses 60 s). */
void t0mi_set_timeout_ms(t0mi_ctx* ctx, uint32_t ms);
/* Null runtime only: make the next dispatch report a timeout. */
int t0mi_null_inject_timeout(t0mi_ctx* ctx);
/* Null runtime only: grid (work-items) and kernarg bytes of the last dispatch. */
int t0mi_null_last_dispatch(t0mi_ctx* ctx, uint32_t grid[3], uint8_t* ka, size_t ka_cap, size_t* ka_len);

/* GpuRuntime::alloc (gpu_context.rs:508-510) through its BufferPool
 * (gpu_context.rs:31-90): the size is rounded up to 4096 bytes, the pool key; a
 * buffer recycled at that size is handed out again, zeroed in stream order
 * before any later work on the runtime's stream; otherwise a fresh allocation
 * (contents undefined).  Not during graph capture when it must allocate. */
int t0mi_alloc(t0mi_ctx* ctx, size_t bytes, uint64_t* dptr);
/* GpuRuntime::alloc_zero (gpu_context.rs:513-517): alloc, zeroed, and waits. */
int t0mi_alloc_zero(t0mi_ctx* ctx, size_t bytes, uint64_t* dptr);
/* GpuRuntime::alloc_f32 (gpu_context.rs:520-525): n floats, max(4n, 512) bytes
 * rounded up to 512, from the pool, zeroed in stream order. */
int t0mi_alloc_f32(t0mi_ctx* ctx, size_t n, uint64_t* dptr);
/* GpuRuntime::recycle (gpu_context.rs:528-531): the buffer returns to the pool
 * (no wait, no free); queued work that uses it still runs before its next
 * hand-out, which zeroes it in stream order. */
int t0mi_recycle(t0mi_ctx* ctx, uint64_t dptr);
/* BufferPool::cached_bytes / clear (gpu_context.rs:83-93); clear waits for the
 * stream, then frees every pooled buffer. */
size_t t0mi_pool_cached_bytes(t0mi_ctx* ctx);
int t0mi_pool_clear(t0mi_ctx* ctx);
/* Frees a buffer now (after the stream's queued work): no reference counterpart
 * (the reference's GpuBuffer frees on drop). */
int t0mi_free(t0mi_ctx* ctx, uint64_t dptr);
/* GpuBuffer::write / read behind GpuRuntime::write_f32 / read_f32
 * (gpu_context.rs:536-552): synchronous copies; read_f32 waits for the stream
 * first, as here. */
int t0mi_h2d(t0mi_ctx* ctx, uint64_t dst, const void* src, size_t bytes);
int t0mi_d2h(t0mi_ctx* ctx, void* dst, uint64_t src, size_t bytes);
int t0mi_memset(t0mi_ctx* ctx, uint64_t dst, int value, size_t bytes);

/* ensure_kernel_t0(cfg.name(), || generate(&cfg), ...) (gpu_context.rs:212-265):
 * instead of generate + compile + GpuKernel::load, look up the prebuilt gfx950
 * code object for this config (cached by name; a reference tile without a
 * kernel of its own shape maps to the covering kernel).  kernarg_size is 40,
 * or 48 for a bias epilogue; wg_size and lds_size are the config's.  The
 * kernel is owned by ctx. */
int t0mi_kernel_get(t0mi_ctx* ctx, const t0mi_gemm_config* cfg, t0mi_kernel** out);
/* T0Kernel::lds_size / wg_size / kernarg_size (compile.rs:641-656). */
int t0mi_kernel_attrs(const t0mi_kernel* k, uint32_t* lds_size, uint32_t* wg_size, uint32_t* kernarg_size);
int t0mi_kernel_name(const t0mi_kernel* k, char* buf, size_t len);

/* GpuRuntime::dispatch (gpu_context.rs:305-357): checks poisoning, requires
 * ka_len == kernarg_size (reference: assert), launches grid_workitems / wg
 * workgroups and waits (with timeout; a timeout poisons the runtime). */
int t0mi_dispatch(t0mi_ctx* ctx, const t0mi_kernel* k, const uint32_t grid_workitems[3],
                  const uint8_t* ka, size_t ka_len);
/* GpuRuntime::dispatch_async (gpu_context.rs:400-410): no wait. */
int t0mi_dispatch_async(t0mi_ctx* ctx, const t0mi_kernel* k, const uint32_t grid_workitems[3],
                        const uint8_t* ka, size_t ka_len);
/* GpuRuntime::wait_idle / synchronize (gpu_context.rs:446-452). */
int t0mi_wait_idle(t0mi_ctx* ctx);

/* One-call GEMM with a given config (what callers of generate + build_kernargs
 * + compute_grid_auto + dispatch do, src/t0/auto_gemm.rs:575-588), without the
 * reference's padding contract: M, N, K need not be tile multiples (K, and N for
 * NN, must be multiples of 8; rows are 16-byte aligned).  Y is [m, n] with the
 * config's out_dtype.  Split-K > 1 is reduced in a deterministic second pass
 * (p = 0..split_k-1 order) using a library-owned workspace.  Asynchronous. */
int t0mi_gemm(t0mi_ctx* ctx, const t0mi_gemm_config* cfg, uint64_t x, uint64_t b, uint64_t y,
              uint64_t bias, uint32_t m, uint32_t n, uint32_t k);

/* Bytes of the per-GPU scratch array behind t0mi_gemm_noalloc. */
#define T0MI_NOALLOC_SCRATCH_BYTES (32u << 20)
/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): t0mi_gemm with the same arguments, kernels and results,
 * except that its split-K partial planes (and the zero plane of K = 0) live
 * in a static array of T0MI_NOALLOC_SCRATCH_BYTES bytes that every GPU the
 * library runs on holds until the process ends, instead of the runtime's
 * growable workspace.  It calls no hipMalloc or hipFree.  A call needing more
 * than that (M * N * 4 * split_k bytes; M * N * 4 when K = 0) fails with
 * T0MI_ERR_INVALID before anything is launched.  Every runtime on one GPU
 * shares that GPU's array: calls on one stream are ordered; a call from
 * another stream while the last call's work on the GPU has not finished is
 * refused with T0MI_ERR_INVALID (an event recorded after each call, made when
 * the first runtime on the device was created); calls recorded into a graph
 * are not tracked, and replays that overlap with other users of the array on
 * one GPU race.  Nothing in the array needs to start at zero.  Asynchronous. */
int t0mi_gemm_noalloc(t0mi_ctx* ctx, const t0mi_gemm_config* cfg, uint64_t x, uint64_t b, uint64_t y,
                      uint64_t bias, uint32_t m, uint32_t n, uint32_t k);

/* No counterpart in the reference (RDNA parts have one L2).  The XCD count of
 * this runtime's device when the W4A16 decode's in-launch split-K exchange is
 * on (workgroup i of a launch was found on XCD i % n for every i by a probe at
 * runtime creation), or 0 when it is off and the decode keeps one workgroup per
 * column strip; and, when `misplaced` is not null, whether an exchange launch
 * on this runtime has found one of its workgroups on another XCD than the
 * numbering planned (waits for the stream).  Informational: the partials are
 * written through to memory, so results do not depend on where the pieces
 * ran; a misplaced piece only costs its reader an L2 miss.  For tests and
 * callers that check what runs. */
int t0mi_xcd_placement(t0mi_ctx* ctx, uint32_t* n_xcd, uint32_t* misplaced);

/* ---- batched submission: DispatchQueue (src/t0/prefill_dispatch.rs:58-214) - */
typedef struct t0mi_dispatch_queue t0mi_dispatch_queue;
/* DispatchQueue::new (prefill_dispatch.rs:73-79). */
int t0mi_dq_new(t0mi_ctx* ctx, t0mi_dispatch_queue** out);
/* DispatchQueue::submit (prefill_dispatch.rs:90-107): dispatch_async with the
 * same checks as t0mi_dispatch (kernarg length, grid); a poisoned runtime
 * refuses with T0MI_ERR_POISONED "[DispatchQueue] Queue poisoned ...". */
int t0mi_dq_submit(t0mi_dispatch_queue* q, const t0mi_kernel* k, const uint32_t grid_workitems[3],
                   const uint8_t* ka, size_t ka_len);
/* DispatchQueue::flush (prefill_dispatch.rs:133-166): one wait for every
 * pending dispatch (timeout / failure poisons the runtime); *count = the
 * number flushed (0 when none were pending, without waiting). */
int t0mi_dq_flush(t0mi_dispatch_queue* q, size_t* count);
/* DispatchQueue::pending (prefill_dispatch.rs:169-171). */
size_t t0mi_dq_pending(const t0mi_dispatch_queue* q);
/* DispatchQueue::drop_async (prefill_dispatch.rs:177-187): frees the queue
 * without waiting (warns on stderr if dispatches are pending); the caller keeps
 * their buffers alive until a later wait. */
void t0mi_dq_drop_async(t0mi_dispatch_queue* q);
/* batch_dispatch (prefill_dispatch.rs:204-214): submit n dispatches
 * (grids = n x 3 work-item counts) and flush once; *count = n on success. */
int t0mi_batch_dispatch(t0mi_ctx* ctx, size_t n, const t0mi_kernel* const* kernels, const uint32_t* grids,
                        const uint8_t* const* kas, const size_t* ka_lens, size_t* count);

/* HIP graphs (no reference counterpart; the MI355X form of batched submission,
 * prefill_dispatch.rs:1-46): between begin and end, library calls on ctx that
 * only launch kernels are recorded from ctx's stream instead of run; end
 * instantiates them, and t0mi_graph_launch replays the batch with one launch
 * call (asynchronous; wait with t0mi_wait_idle).  While capturing, calls that
 * wait, allocate, copy to the host or must grow the library workspace return
 * T0MI_ERR_CAPTURE and leave the capture usable: run a batch once before
 * capturing it so the workspace has its size.  While a graph is alive the
 * workspace cannot move (growth returns T0MI_ERR_CAPTURE); destroy graphs
 * before their runtime.  The runtime's stream must not be the null stream. */
typedef struct t0mi_graph t0mi_graph;
int t0mi_capture_begin(t0mi_ctx* ctx);
int t0mi_capture_end(t0mi_ctx* ctx, t0mi_graph** out);
int t0mi_graph_launch(t0mi_graph* g);
size_t t0mi_graph_node_count(const t0mi_graph* g);
void t0mi_graph_destroy(t0mi_graph* g);

/* ---- tile_ir surface: TileGemm (src/t0/tile_ir.rs:100-152) ---------------- */
/* EpilogueOp of the tile_ir fusion chain (tile_ir.rs:40-58), applied in order
 * to every fp32 result before the store (lowered at tile_ir.rs:3400-3540):
 *   BIAS_ADD  v += bias[col]  (bias: [N] f32)     SCALE  v *= scale
 *   RELU      max(v, 0)                           SILU   v * rcp(1 + exp2(-v log2e))
 *   GELU      v * rcp(1 + exp2(-1.702 v log2e))   (the sigmoid form the reference
 *             lowers, tile_ir.rs:3470-3500, not the tanh form its doc comment names)
 *   ABS |v|   NEG -v   CLAMP min(max(v, clamp_min), clamp_max) */
typedef enum {
  T0MI_TEPI_BIAS_ADD = 0,
  T0MI_TEPI_SCALE = 1,
  T0MI_TEPI_RELU = 2,
  T0MI_TEPI_SILU = 3,
  T0MI_TEPI_GELU = 4,
  T0MI_TEPI_ABS = 5,
  T0MI_TEPI_NEG = 6,
  T0MI_TEPI_CLAMP = 7
} t0mi_tile_epilogue_op;
#define T0MI_TILE_MAX_EPILOGUE 8

/* TileGemm, field for field (booleans as 0/1; waves_per_wg 0 = None), plus
 * out_dtype.  wmma_format must be 0 (BF16_F32): the only format on this path.
 * On gfx950 the RDNA-specific fields (wgp_mode, acc_swap, waves_per_wg) keep
 * their meaning for name() and the grid/LDS arithmetic but do not change the
 * kernel; triple_buffer selects a 3-stage LDS ring where one is prebuilt. */
typedef struct t0mi_tile_spec {
  uint32_t tile_m, tile_n, tile_k;
  uint32_t wgp_mode, double_buffer, triple_buffer;
  uint32_t split_k;
  uint32_t swap_grid;
  uint32_t transpose; /* t0mi_transpose */
  uint32_t acc_swap;
  uint32_t n_epilogue;
  uint32_t epilogue[T0MI_TILE_MAX_EPILOGUE]; /* t0mi_tile_epilogue_op */
  uint32_t persistent;
  uint32_t waves_per_wg;
  uint32_t wmma_format;
  uint32_t out_dtype; /* new: T0MI_OUT_F32 (reference) or T0MI_OUT_BF16 */
} t0mi_tile_spec;

/* TileGemm::tile_* presets by function name, e.g. "tile_128x64_k16",
 * "tile_persistent_decode" (tile_ir.rs:156-604); T0MI_ERR_NOT_FOUND if unknown. */
int t0mi_tile_preset(const char* name, t0mi_tile_spec* out);
/* Comma-separated preset names. */
const char* t0mi_tile_preset_names(void);
/* TileGemm::name (tile_ir.rs:677-701); returns the length, writes at most len-1. */
int t0mi_tile_name(const t0mi_tile_spec* s, char* buf, size_t len);
/* n_waves / wg_size / lds_total (tile_ir.rs:607-653), the reference's arithmetic
 * (wave32 work-items, acc-swap region, +16 B persistent slot). */
uint32_t t0mi_tile_n_waves(const t0mi_tile_spec* s);
uint32_t t0mi_tile_wg_size(const t0mi_tile_spec* s);
uint32_t t0mi_tile_lds_total(const t0mi_tile_spec* s);
/* tile_auto_select(m, k, n, transpose) (tile_ir.rs:740-870): the reference's
 * shape rules, including its 64 KB LDS fallback and auto split-K disabled. */
int t0mi_tile_auto_select(uint32_t m, uint32_t k, uint32_t n, uint32_t transpose, t0mi_tile_spec* out);
/* Kernarg bytes the lowered kernel declares: 44 (64 when persistent), then the
 * epilogue arguments in declaration order with the reference's allocator
 * alignment (compile.rs:120-180): bias u64 (8-aligned), scale f32, clamp_min
 * f32, clamp_max f32 — each only when the chain uses it. */
uint32_t t0mi_tile_kernarg_size(const t0mi_tile_spec* s);
/* build_kernargs (tile_ir.rs:4570-4593): 44 B with the M slot left 0, and
 * build_kernargs_m (:4595-4602): 44 B with M.  Layout [X u64 @0, WT u64 @8,
 * Y u64 @16, K @24, N @28, split_k_shift @32, y_split_stride @36 (0), M @40].
 * Return the byte count written (or needed, if cap is too small: nothing is
 * written then). */
int t0mi_tile_build_kernargs(uint64_t x, uint64_t wt, uint64_t y, uint32_t k, uint32_t n,
                             const t0mi_tile_spec* s, uint8_t* out, size_t cap);
int t0mi_tile_build_kernargs_m(uint64_t x, uint64_t wt, uint64_t y, uint32_t k, uint32_t n, uint32_t m,
                               const t0mi_tile_spec* s, uint8_t* out, size_t cap);
/* build_kernargs_m_with_counter (tile_ir.rs:4604-4637): persistent specs append
 * counter u64 @48, n_tiles_n_shift @56, tiles_per_wg @60 (64 B). */
int t0mi_tile_build_kernargs_m_with_counter(uint64_t x, uint64_t wt, uint64_t y, uint32_t k, uint32_t n,
                                            uint32_t m, const t0mi_tile_spec* s, uint64_t counter,
                                            uint32_t n_tiles_n_shift, uint32_t tiles_per_wg, uint8_t* out,
                                            size_t cap);
/* Appends the epilogue arguments the spec's chain declares to a kernarg buffer
 * of *len bytes (what a reference caller writes after build_kernargs_m, per
 * lower_gemm's declarations at tile_ir.rs:1014-1027).  Updates *len. */
int t0mi_tile_append_epilogue_args(const t0mi_tile_spec* s, uint64_t bias, float scale, float clamp_min,
                                   float clamp_max, uint8_t* buf, size_t cap, size_t* len);
/* compute_grid (tile_ir.rs:4645-4666): work-items, [wg_size, 1, 1] when persistent. */
int t0mi_tile_compute_grid(const t0mi_tile_spec* s, uint32_t m, uint32_t n, uint32_t grid_workitems[3]);
/* lower_gemm + T0Kernel::compile + GpuKernel::load for a TileGemm
 * (tile_ir.rs:887; compile.rs:1398): looks up the prebuilt gfx950 kernel with
 * the spec's tile_m x tile_n x tile_k, or the one covering it (tile_k 48 as
 * three 16-K steps; NN tiles narrower than 64 columns on the 64-column NN
 * kernel).  The handle dispatches with the spec's own kernarg layout and grid;
 * M comes from the kernarg (0 = derive it from the grid, padded as gemm_gen
 * does).  A persistent spec (one workgroup looping over the tiles in the
 * reference, tile_ir.rs:540-604, 1062-1120) runs as one launch of a persistent
 * kernel whose grid is what the GPU holds at once, each workgroup looping over
 * work units with the grid's stride: up to 64 rows with K a multiple of 32 the
 * decode kernel (32 x 16 units over the whole K, the K range split over the 16
 * waves of a workgroup and summed in LDS in wave order), else the spec's tile
 * kernel in a tile loop.  The whole K sum lands in Y (split-K is not part of a
 * persistent run, as in the reference).  The kernarg's counter slot is left
 * untouched.  T0MI_ERR_NO_KERNEL when no prebuilt kernel covers the tile. */
int t0mi_tile_kernel_get(t0mi_ctx* ctx, const t0mi_tile_spec* s, t0mi_kernel** out);
/* One-call tile GEMM: Y[m,n] = epilogue(X[m,k] . B) for the spec's transpose,
 * with the chain's arguments; split_k > 1 is reduced deterministically (the
 * reference's tile_ir split-K writes every partition to one plane,
 * tile_ir.rs:4577-4581; here the sum is correct).  A persistent spec takes the
 * persistent kernels described at t0mi_tile_kernel_get.  Asynchronous. */
int t0mi_tile_gemm(t0mi_ctx* ctx, const t0mi_tile_spec* s, uint64_t x, uint64_t wt, uint64_t y, uint32_t m,
                   uint32_t n, uint32_t k, uint64_t bias, float scale, float clamp_min, float clamp_max);

/* ---- autotuner: GemmTuner (src/t0/auto_gemm.rs:46-527) -------------------- */
typedef struct t0mi_tuner t0mi_tuner;
/* GemmTuner::new (default cache dir $HOME/.t0mi_autotune_gfx950, kept apart
 * from the reference's RDNA cache) / with_cache_dir. */
int t0mi_tuner_create(const char* cache_dir_or_null, t0mi_tuner** out);
void t0mi_tuner_destroy(t0mi_tuner* t);
/* max_candidates (default 8) and n_iters (default 5) (auto_gemm.rs:57-65). */
void t0mi_tuner_set_params(t0mi_tuner* t, uint32_t max_candidates, uint32_t n_iters);
/* GemmTuner::tune(rt, m, n, k) (auto_gemm.rs:82-216): memory cache -> disk JSON
 * -> candidates -> 256^3 smoke test -> median timing -> persist.  transpose
 * and out_dtype select the variant being tuned.  *tflops and *from_cache may
 * be null. */
int t0mi_tuner_tune(t0mi_tuner* t, t0mi_ctx* ctx, uint32_t m, uint32_t n, uint32_t k, uint32_t transpose,
                    uint32_t out_dtype, t0mi_gemm_config* best, double* tflops, int* from_cache);
/* GemmTuner::invalidate / clear (auto_gemm.rs:504-514). */
void t0mi_tuner_invalidate(t0mi_tuner* t, uint32_t m, uint32_t n, uint32_t k, uint32_t transpose,
                           uint32_t out_dtype);
void t0mi_tuner_clear(t0mi_tuner* t);
/* Cache file path for a key (auto_gemm.rs:435-437), and its JSON codec. */
int t0mi_tuner_cache_path(t0mi_tuner* t, uint32_t m, uint32_t n, uint32_t k, uint32_t transpose,
                          uint32_t out_dtype, char* buf, size_t len);
/* GemmTuner::report as text (auto_gemm.rs:517-527). */
int t0mi_tuner_report(t0mi_tuner* t, char* buf, size_t len);
/* auto_gemm(rt, a, b, c, m, n, k) (auto_gemm.rs:555-590) with the process-wide
 * tuner; NT layout, f32 output as in the reference.  Returns the cached
 * TFLOPS in *tflops. */
int t0mi_auto_gemm(t0mi_ctx* ctx, uint64_t a, uint64_t b, uint64_t c, uint32_t m, uint32_t n, uint32_t k,
                   double* tflops);

/* ---- W4A16: INT4-dequant GEMM (new; semantics from src/t0/quant_kernels.rs) */
/* Y[m, n] = sum_k A[m,k] * (q[k][n] - z) * s[k/group][n], fp32 accumulate.
 *  A       bf16 [m, k] row-major.
 *  qweight u32 [k/8][n]: 8 nibbles along K per word, nibble e = bits 4e..4e+3
 *          (the reference's low-nibble-first element order, quant_kernels.rs:3-10).
 *  scales  bf16 [k/group][n].
 *  qzeros  u32 [k/group][n/8] (nibble e of word j = zero of column 8j+e), or 0
 *          to use the constant zp_const for every group.
 *  Y       [m, n] f32 or bf16 (RNE) per out_dtype.
 * Requires k % group == 0, group % 32 == 0, n % 8 == 0; A, qweight and Y
 * 16-byte aligned, scales 8-byte, qzeros 4-byte.  K = 0 writes Y = 0.
 * Asynchronous.
 * Routes by row count: the decode kernel over 16-row slabs (exact dequant inside
 * the MFMA), several slabs per launch sharing one pass over the weights, in up to
 * three launches: up to 191 rows for group 128 (four slabs per launch), 144 for
 * groups 32 and 64, 96 for 256, 80 for other groups (one slab per launch; a
 * single slab whose 64-column strips number at most half the CUs -- e.g. a
 * column-parallel shard -- has each strip's K range split over up to 8
 * workgroups, combined inside the launch through the runtime's exchange
 * buffers); then
 * kernels that dequantize inside the MFMA K loop, rounding the weight once to
 * bf16: from there to 191 rows the 128x128 fused tile
 * kernel, 192..1535 rows (K and group multiples of 64) the 256x256 ping-pong
 * kernel, K split through the library workspace when tiles are fewer than
 * CUs; from 1536 rows (768 when K or the group is not a multiple of 64, and
 * from 81 rows for a group that is not a power of two; from 1025 rows when the
 * ping-pong tiles overflow one round of the GPU and t0mi_auto_gemm_plan splits
 * the dense GEMM's columns) the weight is
 * dequantized once to bf16 into the library's conversion buffer (k * n * 2
 * bytes, kept by the runtime) and the dense NN GEMM runs, unless that is above
 * the runtime's limit (t0mi_set_w4a16_workspace_limit).  The ping-pong and the
 * dequant-once routes give bit-identical results when the dense GEMM takes the
 * same 256x256 tile and K partitions (4096 rows and more: config 5). */
int t0mi_w4a16_gemm(t0mi_ctx* ctx, uint64_t a, uint64_t qweight, uint64_t scales, uint64_t qzeros,
                    uint32_t zp_const, uint64_t y, uint32_t m, uint32_t k, uint32_t n, uint32_t group,
                    uint32_t out_dtype);
/* No counterpart in the reference (which has no fused W4A16 GEMM).  For callers
 * that cannot hold the dequantized weight (k * n * 2 bytes of the runtime's
 * conversion buffer): t0mi_w4a16_gemm calls on this runtime whose dequant-once
 * route would need more than `bytes` run the fused kernels instead -- the
 * 256x256 ping-pong kernel (K and group multiples of 64, any row count from
 * 192 on, and from 81 rows for a group that is not a power of two) or the
 * 128x128 fused tile kernel (other power-of-two groups), the weights crossing
 * HBM once, at 4 bits; with a group that is neither, such calls return
 * T0MI_ERR_INVALID.  Every route rounds each weight (q - z) * s once to bf16;
 * the fused results are bit-identical to dequant-once where the dense GEMM
 * takes the same 256x256 tile and K partitions (4096 rows and more: config 5),
 * and otherwise within the GEMM tolerance of them (another tile or K split sums
 * in another order).  Default: no limit.  0: never dequantize once. */
int t0mi_set_w4a16_workspace_limit(t0mi_ctx* ctx, uint64_t bytes);

/* Standalone dequant, replacing build_dequant_int4_{f32,bf16} (quant_kernels.rs:53-171)
 * on the same layouts as t0mi_w4a16_gemm: out[k][n] = (float)(q - z) * s.
 * round_mode 0: f32 out; 1: bf16 by truncation (the reference's store_bf16,
 * quant_kernels.rs:167-168); 2: bf16 round-to-nearest-even.  Bit-exact.
 * qweight and an f32 out are 16-byte aligned, scales and a bf16 out 8-byte. */
int t0mi_dequant_int4(t0mi_ctx* ctx, uint64_t qweight, uint64_t scales, uint64_t qzeros, uint32_t zp_const,
                      uint64_t out, uint32_t k, uint32_t n, uint32_t group, uint32_t round_mode);

/* ---- GPTQ container (GptqWeight, src/t0/quant_kernels.rs:177-294) ---------- */
/* Byte layout of GptqWeight::from_bytes (quant_kernels.rs:242-286), little-endian:
 *   [rows u32][cols u32][group_size u32][rows*cols/2 packed INT4 bytes, element
 *   2i = low nibble of byte i, row-major [rows][cols]][n_groups*rows f32 scales]
 *   [n_groups*rows i32 zero points], scale/zero of (row, g) at row*n_groups + g,
 *   n_groups = cols / group_size.  rows = output features (N), cols = K. */
typedef struct t0mi_gptq_info {
  uint32_t rows, cols, group_size, n_groups;
  uint64_t packed_offset, packed_bytes;  /* 12, rows*cols/2 */
  uint64_t scales_offset, zeros_offset;  /* f32 and i32 sections */
  uint64_t total_bytes;                  /* 12 + packed + 8 * n_groups * rows */
  uint32_t zeros_in_range;               /* 1: every zero point is 0..15 (packable to INT4) */
  uint32_t scales_bf16_exact;            /* 1: every scale is exactly a bf16 value */
} t0mi_gptq_info;

/* GptqWeight::from_bytes (quant_kernels.rs:242-286): validates the header and
 * section lengths of `raw` and fills `out`.  The reference panics on a short
 * header, a truncated body or a length mismatch; here those return
 * T0MI_ERR_INVALID (as does group_size 0 or an odd rows*cols).  Host only. */
int t0mi_gptq_parse(const void* raw, size_t len, t0mi_gptq_info* out);
/* GptqWeight::gpu_buffer_size (quant_kernels.rs:289-293): packed + 4*scales + 4*zeros bytes. */
uint64_t t0mi_gptq_gpu_buffer_size(const t0mi_gptq_info* info);

/* New: converts the GPTQ sections, already in device memory, to the W4A16
 * layouts of t0mi_w4a16_gemm (K = cols, N = rows), on ctx's stream:
 *   qweight u32 [K/8][N]  <- packed [N][K/2] bytes (a u32 transpose: the GPTQ
 *                            bytes of one row, read as little-endian words, are
 *                            the W4A16 words);
 *   scales  bf16 [K/g][N] <- f32 [N][K/g], rounded to nearest even (exact when
 *                            t0mi_gptq_info.scales_bf16_exact);
 *   qzeros  u32 [K/g][N/8] <- i32 [N][K/g] packed as nibbles (values must be
 *                            0..15: t0mi_gptq_info.zeros_in_range).
 * Requires K % 8 == 0, N % 8 == 0, K % group == 0.  Asynchronous. */
int t0mi_gptq_convert(t0mi_ctx* ctx, uint64_t packed, uint64_t scales_f32, uint64_t zeros_i32, uint32_t rows,
                      uint32_t cols, uint32_t group, uint64_t qweight, uint64_t scales_bf16, uint64_t qzeros);

/* ---- Ignis matmul caller (src/ignis/ops/bf16_matmul.rs:33-423) ------------- */
/* The reference converts f32 -> bf16 on the host (round to nearest even,
 * bf16_matmul.rs:372), transposes W, pads every dimension to tile multiples,
 * runs the NT gemm_gen kernel with f32 output and unpads.  Here the conversion
 * (and, where a GEMM operand needs it, the transpose) runs on the GPU into a
 * library-owned buffer, NN is native and ragged shapes need no padding.  All
 * buffers are device f32, row-major, and the calls are asynchronous. */

/* f32 -> bf16 round-to-nearest-even of `count` elements (bf16_matmul.rs:372). */
int t0mi_f32_to_bf16(t0mi_ctx* ctx, uint64_t src_f32, uint64_t dst_bf16, uint64_t count);
/* matmul forward (bf16_matmul.rs:33-96, dispatch_gemm_forward :159-209):
 * Y[m,n] = bf16(X[m,k]) . bf16(W[k,n]), fp32 accumulate, f32 out. */
int t0mi_matmul_f32(t0mi_ctx* ctx, uint64_t x, uint64_t w, uint64_t y, uint32_t m, uint32_t k, uint32_t n);
/* matmul_with_wt_bf16 (bf16_matmul.rs:99-134): X f32 [m,k], WT bf16 [n,k]
 * (pre-transposed weight) -> Y f32 [m,n].  Requires k % 8 == 0 and n % 8 == 0
 * (WT is used in place). */
int t0mi_matmul_wt_bf16(t0mi_ctx* ctx, uint64_t x, uint64_t wt_bf16, uint64_t y, uint32_t m, uint32_t k,
                        uint32_t n);
/* gemm_backward_data (bf16_matmul.rs:216-262): dX[m,k] = bf16(dY[m,n]) . bf16(W[k,n])^T. */
int t0mi_matmul_backward_data(t0mi_ctx* ctx, uint64_t dy, uint64_t w, uint64_t dx, uint32_t m, uint32_t k,
                              uint32_t n);
/* gemm_backward_weight (bf16_matmul.rs:268-316): dW[k,n] = bf16(X[m,k])^T . bf16(dY[m,n]). */
int t0mi_matmul_backward_weight(t0mi_ctx* ctx, uint64_t x, uint64_t dy, uint64_t dw, uint32_t m, uint32_t k,
                                uint32_t n);

#ifdef __cplusplus
}
#endif
#endif /* T0MI_H */
