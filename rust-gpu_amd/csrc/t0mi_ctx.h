// t0mi_ctx.h — runtime object shared by the libt0mi translation units.
#pragma once
#include <hip/hip_runtime.h>

#include <atomic>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "gemm_bf16_kernel.h"
#include "t0mi_internal.h"

namespace t0mi {
struct XcdExchange;  // xcd_exchange.h
}

namespace t0mi {

typedef void (*GemmLaunchFn)(dim3 grid, hipStream_t stream, const GemmParams& p);
struct GemmLaunchEntry {
  int bm, bn, bk, wm, wn, stages, nn;
  GemmLaunchFn fn;
};
// Tables defined by the gemm_inst.hip objects (one per variant block and layout).
const GemmLaunchEntry* gemm_table_p0_nt(size_t* n);
const GemmLaunchEntry* gemm_table_p1_nt(size_t* n);
const GemmLaunchEntry* gemm_table_p0_nn(size_t* n);
const GemmLaunchEntry* gemm_table_p1_nn(size_t* n);
const GemmLaunchEntry* gemm_table_p2_nt(size_t* n);
const GemmLaunchEntry* gemm_table_p2_nn(size_t* n);
const GemmLaunchEntry* gemm_table_p3_nt(size_t* n);
const GemmLaunchEntry* gemm_table_p3_nn(size_t* n);
const GemmLaunchEntry* find_gemm_launch(const t0mi_gemm_config& c);

enum KernelKind : int { KK_GEMM_GEN = 1, KK_TILE = 2 };

}  // namespace t0mi

struct t0mi_kernel {
  int kind;
  t0mi_gemm_config cfg;       // KK_GEMM_GEN: the caller's config; KK_TILE: the lowered config of `tile`
  t0mi_gemm_config phys;      // the config of the prebuilt kernel that runs (== cfg unless remapped)
  t0mi_tile_spec tile;        // KK_TILE only
  t0mi::TileArgLayout lay;    // KK_TILE only
  t0mi::EpiChain chain;
  std::string name;
  uint32_t kernarg_size, lds_size, wg_size;
  const t0mi::GemmLaunchEntry* gemm;
};

struct t0mi_ctx {
  bool null_backend = false;
  int device = -1;
  hipStream_t stream = nullptr;
  bool own_stream = false;
  std::atomic<bool> poisoned{false};
  uint32_t timeout_ms = 60000;  // aql.rs:481-545: 60 s
  std::mutex mu;
  std::map<std::string, std::unique_ptr<t0mi_kernel>> kernels;  // name -> kernel (ensure_kernel_t0 cache)
  std::map<uint64_t, size_t> allocs;                            // live t0mi_alloc buffers (pool-aligned size)
  // BufferPool (gpu_context.rs:31-90): recycled buffers by 4096-aligned size,
  // handed out again (zeroed) by t0mi_alloc / t0mi_alloc_f32; cached bytes.
  std::map<size_t, std::vector<uint64_t>> pool;
  size_t pool_bytes = 0;
  // Held by every call that launches work or uses ws / cvt, so a runtime can be
  // shared between threads (launches reach the stream in lock order).
  // Recursive: entry points call each other.  Waits run outside it.
  std::recursive_mutex submit_mu;
  // Library-owned workspace (split-K partial planes, W4A16 partials).
  void* ws = nullptr;
  size_t ws_bytes = 0;
  // Library-owned bf16 operand buffer of the Ignis matmul calls (kept apart
  // from ws, which the GEMMs they launch may use for split-K).
  void* cvt = nullptr;
  size_t cvt_bytes = 0;
  // Largest dequantized-weight buffer (bytes) t0mi_w4a16_gemm may use for its
  // dequant-once route; above it the fused kernels run instead.
  uint64_t w4_cvt_limit = ~0ull;
  // This device's copy of the library's static scratch array (device
  // address, looked up once per device when the first runtime on it is
  // created) and the error of that lookup if it failed.  Used only by
  // t0mi_gemm_noalloc; shared by every runtime on the device.
  void* scratch = nullptr;
  int scratch_rc = 0;
  // Instantiated graphs captured on this runtime: their kernel nodes hold ws
  // and cvt addresses, so neither buffer may move while one is alive.
  std::atomic<int> live_graphs{0};
  // Null backend: injected failure and the last recorded dispatch.
  bool inject_timeout = false;
  uint32_t last_grid[3] = {0, 0, 0};
  std::vector<uint8_t> last_ka;
  int cu_count = 256;
  // In-launch split-K exchange of the W4A16 decode (xcd_exchange.h): the XCD
  // count when the placement probe found workgroup i on XCD i % xk_nx for every
  // i (0: the probe failed; the decode then keeps one workgroup per strip), the
  // counters (xk_nx groups of kXkCountersPerXcd, zeroed once, left zeroed by
  // every launch), the misplacement flag after them, and the partial slots.
  uint32_t xk_nx = 0;
  uint32_t* xk_tick = nullptr;
  void* xk_part = nullptr;
  size_t xk_part_bytes = 0;
};

// Scoped hold of ctx->submit_mu (ctx must be non-null).
#define T0MI_SUBMIT_GUARD(ctx) std::lock_guard<std::recursive_mutex> t0mi_submit_guard_((ctx)->submit_mu)

namespace t0mi {
// Grows ctx->ws to at least `bytes` (waits for the stream first).
int ensure_workspace(t0mi_ctx* ctx, size_t bytes);
// Grows ctx->cvt to at least `bytes` (waits for the stream first).
int ensure_cvt_buffer(t0mi_ctx* ctx, size_t bytes);
// Counters of the XCD exchange, per XCD: at most this many tiles per XCD per launch.
// Each counter has a 256-byte slot of its own: atomics on one line (or one L2
// channel) are serialized, and a launch's pieces all arrive at about the same
// time (176 tickets on one line: 19 us for a 8 us decode).
constexpr uint32_t kXkCountersPerXcd = 1024;
constexpr uint32_t kXkCounterStride = 64;  // u32s between counters
// Readies the XCD exchange for a launch of `tiles` tiles with `part_bytes` of
// partial slots: false (no error set) when the device's placement did not
// check out or the tiles do not fit the counters; T0MI_ERR_* when a buffer
// could not be made.  Fills *x.
int xk_prepare(t0mi_ctx* ctx, uint32_t tiles, size_t part_bytes, XcdExchange* x, bool* ok);
// Runs a GEMM with the best prebuilt config for (m, n, k, transpose) and the
// given output type (cost-model ranking, as t0mi_auto_select), as two launches
// over column ranges where plan_column_split says so; NT calls of up to 16 rows
// run the persistent decode kernel instead (run_gemm_decode_nt).  Asynchronous.
int run_gemm_auto(t0mi_ctx* ctx, uint32_t transpose, uint64_t x, uint64_t b, uint64_t y, uint32_t m, uint32_t n,
                  uint32_t k, uint32_t out_dtype = T0MI_OUT_F32, uint64_t bias = 0, const EpiChain* epi = nullptr);
// The schedule of an auto-scheduled GEMM: the ranking's first config with a
// prebuilt kernel over columns [0, n1) and, when n1 < n, the planned tail
// config over [n1, n) (plan_column_split with `cus` compute units).  False
// when no prebuilt kernel fits.  Host only.
struct AutoPlan {
  t0mi_gemm_config head, tail;
  const GemmLaunchEntry *e_head = nullptr, *e_tail = nullptr;
  uint32_t n1 = 0;
};
bool auto_plan(uint32_t m, uint32_t n, uint32_t k, uint32_t transpose, uint32_t out_dtype, uint32_t cus,
               AutoPlan* pl);
// Runs a plan made by auto_plan for the same (m, n, k, transpose, out_dtype).
// Decode-sized NT GEMMs (1..16 rows, K a multiple of 32, N within one round of
// 16-column units): the one-launch persistent decode kernel
// (gemm_persistent.hip), which beats the split-K schedule there (1 / 16 x 4096
// x 4096, f32 out: 8.5 / 11.5 against 13.6 / 12.4 us).  Returns 1, launching
// nothing, when the call is outside that range or its arguments are invalid.
int run_gemm_decode_nt(t0mi_ctx* ctx, uint64_t x, uint64_t b, uint64_t y, uint32_t m, uint32_t n, uint32_t k,
                       uint32_t out_dtype, uint64_t bias, const EpiChain& epi);
int run_gemm_planned(t0mi_ctx* ctx, const AutoPlan& pl, uint32_t transpose, uint64_t x, uint64_t b, uint64_t y,
                     uint32_t m, uint32_t n, uint32_t k, uint32_t out_dtype = T0MI_OUT_F32, uint64_t bias = 0,
                     const EpiChain* epi = nullptr);
// Launches the bf16 GEMM kernel for (cfg, params) on ctx's stream.
int launch_gemm(t0mi_ctx* ctx, const t0mi_gemm_config& cfg, const GemmLaunchEntry* e, GemmParams p);
int check_ctx(t0mi_ctx* ctx);
// T0MI_ERR_CAPTURE when ctx's stream is being captured into a graph (calls
// that wait, allocate or copy to the host cannot be recorded); `what` names
// the refused call.
int refuse_if_capturing(t0mi_ctx* ctx, const char* what);
// Fills `bytes` bytes at dst with `value` on ctx's stream, with a kernel (a
// memset node recorded into a graph has given wrong results on replay).
int fill_async(t0mi_ctx* ctx, void* dst, uint8_t value, size_t bytes);
// Sums sk f32 planes of [M, N] (ascending plane order), applies the epilogue
// chain and stores f32 or bf16 into y (row stride ldy), on ctx's stream.
int launch_splitk_reduce(t0mi_ctx* ctx, const float* ws, void* y, const float* bias, uint32_t M, uint32_t N,
                         uint32_t ldy, uint32_t sk, uint32_t out_bf16, const EpiChain& epi);
// The chain of a gemm_gen EpilogueOp.
EpiChain chain_of(uint32_t gemm_gen_epilogue);
// Y[m,n] = epi(X . B) with a prebuilt kernel: tile-aligned or not, split-K
// through the workspace and a deterministic reduce.  Asynchronous.  ldn (0: n)
// is the row length of Y and of NN's B, so that the GEMM can cover a column
// range of larger matrices (B, Y and bias then point at its first column).
// A fixed workspace handed to run_gemm in place of ctx->ws: never grown; a
// GEMM that needs more than `cap` bytes of it is refused before any launch.
struct FixedWorkspace {
  void* ptr;
  size_t cap;
};
int run_gemm(t0mi_ctx* ctx, const t0mi_gemm_config& cfg, const GemmLaunchEntry* e, uint64_t x, uint64_t b,
             uint64_t y, uint64_t bias, uint32_t m, uint32_t n, uint32_t k, const EpiChain& epi,
             const FixedWorkspace* fixed = nullptr, uint32_t ldn = 0);
// True when the chain contains `op`.
inline bool chain_uses(const EpiChain& e, uint32_t op) {
  for (uint32_t i = 0; i < e.n; ++i)
    if (((e.ops >> (4 * i)) & 0xFu) == op) return true;
  return false;
}
// Persistent TileGemm specs (gemm_persistent.hip): up to this many rows (K a multiple
// of 32, or 0) the decode kernel, else the spec's tile kernel with a grid-stride tile loop.
constexpr uint32_t kPersistentDecodeRows = 64;
// Which kernel a persistent run of `cfg` (the spec's lowered config) takes:
// "decode", "tiles" (persistent tile loop) or "one-shot" (a tile with no persistent
// instantiation: the one-shot kernel of the same tile).
const char* persistent_route(const t0mi_gemm_config& cfg, uint32_t m, uint32_t n, uint32_t k);
// Y = epi(X . B) for a persistent spec: one launch of a persistent kernel, the whole K
// sum in one plane (as the reference's persistent lowering, which ignores split-K).
// Asynchronous.
int run_gemm_persistent(t0mi_ctx* ctx, const t0mi_gemm_config& cfg, const GemmLaunchEntry* e, uint64_t x,
                        uint64_t b, uint64_t y, uint64_t bias, uint32_t m, uint32_t n, uint32_t k,
                        const EpiChain& epi);
}  // namespace t0mi
