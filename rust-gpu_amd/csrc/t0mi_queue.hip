// t0mi_queue.hip — batched submission: the reference's DispatchQueue and its
// MI355X form, a captured HIP graph.
//
//   DispatchQueue::{new, submit, flush, pending, drop_async}, batch_dispatch
//       src/t0/prefill_dispatch.rs:58-214
//
// The reference batches AQL packets (barrier bit, agent-scope fences) so that
// N dispatches cost one wait instead of N.  On HIP the runtime's stream already
// orders launches, so a queue is N asynchronous launches and one wait; the
// per-launch host cost that remains (argument parsing, hipLaunchKernel) is
// what a graph removes: the calls are recorded once from the runtime's stream
// and replayed with one hipGraphLaunch.  Every library call that only launches
// kernels can be recorded (dispatches, t0mi_gemm, tile GEMMs, W4A16, the Ignis
// matmuls, t0mi_memset); calls that wait, allocate or copy to the host are
// refused while capturing (T0MI_ERR_CAPTURE) and leave the capture usable.
#include <stdio.h>

#include "t0mi_ctx.h"

using namespace t0mi;

struct t0mi_dispatch_queue {
  t0mi_ctx* ctx;
  size_t pending;  // dispatches submitted since the last flush
  size_t slot;     // the reference's kernarg ring slot counter (informational)
};

struct t0mi_graph {
  t0mi_ctx* ctx;
  hipGraph_t graph;
  hipGraphExec_t exec;
  size_t nodes;
};

static int hip_fail(hipError_t e, const char* what) {
  return set_error(T0MI_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

// ------------------------------------------------------------ DispatchQueue ----

extern "C" int t0mi_dq_new(t0mi_ctx* ctx, t0mi_dispatch_queue** out) {
  if (!ctx || !out) return set_error(T0MI_ERR_INVALID, "null argument");
  *out = new t0mi_dispatch_queue{ctx, 0, 0};
  return T0MI_OK;
}

extern "C" int t0mi_dq_submit(t0mi_dispatch_queue* q, const t0mi_kernel* k, const uint32_t grid[3],
                              const uint8_t* ka, size_t ka_len) {
  if (!q) return set_error(T0MI_ERR_INVALID, "null queue");
  // prefill_dispatch.rs:96-99: a poisoned runtime refuses new work.
  if (q->ctx->poisoned.load()) return set_error(T0MI_ERR_POISONED, "[DispatchQueue] Queue poisoned — refusing submit");
  int rc = t0mi_dispatch_async(q->ctx, k, grid, ka, ka_len);
  if (rc) return rc;
  q->pending += 1;
  q->slot += 1;
  return T0MI_OK;
}

extern "C" int t0mi_dq_flush(t0mi_dispatch_queue* q, size_t* count) {
  if (!q) return set_error(T0MI_ERR_INVALID, "null queue");
  if (count) *count = 0;
  if (q->pending == 0) return T0MI_OK;
  const size_t n = q->pending;
  q->pending = 0;
  // One wait for the whole batch; a failed or timed-out wait poisons the
  // runtime (prefill_dispatch.rs:145-165).
  int rc = t0mi_wait_idle(q->ctx);
  if (rc) {
    if (rc != T0MI_ERR_CAPTURE) q->ctx->poisoned.store(true);
    if (rc == T0MI_ERR_CAPTURE) q->pending = n;  // nothing waited; the batch is still pending
    return rc;
  }
  if (count) *count = n;
  return T0MI_OK;
}

extern "C" size_t t0mi_dq_pending(const t0mi_dispatch_queue* q) { return q ? q->pending : 0; }

extern "C" void t0mi_dq_drop_async(t0mi_dispatch_queue* q) {
  if (!q) return;
  // prefill_dispatch.rs:177-187: the launches stay in the stream and complete
  // on their own; the caller keeps the buffers alive until a later wait.
  if (q->pending > 0) fprintf(stderr, "[DispatchQueue] Warning: %zu dispatches dropped without flush()\n", q->pending);
  delete q;
}

extern "C" int t0mi_batch_dispatch(t0mi_ctx* ctx, size_t n, const t0mi_kernel* const* kernels, const uint32_t* grids,
                                   const uint8_t* const* kas, const size_t* ka_lens, size_t* count) {
  if (!ctx || (n && (!kernels || !grids || !kas || !ka_lens))) return set_error(T0MI_ERR_INVALID, "null argument");
  if (count) *count = 0;
  t0mi_dispatch_queue q{ctx, 0, 0};
  for (size_t i = 0; i < n; ++i) {
    int rc = t0mi_dq_submit(&q, kernels[i], grids + 3 * i, kas[i], ka_lens[i]);
    if (rc) return rc;  // earlier launches are in the stream, as with the reference's `?`
  }
  return t0mi_dq_flush(&q, count);
}

// ------------------------------------------------------------- HIP graphs ----

extern "C" int t0mi_capture_begin(t0mi_ctx* ctx) {
  int rc = check_ctx(ctx);
  if (rc) return rc;
  if (ctx->null_backend) return set_error(T0MI_ERR_NO_DEVICE, "null runtime has no stream to capture");
  if (!ctx->stream) return set_error(T0MI_ERR_INVALID, "the null (default) stream cannot be captured");
  T0MI_SUBMIT_GUARD(ctx);
  rc = refuse_if_capturing(ctx, "t0mi_capture_begin");
  if (rc) return rc;
  (void)hipSetDevice(ctx->device);
  // Thread-local mode: only this thread's unsafe calls affect the capture.
  hipError_t e = hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal);
  return e == hipSuccess ? T0MI_OK : hip_fail(e, "hipStreamBeginCapture");
}

extern "C" int t0mi_capture_end(t0mi_ctx* ctx, t0mi_graph** out) {
  if (!ctx || !out) return set_error(T0MI_ERR_INVALID, "null argument");
  *out = nullptr;
  if (ctx->null_backend) return set_error(T0MI_ERR_NO_DEVICE, "null runtime has no stream to capture");
  T0MI_SUBMIT_GUARD(ctx);
  hipGraph_t g = nullptr;
  hipError_t e = hipStreamEndCapture(ctx->stream, &g);
  if (e != hipSuccess) {
    if (g) (void)hipGraphDestroy(g);
    return hip_fail(e, "hipStreamEndCapture");
  }
  size_t nodes = 0;
  e = hipGraphGetNodes(g, nullptr, &nodes);
  if (e != hipSuccess) {
    (void)hipGraphDestroy(g);
    return hip_fail(e, "hipGraphGetNodes");
  }
  hipGraphExec_t ex = nullptr;
  e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
  if (e != hipSuccess) {
    (void)hipGraphDestroy(g);
    return hip_fail(e, "hipGraphInstantiate");
  }
  *out = new t0mi_graph{ctx, g, ex, nodes};
  ctx->live_graphs.fetch_add(1);
  return T0MI_OK;
}

extern "C" int t0mi_graph_launch(t0mi_graph* g) {
  if (!g) return set_error(T0MI_ERR_INVALID, "null graph");
  int rc = check_ctx(g->ctx);
  if (rc) return rc;
  T0MI_SUBMIT_GUARD(g->ctx);
  rc = refuse_if_capturing(g->ctx, "t0mi_graph_launch");
  if (rc) return rc;
  hipError_t e = hipGraphLaunch(g->exec, g->ctx->stream);
  return e == hipSuccess ? T0MI_OK : hip_fail(e, "hipGraphLaunch");
}

extern "C" size_t t0mi_graph_node_count(const t0mi_graph* g) { return g ? g->nodes : 0; }

extern "C" void t0mi_graph_destroy(t0mi_graph* g) {
  if (!g) return;
  // A replay may still be running: the executable graph is destroyed only
  // after the stream has drained (a poisoned runtime is not waited on).
  if (!g->ctx->poisoned.load() && refuse_if_capturing(g->ctx, "t0mi_graph_destroy") == T0MI_OK)
    (void)hipStreamSynchronize(g->ctx->stream);
  (void)hipGraphExecDestroy(g->exec);
  (void)hipGraphDestroy(g->graph);
  g->ctx->live_graphs.fetch_sub(1);
  delete g;
}
