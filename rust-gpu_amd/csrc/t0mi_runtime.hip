// t0mi_runtime.hip — the HIP shim that replaces the reference's KFD/AQL runtime.
//
//   GpuRuntime::new / dispatch / dispatch_async / wait_idle / alloc / poison
//       src/ignis/gpu_context.rs:151-545
//   GpuKernel::load + KernelLoadConfig            src/kfd/kernel.rs:26-141
//   AqlQueue::submit / synchronize (timeout)      src/kfd/aql.rs:184-249, 481-545
//
// Kernels are not generated and assembled at run time: every config maps to a
// prebuilt gfx950 kernel in this library (gemm_inst.hip).  Dispatch keeps the
// reference's contract — HSA work-item grids, raw kernarg bytes whose length
// must equal the kernel's declaration, synchronous wait with a timeout that
// poisons the runtime — and turns it into a hipLaunchKernelGGL on the
// runtime's stream.
#include <sched.h>
#include <tuple>
#include <string.h>
#include <time.h>

#include "t0mi_ctx.h"
#include "xcd_exchange.h"

using namespace t0mi;

namespace t0mi {

const GemmLaunchEntry* find_gemm_launch(const t0mi_gemm_config& c) {
  uint32_t wm, wn;
  if (!wave_layout(c, &wm, &wn)) return nullptr;
  const bool nn = c.transpose == T0MI_NN;
  const GemmLaunchEntry* (*tables[])(size_t*) = {nn ? gemm_table_p0_nn : gemm_table_p0_nt,
                                                nn ? gemm_table_p1_nn : gemm_table_p1_nt,
                                                nn ? gemm_table_p2_nn : gemm_table_p2_nt,
                                                nn ? gemm_table_p3_nn : gemm_table_p3_nt};
  for (auto tf : tables) {
    size_t n = 0;
    const GemmLaunchEntry* t = tf(&n);
    for (size_t i = 0; i < n; ++i)
      if ((uint32_t)t[i].bm == c.tile_m && (uint32_t)t[i].bn == c.tile_n && (uint32_t)t[i].bk == c.tile_k &&
          (uint32_t)t[i].wm == wm && (uint32_t)t[i].wn == wn && (uint32_t)t[i].stages == stages_of(c))
        return &t[i];
  }
  return nullptr;
}

int check_ctx(t0mi_ctx* ctx) {
  if (!ctx) return set_error(T0MI_ERR_INVALID, "null runtime");
  if (ctx->poisoned.load())
    return set_error(T0MI_ERR_POISONED,
                     "[t0mi] runtime poisoned after a failed wait; refusing dispatch (create a new runtime)");
  return T0MI_OK;
}

static int hip_fail(hipError_t e, const char* what) {
  return set_error(T0MI_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

int refuse_if_capturing(t0mi_ctx* ctx, const char* what) {
  if (ctx->null_backend || !ctx->stream) return T0MI_OK;  // the null stream cannot be captured
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  hipError_t e = hipStreamIsCapturing(ctx->stream, &st);
  if (e != hipSuccess) return hip_fail(e, "hipStreamIsCapturing");
  if (st != hipStreamCaptureStatusNone)
    return set_error(T0MI_ERR_CAPTURE, "%s cannot run while the runtime's stream is being captured", what);
  return T0MI_OK;
}

// Byte fill: 16-byte stores over the aligned middle, single bytes at the ends.
__global__ __launch_bounds__(256) void t0mi_fill_kernel(uint8_t* __restrict__ dst, uint32_t word, size_t head,
                                                        size_t body16, size_t n) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x, stride = (size_t)gridDim.x * blockDim.x;
  const u32x4 q = {word, word, word, word};
  u32x4* mid = (u32x4*)(dst + head);
  for (size_t j = i; j < body16; j += stride) mid[j] = q;
  const size_t tail0 = head + body16 * 16;
  if (i < head) dst[i] = (uint8_t)word;
  if (i < n - tail0) dst[tail0 + i] = (uint8_t)word;
}

int fill_async(t0mi_ctx* ctx, void* dst, uint8_t value, size_t bytes) {
  if (bytes == 0 || ctx->null_backend) return T0MI_OK;
  const size_t mis = (uintptr_t)dst & 15;
  const size_t head = std::min(bytes, mis ? 16 - mis : (size_t)0);
  const size_t body16 = (bytes - head) / 16;
  // head and tail are < 16 bytes each, covered by the first workgroup.
  const size_t blocks = std::max<size_t>(1, std::min<size_t>((body16 + 255) / 256, (size_t)ctx->cu_count * 8));
  hipLaunchKernelGGL(t0mi_fill_kernel, dim3((uint32_t)blocks), dim3(256), 0, ctx->stream, (uint8_t*)dst,
                     value * 0x01010101u, head, body16, bytes);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? T0MI_OK : hip_fail(e, "fill launch");
}

// A buffer that graphs still reference cannot be replaced; one that must grow
// while the stream is captured cannot be allocated (run the work once eagerly
// first: the buffers only grow, so a captured replay then fits).
static int check_growth(t0mi_ctx* ctx, const char* what, size_t have, size_t want) {
  if (ctx->live_graphs.load() > 0)
    return set_error(T0MI_ERR_CAPTURE,
                     "%s must grow from %zu to %zu bytes but %d live graph(s) reference it; destroy them first",
                     what, have, want, ctx->live_graphs.load());
  int rc = refuse_if_capturing(ctx, "growing the library workspace");
  if (rc)
    set_error(T0MI_ERR_CAPTURE,
              "%s must grow from %zu to %zu bytes while the stream is captured; run the work once before capturing",
              what, have, want);
  return rc;
}

int ensure_workspace(t0mi_ctx* ctx, size_t bytes) {
  if (ctx->ws_bytes >= bytes) return T0MI_OK;
  if (ctx->null_backend) {
    ctx->ws_bytes = bytes;
    return T0MI_OK;
  }
  if (int rc = check_growth(ctx, "the split-K workspace", ctx->ws_bytes, bytes)) return rc;
  hipError_t e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
  if (ctx->ws) (void)hipFree(ctx->ws);
  ctx->ws = nullptr;
  ctx->ws_bytes = 0;
  size_t want = bytes + (bytes >> 2);  // grow with slack
  e = hipMalloc(&ctx->ws, want);
  if (e != hipSuccess) return hip_fail(e, "hipMalloc(workspace)");
  ctx->ws_bytes = want;
  return T0MI_OK;
}

int ensure_cvt_buffer(t0mi_ctx* ctx, size_t bytes) {
  if (ctx->cvt_bytes >= bytes) return T0MI_OK;
  if (ctx->null_backend) {
    ctx->cvt_bytes = bytes;
    return T0MI_OK;
  }
  if (int rc = check_growth(ctx, "the conversion buffer", ctx->cvt_bytes, bytes)) return rc;
  hipError_t e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
  if (ctx->cvt) (void)hipFree(ctx->cvt);
  ctx->cvt = nullptr;
  ctx->cvt_bytes = 0;
  size_t want = bytes + (bytes >> 2);
  e = hipMalloc(&ctx->cvt, want);
  if (e != hipSuccess) return hip_fail(e, "hipMalloc(conversion buffer)");
  ctx->cvt_bytes = want;
  return T0MI_OK;
}

int xk_prepare(t0mi_ctx* ctx, uint32_t tiles, size_t part_bytes, XcdExchange* x, bool* ok) {
  *ok = false;
  if (ctx->null_backend || ctx->xk_nx == 0) return T0MI_OK;
  if ((tiles + ctx->xk_nx - 1) / ctx->xk_nx > kXkCountersPerXcd) return T0MI_OK;
  const size_t tick_bytes = ((size_t)ctx->xk_nx * kXkCountersPerXcd + 1) * kXkCounterStride * 4;  // + the flag
  if (!ctx->xk_tick) {
    if (int rc = check_growth(ctx, "the exchange counters", 0, tick_bytes)) return rc;
    hipError_t e = hipMalloc((void**)&ctx->xk_tick, tick_bytes);
    if (e != hipSuccess) return hip_fail(e, "hipMalloc(exchange counters)");
    if (int rc = fill_async(ctx, ctx->xk_tick, 0, tick_bytes)) return rc;
    e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
  }
  if (ctx->xk_part_bytes < part_bytes) {
    if (int rc = check_growth(ctx, "the exchange slots", ctx->xk_part_bytes, part_bytes)) return rc;
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
    if (ctx->xk_part) (void)hipFree(ctx->xk_part);
    ctx->xk_part = nullptr;
    ctx->xk_part_bytes = 0;
    const size_t want = part_bytes + (part_bytes >> 2);
    e = hipMalloc(&ctx->xk_part, want);
    if (e != hipSuccess) return hip_fail(e, "hipMalloc(exchange slots)");
    ctx->xk_part_bytes = want;
  }
  x->part = (float*)ctx->xk_part;
  x->tick = ctx->xk_tick;
  x->flag = ctx->xk_tick + (size_t)ctx->xk_nx * kXkCountersPerXcd * kXkCounterStride;
  x->nx = ctx->xk_nx;
  x->tpx = kXkCountersPerXcd;
  x->stride = kXkCounterStride;
  *ok = true;
  return T0MI_OK;
}

int launch_gemm(t0mi_ctx* ctx, const t0mi_gemm_config& cfg, const GemmLaunchEntry* e, GemmParams p) {
  const uint32_t nwg = p.tiles_m * p.tiles_n * p.split_k;
  if (nwg == 0) return T0MI_OK;
  // Grid axes follow the reference convention (swap_grid: x -> N tiles); the
  // kernel decodes the tile from the linear workgroup id either way.
  dim3 grid = cfg.swap_grid ? dim3(p.tiles_n, p.tiles_m * p.split_k) : dim3(p.tiles_m, p.tiles_n * p.split_k);
  p.swap_grid = cfg.swap_grid;
  // With every workgroup resident from the start, all tiles finish together and
  // the whole output is written at the end of the launch: stream it past the
  // L2 (non-temporal) instead of leaving it dirty there (4096^3 NN: ~1% faster;
  // with more tiles than CUs, normal stores are faster).
  p.stream_out = nwg <= (uint32_t)ctx->cu_count;
  if (ctx->null_backend) return T0MI_OK;
  e->fn(grid, ctx->stream, p);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return hip_fail(err, "gemm launch");
  return T0MI_OK;
}

}  // namespace t0mi

// ------------------------------------------------------------ split-K reduce --
// Deterministic reduction of split-K partial planes: y = sum_{p=0..sk-1} ws[p]
// in ascending p, then the epilogue chain, then f32 or bf16 (RNE) store.
// Each thread owns one 4-column vector and issues the loads of up to 16
// planes before the first add, so a call's partials stream in one round trip
// (the planes were just written and are mostly served by the Infinity Cache).
template <int SK>  // planes handled with all loads in flight (0: any count, 4 at a time)
__global__ __launch_bounds__(256) void t0mi_splitk_reduce(const float* __restrict__ ws, void* __restrict__ y,
                                                          const float* __restrict__ bias, uint32_t M, uint32_t N,
                                                          uint32_t ldy, uint32_t sk, uint32_t out_bf16,
                                                          EpiChain epi) {
  const size_t plane = (size_t)M * N;
  const size_t nvec = plane / 4;
  const uint32_t nq = N / 4;  // N % 8 == 0: a vector never straddles rows
  for (size_t v = blockIdx.x * (size_t)blockDim.x + threadIdx.x; v < nvec; v += (size_t)gridDim.x * blockDim.x) {
    const size_t idx = v * 4;
    const uint32_t m = (uint32_t)(v / nq), n = (uint32_t)(v % nq) * 4;
    f32x4 s;
    if constexpr (SK > 0) {
      f32x4 t[SK];
#pragma unroll
      for (int j = 0; j < SK; ++j) t[j] = __builtin_nontemporal_load((const f32x4*)(ws + j * plane + idx));
      s = t[0];
#pragma unroll
      for (int j = 1; j < SK; ++j) {
        s.x += t[j].x;
        s.y += t[j].y;
        s.z += t[j].z;
        s.w += t[j].w;
      }
    } else {
      // Planes read four at a time (independent loads in flight together) and
      // summed in plane order, so the result does not depend on timing.
      s = f32x4{0.f, 0.f, 0.f, 0.f};
      for (uint32_t q0 = 0; q0 < sk; q0 += 4) {
        f32x4 t[4];
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) {
          const uint32_t q = q0 + j < sk ? q0 + j : q0;  // past the last plane: a repeat, not added
          t[j] = *(const f32x4*)(ws + q * plane + idx);
        }
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) {
          if (q0 + j >= sk) break;
          if (q0 + j == 0) {
            s = t[0];
          } else {
            s.x += t[j].x;
            s.y += t[j].y;
            s.z += t[j].z;
            s.w += t[j].w;
          }
        }
      }
    }
    if (epi.n) {
      f32x4 bv = {0.f, 0.f, 0.f, 0.f};
      if (bias) bv = f32x4{bias[n], bias[n + 1], bias[n + 2], bias[n + 3]};
      s.x = epi_apply(s.x, bv.x, epi);
      s.y = epi_apply(s.y, bv.y, epi);
      s.z = epi_apply(s.z, bv.z, epi);
      s.w = epi_apply(s.w, bv.w, epi);
    }
    if (out_bf16) {
      u32x2 o;
      o.x = (uint32_t)f32_to_bf16_rne(s.x) | ((uint32_t)f32_to_bf16_rne(s.y) << 16);
      o.y = (uint32_t)f32_to_bf16_rne(s.z) | ((uint32_t)f32_to_bf16_rne(s.w) << 16);
      *(u32x2*)((uint16_t*)y + (size_t)m * ldy + n) = o;
    } else {
      *(f32x4*)((float*)y + (size_t)m * ldy + n) = s;
    }
  }
}

namespace t0mi {
EpiChain chain_of(uint32_t gemm_gen_epilogue) {
  EpiChain e;
  memset(&e, 0, sizeof e);
  if (gemm_gen_epilogue == T0MI_EPI_BIAS_ADD_STORE_F32) {
    e.n = 1;
    e.ops = EOP_BIAS;
  } else if (gemm_gen_epilogue == T0MI_EPI_BIAS_ADD_RELU_STORE_F32) {
    e.n = 2;
    e.ops = EOP_BIAS | (EOP_RELU << 4);
  }
  return e;
}


int launch_splitk_reduce(t0mi_ctx* ctx, const float* ws, void* y, const float* bias, uint32_t M, uint32_t N,
                         uint32_t ldy, uint32_t sk, uint32_t out_bf16, const EpiChain& epilogue) {
  if (ctx->null_backend) return T0MI_OK;
  const size_t nvec = (size_t)M * N / 4;
  if (nvec == 0) return T0MI_OK;
  const uint32_t blocks = (uint32_t)std::min<size_t>((nvec + 255) / 256, (size_t)ctx->cu_count * 8);
#define T0MI_REDUCE(SKC)                                                                                     \
  hipLaunchKernelGGL(t0mi_splitk_reduce<SKC>, dim3(blocks), dim3(256), 0, ctx->stream, ws, y, bias, M, N, ldy, sk, \
                     out_bf16, epilogue)
  switch (sk) {
    case 1: T0MI_REDUCE(1); break;
    case 2: T0MI_REDUCE(2); break;
    case 4: T0MI_REDUCE(4); break;
    case 8: T0MI_REDUCE(8); break;
    case 16: T0MI_REDUCE(16); break;
    default: T0MI_REDUCE(0); break;
  }
#undef T0MI_REDUCE
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? T0MI_OK : hip_fail(e, "reduce launch");
}
}  // namespace t0mi

// ------------------------------------------- scratch of t0mi_gemm_noalloc ----

// Split-K partial planes of t0mi_gemm_noalloc.  Every GPU the library runs on
// holds its own copy until the process ends.  In host code `scratch` names a
// host-side stand-in: only the address hipGetSymbolAddress returns for a
// device may reach a kernel or a copy.
static __device__ __align__(256) uint8_t scratch[T0MI_NOALLOC_SCRATCH_BYTES];

// This device's address of `scratch`, looked up once per device with that
// device current (the caller has made it current).
static int scratch_for_device(int dev, void** out) {
  static std::mutex mu;
  static std::map<int, std::pair<void*, hipError_t>> known;
  std::lock_guard<std::mutex> lock(mu);
  auto it = known.find(dev);
  if (it == known.end()) {
    void* ptr = nullptr;
    hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) ptr = nullptr;
    it = known.emplace(dev, std::make_pair(ptr, e)).first;
  }
  *out = it->second.first;
  if (it->second.second != hipSuccess)
    return set_error(T0MI_ERR_HIP, "hipGetSymbolAddress(scratch) on device %d: %s", dev,
                     hipGetErrorString(it->second.second));
  return T0MI_OK;
}

// Who used this device's scratch last: the stream of the last
// t0mi_gemm_noalloc call on the device and an event recorded after its
// launches.  A call from another stream while that event has not completed
// would overwrite planes still being summed: it is refused instead.  The
// event is made at set-up (the first runtime created on the device), so the
// entry point itself creates nothing.
struct ScratchUse {
  std::mutex mu;
  hipStream_t last = nullptr;
  hipEvent_t done = nullptr;
  bool recorded = false;
};
static ScratchUse* scratch_use_for_device(int dev, bool create) {
  static std::mutex mu;
  static std::map<int, ScratchUse*> known;  // held until the process ends, like the scratch itself
  std::lock_guard<std::mutex> lock(mu);
  auto it = known.find(dev);
  if (it != known.end()) return it->second;
  if (!create) return nullptr;
  ScratchUse* u = new ScratchUse();
  if (hipEventCreateWithFlags(&u->done, hipEventDisableTiming) != hipSuccess) u->done = nullptr;
  (void)hipGetLastError();
  known.emplace(dev, u);
  return u;
}

// ------------------------------------------------ XCD placement probe ----

// Workgroup i records the XCD it runs on.
__global__ void t0mi_placement_kernel(uint32_t* out) {
  if (threadIdx.x == 0) out[blockIdx.x] = t0mi::xcc_id();
}

// Once per device (the caller has made it current): launches the probe at
// several grid sizes and returns nx when every workgroup i of every launch ran
// on XCD i % nx (nx = the number of XCDs seen), else 0.  The in-launch
// exchange of split-K partials relies on it.
static uint32_t placement_for_device(int dev) {
  static std::mutex mu;
  static std::map<int, uint32_t> known;
  std::lock_guard<std::mutex> lock(mu);
  auto it = known.find(dev);
  if (it != known.end()) return it->second;
  uint32_t nx = 0;
  constexpr uint32_t kMaxGrid = 4096;
  uint32_t* d = nullptr;
  hipStream_t st = nullptr;
  std::vector<uint32_t> h(kMaxGrid);
  bool ok = hipMalloc((void**)&d, kMaxGrid * 4) == hipSuccess &&
            hipStreamCreateWithFlags(&st, hipStreamNonBlocking) == hipSuccess;
  for (uint32_t grid : {64u, 1000u, kMaxGrid}) {
    if (!ok) break;
    hipLaunchKernelGGL(t0mi_placement_kernel, dim3(grid), dim3(64), 0, st, d);
    ok = hipGetLastError() == hipSuccess && hipMemcpyAsync(h.data(), d, grid * 4, hipMemcpyDeviceToHost, st) == hipSuccess &&
         hipStreamSynchronize(st) == hipSuccess;
    if (!ok) break;
    uint32_t seen = 0;
    for (uint32_t i = 0; i < grid; ++i) seen = std::max(seen, h[i] + 1);
    for (uint32_t i = 0; i < grid && ok; ++i) ok = h[i] == i % seen;
    if (ok && nx && seen != nx) ok = false;
    nx = seen;
  }
  if (st) (void)hipStreamDestroy(st);
  if (d) (void)hipFree(d);
  (void)hipGetLastError();  // a failed probe only turns the exchange off
  const uint32_t res = ok && nx >= 1 && nx <= 16 ? nx : 0;
  known.emplace(dev, res);
  return res;
}

extern "C" int t0mi_xcd_placement(t0mi_ctx* ctx, uint32_t* n_xcd, uint32_t* misplaced) {
  if (!ctx) return set_error(T0MI_ERR_INVALID, "null runtime");
  if (n_xcd) *n_xcd = ctx->xk_nx;
  if (misplaced) *misplaced = 0;
  if (ctx->null_backend || !ctx->xk_tick || !misplaced) return T0MI_OK;
  if (int rc = refuse_if_capturing(ctx, "t0mi_xcd_placement")) return rc;
  hipError_t e = hipMemcpyAsync(misplaced, ctx->xk_tick + (size_t)ctx->xk_nx * kXkCountersPerXcd * kXkCounterStride, 4,
                                hipMemcpyDeviceToHost, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  return e == hipSuccess ? T0MI_OK : hip_fail(e, "reading the placement flag");
}

// ===================================================================== C ABI ==

static int ctx_create(int device, bool use_given_stream, void* hip_stream, t0mi_ctx** out) {
  if (!out) return set_error(T0MI_ERR_INVALID, "null out");
  *out = nullptr;
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n == 0) return set_error(T0MI_ERR_NO_DEVICE, "no HIP device visible (%s)", hipGetErrorString(e));
  int dev = device;
  if (dev < 0) {
    for (int i = 0; i < n; ++i) {
      hipDeviceProp_t pr;
      if (hipGetDeviceProperties(&pr, i) == hipSuccess && strncmp(pr.gcnArchName, "gfx950", 6) == 0) {
        dev = i;
        break;
      }
    }
    if (dev < 0) return set_error(T0MI_ERR_NO_DEVICE, "no gfx950 device among %d HIP devices", n);
  }
  if (dev >= n) return set_error(T0MI_ERR_NO_DEVICE, "device %d out of range (%d devices)", dev, n);
  hipDeviceProp_t pr;
  e = hipGetDeviceProperties(&pr, dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDeviceProperties");
  if (strncmp(pr.gcnArchName, "gfx950", 6) != 0)
    return set_error(T0MI_ERR_NO_DEVICE, "device %d is %s; kernels are built for gfx950 only", dev, pr.gcnArchName);
  e = hipSetDevice(dev);
  if (e != hipSuccess) return hip_fail(e, "hipSetDevice");
  t0mi_ctx* c = new t0mi_ctx();
  c->device = dev;
  c->cu_count = pr.multiProcessorCount;
  if (use_given_stream) {
    // The caller's stream, including the null (default) stream.
    c->stream = (hipStream_t)hip_stream;
    c->own_stream = false;
  } else {
    e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
      delete c;
      return hip_fail(e, "hipStreamCreate");
    }
    c->own_stream = true;
  }
  // A failed lookup leaves the runtime usable; only t0mi_gemm_noalloc reports it.
  c->scratch_rc = scratch_for_device(dev, &c->scratch);
  (void)scratch_use_for_device(dev, true);
  c->xk_nx = placement_for_device(dev);
  *out = c;
  return T0MI_OK;
}

extern "C" int t0mi_ctx_create_on_stream(int device, void* hip_stream, t0mi_ctx** out) {
  return ctx_create(device, true, hip_stream, out);
}

extern "C" int t0mi_ctx_create(int device, t0mi_ctx** out) { return ctx_create(device, false, nullptr, out); }

extern "C" int t0mi_ctx_create_null(t0mi_ctx** out) {
  if (!out) return set_error(T0MI_ERR_INVALID, "null out");
  t0mi_ctx* c = new t0mi_ctx();
  c->null_backend = true;
  *out = c;
  return T0MI_OK;
}

extern "C" void t0mi_ctx_destroy(t0mi_ctx* ctx) {
  if (!ctx) return;
  if (!ctx->null_backend) {
    (void)hipSetDevice(ctx->device);
    if (!ctx->poisoned.load()) (void)hipStreamSynchronize(ctx->stream);
    for (auto& kv : ctx->allocs) (void)hipFree((void*)kv.first);
    for (auto& kv : ctx->pool)
      for (uint64_t p : kv.second) (void)hipFree((void*)p);
    if (ctx->ws) (void)hipFree(ctx->ws);
    if (ctx->cvt) (void)hipFree(ctx->cvt);
    if (ctx->xk_tick) (void)hipFree(ctx->xk_tick);
    if (ctx->xk_part) (void)hipFree(ctx->xk_part);
    if (ctx->own_stream) (void)hipStreamDestroy(ctx->stream);
  }
  delete ctx;
}

extern "C" void* t0mi_ctx_stream(t0mi_ctx* ctx) { return ctx ? (void*)ctx->stream : nullptr; }
extern "C" int t0mi_is_poisoned(t0mi_ctx* ctx) { return ctx && ctx->poisoned.load() ? 1 : 0; }
extern "C" void t0mi_mark_poisoned(t0mi_ctx* ctx) {
  if (ctx) ctx->poisoned.store(true);
}
extern "C" void t0mi_set_timeout_ms(t0mi_ctx* ctx, uint32_t ms) {
  if (ctx) ctx->timeout_ms = ms;
}

extern "C" int t0mi_null_inject_timeout(t0mi_ctx* ctx) {
  if (!ctx || !ctx->null_backend) return set_error(T0MI_ERR_INVALID, "not a null runtime");
  ctx->inject_timeout = true;
  return T0MI_OK;
}

extern "C" int t0mi_null_last_dispatch(t0mi_ctx* ctx, uint32_t grid[3], uint8_t* ka, size_t ka_cap, size_t* ka_len) {
  if (!ctx || !ctx->null_backend) return set_error(T0MI_ERR_INVALID, "not a null runtime");
  if (grid) memcpy(grid, ctx->last_grid, sizeof ctx->last_grid);
  if (ka_len) *ka_len = ctx->last_ka.size();
  if (ka && ka_cap) memcpy(ka, ctx->last_ka.data(), std::min(ka_cap, ctx->last_ka.size()));
  return T0MI_OK;
}

// ---------------------------------------------------------------- memory ----

// BufferPool::alloc (gpu_context.rs:54-73): the size rounded up to 4096 bytes
// is the pool key; a recycled buffer of that size is handed out again, zeroed
// on the stream before any later work (a fill kernel, so that no stale
// contents reach the next user), else a fresh one is allocated (contents
// undefined, as the reference's alloc_vram).
static int pool_alloc(t0mi_ctx* ctx, size_t bytes, uint64_t* dptr, bool* reused) {
  const size_t aligned = ((bytes ? bytes : 1) + 4095) / 4096 * 4096;
  uint64_t p = 0;
  {
    std::lock_guard<std::mutex> lk(ctx->mu);
    auto it = ctx->pool.find(aligned);
    if (it != ctx->pool.end() && !it->second.empty()) {
      p = it->second.back();
      it->second.pop_back();
      ctx->pool_bytes -= aligned;
      ctx->allocs[p] = aligned;
    }
  }
  *reused = p != 0;
  if (p) {
    T0MI_SUBMIT_GUARD(ctx);
    int rc = fill_async(ctx, (void*)p, 0, aligned);
    if (rc) return rc;
    *dptr = p;
    return T0MI_OK;
  }
  if (int rc = refuse_if_capturing(ctx, "t0mi_alloc")) return rc;
  void* q = nullptr;
  hipError_t e = hipMalloc(&q, aligned);
  if (e != hipSuccess) return hip_fail(e, "hipMalloc");
  std::lock_guard<std::mutex> lk(ctx->mu);
  ctx->allocs[(uint64_t)q] = aligned;
  *dptr = (uint64_t)q;
  return T0MI_OK;
}

extern "C" int t0mi_alloc(t0mi_ctx* ctx, size_t bytes, uint64_t* dptr) {
  if (!ctx || !dptr) return set_error(T0MI_ERR_INVALID, "null argument");
  if (ctx->null_backend) return set_error(T0MI_ERR_NO_DEVICE, "null runtime has no memory");
  bool reused = false;
  return pool_alloc(ctx, bytes, dptr, &reused);
}

// GpuRuntime::alloc_f32 (gpu_context.rs:520-525): n floats, at least 512 bytes,
// rounded up to 512, zeroed (in stream order).
extern "C" int t0mi_alloc_f32(t0mi_ctx* ctx, size_t n, uint64_t* dptr) {
  if (!ctx || !dptr) return set_error(T0MI_ERR_INVALID, "null argument");
  if (ctx->null_backend) return set_error(T0MI_ERR_NO_DEVICE, "null runtime has no memory");
  if (n > (SIZE_MAX - 511) / 4) return set_error(T0MI_ERR_INVALID, "n=%zu floats overflow", n);
  const size_t bytes = (std::max<size_t>(n * 4, 512) + 511) & ~(size_t)511;
  bool reused = false;
  int rc = pool_alloc(ctx, bytes, dptr, &reused);
  if (rc || reused) return rc;  // a recycled buffer is zeroed by pool_alloc
  T0MI_SUBMIT_GUARD(ctx);
  return fill_async(ctx, (void*)*dptr, 0, (bytes + 4095) / 4096 * 4096);
}

// GpuRuntime::recycle / BufferPool::recycle (gpu_context.rs:76-81, 528-531):
// the buffer goes back to the pool under its aligned size; nothing waits and
// nothing is freed.  Work already queued on the stream that uses it still
// runs first: the buffer's next hand-out is zeroed in stream order after it.
extern "C" int t0mi_recycle(t0mi_ctx* ctx, uint64_t dptr) {
  if (!ctx) return set_error(T0MI_ERR_INVALID, "null runtime");
  std::lock_guard<std::mutex> lk(ctx->mu);
  auto it = ctx->allocs.find(dptr);
  if (it == ctx->allocs.end())
    return set_error(T0MI_ERR_INVALID, "pointer 0x%llx was not allocated by t0mi_alloc", (unsigned long long)dptr);
  ctx->pool[it->second].push_back(dptr);
  ctx->pool_bytes += it->second;
  ctx->allocs.erase(it);
  return T0MI_OK;
}

// BufferPool::cached_bytes (gpu_context.rs:90-93).
extern "C" size_t t0mi_pool_cached_bytes(t0mi_ctx* ctx) {
  if (!ctx) return 0;
  std::lock_guard<std::mutex> lk(ctx->mu);
  return ctx->pool_bytes;
}

// BufferPool::clear (gpu_context.rs:83-88): frees every cached buffer (after
// the stream's queued work, which may still use them).
extern "C" int t0mi_pool_clear(t0mi_ctx* ctx) {
  if (!ctx) return set_error(T0MI_ERR_INVALID, "null runtime");
  if (ctx->null_backend) return T0MI_OK;
  if (int rc = refuse_if_capturing(ctx, "t0mi_pool_clear")) return rc;
  (void)hipStreamSynchronize(ctx->stream);
  std::lock_guard<std::mutex> lk(ctx->mu);
  hipError_t first = hipSuccess;
  for (auto& kv : ctx->pool)
    for (uint64_t p : kv.second) {
      hipError_t e = hipFree((void*)p);
      if (first == hipSuccess) first = e;
    }
  ctx->pool.clear();
  ctx->pool_bytes = 0;
  return first == hipSuccess ? T0MI_OK : hip_fail(first, "hipFree");
}

extern "C" int t0mi_alloc_zero(t0mi_ctx* ctx, size_t bytes, uint64_t* dptr) {
  int rc = t0mi_alloc(ctx, bytes, dptr);
  if (rc) return rc;
  {
    T0MI_SUBMIT_GUARD(ctx);
    rc = fill_async(ctx, (void*)*dptr, 0, bytes);
  }
  if (rc) return rc;
  hipError_t e = hipStreamSynchronize(ctx->stream);
  return e == hipSuccess ? T0MI_OK : hip_fail(e, "hipStreamSynchronize");
}

extern "C" int t0mi_free(t0mi_ctx* ctx, uint64_t dptr) {
  if (!ctx) return set_error(T0MI_ERR_INVALID, "null runtime");
  std::lock_guard<std::mutex> lk(ctx->mu);
  auto it = ctx->allocs.find(dptr);
  if (it == ctx->allocs.end()) return set_error(T0MI_ERR_INVALID, "pointer 0x%llx was not allocated by t0mi_alloc", (unsigned long long)dptr);
  if (int rc = refuse_if_capturing(ctx, "t0mi_free")) return rc;
  (void)hipStreamSynchronize(ctx->stream);
  hipError_t e = hipFree((void*)dptr);
  ctx->allocs.erase(it);
  return e == hipSuccess ? T0MI_OK : hip_fail(e, "hipFree");
}

extern "C" int t0mi_h2d(t0mi_ctx* ctx, uint64_t dst, const void* src, size_t bytes) {
  if (!ctx || ctx->null_backend) return set_error(T0MI_ERR_INVALID, "no device runtime");
  if (int rc = refuse_if_capturing(ctx, "t0mi_h2d")) return rc;
  hipError_t e = hipMemcpyAsync((void*)dst, src, bytes, hipMemcpyHostToDevice, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  return e == hipSuccess ? T0MI_OK : hip_fail(e, "hipMemcpy H2D");
}

extern "C" int t0mi_d2h(t0mi_ctx* ctx, void* dst, uint64_t src, size_t bytes) {
  if (!ctx || ctx->null_backend) return set_error(T0MI_ERR_INVALID, "no device runtime");
  if (int rc = refuse_if_capturing(ctx, "t0mi_d2h")) return rc;
  hipError_t e = hipMemcpyAsync(dst, (const void*)src, bytes, hipMemcpyDeviceToHost, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  return e == hipSuccess ? T0MI_OK : hip_fail(e, "hipMemcpy D2H");
}

extern "C" int t0mi_memset(t0mi_ctx* ctx, uint64_t dst, int value, size_t bytes) {
  if (!ctx || ctx->null_backend) return set_error(T0MI_ERR_INVALID, "no device runtime");
  if (bytes && !dst) return set_error(T0MI_ERR_INVALID, "null destination");
  T0MI_SUBMIT_GUARD(ctx);
  return fill_async(ctx, (void*)dst, (uint8_t)value, bytes);
}

// --------------------------------------------------------------- kernels ----

extern "C" int t0mi_kernel_get(t0mi_ctx* ctx, const t0mi_gemm_config* cfg, t0mi_kernel** out) {
  if (!ctx || !cfg || !out) return set_error(T0MI_ERR_INVALID, "null argument");
  std::string why;
  t0mi_gemm_config phys;
  if (!config_physical(*cfg, &phys, &why))
    return set_error(T0MI_ERR_INVALID, "[t0mi] config '%s' infeasible on gfx950: %s", config_name(*cfg).c_str(),
                     why.c_str());
  const std::string name = config_name(*cfg);
  std::lock_guard<std::mutex> lk(ctx->mu);
  auto it = ctx->kernels.find(name);
  if (it != ctx->kernels.end()) {
    *out = it->second.get();
    return T0MI_OK;
  }
  const GemmLaunchEntry* e = find_gemm_launch(phys);
  if (!e) return set_error(T0MI_ERR_NO_KERNEL, "[t0mi] no prebuilt gfx950 kernel for '%s'", name.c_str());
  std::unique_ptr<t0mi_kernel> k(new t0mi_kernel());
  k->kind = KK_GEMM_GEN;
  k->cfg = *cfg;
  k->phys = phys;
  k->name = name;
  k->kernarg_size = cfg->epilogue == T0MI_EPI_STORE_F32 ? 40u : 48u;
  k->lds_size = t0mi_config_lds_total(cfg);
  k->wg_size = cfg->wg_size;
  k->gemm = e;
  *out = k.get();
  ctx->kernels[name] = std::move(k);
  return T0MI_OK;
}

extern "C" int t0mi_kernel_attrs(const t0mi_kernel* k, uint32_t* lds_size, uint32_t* wg_size, uint32_t* kernarg_size) {
  if (!k) return set_error(T0MI_ERR_INVALID, "null kernel");
  if (lds_size) *lds_size = k->lds_size;
  if (wg_size) *wg_size = k->wg_size;
  if (kernarg_size) *kernarg_size = k->kernarg_size;
  return T0MI_OK;
}

extern "C" int t0mi_kernel_name(const t0mi_kernel* k, char* buf, size_t len) {
  if (!k) return set_error(T0MI_ERR_INVALID, "null kernel");
  if (buf && len) {
    strncpy(buf, k->name.c_str(), len - 1);
    buf[len - 1] = 0;
  }
  return (int)k->name.size();
}

static uint64_t rd_u64(const uint8_t* p) {
  uint64_t v = 0;
  for (int i = 7; i >= 0; --i) v = (v << 8) | p[i];
  return v;
}
static uint32_t rd_u32(const uint8_t* p) { return (uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 | (uint32_t)p[3] << 24; }

static int wait_stream(t0mi_ctx* ctx) {
  // AqlQueue::synchronize (aql.rs:481-545): poll completion with a timeout;
  // a timeout poisons the runtime (gpu_context.rs:352-355).
  if (ctx->null_backend) {
    if (ctx->inject_timeout) {
      ctx->inject_timeout = false;
      ctx->poisoned.store(true);
      return set_error(T0MI_ERR_TIMEOUT, "[t0mi] dispatch timed out after %u ms; runtime poisoned", ctx->timeout_ms);
    }
    return T0MI_OK;
  }
  if (int rc = refuse_if_capturing(ctx, "a synchronous wait")) return rc;
  hipEvent_t ev;
  hipError_t e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
  if (e != hipSuccess) return hip_fail(e, "hipEventCreate");
  e = hipEventRecord(ev, ctx->stream);
  if (e != hipSuccess) {
    (void)hipEventDestroy(ev);
    return hip_fail(e, "hipEventRecord");
  }
  struct timespec t0, t1;
  clock_gettime(CLOCK_MONOTONIC, &t0);
  int rc = T0MI_OK;
  for (;;) {
    e = hipEventQuery(ev);
    if (e == hipSuccess) break;
    if (e != hipErrorNotReady) {
      ctx->poisoned.store(true);
      rc = hip_fail(e, "dispatch failed; runtime poisoned");
      break;
    }
    clock_gettime(CLOCK_MONOTONIC, &t1);
    const double ms = (t1.tv_sec - t0.tv_sec) * 1e3 + (t1.tv_nsec - t0.tv_nsec) * 1e-6;
    if (ms > ctx->timeout_ms) {
      ctx->poisoned.store(true);
      rc = set_error(T0MI_ERR_TIMEOUT, "[t0mi] dispatch timed out after %u ms; runtime poisoned", ctx->timeout_ms);
      break;
    }
    // aql.rs:486 sleeps 10 us per poll; a sleep that short still costs the
    // kernel's timer slack (~50 us), so the first millisecond only yields.
    if (ms < 1.0) {
      sched_yield();
    } else {
      struct timespec sl = {0, 10000};
      nanosleep(&sl, nullptr);
    }
  }
  if (rc == T0MI_OK) (void)hipEventDestroy(ev);  // a timed-out event is leaked on purpose
  return rc;
}

static float rd_f32(const uint8_t* p) {
  const uint32_t u = rd_u32(p);
  float f;
  memcpy(&f, &u, 4);
  return f;
}

// Dispatch of a lowered TileGemm with its own kernarg layout (tile_ir.rs:4570-4637
// plus the epilogue arguments declared at :1014-1027).
static int dispatch_tile(t0mi_ctx* ctx, const t0mi_kernel* k, const uint32_t grid[3], const uint8_t* ka) {
  const t0mi_tile_spec& s = k->tile;
  const uint64_t x = rd_u64(ka + 0), wt = rd_u64(ka + 8), y = rd_u64(ka + 16);
  const uint32_t K = rd_u32(ka + 24), N = rd_u32(ka + 28), sks = rd_u32(ka + 32), yss = rd_u32(ka + 36);
  uint32_t M = rd_u32(ka + 40);
  const uint32_t sk = tile_split_k(s);
  if (sks != (sk > 1 ? (uint32_t)__builtin_ctz(sk) : 0u))
    return set_error(T0MI_ERR_INVALID, "split_k_shift %u does not match the spec's split_k %u", sks, sk);
  if (!s.persistent) {
    const uint32_t gx = grid[0] / k->wg_size, gy = grid[1] ? grid[1] : 1;
    if (gy % sk) return set_error(T0MI_ERR_INVALID, "grid_y=%u not a multiple of split_k=%u", gy, sk);
    const uint32_t tn = s.swap_grid ? gx : gy / sk, tm = s.swap_grid ? gy / sk : gx;
    // build_kernargs leaves M = 0: fall back to the grid's (padded) row count.
    if (M == 0) M = tm * s.tile_m;
    if ((uint64_t)tn * s.tile_n < N || (uint64_t)tm * s.tile_m < M)
      return set_error(T0MI_ERR_INVALID, "grid (%u x %u tiles) does not cover M=%u N=%u", tm, tn, M, N);
  } else if (M == 0) {
    return set_error(T0MI_ERR_INVALID, "persistent TileGemm dispatch needs M in the kernarg");
  }
  EpiChain chain = k->chain;
  const uint64_t bias = k->lay.bias ? rd_u64(ka + k->lay.bias) : 0;
  if (k->lay.scale) chain.scale = rd_f32(ka + k->lay.scale);
  if (k->lay.clamp_min) {
    chain.lo = rd_f32(ka + k->lay.clamp_min);
    chain.hi = rd_f32(ka + k->lay.clamp_max);
  }
  if (s.persistent)
    // tile_ir.rs:540-604, 1062-1120: one workgroup loops over every tile so that a
    // decode-sized GEMM is one dispatch; split-K is not part of a persistent run
    // (split_k_id = 0), so the whole sum lands in Y.  Here: one launch of a
    // persistent kernel whose grid is what the GPU holds at once.  The kernarg's
    // counter, n_tiles_n_shift and tiles_per_wg describe the reference's
    // one-workgroup schedule; the grid-stride schedule derives its own from M, N.
    return run_gemm_persistent(ctx, k->cfg, k->gemm, x, wt, y, bias, M, N, K, chain);
  if (sk == 1 || yss == 0)
    // One output plane: split-K partitions are summed by the library.
    return run_gemm(ctx, k->cfg, k->gemm, x, wt, y, bias, M, N, K, chain);
  // Caller-provided partial planes (gemm_gen convention): partition p writes
  // the raw f32 sum of its K range at Y + p * y_split_stride; no epilogue.
  if (K % 8 || N % 8 || (K / sk) % 8)
    return set_error(T0MI_ERR_INVALID, "K=%u and N=%u (and K/split_k) must be multiples of 8", K, N);
  if ((uint64_t)yss < (uint64_t)M * N * 4u) return set_error(T0MI_ERR_INVALID, "y_split_stride smaller than a plane");
  GemmParams p;
  memset(&p, 0, sizeof p);
  p.a = (const uint16_t*)x;
  p.b = (const uint16_t*)wt;
  p.y = (void*)y;
  p.M = M;
  p.N = N;
  p.K = K;
  p.lda = K;
  p.ldb = s.transpose == T0MI_NN ? N : K;
  p.ldy = N;
  p.tiles_m = (M + k->cfg.tile_m - 1) / k->cfg.tile_m;
  p.tiles_n = (N + k->cfg.tile_n - 1) / k->cfg.tile_n;
  p.split_k = sk;
  p.k_per_split = K / sk;
  p.y_split_stride = yss;
  p.xcd_remap = 1;
  return launch_gemm(ctx, k->cfg, k->gemm, p);
}

static int dispatch_impl(t0mi_ctx* ctx, const t0mi_kernel* k, const uint32_t grid[3], const uint8_t* ka,
                         size_t ka_len) {
  int rc = check_ctx(ctx);
  if (rc) return rc;
  T0MI_SUBMIT_GUARD(ctx);
  if (!k || !grid || (!ka && ka_len)) return set_error(T0MI_ERR_INVALID, "null argument");
  // gpu_context.rs:319-323: builder and kernel declaration must agree.
  if (ka_len != k->kernarg_size)
    return set_error(T0MI_ERR_KERNARG,
                     "[t0mi] kernarg mismatch: builder produced %zuB, kernel '%s' declares %uB", ka_len,
                     k->name.c_str(), k->kernarg_size);
  if (grid[0] % k->wg_size)
    return set_error(T0MI_ERR_INVALID, "grid_x=%u is not a multiple of wg_size=%u", grid[0], k->wg_size);
  if (ctx->null_backend) {
    memcpy(ctx->last_grid, grid, sizeof ctx->last_grid);
    ctx->last_ka.assign(ka, ka + ka_len);
  }
  if (k->kind == KK_TILE) return dispatch_tile(ctx, k, grid, ka);
  const t0mi_gemm_config& c = k->cfg;
  const uint32_t sk = split_k_of(c);
  const uint32_t gx = grid[0] / k->wg_size, gy = grid[1] ? grid[1] : 1;
  if (gy % sk) return set_error(T0MI_ERR_INVALID, "grid_y=%u not a multiple of split_k=%u", gy, sk);
  GemmParams p;
  memset(&p, 0, sizeof p);
  p.a = (const uint16_t*)rd_u64(ka + 0);
  p.b = (const uint16_t*)rd_u64(ka + 8);
  p.y = (void*)rd_u64(ka + 16);
  p.K = rd_u32(ka + 24);
  p.N = rd_u32(ka + 28);
  p.y_split_stride = rd_u32(ka + 36);
  p.bias = ka_len >= 48 ? (const float*)rd_u64(ka + 40) : nullptr;
  const uint32_t grid_tn = c.swap_grid ? gx : gy / sk;
  const uint32_t grid_tm = c.swap_grid ? gy / sk : gx;
  // gemm_gen kernargs carry no M: the grid defines it, and callers pad Y to
  // tiles_m * tile_m rows (gemm_gen.rs:299-307).
  p.M = grid_tm * c.tile_m;
  if ((uint64_t)grid_tn * c.tile_n < p.N)
    return set_error(T0MI_ERR_INVALID, "grid (%u tiles of %u columns) does not cover N=%u", grid_tn, c.tile_n, p.N);
  // The launched kernel's own tiles (a remapped reference tile, e.g. 16 rows on
  // a 32-row kernel, covers the same M x N).
  const t0mi_gemm_config& ph = k->phys;
  p.tiles_m = (p.M + ph.tile_m - 1) / ph.tile_m;
  p.tiles_n = (p.N + ph.tile_n - 1) / ph.tile_n;
  p.lda = p.K;
  p.ldb = c.transpose == T0MI_NN ? p.N : p.K;
  p.ldy = p.N;
  p.split_k = sk;
  p.k_per_split = sk > 1 ? p.K / sk : p.K;  // K >> split_k_shift (gemm_gen.rs:769-775)
  p.out_bf16 = c.out_dtype == T0MI_OUT_BF16;
  p.epi = chain_of(c.epilogue);
  p.xcd_remap = 1;
  if (p.K % 8 || p.N % 8 || p.k_per_split % 8)
    return set_error(T0MI_ERR_INVALID, "K=%u and N=%u (and K/split_k) must be multiples of 8", p.K, p.N);
  if (p.epi.n && !p.bias) return set_error(T0MI_ERR_INVALID, "bias epilogue with null bias");
  if (sk > 1 && p.y_split_stride < (uint64_t)p.M * p.N * 4u)
    return set_error(T0MI_ERR_INVALID, "y_split_stride %llu smaller than an f32 plane", (unsigned long long)p.y_split_stride);
  return launch_gemm(ctx, ph, k->gemm, p);
}

extern "C" int t0mi_dispatch_async(t0mi_ctx* ctx, const t0mi_kernel* k, const uint32_t grid[3], const uint8_t* ka,
                                   size_t ka_len) {
  return dispatch_impl(ctx, k, grid, ka, ka_len);
}

extern "C" int t0mi_dispatch(t0mi_ctx* ctx, const t0mi_kernel* k, const uint32_t grid[3], const uint8_t* ka,
                             size_t ka_len) {
  // A synchronous dispatch cannot be recorded: refuse before launching.
  int rc = ctx ? refuse_if_capturing(ctx, "t0mi_dispatch (synchronous)") : T0MI_OK;
  if (rc) return rc;
  rc = dispatch_impl(ctx, k, grid, ka, ka_len);
  if (rc) return rc;
  return wait_stream(ctx);
}

extern "C" int t0mi_wait_idle(t0mi_ctx* ctx) {
  if (!ctx) return set_error(T0MI_ERR_INVALID, "null runtime");
  if (ctx->poisoned.load()) return set_error(T0MI_ERR_POISONED, "[t0mi] runtime poisoned");
  return wait_stream(ctx);
}

// ---------------------------------------------------------- one-call GEMM ----

namespace t0mi {
int run_gemm(t0mi_ctx* ctx, const t0mi_gemm_config& cfg, const GemmLaunchEntry* e, uint64_t x, uint64_t b,
             uint64_t y, uint64_t bias, uint32_t m, uint32_t n, uint32_t k, const EpiChain& epi,
             const FixedWorkspace* fixed, uint32_t ldn) {
  if (m == 0 || n == 0) return T0MI_OK;
  const uint32_t ld = ldn ? ldn : n;
  if (ld < n || ld % 8) return set_error(T0MI_ERR_INVALID, "row length %u for N=%u", ld, n);
  if (k % 8) return set_error(T0MI_ERR_INVALID, "K=%u must be a multiple of 8", k);
  if (n % 8) return set_error(T0MI_ERR_INVALID, "N=%u must be a multiple of 8", n);
  if ((x | b | y) & 15) return set_error(T0MI_ERR_INVALID, "X, B and Y must be 16-byte aligned");
  if (chain_uses(epi, EOP_BIAS) && !bias) return set_error(T0MI_ERR_INVALID, "bias epilogue with null bias");
  if (bias & 3) return set_error(T0MI_ERR_INVALID, "bias must be 4-byte aligned");
  const uint32_t sk = split_k_of(cfg);
  GemmParams p;
  memset(&p, 0, sizeof p);
  p.a = (const uint16_t*)x;
  p.b = (const uint16_t*)b;
  p.bias = (const float*)bias;
  p.M = m;
  p.N = n;
  p.K = k;
  p.lda = k;
  p.ldb = cfg.transpose == T0MI_NN ? ld : k;
  p.ldy = ld;
  p.tiles_m = (m + cfg.tile_m - 1) / cfg.tile_m;
  p.tiles_n = (n + cfg.tile_n - 1) / cfg.tile_n;
  p.split_k = sk;
  p.epi = epi;
  p.out_bf16 = cfg.out_dtype == T0MI_OUT_BF16;
  p.xcd_remap = 1;
  const size_t plane = (size_t)m * n * 4;
  // The f32 workspace this call needs: none, one zero plane (K = 0) or one
  // plane per K partition.  A fixed workspace is checked before any launch.
  const size_t ws_need = k == 0 ? plane : sk > 1 ? plane * sk : 0;
  if (fixed && ws_need > fixed->cap)
    return set_error(T0MI_ERR_INVALID,
                     "%ux%u with split_k=%u needs %zu bytes of scratch; the fixed workspace holds %zu", m, n,
                     k == 0 ? 1u : sk, ws_need, fixed->cap);
  void* ws = nullptr;
  if (ws_need) {
    if (fixed) {
      ws = fixed->ptr;
    } else {
      int rc = ensure_workspace(ctx, ws_need);
      if (rc) return rc;
      ws = ctx->ws;
    }
  }
  int rc;
  if (k == 0) {
    // Empty contraction: the sum is zero (plus epilogue).
    if (ctx->null_backend) return T0MI_OK;
    rc = fill_async(ctx, ws, 0, plane);
    if (rc) return rc;
    return launch_splitk_reduce(ctx, (const float*)ws, (void*)y, (const float*)bias, m, n, ld, 1u, p.out_bf16, epi);
  }
  if (sk == 1) {
    p.k_per_split = k;
    p.y = (void*)y;
    return launch_gemm(ctx, cfg, e, p);
  }
  // Split-K: partitions of whole K tiles write f32 planes into the workspace,
  // then a reduce pass sums them in partition order.
  const uint32_t kt = (k + cfg.tile_k - 1) / cfg.tile_k;
  p.k_per_split = ((kt + sk - 1) / sk) * cfg.tile_k;
  p.y = ws;
  p.ldy = n;
  p.y_split_stride = plane;
  rc = launch_gemm(ctx, cfg, e, p);
  if (rc || ctx->null_backend) return rc;
  return launch_splitk_reduce(ctx, (const float*)ws, (void*)y, (const float*)bias, m, n, ld, sk, p.out_bf16, epi);
}
}  // namespace t0mi

extern "C" int t0mi_gemm(t0mi_ctx* ctx, const t0mi_gemm_config* cfg, uint64_t x, uint64_t b, uint64_t y,
                         uint64_t bias, uint32_t m, uint32_t n, uint32_t k) {
  int rc = check_ctx(ctx);
  if (rc) return rc;
  T0MI_SUBMIT_GUARD(ctx);
  if (!cfg) return set_error(T0MI_ERR_INVALID, "null config");
  std::string why;
  t0mi_gemm_config phys;
  if (!config_physical(*cfg, &phys, &why))
    return set_error(T0MI_ERR_INVALID, "[t0mi] config '%s' infeasible on gfx950: %s", config_name(*cfg).c_str(),
                     why.c_str());
  const GemmLaunchEntry* e = find_gemm_launch(phys);
  if (!e) return set_error(T0MI_ERR_NO_KERNEL, "[t0mi] no prebuilt gfx950 kernel for '%s'", config_name(*cfg).c_str());
  return run_gemm(ctx, phys, e, x, b, y, bias, m, n, k, chain_of(cfg->epilogue));
}

extern "C" int t0mi_gemm_noalloc(t0mi_ctx* ctx, const t0mi_gemm_config* cfg, uint64_t x, uint64_t b, uint64_t y,
                                 uint64_t bias, uint32_t m, uint32_t n, uint32_t k) {
  int rc = check_ctx(ctx);
  if (rc) return rc;
  T0MI_SUBMIT_GUARD(ctx);
  if (!cfg) return set_error(T0MI_ERR_INVALID, "null config");
  if (!ctx->null_backend && ctx->scratch_rc)
    return set_error(ctx->scratch_rc, "t0mi_gemm_noalloc: the library scratch of device %d is unavailable",
                     ctx->device);
  std::string why;
  t0mi_gemm_config phys;
  if (!config_physical(*cfg, &phys, &why))
    return set_error(T0MI_ERR_INVALID, "[t0mi] config '%s' infeasible on gfx950: %s", config_name(*cfg).c_str(),
                     why.c_str());
  const GemmLaunchEntry* e = find_gemm_launch(phys);
  if (!e) return set_error(T0MI_ERR_NO_KERNEL, "[t0mi] no prebuilt gfx950 kernel for '%s'", config_name(*cfg).c_str());
  const FixedWorkspace fixed{ctx->scratch, (size_t)T0MI_NOALLOC_SCRATCH_BYTES};
  ScratchUse* u = ctx->null_backend ? nullptr : scratch_use_for_device(ctx->device, false);
  if (!u || !u->done) return run_gemm(ctx, phys, e, x, b, y, bias, m, n, k, chain_of(cfg->epilogue), &fixed);
  std::lock_guard<std::mutex> lk(u->mu);
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  (void)hipStreamIsCapturing(ctx->stream, &cap);
  const bool capturing = cap != hipStreamCaptureStatusNone;  // captured calls are not tracked
  if (!capturing && u->recorded && u->last != ctx->stream) {
    const hipError_t q = hipEventQuery(u->done);
    if (q == hipErrorNotReady)
      return set_error(T0MI_ERR_INVALID,
                       "t0mi_gemm_noalloc: device %d's scratch is still in use by a call on another stream; calls "
                       "that overlap on one GPU would race (wait for that stream first)",
                       ctx->device);
  }
  rc = run_gemm(ctx, phys, e, x, b, y, bias, m, n, k, chain_of(cfg->epilogue), &fixed);
  if (rc == T0MI_OK && !capturing && hipEventRecord(u->done, ctx->stream) == hipSuccess) {
    u->last = ctx->stream;
    u->recorded = true;
  }
  return rc;
}

bool t0mi::auto_plan(uint32_t m, uint32_t n, uint32_t k, uint32_t transpose, uint32_t out_dtype, uint32_t cus,
                     AutoPlan* pl) {
  for (const t0mi_gemm_config& c : rank_candidates(m, n, k, transpose, out_dtype, nullptr)) {
    const GemmLaunchEntry* e = find_gemm_launch(c);
    if (!e) continue;
    pl->head = c;
    pl->e_head = e;
    pl->n1 = n;
    uint32_t n1 = 0;
    t0mi_gemm_config tail;
    if (plan_column_split(c, m, n, k, transpose, out_dtype, &n1, &tail, cus)) {
      const GemmLaunchEntry* et = find_gemm_launch(tail);
      if (et) {
        pl->tail = tail;
        pl->e_tail = et;
        pl->n1 = n1;
      }
    }
    return true;
  }
  return false;
}

namespace {
// auto_plan results by shape (the ranking walks every prebuilt variant and
// split: microseconds of host time per call otherwise).  Process-wide, like
// cached_auto_select's cache; cleared when it grows past kPlanCacheMax.
struct PlanKey {
  uint32_t m, n, k, transpose, out_dtype, cus;
  bool operator<(const PlanKey& o) const {
    return std::tie(m, n, k, transpose, out_dtype, cus) < std::tie(o.m, o.n, o.k, o.transpose, o.out_dtype, o.cus);
  }
};
constexpr size_t kPlanCacheMax = 4096;
std::mutex g_plan_mu;
std::map<PlanKey, AutoPlan> g_plans;
bool cached_auto_plan(uint32_t m, uint32_t n, uint32_t k, uint32_t transpose, uint32_t out_dtype, uint32_t cus,
                      AutoPlan* pl) {
  const PlanKey key{m, n, k, transpose, out_dtype, cus};
  {
    std::lock_guard<std::mutex> lk(g_plan_mu);
    auto it = g_plans.find(key);
    if (it != g_plans.end()) {
      *pl = it->second;
      return true;
    }
  }
  if (!t0mi::auto_plan(m, n, k, transpose, out_dtype, cus, pl)) return false;
  std::lock_guard<std::mutex> lk(g_plan_mu);
  if (g_plans.size() >= kPlanCacheMax) g_plans.clear();
  g_plans[key] = *pl;
  return true;
}
}  // namespace

int t0mi::run_gemm_auto(t0mi_ctx* ctx, uint32_t transpose, uint64_t x, uint64_t b, uint64_t y, uint32_t m, uint32_t n,
                        uint32_t k, uint32_t out_dtype, uint64_t bias, const EpiChain* epi) {
  if (transpose == T0MI_NT) {
    const int rc = run_gemm_decode_nt(ctx, x, b, y, m, n, k, out_dtype, bias, epi ? *epi : EpiChain{});
    if (rc <= 0) return rc;
  }
  AutoPlan pl;
  if (!cached_auto_plan(m, n, k, transpose, out_dtype, (uint32_t)ctx->cu_count, &pl))
    return set_error(T0MI_ERR_NO_KERNEL, "[t0mi] no prebuilt gfx950 kernel for %ux%ux%u (%s)", m, n, k,
                     transpose == T0MI_NN ? "NN" : "NT");
  return run_gemm_planned(ctx, pl, transpose, x, b, y, m, n, k, out_dtype, bias, epi);
}

int t0mi::run_gemm_planned(t0mi_ctx* ctx, const AutoPlan& pl, uint32_t transpose, uint64_t x, uint64_t b, uint64_t y,
                           uint32_t m, uint32_t n, uint32_t k, uint32_t out_dtype, uint64_t bias,
                           const EpiChain* epi) {
  const EpiChain chain = epi ? *epi : EpiChain{};
  if (pl.n1 == n) return run_gemm(ctx, pl.head, pl.e_head, x, b, y, bias, m, n, k, chain);
  // Columns [0, n1) on the head config, [n1, n) on the tail's; B, Y and bias
  // advance to column n1 (NN's B and Y keep their row length n; NT's B rows
  // are columns).
  const uint32_t n1 = pl.n1;
  const uint64_t ob = out_dtype == T0MI_OUT_BF16 ? 2 : 4;
  int rc = run_gemm(ctx, pl.head, pl.e_head, x, b, y, bias, m, n1, k, chain, nullptr, n);
  if (rc) return rc;
  const uint64_t b_tail = b + (transpose == T0MI_NN ? (uint64_t)n1 * 2 : (uint64_t)n1 * k * 2);
  return run_gemm(ctx, pl.tail, pl.e_tail, x, b_tail, y + (uint64_t)n1 * ob, bias ? bias + (uint64_t)n1 * 4 : 0, m,
                  n - n1, k, chain, nullptr, n);
}

extern "C" int t0mi_auto_gemm_plan(uint32_t m, uint32_t n, uint32_t k, uint32_t transpose, uint32_t out_dtype,
                                   t0mi_gemm_config* head, uint32_t* n_main, t0mi_gemm_config* tail) {
  if (!head || !n_main || !tail) return set_error(T0MI_ERR_INVALID, "null output");
  if (!m || !n || !k) return set_error(T0MI_ERR_INVALID, "zero dimension");
  if (transpose > T0MI_NN || out_dtype > T0MI_OUT_BF16) return set_error(T0MI_ERR_INVALID, "bad layout or out_dtype");
  AutoPlan pl;
  if (!auto_plan(m, n, k, transpose, out_dtype, 256, &pl))
    return set_error(T0MI_ERR_NO_KERNEL, "[t0mi] no prebuilt gfx950 kernel for %ux%ux%u", m, n, k);
  *head = pl.head;
  *n_main = pl.n1;
  *tail = pl.n1 < n ? pl.tail : pl.head;
  return T0MI_OK;
}

// ------------------------------------------------------------ tile_ir GEMM ----

extern "C" int t0mi_tile_kernel_get(t0mi_ctx* ctx, const t0mi_tile_spec* s, t0mi_kernel** out) {
  if (!ctx || !s || !out) return set_error(T0MI_ERR_INVALID, "null argument");
  EpiChain chain;
  std::string why;
  if (!tile_valid(*s, &chain, &why))
    return set_error(T0MI_ERR_INVALID, "[t0mi] TileGemm '%s' invalid: %s", tile_name(*s).c_str(), why.c_str());
  t0mi_gemm_config cfg;
  if (!tile_lower(*s, &cfg, &why))
    return set_error(T0MI_ERR_NO_KERNEL, "[t0mi] TileGemm '%s': %s", tile_name(*s).c_str(), why.c_str());
  const GemmLaunchEntry* e = find_gemm_launch(cfg);
  if (!e) return set_error(T0MI_ERR_NO_KERNEL, "[t0mi] no prebuilt gfx950 kernel for '%s'", tile_name(*s).c_str());
  const std::string name = tile_name(*s);
  std::lock_guard<std::mutex> lk(ctx->mu);
  auto it = ctx->kernels.find(name);
  if (it != ctx->kernels.end()) {
    *out = it->second.get();
    return T0MI_OK;
  }
  std::unique_ptr<t0mi_kernel> k(new t0mi_kernel());
  k->kind = KK_TILE;
  k->cfg = cfg;
  k->phys = cfg;
  k->tile = *s;
  k->lay = tile_arg_layout(*s);
  k->chain = chain;
  k->name = name;
  k->kernarg_size = k->lay.size;
  k->lds_size = t0mi_tile_lds_total(s);
  k->wg_size = tile_wg_size(*s);
  k->gemm = e;
  *out = k.get();
  ctx->kernels[name] = std::move(k);
  return T0MI_OK;
}

extern "C" int t0mi_tile_gemm(t0mi_ctx* ctx, const t0mi_tile_spec* s, uint64_t x, uint64_t wt, uint64_t y,
                              uint32_t m, uint32_t n, uint32_t k, uint64_t bias, float scale, float clamp_min,
                              float clamp_max) {
  int rc = check_ctx(ctx);
  if (rc) return rc;
  T0MI_SUBMIT_GUARD(ctx);
  if (!s) return set_error(T0MI_ERR_INVALID, "null spec");
  EpiChain chain;
  std::string why;
  if (!tile_valid(*s, &chain, &why))
    return set_error(T0MI_ERR_INVALID, "[t0mi] TileGemm '%s' invalid: %s", tile_name(*s).c_str(), why.c_str());
  t0mi_gemm_config cfg;
  if (!tile_lower(*s, &cfg, &why))
    return set_error(T0MI_ERR_NO_KERNEL, "[t0mi] TileGemm '%s': %s", tile_name(*s).c_str(), why.c_str());
  const GemmLaunchEntry* e = find_gemm_launch(cfg);
  if (!e) return set_error(T0MI_ERR_NO_KERNEL, "[t0mi] no prebuilt gfx950 kernel for '%s'", tile_name(*s).c_str());
  chain.scale = scale;
  chain.lo = clamp_min;
  chain.hi = clamp_max;
  if (s->persistent) return run_gemm_persistent(ctx, cfg, e, x, wt, y, bias, m, n, k, chain);
  return run_gemm(ctx, cfg, e, x, wt, y, bias, m, n, k, chain);
}
