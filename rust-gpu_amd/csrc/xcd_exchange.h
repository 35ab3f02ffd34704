// xcd_exchange.h — split-K partial sums combined inside one launch, normally
// within one XCD.
//
// MI355X has 8 XCDs, each with its own L2; workgroup i of a launch usually runs
// on XCD i % nx (nx = 8 on a whole MI355X; checked per runtime by t0mi's
// placement probe, and per workgroup by the kernels: a mismatch sets a flag the
// host can read).  A kernel that splits an output tile's K range over P
// workgroups numbers them so that all P land on the tile's XCD:
//     id = ((tile / nx) * P + piece) * nx + tile % nx.
// Each piece stores its fp32 partial into its own slot, waits for the stores to
// be acknowledged, and takes a ticket on the tile's counter.  The piece that
// draws ticket P - 1 is the last: it reads the other pieces' slots, sums all P
// in piece order -- so the result does not depend on which piece arrived last
// -- stores the output, and puts the counter back to 0 for the next launch.
// Nobody waits for anybody: a launch ends however its workgroups are scheduled.
//
// The slots are written and read with the device-scope cache policy (sc1: what
// the compiler emits for device-scope atomic stores and loads, coherent across
// XCDs; the stores are written through to memory), so the exchange is correct
// wherever the pieces run.  The numbering only makes one XCD the usual case
// (the reader then finds the lines in its own L2): the placement has been seen
// to differ (a workgroup on another XCD than i % nx), which the kernels flag
// for the host.
//
// Counters live in a per-runtime array that starts zeroed; they are
// device-scope atomics (coherent across XCDs), grouped by the tile's XCD (`tpx`
// per XCD), and every counter has a 256-byte slot of its own: the pieces of all
// tiles arrive at about the same time, and atomics on one line are serialized.
// Launches that overlap on one runtime would share counters and slots: the
// runtime orders its launches on one stream.
#pragma once
#include <stdint.h>

#include "index_maps.h"

namespace t0mi {

struct XcdExchange {
  float* part;      // partial slots
  uint32_t* tick;   // counters, nx groups of tpx, `stride` u32s apart
  uint32_t* flag;   // set to 1 by a workgroup found on another XCD than planned
  uint32_t nx;      // XCDs
  uint32_t tpx;     // counters per XCD
  uint32_t stride;  // u32s between counters (64: 256 bytes)
};

// XCC_ID hardware register (gfx940+): the XCD this wave runs on.
__device__ __forceinline__ uint32_t xcc_id() {
  uint32_t x;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID, 0, 4)" : "=s"(x));
  return x;
}

// xk_unpack, the workgroup numbering above inverted: index_maps.h.

// Counter of `tile`.
__device__ __forceinline__ uint32_t* xk_counter(const XcdExchange& x, uint32_t tile) {
  return x.tick + ((size_t)(tile % x.nx) * x.tpx + tile / x.nx) * x.stride;
}

// Flags a workgroup that is not on the XCD the numbering assumes: diagnostic
// only, results do not depend on it.
__device__ __forceinline__ void xk_check_placement(const XcdExchange& x) {
  if (threadIdx.x == 0 && xcc_id() != blockIdx.x % x.nx) atomicOr(x.flag, 1u);
}

// Slot access: buffer operations on a slot region (record count = its bytes)
// with the device-scope cache policy (sc1): stores written through to memory,
// loads that see what other XCDs wrote through.
typedef float xk_f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t xk_u32x4 __attribute__((ext_vector_type(4)));
constexpr int kXkCachePolicy = 16;  // sc1
__device__ __forceinline__ __amdgpu_buffer_rsrc_t xk_slots(const float* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ void xk_store(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, xk_f32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(xk_u32x4, v), r, (int)byte_off, 0, kXkCachePolicy);
}
__device__ __forceinline__ xk_f32x4 xk_load(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_bit_cast(xk_f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)byte_off, 0, kXkCachePolicy));
}

// After every thread of the workgroup has stored its share of the partial:
// waits for the stores, takes the tile's ticket (thread 0) and returns true in
// every thread of the last piece.  Contains two workgroup barriers: call it
// from all threads.
__device__ __forceinline__ bool xk_arrive(const XcdExchange& x, uint32_t tile, uint32_t pieces) {
  __shared__ uint32_t ticket;
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0);  // this thread's partial stores have reached memory
  __syncthreads();
  if (threadIdx.x == 0) ticket = __hip_atomic_fetch_add(xk_counter(x, tile), 1u, __ATOMIC_RELAXED,
                                                        __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  return ticket == pieces - 1;
}

// The last piece's reset of the tile's counter (after it has read the slots).
__device__ __forceinline__ void xk_reset(const XcdExchange& x, uint32_t tile) {
  if (threadIdx.x == 0) __hip_atomic_store(xk_counter(x, tile), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace t0mi
