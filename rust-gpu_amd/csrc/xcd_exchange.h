// xcd_exchange.h — split-K partial sums combined inside one launch, through one
// XCD's L2.
//
// MI355X has 8 XCDs, each with its own L2; workgroup i of a launch runs on XCD
// i % nx (nx = 8 on a whole MI355X; checked per runtime by t0mi's placement
// probe, and per workgroup by the kernels: a mismatch sets a flag the host can
// read).  A kernel that splits an output tile's K range over P workgroups
// numbers them so that all P land on the tile's XCD:
//     id = ((tile / nx) * P + piece) * nx + tile % nx.
// Each piece stores its fp32 partial into its own slot (plain stores: written
// through the CU's L1 into the XCD's L2), waits for the stores to be
// acknowledged, and takes a ticket on the tile's counter.  The piece that draws
// ticket P - 1 is the last: it reads the other pieces' slots (L2 hits; no CU
// read those lines earlier in the launch, and L1 is invalidated at launch),
// sums all P in piece order -- so the result does not depend on which piece
// arrived last -- stores the output, and puts the counter back to 0 for the
// next launch.  Nobody waits for anybody: a launch ends however its
// workgroups are scheduled.
//
// Counters live in a per-runtime array that starts zeroed; a tile's counter is
// touched only by its XCD (counters are grouped by XCD, `tpx` per XCD), and
// every counter has a 256-byte slot of its own: the pieces of all tiles arrive
// at about the same time, and atomics on one line are serialized.  Launches that overlap on one runtime
// would share counters and slots: the runtime orders its launches on one stream.
#pragma once
#include <stdint.h>

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

// The workgroup numbering above, inverted: (tile, piece) of workgroup `id`.
__device__ __forceinline__ void xk_unpack(uint32_t id, uint32_t nx, uint32_t pieces, uint32_t* tile,
                                          uint32_t* piece) {
  const uint32_t xs = id % nx, r = id / nx;
  *piece = r % pieces;
  *tile = (r / pieces) * nx + xs;
}

// Counter of `tile`.
__device__ __forceinline__ uint32_t* xk_counter(const XcdExchange& x, uint32_t tile) {
  return x.tick + ((size_t)(tile % x.nx) * x.tpx + tile / x.nx) * x.stride;
}

// Flags a workgroup that is not on the XCD the numbering assumes.
__device__ __forceinline__ void xk_check_placement(const XcdExchange& x) {
  if (threadIdx.x == 0 && xcc_id() != blockIdx.x % x.nx) atomicOr(x.flag, 1u);
}

// After every thread of the workgroup has stored its share of the partial:
// waits for the stores, takes the tile's ticket (thread 0) and returns true in
// every thread of the last piece.  Contains two workgroup barriers: call it
// from all threads.
__device__ __forceinline__ bool xk_arrive(const XcdExchange& x, uint32_t tile, uint32_t pieces) {
  __shared__ uint32_t ticket;
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0);  // this thread's partial stores are in L2
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
