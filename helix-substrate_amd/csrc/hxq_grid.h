// Grid-wide barrier for persistent kernels (every block of the grid resident,
// guaranteed by a cooperative launch).
//
// State in device memory: an arrival counter and a generation number.  Block
// thread 0 reads the generation, adds itself to the counter; the last block to
// arrive resets the counter and bumps the generation; the others wait for the
// generation to change.  The counter is back at 0 after every barrier, so the
// state carries over from one launch to the next without host resets.
//
// Every wait is bounded: a block that waits longer than `timeout_ticks` of the
// 100 MHz wall clock, or that sees the error word set, sets the error word and
// reports failure; the caller then leaves the kernel, so every wave of the
// grid ends even if the barrier cannot complete.
//
// Memory ordering: every thread releases its global writes at agent scope
// before the block joins, and acquires at agent scope after it leaves, so data
// written by any block before the barrier is visible to every block after it
// (the per-XCD L2 caches are written back / invalidated by those fences).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hxq {

struct GridBarrier {
    uint32_t count;
    uint32_t gen;
    int32_t err;      // nonzero: a wait timed out (or another block gave up)
    int32_t pad_;
};

// Thread 0 of the block arrives and waits; returns 1 (passed) or 0 (gave up).
__device__ __forceinline__ int grid_arrive_wait(GridBarrier *gb, uint32_t nblocks,
                                                uint64_t timeout_ticks) {
    const uint32_t g = __hip_atomic_load(&gb->gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t old =
        __hip_atomic_fetch_add(&gb->count, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    if (old == nblocks - 1) {
        __hip_atomic_store(&gb->count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_fetch_add(&gb->gen, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        return 1;
    }
    const uint64_t t0 = wall_clock64();
    while (__hip_atomic_load(&gb->gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == g) {
        if (__hip_atomic_load(&gb->err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0 ||
            wall_clock64() - t0 > timeout_ticks) {
            __hip_atomic_store(&gb->err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return 0;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    return 1;
}

// Whole-block grid barrier; `flag` is a __shared__ int of the caller.  Returns
// false when the barrier gave up (the caller must return from the kernel).
__device__ __forceinline__ bool grid_sync(GridBarrier *gb, int *flag, uint64_t timeout_ticks) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    __syncthreads();
    if (threadIdx.x == 0) *flag = grid_arrive_wait(gb, gridDim.x, timeout_ticks);
    __syncthreads();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    return *flag != 0;
}

}  // namespace hxq
