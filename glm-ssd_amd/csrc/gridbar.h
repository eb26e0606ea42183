// Grid-wide barrier of the fused routed-expert FFN kernels (one per launch, every workgroup
// co-resident), correct under the HIP/HSA memory model:
//   * arrival is a release at agent scope (a fence, then the counter increment), so every global
//     store the workgroup made before the barrier (after its own workgroup barrier) happens-before
//     the arrival;
//   * the last arrival publishes a new generation with a release; the waiter's loop ends with an
//     acquire fence at agent scope, then a workgroup barrier, so every wave's later loads see all
//     the arrivals' stores on any XCD (the fences emit the L2 write-back / invalidate they need).
// Counters are per slot, and the host gives each launch a slot of its own (a rotation over
// GS_BAR_SLOTS per device), so launches that overlap on one device never share counters. Within a
// slot the barrier resets itself (the last arrival of a group clears the group counter before the
// generation moves on), so it works for any grid size and for replays of a captured launch.
// Arrivals are spread over up to 8 group counters (blockIdx % 8) on separate 128-byte lines, so
// 256 workgroups' atomics do not all queue on one address.
// The wait is bounded in time (ticks of the 100 MHz s_memrealtime clock): on expiry the kernel
// sets a flag the host reads (gs_moe_ffn_status) and runs on with undefined results instead of
// hanging the device.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define GS_BAR_SLOTS 64
#define GS_BAR_GROUPS 8u

struct __attribute__((aligned(128))) BarLine {
    unsigned v;
    unsigned pad[31];
};
struct BarSlot {
    BarLine group[GS_BAR_GROUPS];   // arrivals per workgroup group (reset by the group's last)
    BarLine top;                    // completed groups (reset by the last group)
    BarLine gen;                    // generation: advanced once per completed barrier
};
__device__ BarSlot gs_bar[GS_BAR_SLOTS];
__device__ unsigned gs_ffn_timeout;   // set when a barrier wait expired (results undefined)

// Generation of the slot, read by thread 0 at kernel start (before this workgroup can arrive,
// hence before the generation this launch waits for can be published).
__device__ __forceinline__ unsigned bar_generation(int slot) {
    return __hip_atomic_load(&gs_bar[slot].gen.v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Arrival of this workgroup (thread 0, after a workgroup barrier).
__device__ __forceinline__ void bar_arrive(int slot) {
    BarSlot &b = gs_bar[slot];
    const unsigned nblk = gridDim.x;
    const unsigned ng = nblk < GS_BAR_GROUPS ? nblk : GS_BAR_GROUPS;
    const unsigned g = blockIdx.x % ng;
    const unsigned size_g = (nblk - g + ng - 1) / ng;   // workgroups in group g
    const unsigned old = __hip_atomic_fetch_add(&b.group[g].v, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    if (old + 1 != size_g) return;
    __hip_atomic_store(&b.group[g].v, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const unsigned done = __hip_atomic_fetch_add(&b.top.v, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    if (done + 1 != ng) return;
    __hip_atomic_store(&b.top.v, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_fetch_add(&b.gen.v, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
}

// Wait (thread 0) until the slot's generation moves past gen0; bounded in time. Ends with an
// acquire at agent scope.
__device__ __forceinline__ void bar_wait(int slot, unsigned gen0, uint64_t ticks) {
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    while (__hip_atomic_load(&gs_bar[slot].gen.v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gen0) {
        if (__builtin_amdgcn_s_memrealtime() - t0 > ticks) {
            __hip_atomic_store(&gs_ffn_timeout, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            break;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
}

// Release of this workgroup's global stores before its arrival (thread 0, after a workgroup
// barrier that ordered the other waves' stores before it).
__device__ __forceinline__ void bar_release() { __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent"); }
