// moa_sync.h -- cross-workgroup hand-off primitives shared by the single-launch kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "moa_internal.h"

namespace moa {

// Cross-workgroup hand-off for the grid-wide epilogues.
//
// Workgroups publish() their results and then arrive on device-scope counters; the workgroup
// that arrives last reads every result with collect(). Results are agent-scope atomic
// stores/loads (global_store/load sc1 on gfx950: coherent across the XCDs' L2s without cache
// maintenance). Each wave waits for its own stores to complete (s_waitcnt vmcnt(0)) before its
// workgroup arrives, so a value is visible once the counters have counted its workgroup. No L2
// writeback/invalidate is issued (a fence per wave costs more than these kernels' weight
// stream), and each workgroup arrives once, on counters that never share a 256-byte line:
// device-scope atomics to one line serialise. Counters reset themselves, so consecutive launches
// on one stream reuse them.
__device__ __forceinline__ void publish(uint16_t* p, uint32_t v) {
    __hip_atomic_store(p, (uint16_t)v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint32_t collect(const uint16_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Eight published bf16 values (16 bytes) read coherently.
__device__ __forceinline__ uint4 collect16(const uint16_t* p) {
    const uint32_t* q = reinterpret_cast<const uint32_t*>(p);
    return make_uint4(__hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT),
                      __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT),
                      __hip_atomic_load(q + 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT),
                      __hip_atomic_load(q + 3, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}

__device__ __forceinline__ uint32_t counter_add(uint32_t* c) {
    return __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Launch epochs of the single-launch kernels. An epoch counter is a 64-bit word that each of a
// fixed number `per` (a power of two) of the launch's workgroups advances by one at entry, and
// the value a workgroup reads, divided by `per`, is the number of earlier launches. Because
// every launch adds exactly `per`, all workgroups of one launch read values in the same block
// of `per`, and 64 bits never wrap. The launch's tag is that count modulo 2^32 - 1, plus one:
// 1 .. 2^32 - 1, never 0 (the value of a zero-filled slot), and consecutive launches always
// differ. A tagged word is rewritten by every launch that reads it, so a word left by an
// earlier launch never carries the current tag (a word skipped by 2^32 - 2 launches in a row
// could: the FFN's post-norm words when no post-norm is asked for that many times).
__device__ __forceinline__ uint64_t epoch_add(uint32_t* c) {
    return __hip_atomic_fetch_add(reinterpret_cast<uint64_t*>(c), 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <int per>
__host__ __device__ __forceinline__ uint32_t epoch_tag(uint64_t old) {
    static_assert(per > 0 && (per & (per - 1)) == 0, "a power of two of workgroups per epoch counter");
    return (uint32_t)((old / per) % 0xffffffffull) + 1u;
}
__device__ __forceinline__ void counter_reset(uint32_t* c) {
    __hip_atomic_store(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Tagged hand-off (single-launch kernels). A 64-bit word carries a value in its low half and the
// launch's tag in its high half, written by one agent-scope store: a reader that sees the tag has
// the whole value, so no counter has to follow the data. Tags come from monotonic counters (a
// launch's epoch), so words left by an earlier launch never carry the current tag.
constexpr uint64_t kSpinTicks = 1ull << 24;  // bound of every poll: ~168 ms of the 100 MHz wall clock

typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) void glb_void;

__device__ __forceinline__ void publish32(void* p, uint32_t v) {
    __hip_atomic_store(reinterpret_cast<uint32_t*>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void publish64(uint64_t* p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t collect64(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t tagged(uint32_t tag, uint32_t v) { return ((uint64_t)tag << 32) | v; }

}  // namespace moa
