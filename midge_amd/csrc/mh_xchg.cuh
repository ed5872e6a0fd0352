// mh_xchg.cuh — words that the blocks of one launch exchange while it runs
// (the one-launch decode step and attention): a 64-bit device-scope store
// carries the producer's sequence number next to a 32-bit value, so that a
// consumer polls the data itself; device-scope loads and stores are coherent
// across the XCDs' L2 caches. Every wait on such a word is bounded.
#pragma once

#include "mh_internal.h"

namespace mh {
namespace {

constexpr unsigned kSpinLimit = 1u << 20;   // polls before a wait gives up (~1 s)

__device__ __forceinline__ void raise_err(unsigned *err) {
    __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Tagged words: (tag << 32) | payload in one device-scope 64-bit store.
__device__ __forceinline__ void st_tag_u(uint64_t *p, unsigned tag, uint32_t v) {
    __hip_atomic_store(p, ((uint64_t)tag << 32) | v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_tag(uint64_t *p, unsigned tag, float v) { st_tag_u(p, tag, __float_as_uint(v)); }
__device__ __forceinline__ uint64_t ld_tag(const uint64_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool tag_is(uint64_t w, unsigned tag) { return (unsigned)(w >> 32) == tag; }
__device__ __forceinline__ float tag_val(uint64_t w) { return __uint_as_float((uint32_t)w); }

// An opaque copy of v: values derived from it are recomputed where they are
// used instead of being hoisted out of a loop and held in registers.
__device__ __forceinline__ int opaque(int v) {
    asm volatile("" : "+v"(v));
    return v;
}

}  // namespace
}  // namespace mh
