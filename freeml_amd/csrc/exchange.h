// Exchange words between the workgroups (WGs) of one resident launch, device code.
//
// A word is 64 bits: {payload bits, epoch}.  The producer stores it in one instruction; a
// consumer loads it until the epoch is the one it waits for, so a hand-off needs no barrier and
// no separate flag.  Two scopes, chosen by where producer and consumer run:
//
//  * device scope: agent-scope relaxed atomics.  On MI355X each XCD (accelerator complex die,
//    32 CUs) has its own L2 and the L2s are not coherent with each other, so these loads and
//    stores bypass the L2 (sc1) and meet in the memory-side cache.  Correct between any WGs;
//    every decode kernel exchanges at this scope.
//  * the "XCD scope" below (buffer loads and stores with sc0 only) is NOT a working hand-off:
//    measured on MI355X (the exchange probe, scopes 1-5), a consumer polling with sc0 never saw
//    a producer's word, even between two WGs on the same XCD (every bounded wait gave up).
//    The one XCD-local form that was observed to
//    work, a plain store polled with an sc1 load (the L2 returns its dirty line), is no faster
//    than device scope (~1.1 vs ~1.0 us per hop) and is not a scope the memory model defines.
//    xcd_buf / xcd_load / xcd_store exist for the probe's measurements only.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace fmlh {
namespace xchg {

typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

// Index of the XCD the calling wave runs on (hardware register XCC_ID, bits 3:0).
__device__ __forceinline__ int xcc_id() {
    unsigned v;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
    return static_cast<int>(v & 0xf);
}

__device__ __forceinline__ uint64_t pack(uint32_t bits, uint32_t epoch) {
    return (static_cast<uint64_t>(epoch) << 32) | bits;
}
__device__ __forceinline__ bool current(uint64_t v, uint32_t epoch) { return static_cast<uint32_t>(v >> 32) == epoch; }
__device__ __forceinline__ float payload(uint64_t v) { return __uint_as_float(static_cast<uint32_t>(v)); }

// ---- device scope ----------------------------------------------------------------------------

__device__ __forceinline__ uint64_t dev_load(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void dev_store(uint64_t* p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---- "XCD scope" (probe only: not coherent between CUs, see above) --------------------------
// Buffer instructions with cache policy sc0 (bit 0 of the policy operand).  The empty asm with
// a memory clobber before each load keeps the compiler from reusing an earlier load's value in
// a polling loop (the buffer-load builtin is otherwise treated as a plain read).

struct XcdBuf {
    __amdgpu_buffer_rsrc_t r;
};

__device__ __forceinline__ XcdBuf xcd_buf(const uint64_t* base) {
    // num_records: the whole range reachable by 32-bit byte offsets; flags 0x00020000 is the
    // default data format of a raw buffer.
    return XcdBuf{__builtin_amdgcn_make_buffer_rsrc(const_cast<uint64_t*>(base), 0, 0x7fffffff, 0x00020000)};
}
__device__ __forceinline__ uint64_t xcd_load(XcdBuf b, uint32_t index) {
    asm volatile("" ::: "memory");
    const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(b.r, index * 8u, 0, 1);
    return (static_cast<uint64_t>(v.y) << 32) | v.x;
}
__device__ __forceinline__ void xcd_store(XcdBuf b, uint32_t index, uint64_t w) {
    u32x2 v;
    v.x = static_cast<uint32_t>(w);
    v.y = static_cast<uint32_t>(w >> 32);
    __builtin_amdgcn_raw_buffer_store_b64(v, b.r, index * 8u, 0, 1);
}

}  // namespace xchg
}  // namespace fmlh
