// Buffer-resource loads shared by the matmul and attention kernels.
//
// A buffer resource holds a base address and a byte size in scalar registers;
// a load adds a per-lane vector offset and a wave-uniform scalar offset, so
// loop bodies do no 64-bit address arithmetic.  Reads past the resource's size
// return zero without touching memory.
#pragma once
#include "sd_common.hpp"

namespace sd {

typedef __amdgpu_buffer_rsrc_t rsrc_t;
__device__ __forceinline__ rsrc_t make_rsrc(const void *base, uint32_t bytes) {
    // the operands are wave-uniform; readfirstlane makes that visible to the
    // compiler, which otherwise may keep them in vector registers and wrap
    // every buffer load in a per-lane loop
    const uint64_t a = (uint64_t)base;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
    const uint64_t u = ((uint64_t)hi << 32) | lo;
    return __builtin_amdgcn_make_buffer_rsrc((void *)u, (short)0, (int)__builtin_amdgcn_readfirstlane(bytes),
                                             0x00020000);
}
// wave-uniform value pinned to a scalar register (the soffset operand)
__device__ __forceinline__ uint32_t uni(uint32_t v) { return __builtin_amdgcn_readfirstlane(v); }
// CP: the load's cache-policy bits; kLoadDev (sc1) reads at device scope,
// past the XCD's L2 (data another XCD wrote during this launch)
constexpr int kLoadDev = 16;
template <int CP = 0> __device__ __forceinline__ uintx4 bld16(rsrc_t r, uint32_t vo, uint32_t so) {
    return __builtin_bit_cast(uintx4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)vo, (int)so, CP));
}
__device__ __forceinline__ uintx2 bld8(rsrc_t r, uint32_t vo, uint32_t so) {
    return __builtin_bit_cast(uintx2, __builtin_amdgcn_raw_buffer_load_b64(r, (int)vo, (int)so, 0));
}
__device__ __forceinline__ uint32_t bld4(rsrc_t r, uint32_t vo, uint32_t so) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, (int)vo, (int)so, 0);
}
__device__ __forceinline__ uint32_t bld2(rsrc_t r, uint32_t vo, uint32_t so) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, (int)vo, (int)so, 0);
}

// Device-scope (sc1) 8- and 2-byte accesses, for data that workgroups of one
// launch hand to each other.  Each XCD has its own L2: a plain store may stay there
// until the kernel ends and a plain load may hit a line another XCD has since
// rewritten, while an sc1 store is written through to memory and an sc1 load
// reads past the XCD's L2, without writing back or invalidating whole caches.
// (Plain stores handed over inside one launch were measured to deliver stale
// data to other XCDs.)  Device-scope atomics are coherent across the XCDs.
__device__ __forceinline__ void st_dev64(void *p, uint64_t v) {
    __hip_atomic_store((uint64_t *)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_dev64(const void *p) {
    return __hip_atomic_load((const uint64_t *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev16(uint16_t *p, uint16_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The kernel's argument block (or the part at byte offset OFF) as a
// reference into the kernarg segment.  A kernel that hands its by-value
// parameter to a device function has the compiler copy it to the stack and,
// once inlined, load every field at entry and keep them all in scalar
// registers (spilling them); reads through the segment stay constant loads
// that the compiler repeats where they are used.
template <typename T, int OFF = 0> __device__ __forceinline__ const T &kernarg() {
    return *(const T *)((const __attribute__((address_space(4))) char *)__builtin_amdgcn_kernarg_segment_ptr() + OFF);
}

// A kernel's argument block reaches its waves through the scalar cache.  A
// kernel that reads a large parameter struct field by field, with branches
// between the reads, waits one memory round trip (~0.5 us) per cache line it
// first touches.  Touching every 64-byte line of the first BYTES bytes at
// once fills them in a single round trip; later reads of any field then hit.
// The loads (eight, or sixteen for blocks over 512 bytes, the last line
// repeated) sit in one asm statement with their wait, so the compiler cannot
// split them into batches with a wait between each.
template <int BYTES> __device__ __forceinline__ void warm_kernargs() {
    constexpr int L = (BYTES + 63) / 64 - 1;  // last line
    static_assert(L >= 0 && L < 16, "argument blocks of at most 1 KiB");
    const auto ka = __builtin_amdgcn_kernarg_segment_ptr();
    if constexpr (L < 8) {
        uint32_t v0, v1, v2, v3, v4, v5, v6, v7;
        asm volatile(
            "s_load_dword %0, %8, %9\n\t"
            "s_load_dword %1, %8, %10\n\t"
            "s_load_dword %2, %8, %11\n\t"
            "s_load_dword %3, %8, %12\n\t"
            "s_load_dword %4, %8, %13\n\t"
            "s_load_dword %5, %8, %14\n\t"
            "s_load_dword %6, %8, %15\n\t"
            "s_load_dword %7, %8, %16\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&s"(v0), "=&s"(v1), "=&s"(v2), "=&s"(v3), "=&s"(v4), "=&s"(v5), "=&s"(v6), "=&s"(v7)
            : "s"(ka), "i"(0), "i"((L < 1 ? L : 1) * 64), "i"((L < 2 ? L : 2) * 64), "i"((L < 3 ? L : 3) * 64),
              "i"((L < 4 ? L : 4) * 64), "i"((L < 5 ? L : 5) * 64), "i"((L < 6 ? L : 6) * 64), "i"(L * 64)
            : "memory");
    } else {
        // every load writes the same (discarded) register, complete at the wait
        uint32_t v;
        asm volatile(
            "s_load_dword %0, %1, 0x0\n\t"
            "s_load_dword %0, %1, 0x40\n\t"
            "s_load_dword %0, %1, 0x80\n\t"
            "s_load_dword %0, %1, 0xc0\n\t"
            "s_load_dword %0, %1, 0x100\n\t"
            "s_load_dword %0, %1, 0x140\n\t"
            "s_load_dword %0, %1, 0x180\n\t"
            "s_load_dword %0, %1, 0x1c0\n\t"
            "s_load_dword %0, %1, %2\n\t"
            "s_load_dword %0, %1, %3\n\t"
            "s_load_dword %0, %1, %4\n\t"
            "s_load_dword %0, %1, %5\n\t"
            "s_load_dword %0, %1, %6\n\t"
            "s_load_dword %0, %1, %7\n\t"
            "s_load_dword %0, %1, %8\n\t"
            "s_load_dword %0, %1, %9\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&s"(v)
            : "s"(ka), "i"(8 * 64), "i"((L < 9 ? L : 9) * 64), "i"((L < 10 ? L : 10) * 64),
              "i"((L < 11 ? L : 11) * 64), "i"((L < 12 ? L : 12) * 64), "i"((L < 13 ? L : 13) * 64),
              "i"((L < 14 ? L : 14) * 64), "i"(L * 64)
            : "memory");
    }
}

}  // namespace sd
