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
__device__ __forceinline__ uintx4 bld16(rsrc_t r, uint32_t vo, uint32_t so) {
    return __builtin_bit_cast(uintx4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)vo, (int)so, 0));
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

// A kernel's argument block reaches its waves through the scalar cache.  A
// kernel that reads a large parameter struct field by field, with branches
// between the reads, waits one memory round trip (~0.5 us) per cache line it
// first touches.  Touching every 64-byte line of the first BYTES bytes at once
// fills them in a single round trip; later reads of any field then hit.
template <int BYTES> __device__ __forceinline__ void warm_kernargs() {
    typedef const uint32_t __attribute__((address_space(4))) cu32;
    const cu32 *ka = (const cu32 *)__builtin_amdgcn_kernarg_segment_ptr();
    uint32_t acc = 0;
#pragma unroll
    for (int i = 0; i < (BYTES + 63) / 64; i++) acc ^= ka[16 * i];
    asm volatile("" ::"s"(acc));  // waits for every line once, here
}

}  // namespace sd
