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

}  // namespace sd
