// Lane view of the tile-interleaved weight layout and the integer part of the
// in-register dequantisation (shared by the matmul kernels and by the
// host-side layout tests, hence __host__ __device__).
//
// A lane (r = lane & 15, g = lane >> 4) of a 16x16x32 MFMA owns row r of a
// 16-row tile and the elements 64g .. 64g+63 of each 256-element superblock.
// For each superblock it loads a few fixed byte ranges of the tile block
// (offsets below, relative to the block start) and, for K-chunk c = 0..7,
// builds four 32-bit words p0..p3 of two fp16 "codes" each:
//   p0: slots 0,1   p1: slots 2,3   (half s' = 0 of the lane's elements)
//   p2: slots 4,5   p3: slots 6,7   (half s' = 1)
// A code is an fp16 number 1024 + q (p0, p1: 0x6400 | q) or 64 + q (p2, p3:
// 0x5400 | q << 4) holding the element's unsigned quant value q exactly, so
// one packed fp16 FMA or multiply per pair of codes removes the offset and
// applies the scale (the matmul kernels' QFmt::frag / ifrag).
#pragma once
#include <stdint.h>

#include "sd_common.hpp"

namespace sd {

// ---- bit helpers (one VALU instruction each on the device) -------------------
// (a & m) | o as one v_and_or_b32: a gfx9 VOP3 takes no literal operand and
// reads at most one scalar register, so the mask goes in a scalar register and
// the OR operand in a vector register (the compiler would otherwise split the
// expression into v_and + v_or).
__host__ __device__ inline uint32_t and_or(uint32_t a, uint32_t m, uint32_t o) {
#if defined(__HIP_DEVICE_COMPILE__)
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "s"(m), "v"(o));
    return r;
#else
    return (a & m) | o;
#endif
}
// v_perm_b32: byte i of the result = byte sel_i of the 8 bytes {hi, lo}
// (selectors 0-3 pick lo's bytes, 4-7 hi's)
__host__ __device__ inline uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __builtin_amdgcn_perm(hi, lo, sel);
#else
    const uint64_t v = ((uint64_t)hi << 32) | lo;
    uint32_t r = 0;
    for (int i = 0; i < 4; i++) r |= (uint32_t)((v >> (8 * ((sel >> (8 * i)) & 7))) & 0xff) << (8 * i);
    return r;
#endif
}
// rotate right (v_alignbit_b32 x, x, n)
__host__ __device__ inline uint32_t rotr(uint32_t x, int n) {
#if defined(__HIP_DEVICE_COMPILE__)
    return n ? __builtin_amdgcn_alignbit(x, x, n) : x;
#else
    return n ? (x >> n) | (x << (32 - n)) : x;
#endif
}
// word c (0..7) of the 32 bytes a|b; c is a compile-time constant after unrolling
__host__ __device__ inline uint32_t wsel(const uintx4 &a, const uintx4 &b, int c) {
    const uintx4 &v = c < 4 ? a : b;
    const int i = c & 3;
    return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

// ---- per-format lane data: byte offsets in the tile block and code extraction ----
struct LaneQ4K {
    uintx4 hdr, q0, q1;
    static constexpr int TBB = 2304;
    __host__ __device__ static int off_hdr(int lane) { return (lane & 15) * 16; }
    __host__ __device__ static int off_q0(int lane) { return 256 + lane * 16; }
    __host__ __device__ static int off_q1(int lane) { return 1280 + lane * 16; }
    __host__ __device__ void codes(int g, int c, uint32_t p[4]) const {
        const uint32_t w = wsel(q0, q1, c), w8 = w >> 8;
        const uint32_t e64 = 0x64006400u, e54 = 0x54005400u;
        p[0] = and_or(w, 0x000F000Fu, e64);   // bytes 0,2 low: 1024 + q
        p[1] = and_or(w8, 0x000F000Fu, e64);  // bytes 1,3 low
        p[2] = and_or(w, 0x00F000F0u, e54);   // bytes 0,2 high: 64 + q
        p[3] = and_or(w8, 0x00F000F0u, e54);  // bytes 1,3 high
    }
};

// Q5_K: fifth bits of chunk c in word c >> 2 rotated left by {0, 2, 8, 10}[c & 3];
// unrotated, the low-nibble element t sits at bit 4 / 20 (t = 0 / 2, +1 for
// odd t) and the high-nibble element at 8 / 24 (+1).
struct LaneQ5K {
    uintx4 hdr, q0, q1;
    uintx2 qh;
    static constexpr int TBB = 2816;
    __host__ __device__ static int off_hdr(int lane) { return (lane & 15) * 16; }
    __host__ __device__ static int off_qh(int lane) { return 256 + lane * 8; }
    __host__ __device__ static int off_q0(int lane) { return 768 + lane * 16; }
    __host__ __device__ static int off_q1(int lane) { return 1792 + lane * 16; }
    __host__ __device__ static int rot(int c) { return (c & 1) * 2 + (c & 2) * 4; }  // 0, 2, 8, 10
    __host__ __device__ void codes(int g, int c, uint32_t p[4]) const {
        const uint32_t w = wsel(q0, q1, c), w8 = w >> 8;
        const uint32_t R = rotr(c < 4 ? qh.x : qh.y, rot(c)), R1 = R >> 1;
        const uint32_t x02 = and_or(R, 0x00100010u, 0x64006400u);  // fifth bit -> 16 in the 1024 binade
        const uint32_t x13 = and_or(R1, 0x00100010u, 0x64006400u);
        const uint32_t y02 = and_or(R, 0x01000100u, 0x54005400u);  // fifth bit -> 16 in the 64 binade
        const uint32_t y13 = and_or(R1, 0x01000100u, 0x54005400u);
        p[0] = and_or(w, 0x000F000Fu, x02);  // 1024 + q5
        p[1] = and_or(w8, 0x000F000Fu, x13);
        p[2] = and_or(w, 0x00F000F0u, y02);  // 64 + q5
        p[3] = and_or(w8, 0x00F000F0u, y13);
    }
};

// Q6_K: nibble byte l = low 4 bits of element (s'=0, l) | (s'=1, l) << 4; the
// 2-bit high parts of chunk c in word c >> 1 rotated left by 8 * (c & 1);
// unrotated, low-nibble element t at bits 4 / 20 (+2 for odd t), high at 8 / 24 (+2).
struct LaneQ6K {
    uintx4 n0, n1, hb;
    uint32_t sc, d;
    static constexpr int TBB = 3360;
    __host__ __device__ static int off_n0(int lane) { return lane * 16; }
    __host__ __device__ static int off_n1(int lane) { return 1024 + lane * 16; }
    __host__ __device__ static int off_hb(int lane) { return 2048 + lane * 16; }
    __host__ __device__ static int off_sc(int lane) { return 3072 + (lane & 15) * 16 + 4 * (lane >> 4); }
    __host__ __device__ static int off_d(int lane) { return 3328 + (lane & 15) * 2; }
    __host__ __device__ void codes(int g, int c, uint32_t p[4]) const {
        const uint32_t w = wsel(n0, n1, c), w8 = w >> 8;
        const int k = c >> 1;
        const uint32_t hw = k == 0 ? hb.x : k == 1 ? hb.y : k == 2 ? hb.z : hb.w;
        const uint32_t R = rotr(hw, 8 * (c & 1)), R2 = R >> 2;
        const uint32_t x02 = and_or(R, 0x00300030u, 0x64006400u);  // high bits -> 16, 32 in the 1024 binade
        const uint32_t x13 = and_or(R2, 0x00300030u, 0x64006400u);
        const uint32_t y02 = and_or(R, 0x03000300u, 0x54005400u);  // high bits -> 16, 32 in the 64 binade
        const uint32_t y13 = and_or(R2, 0x03000300u, 0x54005400u);
        p[0] = and_or(w, 0x000F000Fu, x02);  // s' = 0: 1024 + q6
        p[1] = and_or(w8, 0x000F000Fu, x13);
        p[2] = and_or(w, 0x00F000F0u, y02);  // s' = 1: 64 + q6
        p[3] = and_or(w8, 0x00F000F0u, y13);
    }
};

// Q8_0: the lane's 64 bytes are blocks 2g (parts 0, 1) and 2g+1 (parts 2, 3),
// stored as q + 128 (the relayout flips each byte's top bit); codes 1024 + (q + 128)
struct LaneQ80 {
    uintx4 a0, a1, b0, b1;
    uint32_t d;
    static constexpr int TBB = 4352;
    __host__ __device__ static int off_part(int lane, int p) { return 1024 * p + lane * 16; }
    __host__ __device__ static int off_d(int lane) { return 4096 + (lane & 15) * 16 + 4 * (lane >> 4); }
    __host__ __device__ void codes(int g, int c, uint32_t p[4]) const {
        const uint32_t qa = wsel(a0, a1, c), qb = wsel(b0, b1, c);
        const uint32_t M = 0x64646464u;
        p[0] = perm(qa, M, 0x00060004u);  // {qa.b0, 0x64, qa.b2, 0x64}
        p[1] = perm(qa, M, 0x00070005u);  // {qa.b1, 0x64, qa.b3, 0x64}
        p[2] = perm(qb, M, 0x00060004u);
        p[3] = perm(qb, M, 0x00070005u);
    }
};

}  // namespace sd
