// Shared definitions for the MI355X (gfx950) target-verify library.
//
// Weights arrive in their GGUF block layouts (row-major [N][K/elems] blocks, as
// candle's QMatMul holds them: crates/speculate/src/model/quantized_llama_local.rs:258-281):
//   Q4_K  144 B / 256: f16 d | f16 dmin | u8 scales[12] | u8 qs[128]
//   Q5_K  176 B / 256: f16 d | f16 dmin | u8 scales[12] | u8 qh[32] | u8 qs[128]
//   Q6_K  210 B / 256: u8 ql[128] | u8 qh[64] | i8 scales[16] | f16 d
//   Q8_0   34 B /  32: f16 d | i8 qs[32]
// and are kept in HBM in a tile-interleaved layout (sd_layout.hip): a matrix of
// R rows (R % 16 == 0) is R/16 x K/256 tile blocks, tile-major, each holding
// the 16 rows' blocks of one 256-column superblock rearranged so that every
// load of the MFMA lane mapping (lane = r + 16 g) reads contiguous bytes.  The
// byte size is the GGUF size; only the order changes.
//
// Activations feeding a quantised matmul are fp16 in a "fragment" order: within
// each 256-element superblock, slot p = c*32 + g*8 + s (chunk c = 0..7, lane
// group g = 0..3, slot s = 0..7) holds element
//     e(c, g, s) = 64*g + 32*(s >> 2) + 4*c + {0, 2, 1, 3}[s & 3].
// That is the order in which one lane of a 16x16x32 MFMA unpacks its 8 weights
// from a 4-byte quant word, so the B operand is one 16-byte load.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sd {

enum Fmt : int { F32 = 0, Q8_0 = 8, Q4_K = 12, Q5_K = 13, Q6_K = 14 };

__host__ __device__ inline int fmt_block_bytes(int f) {
    return f == Q4_K ? 144 : f == Q5_K ? 176 : f == Q6_K ? 210 : f == Q8_0 ? 34 : 0;
}
__host__ __device__ inline int fmt_block_elems(int f) { return f == Q8_0 ? 32 : 256; }
// bytes of one 256-element superblock of one row (8 Q8_0 blocks for Q8_0)
__host__ __device__ inline int fmt_sb_bytes(int f) { return f == Q8_0 ? 272 : fmt_block_bytes(f); }
// bytes of one tile block (16 rows x one superblock) of the device layout
__host__ __device__ inline int tile_block_bytes(int f) { return 16 * fmt_sb_bytes(f); }
// bytes of a whole [rows][K] tensor (F32: plain row-major)
__host__ __device__ inline int64_t dev_tensor_bytes(int f, int64_t rows, int64_t K) {
    return f == F32 ? 4 * rows * K : rows * (K / 256) * fmt_sb_bytes(f);
}

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef unsigned int uintx4 __attribute__((ext_vector_type(4)));
typedef unsigned int uintx2 __attribute__((ext_vector_type(2)));

// element index inside a superblock for fragment slot p (see header comment)
__host__ __device__ inline int frag_elem(int p) {
    const int c = p >> 5, g = (p >> 3) & 3, s = p & 7;
    const int t = (s & 3) == 1 ? 2 : (s & 3) == 2 ? 1 : (s & 3);
    return 64 * g + 32 * (s >> 2) + 4 * c + t;
}
// inverse: fragment slot of element e inside a superblock
__host__ __device__ inline int frag_slot(int e) {
    const int g = e >> 6, hi = (e >> 5) & 1, r = e & 31, c = r >> 2, t = r & 3;
    const int s = hi * 4 + ((t == 1) ? 2 : (t == 2) ? 1 : t);
    return c * 32 + g * 8 + s;
}
__host__ __device__ inline int64_t frag_index(int64_t k) { return (k & ~int64_t(255)) + frag_slot((int)(k & 255)); }

// ---- KV cache layout ----------------------------------------------------
// The cache holds, per (layer, K/V, kv head) "stream", cap positions x hd
// fp16 values (cap a multiple of 32), blocked so that every MFMA operand the
// attention kernel loads is one contiguous 16-byte piece per lane and 1 KiB
// per wave:
//   K: [pos / 16][d / 32][pos % 16][d % 32]  (A operand of S^T = K Q^T: a lane
//      reads 8 consecutive d of one key)
//   V: [pos / 32][d][slot(pos % 32)]         (A operand of O^T = V^T P^T: a lane
//      reads the 8 keys its P^T fragment holds, {4g..4g+3, 16+4g..16+4g+3},
//      as slots 8g..8g+7)
__host__ __device__ inline int64_t kv_k_off(int64_t pos, int d, int hd) {
    return (pos >> 4) * 16 * hd + (d >> 5) * 512 + (pos & 15) * 32 + (d & 31);
}
__host__ __device__ inline int kv_v_slot(int r) { return 8 * ((r & 15) >> 2) + 4 * (r >> 4) + (r & 3); }
__host__ __device__ inline int64_t kv_v_off(int64_t pos, int d, int hd) {
    return (pos >> 5) * 32 * hd + d * 32 + kv_v_slot((int)(pos & 31));
}
__host__ __device__ inline int64_t kv_off(int which, int64_t pos, int d, int hd) {
    return which ? kv_v_off(pos, d, hd) : kv_k_off(pos, d, hd);
}

// ---- fp16 bit helpers --------------------------------------------------
__device__ inline float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
// f32 -> fp16 (round to nearest even) of the f32 value as the source computed
// it.  The empty asm keeps the compiler from fusing a producing multiply or
// multiply-add into the conversion (v_fma_mix*_f16: one rounding instead of
// two), which it does in some kernels and not in others; the same source then
// rounds the same way in every kernel that inlines it.
__device__ inline uint16_t f2h(float f) {
    asm("" : "+v"(f));
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// ---- seeded synthetic values (same arithmetic as the CPU generator) -----
__host__ __device__ inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
// Irwin-Hall(4) of 16-bit uniforms, centred: s in [-131070, 131070]; value = s * mult
__host__ __device__ inline float synth_value(uint64_t seed, uint64_t idx, float mult) {
    const uint64_t h = mix64(seed + (idx + 1ull) * 0x9E3779B97F4A7C15ull);
    const int32_t s = (int32_t)(h & 0xffff) + (int32_t)((h >> 16) & 0xffff) + (int32_t)((h >> 32) & 0xffff) +
                      (int32_t)(h >> 48) - 131070;
    return (float)s * mult;
}
inline uint64_t tensor_seed(uint64_t model_seed, int layer, int kind) {
    const uint64_t tag = ((uint64_t)(((layer + 1) << 8) | kind)) * 0xD1B54A32D192ED03ull;
    return mix64(model_seed ^ tag);
}

// 1 / rms of one token from its np partial sums of squares (RMSNorm split
// around a matmul): four running sums over j = i, i + 4, ... added as
// ((s0 + s1) + (s2 + s3)), the order in which four lanes combine them
__device__ inline float norm_inv_rms(const float *ssq_row, int np, int K, float eps) {
    float q[4] = {0.f, 0.f, 0.f, 0.f};
    for (int j = 0; j < np; j++) q[j & 3] += ssq_row[j];
    return 1.0f / sqrtf(((q[0] + q[1]) + (q[2] + q[3])) / (float)K + eps);
}

}  // namespace sd

#define SD_HIP_CHECK(expr)                                                        \
    do {                                                                          \
        hipError_t _e = (expr);                                                   \
        if (_e != hipSuccess) {                                                   \
            throw sd::BackendError(std::string(#expr) + ": " + hipGetErrorString(_e)); \
        }                                                                         \
    } while (0)
