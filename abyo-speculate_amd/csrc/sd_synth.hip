// Seeded synthetic weights / KV contents, and the bit-exact f32 dequantiser.
//
// The generator draws N(0, std)-like values from a counter hash (Irwin-Hall of
// four 16-bit uniforms) and quantises each block with this library's own
// deterministic quantiser.  The value of element i of a tensor depends only on
// (seed, i), so the blocks are independent of launch shape; the CPU generator
// used by the tests computes the same blocks bit for bit.
//
// The dequantiser evaluates the GGUF block expressions in f32 with two
// roundings (no FMA), as candle's CPU dequantize does for the tensors loaded at
// crates/speculate/src/model/quantized_llama_local.rs:242-243 (token_embd) and
// behind every QMatMul (:47-49, 73-90, 135, 317).
#include "sd_common.hpp"
#include "sd_kernels.hpp"
#include "sd_tiles.hpp"

namespace sd {

#pragma clang fp contract(off)

__device__ inline float clampf_(float v, float lo, float hi) { return v < lo ? lo : (v > hi ? hi : v); }
__device__ inline float f16_round(float x) { return (float)(_Float16)x; }

__device__ inline void st_u16(uint8_t *p, uint16_t v) {
    p[0] = (uint8_t)(v & 0xff);
    p[1] = (uint8_t)(v >> 8);
}

// Q4_K (nmax 15) / Q5_K (nmax 31): per 32-element sub-block scale=(max-min)/nmax,
// min=-min(0,min); 6-bit scales against f16 super-scales d=max_scale/63, dmin=max_min/63.
template <int NMAX>
__device__ void quant_kasym_dev(uint64_t seed, uint64_t base, float mult, uint8_t sc6[8], uint8_t mn6[8], float &df,
                                float &dmf) {
    float scale[8], minv[8], max_scale = 0.f, max_min = 0.f;
    for (int j = 0; j < 8; j++) {
        float mn = synth_value(seed, base + 32 * j, mult), mx = mn;
        for (int l = 1; l < 32; l++) {
            const float v = synth_value(seed, base + 32 * j + l, mult);
            if (v < mn) mn = v;
            if (v > mx) mx = v;
        }
        if (mn > 0.f) mn = 0.f;
        scale[j] = (mx - mn) / (float)NMAX;
        minv[j] = -mn;
        if (scale[j] > max_scale) max_scale = scale[j];
        if (minv[j] > max_min) max_min = minv[j];
    }
    df = f16_round(max_scale / 63.f);
    dmf = f16_round(max_min / 63.f);
    for (int j = 0; j < 8; j++) {
        sc6[j] = df > 0.f ? (uint8_t)clampf_(rintf(scale[j] / df), 0.f, 63.f) : 0;
        mn6[j] = dmf > 0.f ? (uint8_t)clampf_(rintf(minv[j] / dmf), 0.f, 63.f) : 0;
    }
}

__device__ inline void pack_scale_min(const uint8_t sc[8], const uint8_t mn[8], uint8_t *q) {
    for (int j = 0; j < 4; j++) {
        q[j] = (uint8_t)(sc[j] | ((sc[j + 4] >> 4) << 6));
        q[j + 4] = (uint8_t)(mn[j] | ((mn[j + 4] >> 4) << 6));
        q[j + 8] = (uint8_t)((sc[j + 4] & 0xF) | ((mn[j + 4] & 0xF) << 4));
    }
}

template <int NMAX>
__device__ inline uint8_t quant_kasym_elem(uint64_t seed, uint64_t idx, float mult, float d1, float m1) {
    const float v = synth_value(seed, idx, mult);
    return d1 > 0.f ? (uint8_t)clampf_(rintf((v + m1) / d1), 0.f, (float)NMAX) : 0;
}

__global__ void k_synth_q4k(uint8_t *out, int64_t nsb_total, int64_t K, uint64_t seed, float mult) {
    const int64_t sb = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (sb >= nsb_total) return;
    const uint64_t base = (uint64_t)sb * 256;  // rows*K laid out row-major; K % 256 == 0
    uint8_t sc6[8], mn6[8];
    float df, dmf;
    quant_kasym_dev<15>(seed, base, mult, sc6, mn6, df, dmf);
    uint8_t *o = out + sb * 144;
    st_u16(o, f2h(df));
    st_u16(o + 2, f2h(dmf));
    pack_scale_min(sc6, mn6, o + 4);
    for (int j = 0; j < 4; j++) {
        const float d1 = df * (float)sc6[2 * j], m1 = dmf * (float)mn6[2 * j];
        const float d2 = df * (float)sc6[2 * j + 1], m2 = dmf * (float)mn6[2 * j + 1];
        for (int l = 0; l < 32; l++) {
            const uint8_t lo = quant_kasym_elem<15>(seed, base + 64 * j + l, mult, d1, m1);
            const uint8_t hi = quant_kasym_elem<15>(seed, base + 64 * j + 32 + l, mult, d2, m2);
            o[16 + 32 * j + l] = (uint8_t)(lo | (hi << 4));
        }
    }
}

__global__ void k_synth_q5k(uint8_t *out, int64_t nsb_total, int64_t K, uint64_t seed, float mult) {
    const int64_t sb = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (sb >= nsb_total) return;
    const uint64_t base = (uint64_t)sb * 256;
    uint8_t sc6[8], mn6[8];
    float df, dmf;
    quant_kasym_dev<31>(seed, base, mult, sc6, mn6, df, dmf);
    uint8_t *o = out + sb * 176;
    st_u16(o, f2h(df));
    st_u16(o + 2, f2h(dmf));
    pack_scale_min(sc6, mn6, o + 4);
    uint8_t *qh = o + 16, *ql = o + 48;
    for (int l = 0; l < 32; l++) qh[l] = 0;
    for (int j = 0; j < 4; j++) {
        const float d1 = df * (float)sc6[2 * j], m1 = dmf * (float)mn6[2 * j];
        const float d2 = df * (float)sc6[2 * j + 1], m2 = dmf * (float)mn6[2 * j + 1];
        for (int l = 0; l < 32; l++) {
            const uint8_t lo = quant_kasym_elem<31>(seed, base + 64 * j + l, mult, d1, m1);
            const uint8_t hi = quant_kasym_elem<31>(seed, base + 64 * j + 32 + l, mult, d2, m2);
            ql[32 * j + l] = (uint8_t)((lo & 0xF) | ((hi & 0xF) << 4));
            qh[l] |= (uint8_t)((((lo >> 4) & 1) << (2 * j)) | (((hi >> 4) & 1) << (2 * j + 1)));
        }
    }
}

__global__ void k_synth_q6k(uint8_t *out, int64_t nsb_total, int64_t K, uint64_t seed, float mult) {
    const int64_t sb = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (sb >= nsb_total) return;
    const uint64_t base = (uint64_t)sb * 256;
    float scale[16], max_scale = 0.f;
    for (int j = 0; j < 16; j++) {
        float amax = 0.f;
        for (int l = 0; l < 16; l++) {
            const float a = fabsf(synth_value(seed, base + 16 * j + l, mult));
            if (a > amax) amax = a;
        }
        scale[j] = amax / 31.f;
        if (scale[j] > max_scale) max_scale = scale[j];
    }
    const float df = f16_round(max_scale / 127.f);
    uint8_t *o = out + sb * 210;
    int8_t sc[16];
    for (int j = 0; j < 16; j++) {
        sc[j] = (int8_t)(df > 0.f ? (int)clampf_(rintf(scale[j] / df), 0.f, 127.f) : 0);
        o[192 + j] = (uint8_t)sc[j];
    }
    auto q6 = [&](int e) -> uint8_t {
        const float ds = df * (float)sc[e >> 4];
        const float v = synth_value(seed, base + e, mult);
        const int qi = ds > 0.f ? (int)clampf_(rintf(v / ds), -32.f, 31.f) : 0;
        return (uint8_t)(qi + 32);
    };
    for (int h = 0; h < 2; h++)
        for (int l = 0; l < 32; l++) {
            const uint8_t q1 = q6(128 * h + l), q2 = q6(128 * h + 32 + l), q3 = q6(128 * h + 64 + l),
                          q4 = q6(128 * h + 96 + l);
            o[64 * h + l] = (uint8_t)((q1 & 0xF) | ((q3 & 0xF) << 4));
            o[64 * h + 32 + l] = (uint8_t)((q2 & 0xF) | ((q4 & 0xF) << 4));
            o[128 + 32 * h + l] = (uint8_t)((q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6));
        }
    st_u16(o + 208, f2h(df));
}

__global__ void k_synth_q80(uint8_t *out, int64_t nblk_total, uint64_t seed, float mult) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblk_total) return;
    const uint64_t base = (uint64_t)b * 32;
    float amax = 0.f;
    for (int l = 0; l < 32; l++) {
        const float a = fabsf(synth_value(seed, base + l, mult));
        if (a > amax) amax = a;
    }
    const float df = f16_round(amax / 127.f);
    uint8_t *o = out + b * 34;
    st_u16(o, f2h(df));
    for (int l = 0; l < 32; l++) {
        const float v = synth_value(seed, base + l, mult);
        o[2 + l] = (uint8_t)(int8_t)(df > 0.f ? (int)clampf_(rintf(v / df), -127.f, 127.f) : 0);
    }
}

__global__ void k_synth_f32(float *out, int64_t n, uint64_t seed, float mult) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = synth_value(seed, (uint64_t)i, mult);
}

__global__ void k_fill_f32(float *out, int64_t n, float v) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = v;
}

// KV rows [0, P) of every (layer, K/V, head): fp16(N(0,1)-like), value index
// (stream << 32) | (pos * hd + d) with stream = (layer*2 + kv)*n_kv + head,
// stored at the element's place in the blocked cache layout (kv_off).
__global__ void k_fill_kv(uint16_t *kv, int L, int n_kv, int64_t cap, int hd, int P, uint64_t seed, float mult) {
    const int64_t per_stream = (int64_t)P * hd;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t total = (int64_t)L * 2 * n_kv * per_stream;
    if (i >= total) return;
    const int64_t stream = i / per_stream, r = i % per_stream;
    const uint64_t idx = ((uint64_t)stream << 32) | (uint64_t)r;
    const int which = (int)((stream / n_kv) & 1);
    kv[stream * cap * hd + kv_off(which, r / hd, (int)(r % hd), hd)] = f2h(synth_value(seed, idx, mult));
}

// ---- exact f32 dequantisation: one thread per 32 outputs ----------------
__device__ inline float ldh(const uint8_t *p) { return h2f((uint16_t)(p[0] | (p[1] << 8))); }

__global__ void k_dequant(int fmt, const uint8_t *w, int64_t n_groups, float *y) {
    // a "group" = 32 consecutive output elements
    const int64_t gi = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gi >= n_groups) return;
    float *o = y + gi * 32;
    if (fmt == Q8_0) {
        const uint8_t *b = w + gi * 34;
        const float d = ldh(b);
        for (int l = 0; l < 32; l++) o[l] = d * (float)(int8_t)b[2 + l];
        return;
    }
    const int64_t sb = gi >> 3;
    const int part = (int)(gi & 7);  // 32-element part of the superblock
    if (fmt == Q4_K || fmt == Q5_K) {
        const int bb = fmt == Q4_K ? 144 : 176;
        const uint8_t *b = w + sb * bb;
        const float d = ldh(b), mn = ldh(b + 2);
        int s, m;
        kq_scale_min(b + 4, part, s, m);  // GGUF's 6-bit scale / min packing
        const float d1 = d * (float)s, m1 = mn * (float)m;
        const int j = part >> 1, hi = part & 1;
        if (fmt == Q4_K) {
            const uint8_t *q = b + 16 + 32 * j;
            for (int l = 0; l < 32; l++) o[l] = d1 * (float)(hi ? (q[l] >> 4) : (q[l] & 0xF)) - m1;
        } else {
            const uint8_t *qh = b + 16, *q = b + 48 + 32 * j;
            const int u = 1 << (2 * j + hi);
            for (int l = 0; l < 32; l++)
                o[l] = d1 * (float)((hi ? (q[l] >> 4) : (q[l] & 0xF)) + ((qh[l] & u) ? 16 : 0)) - m1;
        }
        return;
    }
    if (fmt == Q6_K) {
        const uint8_t *b = w + sb * 210;
        const float d = ldh(b + 208);
        const int h = part >> 2, qd = part & 3;  // elements 128h + 32qd + l
        const uint8_t *ql = b + 64 * h + 32 * (qd & 1), *qh = b + 128 + 32 * h;
        const int8_t *sc = (const int8_t *)(b + 192 + 8 * h);
        for (int l = 0; l < 32; l++) {
            const int nib = qd < 2 ? (ql[l] & 0xF) : (ql[l] >> 4);
            const int q = (nib | (((qh[l] >> (2 * qd)) & 3) << 4)) - 32;
            o[l] = d * (float)sc[l / 16 + 2 * qd] * (float)q;
        }
    }
}

// ---- launchers -----------------------------------------------------------
void launch_synth_quant(int fmt, uint8_t *out, int64_t rows, int64_t K, uint64_t seed, float mult, hipStream_t st) {
    const int T = 64;
    if (fmt == Q8_0) {
        const int64_t nb = rows * K / 32;
        hipLaunchKernelGGL(k_synth_q80, dim3((unsigned)((nb + T - 1) / T)), dim3(T), 0, st, out, nb, seed, mult);
        return;
    }
    const int64_t nsb = rows * K / 256;
    const dim3 g((unsigned)((nsb + T - 1) / T));
    if (fmt == Q4_K) hipLaunchKernelGGL(k_synth_q4k, g, dim3(T), 0, st, out, nsb, K, seed, mult);
    else if (fmt == Q5_K) hipLaunchKernelGGL(k_synth_q5k, g, dim3(T), 0, st, out, nsb, K, seed, mult);
    else if (fmt == Q6_K) hipLaunchKernelGGL(k_synth_q6k, g, dim3(T), 0, st, out, nsb, K, seed, mult);
}

void launch_synth_f32(float *out, int64_t n, uint64_t seed, float mult, hipStream_t st) {
    hipLaunchKernelGGL(k_synth_f32, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, out, n, seed, mult);
}

void launch_fill_f32(float *out, int64_t n, float v, hipStream_t st) {
    hipLaunchKernelGGL(k_fill_f32, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, out, n, v);
}

void launch_fill_kv(uint16_t *kv, int L, int n_kv, int64_t cap, int hd, int P, uint64_t seed, float mult,
                    hipStream_t st) {
    const int64_t total = (int64_t)L * 2 * n_kv * P * hd;
    if (total == 0) return;
    hipLaunchKernelGGL(k_fill_kv, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, kv, L, n_kv, cap, hd, P,
                       seed, mult);
}

void launch_dequant(int fmt, const uint8_t *w, int64_t n_elems, float *y, hipStream_t st) {
    const int64_t groups = n_elems / 32;
    hipLaunchKernelGGL(k_dequant, dim3((unsigned)((groups + 127) / 128)), dim3(128), 0, st, fmt, w, groups, y);
}

}  // namespace sd
