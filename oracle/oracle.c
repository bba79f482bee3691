/*
 * CPU oracle for the target-verify path: TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only to check results against (or as the timed CPU baseline).
 * The product library (abyo-speculate_amd/) never links, loads or calls it.
 *
 * What is restated here, and from where (paths relative to the reference
 * checkout):
 *   - GGUF block dequantisation for Q4_K / Q5_K / Q6_K / Q8_0.  The reference
 *     calls it through candle-core 0.8.4 (external, not vendored):
 *     `QMatMul::forward` at crates/speculate/src/model/quantized_llama_local.rs:47-49,
 *     73-90, 135, 317 and `tok_q.dequantize` at :242-243.  The block layouts
 *     and the f32 expressions follow the published ggml k-quants format that
 *     candle mirrors (d*sc*q - dmin*m for Q4_K/Q5_K, (d*sc)*(q-32) for Q6_K,
 *     d*q for Q8_0), evaluated without FMA contraction as Rust does.
 *   - IEEE binary16 <-> binary32 conversion (round to nearest even), as the
 *     `half` 2.7.1 crate does for the block super-scales.
 *   - softmax_with_temperature / sample_from_distribution
 *     (crates/speculate/src/sampling/tokens.rs:15-55, 99-120),
 *     modified_rejection_step / adjusted_distribution
 *     (crates/speculate/src/methods/vanilla.rs:59-73, 83-106) and the
 *     first-max argmax fold (crates/speculate/src/methods/eagle.rs:626-637):
 *     sequential f32 folds with libm expf, in the reference's order.
 *   - Synthetic weights: a seeded counter hash -> Irwin-Hall normal ->
 *     the library's own deterministic block quantiser.  The reference has no
 *     quantiser of its own (candle's QTensor::quantize is external); parity
 *     is defined on the blocks, and this generator must equal the product's
 *     GPU generator bit for bit.
 *
 * Build: gcc -O2 -ffp-contract=off -fno-fast-math -fopenmp -shared -fPIC.
 * FP contraction is off so every a*b-c below rounds twice, like the Rust code.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#include <stdlib.h>

#define QK_K 256

/* ------------------------------------------------------------------ */
/* binary16 conversions (IEEE 754-2008, round to nearest, ties to even) */
/* ------------------------------------------------------------------ */
float or_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1f;
    uint32_t man = h & 0x3ff;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else { /* subnormal: man * 2^-24 */
            float v = (float)man * 5.9604644775390625e-08f; /* exact */
            memcpy(&bits, &v, 4);
            bits |= sign;
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t or_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xffu;
    uint32_t man = x & 0x7fffffu;
    if (exp == 0xff) return (uint16_t)(sign | 0x7c00u | (man ? 0x200u : 0u));
    int e = (int)exp - 112; /* rebias 127 -> 15 */
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        /* subnormal result: m = full * 2^(exp-126), rounded to nearest even */
        if (exp == 0) return (uint16_t)sign; /* f32 subnormals are far below 2^-25 */
        uint32_t full = man | 0x800000u;
        int shift = 14 - e; /* >= 14 */
        if (shift > 24) return (uint16_t)sign;
        uint32_t m = full >> shift;
        uint32_t rem = full & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (m & 1u))) m++;
        return (uint16_t)(sign | m);
    }
    uint32_t h = sign | ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)h;
}

void or_f32_to_f16_array(const float *x, int64_t n, uint16_t *y) {
    for (int64_t i = 0; i < n; i++) y[i] = or_f32_to_f16(x[i]);
}
void or_f16_to_f32_array(const uint16_t *x, int64_t n, float *y) {
    for (int64_t i = 0; i < n; i++) y[i] = or_f16_to_f32(x[i]);
}

static float ld_f16(const uint8_t *p) {
    uint16_t h;
    memcpy(&h, p, 2);
    return or_f16_to_f32(h);
}
static void st_f16(uint8_t *p, float v) {
    uint16_t h = or_f32_to_f16(v);
    memcpy(p, &h, 2);
}

/* ------------------------------------------------------------------ */
/* GGUF block dequantisation                                            */
/* ------------------------------------------------------------------ */
/* 6-bit scale/min unpacking of the 12-byte K-quant scale field. */
void or_get_scale_min_k4(int j, const uint8_t *q, uint8_t *d, uint8_t *m) {
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j - 0] >> 6) << 4));
    }
}

/* Q4_K: half d | half dmin | u8 scales[12] | u8 qs[128]   (144 bytes) */
void or_dequant_q4k(const uint8_t *blk, int64_t nblocks, float *y) {
    for (int64_t b = 0; b < nblocks; b++, blk += 144) {
        const float d = ld_f16(blk), min = ld_f16(blk + 2);
        const uint8_t *sc = blk + 4, *q = blk + 16;
        int is = 0;
        for (int j = 0; j < QK_K; j += 64) {
            uint8_t s, m;
            or_get_scale_min_k4(is + 0, sc, &s, &m);
            const float d1 = d * (float)s, m1 = min * (float)m;
            or_get_scale_min_k4(is + 1, sc, &s, &m);
            const float d2 = d * (float)s, m2 = min * (float)m;
            for (int l = 0; l < 32; l++) *y++ = d1 * (float)(q[l] & 0xF) - m1;
            for (int l = 0; l < 32; l++) *y++ = d2 * (float)(q[l] >> 4) - m2;
            q += 32;
            is += 2;
        }
    }
}

/* Q5_K: half d | half dmin | u8 scales[12] | u8 qh[32] | u8 qs[128]   (176 bytes) */
void or_dequant_q5k(const uint8_t *blk, int64_t nblocks, float *y) {
    for (int64_t b = 0; b < nblocks; b++, blk += 176) {
        const float d = ld_f16(blk), min = ld_f16(blk + 2);
        const uint8_t *sc = blk + 4, *qh = blk + 16, *ql = blk + 48;
        int is = 0;
        uint8_t u1 = 1, u2 = 2;
        for (int j = 0; j < QK_K; j += 64) {
            uint8_t s, m;
            or_get_scale_min_k4(is + 0, sc, &s, &m);
            const float d1 = d * (float)s, m1 = min * (float)m;
            or_get_scale_min_k4(is + 1, sc, &s, &m);
            const float d2 = d * (float)s, m2 = min * (float)m;
            for (int l = 0; l < 32; l++) *y++ = d1 * (float)((ql[l] & 0xF) + ((qh[l] & u1) ? 16 : 0)) - m1;
            for (int l = 0; l < 32; l++) *y++ = d2 * (float)((ql[l] >> 4) + ((qh[l] & u2) ? 16 : 0)) - m2;
            ql += 32;
            is += 2;
            u1 <<= 2;
            u2 <<= 2;
        }
    }
}

/* Q6_K: u8 ql[128] | u8 qh[64] | i8 scales[16] | half d   (210 bytes) */
void or_dequant_q6k(const uint8_t *blk, int64_t nblocks, float *y) {
    for (int64_t b = 0; b < nblocks; b++, blk += 210) {
        const float d = ld_f16(blk + 208);
        const uint8_t *ql = blk, *qh = blk + 128;
        const int8_t *sc = (const int8_t *)(blk + 192);
        for (int n = 0; n < QK_K; n += 128) {
            for (int l = 0; l < 32; l++) {
                int is = l / 16;
                const int q1 = (int)((ql[l + 0] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
                const int q2 = (int)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                const int q3 = (int)((ql[l + 0] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                const int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                y[l + 0] = d * (float)sc[is + 0] * (float)q1;
                y[l + 32] = d * (float)sc[is + 2] * (float)q2;
                y[l + 64] = d * (float)sc[is + 4] * (float)q3;
                y[l + 96] = d * (float)sc[is + 6] * (float)q4;
            }
            y += 128;
            ql += 64;
            qh += 32;
            sc += 8;
        }
    }
}

/* Q8_0: half d | i8 qs[32]   (34 bytes, 32 elements) */
void or_dequant_q80(const uint8_t *blk, int64_t nblocks, float *y) {
    for (int64_t b = 0; b < nblocks; b++, blk += 34) {
        const float d = ld_f16(blk);
        const int8_t *q = (const int8_t *)(blk + 2);
        for (int l = 0; l < 32; l++) *y++ = d * (float)q[l];
    }
}

/* format ids shared with the python side: 0=F32 (raw), 12=Q4_K, 13=Q5_K, 14=Q6_K, 8=Q8_0
 * (the GGML type ids) */
int64_t or_block_bytes(int fmt) {
    switch (fmt) {
    case 12: return 144;
    case 13: return 176;
    case 14: return 210;
    case 8: return 34;
    default: return 0;
    }
}
int64_t or_block_elems(int fmt) { return fmt == 8 ? 32 : QK_K; }

int or_dequant(int fmt, const uint8_t *blk, int64_t nblocks, float *y) {
    switch (fmt) {
    case 12: or_dequant_q4k(blk, nblocks, y); return 0;
    case 13: or_dequant_q5k(blk, nblocks, y); return 0;
    case 14: or_dequant_q6k(blk, nblocks, y); return 0;
    case 8: or_dequant_q80(blk, nblocks, y); return 0;
    default: return -1;
    }
}

/* Dequantise rows [r0, r1) of a row-major [N][K] block matrix (threads over rows). */
int or_dequant_rows(int fmt, const uint8_t *w, int64_t K, int64_t r0, int64_t r1, float *y) {
    const int64_t bb = or_block_bytes(fmt), be = or_block_elems(fmt);
    if (!bb || K % be) return -1;
    const int64_t nb = K / be, row_bytes = nb * bb;
#pragma omp parallel for schedule(static)
    for (int64_t r = r0; r < r1; r++) or_dequant(fmt, w + r * row_bytes, nb, y + (r - r0) * K);
    return 0;
}

/* y[m][n] = sum_k x[m][k] * deq(W)[n][k], f32 dequant values, f64 accumulation.
 * rows of W dequantised on the fly (threads over n). */
int or_qmatmul(int fmt, const uint8_t *w, int64_t N, int64_t K, const float *x, int64_t M, float *y) {
    const int64_t bb = or_block_bytes(fmt), be = or_block_elems(fmt);
    if (!bb || K % be) return -1;
    const int64_t nb = K / be, row_bytes = nb * bb;
#pragma omp parallel
    {
        float *row = (float *)malloc(sizeof(float) * K);
#pragma omp for schedule(static)
        for (int64_t n = 0; n < N; n++) {
            or_dequant(fmt, w + n * row_bytes, nb, row);
            for (int64_t m = 0; m < M; m++) {
                const float *xm = x + m * K;
                double acc = 0.0;
                for (int64_t k = 0; k < K; k++) acc += (double)xm[k] * (double)row[k];
                y[m * N + n] = (float)acc;
            }
        }
        free(row);
    }
    return 0;
}

/* ------------------------------------------------------------------ */
/* Synthetic weights (seeded, deterministic; equals the GPU generator)   */
/* ------------------------------------------------------------------ */
uint64_t or_mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
/* Irwin-Hall(4) approximation of N(0, std): mult = std*sqrt(3)/65536 (precomputed in f64 -> f32). */
float or_synth_value(uint64_t seed, uint64_t idx, float mult) {
    uint64_t h = or_mix64(seed + (idx + 1ull) * 0x9E3779B97F4A7C15ull);
    int32_t s = (int32_t)(h & 0xffff) + (int32_t)((h >> 16) & 0xffff) + (int32_t)((h >> 32) & 0xffff) +
                (int32_t)(h >> 48) - 131070;
    return (float)s * mult;
}
void or_synth_f32(uint64_t seed, int64_t n, float mult, float *y) {
    for (int64_t i = 0; i < n; i++) y[i] = or_synth_value(seed, (uint64_t)i, mult);
}

static float clampf(float v, float lo, float hi) { return v < lo ? lo : (v > hi ? hi : v); }

static void pack_scale_min_k4(const uint8_t *sc, const uint8_t *mn, uint8_t *q) {
    for (int j = 0; j < 4; j++) {
        q[j] = (uint8_t)(sc[j] | ((sc[j + 4] >> 4) << 6));
        q[j + 4] = (uint8_t)(mn[j] | ((mn[j + 4] >> 4) << 6));
        q[j + 8] = (uint8_t)((sc[j + 4] & 0xF) | ((mn[j + 4] & 0xF) << 4));
    }
}

/* Q4_K (nmax=15) and Q5_K (nmax=31) share the asymmetric 8x32 quantiser. */
static void quant_kasym(const float *x, int nmax, uint8_t *sc6, uint8_t *mn6, float *dd, float *dm, uint8_t *q) {
    float scale[8], minv[8], max_scale = 0.f, max_min = 0.f;
    for (int j = 0; j < 8; j++) {
        float mn = x[32 * j], mx = x[32 * j];
        for (int l = 1; l < 32; l++) {
            float v = x[32 * j + l];
            if (v < mn) mn = v;
            if (v > mx) mx = v;
        }
        if (mn > 0.f) mn = 0.f;
        scale[j] = (mx - mn) / (float)nmax;
        minv[j] = -mn;
        if (scale[j] > max_scale) max_scale = scale[j];
        if (minv[j] > max_min) max_min = minv[j];
    }
    const float df = or_f16_to_f32(or_f32_to_f16(max_scale / 63.f));
    const float dminf = or_f16_to_f32(or_f32_to_f16(max_min / 63.f));
    for (int j = 0; j < 8; j++) {
        sc6[j] = df > 0.f ? (uint8_t)clampf(rintf(scale[j] / df), 0.f, 63.f) : 0;
        mn6[j] = dminf > 0.f ? (uint8_t)clampf(rintf(minv[j] / dminf), 0.f, 63.f) : 0;
        const float d1 = df * (float)sc6[j], m1 = dminf * (float)mn6[j];
        for (int l = 0; l < 32; l++) {
            float v = x[32 * j + l];
            q[32 * j + l] = d1 > 0.f ? (uint8_t)clampf(rintf((v + m1) / d1), 0.f, (float)nmax) : 0;
        }
    }
    *dd = df;
    *dm = dminf;
}

void or_quantize_q4k(const float *x, int64_t nblocks, uint8_t *out) {
    for (int64_t b = 0; b < nblocks; b++, x += QK_K, out += 144) {
        uint8_t sc6[8], mn6[8], q[QK_K];
        float df, dm;
        quant_kasym(x, 15, sc6, mn6, &df, &dm, q);
        st_f16(out, df);
        st_f16(out + 2, dm);
        pack_scale_min_k4(sc6, mn6, out + 4);
        for (int j = 0; j < 4; j++)
            for (int l = 0; l < 32; l++) out[16 + 32 * j + l] = (uint8_t)(q[64 * j + l] | (q[64 * j + 32 + l] << 4));
    }
}

void or_quantize_q5k(const float *x, int64_t nblocks, uint8_t *out) {
    for (int64_t b = 0; b < nblocks; b++, x += QK_K, out += 176) {
        uint8_t sc6[8], mn6[8], q[QK_K];
        float df, dm;
        quant_kasym(x, 31, sc6, mn6, &df, &dm, q);
        st_f16(out, df);
        st_f16(out + 2, dm);
        pack_scale_min_k4(sc6, mn6, out + 4);
        uint8_t *qh = out + 16, *ql = out + 48;
        memset(qh, 0, 32);
        for (int j = 0; j < 4; j++)
            for (int l = 0; l < 32; l++) {
                const uint8_t lo = q[64 * j + l], hi = q[64 * j + 32 + l];
                ql[32 * j + l] = (uint8_t)((lo & 0xF) | ((hi & 0xF) << 4));
                qh[l] |= (uint8_t)(((lo >> 4) & 1) << (2 * j));
                qh[l] |= (uint8_t)(((hi >> 4) & 1) << (2 * j + 1));
            }
    }
}

void or_quantize_q6k(const float *x, int64_t nblocks, uint8_t *out) {
    for (int64_t b = 0; b < nblocks; b++, x += QK_K, out += 210) {
        float scale[16], max_scale = 0.f;
        for (int j = 0; j < 16; j++) {
            float amax = 0.f;
            for (int l = 0; l < 16; l++) {
                float a = fabsf(x[16 * j + l]);
                if (a > amax) amax = a;
            }
            scale[j] = amax / 31.f;
            if (scale[j] > max_scale) max_scale = scale[j];
        }
        const float df = or_f16_to_f32(or_f32_to_f16(max_scale / 127.f));
        uint8_t q[QK_K];
        int8_t *sc = (int8_t *)(out + 192);
        for (int j = 0; j < 16; j++) {
            int s = df > 0.f ? (int)clampf(rintf(scale[j] / df), 0.f, 127.f) : 0;
            sc[j] = (int8_t)s;
            const float ds = df * (float)s;
            for (int l = 0; l < 16; l++) {
                float v = x[16 * j + l];
                int qi = ds > 0.f ? (int)clampf(rintf(v / ds), -32.f, 31.f) : 0;
                q[16 * j + l] = (uint8_t)(qi + 32);
            }
        }
        uint8_t *ql = out, *qh = out + 128;
        for (int h = 0; h < 2; h++)
            for (int l = 0; l < 32; l++) {
                const uint8_t q1 = q[128 * h + l], q2 = q[128 * h + 32 + l], q3 = q[128 * h + 64 + l],
                              q4 = q[128 * h + 96 + l];
                ql[64 * h + l] = (uint8_t)((q1 & 0xF) | ((q3 & 0xF) << 4));
                ql[64 * h + 32 + l] = (uint8_t)((q2 & 0xF) | ((q4 & 0xF) << 4));
                qh[32 * h + l] = (uint8_t)((q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6));
            }
        st_f16(out + 208, df);
    }
}

void or_quantize_q80(const float *x, int64_t nblocks, uint8_t *out) {
    for (int64_t b = 0; b < nblocks; b++, x += 32, out += 34) {
        float amax = 0.f;
        for (int l = 0; l < 32; l++) {
            float a = fabsf(x[l]);
            if (a > amax) amax = a;
        }
        const float df = or_f16_to_f32(or_f32_to_f16(amax / 127.f));
        st_f16(out, df);
        int8_t *q = (int8_t *)(out + 2);
        for (int l = 0; l < 32; l++) q[l] = df > 0.f ? (int8_t)clampf(rintf(x[l] / df), -127.f, 127.f) : 0;
    }
}

int or_quantize(int fmt, const float *x, int64_t nblocks, uint8_t *out) {
    switch (fmt) {
    case 12: or_quantize_q4k(x, nblocks, out); return 0;
    case 13: or_quantize_q5k(x, nblocks, out); return 0;
    case 14: or_quantize_q6k(x, nblocks, out); return 0;
    case 8: or_quantize_q80(x, nblocks, out); return 0;
    default: return -1;
    }
}

/* Synthesise a [rows][K] tensor of N(0,std)-like values with `seed` and quantise
 * it block by block (threads over rows; per-element values depend only on
 * (seed, flat index), so the result is thread-count independent). */
int or_synth_quant(int fmt, uint64_t seed, int64_t rows, int64_t K, float mult, uint8_t *out) {
    const int64_t bb = or_block_bytes(fmt), be = or_block_elems(fmt);
    if (!bb || K % be) return -1;
    const int64_t nb = K / be;
#pragma omp parallel
    {
        float *row = (float *)malloc(sizeof(float) * K);
#pragma omp for schedule(static)
        for (int64_t r = 0; r < rows; r++) {
            for (int64_t k = 0; k < K; k++) row[k] = or_synth_value(seed, (uint64_t)(r * K + k), mult);
            or_quantize(fmt, row, nb, out + r * nb * bb);
        }
        free(row);
    }
    return 0;
}

/* ------------------------------------------------------------------ */
/* Sampling / acceptance primitives: sequential f32, reference order    */
/* ------------------------------------------------------------------ */
/* first-max argmax fold from (0, -inf) with strict '>' (NaN never wins,
 * an all -inf/NaN row gives 0): eagle.rs:626-637, tokens.rs:26-35 */
int64_t or_argmax_fold(const float *v, int64_t n) {
    int64_t bi = 0;
    float bv = -INFINITY;
    for (int64_t i = 0; i < n; i++)
        if (v[i] > bv) {
            bi = i;
            bv = v[i];
        }
    return bi;
}

/* softmax_with_temperature (tokens.rs:15-55).  Returns 0, or -1 on the
 * reference's error cases (empty, bad temperature, non-positive/non-finite sum). */
int or_softmax_t(const float *logits, int64_t n, float temperature, float *out) {
    if (n <= 0) return -1;
    if (!isfinite(temperature) || temperature < 0.f) return -1;
    if (temperature == 0.f) {
        int64_t am = or_argmax_fold(logits, n);
        for (int64_t i = 0; i < n; i++) out[i] = 0.f;
        out[am] = 1.f;
        return 0;
    }
    const float inv_t = 1.0f / temperature;
    float mx = -INFINITY;
    for (int64_t i = 0; i < n; i++) mx = fmaxf(mx, logits[i]); /* f32::max ignores NaN */
    float sum = 0.f;
    for (int64_t i = 0; i < n; i++) {
        out[i] = expf((logits[i] - mx) * inv_t);
        sum += out[i];
    }
    if (sum <= 0.f || !isfinite(sum)) return -1;
    for (int64_t i = 0; i < n; i++) out[i] /= sum;
    return 0;
}

/* sample_from_distribution with an explicit uniform u in [0,1) (tokens.rs:99-120). */
int64_t or_sample_u(const float *probs, int64_t n, float u) {
    if (n <= 0) return -1;
    float sum = 0.f;
    for (int64_t i = 0; i < n; i++) sum += probs[i];
    if (!isfinite(sum) || sum <= 0.f) return -1;
    const float uu = u * sum;
    float acc = 0.f;
    for (int64_t i = 0; i < n; i++) {
        const float p = probs[i];
        if (!isfinite(p) || p < 0.f) return -2;
        acc += p;
        if (uu < acc) return i;
    }
    return n - 1;
}

/* modified_rejection_step (vanilla.rs:59-73): 1 = Accepted, 0 = Rejected. */
int or_rejection_step(float q_draft, float p_target, float u) {
    if (q_draft <= 0.f) return 1;
    float ratio = p_target / q_draft;
    if (ratio > 1.f) ratio = 1.f;
    return u <= ratio ? 1 : 0;
}

/* adjusted_distribution (vanilla.rs:83-106): max(0, p-q) / sum.  -1 on zero/non-finite mass. */
int or_adjusted(const float *p, const float *q, int64_t n, float *out) {
    float sum = 0.f;
    for (int64_t i = 0; i < n; i++) {
        float d = p[i] - q[i];
        out[i] = d > 0.f ? d : 0.f; /* f32::max(0.0) */
        sum += out[i];
    }
    if (sum <= 0.f || !isfinite(sum)) return -1;
    for (int64_t i = 0; i < n; i++) out[i] /= sum;
    return 0;
}

/* ------------------------------------------------------------------ */
/* RoPE tables (quantized_llama_local.rs:189-205): theta_i = 1/base^(i/d) */
/* for even i (f32 powf), table[t][i/2] = cos/sin(t * theta) in f32.      */
/* ------------------------------------------------------------------ */
void or_rope_tables(int64_t dim, float base, int64_t ctx, float *cos_t, float *sin_t) {
    const int64_t h = dim / 2;
    float *theta = (float *)malloc(sizeof(float) * h);
    for (int64_t i = 0; i < h; i++) theta[i] = 1.0f / powf(base, (float)(2 * i) / (float)dim);
    for (int64_t t = 0; t < ctx; t++)
        for (int64_t i = 0; i < h; i++) {
            const float a = (float)t * theta[i];
            cos_t[t * h + i] = cosf(a);
            sin_t[t * h + i] = sinf(a);
        }
    free(theta);
}
