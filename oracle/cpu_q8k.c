/*
 * CPU baseline of the verify step: TEST AND MEASUREMENT INFRASTRUCTURE ONLY
 * (bench.py's cpu_baseline leg and tests/ load it; the product library never
 * does).
 *
 * A C restatement of the CPU algorithm the reference's quantised matmul runs
 * when candle executes on the CPU (`QMatMul::forward`,
 * crates/speculate/src/model/quantized_llama_local.rs:47-49, 73-90, 135,
 * 317; candle-core 0.8.4's k-quants, external and not vendored, which follow
 * the published ggml k-quants dot products):
 *   - every activation row is quantised to Q8_K blocks of 256: the element of
 *     largest magnitude, max, sets iscale = -128 / max; q = nearest integer of
 *     iscale * x, capped at 127; d = 1 / iscale; bsums[16] = the sums of q
 *     over groups of 16 (ggml's quantize_row_q8_K);
 *   - each output is a sum over superblocks of integer dot products of the
 *     weight codes with those int8 values, scaled in f32:
 *       Q4_K: y += d_x * (d * sum_j sc_j * sum(q4 * q8) - dmin * sum_j m_j * bsum_j)
 *       Q6_K: y += d_x * d * sum_g sc_g * sum((q6 - 32) * q8)
 *     (ggml's vec_dot_q4_K_q8_K / vec_dot_q6_K_q8_K);
 *   - threads over output rows (OpenMP here, rayon there), SIMD over the 256
 *     elements (AVX2 byte-multiply-add, as ggml's and candle's x86 paths),
 *     with a plain C version of the same integer sums where AVX2 is missing.
 * Also the f32 attention of one layer for M new rows over the cached rows
 * (scores, masked softmax with expf, weighted V sum), threads over heads.
 *
 * The integer sums are exact; only the f32 scaling and the order of the
 * per-superblock f32 accumulation can differ from candle's, which does not
 * matter for a timing baseline.  tests/test_cpu_baseline.py pins the
 * quantiser and both dot products against exact restatements.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#include <immintrin.h>

#define QK_K 256

typedef struct {
    float d;
    int8_t qs[QK_K];
    int16_t bsums[QK_K / 16];
} or_block_q8k;

float or_f16_to_f32(uint16_t h);

static inline float f16_at(const uint8_t *p) {
    uint16_t h;
    memcpy(&h, p, 2);
    return or_f16_to_f32(h);
}

/* ggml's nearest_int: round half away from zero via the 1.5*2^23 trick */
static inline int nearest_int(float fval) {
    float val = fval + 12582912.f;
    int i;
    memcpy(&i, &val, sizeof(int));
    return (i & 0x007fffff) - 0x00400000;
}

void or_quantize_row_q8k(const float *x, int64_t K, or_block_q8k *y) {
    const int64_t nb = K / QK_K;
    for (int64_t i = 0; i < nb; i++) {
        const float *xb = x + i * QK_K;
        float max = 0, amax = 0;
        for (int j = 0; j < QK_K; j++) {
            const float ax = fabsf(xb[j]);
            if (ax > amax) {
                amax = ax;
                max = xb[j];
            }
        }
        if (!amax) {
            y[i].d = 0;
            memset(y[i].qs, 0, QK_K);
            memset(y[i].bsums, 0, sizeof y[i].bsums);
            continue;
        }
        const float iscale = -128.f / max;
        for (int j = 0; j < QK_K; j++) {
            const int v = nearest_int(iscale * xb[j]);
            y[i].qs[j] = (int8_t)(v < 127 ? v : 127);
        }
        for (int j = 0; j < QK_K / 16; j++) {
            int sum = 0;
            for (int ii = 0; ii < 16; ii++) sum += y[i].qs[j * 16 + ii];
            y[i].bsums[j] = (int16_t)sum;
        }
        y[i].d = 1 / iscale;
    }
}

/* 6-bit scales and mins of the 8 sub-blocks (get_scale_min_k4) */
static inline void q4k_scales(const uint8_t *s, uint8_t *sc, uint8_t *mn) {
    for (int j = 0; j < 4; j++) {
        sc[j] = s[j] & 63;
        mn[j] = s[j + 4] & 63;
    }
    for (int j = 4; j < 8; j++) {
        sc[j] = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
        mn[j] = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

/* Q4_K block: d f16, dmin f16, scales[12], qs[128] (144 bytes); element
 * 64 j + l is the low nibble of qs[32 j + l], 64 j + 32 + l its high nibble */
static float dot_q4k_q8k_c(const uint8_t *w, const or_block_q8k *y, int64_t nb) {
    float sumf = 0;
    for (int64_t i = 0; i < nb; i++) {
        const uint8_t *b = w + i * 144;
        uint8_t sc[8], mn[8];
        q4k_scales(b + 4, sc, mn);
        const uint8_t *qs = b + 16;
        const int8_t *q8 = y[i].qs;
        int32_t sumi = 0, summ = 0;
        for (int j = 0; j < 4; j++) {
            int32_t lo = 0, hi = 0;
            for (int l = 0; l < 32; l++) {
                lo += (qs[32 * j + l] & 0xF) * q8[64 * j + l];
                hi += (qs[32 * j + l] >> 4) * q8[64 * j + 32 + l];
            }
            sumi += sc[2 * j] * lo + sc[2 * j + 1] * hi;
        }
        for (int j = 0; j < 8; j++) summ += mn[j] * (y[i].bsums[2 * j] + y[i].bsums[2 * j + 1]);
        sumf += y[i].d * (f16_at(b) * (float)sumi - f16_at(b + 2) * (float)summ);
    }
    return sumf;
}

/* Q6_K block: ql[128], qh[64], scales[16] (int8), d f16 (210 bytes) */
static inline int q6_at(const uint8_t *ql, const uint8_t *qh, int e) {
    const int h = e >> 7, r = e & 127, l = r & 31, quarter = r >> 5;
    const uint8_t *L = ql + 64 * h, *H = qh + 32 * h;
    const int low = quarter == 0 ? (L[l] & 0xF) : quarter == 1 ? (L[l + 32] & 0xF) : quarter == 2 ? (L[l] >> 4) : (L[l + 32] >> 4);
    const int high = (H[l] >> (2 * quarter)) & 3;
    return (low | (high << 4)) - 32;
}
static float dot_q6k_q8k_c(const uint8_t *w, const or_block_q8k *y, int64_t nb) {
    float sumf = 0;
    for (int64_t i = 0; i < nb; i++) {
        const uint8_t *b = w + i * 210;
        const int8_t *sc = (const int8_t *)(b + 192);
        int32_t sumi = 0;
        for (int g = 0; g < 16; g++) {
            int32_t s = 0;
            for (int ii = 0; ii < 16; ii++) s += q6_at(b, b + 128, 16 * g + ii) * y[i].qs[16 * g + ii];
            sumi += sc[g] * s;
        }
        sumf += y[i].d * f16_at(b + 208) * (float)sumi;
    }
    return sumf;
}

__attribute__((target("avx2,fma"))) static inline int32_t hsum_i32_8(__m256i v) {
    const __m128i s = _mm_add_epi32(_mm256_castsi256_si128(v), _mm256_extracti128_si256(v, 1));
    const __m128i s2 = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0x4E));
    return _mm_cvtsi128_si32(_mm_add_epi32(s2, _mm_shuffle_epi32(s2, 0xB1)));
}

__attribute__((target("avx2,fma"))) static float dot_q4k_q8k_avx2(const uint8_t *w, const or_block_q8k *y,
                                                                  int64_t nb) {
    const __m256i m4 = _mm256_set1_epi8(0xF);
    float sumf = 0;
    for (int64_t i = 0; i < nb; i++) {
        const uint8_t *b = w + i * 144;
        uint8_t sc[8], mn[8];
        q4k_scales(b + 4, sc, mn);
        const uint8_t *qs = b + 16;
        const int8_t *q8 = y[i].qs;
        __m256i acc = _mm256_setzero_si256();
        for (int j = 0; j < 4; j++) {
            const __m256i q4 = _mm256_loadu_si256((const __m256i *)(qs + 32 * j));
            const __m256i lo = _mm256_and_si256(q4, m4), hi = _mm256_and_si256(_mm256_srli_epi16(q4, 4), m4);
            const __m256i plo = _mm256_maddubs_epi16(lo, _mm256_loadu_si256((const __m256i *)(q8 + 64 * j)));
            const __m256i phi = _mm256_maddubs_epi16(hi, _mm256_loadu_si256((const __m256i *)(q8 + 64 * j + 32)));
            acc = _mm256_add_epi32(acc, _mm256_madd_epi16(plo, _mm256_set1_epi16(sc[2 * j])));
            acc = _mm256_add_epi32(acc, _mm256_madd_epi16(phi, _mm256_set1_epi16(sc[2 * j + 1])));
        }
        int32_t summ = 0;
        for (int j = 0; j < 8; j++) summ += mn[j] * (y[i].bsums[2 * j] + y[i].bsums[2 * j + 1]);
        sumf += y[i].d * (f16_at(b) * (float)hsum_i32_8(acc) - f16_at(b + 2) * (float)summ);
    }
    return sumf;
}

__attribute__((target("avx2,fma"))) static float dot_q6k_q8k_avx2(const uint8_t *w, const or_block_q8k *y,
                                                                  int64_t nb) {
    const __m256i m4 = _mm256_set1_epi8(0xF), m3 = _mm256_set1_epi8(3);
    float sumf = 0;
    for (int64_t i = 0; i < nb; i++) {
        const uint8_t *b = w + i * 210;
        const int8_t *sc = (const int8_t *)(b + 192);
        const int8_t *q8 = y[i].qs;
        __m256i acc = _mm256_setzero_si256();
        int32_t off = 0;  // 32 * sum_g sc_g * bsum_g
        for (int g = 0; g < 16; g++) off += sc[g] * y[i].bsums[g];
        for (int h = 0; h < 2; h++) {
            const __m256i L0 = _mm256_loadu_si256((const __m256i *)(b + 64 * h));
            const __m256i L1 = _mm256_loadu_si256((const __m256i *)(b + 64 * h + 32));
            const __m256i H = _mm256_loadu_si256((const __m256i *)(b + 128 + 32 * h));
            // the four 32-element quarters of this half, unsigned 0..63
            __m256i q[4];
            q[0] = _mm256_or_si256(_mm256_and_si256(L0, m4), _mm256_slli_epi16(_mm256_and_si256(H, m3), 4));
            q[1] = _mm256_or_si256(_mm256_and_si256(L1, m4),
                                   _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(H, 2), m3), 4));
            q[2] = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(L0, 4), m4),
                                   _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(H, 4), m3), 4));
            q[3] = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(L1, 4), m4),
                                   _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(H, 6), m3), 4));
            for (int k = 0; k < 4; k++) {
                const int e0 = 128 * h + 32 * k;  // first element; groups e0/16 and e0/16 + 1
                const __m256i p = _mm256_maddubs_epi16(q[k], _mm256_loadu_si256((const __m256i *)(q8 + e0)));
                const __m256i s = _mm256_set_m128i(_mm_set1_epi16(sc[e0 / 16 + 1]), _mm_set1_epi16(sc[e0 / 16]));
                acc = _mm256_add_epi32(acc, _mm256_madd_epi16(p, s));
            }
        }
        sumf += y[i].d * f16_at(b + 208) * (float)(hsum_i32_8(acc) - 32 * off);
    }
    return sumf;
}

static int have_avx2(void) {
    static int v = -1;
    if (v < 0) v = __builtin_cpu_supports("avx2") ? 1 : 0;
    return v;
}

/* one dot product of a weight row with a Q8_K row; simd = 0 forces plain C */
float or_dot_q8k(int fmt, const uint8_t *wrow, const or_block_q8k *y, int64_t nb, int simd) {
    const int v = simd && have_avx2();
    if (fmt == 12) return v ? dot_q4k_q8k_avx2(wrow, y, nb) : dot_q4k_q8k_c(wrow, y, nb);
    if (fmt == 14) return v ? dot_q6k_q8k_avx2(wrow, y, nb) : dot_q6k_q8k_c(wrow, y, nb);
    return NAN;
}

/* y[m][n] = dot(W row n, Q8_K(x row m)); xq: M * K / 256 blocks of scratch.
 * Threads over the output rows. */
int or_cpu_qmatmul_q8k(int fmt, const uint8_t *w, int64_t N, int64_t K, const float *x, int64_t M, float *y,
                       or_block_q8k *xq, int simd) {
    if ((fmt != 12 && fmt != 14) || K % QK_K) return -1;
    const int64_t nb = K / QK_K, rb = fmt == 12 ? nb * 144 : nb * 210;
    for (int64_t m = 0; m < M; m++) or_quantize_row_q8k(x + m * K, K, xq + m * nb);
#pragma omp parallel for schedule(static)
    for (int64_t n = 0; n < N; n++)
        for (int64_t m = 0; m < M; m++) y[m * N + n] = or_dot_q8k(fmt, w + n * rb, xq + m * nb, nb, simd);
    return 0;
}

/* One layer's attention for M new rows (positions P .. P+M-1) over the cached
 * rows: q [M][n_heads][hd], k/v caches [n_kv][T][hd] with T = P + M rows
 * filled, out [M][n_heads][hd].  Query i sees keys < P + i + 1 (a causal
 * chain).  Threads over heads. */
int or_cpu_attention(const float *q, const float *kc, const float *vc, int64_t M, int64_t P, int n_heads, int n_kv,
                     int hd, float *out) {
    const int64_t T = P + M;
    const int rep = n_heads / n_kv;
    const float scale = 1.0f / sqrtf((float)hd);
#pragma omp parallel for schedule(static)
    for (int h = 0; h < n_heads; h++) {
        const float *K = kc + (int64_t)(h / rep) * T * hd, *V = vc + (int64_t)(h / rep) * T * hd;
        float *sc = (float *)__builtin_alloca((size_t)T * sizeof(float));
        for (int64_t i = 0; i < M; i++) {
            const float *qi = q + (i * n_heads + h) * hd;
            float *o = out + (i * n_heads + h) * hd;
            const int64_t nk = P + i + 1;
            float mx = -INFINITY;
            for (int64_t j = 0; j < nk; j++) {
                float a = 0.f;
                for (int d = 0; d < hd; d++) a += qi[d] * K[j * hd + d];
                sc[j] = a * scale;
                if (sc[j] > mx) mx = sc[j];
            }
            float sum = 0.f;
            for (int64_t j = 0; j < nk; j++) {
                sc[j] = expf(sc[j] - mx);
                sum += sc[j];
            }
            for (int d = 0; d < hd; d++) o[d] = 0.f;
            for (int64_t j = 0; j < nk; j++) {
                const float p = sc[j] / sum;
                for (int d = 0; d < hd; d++) o[d] += p * V[j * hd + d];
            }
        }
    }
    return 0;
}
