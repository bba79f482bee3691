// Embedding gather, RMSNorm, device-layout dequantisation, KV compaction.
//
//  * embedding: Embedding::forward over the f32-dequantised token table
//    (crates/speculate/src/model/quantized_llama_local.rs:242-243, 380, 419);
//    rows are dequantised on the fly from the quantised table with the exact
//    f32 expressions, so no 2 GB f32 copy of the table is kept.
//  * rms_norm: RmsNorm::forward (:385, 389, 398): x / sqrt(mean(x^2) + eps) * w.
//    Writes the fp16 fragment-layout operand of the next matmul, and optionally
//    the f32 row (the final hidden state returned by tree_logits_keep_kv).
//  * keep_kv_tail: LayerWeights::keep_kv_indices (:177-186) for the only index
//    lists the decoder builds, [0..P) ++ [P + ti] (quantized_llama.rs:426-432):
//    the prefix never moves, the accepted tree rows are gathered to [P, P+n).
#include "sd_common.hpp"
#include "sd_kernels_elem.hpp"

namespace sd {

#pragma clang fp contract(off)

__device__ inline float ld_h(const uint8_t *p) { return h2f((uint16_t)(p[0] | (p[1] << 8))); }

// element e of a device-layout row (exact f32, two roundings per expression)
__device__ float deq_elem(int fmt, const uint8_t *row, int nsb, int e) {
    if (fmt == F32) return ((const float *)row)[e];
    if (fmt == Q8_0) {
        const int nb = nsb * 8, b = e >> 5, l = e & 31;
        const float d = ld_h(row + 32 * nb + 2 * b);
        return d * (float)(int8_t)row[32 * b + l];
    }
    const int sb = e >> 8, r = e & 255;
    if (fmt == Q4_K || fmt == Q5_K) {
        const uint8_t *b = row + (int64_t)sb * (fmt == Q4_K ? 144 : 176);
        const float d = ld_h(b), mn = ld_h(b + 2);
        const uint8_t *sc = b + 4;
        const int part = r >> 5, j = r >> 6, hi = (r >> 5) & 1, l = r & 31;
        int s, m;
        if (part < 4) {
            s = sc[part] & 63;
            m = sc[part + 4] & 63;
        } else {
            s = (sc[part + 4] & 0xF) | ((sc[part - 4] >> 6) << 4);
            m = (sc[part + 4] >> 4) | ((sc[part] >> 6) << 4);
        }
        const float d1 = d * (float)s, m1 = mn * (float)m;
        int q;
        if (fmt == Q4_K) {
            const uint8_t qb = b[16 + 32 * j + l];
            q = hi ? (qb >> 4) : (qb & 0xF);
        } else {
            const uint8_t qb = b[48 + 32 * j + l], qh = b[16 + l];
            q = (hi ? (qb >> 4) : (qb & 0xF)) + (((qh >> (2 * j + hi)) & 1) ? 16 : 0);
        }
        return d1 * (float)q - m1;
    }
    // Q6_K planar
    const float d = ld_h(row + (int64_t)nsb * 208 + 2 * sb);
    const int h = r >> 7, qd = (r >> 5) & 3, l = r & 31;
    const uint8_t qlb = row[(int64_t)sb * 128 + 64 * h + 32 * (qd & 1) + l];
    const uint8_t qhb = row[(int64_t)nsb * 128 + (int64_t)sb * 64 + 32 * h + l];
    const int8_t sc = (int8_t)row[(int64_t)nsb * 192 + (int64_t)sb * 16 + 8 * h + l / 16 + 2 * qd];
    const int nib = qd < 2 ? (qlb & 0xF) : (qlb >> 4);
    const int q = (nib | (((qhb >> (2 * qd)) & 3) << 4)) - 32;
    return d * (float)sc * (float)q;
}

__global__ void k_dequant_dev(int fmt, const uint8_t *w, int64_t rows, int K, int64_t stride, float *y) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * K) return;
    const int64_t r = i / K;
    const int e = (int)(i % K);
    y[i] = deq_elem(fmt, w + r * stride, K / 256, e);
}

// h[m][k] = table[ids[m]][k]
__global__ void k_embed(int fmt, const uint8_t *table, int64_t stride, int K, const int *ids, float *h) {
    const int m = blockIdx.y;
    const int k = blockIdx.x * blockDim.x + threadIdx.x;
    if (k >= K) return;
    h[(int64_t)m * K + k] = deq_elem(fmt, table + (int64_t)ids[m] * stride, K / 256, k);
}

// one workgroup (256 threads) per row
__global__ __launch_bounds__(256) void k_rmsnorm(const float *x, const float *w, int K, float eps, uint16_t *out16,
                                                 int ld16, float *out32) {
    const int m = blockIdx.x;
    const float *row = x + (int64_t)m * K;
    float ss = 0.f;
    for (int k = threadIdx.x; k < K; k += 256) {
        const float v = row[k];
        ss += v * v;
    }
    __shared__ float red[256];
    red[threadIdx.x] = ss;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if (threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
        __syncthreads();
    }
    const float mrms = sqrtf(red[0] / (float)K + eps);
    for (int k = threadIdx.x; k < K; k += 256) {
        const float y = row[k] / mrms * w[k];
        if (out16) out16[(int64_t)m * ld16 + frag_index(k)] = f2h(y);
        if (out32) out32[(int64_t)m * K + k] = y;
    }
}

// f32 rows -> fp16 fragment layout (hidden states handed to apply_lm_head)
__global__ void k_to_frag16(const float *x, int K, uint16_t *out16, int ld16) {
    const int m = blockIdx.y;
    const int k = blockIdx.x * blockDim.x + threadIdx.x;
    if (k >= K) return;
    out16[(int64_t)m * ld16 + frag_index(k)] = f2h(x[(int64_t)m * K + k]);
}

// ---- argmax over per-workgroup partials (first max wins, NaN/-inf skipped) ----
// grid M, block 256
__global__ __launch_bounds__(256) void k_argmax_reduce(const float *pv, const int *pi, int nwg, int *out) {
    const int m = blockIdx.x;
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int w = threadIdx.x; w < nwg; w += 256) {
        const float v = pv[(int64_t)m * nwg + w];
        const int i = pi[(int64_t)m * nwg + w];
        if (i != 0x7fffffff && (v > bv || (v == bv && i < bi) || bi == 0x7fffffff)) {
            bv = v;
            bi = i;
        }
    }
    __shared__ float sv[256];
    __shared__ int si[256];
    sv[threadIdx.x] = bv;
    si[threadIdx.x] = bi;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if (threadIdx.x < o) {
            const float v = sv[threadIdx.x + o];
            const int i = si[threadIdx.x + o];
            if (i != 0x7fffffff &&
                (v > sv[threadIdx.x] || (v == sv[threadIdx.x] && i < si[threadIdx.x]) || si[threadIdx.x] == 0x7fffffff)) {
                sv[threadIdx.x] = v;
                si[threadIdx.x] = i;
            }
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) out[m] = si[0] == 0x7fffffff ? 0 : si[0];
}

// ---- argmax directly over f32 rows (rows not produced by the fused lm_head) ----
__global__ __launch_bounds__(256) void k_argmax_rows(const float *x, int64_t ld, int n, int *out) {
    const int m = blockIdx.x;
    const float *row = x + (int64_t)m * ld;
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int i = threadIdx.x; i < n; i += 256) {
        const float v = row[i];
        if (v > -INFINITY && (v > bv || bi == 0x7fffffff)) {  // i increases per thread: first max kept
            bv = v;
            bi = i;
        }
    }
    __shared__ float sv[256];
    __shared__ int si[256];
    sv[threadIdx.x] = bv;
    si[threadIdx.x] = bi;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if (threadIdx.x < o) {
            const float v = sv[threadIdx.x + o];
            const int i = si[threadIdx.x + o];
            if (i != 0x7fffffff &&
                (v > sv[threadIdx.x] || (v == sv[threadIdx.x] && i < si[threadIdx.x]) || si[threadIdx.x] == 0x7fffffff)) {
                sv[threadIdx.x] = v;
                si[threadIdx.x] = i;
            }
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) out[m] = si[0] == 0x7fffffff ? 0 : si[0];
}

// ---- KV compaction: rows P + src[j] -> P + j, j = 1..n-1 (src[0] == 0) -------
// grid (L * 2 * n_kv), block 256: each workgroup gathers its stream's rows into
// LDS first, so the in-place move is race free.
__global__ __launch_bounds__(256) void k_keep_kv_tail(uint16_t *kv, int64_t stream_stride, int hd, int P,
                                                      const int *src, int n) {
    extern __shared__ uint16_t buf[];
    uint16_t *base = kv + (int64_t)blockIdx.x * stream_stride;
    const int per = n * hd;
    for (int i = threadIdx.x; i < per; i += 256) {
        const int j = i / hd, d = i % hd;
        buf[i] = base[(int64_t)(P + src[j]) * hd + d];
    }
    __syncthreads();
    for (int i = threadIdx.x; i < per; i += 256) {
        const int j = i / hd, d = i % hd;
        base[(int64_t)(P + j) * hd + d] = buf[i];
    }
}

// ---- launchers ----
void launch_dequant_dev(int fmt, const uint8_t *w, int64_t rows, int K, float *y, hipStream_t st) {
    const int64_t n = rows * K;
    hipLaunchKernelGGL(k_dequant_dev, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, fmt, w, rows, K,
                       dev_row_stride(fmt, K), y);
}
void launch_embed(int fmt, const uint8_t *table, int K, const int *ids, int M, float *h, hipStream_t st) {
    hipLaunchKernelGGL(k_embed, dim3((K + 255) / 256, M), dim3(256), 0, st, fmt, table, dev_row_stride(fmt, K), K,
                       ids, h);
}
void launch_rmsnorm(const float *x, const float *w, int M, int K, float eps, uint16_t *out16, int ld16, float *out32,
                    hipStream_t st) {
    hipLaunchKernelGGL(k_rmsnorm, dim3(M), dim3(256), 0, st, x, w, K, eps, out16, ld16, out32);
}
void launch_to_frag16(const float *x, int M, int K, uint16_t *out16, int ld16, hipStream_t st) {
    hipLaunchKernelGGL(k_to_frag16, dim3((K + 255) / 256, M), dim3(256), 0, st, x, K, out16, ld16);
}
void launch_argmax_reduce(const float *pv, const int *pi, int nwg, int M, int *out, hipStream_t st) {
    hipLaunchKernelGGL(k_argmax_reduce, dim3(M), dim3(256), 0, st, pv, pi, nwg, out);
}
void launch_argmax_rows(const float *x, int64_t ld, int n, int M, int *out, hipStream_t st) {
    hipLaunchKernelGGL(k_argmax_rows, dim3(M), dim3(256), 0, st, x, ld, n, out);
}
void launch_keep_kv_tail(uint16_t *kv, int nstreams, int64_t stream_stride, int hd, int P, const int *src, int n,
                         hipStream_t st) {
    const size_t lds = (size_t)n * hd * sizeof(uint16_t);
    hipLaunchKernelGGL(k_keep_kv_tail, dim3(nstreams), dim3(256), lds, st, kv, stream_stride, hd, P, src, n);
}

}  // namespace sd
