// RMSNorm, argmax reductions, KV compaction.
//
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

// One workgroup (NT threads) per row.  Each thread keeps its K/NT values in
// registers (vector loads, all issued before the first use), so the row is
// read from memory once and there is one memory round trip, not K/NT of them.
// With nks > 1 the residual matmul that produced x left K-slice partial sums
// part[ks][M][K] (nks <= 8): they are added to x in slice order first (and x
// is stored); every slice's loads are in flight before the first add.
template <int NV, int NT>  // NT threads, NV float4 vectors per thread: K = 4 * NT * NV
__global__ __launch_bounds__(NT) void k_rmsnorm(float *x, const float *w, int K, float eps, uint16_t *out16,
                                                int ld16, float *out32, const float *part, int nks,
                                                int64_t pstride) {
    const int m = blockIdx.x, t = threadIdx.x;
    float4 *row = (float4 *)(x + (int64_t)m * K);
    const float4 *wv = (const float4 *)w;
    float4 v[NV], wr[NV];
#pragma unroll
    for (int i = 0; i < NV; i++) v[i] = row[t + NT * i];
#pragma unroll
    for (int i = 0; i < NV; i++) wr[i] = wv[t + NT * i];
    if (nks > 1) {
        constexpr int KS = NV <= 4 ? 8 : 4;  // slices per batch of loads (registers: KS * NV float4)
        for (int k0 = 0; k0 < nks; k0 += KS) {
            float4 a[KS][NV];
#pragma unroll
            for (int k = 0; k < KS; k++) {
                const float4 *pr = (const float4 *)(part + (k0 + k) * pstride + (int64_t)m * K);
#pragma unroll
                for (int i = 0; i < NV; i++) a[k][i] = k0 + k < nks ? pr[t + NT * i] : make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int k = 0; k < KS; k++)
#pragma unroll
                for (int i = 0; i < NV; i++) {
                    if (k0 + k >= nks) continue;
                    v[i].x += a[k][i].x;
                    v[i].y += a[k][i].y;
                    v[i].z += a[k][i].z;
                    v[i].w += a[k][i].w;
                }
        }
#pragma unroll
        for (int i = 0; i < NV; i++) row[t + NT * i] = v[i];
    }
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < NV; i++) ss += v[i].x * v[i].x + v[i].y * v[i].y + v[i].z * v[i].z + v[i].w * v[i].w;
    ss += __shfl_xor(ss, 1);
    ss += __shfl_xor(ss, 2);
    ss += __shfl_xor(ss, 4);
    ss += __shfl_xor(ss, 8);
    ss += __shfl_xor(ss, 16);
    ss += __shfl_xor(ss, 32);
    constexpr int NW = NT / 64;
    __shared__ float red[NW];
    if ((t & 63) == 0) red[t >> 6] = ss;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int i = 0; i < NW; i++) tot += red[i];  // fixed order
    const float mrms = sqrtf(tot / (float)K + eps);
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int k = 4 * (t + NT * i);
        const float y[4] = {v[i].x / mrms * wr[i].x, v[i].y / mrms * wr[i].y, v[i].z / mrms * wr[i].z,
                            v[i].w / mrms * wr[i].w};
        if (out16) {
            // elements k .. k+3 sit in fragment slots f, f+2, f+1, f+3: one 8-byte store
            const uint32_t lo = (uint32_t)f2h(y[0]) | ((uint32_t)f2h(y[2]) << 16);
            const uint32_t hi = (uint32_t)f2h(y[1]) | ((uint32_t)f2h(y[3]) << 16);
            *(uint2 *)(out16 + (int64_t)m * ld16 + frag_index(k)) = make_uint2(lo, hi);
        }
        if (out32) *(float4 *)(out32 + (int64_t)m * K + k) = make_float4(y[0], y[1], y[2], y[3]);
    }
}

// generic K (multiple of 4): strided loop
__global__ __launch_bounds__(256) void k_rmsnorm_any(float *x, const float *w, int K, float eps, uint16_t *out16,
                                                     int ld16, float *out32, const float *part, int nks,
                                                     int64_t pstride) {
    const int m = blockIdx.x;
    float *row = x + (int64_t)m * K;
    if (nks > 1) {
        for (int k = threadIdx.x; k < K; k += 256) {
            float v = row[k];
            for (int s = 0; s < nks; s++) v += part[s * pstride + (int64_t)m * K + k];
            row[k] = v;
        }
        __syncthreads();
    }
    float ss = 0.f;
    for (int k = threadIdx.x; k < K; k += 256) ss += row[k] * row[k];
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

// Residual finalisation spread over each row (17..64 rows): x += the K-slice
// partials of the residual matmul (slice order, nks <= 8), u = fp16(x * w) in
// fragment order, and one sum of x^2 per token and block of 4 * NT columns,
// ssq[m * (K / (4 NT)) + b]; the matmul reading u applies
// 1 / sqrt(sum / K + eps) (RMSNorm::forward split around it).  The rows of one
// token spread over K / (4 NT) workgroups instead of one.  grid (M, K / (4 NT)).
template <int NT>
__global__ __launch_bounds__(NT) void k_resid_u(float *x, const float *w, int K, const float *part, int nks,
                                                int64_t pstride, uint16_t *out16, int ld16, float *ssq) {
    const int m = blockIdx.x, b = blockIdx.y, t = threadIdx.x;
    const int k = (b * NT + t) * 4;
    float4 *rp = (float4 *)(x + (int64_t)m * K + k);
    float4 v = *rp;
    const float4 wv = *(const float4 *)(w + k);
    if (nks > 1) {
        float4 a[8];
#pragma unroll
        for (int ks = 0; ks < 8; ks++)
            a[ks] = ks < nks ? *(const float4 *)(part + ks * pstride + (int64_t)m * K + k) : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int ks = 0; ks < 8; ks++) {
            if (ks >= nks) continue;
            v.x += a[ks].x;
            v.y += a[ks].y;
            v.z += a[ks].z;
            v.w += a[ks].w;
        }
        *rp = v;
    }
    // elements k .. k+3 sit in fragment slots f, f+2, f+1, f+3: one 8-byte store
    const uint32_t lo = (uint32_t)f2h(v.x * wv.x) | ((uint32_t)f2h(v.z * wv.z) << 16);
    const uint32_t hi = (uint32_t)f2h(v.y * wv.y) | ((uint32_t)f2h(v.w * wv.w) << 16);
    *(uint2 *)(out16 + (int64_t)m * ld16 + frag_index(k)) = make_uint2(lo, hi);
    float ss = v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
    ss += __shfl_xor(ss, 1);
    ss += __shfl_xor(ss, 2);
    ss += __shfl_xor(ss, 4);
    ss += __shfl_xor(ss, 8);
    ss += __shfl_xor(ss, 16);
    ss += __shfl_xor(ss, 32);
    constexpr int NW = NT / 64;
    __shared__ float red[NW];
    if ((t & 63) == 0) red[t >> 6] = ss;
    __syncthreads();
    if (t == 0) {
        float tot = 0.f;
#pragma unroll
        for (int i = 0; i < NW; i++) tot += red[i];  // fixed order
        ssq[(int64_t)m * gridDim.y + b] = tot;
    }
}

// Input of a matmul with the RMSNorm fused into it (M <= 16): u = fp16(x * w)
// in fragment order and, per 16-element tile, the sum of x^2 (the matmul's
// epilogue applies 1 / sqrt(sum / K + eps)).  grid M, block 256; K % 16 == 0.
__global__ __launch_bounds__(256) void k_norm_u(const float *x, const float *w, int K, uint16_t *out16, int ld16,
                                                float *ssq) {
    const int m = blockIdx.x;
    const float *row = x + (int64_t)m * K;
    for (int t = threadIdx.x; t < K / 16; t += 256) {
        float4 v[4], wv[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            v[j] = ((const float4 *)(row + 16 * t))[j];
            wv[j] = ((const float4 *)(w + 16 * t))[j];
        }
        float s = 0.f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            s += (v[j].x * v[j].x + v[j].y * v[j].y) + (v[j].z * v[j].z + v[j].w * v[j].w);
            const int k = 16 * t + 4 * j;
            uint16_t *dst = out16 + (int64_t)m * ld16 + frag_index(k);  // slots of k, k+2, k+1, k+3
            dst[0] = f2h(v[j].x * wv[j].x);
            dst[1] = f2h(v[j].z * wv[j].z);
            dst[2] = f2h(v[j].y * wv[j].y);
            dst[3] = f2h(v[j].w * wv[j].w);
        }
        ssq[(int64_t)m * (K / 16) + t] = s;
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
// grid M, block 256.  Each thread loads its (up to 32) partials before
// comparing, so the reduction costs one memory round trip.
__device__ __forceinline__ void amax_take(float &bv, int &bi, float v, int i) {
    if (i != 0x7fffffff && (v > bv || (v == bv && i < bi) || bi == 0x7fffffff)) {
        bv = v;
        bi = i;
    }
}
__global__ __launch_bounds__(256) void k_argmax_reduce(const float *pv, const int *pi, int nwg, int *out) {
    const int m = blockIdx.x;
    constexpr int PER = 32;
    float v[PER];
    int ix[PER];
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int w = threadIdx.x + 256 * j;
        const bool ok = w < nwg;
        v[j] = ok ? pv[(int64_t)m * nwg + w] : -INFINITY;
        ix[j] = ok ? pi[(int64_t)m * nwg + w] : 0x7fffffff;
    }
    float bv = -INFINITY;
    int bi = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < PER; j++) amax_take(bv, bi, v[j], ix[j]);
    for (int w = threadIdx.x + 256 * PER; w < nwg; w += 256) amax_take(bv, bi, pv[(int64_t)m * nwg + w], pi[(int64_t)m * nwg + w]);
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) amax_take(bv, bi, __shfl_xor(bv, off), __shfl_xor(bi, off));
    __shared__ float sv[4];
    __shared__ int si[4];
    if ((threadIdx.x & 63) == 0) {
        sv[threadIdx.x >> 6] = bv;
        si[threadIdx.x >> 6] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int k = 1; k < 4; k++) amax_take(bv, bi, sv[k], si[k]);
        out[m] = bi == 0x7fffffff ? 0 : bi;
    }
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
// LDS first, so the in-place move is race free.  Streams alternate K, V every
// n_kv streams; element places follow the blocked cache layout (kv_off).
__global__ __launch_bounds__(256) void k_keep_kv_tail(uint16_t *kv, int64_t stream_stride, int n_kv, int hd, int P,
                                                      const int *src, int n) {
    extern __shared__ uint16_t buf[];
    uint16_t *base = kv + (int64_t)blockIdx.x * stream_stride;
    const int which = (int)((blockIdx.x / n_kv) & 1);
    const int per = n * hd;
    for (int i = threadIdx.x; i < per; i += 256) {
        const int j = i / hd, d = i % hd;
        buf[i] = base[kv_off(which, P + src[j], d, hd)];
    }
    __syncthreads();
    for (int i = threadIdx.x; i < per; i += 256) {
        const int j = i / hd, d = i % hd;
        base[kv_off(which, P + j, d, hd)] = buf[i];
    }
}

// ---- launchers ----
void launch_rmsnorm(float *x, const float *w, int M, int K, float eps, uint16_t *out16, int ld16, float *out32,
                    hipStream_t st, const float *part, int nks) {
    const int64_t ps = (int64_t)M * K;
#define SD_RMS(KERN, NT) hipLaunchKernelGGL(KERN, dim3(M), dim3(NT), 0, st, x, w, K, eps, out16, ld16, out32, part, nks, ps)
    // one float4 per thread (and slice) where K allows: the row's loads spread
    // over 16 waves
    switch (K) {
    case 1024: SD_RMS((k_rmsnorm<1, 256>), 256); break;
    case 2048: SD_RMS((k_rmsnorm<2, 256>), 256); break;
    case 3072: SD_RMS((k_rmsnorm<3, 256>), 256); break;
    case 4096: SD_RMS((k_rmsnorm<1, 1024>), 1024); break;
    case 5120: SD_RMS((k_rmsnorm<5, 256>), 256); break;
    case 8192: SD_RMS((k_rmsnorm<2, 1024>), 1024); break;
    default: SD_RMS(k_rmsnorm_any, 256); break;
    }
#undef SD_RMS
}
void launch_norm_u(const float *x, const float *w, int M, int K, uint16_t *out16, int ld16, float *ssq,
                   hipStream_t st) {
    if (K % 16) throw BackendError("norm_u: K must be a multiple of 16");
    hipLaunchKernelGGL(k_norm_u, dim3(M), dim3(256), 0, st, x, w, K, out16, ld16, ssq);
}
int resid_u_parts(int K) { return K % 1024 == 0 ? K / 1024 : K % 512 == 0 ? K / 512 : K / 256; }
void launch_resid_u(float *x, const float *w, int M, int K, const float *part, int nks, uint16_t *out16, int ld16,
                    float *ssq, hipStream_t st) {
    if (K % 256 || nks > 8) throw BackendError("resid_u: K must be a multiple of 256, at most 8 slices");
    const int64_t ps = (int64_t)M * K;
    const int nb = resid_u_parts(K);
    if (nb > 64) throw BackendError("resid_u: too many column blocks");
    if (K % 1024 == 0) hipLaunchKernelGGL(k_resid_u<256>, dim3(M, nb), dim3(256), 0, st, x, w, K, part, nks, ps, out16, ld16, ssq);
    else if (K % 512 == 0) hipLaunchKernelGGL(k_resid_u<128>, dim3(M, nb), dim3(128), 0, st, x, w, K, part, nks, ps, out16, ld16, ssq);
    else hipLaunchKernelGGL(k_resid_u<64>, dim3(M, nb), dim3(64), 0, st, x, w, K, part, nks, ps, out16, ld16, ssq);
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
void launch_keep_kv_tail(uint16_t *kv, int nstreams, int64_t stream_stride, int n_kv, int hd, int P, const int *src,
                         int n, hipStream_t st) {
    const size_t lds = (size_t)n * hd * sizeof(uint16_t);
    hipLaunchKernelGGL(k_keep_kv_tail, dim3(nstreams), dim3(256), lds, st, kv, stream_stride, n_kv, hd, P, src, n);
}

}  // namespace sd
