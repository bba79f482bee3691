// Launchers of the element-wise / reduction kernels (sd_elem.hip).
#pragma once
#include "sd_kernels.hpp"

namespace sd {

// sd_layout.hip: exact f32 dequantisation of device-layout rows, and the
// embedding gather (Embedding::forward over the dequantised token table,
// crates/speculate/src/model/quantized_llama_local.rs:242-243, 380, 419; rows
// are dequantised on the fly, so no f32 copy of the table is kept)
void launch_dequant_dev(int fmt, const uint8_t *w, int64_t rows, int K, float *y, hipStream_t st);
void launch_embed(int fmt, const uint8_t *table, int K, const int *ids, int M, float *h, hipStream_t st);
// x: [M][K]; with nks > 1, part[ks][M][K] (K-slice partial sums of the
// residual matmul that produced x) are first added to x in slice order.
void launch_rmsnorm(float *x, const float *w, int M, int K, float eps, uint16_t *out16, int ld16, float *out32,
                    hipStream_t st, const float *part = nullptr, int nks = 1);
// 17..64 rows: x += part slices (nks > 1), u = fp16(x * w) in fragment order and
// one sum of x^2 per token and column block (ssq [M][resid_u_parts(K)]) for a
// matmul that applies the norm's 1 / rms itself
int resid_u_parts(int K);
void launch_resid_u(float *x, const float *w, int M, int K, const float *part, int nks, uint16_t *out16, int ld16,
                    float *ssq, hipStream_t st);
void launch_to_frag16(const float *x, int M, int K, uint16_t *out16, int ld16, hipStream_t st);
// u = fp16(x * w) in fragment order + per-16-element sums of x^2 (ssq [M][K/16])
// for a matmul with the RMSNorm fused into its epilogue
void launch_norm_u(const float *x, const float *w, int M, int K, uint16_t *out16, int ld16, float *ssq,
                   hipStream_t st);
void launch_argmax_reduce(const float *pv, const int *pi, int nwg, int M, int *out, hipStream_t st);
void launch_argmax_rows(const float *x, int64_t ld, int n, int M, int *out, hipStream_t st);
void launch_keep_kv_tail(uint16_t *kv, int nstreams, int64_t stream_stride, int n_kv, int hd, int P, const int *src,
                         int n, hipStream_t st);

}  // namespace sd
