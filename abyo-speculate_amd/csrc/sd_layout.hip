// GGUF rows <-> device rows.
//
// Q4_K (144 B) and Q5_K (176 B) blocks are 16-byte multiples and stay as GGUF
// stores them.  Q6_K (210 B) and Q8_0 (34 B) blocks are not 16-byte aligned,
// so each row's bytes are regrouped into planes (a permutation of the same
// bytes, so HBM traffic is unchanged):
//   Q6_K row: ql[128*nsb] | qh[64*nsb] | scales[16*nsb] | d[2*nsb]   (stride padded to 16 B)
//   Q8_0 row: qs[32*nb]   | d[2*nb]
#include "sd_common.hpp"
#include "sd_kernels.hpp"

namespace sd {

// one thread per block; dir 0: gguf -> dev, 1: dev -> gguf
__global__ void k_relayout(int fmt, const uint8_t *src, uint8_t *dst, int64_t rows, int64_t nb, int64_t stride_dev,
                           int dir) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * nb) return;
    const int64_t r = i / nb, b = i % nb;
    const int bb = fmt_block_bytes(fmt);
    const int64_t g_off = r * nb * bb + b * bb;  // gguf row stride is unpadded
    const int64_t d_row = r * stride_dev;
    if (fmt == Q6_K) {
        // gguf block: ql[0..128) qh[128..192) sc[192..208) d[208..210)
        const int64_t off_ql = d_row + 128 * b, off_qh = d_row + 128 * nb + 64 * b,
                      off_sc = d_row + 192 * nb + 16 * b, off_d = d_row + 208 * nb + 2 * b;
        for (int j = 0; j < 210; j++) {
            const int64_t dev = j < 128 ? off_ql + j : j < 192 ? off_qh + (j - 128) : j < 208 ? off_sc + (j - 192)
                                                                                            : off_d + (j - 208);
            if (dir == 0) dst[dev] = src[g_off + j];
            else dst[g_off + j] = src[dev];
        }
    } else if (fmt == Q8_0) {
        const int64_t off_q = d_row + 32 * b, off_d = d_row + 32 * nb + 2 * b;
        for (int j = 0; j < 34; j++) {
            const int64_t dev = j < 2 ? off_d + j : off_q + (j - 2);
            if (dir == 0) dst[dev] = src[g_off + j];
            else dst[g_off + j] = src[dev];
        }
    } else {
        for (int j = 0; j < bb; j++) {
            if (dir == 0) dst[d_row + b * bb + j] = src[g_off + j];
            else dst[g_off + j] = src[d_row + b * bb + j];
        }
    }
}

static void relayout(int fmt, const uint8_t *src, uint8_t *dst, int64_t rows, int64_t K, int dir, hipStream_t st) {
    const int64_t nb = K / fmt_block_elems(fmt);
    const int64_t n = rows * nb;
    hipLaunchKernelGGL(k_relayout, dim3((unsigned)((n + 127) / 128)), dim3(128), 0, st, fmt, src, dst, rows, nb,
                       dev_row_stride(fmt, K), dir);
}

void launch_gguf_to_dev(int fmt, const uint8_t *src, uint8_t *dst, int64_t rows, int64_t K, hipStream_t st) {
    relayout(fmt, src, dst, rows, K, 0, st);
}
void launch_dev_to_gguf(int fmt, const uint8_t *src, uint8_t *dst, int64_t rows, int64_t K, hipStream_t st) {
    relayout(fmt, src, dst, rows, K, 1, st);
}

}  // namespace sd
