// Device weight layout: GGUF rows <-> tile-interleaved tile blocks, and the
// exact f32 dequantisation of device-layout tensors.
//
// A tile block holds the superblock sb of rows 16t .. 16t+15.  Inside it, the
// bytes a lane (r, g) of the matmul kernel needs (r = row within the tile, g =
// lane group, lane = r + 16 g) are packed so that each of its loads reads a
// contiguous range across the wave:
//
//   Q4_K (2304 B): hdr[r][16]                     (d, dmin, then the 6-bit scales
//                                                 and mins regrouped per lane group:
//                                                 kq_hdr_pack in sd_tiles.hpp; 256 B)
//                  qs  part p = 0,1: [lane][16]   (qs bytes 32g + 16p .. +16)
//   Q5_K (2816 B): hdr[r][16] | qhp[lane][8] | qs part 0,1 as Q4_K
//                  qhp holds the lane's 64 fifth bits, placed where the matmul
//                  ORs them into its fp16 codes (layout_q5_bit below)
//   Q6_K (3360 B): nib part 0,1: [lane][16]       nib byte l = low 4 bits of the
//                  elements (s'=0, l) | (s'=1, l) << 4, s' = element half
//                  hbp[lane][16]                  2-bit high parts (layout_q6_bit)
//                  sc[r][16] | d[r][2]
//   Q8_0 (4352 B): qs part p = 0..3: [lane][16]   (blocks 2g, 2g+1: 64 bytes, each q + 128)
//                  d[r][8 x f16]
//
// Lane (r, g) covers elements 64g .. 64g+63 of the superblock: for the K-quants
// low/high nibble of qs group g (sub-blocks 2g and 2g+1); for Q6_K the elements
// 128h + 32(2 odd + s') + l with h = g >> 1, odd = g & 1; for Q8_0 the blocks
// 2g and 2g+1.  Chunk c of a lane = bytes 4c .. 4c+3 of its 32-byte group, i.e.
// elements l = 4c .. 4c+3 of both halves.
#include "sd_common.hpp"
#include "sd_kernels.hpp"
#include "sd_kernels_elem.hpp"
#include "sd_tiles.hpp"

namespace sd {

#pragma clang fp contract(off)

// one thread per (row, superblock); dir 0: GGUF -> device, 1: device -> GGUF
__global__ void k_relayout(int fmt, const uint8_t *src, uint8_t *dst, int64_t rows, int64_t nsb, int dir) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * nsb) return;
    const int64_t row = i / nsb, sb = i % nsb;
    const int sbb = fmt_sb_bytes(fmt), tbb = tile_block_bytes(fmt);
    const int64_t g_off = (row * nsb + sb) * sbb;               // GGUF row-major
    const int64_t t_off = ((row >> 4) * nsb + sb) * (int64_t)tbb;  // tile block
    if (dir == 0) pack_sb(fmt, src + g_off, dst + t_off, (int)(row & 15));
    else unpack_sb(fmt, src + t_off, (int)(row & 15), dst + g_off);
}

// ---- exact f32 dequantisation of one GGUF superblock (no FMA contraction) ------
__device__ inline float ldh(const uint8_t *p) { return h2f((uint16_t)(p[0] | (p[1] << 8))); }

// element e (0..255) of a GGUF superblock
__device__ float deq_gguf(int fmt, const uint8_t *b, int e) {
    if (fmt == Q8_0) {
        const uint8_t *blk = b + 34 * (e >> 5);
        return ldh(blk) * (float)(int8_t)blk[2 + (e & 31)];
    }
    if (fmt == Q4_K || fmt == Q5_K) {
        const int part = e >> 5, j = e >> 6, hi = part & 1, l = e & 31;
        int s, m;
        kq_scale_min(b + 4, part, s, m);
        const float d1 = ldh(b) * (float)s, m1 = ldh(b + 2) * (float)m;
        int q;
        if (fmt == Q4_K) {
            const uint8_t qb = b[16 + 32 * j + l];
            q = hi ? (qb >> 4) : (qb & 0xF);
        } else {
            const uint8_t qb = b[48 + 32 * j + l];
            q = (hi ? (qb >> 4) : (qb & 0xF)) + (((b[16 + l] >> (2 * j + hi)) & 1) ? 16 : 0);
        }
        return d1 * (float)q - m1;
    }
    // Q6_K: element 128h + 32qd + l
    const int h = e >> 7, qd = (e >> 5) & 3, l = e & 31;
    const uint8_t qlb = b[64 * h + 32 * (qd & 1) + l], qhb = b[128 + 32 * h + l];
    const int nib = qd < 2 ? (qlb & 0xF) : (qlb >> 4);
    const int q = (nib | (((qhb >> (2 * qd)) & 3) << 4)) - 32;
    return ldh(b + 208) * (float)(int8_t)b[192 + 8 * h + l / 16 + 2 * qd] * (float)q;
}

// y[row][k] of a device-layout tensor: one thread per (row, superblock)
__global__ void k_dequant_dev(int fmt, const uint8_t *w, int64_t rows, int64_t nsb, float *y) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * nsb) return;
    const int64_t row = i / nsb, sb = i % nsb;
    if (fmt == F32) {
        for (int e = 0; e < 256; e++) y[row * nsb * 256 + sb * 256 + e] = ((const float *)w)[row * nsb * 256 + sb * 256 + e];
        return;
    }
    uint8_t gg[272];
    unpack_sb(fmt, w + ((row >> 4) * nsb + sb) * (int64_t)tile_block_bytes(fmt), (int)(row & 15), gg);
    float *o = y + (row * nsb + sb) * 256;
    for (int e = 0; e < 256; e++) o[e] = deq_gguf(fmt, gg, e);
}

// h[m][k] = table[ids[m]][k] (Embedding over the dequantised token table),
// from the table's GGUF-order copy: grid (M, K/256), one thread per element
__global__ __launch_bounds__(256) void k_embed(int fmt, const uint8_t *table, int64_t nsb, const int *ids, float *h) {
    const int m = blockIdx.x, sb = blockIdx.y, e = threadIdx.x;
    const int64_t row = ids[m];
    float *o = h + ((int64_t)m * nsb + sb) * 256;
    if (fmt == F32) {
        o[e] = ((const float *)table)[(row * nsb + sb) * 256 + e];
        return;
    }
    o[e] = deq_gguf(fmt, table + (row * nsb + sb) * (int64_t)fmt_sb_bytes(fmt), e);
}

// ---- launchers ----
static void relayout(int fmt, const uint8_t *src, uint8_t *dst, int64_t rows, int64_t K, int dir, hipStream_t st) {
    if (rows % 16 || K % 256) throw BackendError("relayout: rows must be a multiple of 16 and K of 256");
    const int64_t nsb = K / 256, n = rows * nsb;
    hipLaunchKernelGGL(k_relayout, dim3((unsigned)((n + 127) / 128)), dim3(128), 0, st, fmt, src, dst, rows, nsb, dir);
}
void launch_gguf_to_dev(int fmt, const uint8_t *src, uint8_t *dst, int64_t rows, int64_t K, hipStream_t st) {
    relayout(fmt, src, dst, rows, K, 0, st);
}
void launch_dev_to_gguf(int fmt, const uint8_t *src, uint8_t *dst, int64_t rows, int64_t K, hipStream_t st) {
    relayout(fmt, src, dst, rows, K, 1, st);
}
void launch_dequant_dev(int fmt, const uint8_t *w, int64_t rows, int K, float *y, hipStream_t st) {
    const int64_t nsb = K / 256, n = rows * nsb;
    hipLaunchKernelGGL(k_dequant_dev, dim3((unsigned)((n + 127) / 128)), dim3(128), 0, st, fmt, w, rows, nsb, y);
}
void launch_embed(int fmt, const uint8_t *table, int K, const int *ids, int M, float *h, hipStream_t st) {
    if (!table) throw BackendError("embedding table not set");
    const int64_t nsb = K / 256;
    hipLaunchKernelGGL(k_embed, dim3((unsigned)M, (unsigned)nsb), dim3(256), 0, st, fmt, table, nsb, ids, h);
}

}  // namespace sd
