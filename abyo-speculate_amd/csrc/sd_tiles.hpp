// One row's GGUF superblock <-> its share of a tile block of the device
// weight layout (described in sd_layout.hip).  __host__ __device__: the
// relayout kernels and the host-side repacking entry points share it.
#pragma once
#include <stdint.h>

#include "sd_common.hpp"
#include "sd_qcodes.hpp"

namespace sd {

// ---- fifth / high bits: where the matmul expects them -------------------------
// For chunk c, element t = l & 3 of half s' (0 = low nibble, 1 = high nibble):
// unrotated bit position in the chunk's 32-bit word; the word is then rotated
// left by a chunk-dependent amount so that several chunks share one word.
__host__ __device__ inline int q5_base_bit(int t, int hi) {
    // p0: t=0 -> 4, t=2 -> 20; p2 (hi): 8, 24; p1/p3 read (word >> 1): t=1 -> 5/9, t=3 -> 21/25
    const int base = (t & 2) ? 20 : 4;
    return base + (hi ? 4 : 0) + (t & 1);
}
__host__ __device__ inline int q5_rot(int c) { return LaneQ5K::rot(c); }  // 0, 2, 8, 10
// Q5_K: word (c >> 2) of the lane's 8 bytes, bit (base + rot) & 31
__host__ __device__ inline int layout_q5_bit(int l, int hi) {
    const int c = l >> 2;
    return 32 * (c >> 2) + ((q5_base_bit(l & 3, hi) + q5_rot(c)) & 31);
}
__host__ __device__ inline int q6_base_bit(int t, int hi) {
    // p0: t=0 -> 4..5, t=2 -> 20..21; p2 (hi): 8..9, 24..25; p1/p3 read (word >> 2)
    const int base = (t & 2) ? 20 : 4;
    return base + (hi ? 4 : 0) + 2 * (t & 1);
}
// Q6_K: word (c >> 1) of the lane's 16 bytes, 2 bits at (base + 8*(c & 1)) & 31
__host__ __device__ inline int layout_q6_bit(int l, int hi) {
    const int c = l >> 2;
    return 32 * (c >> 1) + ((q6_base_bit(l & 3, hi) + 8 * (c & 1)) & 31);
}

__host__ __device__ inline void set_bits(uint8_t *p, int bit, int nbits, int v) {
    for (int i = 0; i < nbits; i++) {
        const int b = bit + i;
        if ((v >> i) & 1) p[b >> 3] |= (uint8_t)(1u << (b & 7));
    }
}
__host__ __device__ inline int get_bits(const uint8_t *p, int bit, int nbits) {
    int v = 0;
    for (int i = 0; i < nbits; i++) {
        const int b = bit + i;
        v |= ((p[b >> 3] >> (b & 7)) & 1) << i;
    }
    return v;
}

// ---- K-quant header: scales and mins regrouped per lane group --------------
// Bytes 0..3 of a row's 16-byte header are GGUF's (d, dmin).  Bytes 4..15 hold
// the 8 six-bit scales sc_j and mins m_j regrouped: lane group g needs
// sc_2g, sc_2g+1, m_2g, m_2g+1, the 24-bit word
//   w_g = sc_2g | sc_2g+1 << 6 | m_2g << 12 | m_2g+1 << 18,
// and byte k of w_g sits at byte g of header word 1 + k (byte 4 + 4k + g), so
// a lane gathers it with two byte permutes.  The 96 bits are a permutation of
// GGUF's 12 scale bytes (get_scale_min_k4's packing), so unpacking is exact.
__host__ __device__ inline void kq_scale_min(const uint8_t *q, int j, int &sc, int &m) {
    if (j < 4) {
        sc = q[j] & 63;
        m = q[j + 4] & 63;
    } else {
        sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}
// q: GGUF scale bytes (12); h: the header's bytes 4..15
__host__ __device__ inline void kq_hdr_pack(const uint8_t *q, uint8_t *h) {
    int sc[8], mn[8];
    for (int j = 0; j < 8; j++) kq_scale_min(q, j, sc[j], mn[j]);
    for (int g = 0; g < 4; g++) {
        const uint32_t w = (uint32_t)sc[2 * g] | (uint32_t)sc[2 * g + 1] << 6 | (uint32_t)mn[2 * g] << 12 |
                           (uint32_t)mn[2 * g + 1] << 18;
        for (int k = 0; k < 3; k++) h[4 * k + g] = (uint8_t)(w >> (8 * k));
    }
}
__host__ __device__ inline void kq_hdr_unpack(const uint8_t *h, uint8_t *q) {
    int sc[8], mn[8];
    for (int g = 0; g < 4; g++) {
        const uint32_t w = (uint32_t)h[g] | (uint32_t)h[4 + g] << 8 | (uint32_t)h[8 + g] << 16;
        sc[2 * g] = (int)(w & 63);
        sc[2 * g + 1] = (int)((w >> 6) & 63);
        mn[2 * g] = (int)((w >> 12) & 63);
        mn[2 * g + 1] = (int)((w >> 18) & 63);
    }
    for (int j = 0; j < 4; j++) {
        q[j] = (uint8_t)(sc[j] | ((sc[j + 4] >> 4) << 6));
        q[j + 4] = (uint8_t)(mn[j] | ((mn[j + 4] >> 4) << 6));
        q[j + 8] = (uint8_t)((sc[j + 4] & 0xF) | ((mn[j + 4] & 0xF) << 4));
    }
}

// ---- one row's GGUF superblock <-> its share of a tile block -----------------
// gg: the row's GGUF bytes of the superblock (fmt_sb_bytes); tb: tile block; r: row in tile.
// pack writes only bytes owned by row r (its lanes r + 16g), so threads of the
// 16 rows never touch the same byte.
__host__ __device__ inline void pack_sb(int fmt, const uint8_t *gg, uint8_t *tb, int r) {
    if (fmt == Q4_K || fmt == Q5_K) {
        for (int j = 0; j < 4; j++) tb[r * 16 + j] = gg[j];
        kq_hdr_pack(gg + 4, tb + r * 16 + 4);
        const uint8_t *qs = gg + (fmt == Q4_K ? 16 : 48);
        const int qoff = fmt == Q4_K ? 256 : 768;
        for (int q = 0; q < 128; q++) {
            const int g = q >> 5, o = q & 31, lane = r + 16 * g;
            tb[qoff + (o >> 4) * 1024 + lane * 16 + (o & 15)] = qs[q];
        }
        if (fmt == Q5_K) {
            const uint8_t *qh = gg + 16;
            for (int g = 0; g < 4; g++) {
                uint8_t *w = tb + 256 + (r + 16 * g) * 8;
                for (int i = 0; i < 8; i++) w[i] = 0;
                for (int l = 0; l < 32; l++)
                    for (int hi = 0; hi < 2; hi++)
                        set_bits(w, layout_q5_bit(l, hi), 1, (qh[l] >> (2 * g + hi)) & 1);
            }
        }
        return;
    }
    if (fmt == Q6_K) {
        const uint8_t *ql = gg, *qh = gg + 128;
        for (int g = 0; g < 4; g++) {
            const int h = g >> 1, odd = g & 1, lane = r + 16 * g;
            uint8_t *hb = tb + 2048 + lane * 16;
            for (int i = 0; i < 16; i++) hb[i] = 0;
            for (int l = 0; l < 32; l++) {
                const int n0 = (ql[64 * h + l] >> (4 * odd)) & 0xF;       // s' = 0 (qd = 2 odd)
                const int n1 = (ql[64 * h + 32 + l] >> (4 * odd)) & 0xF;  // s' = 1 (qd = 2 odd + 1)
                tb[(l >> 4) * 1024 + lane * 16 + (l & 15)] = (uint8_t)(n0 | (n1 << 4));
                const int h0 = (qh[32 * h + l] >> (2 * (2 * odd))) & 3;
                const int h1 = (qh[32 * h + l] >> (2 * (2 * odd + 1))) & 3;
                set_bits(hb, layout_q6_bit(l, 0), 2, h0);
                set_bits(hb, layout_q6_bit(l, 1), 2, h1);
            }
        }
        for (int j = 0; j < 16; j++) tb[3072 + r * 16 + j] = gg[192 + j];
        tb[3328 + r * 2] = gg[208];
        tb[3328 + r * 2 + 1] = gg[209];
        return;
    }
    if (fmt == Q8_0) {
        for (int b = 0; b < 8; b++) {
            const uint8_t *blk = gg + 34 * b;
            tb[4096 + r * 16 + 2 * b] = blk[0];
            tb[4096 + r * 16 + 2 * b + 1] = blk[1];
            const int g = b >> 1, lane = r + 16 * g;
            for (int i = 0; i < 32; i++) {
                const int o = 32 * (b & 1) + i;  // byte within the lane's 64
                tb[(o >> 4) * 1024 + lane * 16 + (o & 15)] = (uint8_t)(blk[2 + i] ^ 0x80);  // q + 128
            }
        }
    }
}

__host__ __device__ inline void unpack_sb(int fmt, const uint8_t *tb, int r, uint8_t *gg) {
    if (fmt == Q4_K || fmt == Q5_K) {
        for (int j = 0; j < 4; j++) gg[j] = tb[r * 16 + j];
        kq_hdr_unpack(tb + r * 16 + 4, gg + 4);
        uint8_t *qs = gg + (fmt == Q4_K ? 16 : 48);
        const int qoff = fmt == Q4_K ? 256 : 768;
        for (int q = 0; q < 128; q++) {
            const int g = q >> 5, o = q & 31, lane = r + 16 * g;
            qs[q] = tb[qoff + (o >> 4) * 1024 + lane * 16 + (o & 15)];
        }
        if (fmt == Q5_K) {
            uint8_t *qh = gg + 16;
            for (int l = 0; l < 32; l++) qh[l] = 0;
            for (int g = 0; g < 4; g++) {
                const uint8_t *w = tb + 256 + (r + 16 * g) * 8;
                for (int l = 0; l < 32; l++)
                    for (int hi = 0; hi < 2; hi++)
                        qh[l] |= (uint8_t)(get_bits(w, layout_q5_bit(l, hi), 1) << (2 * g + hi));
            }
        }
        return;
    }
    if (fmt == Q6_K) {
        uint8_t *ql = gg, *qh = gg + 128;
        for (int i = 0; i < 192; i++) gg[i] = 0;
        for (int g = 0; g < 4; g++) {
            const int h = g >> 1, odd = g & 1, lane = r + 16 * g;
            const uint8_t *hb = tb + 2048 + lane * 16;
            for (int l = 0; l < 32; l++) {
                const int nb = tb[(l >> 4) * 1024 + lane * 16 + (l & 15)];
                ql[64 * h + l] |= (uint8_t)((nb & 0xF) << (4 * odd));
                ql[64 * h + 32 + l] |= (uint8_t)((nb >> 4) << (4 * odd));
                qh[32 * h + l] |= (uint8_t)(get_bits(hb, layout_q6_bit(l, 0), 2) << (2 * (2 * odd)));
                qh[32 * h + l] |= (uint8_t)(get_bits(hb, layout_q6_bit(l, 1), 2) << (2 * (2 * odd + 1)));
            }
        }
        for (int j = 0; j < 16; j++) gg[192 + j] = tb[3072 + r * 16 + j];
        gg[208] = tb[3328 + r * 2];
        gg[209] = tb[3328 + r * 2 + 1];
        return;
    }
    if (fmt == Q8_0) {
        for (int b = 0; b < 8; b++) {
            uint8_t *blk = gg + 34 * b;
            blk[0] = tb[4096 + r * 16 + 2 * b];
            blk[1] = tb[4096 + r * 16 + 2 * b + 1];
            const int g = b >> 1, lane = r + 16 * g;
            for (int i = 0; i < 32; i++) {
                const int o = 32 * (b & 1) + i;
                blk[2 + i] = (uint8_t)(tb[(o >> 4) * 1024 + lane * 16 + (o & 15)] ^ 0x80);
            }
        }
    }
}

}  // namespace sd
