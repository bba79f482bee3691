// K1: fused GGUF dequant-matmul on CDNA4 MFMA, y[m][n] = sum_k x[m][k] * W[n][k].
//
// Replaces candle's QMatMul::forward at the reference's call sites
// (crates/speculate/src/model/quantized_llama_local.rs:47-49 MLP, :73-90 Q/K/V,
// :135 wo, :317 lm_head; quantized_qwen2_local.rs:41-44, 71-82, 138, 315).
//
// Tiling.  A = 16 weight rows x 32 K (dequantised to fp16 in registers),
// B = 32 K x 16 tokens (fp16 activations, fragment layout), one
// v_mfma_f32_16x16x32_f16 per (row tile, token tile, 32-K chunk), f32
// accumulation.  A workgroup owns RT row tiles; its KW waves split the K
// superblocks (wave w takes w, w+KW, ...); partial sums meet in LDS and are
// added in fixed wave order, so every output is independent of M and of the
// launch: row i of an M-row call equals the M=1 call bit for bit.
//
// Dequant to fp16: a quant nibble pair is OR'ed into the mantissa of 1024.0h
// (0x6400 | q == 1024 + q exactly) and v_fma_mix computes
// round_f16((1024 + q) * d1 + (-(1024 * d1 + m1))) in f32 inside the
// instruction, i.e. the f32 value d1*q - m1 rounded once to fp16.
#include "sd_common.hpp"
#include "sd_kernels.hpp"

namespace sd {

__device__ inline uint32_t fmix2(uint32_t p, float s, float c) {
    const _Float16 lo = __builtin_bit_cast(_Float16, (uint16_t)(p & 0xffffu));
    const _Float16 hi = __builtin_bit_cast(_Float16, (uint16_t)(p >> 16));
    const _Float16 r0 = (_Float16)__builtin_fmaf((float)lo, s, c);
    const _Float16 r1 = (_Float16)__builtin_fmaf((float)hi, s, c);
    return (uint32_t)__builtin_bit_cast(uint16_t, r0) | ((uint32_t)__builtin_bit_cast(uint16_t, r1) << 16);
}

__device__ inline half8 as_half8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    uintx4 u = {a, b, c, d};
    return __builtin_bit_cast(half8, u);
}

__device__ inline uint32_t byte_of(uint32_t w0, uint32_t w1, uint32_t w2, int i) {
    const uint32_t w = i < 4 ? w0 : (i < 8 ? w1 : w2);
    return (w >> (8 * (i & 3))) & 0xffu;
}

// --------------------------------------------------------------------------
// Per-format lane loaders.  Lane (r16 = lane & 15, g = lane >> 4) handles row
// r16 of the tile and fragment group g: 64 elements of each superblock.
// --------------------------------------------------------------------------
struct LdQ4K {
    uintx4 hdr, q0, q1;
};
struct LdQ5K {
    uintx4 hdr, h0, h1, q0, q1;
};
struct LdQ6K {
    uintx4 l0, l1, l2, l3, h0, h1;
    uint32_t sc;
    uint32_t d;
};
struct LdQ80 {
    uintx4 a0, a1, b0, b1;
    uint32_t d;
};

template <int FMT> struct Ld;
template <> struct Ld<Q4_K> { typedef LdQ4K T; };
template <> struct Ld<Q5_K> { typedef LdQ5K T; };
template <> struct Ld<Q6_K> { typedef LdQ6K T; };
template <> struct Ld<Q8_0> { typedef LdQ80 T; };

__device__ inline uintx4 ld16(const uint8_t *p) { return *(const uintx4 *)p; }

// row: device-layout row base, nsb: superblocks per row
__device__ inline void load_sb(LdQ4K &r, const uint8_t *row, int nsb, int sb, int g) {
    const uint8_t *b = row + (int64_t)sb * 144;
    r.hdr = ld16(b);
    r.q0 = ld16(b + 16 + 32 * g);
    r.q1 = ld16(b + 32 + 32 * g);
}
__device__ inline void load_sb(LdQ5K &r, const uint8_t *row, int nsb, int sb, int g) {
    const uint8_t *b = row + (int64_t)sb * 176;
    r.hdr = ld16(b);
    r.h0 = ld16(b + 16);
    r.h1 = ld16(b + 32);
    r.q0 = ld16(b + 48 + 32 * g);
    r.q1 = ld16(b + 64 + 32 * g);
}
__device__ inline void load_sb(LdQ6K &r, const uint8_t *row, int nsb, int sb, int g) {
    const int h = g >> 1;
    const uint8_t *ql = row + (int64_t)sb * 128 + 64 * h;
    r.l0 = ld16(ql);
    r.l1 = ld16(ql + 16);
    r.l2 = ld16(ql + 32);
    r.l3 = ld16(ql + 48);
    const uint8_t *qh = row + (int64_t)nsb * 128 + (int64_t)sb * 64 + 32 * h;
    r.h0 = ld16(qh);
    r.h1 = ld16(qh + 16);
    r.sc = *(const uint32_t *)(row + (int64_t)nsb * 192 + (int64_t)sb * 16 + 4 * g);
    r.d = *(const uint16_t *)(row + (int64_t)nsb * 208 + (int64_t)sb * 2);
}
__device__ inline void load_sb(LdQ80 &r, const uint8_t *row, int nsb, int sb, int g) {
    const uint8_t *q = row + (int64_t)sb * 256 + 64 * g;
    r.a0 = ld16(q);
    r.a1 = ld16(q + 16);
    r.b0 = ld16(q + 32);
    r.b1 = ld16(q + 48);
    r.d = *(const uint32_t *)(row + (int64_t)nsb * 256 + (int64_t)sb * 16 + 4 * g);
}

// Per-superblock scale constants and the fp16 A fragment of chunk c.
struct ScQ {
    float s0, c0, s1, c1, s2, c2, s3, c3;
};

__device__ inline void get_k4(uint32_t w0, uint32_t w1, uint32_t w2, int j, int &sc, int &m) {
    if (j < 4) {
        sc = byte_of(w0, w1, w2, j) & 63;
        m = byte_of(w0, w1, w2, j + 4) & 63;
    } else {
        sc = (byte_of(w0, w1, w2, j + 4) & 0xF) | ((byte_of(w0, w1, w2, j - 4) >> 6) << 4);
        m = (byte_of(w0, w1, w2, j + 4) >> 4) | ((byte_of(w0, w1, w2, j) >> 6) << 4);
    }
}

__device__ inline ScQ scales_kasym(const uintx4 &hdr, int g) {
    const float d = h2f((uint16_t)(hdr.x & 0xffff)), dmin = h2f((uint16_t)(hdr.x >> 16));
    int s, m;
    ScQ r;
    get_k4(hdr.y, hdr.z, hdr.w, 2 * g, s, m);
    float d1 = d * (float)s, m1 = dmin * (float)m;
    r.s0 = d1;
    r.c0 = -(1024.f * d1 + m1);
    get_k4(hdr.y, hdr.z, hdr.w, 2 * g + 1, s, m);
    d1 = d * (float)s;
    m1 = dmin * (float)m;
    r.s1 = d1;
    r.c1 = -(1024.f * d1 + m1);
    return r;
}

__device__ inline ScQ get_scales(const LdQ4K &r, int g) { return scales_kasym(r.hdr, g); }
__device__ inline ScQ get_scales(const LdQ5K &r, int g) { return scales_kasym(r.hdr, g); }
__device__ inline ScQ get_scales(const LdQ6K &r, int g) {
    const float d = h2f((uint16_t)r.d);
    ScQ q;
    // sub-block scales for part A (chunks 0-3 / 4-7) and part B (same)
    const float a0 = d * (float)(int8_t)(r.sc & 0xff), a1 = d * (float)(int8_t)((r.sc >> 8) & 0xff);
    const float b0 = d * (float)(int8_t)((r.sc >> 16) & 0xff), b1 = d * (float)(int8_t)(r.sc >> 24);
    q.s0 = a0; q.c0 = -1056.f * a0;
    q.s1 = a1; q.c1 = -1056.f * a1;
    q.s2 = b0; q.c2 = -1056.f * b0;
    q.s3 = b1; q.c3 = -1056.f * b1;
    return q;
}
__device__ inline ScQ get_scales(const LdQ80 &r, int g) {
    const float da = h2f((uint16_t)(r.d & 0xffff)), db = h2f((uint16_t)(r.d >> 16));
    ScQ q;
    q.s0 = da; q.c0 = -1152.f * da;
    q.s1 = db; q.c1 = -1152.f * db;
    return q;
}

__device__ inline uint32_t wsel(const uintx4 &a, const uintx4 &b, int c) {
    // word c (0..7) of the 32 bytes a|b
    const uintx4 &v = c < 4 ? a : b;
    const int i = c & 3;
    return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

// pairs of bytes (0,2) and (1,3) of a word of 8-bit quant values -> fp16(1024+q)
__device__ inline uint32_t pr02(uint32_t q) { return (q & 0x00FF00FFu) | 0x64006400u; }
__device__ inline uint32_t pr13(uint32_t q) { return ((q >> 8) & 0x00FF00FFu) | 0x64006400u; }

__device__ inline half8 frag(const LdQ4K &r, const ScQ &s, int g, int c) {
    const uint32_t w = wsel(r.q0, r.q1, c);
    const uint32_t p0 = (w & 0x000F000Fu) | 0x64006400u;
    const uint32_t p1 = ((w >> 8) & 0x000F000Fu) | 0x64006400u;
    const uint32_t p2 = ((w >> 4) & 0x000F000Fu) | 0x64006400u;
    const uint32_t p3 = ((w >> 12) & 0x000F000Fu) | 0x64006400u;
    return as_half8(fmix2(p0, s.s0, s.c0), fmix2(p1, s.s0, s.c0), fmix2(p2, s.s1, s.c1), fmix2(p3, s.s1, s.c1));
}
__device__ inline half8 frag(const LdQ5K &r, const ScQ &s, int g, int c) {
    const uint32_t w = wsel(r.q0, r.q1, c);
    const uint32_t h = wsel(r.h0, r.h1, c);
    const uint32_t lo = (w & 0x0F0F0F0Fu) | (((h >> (2 * g)) & 0x01010101u) << 4);
    const uint32_t hi = ((w >> 4) & 0x0F0F0F0Fu) | (((h >> (2 * g + 1)) & 0x01010101u) << 4);
    return as_half8(fmix2(pr02(lo), s.s0, s.c0), fmix2(pr13(lo), s.s0, s.c0), fmix2(pr02(hi), s.s1, s.c1),
                    fmix2(pr13(hi), s.s1, s.c1));
}
__device__ inline half8 frag(const LdQ6K &r, const ScQ &s, int g, int c) {
    const int odd = g & 1;
    const uint32_t wa = wsel(r.l0, r.l1, c), wb = wsel(r.l2, r.l3, c), wh = wsel(r.h0, r.h1, c);
    const uint32_t na = odd ? (wa >> 4) : wa, nb = odd ? (wb >> 4) : wb;
    const uint32_t qa = (na & 0x0F0F0F0Fu) | (((wh >> (4 * odd)) & 0x03030303u) << 4);
    const uint32_t qb = (nb & 0x0F0F0F0Fu) | (((wh >> (4 * odd + 2)) & 0x03030303u) << 4);
    const float sa = c < 4 ? s.s0 : s.s1, ca = c < 4 ? s.c0 : s.c1;
    const float sb = c < 4 ? s.s2 : s.s3, cb = c < 4 ? s.c2 : s.c3;
    return as_half8(fmix2(pr02(qa), sa, ca), fmix2(pr13(qa), sa, ca), fmix2(pr02(qb), sb, cb), fmix2(pr13(qb), sb, cb));
}
__device__ inline half8 frag(const LdQ80 &r, const ScQ &s, int g, int c) {
    const uint32_t qa = wsel(r.a0, r.a1, c) ^ 0x80808080u, qb = wsel(r.b0, r.b1, c) ^ 0x80808080u;
    return as_half8(fmix2(pr02(qa), s.s0, s.c0), fmix2(pr13(qa), s.s0, s.c0), fmix2(pr02(qb), s.s1, s.c1),
                    fmix2(pr13(qb), s.s1, s.c1));
}

__device__ inline float silu_f(float g) { return g / (1.0f + __expf(-g)); }

// --------------------------------------------------------------------------
// Main body for one format.  acc[rt][ct] accumulates the wave's superblocks.
// --------------------------------------------------------------------------
template <int FMT, int RT, int CT, int KW>
__device__ void gemm_body(const GemmParams &p, const uint8_t *rowp[RT], floatx4 (&acc)[RT][CT]) {
    typedef typename Ld<FMT>::T L;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r16 = lane & 15, g = lane >> 4;
    const int K = p.K, nsb = K >> 8;
    const uint16_t *xb[CT];
#pragma unroll
    for (int ct = 0; ct < CT; ct++) xb[ct] = p.xp + (int64_t)(ct * 16 + r16) * K + g * 8;

    int sb = wave;
    if (sb >= nsb) return;
    L cur[RT];
#pragma unroll
    for (int rt = 0; rt < RT; rt++) load_sb(cur[rt], rowp[rt], nsb, sb, g);
    for (; sb < nsb; sb += KW) {
        const int nx = sb + KW < nsb ? sb + KW : sb;
        L nxt[RT];
#pragma unroll
        for (int rt = 0; rt < RT; rt++) load_sb(nxt[rt], rowp[rt], nsb, nx, g);
        uintx4 bf[CT][8];
#pragma unroll
        for (int ct = 0; ct < CT; ct++)
#pragma unroll
            for (int c = 0; c < 8; c++) bf[ct][c] = *(const uintx4 *)(xb[ct] + (int64_t)sb * 256 + c * 32);
        ScQ sc[RT];
#pragma unroll
        for (int rt = 0; rt < RT; rt++) sc[rt] = get_scales(cur[rt], g);
#pragma unroll
        for (int c = 0; c < 8; c++) {
#pragma unroll
            for (int rt = 0; rt < RT; rt++) {
                const half8 a = frag(cur[rt], sc[rt], g, c);
#pragma unroll
                for (int ct = 0; ct < CT; ct++)
                    acc[rt][ct] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, __builtin_bit_cast(half8, bf[ct][c]),
                                                                         acc[rt][ct], 0, 0, 0);
            }
        }
#pragma unroll
        for (int rt = 0; rt < RT; rt++) cur[rt] = nxt[rt];
    }
}

template <int RT, int CT, int KW>
__global__ __launch_bounds__(64 * KW) void k_qgemm(GemmParams p) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r16 = lane & 15, g = lane >> 4;
    const int tile_base = blockIdx.x * RT;  // first tile (non-SWIGLU); SWIGLU: tile index within gate/up

    // segment of this workgroup (segments never straddle a workgroup)
    int si = 0;
    if (p.mode != GM_SWIGLU) {
        while (si + 1 < p.nseg && tile_base >= p.seg[si + 1].tile0) si++;
    }
    const GemmSeg &S = p.seg[si];
    const int fmt = S.fmt;
    const int64_t stride = dev_row_stride(fmt, p.K);

    const uint8_t *rowp[RT];
    int rloc[RT];  // local first row of each tile within its segment
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        const GemmSeg &Sr = p.mode == GM_SWIGLU ? p.seg[rt] : S;
        rloc[rt] = p.mode == GM_SWIGLU ? blockIdx.x * 16 : (tile_base + rt - S.tile0) * 16;
        rowp[rt] = Sr.w + (int64_t)(rloc[rt] + r16) * stride;
    }

    floatx4 acc[RT][CT];
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int ct = 0; ct < CT; ct++) acc[rt][ct] = floatx4{0.f, 0.f, 0.f, 0.f};

    switch (fmt) {
    case Q4_K: gemm_body<Q4_K, RT, CT, KW>(p, rowp, acc); break;
    case Q5_K: gemm_body<Q5_K, RT, CT, KW>(p, rowp, acc); break;
    case Q6_K: gemm_body<Q6_K, RT, CT, KW>(p, rowp, acc); break;
    case Q8_0: gemm_body<Q8_0, RT, CT, KW>(p, rowp, acc); break;
    default: break;
    }

    // ---- fixed-order cross-wave reduction through LDS ----
    __shared__ floatx4 red[KW][RT][CT][64];
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int ct = 0; ct < CT; ct++) red[wave][rt][ct][lane] = acc[rt][ct];
    __syncthreads();

    // each wave finishes the token tiles ct = wave, wave+KW, ... (all rt of it)
    for (int ct = wave; ct < CT; ct += KW) {
        floatx4 v[RT];
#pragma unroll
        for (int rt = 0; rt < RT; rt++) {
            floatx4 s = red[0][rt][ct][lane];
#pragma unroll
            for (int w = 1; w < KW; w++) s += red[w][rt][ct][lane];
            v[rt] = s;
        }
        const int m = ct * 16 + r16;
        const bool live = m < p.M;
        if (p.mode == GM_SWIGLU) {
            // v[0] = gate rows, v[1] = up rows, same output features
            const int n0 = rloc[0] + 4 * g;
            if (live) {
                uint16_t *dst = p.act + (int64_t)m * p.act_ld;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float a = silu_f(v[0][i]) * v[RT - 1][i];
                    dst[frag_index(n0 + i)] = f2h(a);
                }
            }
            continue;
        }
        float bv = -INFINITY;
        int bi = 0x7fffffff;
#pragma unroll
        for (int rt = 0; rt < RT; rt++) {
            const int n0 = rloc[rt] + 4 * g;
            if (!live) continue;
            float *o = S.out + (int64_t)m * S.ldo + S.col0 + n0;
            floatx4 r = v[rt];
            if (p.mode == GM_RESID) {
                r += *(floatx4 *)o;
            } else if (S.bias) {
                r += *(const floatx4 *)(S.bias + n0);
            }
            *(floatx4 *)o = r;
            if (p.mode == GM_LOGITS) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float x = r[i];
                    const int idx = S.col0 + n0 + i;
                    if (x > -INFINITY && (x > bv || (x == bv && idx < bi))) {
                        bv = x;
                        bi = idx;
                    }
                }
            }
        }
        if (p.mode == GM_LOGITS) {
            // combine the 4 lanes (g = 0..3) that hold the same token
#pragma unroll
            for (int off = 16; off < 64; off <<= 1) {
                const float ov = __shfl_xor(bv, off);
                const int oi = __shfl_xor(bi, off);
                if (oi != 0x7fffffff && (ov > bv || (ov == bv && oi < bi) || bi == 0x7fffffff)) {
                    bv = ov;
                    bi = oi;
                }
            }
            if (g == 0 && live) {
                p.amax_v[(int64_t)m * p.amax_ld + blockIdx.x] = bv;
                p.amax_i[(int64_t)m * p.amax_ld + blockIdx.x] = bi;
            }
        }
    }
}

// --------------------------------------------------------------------------
template <int RT, int CT>
static void launch_rt_ct(const GemmParams &p, int nwg, hipStream_t st) {
    constexpr int KW = 4;
    hipLaunchKernelGGL((k_qgemm<RT, CT, KW>), dim3(nwg), dim3(64 * KW), 0, st, p);
}

static int pick_ct(int M) { return M <= 16 ? 1 : M <= 32 ? 2 : M <= 64 ? 4 : 8; }

static int pick_rt(const GemmParams &p) {
    if (p.mode == GM_SWIGLU) return 2;
    if (pick_ct(p.M) >= 8) return 1;
    for (int i = 0; i < p.nseg; i++)
        if (p.seg[i].rows % 32) return 1;
    return 2;
}

int qgemm_workgroups(const GemmParams &p) {
    if (p.mode == GM_SWIGLU) return p.seg[0].rows / 16;
    return p.ntiles / pick_rt(p);
}

int launch_qgemm(const GemmParams &p, hipStream_t st) {
    const int ct = pick_ct(p.M), rt = pick_rt(p);
    const int nwg = qgemm_workgroups(p);
    if (rt == 2) {
        switch (ct) {
        case 1: launch_rt_ct<2, 1>(p, nwg, st); break;
        case 2: launch_rt_ct<2, 2>(p, nwg, st); break;
        case 4: launch_rt_ct<2, 4>(p, nwg, st); break;
        case 8: launch_rt_ct<2, 8>(p, nwg, st); break;
        default: throw BackendError("qgemm: unsupported tile");
        }
    } else {
        switch (ct) {
        case 1: launch_rt_ct<1, 1>(p, nwg, st); break;
        case 2: launch_rt_ct<1, 2>(p, nwg, st); break;
        case 4: launch_rt_ct<1, 4>(p, nwg, st); break;
        case 8: launch_rt_ct<1, 8>(p, nwg, st); break;
        default: throw BackendError("qgemm: unsupported tile");
        }
    }
    return nwg;
}

}  // namespace sd
