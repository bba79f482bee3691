// K1: fused GGUF dequant-matmul on CDNA4 MFMA, y[m][n] = sum_k x[m][k] * W[n][k].
//
// Replaces candle's QMatMul::forward at the reference's call sites
// (crates/speculate/src/model/quantized_llama_local.rs:47-49 MLP, :73-90 Q/K/V,
// :135 wo, :317 lm_head; quantized_qwen2_local.rs:41-44, 71-82, 138, 315).
//
// Both kernels multiply 16 weight rows x 32 K (dequantised to fp16 in
// registers) by 32 K x 16 tokens (fp16 activations in fragment order) with
// v_mfma_f32_16x16x32_f16 and accumulate in f32.
//
//  * k_qgemv (M <= 16, the linear-verify shape): one 16-token tile; only the
//    lanes of real tokens fetch distinct activation rows.  A workgroup owns one
//    row tile (two in SWIGLU mode) and KW waves per tile that split the K
//    superblocks (wave w takes w, w+KW, ...), each with the weights of its next
//    two superblocks in flight; KW is chosen per matrix so that every launch
//    puts thousands of waves on the 256 CUs.
//  * k_qgemm (M > 16, tree and prefill shapes): CT token tiles per wave reuse
//    every dequantised fragment CT times.
//
// Accumulation order is fixed by the matrix alone: per wave, superblocks in
// increasing order and chunks c = 0..7 in order; across waves, partial sums
// meet in LDS and are added for w = 0..KW-1 in order.  KW depends only on
// (rows, K), never on M, so row i of an M-row call equals the M=1 call bit for
// bit in both kernels.
//
// Dequantisation to fp16: a 4-bit code is OR'ed into the mantissa of 1024.0h
// (0x6400 | q == 1024 + q) or, for a code already at bits 4-7, of 64.0h
// (0x5400 | q << 4 == 64 + q), and v_fma_mix evaluates
// round_f16((64|1024 + q) * s + c) in f32, c = -((64|1024) * s + m): the f32
// value s*q - m rounded once to fp16.
#include "sd_common.hpp"
#include "sd_kernels.hpp"
#include "sd_qcodes.hpp"

namespace sd {

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

// two fp16 codes -> two fp16 results of round_f16(code * s + c) (f32 inside)
__device__ __forceinline__ uint32_t fm2(uint32_t p, float s, float c) {
    const half2v h = __builtin_bit_cast(half2v, p);
    half2v r;
    r.x = (_Float16)__builtin_fmaf((float)h.x, s, c);
    r.y = (_Float16)__builtin_fmaf((float)h.y, s, c);
    return __builtin_bit_cast(uint32_t, r);
}
__device__ __forceinline__ half8 as_half8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    const uintx4 u = {a, b, c, d};
    return __builtin_bit_cast(half8, u);
}
// Buffer loads: the matrix base and size sit in a scalar resource, the lane's
// byte offset in a vector register and the superblock offset in a scalar one,
// so the inner loop does no 64-bit address arithmetic.  Reads past the
// resource's size return zero.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
__device__ __forceinline__ rsrc_t make_rsrc(const void *base, uint32_t bytes) {
    // the operands are wave-uniform; readfirstlane makes that visible to the
    // compiler, which otherwise may keep them in vector registers and wrap
    // every buffer load in a per-lane loop
    const uint64_t a = (uint64_t)base;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
    const uint64_t u = ((uint64_t)hi << 32) | lo;
    return __builtin_amdgcn_make_buffer_rsrc((void *)u, (short)0, (int)__builtin_amdgcn_readfirstlane(bytes),
                                             0x00020000);
}
// wave-uniform value pinned to a scalar register (the soffset operand)
__device__ __forceinline__ uint32_t uni(uint32_t v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ uintx4 bld16(rsrc_t r, uint32_t vo, uint32_t so) {
    return __builtin_bit_cast(uintx4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)vo, (int)so, 0));
}
__device__ __forceinline__ uint32_t bld4(rsrc_t r, uint32_t vo, uint32_t so) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, (int)vo, (int)so, 0);
}
__device__ __forceinline__ uint32_t bld2(rsrc_t r, uint32_t vo, uint32_t so) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, (int)vo, (int)so, 0);
}
// one lane's view of its weight row: resource of the whole matrix + row start
struct WRow {
    rsrc_t rs;
    uint32_t base;  // byte offset of the tile's first tile block (wave-uniform)
};
__device__ __forceinline__ uintx2 bld8(rsrc_t r, uint32_t vo, uint32_t so) {
    return __builtin_bit_cast(uintx2, __builtin_amdgcn_raw_buffer_load_b64(r, (int)vo, (int)so, 0));
}
// --------------------------------------------------------------------------
// Per-format lane data.  Lane (r16 = lane & 15, g = lane >> 4) holds row r16
// of the tile and the 64 elements [64g, 64g + 64) of each superblock; chunk c
// of the lane covers the fragment slots g*8 .. g*8+7 of K-chunk c, i.e. the
// elements 64g + 32*(s >> 2) + 4c + {0,2,1,3}[s & 3].
// --------------------------------------------------------------------------
template <int FMT> struct QFmt;

// get_scale_min_k4 for sub-blocks 2g and 2g+1 without lane-divergent branches.
// Scale bytes s[0..11] = hdr.y | hdr.z | hdr.w.  For j < 4: sc = s[j] & 63,
// m = s[j+4] & 63; for j >= 4: sc = (s[j+4] & 15) | (s[j-4] >> 6) << 4,
// m = (s[j+4] >> 4) | (s[j] >> 6) << 4.
__device__ __forceinline__ void kquant_scales(const uintx4 &hdr, int g, float &s0, float &c0, float &s1,
                                              float &c1) {
    const float d = h2f((uint16_t)(hdr.x & 0xffffu)), dmin = h2f((uint16_t)(hdr.x >> 16));
    const int sh = (g & 1) * 16;
    const uint32_t A = hdr.y >> sh, B = hdr.z >> sh, C = hdr.w >> sh;  // bytes jj, jj+1 in bits 0..15
    const bool hi = g >= 2;
    int sc[2], mn[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const uint32_t a = (A >> (8 * i)) & 0xffu, b = (B >> (8 * i)) & 0xffu, cc = (C >> (8 * i)) & 0xffu;
        const uint32_t sc_lo = a & 63u, mn_lo = b & 63u;
        const uint32_t sc_hi = (cc & 15u) | ((a >> 6) << 4), mn_hi = (cc >> 4) | ((b >> 6) << 4);
        sc[i] = (int)(hi ? sc_hi : sc_lo);
        mn[i] = (int)(hi ? mn_hi : mn_lo);
    }
    const float d0 = d * (float)sc[0], m0 = dmin * (float)mn[0];
    const float d1 = d * (float)sc[1], m1 = dmin * (float)mn[1];
    s0 = d0;
    c0 = -(1024.f * d0 + m0);  // low nibbles, codes 1024 + q
    s1 = d1;
    c1 = -(64.f * d1 + m1);    // high nibbles, codes 64 + q
}

// Loads address one tile block: the wave-uniform part (tile, superblock) goes
// in the scalar offset, the lane's fixed position inside the block in the
// vector offset (see the tile-block layout in sd_layout.hip).
__device__ __forceinline__ uint32_t tb_off(const WRow &w, int sb, int tbb) { return uni(w.base + (uint32_t)sb * tbb); }

template <> struct QFmt<Q4_K> {
    typedef LaneQ4K D;
    struct S {
        float s0, c0, s1, c1;
    };
    static __device__ __forceinline__ void load(D &r, const WRow &w, int nsb, int sb, int g) {
        const int lane = threadIdx.x & 63;
        const uint32_t so = tb_off(w, sb, D::TBB);
        r.hdr = bld16(w.rs, D::off_hdr(lane), so);
        r.q0 = bld16(w.rs, D::off_q0(lane), so);
        r.q1 = bld16(w.rs, D::off_q1(lane), so);
    }
    static __device__ __forceinline__ S scales(const D &r, int g) {
        S s;
        kquant_scales(r.hdr, g, s.s0, s.c0, s.s1, s.c1);
        return s;
    }
    static __device__ __forceinline__ half8 frag(const D &r, const S &s, int g, int c) {
        uint32_t p[4];
        r.codes(g, c, p);
        return as_half8(fm2(p[0], s.s0, s.c0), fm2(p[1], s.s0, s.c0), fm2(p[2], s.s1, s.c1), fm2(p[3], s.s1, s.c1));
    }
};

template <> struct QFmt<Q5_K> {
    typedef LaneQ5K D;
    typedef QFmt<Q4_K>::S S;
    static __device__ __forceinline__ void load(D &r, const WRow &w, int nsb, int sb, int g) {
        const int lane = threadIdx.x & 63;
        const uint32_t so = tb_off(w, sb, D::TBB);
        r.hdr = bld16(w.rs, D::off_hdr(lane), so);
        r.qh = bld8(w.rs, D::off_qh(lane), so);
        r.q0 = bld16(w.rs, D::off_q0(lane), so);
        r.q1 = bld16(w.rs, D::off_q1(lane), so);
    }
    static __device__ __forceinline__ S scales(const D &r, int g) {
        S s;
        kquant_scales(r.hdr, g, s.s0, s.c0, s.s1, s.c1);
        return s;
    }
    static __device__ __forceinline__ half8 frag(const D &r, const S &s, int g, int c) {
        uint32_t p[4];
        r.codes(g, c, p);
        return as_half8(fm2(p[0], s.s0, s.c0), fm2(p[1], s.s0, s.c0), fm2(p[2], s.s1, s.c1), fm2(p[3], s.s1, s.c1));
    }
};

template <> struct QFmt<Q6_K> {
    typedef LaneQ6K D;
    struct S {
        float s[4], c[4];  // [2 * s' + (c >= 4)]; c = offset for codes 1024 + q6 (s'=0) / 64 + q6 (s'=1)
    };
    static __device__ __forceinline__ void load(D &r, const WRow &w, int nsb, int sb, int g) {
        const int lane = threadIdx.x & 63;
        const uint32_t so = tb_off(w, sb, D::TBB);
        r.n0 = bld16(w.rs, D::off_n0(lane), so);
        r.n1 = bld16(w.rs, D::off_n1(lane), so);
        r.hb = bld16(w.rs, D::off_hb(lane), so);
        r.sc = bld4(w.rs, D::off_sc(lane), so);
        r.d = bld2(w.rs, D::off_d(lane), so);
    }
    static __device__ __forceinline__ S scales(const D &r, int g) {
        const float d = h2f((uint16_t)r.d);
        S s;
        // sc bytes of the lane: [s'=0, l<16], [s'=0, l>=16], [s'=1, l<16], [s'=1, l>=16]
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float v = d * (float)(int8_t)((r.sc >> (8 * i)) & 0xffu);
            s.s[i] = v;
            s.c[i] = (i < 2 ? -1056.f : -96.f) * v;  // value (q6 - 32) * v
        }
        return s;
    }
    static __device__ __forceinline__ half8 frag(const D &r, const S &s, int g, int c) {
        uint32_t p[4];
        r.codes(g, c, p);
        const int hl = c >= 4 ? 1 : 0;
        const float sa = s.s[hl], ca = s.c[hl], sb = s.s[2 + hl], cb = s.c[2 + hl];
        return as_half8(fm2(p[0], sa, ca), fm2(p[1], sa, ca), fm2(p[2], sb, cb), fm2(p[3], sb, cb));
    }
};

template <> struct QFmt<Q8_0> {
    typedef LaneQ80 D;
    typedef QFmt<Q4_K>::S S;
    static __device__ __forceinline__ void load(D &r, const WRow &w, int nsb, int sb, int g) {
        const int lane = threadIdx.x & 63;
        const uint32_t so = tb_off(w, sb, D::TBB);
        r.a0 = bld16(w.rs, D::off_part(lane, 0), so);
        r.a1 = bld16(w.rs, D::off_part(lane, 1), so);
        r.b0 = bld16(w.rs, D::off_part(lane, 2), so);
        r.b1 = bld16(w.rs, D::off_part(lane, 3), so);
        r.d = bld4(w.rs, D::off_d(lane), so);
    }
    static __device__ __forceinline__ S scales(const D &r, int g) {
        const float da = h2f((uint16_t)(r.d & 0xffffu)), db = h2f((uint16_t)(r.d >> 16));
        S s;
        s.s0 = da;
        s.c0 = -1152.f * da;  // codes 1024 + (q + 128)
        s.s1 = db;
        s.c1 = -1152.f * db;
        return s;
    }
    static __device__ __forceinline__ half8 frag(const D &r, const S &s, int g, int c) {
        uint32_t p[4];
        r.codes(g, c, p);
        return as_half8(fm2(p[0], s.s0, s.c0), fm2(p[1], s.s0, s.c0), fm2(p[2], s.s1, s.c1), fm2(p[3], s.s1, s.c1));
    }
};

__device__ __forceinline__ float silu_f(float g) { return g / (1.0f + __expf(-g)); }

// --------------------------------------------------------------------------
// Shared epilogue: v[rt] is the full sum for row tile rt (lane holds rows
// rloc[rt] + 4g + i, token m).  Writes outputs and, for GM_LOGITS, the
// per-workgroup argmax partial of every token (first max wins).
// --------------------------------------------------------------------------
template <int RT>
__device__ __forceinline__ void epilogue(const GemmParams &p, const GemmSeg &S, const int (&rloc)[RT],
                                         floatx4 (&v)[RT], int m, int g) {
    const bool live = m < p.M;
    if (p.mode == GM_SWIGLU) {
        // v[0] = gate rows, v[RT-1] = up rows of the same output features
        if (live) {
            uint16_t *dst = p.act + (int64_t)m * p.act_ld;
            const int n0 = rloc[0] + 4 * g;
#pragma unroll
            for (int i = 0; i < 4; i++) dst[frag_index(n0 + i)] = f2h(silu_f(v[0][i]) * v[RT - 1][i]);
        }
        return;
    }
    float bv = -INFINITY;
    int bi = 0x7fffffff;
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        if (!live) continue;
        const int n0 = rloc[rt] + 4 * g;
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

// The segment holding a row tile, selected with uniform compares (indexing the
// parameter block with a run-time index would copy it to scratch memory).
__device__ __forceinline__ GemmSeg seg_of_tile(const GemmParams &p, int tile) {
    GemmSeg S = p.seg[0];
#pragma unroll
    for (int i = 1; i < 4; i++)
        if (i < p.nseg && tile >= p.seg[i].tile0) S = p.seg[i];
    return S;
}

// row0: first row of the 16-row tile
__device__ __forceinline__ WRow wrow(const GemmSeg &S, int K, int row0) {
    const uint32_t nsb = (uint32_t)K >> 8, tbb = (uint32_t)tile_block_bytes(S.fmt);
    WRow w;
    w.rs = make_rsrc(S.w, (uint32_t)(S.rows >> 4) * nsb * tbb);
    w.base = uni((uint32_t)(row0 >> 4) * nsb * tbb);
    return w;
}

// ==========================================================================
// M <= 16
// ==========================================================================
template <int FMT>
__device__ __forceinline__ void gemv_step(const typename QFmt<FMT>::D &d, rsrc_t xr, uint32_t xvo, int sb, int g,
                                          floatx4 &acc) {
    typedef QFmt<FMT> F;
    // activations of this superblock: issued before the dequantisation so
    // their L2 latency overlaps it
    uintx4 b[8];
#pragma unroll
    for (int c = 0; c < 8; c++) b[c] = bld16(xr, xvo + 64 * c, uni((uint32_t)sb * 512u));
    const typename F::S sc = F::scales(d, g);
    // all fragments first, then the MFMA chain: no MFMA waits on the VALU
    // result it reads (the VALU -> MFMA operand hazard costs wait states)
    half8 a[8];
#pragma unroll
    for (int c = 0; c < 8; c++) a[c] = F::frag(d, sc, g, c);
#pragma unroll
    for (int c = 0; c < 8; c++)
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[c], __builtin_bit_cast(half8, b[c]), acc, 0, 0, 0);
}

// Superblocks sb = ks, ks + KW, ... in order; the weights of the next two are
// in flight (three register buffers in rotation) while one is computed.
template <int FMT, int KW>
__device__ __forceinline__ void gemv_body(const GemmParams &p, const WRow &row, int ks, floatx4 &acc) {
    typedef QFmt<FMT> F;
    const int lane = threadIdx.x & 63;
    const int r16 = lane & 15, g = lane >> 4;
    const int nsb = p.K >> 8;
    // lanes of padding tokens (r16 >= M) read the last real token's row: the
    // loads coalesce with that lane's and the padding columns are never stored
    const rsrc_t xr = make_rsrc(p.xp, (uint32_t)p.M * (uint32_t)p.K * 2u);
    const uint32_t xvo = ((uint32_t)min(r16, p.M - 1) * (uint32_t)p.K + 8u * g) * 2u;
    int sb = ks;
    if (sb >= nsb) return;
    typename F::D w0, w1, w2;
    F::load(w0, row, nsb, sb, g);
    if (sb + KW < nsb) F::load(w1, row, nsb, sb + KW, g);
    while (true) {
        if (sb + 2 * KW < nsb) F::load(w2, row, nsb, sb + 2 * KW, g);
        gemv_step<FMT>(w0, xr, xvo, sb, g, acc);
        sb += KW;
        if (sb >= nsb) break;
        if (sb + 2 * KW < nsb) F::load(w0, row, nsb, sb + 2 * KW, g);
        gemv_step<FMT>(w1, xr, xvo, sb, g, acc);
        sb += KW;
        if (sb >= nsb) break;
        if (sb + 2 * KW < nsb) F::load(w1, row, nsb, sb + 2 * KW, g);
        gemv_step<FMT>(w2, xr, xvo, sb, g, acc);
        sb += KW;
        if (sb >= nsb) break;
    }
}

// Workgroup = NT row tiles x KW waves: wave w works on tile w / KW and on the
// superblocks w % KW, w % KW + KW, ...  NT = 2 only in SWIGLU mode (gate tile,
// up tile of the same 16 features).
template <int NT, int KW>
__global__ __launch_bounds__(64 * KW * NT) void k_qgemv(GemmParams p) {
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r16 = lane & 15, g = lane >> 4;
    const int t = wave / KW, ks = wave % KW;
    GemmSeg S, St;
    int rloc;
    if (NT == 2) {
        S = p.seg[0];
        St = t == 0 ? p.seg[0] : p.seg[1];
        rloc = (int)blockIdx.x * 16;
    } else {
        S = seg_of_tile(p, blockIdx.x);
        St = S;
        rloc = ((int)blockIdx.x - S.tile0) * 16;
    }
    const WRow row = wrow(St, p.K, rloc);
    floatx4 acc = floatx4{0.f, 0.f, 0.f, 0.f};
    switch (St.fmt) {
    case Q4_K: gemv_body<Q4_K, KW>(p, row, ks, acc); break;
    case Q5_K: gemv_body<Q5_K, KW>(p, row, ks, acc); break;
    case Q6_K: gemv_body<Q6_K, KW>(p, row, ks, acc); break;
    case Q8_0: gemv_body<Q8_0, KW>(p, row, ks, acc); break;
    default: break;
    }
    floatx4 v[NT];
    if constexpr (KW * NT > 1) {
        __shared__ floatx4 red[NT][KW][64];
        red[t][ks][lane] = acc;
        __syncthreads();
        if (wave != 0) return;
#pragma unroll
        for (int tt = 0; tt < NT; tt++) {
            floatx4 sum = red[tt][0][lane];
#pragma unroll
            for (int w = 1; w < KW; w++) sum += red[tt][w][lane];
            v[tt] = sum;
        }
    } else {
        v[0] = acc;
    }
    int rl[NT];
#pragma unroll
    for (int tt = 0; tt < NT; tt++) rl[tt] = rloc;
    epilogue<NT>(p, S, rl, v, r16, g);
}

// ==========================================================================
// M > 16
// ==========================================================================
template <int FMT, int CT, int KW>
__device__ __forceinline__ void gemm_body(const GemmParams &p, const WRow &row, floatx4 (&acc)[CT]) {
    typedef QFmt<FMT> F;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r16 = lane & 15, g = lane >> 4;
    const int K = p.K, nsb = K >> 8;
    const rsrc_t xr = make_rsrc(p.xp, (uint32_t)(CT * 16) * (uint32_t)K * 2u);
    const uint32_t xvo = ((uint32_t)r16 * (uint32_t)K + 8u * g) * 2u, xct = 16u * (uint32_t)K * 2u;
    int sb = wave;
    if (sb >= nsb) return;
    typename F::D cur, nxt;
    F::load(cur, row, nsb, sb, g);
    for (; sb < nsb; sb += KW) {
        const int nx = sb + KW < nsb ? sb + KW : sb;
        F::load(nxt, row, nsb, nx, g);
        uintx4 bf[CT][8];
#pragma unroll
        for (int ct = 0; ct < CT; ct++)
#pragma unroll
            for (int c = 0; c < 8; c++) bf[ct][c] = bld16(xr, xvo + ct * xct + 64 * c, uni((uint32_t)sb * 512u));
        const typename F::S sc = F::scales(cur, g);
#pragma unroll
        for (int c = 0; c < 8; c++) {
            const half8 a = F::frag(cur, sc, g, c);
#pragma unroll
            for (int ct = 0; ct < CT; ct++)
                acc[ct] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, __builtin_bit_cast(half8, bf[ct][c]), acc[ct], 0,
                                                                 0, 0);
        }
        cur = nxt;
    }
}

// One row tile per workgroup; in SWIGLU mode the workgroup computes the gate
// tile and then the up tile of the same 16 output features.
template <int CT, int KW>
__global__ __launch_bounds__(64 * KW) void k_qgemm(GemmParams p) {
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r16 = lane & 15, g = lane >> 4;
    const bool swi = p.mode == GM_SWIGLU;
    const int nt = swi ? 2 : 1;
    const GemmSeg S = swi ? p.seg[0] : seg_of_tile(p, blockIdx.x);
    const int rloc = swi ? (int)blockIdx.x * 16 : ((int)blockIdx.x - S.tile0) * 16;
    floatx4 acc[2][CT];
    for (int t = 0; t < nt; t++) {
        const GemmSeg St = (swi && t == 1) ? p.seg[1] : S;
        const WRow row = wrow(St, p.K, rloc);
#pragma unroll
        for (int ct = 0; ct < CT; ct++) acc[t][ct] = floatx4{0.f, 0.f, 0.f, 0.f};
        switch (St.fmt) {
        case Q4_K: gemm_body<Q4_K, CT, KW>(p, row, acc[t]); break;
        case Q5_K: gemm_body<Q5_K, CT, KW>(p, row, acc[t]); break;
        case Q6_K: gemm_body<Q6_K, CT, KW>(p, row, acc[t]); break;
        case Q8_0: gemm_body<Q8_0, CT, KW>(p, row, acc[t]); break;
        default: break;
        }
    }
    // fixed-order cross-wave reduction through LDS, one token tile at a time
    __shared__ floatx4 red[KW][2][64];
    const int r2[2] = {rloc, rloc};
    for (int ct = 0; ct < CT; ct++) {
        __syncthreads();
        for (int t = 0; t < nt; t++) red[wave][t][lane] = acc[t][ct];
        __syncthreads();
        if (wave != 0) continue;
        floatx4 v[2];
        for (int t = 0; t < nt; t++) {
            floatx4 s = red[0][t][lane];
            for (int w = 1; w < KW; w++) s += red[w][t][lane];
            v[t] = s;
        }
        const int m = ct * 16 + r16;
        if (swi) {
            epilogue<2>(p, S, r2, v, m, g);
        } else {
            const int r1[1] = {rloc};
            floatx4 v1[1] = {v[0]};
            epilogue<1>(p, S, r1, v1, m, g);
        }
    }
}

// --------------------------------------------------------------------------
// Launch policy.  KW (waves splitting K) is a function of the matrix only:
// the smallest power of two that puts >= 2048 waves on the chip for the M <= 16
// kernel, capped at 8 and at the number of superblocks.
// --------------------------------------------------------------------------
static int tiles_per_row_group(const GemmParams &p) { return p.mode == GM_SWIGLU ? p.seg[0].rows / 16 : p.ntiles; }

int qgemm_kw(const GemmParams &p) {
    const int nsb = p.K / 256;
    const int groups = tiles_per_row_group(p);  // row groups (16 rows, or gate+up pairs)
    int kw = 1;
    while (kw < 8 && groups * kw < 2048) kw *= 2;
    while (kw > 1 && kw > nsb) kw /= 2;
    if (p.mode == GM_SWIGLU && kw > 4) kw = 4;  // 2 x 8 waves would exceed 128 VGPRs per lane
    return kw;
}

int qgemm_workgroups(const GemmParams &p) {
    if (p.mode == GM_SWIGLU) return p.seg[0].rows / 16;
    return p.ntiles;
}

template <int NT, int KW>
static void launch_gemv(const GemmParams &p, int nwg, hipStream_t st) {
    hipLaunchKernelGGL((k_qgemv<NT, KW>), dim3(nwg), dim3(64 * KW * NT), 0, st, p);
}
template <int CT, int KW>
static void launch_gemm(const GemmParams &p, int nwg, hipStream_t st) {
    hipLaunchKernelGGL((k_qgemm<CT, KW>), dim3(nwg), dim3(64 * KW), 0, st, p);
}

int launch_qgemm(const GemmParams &p, hipStream_t st) {
    if (p.M < 1 || p.M > 128) throw BackendError("qgemm: M out of range");
    const int kw = qgemm_kw(p);
    const int nwg = qgemm_workgroups(p);
    if (p.M <= 16) {
        const int nt = p.mode == GM_SWIGLU ? 2 : 1;
#define SD_GEMV(T, W) if (nt == T && kw == W) { launch_gemv<T, W>(p, nwg, st); return nwg; }
        SD_GEMV(1, 1) SD_GEMV(1, 2) SD_GEMV(1, 4) SD_GEMV(1, 8)
        SD_GEMV(2, 1) SD_GEMV(2, 2) SD_GEMV(2, 4) SD_GEMV(2, 8)
#undef SD_GEMV
        throw BackendError("qgemv: unsupported launch shape");
    }
    const int ct = p.M <= 32 ? 2 : p.M <= 64 ? 4 : 8;
#define SD_GEMM(C, W) if (ct == C && kw == W) { launch_gemm<C, W>(p, nwg, st); return nwg; }
    SD_GEMM(2, 1) SD_GEMM(2, 2) SD_GEMM(2, 4) SD_GEMM(2, 8)
    SD_GEMM(4, 1) SD_GEMM(4, 2) SD_GEMM(4, 4) SD_GEMM(4, 8)
    SD_GEMM(8, 1) SD_GEMM(8, 2) SD_GEMM(8, 4) SD_GEMM(8, 8)
#undef SD_GEMM
    throw BackendError("qgemm: unsupported launch shape");
}

}  // namespace sd
