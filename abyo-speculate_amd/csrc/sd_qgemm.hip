// K1: fused GGUF dequant-matmul on CDNA4 MFMA, y[m][n] = sum_k x[m][k] * W[n][k].
//
// Replaces candle's QMatMul::forward at the reference's call sites
// (crates/speculate/src/model/quantized_llama_local.rs:47-49 MLP, :73-90 Q/K/V,
// :135 wo, :317 lm_head; quantized_qwen2_local.rs:41-44, 71-82, 138, 315).
//
// Both kernels multiply 16 weight rows x 32 K by 32 K x 16 tokens (fp16
// activations in fragment order) with v_mfma_f32_16x16x32_f16 and accumulate
// in f32.
//
//  * k_qmm (M <= 16, the linear-verify shape): one 16-token tile, products
//    transposed (tokens x rows).  A workgroup owns RT row tiles and KW waves
//    that split the K superblocks (wave w takes w, w+KW, ...), each with the
//    next superblock's weights and activations in flight; KW is chosen per
//    matrix so that every launch puts thousands of waves on the 256 CUs.
//    Q4_K / Q5_K weights enter the MFMA as exact integers (see kquant_int).
//  * k_qgx (M > 16, tree and prefill shapes): 4 waves share each superblock's
//    activations through LDS; CT token tiles per wave reuse every dequantised
//    weight fragment CT times.
//
// Accumulation order is fixed by the matrix alone: per wave, superblocks in
// increasing order and chunks c = 0..7 in order; across waves, partial sums
// meet in LDS and are added for w = 0..KW-1 in order.  KW depends only on
// (rows, K), never on M, so row i of an M-row call (M <= 16) equals the M=1
// call bit for bit.
//
// Dequantisation to fp16 (k_qgx, and Q6_K / Q8_0 in k_qmm): a code is OR'ed
// into the mantissa of 1024.0h (0x6400 | q == 1024 + q) or, for a code already
// at bits 4-7, of 64.0h (0x5400 | q << 4 == 64 + q).  Q6_K: q - 32 exactly,
// times the fp16 sub-block scale fp16(d * sc) in one v_pk_mul_f16.  Q8_0: q
// exactly, times the fp16 block scale in one v_pk_mul_f16.  Q4_K / Q5_K (k_qgx): q exactly, then one
// v_pk_fma_f16 with the sub-block's fp16 scale and min, round_f16(q * s16 -
// m16) where s16 = fp16(d * sc) and m16 = fp16(dmin * m).
#include <hip/hip_ext.h>

#include "sd_attn_dev.hpp"
#include "sd_buffer.hpp"
#include "sd_common.hpp"
#include "sd_kernels.hpp"
#include "sd_kernels_attn.hpp"
#include "sd_qcodes.hpp"

namespace sd {

typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// Compiler-visible forms only on the paths into MFMA operands: an inline-asm
// result read by an MFMA (or an MFMA result read by inline asm) escapes the
// compiler's hazard tracking, and the MFMA then sees a stale register.

// two fp16 codes -> code * s + c in one v_pk_fma_f16 (s, c fp16 pairs): exact
// when the result is a small integer (the K-quant integer path below)
__device__ __forceinline__ uint32_t pkfma(uint32_t p, uint32_t s, uint32_t c) {
    const half2v r = __builtin_elementwise_fma(__builtin_bit_cast(half2v, p), __builtin_bit_cast(half2v, s),
                                               __builtin_bit_cast(half2v, c));
    return __builtin_bit_cast(uint32_t, r);
}
// an f32 that fp16 holds exactly, in both halves of a word
__device__ __forceinline__ uint32_t h2pair(float v) {
    const uint32_t h = f2h(v);
    return h | (h << 16);
}
__device__ __forceinline__ half8 as_half8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    const uintx4 u = {a, b, c, d};
    return __builtin_bit_cast(half8, u);
}
// one lane's view of its weight row: resource of the whole matrix + row start
struct WRow {
    rsrc_t rs;
    uint32_t base;  // byte offset of the tile's first tile block (wave-uniform)
};
// --------------------------------------------------------------------------
// Per-format lane data.  Lane (r16 = lane & 15, g = lane >> 4) holds row r16
// of the tile and the 64 elements [64g, 64g + 64) of each superblock; chunk c
// of the lane covers the fragment slots g*8 .. g*8+7 of K-chunk c, i.e. the
// elements 64g + 32*(s >> 2) + 4c + {0,2,1,3}[s & 3].
// --------------------------------------------------------------------------
template <int FMT> struct QFmt;

// The lane group's scales and mins from the header's regrouped scale bytes
// (kq_hdr_pack): w = sc_2g | sc_2g+1 << 6 | m_2g << 12 | m_2g+1 << 18 is byte g
// of header words 1, 2, 3 (permute selector 12 gives a zero byte).
__device__ __forceinline__ uint32_t kquant_word(const uintx4 &hdr, int g) {
    const uint32_t lo = __builtin_amdgcn_perm(hdr.z, hdr.y, 0x0c0c0000u | (uint32_t)(4 + g) << 8 | (uint32_t)g);
    return __builtin_amdgcn_perm(hdr.w, lo, 0x0c000100u | (uint32_t)(4 + g) << 16);
}
__device__ __forceinline__ void kquant_ints(const uintx4 &hdr, int g, int (&sc)[2], int (&mn)[2]) {
    const uint32_t w = kquant_word(hdr, g);
    sc[0] = (int)(w & 63u);
    sc[1] = (int)((w >> 6) & 63u);
    mn[0] = (int)((w >> 12) & 63u);
    mn[1] = (int)(w >> 18);
}

// Loads address one tile block: the wave-uniform part (tile, superblock) goes
// in the scalar offset, the lane's fixed position inside the block in the
// vector offset (see the tile-block layout in sd_layout.hip).
// A negative sb is a load that must not happen: its offset is pushed past any
// resource size (a matrix is < 2 GiB), so the hardware range check returns
// zeros without touching memory (the same trick as composable_kernel's
// out-of-bounds buffer loads).  Loads can then be issued unconditionally,
// which keeps the compiler's wait-count bookkeeping exact across loop turns.
constexpr uint32_t kNoLoad = 0x80000000u;
__device__ __forceinline__ uint32_t tb_off(const WRow &w, int sb, int tbb) {
    return uni(sb < 0 ? kNoLoad : w.base + (uint32_t)sb * tbb);
}

// ---- K-quant integer path (M <= 16 kernel) -------------------------------------
// Q4_K / Q5_K weights are d * sc_j * q - dmin * m_j with 6-bit sc_j, m_j and
// q < 32.  The kernel feeds the MFMA the exact integers sc_j * q <= 63 * 31:
// one v_pk_fma_f16 of the code, (1024 + q) * sc - 1024 * sc (or the 64
// binade's), is exact.  A superblock's products then sum to
// sum_j sc_j sum_k q_k x_k, which is scaled by d in f32, and the mins term
// dmin * sum_j m_j X_j (X_j = sum of the activations of sub-block j) is a
// second small product on the MFMA with exact integer m_j.  Weights are thus
// used exactly instead of rounded to fp16, at two fewer instructions per code
// pair.
constexpr uint32_t kOff1024 = 0xE400E400u;  // (-1024, -1024) in fp16
constexpr uint32_t kOff64 = 0xD400D400u;    // (-64, -64)
struct KInt {
    uint32_t s0, c0, s1, c1;  // fp16 pairs: sc and -1024 sc (low nibbles), sc and -64 sc (high)
    uint32_t m;               // bf16 m of sub-blocks 2g and 2g + 1
    float d, dmin;
};
__device__ __forceinline__ KInt kquant_int(const uintx4 &hdr, int g) {
    int sc[2], mn[2];
    kquant_ints(hdr, g, sc, mn);
    KInt k;
    // (1024 + sc) twice is 0x6400 | sc in both halves; minus 1024 it is sc
    // exactly, and the offsets -1024 sc, -64 sc are exact fp16 products
    const half2v s0 = __builtin_bit_cast(half2v, (uint32_t)sc[0] * 0x10001u + 0x64006400u) +
                      __builtin_bit_cast(half2v, kOff1024);
    const half2v s1 = __builtin_bit_cast(half2v, (uint32_t)sc[1] * 0x10001u + 0x64006400u) +
                      __builtin_bit_cast(half2v, kOff1024);
    k.s0 = __builtin_bit_cast(uint32_t, s0);
    k.c0 = __builtin_bit_cast(uint32_t, s0 * __builtin_bit_cast(half2v, kOff1024));
    k.s1 = __builtin_bit_cast(uint32_t, s1);
    k.c1 = __builtin_bit_cast(uint32_t, s1 * __builtin_bit_cast(half2v, kOff64));
    // bf16 of a small integer: the top half of its f32
    k.m = (__float_as_uint((float)mn[0]) >> 16) | (__float_as_uint((float)mn[1]) & 0xffff0000u);
    k.d = h2f((uint16_t)(hdr.x & 0xffffu));
    k.dmin = h2f((uint16_t)(hdr.x >> 16));
    return k;
}

// fp16 pairs of one lane's two sub-blocks (see QFmt<Q4_K>::S)
struct KS16 {
    uint32_t s0, m0, s1, m1;
};
__device__ __forceinline__ KS16 kquant_s16(const uintx4 &hdr, int g) {
    const float d = h2f((uint16_t)(hdr.x & 0xffffu)), dmin = h2f((uint16_t)(hdr.x >> 16));
    int sc[2], mn[2];
    kquant_ints(hdr, g, sc, mn);
    KS16 k;
    k.s0 = h2pair(d * (float)sc[0]);  // exact f32 products, one rounding each
    k.m0 = h2pair(-(dmin * (float)mn[0]));
    k.s1 = h2pair(d * (float)sc[1]);
    k.m1 = h2pair(-(dmin * (float)mn[1]));
    return k;
}
// codes (off + q) -> round_f16(q * s + nm), q exact
__device__ __forceinline__ uint32_t qsm(uint32_t p, uint32_t off, uint32_t s, uint32_t nm) {
    const half2v q = __builtin_bit_cast(half2v, p) + __builtin_bit_cast(half2v, off);
    return pkfma(__builtin_bit_cast(uint32_t, q), s, nm);
}

template <> struct QFmt<Q4_K> {
    typedef LaneQ4K D;
    static constexpr bool kInt = true;
    static __device__ __forceinline__ KInt iscales(const D &r, int g) { return kquant_int(r.hdr, g); }
    static __device__ __forceinline__ half8 ifrag(const D &r, const KInt &s, int g, int c) {
        uint32_t p[4];
        r.codes(g, c, p);
        return as_half8(pkfma(p[0], s.s0, s.c0), pkfma(p[1], s.s0, s.c0), pkfma(p[2], s.s1, s.c1),
                        pkfma(p[3], s.s1, s.c1));
    }
    // Above 16 rows (weights as the MFMA's fp16 operand): the sub-block
    // scales as fp16 pairs, s = fp16(d * sc) and -m = -fp16(dmin * mn); a code
    // (1024 + q or 64 + q) minus its offset is q exactly, and one
    // v_pk_fma_f16 gives round_f16(q * s - m) (a single rounding of the exact
    // q * s - m).  Two packed instructions per pair of weights.
    typedef KS16 S;
    static __device__ __forceinline__ void load(D &r, const WRow &w, int nsb, int sb, int g) {
        const int lane = threadIdx.x & 63;
        const uint32_t so = tb_off(w, sb, D::TBB);
        r.hdr = bld16(w.rs, D::off_hdr(lane), so);
        r.q0 = bld16(w.rs, D::off_q0(lane), so);
        r.q1 = bld16(w.rs, D::off_q1(lane), so);
    }
    static __device__ __forceinline__ S scales(const D &r, int g) { return kquant_s16(r.hdr, g); }
    static __device__ __forceinline__ half8 frag(const D &r, const S &s, int g, int c) {
        uint32_t p[4];
        r.codes(g, c, p);
        return as_half8(qsm(p[0], kOff1024, s.s0, s.m0), qsm(p[1], kOff1024, s.s0, s.m0),
                        qsm(p[2], kOff64, s.s1, s.m1), qsm(p[3], kOff64, s.s1, s.m1));
    }
};

template <> struct QFmt<Q5_K> {
    typedef LaneQ5K D;
    typedef QFmt<Q4_K>::S S;
    static constexpr bool kInt = true;
    static __device__ __forceinline__ KInt iscales(const D &r, int g) { return kquant_int(r.hdr, g); }
    static __device__ __forceinline__ half8 ifrag(const D &r, const KInt &s, int g, int c) {
        uint32_t p[4];
        r.codes(g, c, p);
        return as_half8(pkfma(p[0], s.s0, s.c0), pkfma(p[1], s.s0, s.c0), pkfma(p[2], s.s1, s.c1),
                        pkfma(p[3], s.s1, s.c1));
    }
    static __device__ __forceinline__ void load(D &r, const WRow &w, int nsb, int sb, int g) {
        const int lane = threadIdx.x & 63;
        const uint32_t so = tb_off(w, sb, D::TBB);
        r.hdr = bld16(w.rs, D::off_hdr(lane), so);
        r.qh = bld8(w.rs, D::off_qh(lane), so);
        r.q0 = bld16(w.rs, D::off_q0(lane), so);
        r.q1 = bld16(w.rs, D::off_q1(lane), so);
    }
    static __device__ __forceinline__ S scales(const D &r, int g) { return kquant_s16(r.hdr, g); }
    static __device__ __forceinline__ half8 frag(const D &r, const S &s, int g, int c) {
        uint32_t p[4];
        r.codes(g, c, p);
        return as_half8(qsm(p[0], kOff1024, s.s0, s.m0), qsm(p[1], kOff1024, s.s0, s.m0),
                        qsm(p[2], kOff64, s.s1, s.m1), qsm(p[3], kOff64, s.s1, s.m1));
    }
};

template <> struct QFmt<Q6_K> {
    typedef LaneQ6K D;
    static constexpr bool kInt = false;  // sc * (q - 32) needs 13 bits, past fp16's exact integers
    // fp16 pairs of d * sc, [2 * s' + (c >= 4)]: a code (1024 + q6 or 64 + q6)
    // minus 1056 (or 96) is q6 - 32 exactly, and one v_pk_mul_f16 gives
    // round_f16((q6 - 32) * fp16(d * sc))
    struct S {
        uint32_t s[4];
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
        for (int i = 0; i < 4; i++) s.s[i] = h2pair(d * (float)(int8_t)((r.sc >> (8 * i)) & 0xffu));  // exact, one rounding
        return s;
    }
    static __device__ __forceinline__ uint32_t qmul(uint32_t p, uint32_t off, uint32_t sc) {
        const half2v q = __builtin_bit_cast(half2v, p) + __builtin_bit_cast(half2v, off);
        return __builtin_bit_cast(uint32_t, q * __builtin_bit_cast(half2v, sc));
    }
    static __device__ __forceinline__ half8 frag(const D &r, const S &s, int g, int c) {
        uint32_t p[4];
        r.codes(g, c, p);
        const int hl = c >= 4 ? 1 : 0;
        const uint32_t sa = s.s[hl], sb = s.s[2 + hl];
        constexpr uint32_t off1056 = 0xE420E420u, off96 = 0xD600D600u;  // (-1056, -1056), (-96, -96) in fp16
        return as_half8(qmul(p[0], off1056, sa), qmul(p[1], off1056, sa), qmul(p[2], off96, sb),
                        qmul(p[3], off96, sb));
    }
};

template <> struct QFmt<Q8_0> {
    typedef LaneQ80 D;
    // d of blocks 2g and 2g+1 in both halves of a word: fp16 (d * q) with d
    // itself fp16 is one v_pk_mul_f16 of the exact integer q, the same single
    // rounding as the f32 route at a third of its cost
    struct S {
        uint32_t d0, d1;
    };
    static constexpr bool kInt = false;  // one scale per 32 elements: an MFMA's K spans 8 of them
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
        S s;
        s.d0 = (r.d & 0xffffu) * 0x10001u;
        s.d1 = (r.d >> 16) * 0x10001u;
        return s;
    }
    // codes 1024 + (q + 128) -> q (exact) -> round_f16(q * d)
    static __device__ __forceinline__ uint32_t qd2(uint32_t p, uint32_t d) {
        const half2v q = __builtin_bit_cast(half2v, p) + (half2v){(_Float16)-1152.f, (_Float16)-1152.f};
        return __builtin_bit_cast(uint32_t, q * __builtin_bit_cast(half2v, d));
    }
    static __device__ __forceinline__ half8 frag(const D &r, const S &s, int g, int c) {
        uint32_t p[4];
        r.codes(g, c, p);
        return as_half8(qd2(p[0], s.d0), qd2(p[1], s.d0), qd2(p[2], s.d1), qd2(p[3], s.d1));
    }
};

__device__ __forceinline__ float silu_f(float g) { return g / (1.0f + __expf(-g)); }

// --------------------------------------------------------------------------
// Epilogue of one wave's row tiles: v[rt] is the full sum of row tile rt (the
// lane holds rows rloc[rt] + 4g + i of token m).  SWIGLU: tiles [0, RT/2) are
// gate tiles and [RT/2, RT) the up tiles of the same features.  GM_LOGITS also
// writes the tiles' argmax partial of every token (first max wins) to `slot`.
// --------------------------------------------------------------------------
// four fp16 values to one 8-byte store
// DEV: a device-scope store (read by other workgroups of the same launch)
template <bool DEV = false> __device__ __forceinline__ void st4h(uint16_t *dst, float a, float b, float c, float d) {
    const uintx2 v{(uint32_t)f2h(a) | ((uint32_t)f2h(b) << 16), (uint32_t)f2h(c) | ((uint32_t)f2h(d) << 16)};
    if constexpr (DEV) st_dev64(dst, (uint64_t)v.x | ((uint64_t)v.y << 32));
    else *(uintx2 *)dst = v;
}

// Operands the epilogue reads besides the accumulators, requested when the
// kernel starts so that they arrive during the main loop instead of costing a
// memory round trip after it: the residual rows (GM_RESID), the next norm's
// weights, the bias and, for RoPE, the position and its cos/sin entries.
template <int RT> struct EpiPre {
    floatx4 a[RT];  // GM_RESID: the residual rows; otherwise the bias
    floatx4 w[RT];  // GM_RESID with next_w: the next norm's weights
    int pos;
    float cs[4], sn[4];
};

// RoPE geometry of a lane (RT == 2): tile 0 holds elements d..d+3 of a head
// (d < hd/2), tile 1 elements d+hd/2..; which = 0 q, 1 k, 2 v
struct RopeLane {
    int which, head, d;
};
template <int RT>
__device__ __forceinline__ RopeLane rope_lane(const GemmParams &p, const GemmSeg (&S)[RT], const int (&rloc)[RT],
                                              int g) {
    const RopeOut &R = p.rope;
    const int qd = R.n_heads * R.hd, kvd = R.n_kv * R.hd;
    const int col = S[0].col0 + rloc[0] + 4 * g;
    RopeLane L;
    L.which = col < qd ? 0 : col < qd + kvd ? 1 : 2;
    const int rel = col - (L.which == 0 ? 0 : L.which == 1 ? qd : qd + kvd);
    L.head = rel / R.hd;
    L.d = rel % R.hd;
    return L;
}

// all loads unconditional (padding tokens read the last real token's data)
template <int RT>
__device__ __forceinline__ void epi_prefetch(const GemmParams &p, const GemmSeg (&S)[RT], const int (&rloc)[RT],
                                             int m, int g, EpiPre<RT> &e) {
    const int ml = min(m, p.M - 1);
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        const int n0 = rloc[rt] + 4 * g;
        if (p.mode == GM_RESID) {
            e.a[rt] = *(const floatx4 *)(S[rt].out + (int64_t)ml * S[rt].ldo + S[rt].col0 + n0);
            if (p.next_w) e.w[rt] = *(const floatx4 *)(p.next_w + S[rt].col0 + n0);
        } else if (S[rt].bias) {
            e.a[rt] = *(const floatx4 *)(S[rt].bias + n0);
        }
    }
    if (p.rope.q16) e.pos = p.rope.pos[ml];
}
// after the position has arrived (called once the weight prologue is in flight)
template <int RT>
__device__ __forceinline__ void epi_prefetch_rope(const GemmParams &p, const GemmSeg (&S)[RT], const int (&rloc)[RT],
                                                  int g, EpiPre<RT> &e) {
    if (!p.rope.q16) return;
    const RopeOut &R = p.rope;
    const RopeLane L = rope_lane<RT>(p, S, rloc, g);
    const int half = R.hd / 2;
    const float *ct = R.cos_t + (int64_t)e.pos * half, *sn = R.sin_t + (int64_t)e.pos * half;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        // rope_i: pair index (d + rt * hd/2 + 2j) / 2 for slot i = 2 rt + j; rope: d + i
        const int f = R.interleaved ? (L.d + (i >> 1) * half + 2 * (i & 1)) >> 1 : L.d + i;
        e.cs[i] = ct[f];
        e.sn[i] = sn[f];
    }
}

// RoPE + KV append of one lane's rows (RT == 2).  Rotation as
// LayerWeights::rope_at_positions (quantized_llama_local.rs:94-105,
// quantized_qwen2_local.rs:98-109): (x0 c - x1 s, x0 s + x1 c) on the pairs
// (2i, 2i+1) inside a tile (rope_i) or (i, i + hd/2) across the two (rope).
// DEV: device-scope stores, for the attention workgroups of the same launch.
template <int RT, bool DEV>
__device__ __forceinline__ void rope_epilogue(const GemmParams &p, const GemmSeg (&S)[RT], const int (&rloc)[RT],
                                              const floatx4 (&v)[RT], const EpiPre<RT> &e, int m, int g) {
    if constexpr (RT == 2) {
        const RopeOut &R = p.rope;
        const int hd = R.hd, half = hd / 2;
        const RopeLane L = rope_lane<RT>(p, S, rloc, g);
        float x[2][4];
#pragma unroll
        for (int rt = 0; rt < 2; rt++) {
            floatx4 r = v[rt];
            if (S[rt].bias) r += e.a[rt];
#pragma unroll
            for (int i = 0; i < 4; i++) x[rt][i] = r[i];
        }
        const int64_t t = (int64_t)R.P + m;
        if (L.which < 2) {
            float y[2][4];
            if (R.interleaved) {
#pragma unroll
                for (int rt = 0; rt < 2; rt++)
#pragma unroll
                    for (int i = 0; i < 4; i += 2) {
                        const float c = e.cs[2 * rt + i / 2], s = e.sn[2 * rt + i / 2];
                        y[rt][i] = x[rt][i] * c - x[rt][i + 1] * s;
                        y[rt][i + 1] = x[rt][i] * s + x[rt][i + 1] * c;
                    }
            } else {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float c = e.cs[i], s = e.sn[i];
                    y[0][i] = x[0][i] * c - x[1][i] * s;
                    y[1][i] = x[0][i] * s + x[1][i] * c;
                }
            }
#pragma unroll
            for (int rt = 0; rt < 2; rt++) {
                const int dd = L.d + rt * half;
                uint16_t *dst = L.which == 0 ? R.q16 + ((int64_t)L.head * p.M + m) * hd + dd
                                             : R.kc + (int64_t)L.head * R.cap * hd + kv_k_off(t, dd, hd);
                st4h<DEV>(dst, y[rt][0], y[rt][1], y[rt][2], y[rt][3]);
            }
        } else {
            uint16_t *vs = R.vc + (int64_t)L.head * R.cap * hd;
#pragma unroll
            for (int rt = 0; rt < 2; rt++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    uint16_t *dst = vs + kv_v_off(t, L.d + rt * half + i, hd);
                    if constexpr (DEV) st_dev16(dst, f2h(x[rt][i]));
                    else *dst = f2h(x[rt][i]);
                }
        }
    }
}

template <int RT, bool DEV = false>
__device__ __forceinline__ void epilogue(const GemmParams &p, const GemmSeg (&S)[RT], const int (&rloc)[RT],
                                         const floatx4 (&v)[RT], const EpiPre<RT> &e, int m, int g, int slot) {
    const bool live = m < p.M;
    if (p.rope.q16) {
        if (live) rope_epilogue<RT, DEV>(p, S, rloc, v, e, m, g);
        return;
    }
    if (p.mode == GM_SWIGLU) {
        if (live) {
            uint16_t *dst = p.act + (int64_t)m * p.act_ld;
#pragma unroll
            for (int f = 0; f < RT / 2; f++) {
                const int n0 = rloc[f] + 4 * g;
#pragma unroll
                for (int i = 0; i < 4; i++) dst[frag_index(n0 + i)] = f2h(silu_f(v[f][i]) * v[RT / 2 + f][i]);
            }
        }
        return;
    }
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    float ss[RT];  // next_w: this lane's share of the tile's sum of squares
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        ss[rt] = 0.f;
        if (!live) continue;
        const int n0 = rloc[rt] + 4 * g;
        float *o = S[rt].out + (int64_t)m * S[rt].ldo + S[rt].col0 + n0;
        floatx4 r = v[rt];
        if (p.mode == GM_RESID) {
            r += e.a[rt];
        } else if (S[rt].bias) {
            r += e.a[rt];
        }
        *(floatx4 *)o = r;
        if (p.next_w) {
            // features n .. n+3 sit in fragment slots f, f+2, f+1, f+3 (frag_slot)
            const int n = S[rt].col0 + n0;
            const floatx4 w = e.w[rt];
            st4h(p.next_u + (int64_t)m * p.next_ld + frag_index(n), r[0] * w[0], r[2] * w[2], r[1] * w[1],
                 r[3] * w[3]);
            ss[rt] = (r[0] * r[0] + r[1] * r[1]) + (r[2] * r[2] + r[3] * r[3]);
        }
        if (p.mode == GM_LOGITS) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float x = r[i];
                const int idx = S[rt].col0 + n0 + i;
                if (x > -INFINITY && (x > bv || (x == bv && idx < bi))) {
                    bv = x;
                    bi = idx;
                }
            }
        }
    }
    if (p.next_w) {
        // per tile: the 4 lanes of a token (g = 0..3) add their rows in a fixed order
#pragma unroll
        for (int rt = 0; rt < RT; rt++) {
            float s = ss[rt];
            s += __shfl_xor(s, 16);
            s += __shfl_xor(s, 32);
            if (g == 0 && live) p.next_ssq[(int64_t)m * p.ntiles + (S[rt].col0 + rloc[rt]) / 16] = s;
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
            p.amax_v[(int64_t)m * p.amax_ld + slot] = bv;
            p.amax_i[(int64_t)m * p.amax_ld + slot] = bi;
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
// The kernel: a workgroup owns RT row tiles (a "row group") and KW waves that
// split the K superblocks (wave w takes w, w + KW, ...); each wave multiplies
// its RT tiles by CT token tiles, so every activation fragment it loads feeds
// RT MFMAs and every dequantised weight fragment CT of them.
// ==========================================================================
// Vector-memory loads complete in issue order, so a wait on one load also
// waits for every older one.  Each step therefore issues the loads it will
// wait on first and the prefetch of the next step's operands after them.

// One superblock of the token tile: the activations arrive with the weights
// (both prefetched one step ahead, in two register sets).  The products are
// transposed, D[token][row] = x . W^T (activations as the MFMA's A operand),
// so that a lane's accumulators belong to its own weight row (r16) and that
// row's scales apply to them directly; the reduction transposes back.
// `sel` picks, per lane, the sub-block sums X_2g, X_2g+1 of the lane's token
// out of one extra product per chunk (see kquant_int).
// The integer path's per-superblock products (sum_j sc_j sum q x per row, the
// sub-block sums X of the token) are applied one superblock late, while the
// next superblock's MFMAs run: reading an MFMA result right after the MFMA
// waits for its whole pipeline, which would otherwise stall every superblock.
template <int RT> struct IntCarry {
    floatx4 part[RT], xs;
    float d[RT], dmin[RT];
    uint32_t m[RT];
    bool live;
};
// acc += d * part - dmin * sum_j m_j X_j for the carried superblock
template <int RT>
__device__ __forceinline__ void int_drain(IntCarry<RT> &cy, floatx4 (&acc)[RT]) {
    if (!cy.live) return;
    const floatx4 zero = {0.f, 0.f, 0.f, 0.f};
    // X_2g, X_2g+1 of the lane's token as bf16 hi + lo: 16 significant bits
    // and the f32 range (a sum of 32 activations can exceed fp16's), times
    // the integer mins, exact in bf16; hi and lo take slots 0, 1 and 2, 3 of
    // one product (the mins repeated), so one MFMA sums all four
    const __bf16 h0 = (__bf16)cy.xs[0], h1 = (__bf16)cy.xs[1];
    const __bf16 l0 = (__bf16)(cy.xs[0] - (float)h0), l1 = (__bf16)(cy.xs[1] - (float)h1);
    const bf16x8 xa = {h0, h1, l0, l1, 0, 0, 0, 0};
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        const bf16x8 mb = __builtin_bit_cast(bf16x8, uintx4{cy.m[rt], cy.m[rt], 0u, 0u});
        const floatx4 pm = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa, mb, zero, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; i++)
            acc[rt][i] = __builtin_fmaf(-cy.dmin[rt], pm[i], __builtin_fmaf(cy.d[rt], cy.part[rt][i], acc[rt][i]));
    }
    cy.live = false;
}

// One superblock of the token tile: the activations arrive with the weights
// (both prefetched one step ahead, in two register sets).  The products are
// transposed, D[token][row] = x . W^T (activations as the MFMA's A operand),
// so that a lane's accumulators belong to its own weight row (r16) and that
// row's scales apply to them directly; the reduction transposes back.
// `sel` picks, per lane, the sub-block sums X_2g, X_2g+1 of the lane's token
// out of one extra product per chunk (see kquant_int).
template <int FMT, int RT>
__device__ __forceinline__ void qmm_step1(const typename QFmt<FMT>::D (&w)[RT], const uintx4 (&b)[8], int g,
                                          floatx4 (&acc)[RT], const half8 &sel, IntCarry<RT> &cy) {
    typedef QFmt<FMT> F;
    const floatx4 zero = {0.f, 0.f, 0.f, 0.f};
    if constexpr (F::kInt) {
        KInt ks[RT];
#pragma unroll
        for (int rt = 0; rt < RT; rt++) ks[rt] = F::iscales(w[rt], g);
        floatx4 xs = zero, part[RT];
#pragma unroll
        for (int c = 0; c < 8; c++) {
            const half8 xc = __builtin_bit_cast(half8, b[c]);
            xs = __builtin_amdgcn_mfma_f32_16x16x32_f16(sel, xc, xs, 0, 0, 0);
#pragma unroll
            for (int rt = 0; rt < RT; rt++)
                part[rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xc, F::ifrag(w[rt], ks[rt], g, c),
                                                                  c == 0 ? zero : part[rt], 0, 0, 0);
            if (c == 0) int_drain<RT>(cy, acc);  // the previous superblock, behind this one's MFMAs
        }
        cy.xs = xs;
#pragma unroll
        for (int rt = 0; rt < RT; rt++) {
            cy.part[rt] = part[rt];
            cy.d[rt] = ks[rt].d;
            cy.dmin[rt] = ks[rt].dmin;
            cy.m[rt] = ks[rt].m;
        }
        cy.live = true;
    } else {
        typename F::S sc[RT];
#pragma unroll
        for (int rt = 0; rt < RT; rt++) sc[rt] = F::scales(w[rt], g);
#pragma unroll
        for (int c = 0; c < 8; c++) {
            const half8 xc = __builtin_bit_cast(half8, b[c]);
#pragma unroll
            for (int rt = 0; rt < RT; rt++)
                acc[rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xc, F::frag(w[rt], sc[rt], g, c), acc[rt], 0, 0, 0);
        }
    }
}

// The activations of superblock sb: XL loads of 16 bytes per lane.  XL = 8:
// load c is chunk c of token r16.  XL = 4 (up to 8 tokens): lanes r16 < 8 load
// chunk 2j of token r16 and lanes r16 >= 8 chunk 2j + 1 of token r16 - 8 (the
// lane's xvo carries the chunk and token), so load j holds chunk 2j for the
// live tokens and chunk 2j + 1 one row of 8 lanes up (see x_chunks).  XL = 2
// (up to 4 tokens): lane group q = r16 / 4 loads chunk 4j + q of token r16 % 4.
template <int XL>
__device__ __forceinline__ void load_x(uintx4 (&b)[XL], rsrc_t xr, uint32_t xvo, int sb) {
    const uint32_t so = uni(sb < 0 ? kNoLoad : (uint32_t)sb * 512u);
#pragma unroll
    for (int c = 0; c < XL; c++) b[c] = bld16(xr, xvo + (512 / XL) * c, so);
}
// the 8 chunk operands of a superblock: with XL = 4, chunk 2j + 1 of token t
// comes from lane t + 8 of the same 16-lane row (rows t >= 8 of the MFMA
// tile hold other data; their products belong to no token and are dropped)
// DPP row_shl:N: lane i of each 16-lane row takes lane i + N (i < 16 - N);
// the upper N lanes, whose token rows are padding wherever a shift is used,
// read zero (bound_ctrl), so the move needs no copy of the old value
template <int N> __device__ __forceinline__ uint32_t row_shl(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x100 + N, 0xF, 0xF, true);
}
template <int N> __device__ __forceinline__ uintx4 row_shl4(const uintx4 &v) {
    return uintx4{row_shl<N>(v.x), row_shl<N>(v.y), row_shl<N>(v.z), row_shl<N>(v.w)};
}
template <int XL>
__device__ __forceinline__ void x_chunks(const uintx4 (&b)[XL], uintx4 (&x)[8]) {
    if constexpr (XL == 8) {
#pragma unroll
        for (int c = 0; c < 8; c++) x[c] = b[c];
    } else if constexpr (XL == 4) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            x[2 * j] = b[j];
            x[2 * j + 1] = row_shl4<8>(b[j]);
        }
    } else {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            x[4 * j] = b[j];
            x[4 * j + 1] = row_shl4<4>(b[j]);
            x[4 * j + 2] = row_shl4<8>(b[j]);
            x[4 * j + 3] = row_shl4<12>(b[j]);
        }
    }
}

// ---- fused RMSNorm, input side ------------------------------------------------
// The sums of squares of token m arrive as K/16 partials, one per 16-element
// tile of h, i.e. 16 per superblock.  They travel with the superblocks: the
// wave that multiplies superblock sb also loads its 16 partials (lane (r16, g)
// the 4 of token r16 at 4g) and adds them to a running sum; the waves' sums
// meet in the cross-wave reduction and the 4 lane groups' by xor-shuffles,
// in a fixed order that depends on the matrix only.
struct NormSrc {
    rsrc_t r;
    uint32_t vo;  // the lane's float4 inside a superblock's 16 partials
};
__device__ __forceinline__ NormSrc norm_src(const GemmParams &p) {
    const int lane = threadIdx.x & 63, r16 = lane & 15, g = lane >> 4;
    NormSrc n;
    // no norm: an empty resource, every load reads zero without a memory access
    n.r = make_rsrc(p.norm_ssq, p.norm_ssq ? (uint32_t)(p.M * p.norm_parts * 4) : 0u);
    n.vo = (uint32_t)(min(r16, p.M - 1) * p.norm_parts + 4 * g) * 4u;
    return n;
}
__device__ __forceinline__ floatx4 norm_load(const NormSrc &n, int sb) {
    return __builtin_bit_cast(floatx4, bld16(n.r, n.vo, uni(sb < 0 ? kNoLoad : (uint32_t)sb * 64u)));
}
__device__ __forceinline__ float norm_add(float s, const floatx4 &v) { return s + ((v.x + v.y) + (v.z + v.w)); }

// Superblocks sb = ks, ks + KW, ... in increasing order, x and weights of the
// next superblock in flight during this one; `after_prologue` runs once the
// first superblock's loads are in flight.
template <int FMT, int RT, int KW, int XL, typename Hook>
__device__ __forceinline__ void qmm_body(const GemmParams &p, const WRow (&row)[RT], int ks, floatx4 (&acc)[RT],
                                         float &nsum, const half8 &sel, Hook &&after_prologue) {
    typedef QFmt<FMT> F;
    const int lane = threadIdx.x & 63;
    const int r16 = lane & 15, g = lane >> 4;
    const int nsb = p.K >> 8;
    // token rows past M read the last real token's row: the loads coalesce
    // with that lane's and the padding tokens are never stored
    const rsrc_t xr = make_rsrc(p.xp, (uint32_t)p.M * (uint32_t)p.K * 2u);
    const uint32_t xvo = XL == 8   ? ((uint32_t)min(r16, p.M - 1) * (uint32_t)p.K + 8u * g) * 2u
                         : XL == 4 ? ((uint32_t)min(r16 & 7, p.M - 1) * (uint32_t)p.K + 8u * g) * 2u + (r16 >= 8 ? 64u : 0u)
                                   : ((uint32_t)min(r16 & 3, p.M - 1) * (uint32_t)p.K + 8u * g) * 2u + 64u * (uint32_t)(r16 >> 2);
    if (ks >= nsb) return;
    const int nst = (nsb - ks + KW - 1) / KW;  // superblocks of this wave: ks + i * KW, i < nst
    auto sbi = [&](int i) { return i < nst ? ks + i * KW : -1; };
    typename F::D w0[RT], w1[RT];
    uintx4 b0[XL], b1[XL], xc[8];
    const NormSrc ns = norm_src(p);
    load_x<XL>(b0, xr, xvo, sbi(0));
#pragma unroll
    for (int rt = 0; rt < RT; rt++) F::load(w0[rt], row[rt], nsb, sbi(0), g);
    floatx4 n0 = norm_load(ns, sbi(0)), n1;  // after the weights: waiting for them does not wait for it
    after_prologue();
    IntCarry<RT> cy;
    cy.live = false;
    for (int i = 0;; i += 2) {
        load_x<XL>(b1, xr, xvo, sbi(i + 1));
#pragma unroll
        for (int rt = 0; rt < RT; rt++) F::load(w1[rt], row[rt], nsb, sbi(i + 1), g);
        n1 = norm_load(ns, sbi(i + 1));
        x_chunks<XL>(b0, xc);
        qmm_step1<FMT, RT>(w0, xc, g, acc, sel, cy);
        nsum = norm_add(nsum, n0);
        if (i + 1 >= nst) break;
        load_x<XL>(b0, xr, xvo, sbi(i + 2));
#pragma unroll
        for (int rt = 0; rt < RT; rt++) F::load(w0[rt], row[rt], nsb, sbi(i + 2), g);
        n0 = norm_load(ns, sbi(i + 2));
        x_chunks<XL>(b1, xc);
        qmm_step1<FMT, RT>(w1, xc, g, acc, sel, cy);
        nsum = norm_add(nsum, n1);
        if (i + 2 >= nst) break;
    }
    int_drain<RT>(cy, acc);
}

// One workgroup (index wg) of the M <= 16 launch.  DONE (the fused Q/K/V +
// attention launch): the epilogue's stores are made at device scope and, once
// they are complete, the workgroup writes epoch to flags[wg].
template <int RT, int KW, int XL, bool DONE = false>
__device__ __forceinline__ void qmm_wg(const GemmParams &p, int wg, unsigned *flags = nullptr, unsigned epoch = 0) {
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r16 = lane & 15, g = lane >> 4;
    GemmSeg S[RT];
    int rloc[RT];
    if (p.mode == GM_SWIGLU) {
        // feature tiles f0 .. f0 + RT/2 - 1: their gate tiles, then their up tiles
        const int f0 = wg * (RT / 2);
#pragma unroll
        for (int rt = 0; rt < RT; rt++) {
            S[rt] = rt < RT / 2 ? p.seg[0] : p.seg[1];
            rloc[rt] = (f0 + rt % (RT / 2)) * 16;
        }
    } else {
        // RT consecutive tiles of one segment (segment sizes are multiples of
        // RT).  With RoPE in the epilogue (RT == 2) the pair is instead tiles j
        // and j + hd/32 of one head, so the lane holding element d of a head
        // also holds d + hd/2, the partner of the half rotation.
        int t0 = wg * RT, tstep = 1;
        if (RT == 2 && p.rope.q16) {
            const int half = p.rope.hd / 32;
            t0 = (wg / half) * 2 * half + wg % half;
            tstep = half;
        }
        const GemmSeg s = seg_of_tile(p, t0);
#pragma unroll
        for (int rt = 0; rt < RT; rt++) {
            S[rt] = s;
            rloc[rt] = (t0 - s.tile0 + rt * tstep) * 16;
        }
    }
    WRow row[RT];
#pragma unroll
    for (int rt = 0; rt < RT; rt++) row[rt] = wrow(S[rt], p.K, rloc[rt]);
    floatx4 acc[RT];
#pragma unroll
    for (int rt = 0; rt < RT; rt++) acc[rt] = floatx4{0.f, 0.f, 0.f, 0.f};
    // Sub-block selector of the K-quant integer path: row r = 4 * gq + u
    // (u < 2) of the 16 x 32 selector is 1 on the elements of sub-block
    // 2 * gq + u, so selector x x^T puts X_2g, X_2g+1 of token t in the first
    // two accumulators of lane (t, g).  Lane (r, g) holds the selector's
    // elements of sub-blocks 2g (slots 0-3) and 2g + 1 (slots 4-7).
    half8 sel;
    {
        const int u = r16 & 3, gq = r16 >> 2;
#pragma unroll
        for (int j = 0; j < 8; j++) sel[j] = (_Float16)((gq == g && u == (j >> 2)) ? 1.f : 0.f);
    }
    // Wave 0 runs the epilogue: it requests the epilogue's operands first and
    // the RoPE table entries (which need the position) once its weights are in
    // flight.  Every wave sums the fused-norm partials of its superblocks.
    EpiPre<RT> e;
    if (wave == 0) epi_prefetch<RT>(p, S, rloc, r16, g, e);
    auto after_prologue = [&]() {
        if (wave == 0) epi_prefetch_rope<RT>(p, S, rloc, g, e);
    };
    float nsum = 0.f;
    switch (S[0].fmt) {
    case Q4_K: qmm_body<Q4_K, RT, KW, XL>(p, row, wave, acc, nsum, sel, after_prologue); break;
    case Q5_K: qmm_body<Q5_K, RT, KW, XL>(p, row, wave, acc, nsum, sel, after_prologue); break;
    case Q6_K: qmm_body<Q6_K, RT, KW, XL>(p, row, wave, acc, nsum, sel, after_prologue); break;
    case Q8_0: qmm_body<Q8_0, RT, KW, XL>(p, row, wave, acc, nsum, sel, after_prologue); break;
    default: break;
    }
    // Fixed-order cross-wave reduction (w = 0, 1, ..., KW-1) through LDS, which
    // also transposes the products back: wave w's lane (row r, g) holds tokens
    // 4g .. 4g+3 of row r; wave 0's lane (token t, g) reads rows 4g .. 4g+3 of
    // token t, the layout of the epilogue.  The norm sums ride along.
    constexpr int kPitch = 20;  // floats per token row: 16 rows + 4, keeps 16-byte reads aligned
    __shared__ __attribute__((aligned(16))) float red[KW][RT][16][kPitch];
    __shared__ float nred[KW][64];
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int i = 0; i < 4; i++) red[wave][rt][4 * g + i][r16] = acc[rt][i];
    nred[wave][lane] = nsum;
    __syncthreads();
    if (wave != 0) return;
    floatx4 v[RT];
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        floatx4 t = *(const floatx4 *)&red[0][rt][r16][4 * g];
#pragma unroll
        for (int w = 1; w < KW; w++) t += *(const floatx4 *)&red[w][rt][r16][4 * g];
        v[rt] = t;
    }
    float ns = nred[0][lane];
#pragma unroll
    for (int w = 1; w < KW; w++) ns += nred[w][lane];
    if (p.norm_ssq) {
        // the token's four lane groups (g = 0..3) in a fixed order
        ns += __shfl_xor(ns, 16);
        ns += __shfl_xor(ns, 32);
        const float inv = 1.0f / sqrtf(ns / (float)p.K + p.norm_eps);
#pragma unroll
        for (int rt = 0; rt < RT; rt++) v[rt] *= inv;
    }
    if constexpr (!DONE) {
        epilogue<RT>(p, S, rloc, v, e, r16, g, wg);
        return;
    }
    epilogue<RT, true>(p, S, rloc, v, e, r16, g, wg);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (lane == 0) __hip_atomic_store(flags + wg, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int RT, int KW, int XL>
__global__ __launch_bounds__(64 * KW) __attribute__((amdgpu_waves_per_eu(2))) void k_qmm(GemmParams p) {
    warm_kernargs<sizeof(GemmParams)>();
    qmm_wg<RT, KW, XL>(kernarg<GemmParams>(), blockIdx.x);
}

// ---- the fused Q/K/V + attention launch (M <= 16) ----
// Workgroups [0, nprod) are the Q/K/V matmul's (k_qmm<2, 8, XL>, RoPE and the
// KV append in the epilogue, stored at device scope), the rest the
// attention's (attn_wg): those request their first cached keys at once, wait
// until the Q/K/V workgroups of their KV head's rows have flagged them stored
// (attn_wait), then read the queries and the new rows.  The attention's
// launch, argument fetch and first cache reads so overlap the matmul instead
// of following it.  Progress: a workgroup of either kind fills a CU (two waves
// per SIMD), the launch has no more workgroups than CUs (qkv_attention_fits),
// and the Q/K/V workgroups never wait.
struct QkvAttnArgs {
    GemmParams g;
    AttnWait w;
    int nprod;
    AttnParams a;
};

template <int HD, int XL>
__global__ __launch_bounds__(kAttnThreads) __attribute__((amdgpu_waves_per_eu(2))) void k_qkv_attn(QkvAttnArgs) {
    warm_kernargs<sizeof(QkvAttnArgs)>();
    const GemmParams &g = kernarg<GemmParams, offsetof(QkvAttnArgs, g)>();
    const AttnWait &w = kernarg<AttnWait, offsetof(QkvAttnArgs, w)>();
    const int nprod = kernarg<int, offsetof(QkvAttnArgs, nprod)>();
    const AttnParams &a = kernarg<AttnParams, offsetof(QkvAttnArgs, a)>();
    if ((int)blockIdx.x < nprod) {
        qmm_wg<2, 8, XL, true>(g, blockIdx.x, w.flags, w.epoch);
        return;
    }
    // KV head fastest: with n_kv a multiple of the 8 XCDs every workgroup of a
    // head shares one XCD's L2
    const int i = (int)blockIdx.x - nprod, h = i % a.n_kv, r = i / a.n_kv;
    attn_wg<HD, true>(a, h, r % a.nsplit, r / a.nsplit, w);
}

// ==========================================================================
// M > 16 (tree and prefill shapes).  A workgroup of 4 waves owns a row block
// -- 4 x RW row tiles, or for gate/up 4 features' gate and up tiles -- and one
// K slice.  The slice's activations are staged superblock by superblock in
// LDS, so each activation byte is fetched from L2 once per workgroup and read
// by all 4 waves (reading them per wave from L1 made the M = 60 launches L2
// bound); the weights stream into registers one superblock ahead.  With more
// than one K slice the launch writes per-slice partial sums and the kernel
// that consumes the output adds them (GM_STORE / GM_RESID callers only).
// ==========================================================================
constexpr int XG_WAVES = 4;
constexpr int XG_PITCH = 528;  // bytes per staged token row: 512 + 16 keeps ds_read_b128 conflict free

template <int CT> struct XStage {
    uintx4 v[2 * CT];  // CT*16 rows x 32 16-byte pieces over 256 threads
};

// the activations of superblock sb (a negative sb loads nothing)
template <int CT>
__device__ __forceinline__ void xg_load(XStage<CT> &st, rsrc_t xr, int M, int K, int sb) {
    const uint32_t so = uni(sb < 0 ? kNoLoad : (uint32_t)sb * 512u);
#pragma unroll
    for (int i = 0; i < 2 * CT; i++) {
        const int piece = (int)threadIdx.x + 256 * i, r = piece >> 5, col = piece & 31;
        const uint32_t vo = r < M ? (uint32_t)r * (uint32_t)K * 2u + (uint32_t)col * 16u : kNoLoad;
        st.v[i] = bld16(xr, vo, so);
    }
}
template <int CT> __device__ __forceinline__ void xg_store(const XStage<CT> &st, uint8_t *buf) {
#pragma unroll
    for (int i = 0; i < 2 * CT; i++) {
        const int piece = (int)threadIdx.x + 256 * i, r = piece >> 5, col = piece & 31;
        *(uintx4 *)(buf + r * XG_PITCH + col * 16) = st.v[i];
    }
}

template <int FMT, int RW, int CT>
__device__ __forceinline__ void qgx_step(const typename QFmt<FMT>::D (&w)[RW], const uint8_t *xb,
                                         const uint32_t (&boff)[CT], int g, floatx4 (&acc)[RW][CT]) {
    typedef QFmt<FMT> F;
    typename F::S sc[RW];
#pragma unroll
    for (int rt = 0; rt < RW; rt++) sc[rt] = F::scales(w[rt], g);
#pragma unroll
    for (int c = 0; c < 8; c++) {
        half8 b[CT];
#pragma unroll
        for (int ct = 0; ct < CT; ct++) b[ct] = *(const half8 *)(xb + boff[ct] + 64 * c);
#pragma unroll
        for (int rt = 0; rt < RW; rt++) {
            const half8 a = F::frag(w[rt], sc[rt], g, c);
#pragma unroll
            for (int ct = 0; ct < CT; ct++)
                acc[rt][ct] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b[ct], acc[rt][ct], 0, 0, 0);
        }
    }
}

// superblocks [sb0, sb1); every thread stages, waves with live = false only
// keep the barriers
template <int FMT, int RW, int CT>
__device__ __forceinline__ void qgx_body(const GemmParams &p, const WRow (&row)[RW], bool live, int sb0, int sb1,
                                         floatx4 (&acc)[RW][CT], uint8_t *lds) {
    typedef QFmt<FMT> F;
    const int lane = threadIdx.x & 63, r16 = lane & 15, g = lane >> 4;
    const int nsb = p.K >> 8;
    constexpr int STAGE = CT * 16 * XG_PITCH;
    const rsrc_t xr = make_rsrc(p.xp, (uint32_t)p.M * (uint32_t)p.K * 2u);
    uint32_t boff[CT];
#pragma unroll
    for (int ct = 0; ct < CT; ct++) boff[ct] = (uint32_t)min(ct * 16 + r16, p.M - 1) * XG_PITCH + 16u * g;
    typename F::D w0[RW], w1[RW];
    XStage<CT> xs;
    auto wsb = [&](int sb) { return live && sb < sb1 ? sb : -1; };
    xg_load<CT>(xs, xr, p.M, p.K, sb0);
#pragma unroll
    for (int rt = 0; rt < RW; rt++) F::load(w0[rt], row[rt], nsb, wsb(sb0), g);
    xg_store<CT>(xs, lds);
    __syncthreads();
    for (int sb = sb0;; sb += 2) {
        // next superblock: activations first (the LDS store below waits on
        // them only), then weights
        xg_load<CT>(xs, xr, p.M, p.K, sb + 1 < sb1 ? sb + 1 : -1);
#pragma unroll
        for (int rt = 0; rt < RW; rt++) F::load(w1[rt], row[rt], nsb, wsb(sb + 1), g);
        if (live) qgx_step<FMT, RW, CT>(w0, lds, boff, g, acc);
        if (sb + 1 >= sb1) break;
        xg_store<CT>(xs, lds + STAGE);
        __syncthreads();
        xg_load<CT>(xs, xr, p.M, p.K, sb + 2 < sb1 ? sb + 2 : -1);
#pragma unroll
        for (int rt = 0; rt < RW; rt++) F::load(w0[rt], row[rt], nsb, wsb(sb + 2), g);
        if (live) qgx_step<FMT, RW, CT>(w1, lds + STAGE, boff, g, acc);
        if (sb + 2 >= sb1) break;
        xg_store<CT>(xs, lds);
        __syncthreads();
    }
}

template <int RW, int CT>
__global__ __launch_bounds__(256) void k_qgx(GemmParams p, int nks) {
    warm_kernargs<sizeof(GemmParams)>();
    extern __shared__ __attribute__((aligned(16))) uint8_t xlds[];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r16 = lane & 15, g = lane >> 4;
    const int rb = (int)blockIdx.x / nks, ks = (int)blockIdx.x % nks;
    const bool swi = p.mode == GM_SWIGLU;
    const int nfeat = swi ? p.seg[0].rows / 16 : 0;
    // this wave's row tiles and their place among the launch's output rows
    GemmSeg S[RW];
    int rloc[RW], grow[RW];
    bool live;
    if (swi) {
        const int f = rb * XG_WAVES + wave;
        live = f < nfeat;
#pragma unroll
        for (int rt = 0; rt < RW; rt++) {
            S[rt] = rt == 0 ? p.seg[0] : p.seg[1];
            rloc[rt] = (live ? f : 0) * 16;
            grow[rt] = rt * nfeat * 16 + rloc[rt];
        }
    } else {
        const int t0 = (rb * XG_WAVES + wave) * RW;
        live = t0 < p.ntiles;
        const GemmSeg s = seg_of_tile(p, live ? t0 : 0);
#pragma unroll
        for (int rt = 0; rt < RW; rt++) {
            S[rt] = s;
            rloc[rt] = ((live ? t0 : s.tile0) - s.tile0 + rt) * 16;
            grow[rt] = (live ? t0 : 0) * 16 + rt * 16;
        }
    }
    WRow row[RW];
#pragma unroll
    for (int rt = 0; rt < RW; rt++) row[rt] = wrow(S[rt], p.K, rloc[rt]);
    const int nsb = p.K >> 8;
    const int sb0 = ks * nsb / nks, sb1 = (ks + 1) * nsb / nks;
    // Input norm (norm_ssq set, M <= 64, norm_parts <= 64): thread t sums the
    // partials j = t % 4, t % 4 + 4, ... of token t / 4, requested now and
    // added after the main loop (norm_inv_rms's order)
    const bool has_norm = p.norm_ssq != nullptr;
    float nrm[16];
#pragma unroll
    for (int i = 0; i < 16; i++) nrm[i] = 0.f;
    if (has_norm) {
        const int m = min((int)threadIdx.x >> 2, p.M - 1), j0 = (int)threadIdx.x & 3;
        const rsrc_t nr = make_rsrc(p.norm_ssq, (uint32_t)(p.M * p.norm_parts * 4));
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int j = j0 + 4 * i;
            nrm[i] = __uint_as_float(bld4(nr, j < p.norm_parts ? (uint32_t)(m * p.norm_parts + j) * 4u : kNoLoad, 0u));
        }
    }
    floatx4 acc[RW][CT];
#pragma unroll
    for (int rt = 0; rt < RW; rt++)
#pragma unroll
        for (int ct = 0; ct < CT; ct++) acc[rt][ct] = floatx4{0.f, 0.f, 0.f, 0.f};
    switch (S[0].fmt) {
    case Q4_K: qgx_body<Q4_K, RW, CT>(p, row, live, sb0, sb1, acc, xlds); break;
    case Q5_K: qgx_body<Q5_K, RW, CT>(p, row, live, sb0, sb1, acc, xlds); break;
    case Q6_K: qgx_body<Q6_K, RW, CT>(p, row, live, sb0, sb1, acc, xlds); break;
    case Q8_0: qgx_body<Q8_0, RW, CT>(p, row, live, sb0, sb1, acc, xlds); break;
    default: break;
    }
    // 1 / rms of every token
    __shared__ float s_inv[64];
    if (has_norm) {
        float t = 0.f;
#pragma unroll
        for (int i = 0; i < 16; i++) t += nrm[i];
        t += __shfl_xor(t, 1);
        t += __shfl_xor(t, 2);
        if ((threadIdx.x & 3) == 0 && (int)(threadIdx.x >> 2) < p.M)
            s_inv[threadIdx.x >> 2] = 1.0f / sqrtf(t / (float)p.K + p.norm_eps);
        __syncthreads();
    }
    const int slot = rb * XG_WAVES + wave;  // argmax partial slot of this wave
    if (!live) {
        // padding waves of the last row block leave a neutral argmax partial
        if (p.mode == GM_LOGITS && g == 0)
            for (int m = r16; m < p.M; m += 16) {
                p.amax_v[(int64_t)m * p.amax_ld + slot] = -INFINITY;
                p.amax_i[(int64_t)m * p.amax_ld + slot] = 0x7fffffff;
            }
        if (nks == 1) return;
    }
    if (nks == 1) {
#pragma unroll
        for (int ct = 0; ct < CT; ct++) {
            floatx4 v[RW];
#pragma unroll
            for (int rt = 0; rt < RW; rt++) v[rt] = acc[rt][ct];
            if (has_norm) {
                const float inv = s_inv[min(ct * 16 + r16, 63)];
#pragma unroll
                for (int rt = 0; rt < RW; rt++) v[rt] *= inv;
            }
            EpiPre<RW> e;
            epi_prefetch<RW>(p, S, rloc, ct * 16 + r16, g, e);
            epilogue<RW>(p, S, rloc, v, e, ct * 16 + r16, g, slot);
        }
        return;
    }
    // K slices: partial sums [ks][M][R] (R = output rows of the launch); the
    // consumer of the output adds them in slice order (an in-kernel reduction
    // by the last workgroup needs agent-scope fences, i.e. L2 write-back and
    // invalidation on every XCD, which measured slower than the split saved)
    if (!live) return;
    const int R = p.ntiles * 16;
#pragma unroll
    for (int ct = 0; ct < CT; ct++) {
        const int m = ct * 16 + r16;
        if (m >= p.M) continue;
#pragma unroll
        for (int rt = 0; rt < RW; rt++)
            *(floatx4 *)(p.part + ((int64_t)ks * p.M + m) * R + grow[rt] + 4 * g) = acc[rt][ct];
    }
}

// --------------------------------------------------------------------------
// Launch policy.  KW (waves splitting K) is a function of the matrix only --
// the smallest power of two that reaches the policy's wave count, capped at 8
// (two waves per SIMD keep the register file) and at the number of
// superblocks -- so row i of an M-row call equals the M=1 call bit for bit.  RT depends on M only through
// the register budget and changes which tiles share a wave, not any sum.
// --------------------------------------------------------------------------
static int swiglu_features(const GemmParams &p) { return p.seg[0].rows / 16; }
static int total_rows(const GemmParams &p) {
    int r = 0;
    for (int i = 0; i < p.nseg; i++) r += p.seg[i].rows;
    return r;
}

// Row tiles per wave and the wave count K is split towards, per matrix:
// outputs of up to 4096 rows (wo, ffn_down at the 8B shapes) stream best as
// 1 tile per wave and >= 2048 waves, wider ones (fused QKV, gate/up, lm_head)
// as 2 tiles per wave and >= 1024 waves (measured on MI355X; a wave's start-up
// latency is paid once per K range, so few long waves beat many short ones
// once the grid covers the chip).
static int policy_rt(const GemmParams &p) {
    if (p.mode == GM_SWIGLU || p.rope.q16) return 2;  // gate/up pairs; RoPE pairs (j, j + hd/32)
    return total_rows(p) <= 4096 ? 1 : 2;
}

int qgemm_kw(const GemmParams &p) {
    const int nsb = p.K / 256;
    const int rt = policy_rt(p);
    const int groups = p.mode == GM_SWIGLU ? swiglu_features(p) : p.ntiles / rt;
    const int target = rt == 1 ? 2048 : 1024;
    int kw = 1;
    while (kw < 8 && groups * kw < target) kw *= 2;
    while (kw > 1 && kw > nsb) kw /= 2;
    return kw;
}

static int token_tiles(int M) { return M <= 16 ? 1 : M <= 32 ? 2 : M <= 64 ? 4 : 8; }

// Row tiles of a wave: the policy's for up to two token tiles, else 1 (gate/up
// pairs always 2); shrunk until every segment splits evenly.
static int qgemm_rt(const GemmParams &p) {
    if (p.mode == GM_SWIGLU) return 2;
    int rt = token_tiles(p.M) <= 2 ? policy_rt(p) : 1;
    for (; rt > 1; rt /= 2) {
        bool ok = p.ntiles % rt == 0;
        for (int i = 0; i < p.nseg; i++) ok = ok && (p.seg[i].rows / 16) % rt == 0;
        if (ok) break;
    }
    return rt;
}

// ---- M > 16: row blocks of 4 waves, K slices towards one workgroup per CU ----
static int xg_rw(const GemmParams &p) {
    if (p.mode == GM_SWIGLU) return 2;
    if (token_tiles(p.M) > 4) return 1;
    for (int i = 0; i < p.nseg; i++)
        if ((p.seg[i].rows / 16) % 2) return 1;
    return 2;
}
static int xg_row_blocks(const GemmParams &p) {
    const int units = p.mode == GM_SWIGLU ? swiglu_features(p) : p.ntiles / xg_rw(p);
    return (units + XG_WAVES - 1) / XG_WAVES;
}
// K slices: only when the caller finalises them (allow_split), towards 192
// workgroups, up to 8 slices and the partial-sum buffer
int qgemm_slices(const GemmParams &p) {
    if (p.M <= 16 || !p.allow_split || (p.mode != GM_STORE && p.mode != GM_RESID)) return 1;
    const int rb = xg_row_blocks(p), nsb = p.K / 256;
    const int64_t R = 16LL * p.ntiles;
    int ks = 1;
    while (ks < 8 && rb * ks < 192 && 2 * ks <= nsb && (int64_t)2 * ks * p.M * R <= p.part_cap) ks *= 2;
    return ks;
}

// argmax partial slots of a GM_LOGITS launch (= amax_ld)
int qgemm_workgroups(const GemmParams &p) {
    if (p.M > 16) return xg_row_blocks(p) * XG_WAVES;
    const int rt = qgemm_rt(p);
    return p.mode == GM_SWIGLU ? swiglu_features(p) / (rt / 2) : p.ntiles / rt;
}

template <typename Kern, typename... Args>
static void launch_timed(Kern kern, dim3 grid, dim3 block, size_t lds, hipStream_t st, const LaunchTiming &tm,
                         Args... args) {
    if (tm.start && tm.stop) hipExtLaunchKernelGGL(kern, grid, block, lds, st, tm.start, tm.stop, 0, args...);
    else hipLaunchKernelGGL(kern, grid, block, lds, st, args...);
}

template <int RW, int CT>
static void launch_qgx(const GemmParams &p, hipStream_t st, const LaunchTiming &tm) {
    const int rb = xg_row_blocks(p), nks = qgemm_slices(p);
    const size_t lds = 2 * CT * 16 * XG_PITCH;
    launch_timed(k_qgx<RW, CT>, dim3(rb * nks), dim3(64 * XG_WAVES), lds, st, tm, p, nks);
}

template <int RT, int KW>
static void launch_qmm(const GemmParams &p, int nwg, hipStream_t st, const LaunchTiming &tm) {
    // up to 8 (4) tokens the activations of a superblock take half (a quarter)
    // of the loads (load_x)
    if (p.M <= 4) launch_timed(k_qmm<RT, KW, 2>, dim3(nwg), dim3(64 * KW), 0, st, tm, p);
    else if (p.M <= 8) launch_timed(k_qmm<RT, KW, 4>, dim3(nwg), dim3(64 * KW), 0, st, tm, p);
    else launch_timed(k_qmm<RT, KW, 8>, dim3(nwg), dim3(64 * KW), 0, st, tm, p);
}

template <int RT>
static bool launch_kw(const GemmParams &p, int kw, int nwg, hipStream_t st, const LaunchTiming &tm) {
    switch (kw) {
    case 1: launch_qmm<RT, 1>(p, nwg, st, tm); return true;
    case 2: launch_qmm<RT, 2>(p, nwg, st, tm); return true;
    case 4: launch_qmm<RT, 4>(p, nwg, st, tm); return true;
    case 8: launch_qmm<RT, 8>(p, nwg, st, tm); return true;
    default: return false;
    }
}

static void qgemm_check(const GemmParams &p) {
    if (p.M < 1 || p.M > 128) throw BackendError("qgemm: M out of range");
    if (p.K % 256) throw BackendError("qgemm: K must be a multiple of 256");
    if (p.mode == GM_SWIGLU && (p.nseg != 2 || p.seg[0].rows != p.seg[1].rows || p.seg[0].fmt != p.seg[1].fmt))
        throw BackendError("qgemm: gate/up segments must match");
    if (p.mode != GM_SWIGLU)
        for (int i = 1; i < p.nseg; i++)
            if (p.seg[i].tile0 != p.seg[i - 1].tile0 + p.seg[i - 1].rows / 16)
                throw BackendError("qgemm: segments must be consecutive");
    // fused RMSNorm and RoPE: both sides in the M <= 16 kernel's epilogues;
    // above 16 rows (up to 64) only the input side, in k_qgx (its K slices
    // are scaled by the kernel that adds them)
    if ((p.next_w || p.rope.q16) && p.M > 16) throw BackendError("qgemm: fused output epilogues need M <= 16");
    if (p.norm_ssq && p.M <= 16 && p.norm_parts * 16 != p.K) throw BackendError("qgemm: norm partials must be one per 16 of K");
    if (p.norm_ssq && p.M > 16 && (p.M > 64 || p.norm_parts < 1 || p.norm_parts > 64))
        throw BackendError("qgemm: input norm above 16 rows needs M <= 64 and at most 64 partials");
    if (p.next_w && (p.mode != GM_RESID || !p.next_u || !p.next_ssq)) throw BackendError("qgemm: next-norm outputs");
    if (p.rope.q16) {
        const RopeOut &R = p.rope;
        if (p.mode != GM_STORE || p.nseg != 3 || (R.hd != 64 && R.hd != 128))
            throw BackendError("qgemm: RoPE epilogue needs the fused Q/K/V launch");
        if (p.seg[0].rows != R.n_heads * R.hd || p.seg[1].rows != R.n_kv * R.hd || p.seg[2].rows != R.n_kv * R.hd)
            throw BackendError("qgemm: RoPE head layout");
        if (p.seg[1].col0 != p.seg[0].rows || p.seg[2].col0 != p.seg[0].rows + p.seg[1].rows || p.seg[0].col0 != 0)
            throw BackendError("qgemm: RoPE column layout");
        if (R.cap % 32 || (int64_t)R.P + p.M > R.cap) throw BackendError("qgemm: RoPE cache capacity");
    }
}

bool qkv_attention_fits(const GemmParams &g, const AttnParams &a, int cus) {
    if (g.M > 16 || !g.rope.q16 || g.mode != GM_STORE || qgemm_rt(g) != 2 || qgemm_kw(g) != 8) return false;
    if (a.M != g.M || (a.hd != 64 && a.hd != 128)) return false;
    // the producer of head j's columns is workgroup range [j hd/32, (j+1) hd/32)
    if (qgemm_workgroups(g) * 32 != (a.n_heads + 2 * a.n_kv) * a.hd) return false;
    const bool merged = a.nsplit == 1 || (a.split_cnt && a.nsplit <= kFusedMaxSplits);
    // every workgroup of the launch on a CU of its own: attention workgroups
    // that wait on CUs the matmul would use made the Qwen2.5-7B-shaped M = 9
    // step slower than the two launches (measured 2700 against 2656 us)
    return merged && qgemm_workgroups(g) + attn_small_workgroups(a) <= cus;
}

void launch_qkv_attention(const GemmParams &g, const AttnParams &a, const QkvAttnSync &sy, int cus, hipStream_t st,
                          const LaunchTiming &tm) {
    qgemm_check(g);
    if (!qkv_attention_fits(g, a, cus)) throw BackendError("qkv_attention: shape does not fit the fused launch");
    if (!sy.flags || !sy.status || sy.epoch == 0) throw BackendError("qkv_attention: synchronisation words missing");
    QkvAttnArgs p;
    p.g = g;
    p.a = attn_small_params(a);
    p.nprod = qgemm_workgroups(g);
    if (p.nprod > sy.nflags) throw BackendError("qkv_attention: too few producer flags");
    p.w.flags = sy.flags;
    p.w.epoch = sy.epoch;
    p.w.status = sy.status;
    if (sy.fault_polls < 0 || sy.epoch >= 0x80000000u) throw BackendError("qkv_attention: bad synchronisation words");
    p.w.want = sy.fault_polls ? sy.epoch | 0x80000000u : sy.epoch;
    p.w.polls = sy.fault_polls ? sy.fault_polls : kWaitPolls;
    const dim3 grid(p.nprod + attn_small_workgroups(p.a)), block(kAttnThreads);
    if (a.hd == 128) {
        if (g.M <= 4) launch_timed(k_qkv_attn<128, 2>, grid, block, 0, st, tm, p);
        else if (g.M <= 8) launch_timed(k_qkv_attn<128, 4>, grid, block, 0, st, tm, p);
        else launch_timed(k_qkv_attn<128, 8>, grid, block, 0, st, tm, p);
    } else {
        if (g.M <= 4) launch_timed(k_qkv_attn<64, 2>, grid, block, 0, st, tm, p);
        else if (g.M <= 8) launch_timed(k_qkv_attn<64, 4>, grid, block, 0, st, tm, p);
        else launch_timed(k_qkv_attn<64, 8>, grid, block, 0, st, tm, p);
    }
}

int launch_qgemm(const GemmParams &p, hipStream_t st, const LaunchTiming &tm) {
    qgemm_check(p);
    const int ct = token_tiles(p.M);
    if (ct > 1) {
        if (qgemm_slices(p) > 1 && !p.part) throw BackendError("qgemm: split-K workspace missing");
        const int rw = xg_rw(p);
        if (rw == 2 && ct == 2) launch_qgx<2, 2>(p, st, tm);
        else if (rw == 2 && ct == 4) launch_qgx<2, 4>(p, st, tm);
        else if (rw == 2 && ct == 8) launch_qgx<2, 8>(p, st, tm);
        else if (rw == 1 && ct == 2) launch_qgx<1, 2>(p, st, tm);
        else if (rw == 1 && ct == 4) launch_qgx<1, 4>(p, st, tm);
        else launch_qgx<1, 8>(p, st, tm);
        return qgemm_workgroups(p);
    }
    const int kw = qgemm_kw(p), rt = qgemm_rt(p);
    const int nwg = qgemm_workgroups(p);
    bool ok = false;
    if (rt == 2) ok = launch_kw<2>(p, kw, nwg, st, tm);
    else if (rt == 1 && p.mode != GM_SWIGLU) ok = launch_kw<1>(p, kw, nwg, st, tm);
    if (!ok) throw BackendError("qgemm: unsupported launch shape");
    return nwg;
}

}  // namespace sd
