// K2: RoPE + KV append + tree-masked GQA attention over the fp16 KV cache.
//
// Replaces LayerWeights::{rope_at, rope_at_positions, run_attn}
// (crates/speculate/src/model/quantized_llama_local.rs:94-136; Qwen2 half
// rotation at quantized_qwen2_local.rs:98-109) and the additive masks of
// causal_bias (:332-350) / DraftTree::full_attention_bias (tree.rs:220-264).
//
// KV layout per layer: n_kv streams of K and of V, each cap positions x hd
// fp16 in the blocked order of kv_k_off / kv_v_off (sd_common.hpp).  The M new
// rows are written in place at [P, P+M) (no cat, no repeat_kv copies).
// Visibility: key j < P is visible to every query; key P+t is visible to
// query token i iff bit t of mask[i] is set (ancestor-or-self for trees,
// t <= i for a causal chain).
//
// Attention is split flash-decoding with the KV streamed straight from HBM
// into MFMA operand registers (no LDS staging): the blocked cache layout makes
// every operand a 16-byte load per lane, 1 KiB contiguous per wave.  Scores
// are computed transposed, S^T = K Q^T (16 keys x 16 queries per MFMA tile),
// so a lane's accumulator already holds the P^T operand of O^T = V^T P^T.
//
// Grid (kv head, key split, query tile).  A workgroup's 4 waves take 4
// consecutive key ranges of keys_per_wave keys and one query tile (16 of the
// n_rep query heads of the KV head times the M tokens); their partial softmax
// states are merged in LDS in a fixed order, and the splits by the last
// workgroup of the tile to finish (up to 16 tokens; a counter per tile, device-
// scope partials) or by a combine kernel (more tokens), with the same
// arithmetic; nothing to merge when one split covers all keys.  Up to 16 tokens,
// keys_per_wave and the split boundaries depend on P only, so a query's
// result does not depend on how many other queries share the call.
#include <mutex>
#include <vector>

#include "sd_buffer.hpp"
#include "sd_common.hpp"
#include "sd_kernels_attn.hpp"

namespace sd {

#pragma clang fp contract(off)

// ---- RoPE + KV append ------------------------------------------------------
// Four consecutive columns (col % 4 == 0) of the projection output: the
// matmul's values (nks <= 1) or its K-slice partials, requested through
// buffer resources without branches so that every load of a thread -- both
// column groups and the token's norm partials -- is in flight before the
// first wait.
struct QkvCols {
    float4 a[8];
};
constexpr uint32_t kNoCol = 0x80000000u;  // offset past any resource: reads zeros, no memory access
__device__ __forceinline__ void qkv_load4(const RopeKvParams &p, int m, int col, QkvCols &c) {
    const bool split = p.nks > 1;
    const int64_t stride = (int64_t)p.M * p.ld_qkv;
    const rsrc_t r = make_rsrc(split ? (const void *)p.part : (const void *)p.qkv,
                               (uint32_t)((split ? p.nks : 1) * stride * 4));
    const uint32_t at = (uint32_t)(((int64_t)m * p.ld_qkv + col) * 4);
    const int n = split ? p.nks : 1;
#pragma unroll
    for (int k = 0; k < 8; k++)
        c.a[k] = __builtin_bit_cast(float4, bld16(r, k < n ? at + (uint32_t)(k * stride * 4) : kNoCol, 0u));
}
// slices added in slice order, scaled by the input norm (after K slices),
// plus the bias
__device__ __forceinline__ float4 qkv_finish4(const RopeKvParams &p, int col, const QkvCols &c, float inv) {
    if (p.nks <= 1) return c.a[0];
    float4 v = c.a[0];
#pragma unroll
    for (int k = 1; k < 8; k++)
        if (k < p.nks) {
            v.x += c.a[k].x;
            v.y += c.a[k].y;
            v.z += c.a[k].z;
            v.w += c.a[k].w;
        }
    if (p.norm_ssq) {
        v.x *= inv;
        v.y *= inv;
        v.z *= inv;
        v.w *= inv;
    }
    if (!p.bq) return v;
    const int qd = p.n_heads * p.hd, kvd = p.n_kv * p.hd;
    const float *b = col < qd ? p.bq + col : col < qd + kvd ? p.bk + (col - qd) : p.bv + (col - qd - kvd);
    const float4 bb = *(const float4 *)b;
    v.x += bb.x;
    v.y += bb.y;
    v.z += bb.z;
    v.w += bb.w;
    return v;
}
__device__ __forceinline__ void st4h_f(uint16_t *dst, float a, float b, float c, float d) {
    *(uintx2 *)dst = uintx2{(uint32_t)f2h(a) | ((uint32_t)f2h(b) << 16), (uint32_t)f2h(c) | ((uint32_t)f2h(d) << 16)};
}

// grid (M, ceil((n_heads + n_kv) * hd / 4 / 64)), block 64: thread (head hh,
// unit j) owns columns d = 4j .. 4j + 3 of the head (with half rotation the
// q / k units of the lower half also own d + hd/2 .., the upper half's idle);
// a KV head's thread does both its k and its v columns.
__global__ __launch_bounds__(64) void k_rope_kv(RopeKvParams p) {
    warm_kernargs<sizeof(RopeKvParams)>();
    const int m = blockIdx.x, hd = p.hd, half = hd / 2, upr = hd / 4;
    const int t = (int)blockIdx.y * 64 + (int)threadIdx.x;
    if (t >= (p.n_heads + p.n_kv) * upr) return;
    const int hh = t / upr, d = 4 * (t % upr);
    const bool q_head = hh < p.n_heads;
    const int kvh = hh - p.n_heads;
    const int col = q_head ? hh * hd : p.n_heads * hd + kvh * hd;  // q or k columns of the head
    const int vcol = (p.n_heads + p.n_kv) * hd + kvh * hd;          // v columns of a KV head
    const bool pair_hi = !p.interleaved && d < half;                // also rotates d + hd/2
    // every load first: the token's norm partials (up to 16), the columns,
    // then the position and its rotation entries
    const bool has_norm = p.norm_ssq && p.nks > 1 && p.norm_parts <= 16;
    // (the resource reaches 4 partials past the last token's: a 16-byte load
    // never straddles its end; ssq holds hidden >= M * parts + 4 floats)
    const rsrc_t nr = make_rsrc(p.norm_ssq, has_norm ? (uint32_t)((p.M * p.norm_parts + 4) * 4) : 0u);
    float sv[16];
#pragma unroll
    for (int j = 0; j < 16; j += 4) {
        // four partials per load; the resource ends at the token's last one
        const float4 q4 = __builtin_bit_cast(
            float4, bld16(nr, j < p.norm_parts ? (uint32_t)(m * p.norm_parts + j) * 4u : kNoCol, 0u));
        sv[j] = q4.x;
        sv[j + 1] = j + 1 < p.norm_parts ? q4.y : 0.f;
        sv[j + 2] = j + 2 < p.norm_parts ? q4.z : 0.f;
        sv[j + 3] = j + 3 < p.norm_parts ? q4.w : 0.f;
    }
    QkvCols cx, cy, cv;
    qkv_load4(p, m, col + d, cx);
    if (pair_hi) qkv_load4(p, m, col + d + half, cy);
    if (!q_head) qkv_load4(p, m, vcol + d, cv);
    const int pos = p.pos[m];
    const float *ct = p.cos_t + (int64_t)pos * half, *st = p.sin_t + (int64_t)pos * half;
    float inv = 1.f;
    if (has_norm) {
        // norm_inv_rms's order
        float q[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 16; j++) q[j & 3] += sv[j];
        inv = 1.0f / sqrtf(((q[0] + q[1]) + (q[2] + q[3])) / (float)p.norm_K + p.norm_eps);
    } else if (p.norm_ssq && p.nks > 1) {
        inv = norm_inv_rms(p.norm_ssq + (int64_t)m * p.norm_parts, p.norm_parts, p.norm_K, p.norm_eps);
    }
    const int64_t tk = (int64_t)p.P + m;
    if (!q_head) {
        // v: copied (fp16) into the cache
        const float4 v = qkv_finish4(p, vcol + d, cv, inv);
        uint16_t *vs = p.vc + (int64_t)kvh * p.cap * hd;
        vs[kv_v_off(tk, d, hd)] = f2h(v.x);
        vs[kv_v_off(tk, d + 1, hd)] = f2h(v.y);
        vs[kv_v_off(tk, d + 2, hd)] = f2h(v.z);
        vs[kv_v_off(tk, d + 3, hd)] = f2h(v.w);
    }
    uint16_t *lo, *hi;
    if (q_head) {
        lo = p.q16 + ((int64_t)hh * p.M + m) * hd + d;
        hi = lo + half;
    } else {
        uint16_t *ks = p.kc + (int64_t)kvh * p.cap * hd;
        lo = ks + kv_k_off(tk, d, hd);
        hi = ks + kv_k_off(tk, d + half, hd);
    }
    const float4 x = qkv_finish4(p, col + d, cx, inv);
    if (p.interleaved) {
        // pairs (d, d+1), (d+2, d+3): rotation indices d/2, d/2 + 1
        const float c0 = ct[d / 2], s0 = st[d / 2], c1 = ct[d / 2 + 1], s1 = st[d / 2 + 1];
        st4h_f(lo, x.x * c0 - x.y * s0, x.x * s0 + x.y * c0, x.z * c1 - x.w * s1, x.z * s1 + x.w * c1);
        return;
    }
    if (!pair_hi) return;  // the unit of d - hd/2 rotates these columns
    const float4 y = qkv_finish4(p, col + d + half, cy, inv);
    const float c[4] = {ct[d], ct[d + 1], ct[d + 2], ct[d + 3]}, sn[4] = {st[d], st[d + 1], st[d + 2], st[d + 3]};
    const float xa[4] = {x.x, x.y, x.z, x.w}, ya[4] = {y.x, y.y, y.z, y.w};
    float r0[4], r1[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        r0[i] = xa[i] * c[i] - ya[i] * sn[i];
        r1[i] = xa[i] * sn[i] + ya[i] * c[i];
    }
    st4h_f(lo, r0[0], r0[1], r0[2], r0[3]);
    st4h_f(hi, r1[0], r1[1], r1[2], r1[3]);
}

#pragma clang fp contract(fast)

// ---- flash-decode over one key split -------------------------------------------
template <int HD> struct KvStep {
    uintx4 k[2][HD / 32];  // S^T A operands: two 16-key tiles x HD/32 d-chunks
    uintx4 v[HD / 16];     // O^T A operands: HD/16 d-tiles x 32 key slots
};

// One KV head's K and V streams as buffer resources and the lane's fixed byte
// offset inside a 32-key block, (r16 * 32 + g * 8) * 2 in both layouts; the
// block's offset kk * HD * 2 is wave-uniform and goes in a scalar register.
struct KvSrc {
    rsrc_t k, v;
    uint32_t lane;
};
// A load that must not happen gets an offset past the resource (a stream is
// < 2 GiB), which reads zeros without touching memory; loads are then issued
// unconditionally and the compiler's wait counts stay exact across the loop.
constexpr uint32_t kNoKv = 0x80000000u;
__device__ __forceinline__ uint32_t kv_so(int kk, int HD) { return uni(kk < 0 ? kNoKv : (uint32_t)kk * HD * 2u); }

// 32 keys [kk, kk+32) of one stream (kk < 0: none): 16-byte pieces, 1 KiB per wave each
template <int HD>
__device__ __forceinline__ void kv_load_k(KvStep<HD> &b, const KvSrc &s, int kk) {
    const uint32_t so = kv_so(kk, HD);
#pragma unroll
    for (int kt = 0; kt < 2; kt++)
#pragma unroll
        for (int dc = 0; dc < HD / 32; dc++) b.k[kt][dc] = bld16(s.k, s.lane + kt * 32 * HD + dc * 1024, so);
}
template <int HD>
__device__ __forceinline__ void kv_load_v(KvStep<HD> &b, const KvSrc &s, int kk) {
    const uint32_t so = kv_so(kk, HD);
#pragma unroll
    for (int dt = 0; dt < HD / 16; dt++) b.v[dt] = bld16(s.v, s.lane + dt * 1024, so);
}

template <int HD, int QT> struct AttnState {
    half8 qf[QT][HD / 32];
    floatx4 o[QT][HD / 16];
    float m[QT], l[QT];
    uint64_t mk0[QT], mk1[QT];
};

// key of P^T / V^T slot j (0..7) of lane group g within a 32-key step
__device__ __forceinline__ int slot_key(int g, int j) { return j < 4 ? 4 * g + j : 16 + 4 * g + (j - 4); }

// The 4 lanes of one query (lane groups g = 0..3 of a 16x16 MFMA layout)
// combined with lane ^ 16 and lane ^ 32: two VALU swaps instead of LDS
// permutes.  Every lane ends with the same value (the operations commute).
__device__ __forceinline__ float xmax4(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float xsum4(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// A query tile's raw operands for lane (r16 = query row, g): 8 dims of each
// 32-dim chunk and the row's tree-mask words.  Lanes past the last query read
// the last query's row, so every load is in bounds and unconditional and the
// compiler issues them back to back before the first wait; query_init zeroes
// those lanes' fragments.
template <int HD> struct QueryRaw {
    uintx4 q[HD / 32];
    uint64_t mk0, mk1;
    bool live;
};
template <int HD>
__device__ __forceinline__ void query_fetch(QueryRaw<HD> &r, const AttnParams &p, int h, int q, int g) {
    const int nq = p.M * p.n_rep;
    r.live = q < nq;
    const int qc = r.live ? q : nq - 1;
    const int m = qc / p.n_rep, rep = qc % p.n_rep;
    const uint16_t *qr = p.q16 + ((int64_t)(h * p.n_rep + rep) * p.M + m) * HD;
#pragma unroll
    for (int dc = 0; dc < HD / 32; dc++) r.q[dc] = *(const uintx4 *)(qr + dc * 32 + g * 8);
    r.mk0 = p.mask[(int64_t)m * p.mask_words];
    r.mk1 = p.mask_words > 1 ? p.mask[(int64_t)m * p.mask_words + 1] : 0ull;
}
// the query scaled by scale * log2(e) (scores in base-2 softmax units) and an
// empty softmax state
template <int HD, int QT>
__device__ __forceinline__ void query_init(AttnState<HD, QT> &S, int t, const QueryRaw<HD> &r, float sl2) {
#pragma unroll
    for (int dc = 0; dc < HD / 32; dc++) {
        half8 v = r.live ? __builtin_bit_cast(half8, r.q[dc]) : half8{};
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = __builtin_bit_cast(_Float16, f2h((float)v[i] * sl2));
        S.qf[t][dc] = v;
    }
    S.mk0[t] = r.mk0;
    S.mk1[t] = r.mk1;
#pragma unroll
    for (int dt = 0; dt < HD / 16; dt++) S.o[t][dt] = floatx4{0.f, 0.f, 0.f, 0.f};
    S.m[t] = -INFINITY;
    S.l[t] = 0.f;
}

// Softmax of one 32-key step for query tile t: st holds the lane's 8 scores
// (keys kk + 16 kt + 4g + i) in base-2 units; returns the P^T fragment.
//
// The running max m of a query (the same in its 4 lanes) moves only when a
// score exceeds it by more than 8: probabilities exp2(s - m) then stay below
// 256, which fp16 and f32 hold with full relative precision.  Each lane keeps
// its own partial sum l of the probabilities it produced; the 4 partials of a
// query are added once, at the end.  So the common step has no cross-lane
// traffic at all: the max is only gathered (and the accumulators rescaled by
// alpha) when some lane of the wave sees a score above its m + 8.
// Keys at or past lim (<= T) belong to another range and are masked.
template <int HD, int QT>
__device__ __forceinline__ half8 step_softmax(AttnState<HD, QT> &S, int t, floatx4 (&st)[2], int kk, int P, int T,
                                              int lim, int g, float &alpha, bool &moved) {
    const bool full = kk + 32 <= P && kk + 32 <= lim;  // every key of the step is visible to every query
    float lmax = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 2; kt++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float v = st[kt][i];
            if (!full) {
                const int key = kk + kt * 16 + 4 * g + i;
                bool vis = key < P && key < lim;
                if (!vis && key < lim) {
                    const int tt = key - P;
                    vis = (((tt < 64 ? S.mk0[t] : S.mk1[t]) >> (tt & 63)) & 1ull) != 0;
                }
                v = vis ? v : -INFINITY;
            }
            st[kt][i] = v;
            lmax = fmaxf(lmax, v);
        }
    alpha = 1.f;
    // -inf + 8 == -inf: the first finite score always moves the max
    if (__builtin_amdgcn_ballot_w64(lmax > S.m[t] + 8.f) != 0) {
        const float cm = xmax4(lmax);
        if (cm > S.m[t] + 8.f) {  // the same decision in the query's 4 lanes
            alpha = __builtin_amdgcn_exp2f(S.m[t] - cm);
            S.m[t] = cm;
            moved = true;
        }
    }
    const float muse = S.m[t] == -INFINITY ? 0.f : S.m[t];
    float ps = 0.f;
    uint32_t pk[4];
#pragma unroll
    for (int kt = 0; kt < 2; kt++) {
        float e[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            e[i] = __builtin_amdgcn_exp2f(st[kt][i] - muse);
            ps += e[i];
        }
        pk[2 * kt] = (uint32_t)f2h(e[0]) | ((uint32_t)f2h(e[1]) << 16);
        pk[2 * kt + 1] = (uint32_t)f2h(e[2]) | ((uint32_t)f2h(e[3]) << 16);
    }
    S.l[t] = S.l[t] * alpha + ps;
    const uintx4 bu = {pk[0], pk[1], pk[2], pk[3]};
    return __builtin_bit_cast(half8, bu);
}

// keys >= T hold stale cache rows: their P^T entries are 0, and their V entries
// are zeroed so that nothing but finite values meets the MFMA
template <int NDT>
__device__ __forceinline__ void zero_stale_v(uintx4 (&v)[NDT], int kk, int T, int g) {
    if (kk + 32 <= T) return;
    uint32_t keep[4];
#pragma unroll
    for (int w = 0; w < 4; w++)
        keep[w] = (kk + slot_key(g, 2 * w) < T ? 0x0000ffffu : 0u) | (kk + slot_key(g, 2 * w + 1) < T ? 0xffff0000u : 0u);
#pragma unroll
    for (int dt = 0; dt < NDT; dt++) {
        v[dt].x &= keep[0];
        v[dt].y &= keep[1];
        v[dt].z &= keep[2];
        v[dt].w &= keep[3];
    }
}

// O^T += V^T P^T for the live tiles, after the rescale the step asked for
template <int HD, int QT>
__device__ __forceinline__ void step_pv(AttnState<HD, QT> &S, const uintx4 (&v)[HD / 16], const half8 (&bp)[QT],
                                        const float (&alpha)[QT], bool moved, const bool (&tl)[QT]) {
    constexpr int NDT = HD / 16;
    if (__builtin_amdgcn_ballot_w64(moved) != 0) {
#pragma unroll
        for (int t = 0; t < QT; t++)
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) S.o[t][dt] *= alpha[t];
    }
#pragma unroll
    for (int t = 0; t < QT; t++) {
        if (!tl[t]) continue;
#pragma unroll
        for (int dt = 0; dt < NDT; dt++)
            S.o[t][dt] =
                __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, v[dt]), bp[t], S.o[t][dt], 0, 0, 0);
    }
}

// S^T = K Q^T for the live tiles
template <int HD, int QT>
__device__ __forceinline__ void step_scores(const AttnState<HD, QT> &S, const uintx4 (&k)[2][HD / 32], int t,
                                            floatx4 (&st)[2]) {
#pragma unroll
    for (int kt = 0; kt < 2; kt++) {
        st[kt] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int dc = 0; dc < HD / 32; dc++)
            st[kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, k[kt][dc]), S.qf[t][dc], st[kt],
                                                            0, 0, 0);
    }
}

// One 32-key step from registers for all query tiles: scores and softmax,
// then the next step's V loads are issued (the current K is dead by then, so
// the two register buffers never hold four operand sets at once), then PV.
template <int HD, int QT>
__device__ __forceinline__ void attn_step(AttnState<HD, QT> &S, KvStep<HD> &b, KvStep<HD> &nb, const KvSrc &src,
                                          int kk, int k1, int P, int T, int g) {
    half8 bp[QT];
    float alpha[QT];
    bool tl[QT];
    bool moved = false;
#pragma unroll
    for (int t = 0; t < QT; t++) {
        tl[t] = true;
        floatx4 st[2];
        step_scores<HD, QT>(S, b.k, t, st);
        bp[t] = step_softmax<HD, QT>(S, t, st, kk, P, T, T, g, alpha[t], moved);
    }
    kv_load_v<HD>(nb, src, kk + 32 < k1 ? kk + 32 : -1);
    zero_stale_v<HD / 16>(b.v, kk, T, g);
    step_pv<HD, QT>(S, b.v, bp, alpha, moved, tl);
}

// Result of one query (lane (r16, g) holds d = dt*16 + 4g + i): with one
// split the normalised row goes straight into the wo input (fp16, fragment
// order); otherwise o / l as fp16 and (m, l) for the merge of the splits,
// which weighs split s by l_s * exp2(m_s - max m).  DEV: the partials are
// stored at device scope, for a merge inside the same launch.
template <int HD, bool DEV = false>
__device__ __forceinline__ void attn_emit(const AttnParams &p, int s, int head, int m, int g,
                                          const floatx4 (&o)[HD / 16], float mq, float l) {
    const float inv = 1.0f / l;
    if (p.nsplit == 1) {
#pragma unroll
        for (int dt = 0; dt < HD / 16; dt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int64_t k = (int64_t)head * HD + dt * 16 + 4 * g + i;
                p.out16[(int64_t)m * p.out_ld + frag_index(k)] = f2h(o[dt][i] * inv);
            }
        return;
    }
    const int64_t pi = ((int64_t)s * p.n_heads + head) * p.M + m;
    uint16_t *po = (uint16_t *)p.part_o + pi * HD;
#pragma unroll
    for (int dt = 0; dt < HD / 16; dt++) {
        const float w = l > 0.f ? inv : 0.f;  // a query that saw no key of this split has l = 0
        const uintx2 v{(uint32_t)f2h(o[dt][0] * w) | ((uint32_t)f2h(o[dt][1] * w) << 16),
                       (uint32_t)f2h(o[dt][2] * w) | ((uint32_t)f2h(o[dt][3] * w) << 16)};
        if constexpr (DEV) st_dev64(po + dt * 16 + 4 * g, (uint64_t)v.x | ((uint64_t)v.y << 32));
        else *(uintx2 *)(po + dt * 16 + 4 * g) = v;
    }
    if (g == 0) {
        if constexpr (DEV) {
            st_dev64(p.part_ml + 2 * pi, (uint64_t)__float_as_uint(mq) | ((uint64_t)__float_as_uint(l) << 32));
        } else {
            p.part_ml[2 * pi] = mq;
            p.part_ml[2 * pi + 1] = l;
        }
    }
}

// Merge of the splits by the last workgroup of a (KV head h, query tile qg)
// to finish: thread (r = tid / 16, c = tid % 16) owns query qg * 16 + r and
// dims [c HD/16, +HD/16).  The arithmetic, and its order, is k_attn_combine's:
// out = sum_s w_s o_s / sum_s w_s in split order, w_s = l_s exp2(m_s - max m).
constexpr int kFusedMaxSplits = 64;
// The merge when every split's (m, l) and pieces fit in registers at once
// (ns <= NSM): one memory round trip; the same arithmetic and order as the
// general path of attn_merge_tile.
template <int HD, int NSM>
__device__ __forceinline__ void attn_merge_regs(const AttnParams &p, int head, int m, int c, int ns, int64_t stride,
                                                int64_t pi0) {
    constexpr int DPT = HD / 16;
    const uint16_t *po = (const uint16_t *)p.part_o + pi0 * HD + c * DPT;
    uint64_t mlv[NSM], ov[NSM][DPT / 4];
#pragma unroll
    for (int j = 0; j < NSM; j++) {
        mlv[j] = j < ns ? ld_dev64(p.part_ml + 2 * (pi0 + j * stride)) : 0ull;
#pragma unroll
        for (int k = 0; k < DPT / 4; k++) ov[j][k] = j < ns ? ld_dev64(po + j * stride * HD + 4 * k) : 0ull;
    }
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < NSM; j++)
        if (j < ns) mx = fmaxf(mx, __uint_as_float((uint32_t)mlv[j]));
    float W = 0.f, acc[DPT];
#pragma unroll
    for (int i = 0; i < DPT; i++) acc[i] = 0.f;
#pragma unroll
    for (int j = 0; j < NSM; j++) {
        if (j < ns) {
            const float ms = __uint_as_float((uint32_t)mlv[j]);
            const float w = ms == -INFINITY ? 0.f : __uint_as_float((uint32_t)(mlv[j] >> 32)) * exp2f(ms - mx);
            W += w;
#pragma unroll
            for (int i = 0; i < DPT; i++) acc[i] += h2f((uint16_t)(ov[j][i >> 2] >> (16 * (i & 3)))) * w;
        }
    }
    // dims 4k .. 4k + 3 of this thread sit in fragment slots f, f + 2, f + 1, f + 3
#pragma unroll
    for (int k = 0; k < DPT / 4; k++) {
        const int64_t e = (int64_t)head * HD + c * DPT + 4 * k;
        *(uintx2 *)(p.out16 + (int64_t)m * p.out_ld + frag_index(e)) =
            uintx2{(uint32_t)f2h(acc[4 * k] / W) | ((uint32_t)f2h(acc[4 * k + 2] / W) << 16),
                   (uint32_t)f2h(acc[4 * k + 1] / W) | ((uint32_t)f2h(acc[4 * k + 3] / W) << 16)};
    }
}

template <int HD> __device__ __forceinline__ void attn_merge_tile(const AttnParams &p, int h, int qg) {
    constexpr int DPT = HD / 16;  // dims per thread, 4 or 8: one or two 8-byte loads per split
    __shared__ float cml[16][kFusedMaxSplits][2];
    const int r = threadIdx.x >> 4, c = threadIdx.x & 15;
    const int nq = p.M * p.n_rep, ns = p.nsplit;
    const int q = qg * 16 + r;
    const bool live = q < nq;
    const int head = h * p.n_rep + (live ? q % p.n_rep : 0), m = live ? q / p.n_rep : 0;
    const int64_t stride = (int64_t)p.n_heads * p.M;  // partial rows per split
    const int64_t pi0 = (int64_t)head * p.M + m;
    if (ns <= 16) {
        if (!live) return;
        if (ns <= 8) attn_merge_regs<HD, 8>(p, head, m, c, ns, stride, pi0);
        else attn_merge_regs<HD, 16>(p, head, m, c, ns, stride, pi0);
        return;
    }
    for (int s = c; s < ns; s += 16) {
        const uint64_t v = live ? ld_dev64(p.part_ml + 2 * (pi0 + s * stride)) : 0ull;
        cml[r][s][0] = __uint_as_float((uint32_t)v);
        cml[r][s][1] = __uint_as_float((uint32_t)(v >> 32));
    }
    __syncthreads();
    if (!live) return;
    float mx = -INFINITY;
    for (int s = 0; s < ns; s++) mx = fmaxf(mx, cml[r][s][0]);
    const uint16_t *po = (const uint16_t *)p.part_o + pi0 * HD + c * DPT;
    float W = 0.f, acc[DPT];
#pragma unroll
    for (int i = 0; i < DPT; i++) acc[i] = 0.f;
    for (int s0 = 0; s0 < ns; s0 += 8) {
        // 8 splits' pieces requested at once
        uint64_t ov[8][DPT / 4];
#pragma unroll
        for (int j = 0; j < 8; j++)
#pragma unroll
            for (int k = 0; k < DPT / 4; k++) ov[j][k] = s0 + j < ns ? ld_dev64(po + (s0 + j) * stride * HD + 4 * k) : 0ull;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            if (s0 + j < ns) {
                const float ms = cml[r][s0 + j][0];
                const float w = ms == -INFINITY ? 0.f : cml[r][s0 + j][1] * exp2f(ms - mx);
                W += w;
#pragma unroll
                for (int i = 0; i < DPT; i++) acc[i] += h2f((uint16_t)(ov[j][i >> 2] >> (16 * (i & 3)))) * w;
            }
        }
    }
#pragma unroll
    for (int i = 0; i < DPT; i++) {
        const int64_t k = (int64_t)head * HD + c * DPT + i;
        p.out16[(int64_t)m * p.out_ld + frag_index(k)] = f2h(acc[i] / W);
    }
}

template <int HD, int QT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void k_attn(AttnParams p) {
    warm_kernargs<sizeof(AttnParams)>();
    constexpr int NDT = HD / 16;
    const int h = blockIdx.x, s = blockIdx.y, qg = blockIdx.z;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r16 = lane & 15, g = lane >> 4;
    const int nq = p.M * p.n_rep;
    const int T = p.P + p.M;
    const int k0 = (s * 4 + wave) * p.keys_per_wave;
    const int k1 = min(k0 + p.keys_per_wave, T);
    const uint32_t stream_bytes = (uint32_t)p.cap * HD * 2u;
    KvSrc src;
    src.k = make_rsrc(p.kc + (int64_t)h * p.cap * HD, stream_bytes);
    src.v = make_rsrc(p.vc + (int64_t)h * p.cap * HD, stream_bytes);
    src.lane = (uint32_t)(r16 * 32 + g * 8) * 2u;

    // the queries first (just written by the Q/K/V launch), then the first
    // 32 keys; two register buffers: the next 32 keys load while the current
    // ones compute (K at the start of a step, V once the step's scores are done)
    QueryRaw<HD> qr[QT];
#pragma unroll
    for (int t = 0; t < QT; t++) query_fetch<HD>(qr[t], p, h, (qg * QT + t) * 16 + r16, g);
    KvStep<HD> b0, b1;
    int kk = k0;
    kv_load_k<HD>(b0, src, kk < k1 ? kk : -1);
    kv_load_v<HD>(b0, src, kk < k1 ? kk : -1);

    AttnState<HD, QT> S;
    const float sl2 = p.scale * 1.4426950408889634f;  // scale * log2(e): softmax in base 2
#pragma unroll
    for (int t = 0; t < QT; t++) query_init<HD, QT>(S, t, qr[t], sl2);

    while (kk < k1) {
        kv_load_k<HD>(b1, src, kk + 32 < k1 ? kk + 32 : -1);
        attn_step<HD, QT>(S, b0, b1, src, kk, k1, p.P, T, g);
        kk += 32;
        if (kk >= k1) break;
        kv_load_k<HD>(b0, src, kk + 32 < k1 ? kk + 32 : -1);
        attn_step<HD, QT>(S, b1, b0, src, kk, k1, p.P, T, g);
        kk += 32;
    }
#pragma unroll
    for (int t = 0; t < QT; t++) S.l[t] = xsum4(S.l[t]);  // the query's 4 partial sums

    // ---- merge the 4 waves' states: rescale to the common max, then
    // (o0 + o2) + (o1 + o3) through LDS ----
    __shared__ float sml[4][QT][16][2];
    __shared__ floatx4 sob[2][QT][NDT][64];
    if (g == 0) {
#pragma unroll
        for (int t = 0; t < QT; t++) {
            sml[wave][t][r16][0] = S.m[t];
            sml[wave][t][r16][1] = S.l[t];
        }
    }
    __syncthreads();
    float Lt[QT], Mt[QT];
#pragma unroll
    for (int t = 0; t < QT; t++) {
        float mx = -INFINITY;
#pragma unroll
        for (int w = 0; w < 4; w++) mx = fmaxf(mx, sml[w][t][r16][0]);
        float L = 0.f, fme = 0.f;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const float mw = sml[w][t][r16][0];
            const float f = mw == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw - mx);
            L += sml[w][t][r16][1] * f;
            if (w == wave) fme = f;
        }
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) S.o[t][dt] *= fme;
        Lt[t] = L;
        Mt[t] = mx;
    }
    if (wave >= 2) {
#pragma unroll
        for (int t = 0; t < QT; t++)
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) sob[wave - 2][t][dt][lane] = S.o[t][dt];
    }
    __syncthreads();
    if (wave < 2) {
#pragma unroll
        for (int t = 0; t < QT; t++)
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) S.o[t][dt] += sob[wave][t][dt][lane];
    }
    __syncthreads();
    if (wave == 1) {
#pragma unroll
        for (int t = 0; t < QT; t++)
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) sob[0][t][dt][lane] = S.o[t][dt];
    }
    __syncthreads();
    const bool fused = p.fused_combine != 0;
    if (wave == 0) {
#pragma unroll
        for (int t = 0; t < QT; t++) {
            const int q = (qg * QT + t) * 16 + r16;
            if (q >= nq) continue;
            floatx4 y[NDT];
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) y[dt] = S.o[t][dt] + sob[0][t][dt][lane];
            if (fused) attn_emit<HD, true>(p, s, h * p.n_rep + q % p.n_rep, q / p.n_rep, g, y, Mt[t], Lt[t]);
            else attn_emit<HD>(p, s, h * p.n_rep + q % p.n_rep, q / p.n_rep, g, y, Mt[t], Lt[t]);
        }
    }
    if (!fused) return;

    // ---- the last of the tile's nsplit workgroups to arrive merges the splits ----
    // Wave 0 wrote the partials (device scope) and waits for those stores to
    // complete before it counts the arrival; the last arrival resets the count
    // for the next launch and reads every split's partials at device scope.
    __shared__ int s_last;
    if (wave == 0) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        if (lane == 0) {
            int *cnt = p.split_cnt + (int64_t)h * gridDim.z + qg;
            const int last = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == p.nsplit - 1;
            if (last) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            s_last = last;
        }
    }
    __syncthreads();
    if (!s_last) return;
    static_assert(QT == 1, "the merge covers one 16-query tile per workgroup");
    attn_merge_tile<HD>(p, h, qg);
}

// ---- many queries (tree verify): query tiles across waves, keys shared in LDS ----
// Grid (kv head, key split, query block).  The kTWaves waves of a workgroup
// own kTQW query tiles each, the kTWaves * kTQW * 16 queries of one query block
// of a KV head (all of them up to 256 query rows), and walk the split's keys
// together: each 32-key block of K and V (contiguous in the blocked cache
// layout) is copied once into LDS by the workgroup's threads and read there by
// all its waves, so the cache leaves L2 once per query block.  Copies run
// kTStages blocks ahead through registers (as many LDS stages, one barrier per
// block).  Splits are a few blocks long, so the grid covers the chip; the
// combine kernel merges them.  Sixteen waves of one tile each (four per SIMD)
// hide the softmax's and the MFMAs' latencies better than eight of two.
constexpr int kTWaves = 16;
constexpr int kTThreads = 64 * kTWaves;
constexpr int kTQW = 1;
constexpr int kTStages = 3;
constexpr int kTMaxSplits = 32;

// a thread's 16-byte pieces of one 32-key block: pieces i * kTThreads + tid,
// the block's K (4 * HD pieces) first, then its V; which stream a piece comes
// from is the same for a whole wave (4 * HD is a multiple of 64)
template <int HD> constexpr int tile_pieces() { return (8 * HD + kTThreads - 1) / kTThreads; }
template <int HD> struct TileCopy {
    uintx4 r[tile_pieces<HD>()];
};
template <int HD>
__device__ __forceinline__ void tile_fetch(TileCopy<HD> &c, const KvSrc &src, int kk, int tid) {  // kk < 0: none
    const uint32_t so = kv_so(kk, HD);
    const int wave_piece = __builtin_amdgcn_readfirstlane(tid & ~63);
#pragma unroll
    for (int i = 0; i < tile_pieces<HD>(); i++) {
        const int piece = i * kTThreads + tid, wp = i * kTThreads + wave_piece;  // wp: wave-uniform
        const bool is_k = wp < 4 * HD;
        const rsrc_t r = is_k ? src.k : src.v;
        const uint32_t vo = wp >= 8 * HD ? kNoKv : (uint32_t)(is_k ? piece : piece - 4 * HD) * 16u;
        c.r[i] = bld16(r, vo, so);
    }
}
// In LDS each 1 KiB chunk (the 64 16-byte pieces one MFMA operand load reads,
// piece r * 4 + g for lane (r16 = r, g)) is stored with the pieces of a row r
// permuted, g -> g ^ ((r >> 1) & 3): the 8 lanes of one LDS pass (same g,
// r = 8q .. 8q+7) then touch 8 different 4-bank groups instead of 2.
__device__ __forceinline__ int lds_swz(int piece) {
    const int w = piece & 63, r = w >> 2;
    return (piece & ~63) + r * 4 + ((w & 3) ^ ((r >> 1) & 3));
}
template <int HD>
__device__ __forceinline__ void tile_store(uintx4 *stage, const TileCopy<HD> &c, int tid) {
#pragma unroll
    for (int i = 0; i < tile_pieces<HD>(); i++)
        if (i * kTThreads + tid < 8 * HD) stage[lds_swz(i * kTThreads + tid)] = c.r[i];
}

// One 32-key block from LDS for the wave's query tiles (dead tiles skipped)
// (lp: the lane's swizzled piece inside a chunk, lds_swz(r16 * 4 + g))
template <int HD, int QT>
__device__ __forceinline__ void tile_step(AttnState<HD, QT> &S, const uintx4 *stage, int lp, const bool (&tl)[QT],
                                          int kk, int P, int T, int lim, int g) {
    constexpr int NDC = HD / 32, NDT = HD / 16;
    uintx4 kop[2][NDC];
#pragma unroll
    for (int kt = 0; kt < 2; kt++)
#pragma unroll
        for (int dc = 0; dc < NDC; dc++) kop[kt][dc] = stage[kt * 2 * HD + dc * 64 + lp];
    half8 bp[QT];
    float alpha[QT];
    bool moved = false;
#pragma unroll
    for (int t = 0; t < QT; t++) {
        alpha[t] = 1.f;
        bp[t] = half8{};
        if (!tl[t]) continue;
        floatx4 st[2];
        step_scores<HD, QT>(S, kop, t, st);
        bp[t] = step_softmax<HD, QT>(S, t, st, kk, P, T, lim, g, alpha[t], moved);
    }
    uintx4 vop[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; dt++) vop[dt] = stage[4 * HD + dt * 64 + lp];
    zero_stale_v<NDT>(vop, kk, T, g);
    step_pv<HD, QT>(S, vop, bp, alpha, moved, tl);
}

template <int HD> constexpr size_t attn_t_lds() { return (size_t)kTStages * 8 * HD * 16; }

template <int HD>
__global__ __launch_bounds__(kTThreads) void k_attn_t(AttnParams p) {
    warm_kernargs<sizeof(AttnParams)>();
    constexpr int QT = kTQW, SW = 8 * HD;  // SW: 16-byte pieces of one stage
    extern __shared__ uintx4 lds[];
    const int h = blockIdx.x, s = blockIdx.y, qb = blockIdx.z;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int tid = threadIdx.x;
    const int r16 = lane & 15, g = lane >> 4;
    const int nq = p.M * p.n_rep;
    const int T = p.P + p.M;
    const int kps = 4 * p.keys_per_wave;  // keys of a split
    const int k0 = s * kps, lim = min(k0 + kps, T);
    const int nb = (lim - k0 + 31) / 32;
    const uint32_t stream_bytes = (uint32_t)p.cap * HD * 2u;
    KvSrc src;
    src.k = make_rsrc(p.kc + (int64_t)h * p.cap * HD, stream_bytes);
    src.v = make_rsrc(p.vc + (int64_t)h * p.cap * HD, stream_bytes);
    src.lane = (uint32_t)(r16 * 32 + g * 8) * 2u;
    const int lp = lds_swz(r16 * 4 + g);
    auto blk = [&](int j) { return k0 + 32 * j < lim ? k0 + 32 * j : -1; };

    // the queries first, then the first blocks' copies
    QueryRaw<HD> qr[QT];
    bool tl[QT];
#pragma unroll
    for (int t = 0; t < QT; t++) {
        const int tile = (qb * kTWaves + wave) * QT + t;
        tl[t] = tile * 16 < nq;  // wave-uniform: the tile holds a live query
        query_fetch<HD>(qr[t], p, h, tile * 16 + r16, g);
    }
    TileCopy<HD> c0, c1, c2;
    tile_fetch<HD>(c0, src, blk(0), tid);
    tile_fetch<HD>(c1, src, blk(1), tid);
    tile_fetch<HD>(c2, src, blk(2), tid);

    AttnState<HD, QT> S;
    const float sl2 = p.scale * 1.4426950408889634f;
#pragma unroll
    for (int t = 0; t < QT; t++) query_init<HD, QT>(S, t, qr[t], sl2);

    // block j lives in stage j % 3; it is written after every wave passed the
    // barrier of block j - 1, i.e. finished block j - 2 and so block j - 3.
    for (int j = 0; j < nb; j += 3) {
        tile_store<HD>(lds, c0, tid);
        tile_fetch<HD>(c0, src, blk(j + 3), tid);
        __syncthreads();
        tile_step<HD, QT>(S, lds, lp, tl, k0 + 32 * j, p.P, T, lim, g);
        if (j + 1 >= nb) break;
        tile_store<HD>(lds + SW, c1, tid);
        tile_fetch<HD>(c1, src, blk(j + 4), tid);
        __syncthreads();
        tile_step<HD, QT>(S, lds + SW, lp, tl, k0 + 32 * (j + 1), p.P, T, lim, g);
        if (j + 2 >= nb) break;
        tile_store<HD>(lds + 2 * SW, c2, tid);
        tile_fetch<HD>(c2, src, blk(j + 5), tid);
        __syncthreads();
        tile_step<HD, QT>(S, lds + 2 * SW, lp, tl, k0 + 32 * (j + 2), p.P, T, lim, g);
    }
#pragma unroll
    for (int t = 0; t < QT; t++) {
        const int q = ((qb * kTWaves + wave) * QT + t) * 16 + r16;
        const float l = xsum4(S.l[t]);  // the query's 4 partial sums
        if (q < nq) attn_emit<HD>(p, s, h * p.n_rep + q % p.n_rep, q / p.n_rep, g, S.o[t], S.m[t], l);
    }
}

// ---- combine splits -> fp16 fragment-layout input of wo ----------------------
// Thread (row, c) of a 128-thread workgroup owns dims [8c, 8c + 8) of one
// partial row (head, m).  The row's threads stage every split's (m_s, l_s)
// in LDS (thread c loads splits c, c + 16, ...), and each thread requests its
// dims of every split at once (up to NS splits; loads past nsplit read zeros
// without a memory access), so the merge waits for one memory round trip.
// Splits are merged in index order:
// out = sum_s w_s o_s / sum_s w_s, w_s = l_s * exp2(m_s - max m).
constexpr int kCombThreads = 128;
constexpr int kCombMaxSplits = 80;  // >= attn_max_splits for every n_kv
template <int NS> __global__ __launch_bounds__(kCombThreads) void k_attn_combine(AttnParams p) {
    warm_kernargs<sizeof(AttnParams)>();
    const int HD = p.hd, ns = p.nsplit;
    const int tpr = HD / 8, rows = kCombThreads / tpr;  // threads per row, rows per workgroup
    const int rl = (int)threadIdx.x / tpr, c = (int)threadIdx.x % tpr;
    const int64_t nrows = (int64_t)p.n_heads * p.M;
    const int64_t row = min((int64_t)blockIdx.x * rows + rl, nrows - 1);  // = head * M + m
    const rsrc_t ro = make_rsrc(p.part_o, (uint32_t)(ns * nrows * HD * 2));
    const rsrc_t rml = make_rsrc(p.part_ml, (uint32_t)(ns * nrows * 8));
    const uint32_t vo = (uint32_t)((row * HD + 8 * c) * 2), vml = (uint32_t)(row * 8);
    constexpr int NML = (NS + 7) / 8;  // (m, l) loads of a thread (tpr >= 8)
    uintx2 ml[NML];
#pragma unroll
    for (int i = 0; i < NML; i++) {
        const int sp = c + tpr * i;
        ml[i] = bld8(rml, sp < ns ? vml + (uint32_t)(sp * nrows * 8) : 0x80000000u, 0u);
    }
    uintx4 ov[NS];
#pragma unroll
    for (int sp = 0; sp < NS; sp++) ov[sp] = bld16(ro, vo, uni(sp < ns ? (uint32_t)(sp * nrows * HD * 2) : 0x80000000u));
    __shared__ float cml[kCombThreads / 8][kCombMaxSplits][2];
#pragma unroll
    for (int i = 0; i < NML; i++) {
        const int sp = c + tpr * i;
        if (sp < ns) {
            cml[rl][sp][0] = __uint_as_float(ml[i].x);
            cml[rl][sp][1] = __uint_as_float(ml[i].y);
        }
    }
    __syncthreads();
    float mx = -INFINITY;
    for (int sp = 0; sp < ns; sp++) mx = fmaxf(mx, cml[rl][sp][0]);
    float W = 0.f, acc[8];
#pragma unroll
    for (int i = 0; i < 8; i++) acc[i] = 0.f;
#pragma unroll
    for (int sp = 0; sp < NS; sp++) {
        if (sp < ns) {
            const float ms = cml[rl][sp][0];
            const float w = ms == -INFINITY ? 0.f : cml[rl][sp][1] * exp2f(ms - mx);
            W += w;
            const uint32_t wd[4] = {ov[sp].x, ov[sp].y, ov[sp].z, ov[sp].w};
#pragma unroll
            for (int i = 0; i < 8; i++) acc[i] += h2f((uint16_t)(wd[i >> 1] >> (16 * (i & 1)))) * w;
        }
    }
    if ((int64_t)blockIdx.x * rows + rl >= nrows) return;
    const int head = (int)(row / p.M), m = (int)(row % p.M);
    // dims 4k .. 4k + 3 sit in fragment slots f, f + 2, f + 1, f + 3
#pragma unroll
    for (int k = 0; k < 2; k++) {
        const int64_t e = (int64_t)head * HD + 8 * c + 4 * k;
        *(uintx2 *)(p.out16 + (int64_t)m * p.out_ld + frag_index(e)) =
            uintx2{(uint32_t)f2h(acc[4 * k] / W) | ((uint32_t)f2h(acc[4 * k + 2] / W) << 16),
                   (uint32_t)f2h(acc[4 * k + 1] / W) | ((uint32_t)f2h(acc[4 * k + 3] / W) << 16)};
    }
}

// ---- host launchers ----------------------------------------------------------
#define SD_ATTN_CHECK(x)                                                                           \
    do {                                                                                           \
        const hipError_t e_ = (x);                                                                 \
        if (e_ != hipSuccess) throw BackendError(std::string("attention: ") + hipGetErrorString(e_)); \
    } while (0)
void launch_rope_kv(const RopeKvParams &p, hipStream_t st) {
    if (p.hd % 8 || p.ld_qkv % 4) throw BackendError("rope_kv: head_dim must be a multiple of 8");
    const int units = (p.n_heads + p.n_kv) * (p.hd / 4);
    hipLaunchKernelGGL(k_rope_kv, dim3(p.M, (units + 63) / 64), dim3(64), 0, st, p);
}

static int attn_target_splits(int n_kv) { return n_kv >= 64 ? 1 : 64 / n_kv; }

// Up to 16 rows (a linear verify or a decode step) the key ranges are a
// function of P alone, so each row's arithmetic is the same as in a one-row
// call.  Above, the splits shrink as query blocks grow, towards one 8-wave
// workgroup per CU (256).
AttnSplit attn_split(int P, int M, int n_kv, int n_rep) {
    const int T = P + M;
    if (M > 16) {
        // k_attn_t: splits of kps keys (whole 32-key blocks), towards one
        // workgroup per CU over the query blocks
        const int nqt = (M * n_rep + 15) / 16, nqb = (nqt + kTWaves * kTQW - 1) / (kTWaves * kTQW);
        int want = 256 / (n_kv * nqb);
        want = want < 1 ? 1 : want > kTMaxSplits ? kTMaxSplits : want;
        int kps = (P + 1 + want - 1) / want;
        kps = kps < 32 ? 32 : (kps + 31) / 32 * 32;
        return AttnSplit{kps / 4, (T + kps - 1) / kps};
    }
    const int want = attn_target_splits(n_kv);
    int kpw = (P + 1 + 4 * want - 1) / (4 * want);
    kpw = kpw < 32 ? 32 : (kpw + 31) / 32 * 32;
    return AttnSplit{kpw, (T + 4 * kpw - 1) / (4 * kpw)};
}

// split size >= (P + 1) / want and >= 32, so for M <= 128
// nsplit = ceil((P + M) / size) <= want + 1 + 128 / 32
int attn_max_splits(int n_kv) {
    const int t = attn_target_splits(n_kv);
    const int n = (t > kTMaxSplits ? t : kTMaxSplits) + 5;
    return n < kCombMaxSplits ? n : kCombMaxSplits;
}

// LDS beyond the 64 KiB default for the M > 16 kernel: a function attribute
// set once per device (the caller's current device), under a lock, since
// handles on different devices may launch from different threads.
static void allow_attn_t_lds() {
    static std::mutex mu;
    static std::vector<bool> done;
    int dev = 0;
    SD_ATTN_CHECK(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lock(mu);
    if ((size_t)dev < done.size() && done[dev]) return;
    SD_ATTN_CHECK(hipFuncSetAttribute((const void *)k_attn_t<128>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                      (int)attn_t_lds<128>()));
    SD_ATTN_CHECK(hipFuncSetAttribute((const void *)k_attn_t<64>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                      (int)attn_t_lds<64>()));
    if ((size_t)dev >= done.size()) done.resize(dev + 1, false);
    done[dev] = true;
}

void launch_attention(const AttnParams &p, hipStream_t st) {
    // a split covers 4 * keys_per_wave keys: whole 32-key blocks, and whole
    // 32-key steps of each of the 4 waves up to 16 rows
    const int kps_unit = p.M > 16 ? 8 : 32;
    if (p.keys_per_wave < kps_unit || p.keys_per_wave % kps_unit) throw BackendError("attention: keys_per_wave");
    if ((int64_t)p.nsplit * 4 * p.keys_per_wave < (int64_t)p.P + p.M) throw BackendError("attention: splits too few");
    if ((int64_t)(p.nsplit - 1) * 4 * p.keys_per_wave >= (int64_t)p.P + p.M) throw BackendError("attention: empty split");
    if (p.cap % 32 || (int64_t)p.P + p.M > p.cap) throw BackendError("attention: cache capacity");
    if (p.mask_words < 1 || p.mask_words > 2 || p.M > 64 * p.mask_words) throw BackendError("attention: mask words");
    if (p.hd != 128 && p.hd != 64) throw BackendError("attention: head_dim must be 64 or 128");
    const int nq = p.M * p.n_rep, nqt = (nq + 15) / 16;
    if (p.M > 16) {
        // query blocks of kTWaves waves x kTQW tiles sharing each key block through LDS
        const dim3 grid(p.n_kv, p.nsplit, (nqt + kTWaves * kTQW - 1) / (kTWaves * kTQW));
        allow_attn_t_lds();
        if (p.hd == 128) hipLaunchKernelGGL(k_attn_t<128>, grid, dim3(kTThreads), attn_t_lds<128>(), st, p);
        else hipLaunchKernelGGL(k_attn_t<64>, grid, dim3(kTThreads), attn_t_lds<64>(), st, p);
    } else {
        AttnParams a = p;
        a.fused_combine = 0;
        if (p.nsplit > 1 && p.split_cnt) {
            if ((int64_t)p.n_kv * nqt > p.split_cnt_len) throw BackendError("attention: split counters too few");
            a.fused_combine = p.nsplit <= kFusedMaxSplits;
        }
        // One query tile per wave keeps a wave within 256 registers (two
        // double-buffered 32-key operand sets and its accumulators), so two
        // waves share each SIMD.  Query tiles become workgroups along z; with the
        // KV head as blockIdx.x and n_kv a multiple of the 8 XCDs, every
        // workgroup of one head lands on the same XCD, so the query tiles re-read
        // that head's keys from its L2.
        const dim3 grid(p.n_kv, p.nsplit, nqt);
        if (p.hd == 128) hipLaunchKernelGGL((k_attn<128, 1>), grid, dim3(256), 0, st, a);
        else hipLaunchKernelGGL((k_attn<64, 1>), grid, dim3(256), 0, st, a);
        if (a.fused_combine) return;
    }
    if (p.nsplit > 1) {
        if (p.nsplit > kCombMaxSplits) throw BackendError("attention: too many splits to combine");
        const int rows = kCombThreads / (p.hd / 8);
        const int64_t nrows = (int64_t)p.n_heads * p.M;
        if ((int64_t)p.nsplit * nrows * p.hd * 2 >= 0x80000000LL) throw BackendError("attention: partials too large");
        const dim3 grid((unsigned)((nrows + rows - 1) / rows)), block(kCombThreads);
        if (p.nsplit <= 8) hipLaunchKernelGGL(k_attn_combine<8>, grid, block, 0, st, p);
        else if (p.nsplit <= 16) hipLaunchKernelGGL(k_attn_combine<16>, grid, block, 0, st, p);
        else if (p.nsplit <= 24) hipLaunchKernelGGL(k_attn_combine<24>, grid, block, 0, st, p);
        else if (p.nsplit <= 32) hipLaunchKernelGGL(k_attn_combine<32>, grid, block, 0, st, p);
        else if (p.nsplit <= 40) hipLaunchKernelGGL(k_attn_combine<40>, grid, block, 0, st, p);
        else hipLaunchKernelGGL(k_attn_combine<kCombMaxSplits>, grid, block, 0, st, p);
    }
}

}  // namespace sd
