// Device code of the M <= 16 attention workgroup (split flash-decoding over
// the blocked fp16 KV cache) and the helpers the tree kernel shares with it.
// Included by sd_attn.hip (the attention launches) and sd_qgemm.hip (the fused
// Q/K/V + attention launch), so both compile the same arithmetic.
//
// Attention is split flash-decoding with the KV streamed straight from HBM
// into MFMA operand registers (no LDS staging): the blocked cache layout makes
// every operand a 16-byte load per lane, 1 KiB contiguous per wave.  Scores
// are computed transposed, S^T = K Q^T (16 keys x 16 queries per MFMA tile),
// so a lane's accumulator already holds the P^T operand of O^T = V^T P^T.
#pragma once
#include "sd_buffer.hpp"
#include "sd_common.hpp"
#include "sd_kernels_attn.hpp"

// products and sums may fuse within this code (the includer's setting is
// restored at the end of the file: -ffp-contract=on)
#pragma clang fp contract(fast)

namespace sd {

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

// 32 keys [kk, kk+32) of one stream (kk < 0: none): 16-byte pieces, 1 KiB per wave each.
// dev (wave-uniform): some of the keys were written during this launch by
// other workgroups, so they are read at device scope.
template <int HD, int CP>
__device__ __forceinline__ void kv_load_k_cp(KvStep<HD> &b, const KvSrc &s, uint32_t so) {
#pragma unroll
    for (int kt = 0; kt < 2; kt++)
#pragma unroll
        for (int dc = 0; dc < HD / 32; dc++) b.k[kt][dc] = bld16<CP>(s.k, s.lane + kt * 32 * HD + dc * 1024, so);
}
template <int HD, int CP>
__device__ __forceinline__ void kv_load_v_cp(KvStep<HD> &b, const KvSrc &s, uint32_t so) {
#pragma unroll
    for (int dt = 0; dt < HD / 16; dt++) b.v[dt] = bld16<CP>(s.v, s.lane + dt * 1024, so);
}
template <int HD>
__device__ __forceinline__ void kv_load_k(KvStep<HD> &b, const KvSrc &s, int kk, bool dev = false) {
    const uint32_t so = kv_so(kk, HD);
    if (dev) kv_load_k_cp<HD, kLoadDev>(b, s, so);
    else kv_load_k_cp<HD, 0>(b, s, so);
}
template <int HD>
__device__ __forceinline__ void kv_load_v(KvStep<HD> &b, const KvSrc &s, int kk, bool dev = false) {
    const uint32_t so = kv_so(kk, HD);
    if (dev) kv_load_v_cp<HD, kLoadDev>(b, s, so);
    else kv_load_v_cp<HD, 0>(b, s, so);
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
// DEV: the queries were written during this launch by other workgroups and
// are read at device scope.
template <int HD, bool DEV = false>
__device__ __forceinline__ void query_fetch(QueryRaw<HD> &r, const AttnParams &p, int h, int q, int g) {
    const int nq = p.M * p.n_rep;
    r.live = q < nq;
    const int qc = r.live ? q : nq - 1;
    const int m = qc / p.n_rep, rep = qc % p.n_rep;
    const uint16_t *qr = p.q16 + ((int64_t)(h * p.n_rep + rep) * p.M + m) * HD;
#pragma unroll
    for (int dc = 0; dc < HD / 32; dc++) {
        if constexpr (DEV) {
            const uint64_t a = ld_dev64(qr + dc * 32 + g * 8), b = ld_dev64(qr + dc * 32 + g * 8 + 4);
            r.q[dc] = uintx4{(uint32_t)a, (uint32_t)(a >> 32), (uint32_t)b, (uint32_t)(b >> 32)};
        } else {
            r.q[dc] = *(const uintx4 *)(qr + dc * 32 + g * 8);
        }
    }
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
// Steps reaching key dev_from or beyond are read at device scope.
template <int HD, int QT>
__device__ __forceinline__ void attn_step(AttnState<HD, QT> &S, KvStep<HD> &b, KvStep<HD> &nb, const KvSrc &src,
                                          int kk, int k1, int P, int T, int g, int dev_from) {
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
    kv_load_v<HD>(nb, src, kk + 32 < k1 ? kk + 32 : -1, kk + 64 > dev_from);
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

// The merge of one 16-query tile by 256 threads (active; thread t's row and
// dims from t & 255).  Every thread of the workgroup calls it, so a barrier
// (more than 16 splits) is reached by every wave.  cml: LDS scratch.
template <int HD>
__device__ __forceinline__ void attn_merge_tile(const AttnParams &p, int h, int qg, bool active,
                                                float (*cml)[kFusedMaxSplits][2]) {
    constexpr int DPT = HD / 16;  // dims per thread, 4 or 8: one or two 8-byte loads per split
    const int t = threadIdx.x & 255, r = t >> 4, c = t & 15;
    const int nq = p.M * p.n_rep, ns = p.nsplit;
    const int q = qg * 16 + r;
    const bool live = active && q < nq;
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

// ---- one workgroup of the M <= 16 kernel ------------------------------------
// 512 threads, 8 waves, one 16-query tile qg of KV head h (16 of the n_rep
// query heads x M tokens) and split s of the keys.  A split is 8 kpw keys
// (kpw = keys_per_wave, a multiple of 32) taken in 32-key steps dealt round
// the waves: wave w owns steps s * 8 spw + w + 8 j, j < spw (spw = kpw / 32),
// so a wave's first two steps are the split's first 16, each wave holds them
// in its two register buffers, and step j + 2 loads as soon as step j is
// done.  The 8 partial softmax states are merged in LDS in a fixed order
// (((o0 + o4) + (o2 + o6)) + ((o1 + o5) + (o3 + o7))); with one split that
// is the result, else the splits are merged by the last of the tile's
// workgroups to finish (fused_combine) or by the combine kernel.
constexpr int kAttnThreads = 512;

// The attention part of a launch whose first workgroups produce the queries
// and the new K/V rows (the fused Q/K/V launch, M <= 16).  Producer
// workgroup j covers the hd columns of head j of the launch's q | k | v heads
// in hd / 32 workgroups: j * hd / 32 + i, i < hd / 32 (two 16-row tiles each,
// d and d + hd / 2).  When its rows are stored it writes epoch (the launch's
// number, never 0) to flags[its index].  An attention workgroup of KV head h
// waits for the producers of its rows only: q heads h n_rep .. (h + 1) n_rep - 1,
// k head h and v head h.  A flag per producer (distinct words, plain stores)
// instead of one shared counter: device-scope atomics on one word from a few
// hundred workgroups queue for microseconds.  A wait that exceeds `polls`
// device-scope reads (kWaitPolls: about a second) gives up: the workgroup
// writes nothing and sets *status (host-visible memory), which the host
// checks after the step.  The attention waits for `want`, which is epoch
// except under fault injection (a number no producer writes).
struct AttnWait {
    unsigned *flags;
    unsigned epoch, want;
    int *status;
    int polls;
};
constexpr int kWaitPolls = 1 << 21;

// Wave 0 waits until every producer of KV head h's rows has flagged this
// epoch, then the verdict reaches the whole workgroup through LDS.
template <int HD>
__device__ __forceinline__ bool attn_wait(const AttnWait &w, const AttnParams &p, int h) {
    __shared__ int s_go;
    if (threadIdx.x < 64) {
        constexpr int WPH = HD / 32;  // producer workgroups per head
        const int lane = threadIdx.x, nqw = WPH * p.n_rep, cnt = WPH * (p.n_rep + 2);
        bool ok = false;
        for (int it = 0; it < w.polls; it++) {
            bool all = true;
            for (int i = lane; i < cnt; i += 64) {
                const int j = i < nqw ? WPH * h * p.n_rep + i
                            : i < nqw + WPH ? WPH * (p.n_heads + h) + (i - nqw)
                                            : WPH * (p.n_heads + p.n_kv + h) + (i - nqw - WPH);
                all = all && __hip_atomic_load(w.flags + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == w.want;
            }
            if (__builtin_amdgcn_ballot_w64(!all) == 0) {
                ok = true;
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
        if (lane == 0) {
            if (!ok) __hip_atomic_store(w.status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            s_go = ok;
        }
    }
    __syncthreads();
    return s_go != 0;
}

// One 32-key step from a register buffer: scores, softmax, PV.
template <int HD>
__device__ __forceinline__ void attn_step1(AttnState<HD, 1> &S, KvStep<HD> &b, int kk, int P, int T, int g) {
    floatx4 st[2];
    float alpha;
    bool moved = false;
    const bool tl[1] = {true};
    step_scores<HD, 1>(S, b.k, 0, st);
    const half8 bp[1] = {step_softmax<HD, 1>(S, 0, st, kk, P, T, T, g, alpha, moved)};
    const float al[1] = {alpha};
    zero_stale_v<HD / 16>(b.v, kk, T, g);
    step_pv<HD, 1>(S, b.v, bp, al, moved, tl);
}

// FUSED: the workgroup belongs to the fused Q/K/V launch.  Its first two
// steps' cached keys (positions < P) are requested before the wait; the
// queries and the blocks that hold position P or later are read after it, at
// device scope (another XCD wrote them during this launch).
template <int HD, bool FUSED>
__device__ __forceinline__ void attn_wg(const AttnParams &p, int h, int s, int qg, const AttnWait &wt) {
    constexpr int NDT = HD / 16;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r16 = lane & 15, g = lane >> 4;
    const int nq = p.M * p.n_rep;
    const int T = p.P + p.M;
    const int spw = p.keys_per_wave >> 5;
    // key of the wave's step j (-1: none)
    auto key = [&](int j) {
        const int k = 32 * (s * 8 * spw + wave + 8 * j);
        return j < spw && k < T ? k : -1;
    };
    const uint32_t stream_bytes = (uint32_t)p.cap * HD * 2u;
    KvSrc src;
    src.k = make_rsrc(p.kc + (int64_t)h * p.cap * HD, stream_bytes);
    src.v = make_rsrc(p.vc + (int64_t)h * p.cap * HD, stream_bytes);
    src.lane = (uint32_t)(r16 * 32 + g * 8) * 2u;
    // a step holds rows written during a fused launch when it reaches P
    auto fresh = [&](int kk) { return FUSED && kk >= 0 && kk + 32 > p.P; };
    __shared__ float sml[8][16][2];
    __shared__ __attribute__((aligned(16))) floatx4 sob[4][NDT][64];

    // the queries (just written by the Q/K/V launch) and the first two steps
    QueryRaw<HD> qr;
    KvStep<HD> b0, b1;
    if constexpr (!FUSED) query_fetch<HD>(qr, p, h, qg * 16 + r16, g);
    kv_load_k<HD>(b0, src, key(0));
    kv_load_v<HD>(b0, src, key(0));
    kv_load_k<HD>(b1, src, key(1));
    kv_load_v<HD>(b1, src, key(1));
    if constexpr (FUSED) {
        if (!attn_wait<HD>(wt, p, h)) return;
        query_fetch<HD, true>(qr, p, h, qg * 16 + r16, g);
        if (fresh(key(0))) {
            kv_load_k<HD>(b0, src, key(0), true);
            kv_load_v<HD>(b0, src, key(0), true);
        }
        if (fresh(key(1))) {
            kv_load_k<HD>(b1, src, key(1), true);
            kv_load_v<HD>(b1, src, key(1), true);
        }
    }

    AttnState<HD, 1> S;
    const float sl2 = p.scale * 1.4426950408889634f;  // scale * log2(e): softmax in base 2
    query_init<HD, 1>(S, 0, qr, sl2);
    for (int j = 0;; j += 2) {
        const int ka = key(j);
        if (ka < 0) break;
        attn_step1<HD>(S, b0, ka, p.P, T, g);
        kv_load_k<HD>(b0, src, key(j + 2), fresh(key(j + 2)));
        kv_load_v<HD>(b0, src, key(j + 2), fresh(key(j + 2)));
        const int kb = key(j + 1);
        if (kb < 0) break;
        attn_step1<HD>(S, b1, kb, p.P, T, g);
        kv_load_k<HD>(b1, src, key(j + 3), fresh(key(j + 3)));
        kv_load_v<HD>(b1, src, key(j + 3), fresh(key(j + 3)));
    }
    S.l[0] = xsum4(S.l[0]);  // the query's 4 partial sums

    // ---- merge the 8 waves: rescale to the common max, then
    // ((o0 + o4) + (o2 + o6)) + ((o1 + o5) + (o3 + o7)) through LDS ----
    if (g == 0) {
        sml[wave][r16][0] = S.m[0];
        sml[wave][r16][1] = S.l[0];
    }
    __syncthreads();
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < 8; w++) mx = fmaxf(mx, sml[w][r16][0]);
    float L = 0.f, fme = 0.f;
#pragma unroll
    for (int w = 0; w < 8; w++) {
        const float mw = sml[w][r16][0];
        const float f = mw == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw - mx);
        L += sml[w][r16][1] * f;
        if (w == wave) fme = f;
    }
#pragma unroll
    for (int dt = 0; dt < NDT; dt++) S.o[0][dt] *= fme;
    // s_w = o_w + o_(w+4) on waves 0..3 (a wave reads, then rewrites, only its
    // own slot), then wave 0 forms (s0 + s2) + (s1 + s3)
    if (wave >= 4) {
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) sob[wave - 4][dt][lane] = S.o[0][dt];
    }
    __syncthreads();
    if (wave < 4) {
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) {
            S.o[0][dt] += sob[wave][dt][lane];
            if (wave > 0) sob[wave][dt][lane] = S.o[0][dt];
        }
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) S.o[0][dt] = (S.o[0][dt] + sob[2][dt][lane]) + (sob[1][dt][lane] + sob[3][dt][lane]);
    }
    const bool fused = p.fused_combine != 0;
    const int q = qg * 16 + r16;
    if (wave == 0 && q < nq) {
        if (fused) attn_emit<HD, true>(p, s, h * p.n_rep + q % p.n_rep, q / p.n_rep, g, S.o[0], mx, L);
        else attn_emit<HD>(p, s, h * p.n_rep + q % p.n_rep, q / p.n_rep, g, S.o[0], mx, L);
    }
    if (!fused) return;

    // ---- the last of the tile's nsplit workgroups to arrive merges the splits ----
    // Wave 0 wrote the partials (device scope) and waits for those stores to
    // complete before it counts the arrival; the last arrival resets the
    // count for the next launch and reads every split's partials at device
    // scope.
    __shared__ int s_last;
    if (wave == 0) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        if (lane == 0) {
            const int nqt = (nq + 15) >> 4;
            int *cnt = p.split_cnt + (int64_t)h * nqt + qg;
            const int last = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == p.nsplit - 1;
            if (last) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            s_last = last;
        }
    }
    __syncthreads();
    if (!s_last) return;
    // the merge's scratch reuses sob, whose last reads precede the barrier
    // above; threads 256.. only keep its barrier
    static_assert(sizeof(sob) >= 16 * kFusedMaxSplits * 2 * sizeof(float), "merge scratch");
    attn_merge_tile<HD>(p, h, qg, threadIdx.x < 256, (float(*)[kFusedMaxSplits][2])(float *)sob);
}

}  // namespace sd

#pragma clang fp contract(on)
