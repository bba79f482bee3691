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
// Split flash-decoding (sd_attn_dev.hpp).  Up to 16 tokens: grid (kv head,
// key split, query tile); a workgroup's 8 waves take the split's 32-key steps
// in turn for one query tile (16 of the n_rep query heads of the KV head times
// the M tokens); their partial softmax states are merged in LDS in a fixed
// order, and the splits by the last workgroup of the tile to finish (a counter
// per tile, device-scope partials) or by a combine kernel, with the same
// arithmetic; nothing to merge when one split covers all keys.  The same
// workgroups also run inside the fused Q/K/V launch (sd_qgemm.hip).
// keys_per_wave and the split boundaries depend on P only, so a query's result
// does not depend on how many other queries share the call.
#include <algorithm>
#include <mutex>
#include <vector>

#include "sd_attn_dev.hpp"
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

// M <= 16 (decode, linear verify): see attn_wg.  Grid (kv head, key split,
// query tile).
template <int HD>
__global__ __launch_bounds__(kAttnThreads) __attribute__((amdgpu_waves_per_eu(2))) void k_attn(AttnParams) {
    warm_kernargs<sizeof(AttnParams)>();
    attn_wg<HD, false>(kernarg<AttnParams>(), blockIdx.x, blockIdx.y, blockIdx.z, AttnWait{});
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

// Up to 16 rows (a linear verify or a decode step) the key ranges are a
// function of P alone, so each row's arithmetic is the same as in a one-row
// call: a split is 8 waves x 3 steps of 32 keys below 1024 cached positions
// (one split up to ~750), else 8 waves x as many steps as give about 64 / n_kv
// splits; each wave's first two steps sit in its registers (requested while
// the fused launch's matmul runs), later ones stream behind them.  Above 16
// rows, the splits shrink as query blocks grow, towards one 8-wave workgroup
// per CU (256).
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
    // steps per wave: 3 (one split) for short prefixes, else as few as give
    // about 64 / n_kv splits (64 workgroups per query tile), at most 32
    const int want = std::min(kTMaxSplits, n_kv >= 64 ? 1 : 64 / n_kv);
    const int spw = P < 1024 ? 3 : std::max(1, (P + 1 + 8 * 32 * want - 1) / (8 * 32 * want));
    const int kps = 8 * 32 * spw;                                            // keys per split
    return AttnSplit{32 * spw, (T + kps - 1) / kps};
}

// above 16 rows the split size is >= (P + 1) / want and >= 32 with
// want <= kTMaxSplits, so for M <= 128 nsplit = ceil((P + M) / size) <=
// want + 1 + 128 / 32; up to 16 rows a split holds 768 keys below 1024
// cached positions (nsplit <= 2) and >= (P + 1) / want above (nsplit <=
// want + 1 <= kTMaxSplits + 1)
static_assert(kTMaxSplits + 5 <= kCombMaxSplits && kTMaxSplits + 5 <= kFusedMaxSplits, "split bounds");
int attn_max_splits(int) { return kTMaxSplits + 5; }

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

static void attn_check(const AttnParams &p) {
    // a split covers waves x keys_per_wave keys: whole 32-key blocks (4 waves
    // above 16 rows), and whole 32-key steps of each of the 8 waves up to 16
    const int kps_unit = p.M > 16 ? 8 : 32, waves = p.M > 16 ? 4 : 8;
    if (p.keys_per_wave < kps_unit || p.keys_per_wave % kps_unit) throw BackendError("attention: keys_per_wave");
    if ((int64_t)p.nsplit * waves * p.keys_per_wave < (int64_t)p.P + p.M) throw BackendError("attention: splits too few");
    if ((int64_t)(p.nsplit - 1) * waves * p.keys_per_wave >= (int64_t)p.P + p.M)
        throw BackendError("attention: empty split");
    if (p.cap % 32 || (int64_t)p.P + p.M > p.cap) throw BackendError("attention: cache capacity");
    if (p.mask_words < 1 || p.mask_words > 2 || p.M > 64 * p.mask_words) throw BackendError("attention: mask words");
    if (p.hd != 128 && p.hd != 64) throw BackendError("attention: head_dim must be 64 or 128");
}

AttnParams attn_small_params(const AttnParams &p) {
    attn_check(p);
    if (p.M > 16) throw BackendError("attention: more than 16 rows");
    const int nqt = (p.M * p.n_rep + 15) / 16;
    AttnParams a = p;
    a.fused_combine = 0;
    if (p.nsplit > 1 && p.split_cnt) {
        if ((int64_t)p.n_kv * nqt > p.split_cnt_len) throw BackendError("attention: split counters too few");
        a.fused_combine = p.nsplit <= kFusedMaxSplits;
    }
    return a;
}

int attn_small_workgroups(const AttnParams &p) { return p.n_kv * p.nsplit * ((p.M * p.n_rep + 15) / 16); }

void launch_attn_combine(const AttnParams &p, hipStream_t st) {
    if (p.nsplit <= 1) return;
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

void launch_attention(const AttnParams &p, hipStream_t st) {
    if (p.M > 16) {
        attn_check(p);
        // query blocks of kTWaves waves x kTQW tiles sharing each key block through LDS
        const int nqt = (p.M * p.n_rep + 15) / 16;
        const dim3 grid(p.n_kv, p.nsplit, (nqt + kTWaves * kTQW - 1) / (kTWaves * kTQW));
        allow_attn_t_lds();
        if (p.hd == 128) hipLaunchKernelGGL(k_attn_t<128>, grid, dim3(kTThreads), attn_t_lds<128>(), st, p);
        else hipLaunchKernelGGL(k_attn_t<64>, grid, dim3(kTThreads), attn_t_lds<64>(), st, p);
        launch_attn_combine(p, st);
        return;
    }
    const AttnParams a = attn_small_params(p);
    // One query tile per wave keeps a wave within 256 registers (two
    // double-buffered 32-key operand sets and its accumulators), so two waves
    // share each SIMD.  Query tiles become workgroups along z; with the KV head
    // as blockIdx.x and n_kv a multiple of the 8 XCDs, every workgroup of one
    // head lands on the same XCD, so the query tiles re-read that head's keys
    // from its L2.
    const dim3 grid(p.n_kv, p.nsplit, (p.M * p.n_rep + 15) / 16);
    if (p.hd == 128) hipLaunchKernelGGL(k_attn<128>, grid, dim3(kAttnThreads), 0, st, a);
    else hipLaunchKernelGGL(k_attn<64>, grid, dim3(kAttnThreads), 0, st, a);
    if (!a.fused_combine) launch_attn_combine(a, st);
}

}  // namespace sd
