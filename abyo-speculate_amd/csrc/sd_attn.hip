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
// states are merged in LDS in a fixed order, and the splits by a combine
// kernel (skipped when one split covers all keys).  Up to 16 tokens,
// keys_per_wave and the split boundaries depend on P only, so a query's
// result does not depend on how many other queries share the call.
#include "sd_buffer.hpp"
#include "sd_common.hpp"
#include "sd_kernels_attn.hpp"

namespace sd {

#pragma clang fp contract(off)

// ---- RoPE + KV append ------------------------------------------------------
// projection output (m, col): the matmul's value, or its K-slice partials
// added in slice order plus the bias
__device__ __forceinline__ float qkv_at(const RopeKvParams &p, int m, int col) {
    const int64_t at = (int64_t)m * p.ld_qkv + col;
    if (p.nks <= 1) return p.qkv[at];
    const int64_t stride = (int64_t)p.M * p.ld_qkv;
    float v = p.part[at];
    for (int k = 1; k < p.nks; k++) v += p.part[at + k * stride];
    if (!p.bq) return v;
    const int qd = p.n_heads * p.hd, kvd = p.n_kv * p.hd;
    return v + (col < qd ? p.bq[col] : col < qd + kvd ? p.bk[col - qd] : p.bv[col - qd - kvd]);
}

// grid (M, n_heads + n_kv), block hd/2 threads
__global__ void k_rope_kv(RopeKvParams p) {
    const int m = blockIdx.x, hh = blockIdx.y, i = threadIdx.x;
    const int half = p.hd / 2;
    if (i >= half) return;
    const int pos = p.pos[m];
    const float c = p.cos_t[(int64_t)pos * half + i], s = p.sin_t[(int64_t)pos * half + i];
    int a, b;  // element pair
    if (p.interleaved) {
        a = 2 * i;
        b = 2 * i + 1;
    } else {
        a = i;
        b = i + half;
    }
    if (hh < p.n_heads) {
        const int c0 = hh * p.hd;
        const float x0 = qkv_at(p, m, c0 + a), x1 = qkv_at(p, m, c0 + b);
        uint16_t *q = p.q16 + ((int64_t)hh * p.M + m) * p.hd;
        q[a] = f2h(x0 * c - x1 * s);
        q[b] = f2h(x0 * s + x1 * c);
    } else {
        const int h = hh - p.n_heads;
        const int ck = p.n_heads * p.hd + h * p.hd, cv = (p.n_heads + p.n_kv) * p.hd + h * p.hd;
        uint16_t *ks = p.kc + (int64_t)h * p.cap * p.hd, *vs = p.vc + (int64_t)h * p.cap * p.hd;
        const int64_t t = p.P + m;
        const float k0 = qkv_at(p, m, ck + a), k1 = qkv_at(p, m, ck + b);
        ks[kv_k_off(t, a, p.hd)] = f2h(k0 * c - k1 * s);
        ks[kv_k_off(t, b, p.hd)] = f2h(k0 * s + k1 * c);
        vs[kv_v_off(t, a, p.hd)] = f2h(qkv_at(p, m, cv + a));
        vs[kv_v_off(t, b, p.hd)] = f2h(qkv_at(p, m, cv + b));
    }
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

// One 32-key step for all query tiles: scores and softmax first, then the
// next step's V loads are issued (the current K is dead by then, so the two
// register buffers never hold four operand sets at once), then O^T += V^T P^T.
//
// The running max of a query moves only when a score exceeds it by more than
// 8 (base 2).  Probabilities exp2(s - m) then stay below 256, which fp16 and
// f32 hold with full relative precision, and the rescale of the accumulators
// (a read-modify-write of 32 registers per query tile) is skipped by the whole
// wave unless one of its queries moved.  The final normalisation divides by
// the sum taken against the same maxima, so the result is the softmax.
template <int HD, int QT>
__device__ __forceinline__ void attn_step(AttnState<HD, QT> &S, KvStep<HD> &b, KvStep<HD> &nb, const KvSrc &src,
                                          int kk, int k1, int P, int T, float sl2, int g) {
    constexpr int NDC = HD / 32, NDT = HD / 16;
    const bool full = kk + 32 <= P;  // every key of the step is visible to every query
    half8 bp[QT];
    float alpha[QT];
    bool moved = false;
#pragma unroll
    for (int t = 0; t < QT; t++) {
        floatx4 st[2];
#pragma unroll
        for (int kt = 0; kt < 2; kt++) {
            st[kt] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int dc = 0; dc < NDC; dc++)
                st[kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, b.k[kt][dc]), S.qf[t][dc],
                                                                st[kt], 0, 0, 0);
        }
        float cm = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < 2; kt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                float v = st[kt][i] * sl2;
                if (!full) {
                    const int key = kk + kt * 16 + 4 * g + i;
                    bool vis = key < P;
                    if (!vis && key < T) {
                        const int tt = key - P;
                        vis = (((tt < 64 ? S.mk0[t] : S.mk1[t]) >> (tt & 63)) & 1ull) != 0;
                    }
                    v = vis ? v : -INFINITY;
                }
                st[kt][i] = v;
                cm = fmaxf(cm, v);
            }
        cm = fmaxf(cm, __shfl_xor(cm, 16));
        cm = fmaxf(cm, __shfl_xor(cm, 32));
        const bool up = cm > S.m[t] + 8.f;  // -inf + 8 == -inf: the first finite score always moves it
        const float mnew = up ? cm : S.m[t];
        alpha[t] = up ? __builtin_amdgcn_exp2f(S.m[t] - mnew) : 1.f;
        moved = moved || up;
        const float muse = mnew == -INFINITY ? 0.f : mnew;
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
        ps += __shfl_xor(ps, 16);
        ps += __shfl_xor(ps, 32);
        S.l[t] = S.l[t] * alpha[t] + ps;
        S.m[t] = mnew;
        const uintx4 bu = {pk[0], pk[1], pk[2], pk[3]};
        bp[t] = __builtin_bit_cast(half8, bu);
    }
    kv_load_v<HD>(nb, src, kk + 32 < k1 ? kk + 32 : -1);
    if (kk + 32 > T) {
        // keys >= T hold stale cache rows: their P^T entries are 0, and their V
        // entries are zeroed so that nothing but finite values meets the MFMA
        uint32_t keep[4];
#pragma unroll
        for (int w = 0; w < 4; w++)
            keep[w] = (kk + slot_key(g, 2 * w) < T ? 0x0000ffffu : 0u) |
                      (kk + slot_key(g, 2 * w + 1) < T ? 0xffff0000u : 0u);
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) {
            b.v[dt].x &= keep[0];
            b.v[dt].y &= keep[1];
            b.v[dt].z &= keep[2];
            b.v[dt].w &= keep[3];
        }
    }
    if (__builtin_amdgcn_ballot_w64(moved) != 0) {
#pragma unroll
        for (int t = 0; t < QT; t++)
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) S.o[t][dt] *= alpha[t];
    }
#pragma unroll
    for (int t = 0; t < QT; t++)
#pragma unroll
        for (int dt = 0; dt < NDT; dt++)
            S.o[t][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, b.v[dt]), bp[t], S.o[t][dt],
                                                                0, 0, 0);
}

template <int HD, int QT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void k_attn(AttnParams p) {
    constexpr int NDC = HD / 32, NDT = HD / 16;
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

    AttnState<HD, QT> S;
#pragma unroll
    for (int t = 0; t < QT; t++) {
        const int q = (qg * QT + t) * 16 + r16;
        const bool live = q < nq;
        const int m = live ? q / p.n_rep : 0, r = live ? q % p.n_rep : 0;
        const uint16_t *qr = p.q16 + ((int64_t)(h * p.n_rep + r) * p.M + m) * HD;
#pragma unroll
        for (int dc = 0; dc < NDC; dc++) {
            uintx4 v = {0u, 0u, 0u, 0u};
            if (live) v = *(const uintx4 *)(qr + dc * 32 + g * 8);
            S.qf[t][dc] = __builtin_bit_cast(half8, v);
        }
        S.mk0[t] = p.mask[(int64_t)m * p.mask_words];
        S.mk1[t] = p.mask_words > 1 ? p.mask[(int64_t)m * p.mask_words + 1] : 0ull;
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) S.o[t][dt] = floatx4{0.f, 0.f, 0.f, 0.f};
        S.m[t] = -INFINITY;
        S.l[t] = 0.f;
    }
    const float sl2 = p.scale * 1.4426950408889634f;  // scale * log2(e): softmax in base 2

    // two register buffers: the next 32 keys load while the current ones compute
    // (K at the start of a step, V once the step's scores are done)
    KvStep<HD> b0, b1;
    int kk = k0;
    kv_load_k<HD>(b0, src, kk < k1 ? kk : -1);
    kv_load_v<HD>(b0, src, kk < k1 ? kk : -1);
    while (kk < k1) {
        kv_load_k<HD>(b1, src, kk + 32 < k1 ? kk + 32 : -1);
        attn_step<HD, QT>(S, b0, b1, src, kk, k1, p.P, T, sl2, g);
        kk += 32;
        if (kk >= k1) break;
        kv_load_k<HD>(b0, src, kk + 32 < k1 ? kk + 32 : -1);
        attn_step<HD, QT>(S, b1, b0, src, kk, k1, p.P, T, sl2, g);
        kk += 32;
    }

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
    if (wave != 0) return;

#pragma unroll
    for (int t = 0; t < QT; t++) {
        const int q = (qg * QT + t) * 16 + r16;
        if (q >= nq) continue;
        const int m = q / p.n_rep, r = q % p.n_rep;
        const int head = h * p.n_rep + r;
        if (p.nsplit == 1) {
            const float inv = 1.0f / Lt[t];
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) {
                const floatx4 y = S.o[t][dt] + sob[0][t][dt][lane];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int64_t k = (int64_t)head * HD + dt * 16 + 4 * g + i;
                    p.out16[(int64_t)m * p.out_ld + frag_index(k)] = f2h(y[i] * inv);
                }
            }
        } else {
            const int64_t pi = ((int64_t)s * p.n_heads + head) * p.M + m;
            float *po = p.part_o + pi * HD;
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) *(floatx4 *)(po + dt * 16 + 4 * g) = S.o[t][dt] + sob[0][t][dt][lane];
            if (g == 0) {
                p.part_ml[2 * pi] = Mt[t];
                p.part_ml[2 * pi + 1] = Lt[t];
            }
        }
    }
}

// ---- combine splits -> fp16 fragment-layout input of wo ----------------------
// grid (n_heads, M), block hd threads; splits are merged in index order.
__global__ __launch_bounds__(128) void k_attn_combine(AttnParams p) {
    const int head = blockIdx.x, m = blockIdx.y, d = threadIdx.x;
    const int HD = p.hd, ns = p.nsplit;
    const int64_t stride = (int64_t)p.n_heads * p.M;  // partial rows per split
    const int64_t pi0 = (int64_t)head * p.M + m;
    float mx = -INFINITY;
    for (int s = 0; s < ns; s++) mx = fmaxf(mx, p.part_ml[2 * (pi0 + s * stride)]);
    float L = 0.f, acc = 0.f;
#pragma unroll 4
    for (int s = 0; s < ns; s++) {
        const int64_t pi = pi0 + s * stride;
        const float ms = p.part_ml[2 * pi];
        const float f = ms == -INFINITY ? 0.f : exp2f(ms - mx);
        L += p.part_ml[2 * pi + 1] * f;
        acc += p.part_o[pi * HD + d] * f;
    }
    const int64_t k = (int64_t)head * HD + d;
    p.out16[(int64_t)m * p.out_ld + frag_index(k)] = f2h(acc / L);
}

// ---- host launchers ----------------------------------------------------------
void launch_rope_kv(const RopeKvParams &p, hipStream_t st) {
    hipLaunchKernelGGL(k_rope_kv, dim3(p.M, p.n_heads + p.n_kv), dim3(p.hd / 2), 0, st, p);
}

static int attn_target_splits(int n_kv) { return n_kv >= 64 ? 1 : 64 / n_kv; }

// Up to 16 rows (a linear verify or a decode step) the key ranges are a
// function of P alone, so each row's arithmetic is the same as in a one-row
// call.  Above, the splits shrink as query tiles grow, towards 2 resident
// waves per SIMD (512 workgroups of 4 waves).
AttnSplit attn_split(int P, int M, int n_kv, int n_rep) {
    const int target = attn_target_splits(n_kv);
    int want = target;
    if (M > 16) {
        const int nqt = (M * n_rep + 15) / 16;
        want = 512 / (n_kv * nqt);
        want = want < 1 ? 1 : want > target ? target : want;
    }
    int kpw = (P + 1 + 4 * want - 1) / (4 * want);
    kpw = kpw < 32 ? 32 : (kpw + 31) / 32 * 32;
    const int T = P + M;
    return AttnSplit{kpw, (T + 4 * kpw - 1) / (4 * kpw)};
}

// 4 * kpw >= (P + 1) / want, want <= target, and 4 * kpw >= 128 >= M, so
// nsplit = ceil((P + M) / (4 kpw)) <= target + 2
int attn_max_splits(int n_kv) { return attn_target_splits(n_kv) + 3; }

void launch_attention(const AttnParams &p, hipStream_t st) {
    if (p.keys_per_wave < 32 || p.keys_per_wave % 32) throw BackendError("attention: keys_per_wave");
    if ((int64_t)p.nsplit * 4 * p.keys_per_wave < (int64_t)p.P + p.M) throw BackendError("attention: splits too few");
    if (p.cap % 32 || (int64_t)p.P + p.M > p.cap) throw BackendError("attention: cache capacity");
    if (p.mask_words < 1 || p.mask_words > 2 || p.M > 64 * p.mask_words) throw BackendError("attention: mask words");
    // One query tile per wave keeps a wave within 256 registers (two
    // double-buffered 32-key operand sets and its accumulators), so two waves
    // share each SIMD.  Query tiles become workgroups along z; with the KV head
    // as blockIdx.x and n_kv a multiple of the 8 XCDs, every workgroup of one
    // head lands on the same XCD, so the query tiles re-read that head's keys
    // from its L2.
    const int nq = p.M * p.n_rep, nqt = (nq + 15) / 16;
    const dim3 grid(p.n_kv, p.nsplit, nqt);
    if (p.hd == 128) hipLaunchKernelGGL((k_attn<128, 1>), grid, dim3(256), 0, st, p);
    else if (p.hd == 64) hipLaunchKernelGGL((k_attn<64, 1>), grid, dim3(256), 0, st, p);
    else throw BackendError("attention: head_dim must be 64 or 128");
    if (p.nsplit > 1) hipLaunchKernelGGL(k_attn_combine, dim3(p.n_heads, p.M), dim3(p.hd), 0, st, p);
}

}  // namespace sd
