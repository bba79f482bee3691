// K2: RoPE + KV append + tree-masked GQA attention over the fp16 KV cache.
//
// Replaces LayerWeights::{rope_at, rope_at_positions, run_attn}
// (crates/speculate/src/model/quantized_llama_local.rs:94-136; Qwen2 half
// rotation at quantized_qwen2_local.rs:98-109) and the additive masks of
// causal_bias (:332-350) / DraftTree::full_attention_bias (tree.rs:220-264).
//
// KV layout per layer: K[n_kv][cap][hd], V[n_kv][cap][hd] fp16.  The M new
// rows are written in place at [P, P+M) (no cat, no repeat_kv copies).
// Visibility: key j < P is visible to every query; key P+t is visible to
// query token i iff bit t of mask[i] is set (ancestor-or-self for trees,
// t <= i for a causal chain).
//
// Attention runs as split flash-decoding.  A workgroup owns one KV head, one
// contiguous range of 64-key chunks (a split) and up to 256 queries (the
// n_rep query heads of the group times the M tokens).  Scores are computed
// transposed, S^T = K Q^T, so the MFMA result layout is directly the B
// operand of O^T = V^T P^T.  Split boundaries depend only on P, so a query's
// result does not depend on how many other queries share the call.
#include "sd_common.hpp"
#include "sd_kernels_attn.hpp"

namespace sd {

#pragma clang fp contract(off)

// ---- RoPE + KV append ------------------------------------------------------
// grid (M, n_heads + n_kv), block hd/2 threads
__global__ void k_rope_kv(RopeKvParams p) {
    const int m = blockIdx.x, hh = blockIdx.y, i = threadIdx.x;
    const int half = p.hd / 2;
    if (i >= half) return;
    const int pos = p.pos[m];
    const float c = p.cos_t[(int64_t)pos * half + i], s = p.sin_t[(int64_t)pos * half + i];
    const float *row = p.qkv + (int64_t)m * p.ld_qkv;
    int a, b;  // element pair
    if (p.interleaved) {
        a = 2 * i;
        b = 2 * i + 1;
    } else {
        a = i;
        b = i + half;
    }
    if (hh < p.n_heads) {
        const float *x = row + hh * p.hd;
        const float x0 = x[a], x1 = x[b];
        uint16_t *q = p.q16 + ((int64_t)hh * p.M + m) * p.hd;
        q[a] = f2h(x0 * c - x1 * s);
        q[b] = f2h(x0 * s + x1 * c);
    } else {
        const int h = hh - p.n_heads;
        const float *xk = row + p.n_heads * p.hd + h * p.hd;
        const float *xv = row + (p.n_heads + p.n_kv) * p.hd + h * p.hd;
        const int64_t dst = ((int64_t)h * p.cap + p.P + m) * p.hd;
        const float k0 = xk[a], k1 = xk[b];
        p.kc[dst + a] = f2h(k0 * c - k1 * s);
        p.kc[dst + b] = f2h(k0 * s + k1 * c);
        p.vc[dst + a] = f2h(xv[a]);
        p.vc[dst + b] = f2h(xv[b]);
    }
}

#pragma clang fp contract(fast)

// ---- flash-decode over one split --------------------------------------------
constexpr int QPW = 4;   // query tiles per wave
constexpr int KCH = 64;  // keys per chunk

template <int HD>
__global__ __launch_bounds__(256) void k_attn_split(AttnParams p) {
    const int h = blockIdx.x, s = blockIdx.y, qg = blockIdx.z;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r16 = lane & 15, g = lane >> 4;
    const int nq = p.M * p.n_rep;
    const int T = p.P + p.M;
    const int nchunks = (T + KCH - 1) / KCH;
    const int c0 = s * p.cps, c1 = min(c0 + p.cps, nchunks);
    constexpr int NDC = HD / 32, NDT = HD / 16;

    __shared__ uint16_t Ks[KCH][HD + 8];
    __shared__ uint16_t Vt[HD][KCH + 8];

    const uint16_t *kbase = p.kc + (int64_t)h * p.cap * HD;
    const uint16_t *vbase = p.vc + (int64_t)h * p.cap * HD;

    // this wave's query tiles
    int ntl = 0;
    int tq0[QPW];
#pragma unroll
    for (int t = 0; t < QPW; t++) {
        const int tile = qg * (4 * QPW) + wave + 4 * t;
        tq0[t] = tile * 16;
        if (tile * 16 < nq) ntl = t + 1;
    }

    half8 qf[QPW][NDC];
    floatx4 o[QPW][NDT];
    float mrun[QPW], lrun[QPW];
    int tok[QPW];
    bool qlive[QPW];
#pragma unroll
    for (int t = 0; t < QPW; t++) {
        const int q = tq0[t] + r16;
        qlive[t] = t < ntl && q < nq;
        const int m = qlive[t] ? q / p.n_rep : 0, r = qlive[t] ? q % p.n_rep : 0;
        tok[t] = m;
        const uint16_t *qr = p.q16 + ((int64_t)(h * p.n_rep + r) * p.M + m) * HD;
#pragma unroll
        for (int dc = 0; dc < NDC; dc++) {
            uintx4 v = {0u, 0u, 0u, 0u};
            if (qlive[t]) v = *(const uintx4 *)(qr + dc * 32 + g * 8);
            qf[t][dc] = __builtin_bit_cast(half8, v);
        }
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) o[t][dt] = floatx4{0.f, 0.f, 0.f, 0.f};
        mrun[t] = -INFINITY;
        lrun[t] = 0.f;
    }

    const float sl2 = p.scale * 1.4426950408889634f;  // scale * log2(e)

    for (int c = c0; c < c1; c++) {
        __syncthreads();
        // stage K (key-major) and V (dim-major) of keys [c*64, c*64+64)
        for (int piece = threadIdx.x; piece < KCH * HD / 8; piece += 256) {
            const int key = piece / (HD / 8), d8 = piece % (HD / 8);
            const int kg = c * KCH + key;
            uintx4 kv = {0u, 0u, 0u, 0u}, vv = {0u, 0u, 0u, 0u};
            if (kg < T) {
                kv = *(const uintx4 *)(kbase + (int64_t)kg * HD + d8 * 8);
                vv = *(const uintx4 *)(vbase + (int64_t)kg * HD + d8 * 8);
            }
            *(uintx4 *)&Ks[key][d8 * 8] = kv;
            const uint32_t vw[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                Vt[d8 * 8 + 2 * e][key] = (uint16_t)(vw[e] & 0xffff);
                Vt[d8 * 8 + 2 * e + 1][key] = (uint16_t)(vw[e] >> 16);
            }
        }
        __syncthreads();

#pragma unroll
        for (int t = 0; t < QPW; t++) {
            if (t >= ntl) break;
            // S^T tile: keys (4 x 16) x 16 queries
            floatx4 st[4];
#pragma unroll
            for (int kt = 0; kt < 4; kt++) {
                st[kt] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int dc = 0; dc < NDC; dc++) {
                    const half8 a = *(const half8 *)&Ks[kt * 16 + r16][dc * 32 + g * 8];
                    st[kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qf[t][dc], st[kt], 0, 0, 0);
                }
            }
            // scale + mask, column max
            float cm = -INFINITY;
#pragma unroll
            for (int kt = 0; kt < 4; kt++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int key = c * KCH + kt * 16 + 4 * g + i;
                    bool vis;
                    if (key < p.P) {
                        vis = true;
                    } else if (key < T) {
                        const int tt = key - p.P;
                        const uint64_t w = p.mask[(int64_t)tok[t] * p.mask_words + (tt >> 6)];
                        vis = (w >> (tt & 63)) & 1ull;
                    } else {
                        vis = false;
                    }
                    const float v = vis ? st[kt][i] * sl2 : -INFINITY;
                    st[kt][i] = v;
                    cm = fmaxf(cm, v);
                }
            cm = fmaxf(cm, __shfl_xor(cm, 16));
            cm = fmaxf(cm, __shfl_xor(cm, 32));
            const float mnew = fmaxf(mrun[t], cm);
            const float muse = mnew == -INFINITY ? 0.f : mnew;
            const float alpha = exp2f(mrun[t] - muse);
            float ps = 0.f;
            uint32_t pk[4][2];
#pragma unroll
            for (int kt = 0; kt < 4; kt++) {
                float e[4];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    e[i] = exp2f(st[kt][i] - muse);
                    ps += e[i];
                }
                pk[kt][0] = (uint32_t)f2h(e[0]) | ((uint32_t)f2h(e[1]) << 16);
                pk[kt][1] = (uint32_t)f2h(e[2]) | ((uint32_t)f2h(e[3]) << 16);
            }
            ps += __shfl_xor(ps, 16);
            ps += __shfl_xor(ps, 32);
            lrun[t] = lrun[t] * alpha + ps;
            mrun[t] = mnew;
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) o[t][dt] *= alpha;
            // O^T += V^T P^T over two 32-key groups
#pragma unroll
            for (int j = 0; j < 2; j++) {
                uintx4 bu = {pk[2 * j][0], pk[2 * j][1], pk[2 * j + 1][0], pk[2 * j + 1][1]};
                const half8 b = __builtin_bit_cast(half8, bu);
#pragma unroll
                for (int dt = 0; dt < NDT; dt++) {
                    const uint16_t *vr = &Vt[dt * 16 + r16][0];
                    const uint2 lo = *(const uint2 *)(vr + (2 * j) * 16 + 4 * g);
                    const uint2 hi = *(const uint2 *)(vr + (2 * j + 1) * 16 + 4 * g);
                    uintx4 au = {lo.x, lo.y, hi.x, hi.y};
                    o[t][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, au), b, o[t][dt],
                                                                      0, 0, 0);
                }
            }
        }
    }

    // partials: o [split][head][m][HD], ml [split][head][m][2]
#pragma unroll
    for (int t = 0; t < QPW; t++) {
        if (t >= ntl || !qlive[t]) continue;
        const int q = tq0[t] + r16;
        const int m = q / p.n_rep, r = q % p.n_rep;
        const int head = h * p.n_rep + r;
        const int64_t pi = ((int64_t)s * p.n_heads + head) * p.M + m;
        float *po = p.part_o + pi * HD;
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) *(floatx4 *)(po + dt * 16 + 4 * g) = o[t][dt];
        if (g == 0) {
            p.part_ml[2 * pi] = mrun[t];
            p.part_ml[2 * pi + 1] = lrun[t];
        }
    }
}

// ---- combine splits -> fp16 fragment-layout input of wo ----------------------
// grid (n_heads, M), block HD threads.  Every split's (m, l) and output are
// loaded before use (up to 64 splits in registers), so the combine costs one
// memory round trip.
constexpr int MAX_SPLITS = 64;
__global__ void k_attn_combine(AttnParams p, int nsplit) {
    const int head = blockIdx.x, m = blockIdx.y, d = threadIdx.x;
    const int HD = p.hd;
    float ms[MAX_SPLITS], ls[MAX_SPLITS], os[MAX_SPLITS];
#pragma unroll
    for (int s = 0; s < MAX_SPLITS; s++) {
        if (s < nsplit) {
            const int64_t pi = ((int64_t)s * p.n_heads + head) * p.M + m;
            ms[s] = p.part_ml[2 * pi];
            ls[s] = p.part_ml[2 * pi + 1];
            os[s] = p.part_o[pi * HD + d];
        }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int s = 0; s < MAX_SPLITS; s++)
        if (s < nsplit) mx = fmaxf(mx, ms[s]);
    float L = 0.f, acc = 0.f;
#pragma unroll
    for (int s = 0; s < MAX_SPLITS; s++) {
        if (s < nsplit && ms[s] != -INFINITY) {
            const float f = exp2f(ms[s] - mx);
            L += ls[s] * f;
            acc += os[s] * f;
        }
    }
    const float y = acc / L;
    const int64_t k = (int64_t)head * HD + d;
    p.out16[(int64_t)m * p.out_ld + frag_index(k)] = f2h(y);
}

// ---- host launchers ----------------------------------------------------------
void launch_rope_kv(const RopeKvParams &p, hipStream_t st) {
    hipLaunchKernelGGL(k_rope_kv, dim3(p.M, p.n_heads + p.n_kv), dim3(p.hd / 2), 0, st, p);
}

int attn_chunks_per_split(int P, int n_kv) {
    const int nch_p = (P + 1 + KCH - 1) / KCH;
    int target = 256 / (n_kv > 0 ? n_kv : 1);
    if (target > MAX_SPLITS - 3) target = MAX_SPLITS - 3;  // up to 3 more splits for <= 128 new rows
    if (target < 1) target = 1;
    if (target > nch_p) target = nch_p;
    return (nch_p + target - 1) / target;
}

int attn_num_splits(int P, int M, int cps) {
    const int nchunks = (P + M + KCH - 1) / KCH;
    return (nchunks + cps - 1) / cps;
}

void launch_attention(const AttnParams &p, hipStream_t st) {
    const int nsplit = attn_num_splits(p.P, p.M, p.cps);
    const int nq = p.M * p.n_rep;
    const int nqg = (nq + 16 * 4 * QPW - 1) / (16 * 4 * QPW);
    const dim3 grid(p.n_kv, nsplit, nqg);
    if (p.hd == 128) hipLaunchKernelGGL(k_attn_split<128>, grid, dim3(256), 0, st, p);
    else if (p.hd == 64) hipLaunchKernelGGL(k_attn_split<64>, grid, dim3(256), 0, st, p);
    else throw BackendError("attention: head_dim must be 64 or 128");
    if (nsplit > MAX_SPLITS) throw BackendError("attention: too many splits");
    hipLaunchKernelGGL(k_attn_combine, dim3(p.n_heads, p.M), dim3(p.hd), 0, st, p, nsplit);
}

}  // namespace sd
