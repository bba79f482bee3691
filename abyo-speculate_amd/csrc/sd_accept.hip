// K4 (sampling half): rejection-sampling acceptance on the device, over the
// logits rows a verify pass left in HBM.
//
// Restates, per consulted row:
//  * softmax_with_temperature (crates/speculate/src/sampling/tokens.rs:15-55):
//    T = 0 -> one-hot at the first max; else exp((l - max) * (1/T)) / sum;
//  * modified_rejection_step (methods/vanilla.rs:59-73): q <= 0 accepts, else
//    accept iff u <= min(1, p / q);
//  * adjusted_distribution (vanilla.rs:83-106): max(0, p - q) / sum, an error
//    when the sum is not positive and finite;
//  * sample_from_distribution (tokens.rs:99-120): the first index whose
//    running sum exceeds u * sum, the last index on drift;
//  * the verify walk of run_vanilla_sd (vanilla.rs:178-210): one uniform per
//    tested draft, one for the resample or the bonus, in that order.
//
// The walk runs over a draft tree given as a parent table; a chain is the
// reference's linear walk exactly.  For trees (a rule the reference does not
// have: run_eagle / run_eagle3 ignore the temperature, eagle.rs:739-740,
// eagle3.rs:789) the children of a node are tested in BFS order against the
// node's current distribution, and each rejection replaces that distribution
// by its adjusted distribution against the node's draft row before the next
// sibling is tested (multi-candidate speculative sampling); if no child is
// accepted the final token is drawn from the last adjusted distribution, and
// after a leaf from the leaf's own distribution.  Two sibling rules: with
// i.i.d. siblings (each drawn from q with replacement) the draft row q stays
// fixed; with siblings drawn without replacement from q (distinct tokens), q
// is zeroed at every rejected token and renormalised before the next sibling
// is tested (q_r(y) = q(y) / R_r off the rejected set, R_{r+1} = R_r - q(x_r)).
// Either rule leaves the committed token distributed as the target's when
// its precondition on the siblings holds; deterministic top-k siblings meet
// neither.
//
// Sums here are parallel (per-thread sequential chunks, then a fixed-order
// tree), so they can differ from the reference's sequential f32 sums in the
// last bits; a decision can only differ when u lies within a few ulps of a
// threshold.
#include "sd_common.hpp"
#include "sd_kernels_accept.hpp"

namespace sd {

#pragma clang fp contract(off)

// ---- per-row softmax statistics --------------------------------------------
// grid rows, block 1024.  Online (max, sum of exp((l - max) * inv_t)) per
// thread over a strided walk, merged in a fixed order.  Entries unreachable
// through the t2d map (t2d_inv[x] < 0) count as -inf (mask_target_logits,
// eagle3.rs:498-513).  Also the first-max argmax (greedy one-hot).
__global__ __launch_bounds__(1024) void k_row_stats(const float *logits, int64_t ld, int V, float inv_t,
                                                   const int *t2d_inv, float *row_m, float *row_s, int *row_am) {
    const int r = blockIdx.x, t = threadIdx.x;
    const float *row = logits + (int64_t)r * ld;
    float m = -INFINITY, s = 0.f, bv = -INFINITY;
    int bi = 0x7fffffff, bad = 0;
    for (int x = t; x < V; x += 1024) {
        float l = row[x];
        if (t2d_inv && t2d_inv[x] < 0) l = -INFINITY;
        // a NaN or +inf entry makes the reference's sum non-finite (an error there)
        if (l != l || l == INFINITY) bad = 1;
        if (l > bv) {  // strictly greater: first max per thread (x increases)
            bv = l;
            bi = x;
        }
        if (l > m) {
            s = s * expf((m - l) * inv_t) + 1.f;
            m = l;
        } else if (l > -INFINITY) {
            s += expf((l - m) * inv_t);
        }
    }
    __shared__ float sm[1024], ss[1024], sv[1024];
    __shared__ int si[1024];
    const bool any_bad = __syncthreads_or(bad) != 0;
    sm[t] = m;
    ss[t] = s;
    sv[t] = bv;
    si[t] = bi;
    __syncthreads();
    for (int o = 512; o > 0; o >>= 1) {
        if (t < o) {
            const float m1 = sm[t], m2 = sm[t + o];
            const float M = fmaxf(m1, m2);
            float S = 0.f;
            if (M > -INFINITY) {
                S = (m1 > -INFINITY ? ss[t] * expf((m1 - M) * inv_t) : 0.f) +
                    (m2 > -INFINITY ? ss[t + o] * expf((m2 - M) * inv_t) : 0.f);
            }
            sm[t] = M;
            ss[t] = S;
            const float v2 = sv[t + o];
            const int i2 = si[t + o];
            if (i2 != 0x7fffffff && (v2 > sv[t] || (v2 == sv[t] && i2 < si[t]) || si[t] == 0x7fffffff)) {
                sv[t] = v2;
                si[t] = i2;
            }
        }
        __syncthreads();
    }
    if (t == 0) {
        row_m[r] = sm[0];
        row_s[r] = any_bad ? NAN : ss[0];
        row_am[r] = si[0] == 0x7fffffff ? 0 : si[0];
    }
}

// ---- the walk ----------------------------------------------------------------
constexpr int WT = 1024;  // threads of the walk kernel
constexpr int MAX_REJ = 16;

struct WalkShared {
    float red[WT];
    float scan[WT];
    int first[WT];
    float Z[MAX_REJ];  // normalisers of the successive adjusted distributions at the current node
    float R[MAX_REJ];  // without replacement: the mass of q left before rejection r (R[0] = 1)
    int rej[MAX_REJ];  // without replacement: the rejected tokens at the current node
    int node, krej, used, plen, fin, status, go;
    float u;
};

// the draft probability of x (q0 = q(x)) that rejection r at the current
// node tests against: q itself for i.i.d. siblings; without replacement, 0 on
// the tokens rejected before r and q(x) / R_r elsewhere (0 once no mass is left)
__device__ __forceinline__ float walk_q(const AcceptParams &a, const WalkShared &W, float q0, int r, int x) {
    if (!a.wor) return q0;
    for (int i = 0; i < r; i++)
        if (W.rej[i] == x) return 0.f;
    return W.R[r] > 0.f ? q0 / W.R[r] : 0.f;
}

// probability of x at `node` after `krej` rejections there
__device__ __forceinline__ float walk_p(const AcceptParams &a, const WalkShared &W, int node, int krej, int x) {
    const float *row = a.logits + (int64_t)node * a.ld;
    float p;
    if (a.t2d_inv && a.t2d_inv[x] < 0) {
        p = 0.f;
    } else if (a.greedy) {
        p = x == a.row_am[node] ? 1.f : 0.f;
    } else {
        p = expf((row[x] - a.row_m[node]) * a.inv_t) / a.row_s[node];
    }
    if (krej > 0) {
        const int qr = a.q_row_of[node];
        const float q0 = accept_q(a, qr, x);
        for (int r = 0; r < krej; r++) p = fmaxf(p - walk_q(a, W, q0, r, x), 0.f) / W.Z[r];
    }
    return p;
}

// Sum over x of f(x) in a fixed order: thread t sums its contiguous chunk,
// then a fixed tree.  Leaves each thread's chunk sum in W.scan[t] when scan is
// set (an exclusive prefix over threads, for the CDF walk).
template <typename F>
__device__ float block_sum(WalkShared &W, int V, bool scan, F f) {
    const int t = threadIdx.x;
    const int chunk = (V + WT - 1) / WT;
    const int x0 = t * chunk, x1 = min(V, x0 + chunk);
    float s = 0.f;
    for (int x = x0; x < x1; x++) s += f(x);
    W.red[t] = s;
    if (scan) W.scan[t] = s;
    __syncthreads();
    for (int o = WT / 2; o > 0; o >>= 1) {
        if (t < o) W.red[t] = W.red[t] + W.red[t + o];
        __syncthreads();
    }
    const float total = W.red[0];
    if (scan) {
        // exclusive prefix over thread chunks, thread order (sequential by
        // one thread: 1024 adds, no reassociation across chunks)
        if (t == 0) {
            float acc = 0.f;
            for (int i = 0; i < WT; i++) {
                const float v = W.scan[i];
                W.scan[i] = acc;
                acc += v;
            }
        }
        __syncthreads();
    }
    __syncthreads();
    return total;
}

// grid 1, block 1024
__global__ __launch_bounds__(WT) void k_accept_walk(AcceptParams a) {
    __shared__ WalkShared W;
    const int t = threadIdx.x;
    if (t == 0) {
        W.node = 0;
        W.used = 0;
        W.plen = 1;
        W.fin = -1;
        W.status = ACC_OK;
        W.krej = 0;
        a.out_path[0] = 0;
    }
    __syncthreads();
    while (true) {
        // every thread has read the previous turn's W.go / W.node / W.krej
        // before thread 0 rewrites them
        __syncthreads();
        // ---- thread 0: test the children of the current node in BFS order ----
        if (t == 0) {
            W.go = 0;  // 0: descend done / 1: sample at node / 2: normaliser pass needed / 3: stop
            const int node = W.node;
            const float S = a.row_s[node];
            if (!a.greedy && (!(S > 0.f) || !isfinite(S))) {
                W.status = ACC_ERR_SOFTMAX;
                W.go = 3;
            } else if (a.max_commit > 0 && W.plen - 1 >= a.max_commit && W.krej == 0) {
                W.go = 3;  // budget reached after an accepted draft: no final token
            } else {
                int c = node + 1;
                int seen = 0;  // children already tested at this node (= krej)
                int accepted = -1;
                for (; c < a.n; c++) {
                    if (a.parents[c] != node) continue;
                    if (seen++ < W.krej) continue;
                    const float u = a.uniforms[W.used++];
                    const int tok = a.tokens[c];
                    const float p = walk_p(a, W, node, W.krej, tok);
                    if (W.krej == 0) W.R[0] = 1.f;
                    const float q = walk_q(a, W, accept_q(a, a.q_row_of[node], tok), W.krej, tok);
                    // modified_rejection_step (vanilla.rs:59-73)
                    const bool acc = q <= 0.f || u <= fminf(p / q, 1.f);
                    if (acc) {
                        accepted = c;
                        break;
                    }
                    W.go = 2;  // rejected: the adjusted distribution's normaliser is needed
                    if (W.krej < MAX_REJ) {
                        W.rej[W.krej] = tok;
                        if (W.krej + 1 < MAX_REJ) W.R[W.krej + 1] = W.R[W.krej] - accept_q(a, a.q_row_of[node], tok);
                    }
                    break;
                }
                if (accepted >= 0) {
                    a.out_path[W.plen++] = accepted;
                    W.node = accepted;
                    W.krej = 0;
                    W.go = 0;
                } else if (W.go != 2) {
                    W.go = 1;  // no child left to test (or a leaf): final draw
                    W.u = a.uniforms[W.used++];
                }
            }
        }
        __syncthreads();
        const int go = W.go;
        if (go == 0) continue;
        if (go == 3) break;
        const int node = W.node, krej = W.krej;
        if (go == 2) {
            // adjusted_distribution (vanilla.rs:83-106) of the current distribution
            if (krej >= MAX_REJ) {
                if (t == 0) W.status = ACC_ERR_ARG;
                break;
            }
            const int qr = a.q_row_of[node];
            const float Z = block_sum(W, a.V, false, [&](int x) {
                return fmaxf(walk_p(a, W, node, krej, x) - walk_q(a, W, accept_q(a, qr, x), krej, x), 0.f);
            });
            if (t == 0) {
                if (!(Z > 0.f) || !isfinite(Z)) {
                    W.status = ACC_ERR_ADJUSTED;
                } else {
                    W.Z[krej] = Z;
                    W.krej = krej + 1;
                }
            }
            __syncthreads();
            if (W.status != ACC_OK) break;
            continue;
        }
        // go == 1: sample_from_distribution (tokens.rs:99-120) over the current distribution
        const float sum = block_sum(W, a.V, true, [&](int x) { return walk_p(a, W, node, krej, x); });
        if (!(sum > 0.f) || !isfinite(sum)) {
            if (t == 0) W.status = ACC_ERR_SOFTMAX;
            break;
        }
        const float target = W.u * sum;
        {
            const int chunk = (a.V + WT - 1) / WT;
            const int x0 = t * chunk, x1 = min(a.V, x0 + chunk);
            float acc = W.scan[t];
            int hit = 0x7fffffff;
            for (int x = x0; x < x1; x++) {
                acc += walk_p(a, W, node, krej, x);
                if (target < acc) {
                    hit = x;
                    break;
                }
            }
            W.first[t] = hit;
            __syncthreads();
            for (int o = WT / 2; o > 0; o >>= 1) {
                if (t < o) W.first[t] = min(W.first[t], W.first[t + o]);
                __syncthreads();
            }
            if (t == 0) W.fin = W.first[0] == 0x7fffffff ? a.V - 1 : W.first[0];
        }
        break;
    }
    __syncthreads();
    if (t == 0) {
        a.out_info[0] = W.plen;
        a.out_info[1] = W.fin;
        a.out_info[2] = W.used;
        a.out_info[3] = W.status;
    }
}

void launch_row_stats(const float *logits, int64_t ld, int V, int rows, float inv_t, const int *t2d_inv, float *row_m,
                      float *row_s, int *row_am, hipStream_t st) {
    hipLaunchKernelGGL(k_row_stats, dim3(rows), dim3(1024), 0, st, logits, ld, V, inv_t, t2d_inv, row_m, row_s, row_am);
}

void launch_accept_walk(const AcceptParams &a, hipStream_t st) {
    hipLaunchKernelGGL(k_accept_walk, dim3(1), dim3(WT), 0, st, a);
}

}  // namespace sd
