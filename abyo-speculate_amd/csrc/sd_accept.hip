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
// The rows' softmax statistics and distributions, and every V-wide pass the
// walk can make (per node, the normaliser of each possible rejection and the
// final draw), are computed across the GPU; the walk, one workgroup, then
// takes the decisions from those sums and searches one tile for the draw.
// Sums here are parallel (fixed-order trees over slices, tiles and lanes), so
// they can differ from the reference's sequential f32 sums in the last bits;
// a decision can only differ when u lies within a few ulps of a threshold.
#include "sd_buffer.hpp"
#include "sd_common.hpp"
#include "sd_kernels_accept.hpp"

namespace sd {

#pragma clang fp contract(off)

// ---- per-row softmax statistics ----------------------------------------------
// grid (rows, slices of kSlice entries), block kRsT.  A slice's max M and sum
// of exp((l - M) * inv_t) (two workgroup reductions: the max first, then the
// sum relative to it); the slices' (max, sum) pairs are merged in slice order
// by the last workgroup of the row to finish (a per-row arrival count,
// device-scope partials).  Entries unreachable through the t2d map
// (t2d_inv[x] < 0) count as -inf (mask_target_logits, eagle3.rs:498-513).
// Also the first-max argmax (greedy one-hot).
constexpr int kRsT = 256, kSlice = 8192;

__device__ __forceinline__ uint64_t pack2(float a, uint32_t b) { return (uint64_t)__float_as_uint(a) | ((uint64_t)b << 32); }

// (m1, s1) + (m2, s2) of the online softmax sum
__device__ __forceinline__ void ms_merge(float &m1, float &s1, float m2, float s2, float inv_t) {
    const float M = fmaxf(m1, m2);
    float S = 0.f;
    if (M > -INFINITY)
        S = (m1 > -INFINITY ? s1 * expf((m1 - M) * inv_t) : 0.f) + (m2 > -INFINITY ? s2 * expf((m2 - M) * inv_t) : 0.f);
    m1 = M;
    s1 = S;
}
constexpr int kNoIdx = 0x7fffffff;
// the earlier of two first-max candidates
__device__ __forceinline__ void am_merge(float &v1, int &i1, float v2, int i2) {
    if (i2 != kNoIdx && (i1 == kNoIdx || v2 > v1 || (v2 == v1 && i2 < i1))) {
        v1 = v2;
        i1 = i2;
    }
}

// workgroup-wide reductions (kRsT threads = 4 waves): lanes by xor butterflies,
// then the 4 waves in order; every thread gets the result
__device__ __forceinline__ float wg_max(float v, float *sh) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
    __syncthreads();
    const float r = fmaxf(fmaxf(sh[0], sh[1]), fmaxf(sh[2], sh[3]));
    __syncthreads();
    return r;
}
__device__ __forceinline__ float wg_sum(float v, float *sh) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
    __syncthreads();
    const float r = (sh[0] + sh[1]) + (sh[2] + sh[3]);
    __syncthreads();
    return r;
}

__global__ __launch_bounds__(kRsT) void k_row_stats(const float *logits, int64_t ld, int V, float inv_t,
                                                   const int *t2d_inv, uint64_t *part, int *cnt, float *row_m,
                                                   float *row_s, int *row_am) {
    const int r = blockIdx.x, sl = blockIdx.y, nsl = gridDim.y, t = threadIdx.x;
    const float *row = logits + (int64_t)r * ld;
    const int x1 = min(V, (sl + 1) * kSlice);
    // the thread's kPer entries x = slice start + t + kRsT i, all requested at once
    constexpr int kPer = kSlice / kRsT;
    float lv[kPer];
#pragma unroll
    for (int i = 0; i < kPer; i++) {
        const int x = sl * kSlice + t + kRsT * i;
        lv[i] = x < x1 ? row[x] : -INFINITY;
        if (t2d_inv && x < x1 && t2d_inv[x] < 0) lv[i] = -INFINITY;
    }
    float bv = -INFINITY;
    int bi = kNoIdx, bad = 0;
#pragma unroll
    for (int i = 0; i < kPer; i++) {
        const float l = lv[i];
        // a NaN or +inf entry makes the reference's sum non-finite (an error there)
        if (l != l || l == INFINITY) bad = 1;
        if (l > bv) {  // strictly greater: first max per thread (x increases)
            bv = l;
            bi = sl * kSlice + t + kRsT * i;
        }
    }
    __shared__ float sh[4];
    __shared__ float sv[kRsT];
    __shared__ int si[kRsT];
    __shared__ int s_last;
    const bool any_bad = __syncthreads_or(bad) != 0;
    const float M = wg_max(bv, sh);
    float s = 0.f;
    if (M > -INFINITY) {
#pragma unroll
        for (int i = 0; i < kPer; i++)
            if (lv[i] > -INFINITY) s += expf((lv[i] - M) * inv_t);
    }
    const float S = wg_sum(s, sh);
    // first-max argmax: a fixed tree over the threads
    sv[t] = bv;
    si[t] = bi;
    __syncthreads();
    for (int o = kRsT / 2; o > 0; o >>= 1) {
        if (t < o) {
            float v1 = sv[t];
            int i1 = si[t];
            am_merge(v1, i1, sv[t + o], si[t + o]);
            sv[t] = v1;
            si[t] = i1;
        }
        __syncthreads();
    }
    if (t == 0) {
        uint64_t *pp = part + ((int64_t)r * nsl + sl) * 2;
        st_dev64(pp, pack2(M, __float_as_uint(any_bad ? NAN : S)));
        st_dev64(pp + 1, pack2(sv[0], (uint32_t)si[0]));
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the partials are stored before the count
        const int last = __hip_atomic_fetch_add(cnt + r, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == nsl - 1;
        if (last) __hip_atomic_store(cnt + r, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = last;
    }
    __syncthreads();
    if (!s_last) return;
    // the row's slices, in slice order
    __shared__ float pm[kRowStatsMaxSlices], ps[kRowStatsMaxSlices], pv[kRowStatsMaxSlices];
    __shared__ int pi[kRowStatsMaxSlices];
    if (t < nsl) {
        const uint64_t a = ld_dev64(part + ((int64_t)r * nsl + t) * 2);
        const uint64_t b = ld_dev64(part + ((int64_t)r * nsl + t) * 2 + 1);
        pm[t] = __uint_as_float((uint32_t)a);
        ps[t] = __uint_as_float((uint32_t)(a >> 32));
        pv[t] = __uint_as_float((uint32_t)b);
        pi[t] = (int)(uint32_t)(b >> 32);
    }
    __syncthreads();
    if (t == 0) {
        float Mr = pm[0], Sr = ps[0], v = pv[0];
        int i = pi[0];
        bool nan = Sr != Sr;
        for (int k = 1; k < nsl; k++) {
            nan = nan || ps[k] != ps[k];
            ms_merge(Mr, Sr, pm[k], ps[k], inv_t);
            am_merge(v, i, pv[k], pi[k]);
        }
        row_m[r] = Mr;
        row_s[r] = nan ? NAN : Sr;
        row_am[r] = i == kNoIdx ? 0 : i;
    }
}

// ---- the walk ----------------------------------------------------------------
constexpr int WT = 1024;       // threads of the walk kernel (16 waves)
constexpr int kTile = 256;     // entries per tile: lane l of a wave holds x = 256 tile + l + 64 j, j < 4
constexpr int kMaxTiles = 1024;  // vocabularies up to 262144
constexpr int MAX_REJ = kAcceptMaxChildren;

constexpr int kMaxNodes = 256;
struct WalkShared {
    // the tree and its per-node inputs, staged once: the walk's serial part
    // (thread 0) then reads LDS instead of waiting on memory for each node
    int par[kMaxNodes], tok[kMaxNodes], qrow[kMaxNodes];
    float uni[kMaxNodes], rs[kMaxNodes];
    float tsum[kMaxTiles];  // per-tile sums of the last pass
    float total;
    float Z[MAX_REJ];  // normalisers of the successive adjusted distributions at the current node
    float R[MAX_REJ];  // without replacement: the mass of q left before rejection r (R[0] = 1)
    int rej[MAX_REJ];  // without replacement: the rejected tokens at the current node
    // the current node's precomputed values: per k, the pass total (the
    // normaliser of rejection k, or the final draw's sum at k = its children)
    // and the test of child k (p, q and the raw draft probability q0)
    float nz[MAX_REJ + 1], np[MAX_REJ], nq[MAX_REJ], nq0[MAX_REJ];
    int node, krej, used, plen, fin, status, go;
    float u;
};

// The rejection state at the current node: the normalisers Z of the adjusted
// distributions so far and, without replacement, the rejected tokens and the
// mass R of q left before each rejection (R[0] = 1).  Held by the walk
// (WalkShared) and by the precomputation of a node's passes (RejState).
struct RejState {
    float Z[MAX_REJ], R[MAX_REJ];
    int rej[MAX_REJ];
};

// the draft probability of x (q0 = q(x)) that rejection r at the current
// node tests against: q itself for i.i.d. siblings; without replacement, 0 on
// the tokens rejected before r and q(x) / R_r elsewhere (0 once no mass is left)
template <typename St>
__device__ __forceinline__ float walk_q(const AcceptParams &a, const St &W, float q0, int r, int x) {
    if (!a.wor) return q0;
    for (int i = 0; i < r; i++)
        if (W.rej[i] == x) return 0.f;
    return W.R[r] > 0.f ? q0 / W.R[r] : 0.f;
}

// probability of x after `krej` rejections at a node whose distribution is p0
// (its prob row's entry) and whose draft row holds q0 = q(x)
template <typename St>
__device__ __forceinline__ float walk_val(const AcceptParams &a, const St &W, int krej, float p0, float q0, int x) {
    float p = p0;
    for (int r = 0; r < krej; r++) p = fmaxf(p - walk_q(a, W, q0, r, x), 0.f) / W.Z[r];
    return p;
}
// the normaliser term of the adjusted distribution after rejection krej
template <typename St>
__device__ __forceinline__ float walk_adj(const AcceptParams &a, const St &W, int krej, float p0, float q0, int x) {
    return fmaxf(walk_val(a, W, krej, p0, q0, x) - walk_q(a, W, q0, krej, x), 0.f);
}
__device__ __forceinline__ float walk_p(const AcceptParams &a, const WalkShared &W, int node, int krej, int x) {
    const float p0 = a.prob[(int64_t)node * a.V + x];
    return walk_val(a, W, krej, p0, krej > 0 ? accept_q(a, W.qrow[node], x) : 0.f, x);
}

// a wave's 64 values summed in a fixed order, lane 0's result
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return __shfl(v, 0);
}
// inclusive prefix over the wave's lanes
__device__ __forceinline__ float wave_scan(float v) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const float y = __shfl_up(v, o);
        if (lane >= o) v += y;
    }
    return v;
}

// Tiles of 256 entries (lane l of a wave holds x = 256 tile + l + 64 j,
// j < 4); kBatch tiles' entries are requested by a wave before it computes
// any (clamped into the row, so that every load is issued unconditionally).
constexpr int kBatch = 6;

// sample_from_distribution's search (tokens.rs:99-120) over the tile sums of
// the same f in W.tsum, by wave 0: the first x with f(x) > 0 whose running sum exceeds
// target, the running sum taken over the tiles' sums and then entry by entry
// inside a tile; -1 when none does (the reference's drift case).
template <typename F> __device__ __forceinline__ int walk_search(const WalkShared &W, int V, float target, F f) {
    const int lane = threadIdx.x & 63;
    const int ntiles = (V + kTile - 1) / kTile;
    const int per = (ntiles + 63) / 64;
    const int t0 = min(ntiles, lane * per), t1 = min(ntiles, t0 + per);
    float ls = 0.f;
    for (int tl = t0; tl < t1; tl++) ls += W.tsum[tl];
    const float incl = wave_scan(ls);
    float acc = __shfl_up(incl, 1);
    if (lane == 0) acc = 0.f;
    // the lane whose tile range crosses the target: the tile and the sum before it
    int tile = -1;
    float before = 0.f;
    for (int tl = t0; tl < t1; tl++) {
        const float nx = acc + W.tsum[tl];
        if (target < nx) {
            tile = tl;
            before = acc;
            break;
        }
        acc = nx;
    }
    const uint64_t hit = __builtin_amdgcn_ballot_w64(tile >= 0);
    if (hit == 0) return -1;
    const int src = __builtin_ctzll(hit);
    tile = __shfl(tile, src);
    float c = __shfl(before, src);
    // entry by entry from that tile on (past it only when rounding moved the crossing)
    for (int tl = tile; tl < ntiles; tl++) {
#pragma unroll 1
        for (int j = 0; j < 4; j++) {
            const int x = tl * kTile + 64 * j + lane;
            const float v = x < V ? f(x) : 0.f;
            const float inc = wave_scan(v);
            const uint64_t b = __builtin_amdgcn_ballot_w64(v > 0.f && target < c + inc);
            if (b) return tl * kTile + 64 * j + __builtin_ctzll(b);
            c = c + __shfl(inc, 63);
        }
    }
    return -1;
}

// ---- every pass of the walk, precomputed across the GPU ---------------------------
// Children are tested in BFS order, so the r-th rejection at node n is always
// that of n's r-th child, and the distribution after k rejections (k <= c_n,
// the number of children) depends on the node and k alone.  Launch k
// (k = 0 .. max c_n, over the nodes with c_n >= k) computes, for a node with
// k < c_n, the tile sums of the adjusted distribution's terms after k
// rejections (walk_adj: the normaliser pass of rejection k), and for a node
// with k == c_n the tile sums of its distribution after all c_n rejections
// (walk_val: the final draw; for a leaf, p itself) -- the walk's only
// possible passes, in its arithmetic and order: a lane's 4 entries of a tile
// in order, then wave_sum.  The Z of rejections i < k are launch i's tile
// sums totalled as walk_load_tiles totals them.  Workgroup 0 of a node also
// evaluates the test of child k exactly as the walk would (walk_p, walk_q).
// Launch 0 also writes the rows as distributions (softmax_with_temperature,
// tokens.rs:15-55; 0 where the t2d map masks x; at T = 0 the one-hot of the
// first max) from the logits and the row statistics.
// grid (participating nodes, tile groups), block kLtT.
// softmax_with_temperature's value at x of row r from its logit (the row's
// statistics from k_row_stats): 0 where the t2d map masks x, the one-hot of
// the first max at T = 0
__device__ __forceinline__ float row_prob_at(const AcceptParams &a, int r, int x, float logit, bool masked) {
    if (masked) return 0.f;
    if (a.greedy) return x == a.row_am[r] ? 1.f : 0.f;
    return expf((logit - a.row_m[r]) * a.inv_t) / a.row_s[r];
}

constexpr int kLtT = 256;
template <bool FIRST>
__global__ __launch_bounds__(kLtT) void k_tree_tiles(AcceptParams a, int k, const int *recs) {
    warm_kernargs<sizeof(AcceptParams)>();
    // the node's record (kTreeRec ints): node, children, draft row of its
    // children, and child k's token, its draft-row index (-1: none) and
    // whether the t2d map masks it
    const int *rec = recs + (int64_t)blockIdx.x * kTreeRec;
    const int r = rec[0], c = rec[1], qr = rec[2], tk = rec[3], dk = rec[4], mk_t = rec[5];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int V = a.V, n = a.n, ntiles = (V + kTile - 1) / kTile;
    const bool zpass = k < c;
    const bool need_q = zpass || k > 0;
    float *prow = a.prob + (int64_t)r * V;
    const float *qrow = need_q ? a.q + (int64_t)(qr < 0 ? 0 : qr) * a.q_ld : nullptr;
    const int tb = ((int)blockIdx.y * (kLtT / 64) + wave) * kBatch;
    // Every load that depends on nothing loaded here is issued first, in this
    // order: the rejection state (tile sums of rejection i = wave, the
    // rejected children's tokens and draft probabilities), the inputs of child
    // k's test, the entries (p or the logits, the mask, the map or q); then the
    // gathers through the map.
    const bool zi = wave < k;
    float zv[kMaxTiles / 64];
    {
        const float *zt = a.tiles + ((int64_t)(zi ? wave : 0) * n + r) * ntiles;
#pragma unroll
        for (int m2 = 0; m2 < kMaxTiles / 64; m2++) zv[m2] = zi ? zt[min(lane + 64 * m2, ntiles - 1)] : 0.f;
    }
    int s_tok = 0;
    float s_q0 = 0.f;
    if (wave == 0 && lane < k) {
        s_tok = a.kids[r * kAcceptMaxChildren + lane];
        s_q0 = a.test[((int64_t)lane * n + r) * 3 + 2];  // launch lane's test of child lane
    }
    const bool tester = blockIdx.y == 0 && threadIdx.x == 0 && zpass;
    float t_raw = 0.f, t_q0 = 0.f;
    if (tester) {
        t_raw = FIRST ? a.logits[(int64_t)r * a.logits_ld + tk] : prow[tk];
        t_q0 = dk < 0 ? 0.f : a.q[(int64_t)qr * a.q_ld + dk];
    }
    float p0[kBatch][4], q0[kBatch][4], mk[kBatch][4];
    int d[kBatch][4];
#pragma unroll
    for (int b = 0; b < kBatch; b++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int x = min((tb + b) * kTile + lane + 64 * j, V - 1);
            if constexpr (FIRST) {
                p0[b][j] = a.logits[(int64_t)r * a.logits_ld + x];
                mk[b][j] = a.t2d_inv ? (float)a.t2d_inv[x] : 0.f;  // < 0: masked
            } else {
                p0[b][j] = prow[x];
            }
            q0[b][j] = 0.f;
            if (need_q) {
                if (a.q_map) d[b][j] = a.q_map[x];
                else q0[b][j] = qrow[x];
            }
        }
    if (need_q && a.q_map) {
#pragma unroll
        for (int b = 0; b < kBatch; b++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float v = qrow[d[b][j] < 0 ? 0 : d[b][j]];
                q0[b][j] = d[b][j] < 0 ? 0.f : v;
            }
    }
    // the rejection state, one shared copy: Z of rejection i = wave totalled
    // as walk_load_tiles totals a pass (rejections past the wave count, which
    // needs more than 4 children, in further rounds), R[0] = 1 and
    // R[i + 1] = R[i] - q0(child i) as the walk updates it
    __shared__ RejState S;
    __shared__ float s_q[MAX_REJ];
    auto zsum = [&](const float (&v)[kMaxTiles / 64]) {
        float sz = 0.f;
#pragma unroll
        for (int m2 = 0; m2 < kMaxTiles / 64; m2++)
            if (lane + 64 * m2 < ntiles) sz += v[m2];
        return wave_sum(sz);
    };
    if (zi) {
        const float z = zsum(zv);
        if (lane == 0) S.Z[wave] = z;
    }
    for (int i = wave + kLtT / 64; i < k; i += kLtT / 64) {
        const float *zt = a.tiles + ((int64_t)i * n + r) * ntiles;
#pragma unroll
        for (int m2 = 0; m2 < kMaxTiles / 64; m2++) zv[m2] = zt[min(lane + 64 * m2, ntiles - 1)];
        const float z = zsum(zv);
        if (lane == 0) S.Z[i] = z;
    }
    if (wave == 0 && lane < k) {
        S.rej[lane] = s_tok;
        s_q[lane] = s_q0;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float Rr = 1.f;
        for (int i = 0; i <= k && i < MAX_REJ; i++) {
            S.R[i] = Rr;
            if (i < k) Rr = Rr - s_q[i];
        }
    }
    __syncthreads();
    if constexpr (FIRST) {
        // softmax_with_temperature's values, written for the later launches and the walk
#pragma unroll
        for (int b = 0; b < kBatch; b++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int x = (tb + b) * kTile + lane + 64 * j;
                const float pv = row_prob_at(a, r, x, p0[b][j], mk[b][j] < 0.f);
                p0[b][j] = pv;
                if (x < V) prow[x] = pv;
            }
    }
    // the test of child k: walk_p and walk_q at its token, as the walk evaluates them
    if (tester) {
        float *te = a.test + ((int64_t)k * n + r) * 3;
        const float pt = FIRST ? row_prob_at(a, r, tk, t_raw, mk_t != 0) : t_raw;
        te[0] = walk_val(a, S, k, pt, k > 0 ? t_q0 : 0.f, tk);
        te[1] = walk_q(a, S, t_q0, k, tk);
        te[2] = t_q0;
    }
    float *out = a.tiles + ((int64_t)k * n + r) * ntiles;
#pragma unroll
    for (int b = 0; b < kBatch; b++) {
        const int tl = tb + b;
        if (tl >= ntiles) break;
        float sum = 0.f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int x = tl * kTile + lane + 64 * j;
            const float v = zpass ? walk_adj(a, S, k, p0[b][j], q0[b][j], x) : walk_val(a, S, k, p0[b][j], q0[b][j], x);
            sum += x < V ? v : 0.f;
        }
        sum = wave_sum(sum);
        if (lane == 0) out[tl] = sum;
    }
}

// a row of precomputed tile sums into W.tsum and its total: wave 0 adds tiles
// lane, lane + 64, ... per lane, then the lanes (wave_sum)
__device__ __forceinline__ float walk_load_tiles(WalkShared &W, const float *src, int ntiles) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int tl = threadIdx.x; tl < ntiles; tl += WT) W.tsum[tl] = src[tl];
    __syncthreads();
    if (wave == 0) {
        float s = 0.f;
        for (int tl = lane; tl < ntiles; tl += 64) s += W.tsum[tl];
        s = wave_sum(s);
        if (lane == 0) W.total = s;
    }
    __syncthreads();
    return W.total;
}

// grid 1, block 1024.  The decisions read the precomputed values of the
// current node (staged into LDS when the walk arrives there), so thread 0
// tests a node's children without a memory round trip per child; the final
// draw loads the chosen pass's tile sums and searches one tile.
__global__ __launch_bounds__(WT) void k_accept_walk(AcceptParams a) {
    warm_kernargs<sizeof(AcceptParams)>();
    __shared__ WalkShared W;
    const int t = threadIdx.x;
    const int n = a.n;
    for (int i = t; i < n; i += WT) {
        W.par[i] = a.parents[i];
        W.tok[i] = a.tokens[i];
        W.qrow[i] = a.q_row_of[i];
        W.uni[i] = a.uniforms[i];
        W.rs[i] = a.row_s[i];
    }
    if (t == 0) {
        W.node = 0;
        W.used = 0;
        W.plen = 1;
        W.fin = -1;
        W.status = ACC_OK;
        W.krej = 0;
        a.out_path[0] = 0;
    }
    bool draw = false;
    while (true) {
        // stage the current node's pass totals and child tests
        __syncthreads();
        {
            const int node = W.node, c = a.nchild[node];
            const int wave = t >> 6, lane = t & 63, ntl = (a.V + kTile - 1) / kTile;
            if (t < c) {
                const float *te = a.test + ((int64_t)t * n + node) * 3;
                W.np[t] = te[0];
                W.nq[t] = te[1];
                W.nq0[t] = te[2];
            }
            // wave w totals pass k = w's tile sums (k <= c) as walk_load_tiles does
            for (int kk = wave; kk <= c; kk += WT / 64) {
                const float *zt = a.tiles + ((int64_t)kk * n + node) * ntl;
                float zv[kMaxTiles / 64];
#pragma unroll
                for (int m2 = 0; m2 < kMaxTiles / 64; m2++) zv[m2] = zt[min(lane + 64 * m2, ntl - 1)];
                float sz = 0.f;
#pragma unroll
                for (int m2 = 0; m2 < kMaxTiles / 64; m2++)
                    if (lane + 64 * m2 < ntl) sz += zv[m2];
                sz = wave_sum(sz);
                if (lane == 0) W.nz[kk] = sz;
            }
        }
        __syncthreads();
        // ---- thread 0: test the children of the current node in BFS order ----
        if (t == 0) {
            W.go = 3;  // 0: descend / 1: final draw at the node / 3: stop
            const int node = W.node;
            const float S = W.rs[node];
            if (!a.greedy && (!(S > 0.f) || !isfinite(S))) {
                W.status = ACC_ERR_SOFTMAX;
            } else if (a.max_commit > 0 && W.plen - 1 >= a.max_commit) {
                // budget reached after an accepted draft: no final token
            } else {
                W.R[0] = 1.f;
                int accepted = -1, krej = 0;
                for (int ch = node + 1; ch < n; ch++) {
                    if (W.par[ch] != node) continue;
                    const float u = W.uni[W.used++];
                    const float p = W.np[krej], q = W.nq[krej];
                    // modified_rejection_step (vanilla.rs:59-73)
                    if (q <= 0.f || u <= fminf(p / q, 1.f)) {
                        accepted = ch;
                        break;
                    }
                    // rejected: the adjusted distribution's normaliser (vanilla.rs:83-106)
                    const float Z = W.nz[krej];
                    if (!(Z > 0.f) || !isfinite(Z)) {
                        W.status = ACC_ERR_ADJUSTED;
                        break;
                    }
                    W.Z[krej] = Z;
                    W.rej[krej] = W.tok[ch];
                    if (krej + 1 < MAX_REJ) W.R[krej + 1] = W.R[krej] - W.nq0[krej];
                    krej++;
                }
                W.krej = krej;
                if (W.status == ACC_OK) {
                    if (accepted >= 0) {
                        a.out_path[W.plen++] = accepted;
                        W.node = accepted;
                        W.go = 0;
                    } else {
                        W.go = 1;  // no child left to test (or a leaf): final draw
                        W.u = W.uni[W.used++];
                    }
                }
            }
        }
        __syncthreads();
        const int go = W.go;
        if (go == 0) continue;
        draw = go == 1;
        break;
    }
    if (draw) {
        // sample_from_distribution (tokens.rs:99-120) over the distribution
        // after all of the node's children were rejected (a leaf's p itself)
        const int node = W.node, krej = W.krej;
        const int ntl = (a.V + kTile - 1) / kTile;
        const float sum = walk_load_tiles(W, a.tiles + ((int64_t)krej * n + node) * ntl, ntl);
        if (!(sum > 0.f) || !isfinite(sum)) {
            if (t == 0) W.status = ACC_ERR_SOFTMAX;
        } else if (t < 64) {
            auto f = [&](int x) { return walk_p(a, W, node, krej, x); };
            const int x = walk_search(W, a.V, W.u * sum, f);
            if (t == 0) W.fin = x < 0 ? a.V - 1 : x;
        }
    }
    __syncthreads();
    if (t == 0) {
        a.out_info[0] = W.plen;
        a.out_info[1] = W.fin;
        a.out_info[2] = W.used;
        a.out_info[3] = W.status;
    }
}

void launch_row_stats(const float *logits, int64_t ld, int V, int rows, float inv_t, const int *t2d_inv, uint64_t *part,
                      int *cnt, float *row_m, float *row_s, int *row_am, hipStream_t st) {
    if (V < 1 || V > kRowStatsMaxSlices * kSlice) throw BackendError("acceptance: vocabulary too large");
    const dim3 grid(rows, (V + kSlice - 1) / kSlice);
    hipLaunchKernelGGL(k_row_stats, grid, dim3(kRsT), 0, st, logits, ld, V, inv_t, t2d_inv, part, cnt, row_m, row_s,
                       row_am);
}

size_t tree_tiles_floats(int n, int V, int kmax) {
    // tile sums, child tests
    return (size_t)(kmax + 1) * n * ((V + kTile - 1) / kTile) + (size_t)3 * (kmax + 1) * n;
}

void launch_tree_tiles(const AcceptParams &a, int kmax, const int *const *recs, const int *counts, hipStream_t st) {
    if (a.V > kMaxTiles * kTile) throw BackendError("acceptance: vocabulary too large");
    if (a.n < 1 || a.n > kMaxNodes) throw BackendError("acceptance: too many tree nodes");
    if (kmax < 0 || kmax > MAX_REJ) throw BackendError("acceptance: too many children for the precomputed passes");
    if (!a.tiles || !a.test || !a.nchild || !a.kids || !a.logits || !a.prob) throw BackendError("acceptance: pass buffers");
    if (counts[0] != a.n) throw BackendError("acceptance: the first pass covers every node");
    const int ntiles = (a.V + kTile - 1) / kTile, per = (kLtT / 64) * kBatch;
    const unsigned groups = (unsigned)((ntiles + per - 1) / per);
    hipLaunchKernelGGL(k_tree_tiles<true>, dim3(a.n, groups), dim3(kLtT), 0, st, a, 0, recs[0]);
    for (int k = 1; k <= kmax; k++)
        if (counts[k] > 0)
            hipLaunchKernelGGL(k_tree_tiles<false>, dim3(counts[k], groups), dim3(kLtT), 0, st, a, k, recs[k]);
}

void launch_accept_walk(const AcceptParams &a, hipStream_t st) {
    if (a.V > kMaxTiles * kTile) throw BackendError("acceptance: vocabulary too large");
    if (!a.tiles || !a.test || !a.nchild) throw BackendError("acceptance: the walk reads the passes of launch_tree_tiles");
    if (a.n < 1 || a.n > kMaxNodes) throw BackendError("acceptance: too many tree nodes");
    hipLaunchKernelGGL(k_accept_walk, dim3(1), dim3(WT), 0, st, a);
}

}  // namespace sd
