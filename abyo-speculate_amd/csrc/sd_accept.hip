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
// The rows' softmax statistics and distributions are computed across the
// GPU; the walk, one workgroup, then reads the distributions.  Sums here are
// parallel (fixed-order trees over slices, tiles and lanes), so they can
// differ from the reference's sequential f32 sums in the last bits; a
// decision can only differ when u lies within a few ulps of a threshold.
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

__device__ __forceinline__ void st_dev64(void *p, uint64_t v) {
    __hip_atomic_store((uint64_t *)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_dev64(const void *p) {
    return __hip_atomic_load((const uint64_t *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
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

// ---- the rows as distributions ----------------------------------------------
// grid (rows, slices), block kRsT: prob[r][x] = softmax_with_temperature's
// value (tokens.rs:15-55), 0 where the t2d map masks x; at T = 0 the one-hot
// of the first max.
__global__ __launch_bounds__(kRsT) void k_row_prob(const float *logits, int64_t ld, int V, float inv_t, int greedy,
                                                  const int *t2d_inv, const float *row_m, const float *row_s,
                                                  const int *row_am, float *prob) {
    const int r = blockIdx.x, sl = blockIdx.y;
    const float *row = logits + (int64_t)r * ld;
    float *out = prob + (int64_t)r * V;
    const float m = row_m[r], S = row_s[r];
    const int am = row_am[r];
    const int x1 = min(V, (sl + 1) * kSlice);
    constexpr int kPer = kSlice / kRsT;
    float lv[kPer];
    bool live[kPer];
#pragma unroll
    for (int i = 0; i < kPer; i++) {
        const int x = sl * kSlice + threadIdx.x + kRsT * i;
        live[i] = x < x1 && !(t2d_inv && t2d_inv[x] < 0);
        lv[i] = live[i] && !greedy ? row[x] : 0.f;
    }
#pragma unroll
    for (int i = 0; i < kPer; i++) {
        const int x = sl * kSlice + threadIdx.x + kRsT * i;
        if (x >= x1) break;
        float p;
        if (!live[i]) p = 0.f;
        else if (greedy) p = x == am ? 1.f : 0.f;
        else p = expf((lv[i] - m) * inv_t) / S;
        out[x] = p;
    }
}

// ---- the walk ----------------------------------------------------------------
constexpr int WT = 1024;       // threads of the walk kernel (16 waves)
constexpr int kTile = 256;     // entries per tile: lane l of a wave holds x = 256 tile + l + 64 j, j < 4
constexpr int kMaxTiles = 1024;  // vocabularies up to 262144
constexpr int MAX_REJ = 16;

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

// probability of x after `krej` rejections at a node whose distribution is p0
// (its prob row's entry) and whose draft row holds q0 = q(x)
__device__ __forceinline__ float walk_val(const AcceptParams &a, const WalkShared &W, int krej, float p0, float q0,
                                          int x) {
    float p = p0;
    for (int r = 0; r < krej; r++) p = fmaxf(p - walk_q(a, W, q0, r, x), 0.f) / W.Z[r];
    return p;
}
// the normaliser term of the adjusted distribution after rejection krej
__device__ __forceinline__ float walk_adj(const AcceptParams &a, const WalkShared &W, int krej, float p0, float q0,
                                          int x) {
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

// Sum over x < V of the walk's values at `node` in a fixed order: tiles of
// 256 entries (wave w takes tiles w, w + 16, ...; a lane its 4 entries in
// order, then the wave's lanes), then the tiles.  ZPASS: the adjusted
// distribution's unnormalised terms (walk_adj), else the current
// distribution (walk_val).  QM: how q(x) is read -- 0 not at all, 1 from a
// target-vocabulary row, 2 through the t2d map.  Each wave requests kBatch
// tiles' entries (clamped into the row, so that every load is issued
// unconditionally) before it computes any of them.  Leaves the tile sums in
// W.tsum for walk_search.
constexpr int kBatch = 6;
template <bool ZPASS, int QM>
__device__ __forceinline__ void walk_tiles(WalkShared &W, const AcceptParams &a, int node, int krej) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int V = a.V, ntiles = (V + kTile - 1) / kTile;
    const float *prow = a.prob + (int64_t)node * V;
    const int qr = W.qrow[node];
    const float *qrow = QM ? a.q + (int64_t)(qr < 0 ? 0 : qr) * a.q_ld : nullptr;
    for (int tb = wave; tb < ntiles; tb += (WT / 64) * kBatch) {
        float p0[kBatch][4], q0[kBatch][4];
        int d[kBatch][4];
#pragma unroll
        for (int b = 0; b < kBatch; b++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int x = min((tb + (WT / 64) * b) * kTile + lane + 64 * j, V - 1);
                p0[b][j] = prow[x];
                if constexpr (QM == 1) q0[b][j] = qrow[x];
                if constexpr (QM == 2) d[b][j] = a.q_map[x];
            }
        if constexpr (QM == 2) {
#pragma unroll
            for (int b = 0; b < kBatch; b++)
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const float v = qrow[d[b][j] < 0 ? 0 : d[b][j]];
                    q0[b][j] = d[b][j] < 0 ? 0.f : v;
                }
        }
        if constexpr (QM == 0) {
#pragma unroll
            for (int b = 0; b < kBatch; b++)
#pragma unroll
                for (int j = 0; j < 4; j++) q0[b][j] = 0.f;
        }
#pragma unroll
        for (int b = 0; b < kBatch; b++) {
            const int tl = tb + (WT / 64) * b;
            if (tl >= ntiles) break;
            float s = 0.f;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int x = tl * kTile + lane + 64 * j;
                const float v = ZPASS ? walk_adj(a, W, krej, p0[b][j], q0[b][j], x)
                                      : walk_val(a, W, krej, p0[b][j], q0[b][j], x);
                s += x < V ? v : 0.f;
            }
            s = wave_sum(s);
            if (lane == 0) W.tsum[tl] = s;
        }
    }
}
__device__ __forceinline__ float walk_pass(WalkShared &W, const AcceptParams &a, int node, int krej, bool zpass) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int ntiles = (a.V + kTile - 1) / kTile;
    const int qm = !(zpass || krej > 0) ? 0 : a.q_map ? 2 : 1;
    if (zpass) {
        if (qm == 2) walk_tiles<true, 2>(W, a, node, krej);
        else walk_tiles<true, 1>(W, a, node, krej);
    } else {
        if (qm == 0) walk_tiles<false, 0>(W, a, node, krej);
        else if (qm == 2) walk_tiles<false, 2>(W, a, node, krej);
        else walk_tiles<false, 1>(W, a, node, krej);
    }
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

// sample_from_distribution's search (tokens.rs:99-120) after a walk_pass of
// the same f, by wave 0: the first x with f(x) > 0 whose running sum exceeds
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

// ---- a chain's passes, precomputed across the GPU ---------------------------------
// grid (n, tile groups), block kLtT: wave w of group y sums tiles
// (y * 4 + w) * kBatch + b, b < kBatch, of row r exactly as walk_tiles does
// (a lane's 4 entries in order, then wave_sum).  Phase 0: for a node with a
// child, max(0, p - q) (the normaliser pass of its first rejection), for the
// leaf p itself (its final draw); phase 1, after phase 0: max(0, p - q) / Z
// with Z totalled as walk_pass totals (the draw after the rejection).
constexpr int kLtT = 256;
template <int PHASE> __global__ __launch_bounds__(kLtT) void k_linear_tiles(AcceptParams a, float *lin) {
    warm_kernargs<sizeof(AcceptParams)>();
    const int r = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int V = a.V, n = a.n, ntiles = (V + kTile - 1) / kTile;
    const bool leaf = r == n - 1;
    if (PHASE == 1 && leaf) return;
    const float *prow = a.prob + (int64_t)r * V;
    const float *qrow = a.q + (int64_t)(leaf ? 0 : a.q_row_of[r]) * a.q_ld;
    float Z = 1.f;
    if (PHASE == 1) {
        const float *zt = lin + (int64_t)r * ntiles;
        float s = 0.f;
        for (int tl = lane; tl < ntiles; tl += 64) s += zt[tl];
        Z = wave_sum(s);
    }
    float *out = PHASE == 1 ? lin + (int64_t)(n + r) * ntiles : leaf ? lin + 2LL * n * ntiles : lin + (int64_t)r * ntiles;
    const int tb = ((int)blockIdx.y * (kLtT / 64) + wave) * kBatch;
    float p0[kBatch][4], q0[kBatch][4];
#pragma unroll
    for (int b = 0; b < kBatch; b++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int x = min((tb + b) * kTile + lane + 64 * j, V - 1);
            p0[b][j] = prow[x];
            q0[b][j] = leaf ? 0.f : qrow[x];
        }
#pragma unroll
    for (int b = 0; b < kBatch; b++) {
        const int tl = tb + b;
        if (tl >= ntiles) break;
        float s = 0.f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int x = tl * kTile + lane + 64 * j;
            const float v = leaf ? p0[b][j] : PHASE == 0 ? fmaxf(p0[b][j] - q0[b][j], 0.f)
                                                         : fmaxf(p0[b][j] - q0[b][j], 0.f) / Z;
            s += x < V ? v : 0.f;
        }
        s = wave_sum(s);
        if (lane == 0) out[tl] = s;
    }
}

// wave 0: a row of precomputed tile sums into W.tsum and its total (walk_pass's order)
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

// grid 1, block 1024
__global__ __launch_bounds__(WT) void k_accept_walk(AcceptParams a) {
    warm_kernargs<sizeof(AcceptParams)>();
    __shared__ WalkShared W;
    const int t = threadIdx.x;
    for (int i = t; i < a.n; i += WT) {
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
    __syncthreads();
    while (true) {
        // every thread has read the previous turn's W.go / W.node / W.krej
        // before thread 0 rewrites them
        __syncthreads();
        // ---- thread 0: test the children of the current node in BFS order ----
        if (t == 0) {
            W.go = 0;  // 0: descend done / 1: sample at node / 2: normaliser pass needed / 3: stop
            const int node = W.node;
            const float S = W.rs[node];
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
                    if (W.par[c] != node) continue;
                    if (seen++ < W.krej) continue;
                    const float u = W.uni[W.used++];
                    const int tok = W.tok[c];
                    const float p = walk_p(a, W, node, W.krej, tok);
                    if (W.krej == 0) W.R[0] = 1.f;
                    const float q = walk_q(a, W, accept_q(a, W.qrow[node], tok), W.krej, tok);
                    // modified_rejection_step (vanilla.rs:59-73)
                    const bool acc = q <= 0.f || u <= fminf(p / q, 1.f);
                    if (acc) {
                        accepted = c;
                        break;
                    }
                    W.go = 2;  // rejected: the adjusted distribution's normaliser is needed
                    if (W.krej < MAX_REJ) {
                        W.rej[W.krej] = tok;
                        if (W.krej + 1 < MAX_REJ) W.R[W.krej + 1] = W.R[W.krej] - accept_q(a, W.qrow[node], tok);
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
                    W.u = W.uni[W.used++];
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
            const int ntl = (a.V + kTile - 1) / kTile;
            const float Z = a.lin && krej == 0 ? walk_load_tiles(W, a.lin + (int64_t)node * ntl, ntl)
                                               : walk_pass(W, a, node, krej, true);
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
        auto f = [&](int x) { return walk_p(a, W, node, krej, x); };
        const int ntl = (a.V + kTile - 1) / kTile;
        const float sum = a.lin && krej == 1 ? walk_load_tiles(W, a.lin + (int64_t)(a.n + node) * ntl, ntl)
                          : a.lin && krej == 0 && node == a.n - 1 ? walk_load_tiles(W, a.lin + 2LL * a.n * ntl, ntl)
                                                                  : walk_pass(W, a, node, krej, false);
        if (!(sum > 0.f) || !isfinite(sum)) {
            if (t == 0) W.status = ACC_ERR_SOFTMAX;
            break;
        }
        if (t < 64) {
            const int x = walk_search(W, a.V, W.u * sum, f);
            if (t == 0) W.fin = x < 0 ? a.V - 1 : x;
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

void launch_row_stats(const float *logits, int64_t ld, int V, int rows, float inv_t, int greedy, const int *t2d_inv,
                      uint64_t *part, int *cnt, float *row_m, float *row_s, int *row_am, float *prob, hipStream_t st) {
    if (V < 1 || V > kRowStatsMaxSlices * kSlice) throw BackendError("acceptance: vocabulary too large");
    const dim3 grid(rows, (V + kSlice - 1) / kSlice);
    hipLaunchKernelGGL(k_row_stats, grid, dim3(kRsT), 0, st, logits, ld, V, inv_t, t2d_inv, part, cnt, row_m, row_s,
                       row_am);
    hipLaunchKernelGGL(k_row_prob, grid, dim3(kRsT), 0, st, logits, ld, V, inv_t, greedy, t2d_inv, row_m, row_s,
                       row_am, prob);
}

size_t linear_tiles_floats(int n, int V) { return (size_t)(2 * n + 1) * ((V + kTile - 1) / kTile); }

void launch_linear_tiles(const AcceptParams &a, float *lin, hipStream_t st) {
    if (a.V > kMaxTiles * kTile) throw BackendError("acceptance: vocabulary too large");
    if (a.n < 1 || a.n > kMaxNodes || a.q_map) throw BackendError("acceptance: linear tiles need a chain in the target vocabulary");
    const int ntiles = (a.V + kTile - 1) / kTile, per = (kLtT / 64) * kBatch;
    const dim3 grid(a.n, (ntiles + per - 1) / per);
    hipLaunchKernelGGL(k_linear_tiles<0>, grid, dim3(kLtT), 0, st, a, lin);
    hipLaunchKernelGGL(k_linear_tiles<1>, grid, dim3(kLtT), 0, st, a, lin);
}

void launch_accept_walk(const AcceptParams &a, hipStream_t st) {
    if (a.V > kMaxTiles * kTile) throw BackendError("acceptance: vocabulary too large");
    if (a.n < 1 || a.n > kMaxNodes) throw BackendError("acceptance: too many tree nodes");
    hipLaunchKernelGGL(k_accept_walk, dim3(1), dim3(WT), 0, st, a);
}

}  // namespace sd
