// Parameter block and launchers of the rejection-sampling acceptance kernels
// (sd_accept.hip).
#pragma once
#include "sd_kernels.hpp"

namespace sd {

enum AcceptStatus : int { ACC_OK = 0, ACC_ERR_SOFTMAX = 1, ACC_ERR_ADJUSTED = 2, ACC_ERR_ARG = 3 };

struct AcceptParams {
    const float *prob;     // [n][V] the verify rows as distributions (k_row_prob), row i = tree node i
    int V;                 // target vocabulary
    int n;                 // tree nodes (a chain for the linear walk)
    const int *parents;    // [n], parents[0] unused
    const int *tokens;     // [n] target-vocab ids
    const float *row_m, *row_s;  // softmax statistics per row (k_row_stats)
    const int *row_am;     // first-max argmax per row
    float inv_t;           // 1 / temperature (unused when greedy)
    int greedy;            // temperature == 0: one-hot distributions
    const int *t2d_inv;    // nullable: target id -> draft id or -1; -1 entries are masked out of the target rows
    const float *q;        // draft rows [*][q_ld]
    int64_t q_ld;
    const int *q_map;      // nullable: q rows are in the draft vocabulary, target id x reads q[t2d_inv[x]]
    const int *q_row_of;   // [n] q row of each node's children (-1 for leaves)
    const float *uniforms; // >= n values
    int max_commit;        // 0: no limit; else stop after this many committed drafts
    int wor;               // 1: siblings were drawn without replacement from q, so each rejected
                           // token's q is zeroed and q renormalised before the next sibling
    int *out_path;         // [n] accepted node indices, root first
    int *out_info;         // [4]: path length, final token (-1 none), uniforms used, status
    // A chain (node i's child is i + 1) with draft rows in the target
    // vocabulary may carry every pass its walk can make, precomputed across
    // the GPU by launch_linear_tiles: per node the tile sums of max(0, p - q)
    // and of max(0, p - q) / Z, and the leaf's tile sums of p.  Null: the walk
    // makes its passes itself.
    const float *lin;
};

// q(x) of draft row qr
__device__ __forceinline__ float accept_q(const AcceptParams &a, int qr, int x) {
    if (a.q_map) {
        const int d = a.q_map[x];
        return d < 0 ? 0.f : a.q[(int64_t)qr * a.q_ld + d];
    }
    return a.q[(int64_t)qr * a.q_ld + x];
}

// Softmax statistics (max, sum, first-max argmax) of `rows` logits rows and
// the rows as distributions into prob [rows][V].  part: kRowStatsMaxSlices x 2
// words per row; cnt: one zeroed int per row (left zeroed).
constexpr int kRowStatsMaxSlices = 32;
void launch_row_stats(const float *logits, int64_t ld, int V, int rows, float inv_t, int greedy, const int *t2d_inv,
                      uint64_t *part, int *cnt, float *row_m, float *row_s, int *row_am, float *prob, hipStream_t st);
void launch_accept_walk(const AcceptParams &a, hipStream_t st);
// the precomputed passes of a chain's walk into lin [(2 n + 1) x tiles]
// (AcceptParams::lin; a.prob, a.q, a.q_row_of, a.V, a.n as for the walk)
size_t linear_tiles_floats(int n, int V);
void launch_linear_tiles(const AcceptParams &a, float *lin, hipStream_t st);

}  // namespace sd
