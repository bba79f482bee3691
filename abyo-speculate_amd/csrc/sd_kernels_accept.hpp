// Parameter block and launchers of the rejection-sampling acceptance kernels
// (sd_accept.hip).
#pragma once
#include "sd_kernels.hpp"

namespace sd {

enum AcceptStatus : int { ACC_OK = 0, ACC_ERR_SOFTMAX = 1, ACC_ERR_ADJUSTED = 2, ACC_ERR_ARG = 3 };

// children per tree node the walk supports (one normaliser per rejection)
constexpr int kAcceptMaxChildren = 16;
// ints of one node's record in a precomputed pass: node, children, draft row
// of its children, child k's token, its draft-row index (-1: none), whether
// the t2d map masks it, padding
constexpr int kTreeRec = 8;
// ints per tree node of a walk's inputs: parents, tokens, draft row, uniform,
// children count, the children's tokens, and the node's records of each
// precomputed pass
constexpr int kAccTreeInts = 5 + kAcceptMaxChildren + kTreeRec * (kAcceptMaxChildren + 1);

struct AcceptParams {
    float *prob;           // [n][V] the verify rows as distributions (written by the first pass), row i = tree node i
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
    // The logits rows of the verify pass (row i = tree node i), from which the
    // first precomputed pass writes prob.
    const float *logits;
    int64_t logits_ld;
    // The tree's shape for the precomputed passes: children per node, and
    // per node its children's tokens in BFS order ([n][kAcceptMaxChildren]).
    const int *nchild, *kids;
    // Every pass the walk can make, precomputed across the GPU by
    // launch_tree_tiles, per node and k = 0 .. c (its children): the tile
    // sums (tiles + (k * n + node) * tile count) of the adjusted
    // distribution's terms after k rejections (k < c: the normaliser of
    // rejection k is their total) or of the distribution after all c
    // rejections (k = c: the final draw); for k < c the test of child k,
    // (p, q, q0) at test + (k * n + node) * 3.
    float *tiles, *test;
};

// q(x) of draft row qr
__device__ __forceinline__ float accept_q(const AcceptParams &a, int qr, int x) {
    if (a.q_map) {
        const int d = a.q_map[x];
        return d < 0 ? 0.f : a.q[(int64_t)qr * a.q_ld + d];
    }
    return a.q[(int64_t)qr * a.q_ld + x];
}

// Softmax statistics (max, sum, first-max argmax) of `rows` logits rows.
// part: kRowStatsMaxSlices x 2 words per row; cnt: one zeroed int per row
// (left zeroed).
constexpr int kRowStatsMaxSlices = 32;
void launch_row_stats(const float *logits, int64_t ld, int V, int rows, float inv_t, const int *t2d_inv, uint64_t *part,
                      int *cnt, float *row_m, float *row_s, int *row_am, hipStream_t st);
void launch_accept_walk(const AcceptParams &a, hipStream_t st);
// The walk's passes, precomputed into a.tiles / a.test (kmax: the most
// children of a node, <= kAcceptMaxChildren), and the rows as distributions
// into a.prob; tree_tiles_floats is the floats of tiles and tests together.
// recs[k] (device) holds the kTreeRec-int records of the counts[k] nodes
// with at least k children (recs[0]: all of them).  Then launch_accept_walk.
size_t tree_tiles_floats(int n, int V, int kmax);
void launch_tree_tiles(const AcceptParams &a, int kmax, const int *const *recs, const int *counts, hipStream_t st);

}  // namespace sd
