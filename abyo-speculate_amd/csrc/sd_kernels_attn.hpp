// Parameter blocks and launchers of the attention kernels (sd_attn.hip).
#pragma once
#include "sd_kernels.hpp"

namespace sd {

struct RopeKvParams {
    const float *qkv;   // [M][ld_qkv] f32: q (n_heads*hd) | k (n_kv*hd) | v (n_kv*hd)
    int ld_qkv;
    const int *pos;     // [M] absolute positions
    const float *cos_t, *sin_t;  // [ctx][hd/2]
    uint16_t *q16;      // [n_heads][M][hd] fp16 (rotated q)
    uint16_t *kc, *vc;  // this layer's cache streams, [n_kv][cap * hd] in the blocked layout (kv_k_off / kv_v_off)
    int64_t cap;
    int P, M, n_heads, n_kv, hd;
    int interleaved;    // 1: rope_i pairs (2i, 2i+1) (Llama); 0: rope pairs (i, i+hd/2) (Qwen2)
    // nks > 1: the QKV matmul left K-slice partial sums part[ks][M][ld_qkv]
    // (no bias) instead of qkv; they are added in slice order, then the bias
    const float *part;
    int nks;
    const float *bq, *bk, *bv;  // QKV biases (Qwen2) or null
    // with K slices and norm_ssq set, the input was u = fp16(h * w_norm): the
    // slices' sum is scaled by norm_inv_rms(norm_ssq + m * norm_parts, ...)
    // over K columns before the bias
    const float *norm_ssq;
    int norm_parts, norm_K;
    float norm_eps;
};

// Work split of one attention call, a function of the prefix length P and the
// head layout only (never of M), so a query's arithmetic does not depend on
// how many other queries share the call.
struct AttnSplit {
    int keys_per_wave;  // a split covers 4 * keys_per_wave keys (multiple of 32 up to 16 rows, of 8 above)
    int nsplit;         // workgroups along the keys (for T = P + M keys)
};
AttnSplit attn_split(int P, int M, int n_kv, int n_rep);
int attn_max_splits(int n_kv);  // upper bound of nsplit over all P, M <= 128

struct AttnParams {
    const uint16_t *q16;
    const uint16_t *kc, *vc;
    int64_t cap;
    const uint64_t *mask;  // [M][mask_words]
    int mask_words;
    int P, M, n_heads, n_kv, n_rep, hd;
    int keys_per_wave, nsplit;
    float scale;           // 1/sqrt(hd)
    float *part_o;         // [nsplit][n_heads][M][hd]
    float *part_ml;        // [nsplit][n_heads][M][2]
    uint16_t *out16;       // [M][out_ld] fp16 fragment layout (input of wo)
    int out_ld;
    // Up to 16 rows with several splits: per-(KV head, query tile) arrival
    // counts, zero between launches, through which the last split of a tile
    // merges the splits inside the attention kernel (no combine launch).
    // Null: the combine kernel runs.  Launches sharing one array must not
    // overlap.
    int *split_cnt;
    int split_cnt_len;
    int fused_combine;     // set by launch_attention
};

void launch_rope_kv(const RopeKvParams &p, hipStream_t st);
void launch_attention(const AttnParams &p, hipStream_t st);
// Up to 16 rows: the checked parameters of the attention workgroups
// (fused_combine set), how many of them a launch has, and the combine launch
// that follows them when they do not merge the splits themselves (nothing
// with one split).
AttnParams attn_small_params(const AttnParams &p);
int attn_small_workgroups(const AttnParams &p);
void launch_attn_combine(const AttnParams &p, hipStream_t st);

// ---- sd_qgemm.hip: the fused Q/K/V + attention launch (M <= 16) ----
// The Q/K/V matmul with RoPE and the KV append in its epilogue (GemmParams g,
// as launch_qgemm takes it) and the attention over the result (AttnParams a,
// as launch_attention takes it) in one launch.  flags: nflags words, one per
// matmul workgroup, that a launch sets to epoch (non-zero, different from the
// previous launch's on these flags); status: host-visible memory that a launch
// sets to 1 if its attention gave up waiting for the matmul (its outputs are
// then undefined and the split counters must be cleared).  Launches sharing
// these words must not overlap.  cus: the device's CU count.  fault_polls:
// 0, or fault injection for tests: the attention waits for a number no
// producer writes and gives up after fault_polls reads (every workgroup still
// ends normally, and the launch reports through status).
struct QkvAttnSync {
    unsigned *flags;
    int nflags;
    unsigned epoch;
    int *status;
    int fault_polls;
};
bool qkv_attention_fits(const GemmParams &g, const AttnParams &a, int cus);
void launch_qkv_attention(const GemmParams &g, const AttnParams &a, const QkvAttnSync &sy, int cus, hipStream_t st,
                          const LaunchTiming &tm = LaunchTiming{});

}  // namespace sd
