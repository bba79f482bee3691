// Host runtime: device weights, fp16 KV cache, work buffers and the forward
// pass of the quantised Llama / Qwen2 target, plus the decoder state machine
// of the reference's LlamaQuantDecoder (crates/speculate/src/model/quantized_llama.rs).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <array>
#include <string>
#include <vector>

#include "sd_common.hpp"
#include "sd_kernels.hpp"
#include "sd_kernels_attn.hpp"
#include "sd_kernels_accept.hpp"
#include "sd_kernels_elem.hpp"

namespace sd {

// Error classes mapped 1:1 onto the reference's Error variants (error.rs:10-50).
struct SamplingError : std::runtime_error {
    explicit SamplingError(const std::string &m) : std::runtime_error(m) {}
};
struct RollbackError : std::runtime_error {
    explicit RollbackError(const std::string &m) : std::runtime_error(m) {}
};
struct ArgError : std::runtime_error {
    explicit ArgError(const std::string &m) : std::runtime_error(m) {}
};
struct UnsupportedError : std::runtime_error {
    explicit UnsupportedError(const std::string &m) : std::runtime_error(m) {}
};

enum Kind : int {
    K_TOK_EMBD = 0, K_OUTPUT = 1, K_OUTPUT_NORM = 2,
    K_ATTN_Q = 3, K_ATTN_K = 4, K_ATTN_V = 5, K_ATTN_O = 6,
    K_FFN_GATE = 7, K_FFN_UP = 8, K_FFN_DOWN = 9,
    K_ATTN_NORM = 10, K_FFN_NORM = 11, K_BQ = 12, K_BK = 13, K_BV = 14,
    K_NUM = 15
};

struct ModelCfg {
    int arch = 0;  // 0 llama (rope_i, no bias), 1 qwen2 (rope, QKV bias)
    int n_layers = 0, hidden = 0, n_heads = 0, n_kv_heads = 0, head_dim = 0, ffn = 0, vocab = 0;
    float rope_theta = 10000.f, rms_eps = 1e-5f;
    int ctx_len = 0;     // KV capacity (max positions)
    int max_batch = 128; // rows per forward pass
    int tied_output = 0;
    int device = 0;
    int q_dim() const { return n_heads * head_dim; }
    int kv_dim() const { return n_kv_heads * head_dim; }
};

// [rows][K] of a tensor kind under a config (norms and biases: rows = 1), and
// whether the kind is an F32 vector (norm or bias) rather than a matrix
void tensor_shape(const ModelCfg &c, int kind, int &rows, int &K);
bool kind_is_f32(int kind);

struct DevTensor {
    int fmt = -1;
    int rows = 0, K = 0;
    uint8_t *d = nullptr;
    size_t bytes = 0;
    // token_embd only: a second copy in GGUF row order, read by the embedding
    // gather (one row's superblocks are contiguous there, while the tile
    // layout interleaves 16 rows); HBM is plentiful, the gather is on the path
    uint8_t *gguf = nullptr;
    bool set() const { return d != nullptr; }
};

// Per-kernel-class timing collected with HIP events on the model's stream.
// Classes: 0 qkv, 1 wo, 2 gate_up, 3 down, 4 lm_head (the dequant-matmul
// launches), 5 attn (split attention + combine of one layer) and 6 qkv_attn
// (the fused Q/K/V + attention launch of one layer, M <= 16).
enum ProfClass : int {
    PC_QKV = 0, PC_WO = 1, PC_GATE_UP = 2, PC_DOWN = 3, PC_LM_HEAD = 4, PC_ATTN = 5, PC_QKV_ATTN = 6
};
struct ProfEntry {
    int cls;
    double bytes;  // algorithmic bytes of the launch
    int ev;        // index of the start event in the pool; the stop event is ev + 1
};

struct DraftTreeC;

class Model {
  public:
    explicit Model(const ModelCfg &c);
    ~Model();

    ModelCfg cfg;
    hipStream_t st = nullptr;

    // weights
    std::vector<std::array<DevTensor, K_NUM>> lw;  // per layer
    std::array<DevTensor, K_NUM> gw;              // global (layer = -1)

    void set_tensor(int layer, int kind, int fmt, const void *host, size_t bytes);
    void get_tensor(int layer, int kind, void *host, size_t bytes);
    void tensor_info(int layer, int kind, int *fmt, int *rows, int *K, size_t *gguf_bytes);
    void dequant_tensor(int layer, int kind, float *host);
    void synthesize(int mix, uint64_t seed, float std);
    void fill_kv_synthetic(int P, uint64_t seed);
    bool weights_ready() const;

    // raw matmul (test entry): y[M][N] = x[M][K] . W^T (x rounded to fp16)
    void qmatmul(int layer, int kind, const float *x, int M, float *y);
    // the same product on device buffers, enqueued on `stream` (the model's
    // own stream when null), with the fp16 activations staged in `staging`
    // (staging_bytes >= M * K * 2); allocates nothing and does not wait
    void qmatmul_into(int layer, int kind, const float *x_dev, int M, float *y_dev, hipStream_t stream,
                      void *staging, size_t staging_bytes);
    // microbenchmark of one dequant-matmul launch: microseconds per launch
    enum { BENCH_QKV = 100, BENCH_GATE_UP = 101, BENCH_ALL_LAYERS = -2 };
    double bench_qmatmul(int layer, int kind, int M, int iters, double *bytes_out);
    GemmParams bench_params(int layer, int kind, int M, double *bytes_out);

    // forward of M tokens at cache positions [P, P+M); mask words per token.
    // logits_mode: 0 none, 1 last row only (into logits row 0), 2 all rows.
    void forward(const int *ids, const int *pos, const uint64_t *mask, int mask_words, int M, int P, int logits_mode,
                 bool want_hidden, const std::vector<int> &collect, float *collect_out);
    void lm_head_rows(const float *hidden_host, int rows, float *out_host);
    // the lm_head product of M <= 16 rows already on the device, fp16 in the
    // matmul's fragment order (launch_to_frag16), into out [M][vocab] on `s`
    void lm_head_device(const uint16_t *xp, int M, float *out, hipStream_t s);
    void embed_rows(const int *ids, int n, float *out_host);
    void compact_tail(int P, const std::vector<int> &src);

    // profiling of the dominant kernels (events come from a pool that grows
    // on demand and is reused after every read, so timing adds no allocation
    // to a steady-state step)
    bool prof_on = false;
    std::vector<ProfEntry> prof;
    std::vector<hipEvent_t> ev_pool;
    void prof_reset();
    int prof_events();                             // index of a free (start, stop) event pair
    int prof_begin();                              // records a start event, returns its index
    void prof_end(int ev, int cls, double bytes);  // records the stop event

    // device buffers
    uint16_t *kv = nullptr;  // [L][2][n_kv][cap][hd]
    int64_t cap = 0;
    float *cos_t = nullptr, *sin_t = nullptr;
    float *h = nullptr, *qkv = nullptr, *logits = nullptr, *hidden_out = nullptr, *last_row = nullptr;
    float *part_o = nullptr, *part_ml = nullptr, *amax_v = nullptr, *collect_buf = nullptr;
    int collect_cap = 0;     // rows of collect_buf
    uint64_t fwd_count = 0;  // forwards, weight and cache writes so far (the collected rows' validity stamp)
    int *split_cnt = nullptr;  // attention's per-tile split arrival counts (zero between launches)
    // The fused Q/K/V + attention launch (M <= 16, where it fits): a flag per
    // matmul workgroup, the number of the last launch (the value its flags
    // were set to) and the pinned, device-mapped word a launch sets when its
    // attention gave up waiting for the matmul.  fused_qkv_attn: take the
    // fused launch where it fits (the environment variable SD_ATTN_UNFUSED=1
    // at creation turns it off, for comparisons).
    static constexpr int kQaFlags = 4096;
    unsigned *qa_flags = nullptr;
    unsigned qa_epoch = 0;
    int *qa_status = nullptr, *qa_status_dev = nullptr;
    int n_cus = 0;
    bool fused_qkv_attn = true;
    // waits for the stream, then fails (clearing the synchronisation words) if
    // a fused launch gave up
    void sync();
    void check_status();
    int *amax_i = nullptr, *argmax = nullptr, *d_ids = nullptr, *d_pos = nullptr, *d_src = nullptr;
    uint64_t *d_mask = nullptr;
    // split-K partial sums of the M > 16 matmul (see GemmParams::allow_split)
    float *qg_part = nullptr;
    int64_t qg_part_cap = 0;
    // fused RMSNorm (M <= 16): per-16-row-tile sums of h^2, [16][hidden / 16]
    float *ssq = nullptr;
    void gemm_workspace(GemmParams &p) const {
        p.part = qg_part;
        p.part_cap = qg_part_cap;
    }
    // rejection-sampling acceptance: per-row softmax statistics, the tree,
    // draft rows, uniforms and results (draft rows grow on demand)
    float *acc_m = nullptr, *acc_s = nullptr, *acc_q = nullptr;
    size_t acc_q_cap = 0;  // floats
    uint64_t *acc_part = nullptr;  // row statistics' per-slice partials
    int *acc_cnt = nullptr;        // their per-row arrival counts (zero between launches)
    float *acc_lin = nullptr;      // the walk's precomputed passes (launch_tree_tiles)
    size_t acc_lin_cap = 0;        // floats
    float *acc_prob = nullptr;     // the verify rows as distributions
    size_t acc_prob_cap = 0;       // floats
    int *acc_am = nullptr, *acc_tree = nullptr, *acc_out = nullptr;
    // d2t map of an EAGLE-3 draft (eagle3.rs:377-397): target id -> draft id or -1
    int *t2d_inv = nullptr;
    int d2t_draft_vocab = 0;
    uint16_t *xp = nullptr, *ap = nullptr, *act = nullptr, *q16 = nullptr;
    int xp_ld = 0, ap_ld = 0, act_ld = 0;
    int amax_ld = 0;
    int nsplit_max = 0;
    int logits_rows_last = 0;  // rows of `logits` / `argmax` produced by the last forward
    // apply_lm_head / embed_tokens work buffers (kAuxRows rows per chunk),
    // apart from the verify pass's
    static constexpr int kAuxRows = 16;
    float *aux_h = nullptr, *aux_y = nullptr;
    uint16_t *aux_x = nullptr;
    int *aux_ids = nullptr;
    // pinned staging for small H2D transfers
    int *h_stage = nullptr;
    int *acc_stage = nullptr;  // pinned: a walk's inputs [kAccTreeInts max_batch] and outputs [max_batch + 4]
    size_t h_stage_bytes = 0;
    hipEvent_t stage_ev = nullptr;  // recorded after the last copy out of h_stage
    void stage_wait();               // host waits until h_stage may be rewritten
    void stage_done();

    // token table in GGUF row order (F32 tables are row-major either way)
    const uint8_t *embed_table() const { return gw[K_TOK_EMBD].fmt == F32 ? gw[K_TOK_EMBD].d : gw[K_TOK_EMBD].gguf; }

  private:
    void alloc_buffers();
    void run_gemm(GemmParams &p, int cls, double bytes);
    uint16_t *kc(int layer) const { return kv + (int64_t)layer * 2 * cfg.n_kv_heads * cap * cfg.head_dim; }
    uint16_t *vc(int layer) const { return kc(layer) + (int64_t)cfg.n_kv_heads * cap * cfg.head_dim; }
};

// Decoder contract of LlamaQuantDecoder (quantized_llama.rs:443-600) over Model.
class Decoder {
  public:
    explicit Decoder(Model *m) : model(m) {}
    Model *model;
    std::vector<uint32_t> history;
    int cache_len = 0;
    bool last_valid = false;  // last_logits cache (device row model->last_row)
    std::vector<uint32_t> eos;

    void reset();
    void observe(const uint32_t *ids, size_t n);
    void next_logits(float *out);
    void batched_logits(const uint32_t *drafts, size_t k, float *out);
    void rollback_to(size_t len);
    void tree_logits_keep_kv(const uint32_t *tokens, const uint32_t *parents, size_t n, float *out_logits,
                             float *out_hidden);
    void tree_logits(const uint32_t *tokens, const uint32_t *parents, size_t n, float *out_logits);
    void commit_tree_path(const uint32_t *tokens, const uint32_t *parents, size_t n, const uint32_t *acc,
                          size_t n_acc);
    void last_hidden_state(float *out);
    void observe_returning_last_hidden(const uint32_t *ids, size_t n, float *out);
    void last_hidden_states_multi(const uint32_t *layers, size_t nl, float *out_final, float *out_layers);
    const float *collect_hidden_device(const uint32_t *layers, size_t nl);
    // The layers of the last collection; a one-token observe collects them
    // as it goes, so that the next collection for that token (the EAGLE-3
    // round after the bonus token's observe) reads them instead of running
    // the same M=1 forward again.  Valid while the history length and the
    // model's forward count are the ones recorded.
    std::vector<int> collect_keep;
    size_t collect_hist = 0;
    uint64_t collect_fwd = 0;

    // device acceptance
    void verify_greedy_linear(const uint32_t *drafts, size_t k, uint32_t *commits, size_t *n_commit,
                              size_t *n_accepted);
    void verify_greedy_tree(const uint32_t *tokens, const uint32_t *parents, size_t n, int strict,
                            uint32_t *path, size_t *path_len, uint32_t *bonus, int32_t *bonus_node,
                            uint32_t *committed, size_t *n_committed, size_t *keep_len, int32_t *stop);
    void argmax_rows(int32_t *out, size_t n);
    // batched_logits + the rejection walk of vanilla.rs:178-210 on the device
    // (q_on_device: q_rows is a device pointer on the model's GPU, not uploaded)
    void verify_rejection_linear(const uint32_t *drafts, size_t k, const float *q_rows, const float *uniforms,
                                 size_t n_uniforms, float temperature, size_t max_commit, uint32_t *commits,
                                 size_t *n_commit, size_t *n_accepted, size_t *n_used, bool q_on_device = false);
    // tree_logits_keep_kv + the tree rejection walk (sd_accept.hip)
    void verify_rejection_tree(const uint32_t *tokens, const uint32_t *parents, size_t n, const float *q_rows,
                               size_t q_rows_n, size_t q_vocab, const int32_t *q_row_of, const float *uniforms,
                               size_t n_uniforms, float temperature, int use_t2d, int siblings, size_t max_commit,
                               uint32_t *path, size_t *path_len, int32_t *token, size_t *n_used,
                               bool q_on_device = false);
    // EAGLE-3 vocabulary map (eagle3.rs:377-397, 476-513)
    void set_d2t(const int64_t *d2t, size_t n);
    std::vector<int64_t> d2t_host;
    std::vector<int32_t> t2d_host;  // target id -> draft id or -1 (last writer wins, like the HashMap insert)

    // sets history and KV [0, n) to synthetic values (benchmarks, full-size tests)
    void prime_synthetic(const uint32_t *ids, size_t n, uint64_t kv_seed);

  private:
    void forward_advance(const uint32_t *tokens, size_t n, bool all_rows);
    // the acceptance walk over logits rows [0, n) of the last pass
    void accept_walk(const int *parents, const int *tokens, int n, const float *q_rows, bool q_on_device,
                     size_t q_rows_n, size_t q_vocab, const int *q_row_of, const float *uniforms, float temperature,
                     int use_t2d, int wor, size_t max_commit, std::vector<int> &path, int &fin, size_t &used);
    void truncate(size_t len);
    void tree_forward(const uint32_t *tokens, const uint32_t *parents, size_t n, bool want_hidden, int &prefix);
};

// Host DraftTree (tree.rs:38-282): parent table validation, depths, paths, masks.
struct DraftTreeC {
    std::vector<uint32_t> tokens;
    std::vector<uint32_t> parents;
    static DraftTreeC from_arrays(const uint32_t *tokens, const uint32_t *parents, size_t n);
    size_t size() const { return tokens.size(); }
    int depth_of(size_t i) const;
    bool is_ancestor_of(size_t a, size_t n) const;
    std::vector<std::vector<size_t>> paths() const;
    void masks(std::vector<uint64_t> &words, int &nw) const;
};

// Tree builders (sd_tree.cpp): medusa.rs:172-193 and eagle.rs:763-845.
DraftTreeC cartesian_tree(uint32_t root, const uint32_t *cand, const uint32_t *branching, size_t depth);
size_t cartesian_size(const uint32_t *branching, size_t depth);
DraftTreeC prune_cartesian(const DraftTreeC &full, const float *log_probs, const uint32_t *branching, size_t depth,
                           size_t max_total);

}  // namespace sd
