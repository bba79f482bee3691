// EAGLE drafts on the device: EAGLE-3 (crates/speculate/src/methods/eagle3.rs:
// the f16 midlayer, norm + lm_head, per-step top-k / log-probs and d2t) and
// EAGLE-2 (methods/eagle.rs: fc over [hidden, embedding], one Llama block,
// the target's lm_head), run on the target model's stream so that a whole
// draft round needs no host round trip (sd_draft.hip holds the kernels,
// sd_draft.cpp these classes).
#pragma once
#include <stdint.h>

#include <vector>

#include "sd_kernels.hpp"

namespace sd {

class Model;
class Decoder;

constexpr int kDraftMaxK = 32768;    // inputs of one matrix-vector product
constexpr int kDraftMaxSteps = 16;   // draft steps of one round (the draft's own KV cache)
constexpr int kDraftMaxTopk = 8;     // candidates per step
constexpr size_t kDraftOut = (size_t)kDraftMaxSteps * kDraftMaxTopk;  // entries of one round's output array

enum DraftGemvMode : int { DG_STORE = 0, DG_ADD = 1, DG_SWIGLU = 2, DG_LOGITS = 3 };

struct DraftGemv {
    const uint16_t *w;  // [N][K] f16 (SwiGLU: [2N][K], gate rows then up rows)
    const uint16_t *x;  // [K] f16
    int N, K;           // SwiGLU: N = features
    uint16_t *y16;      // STORE / ADD / SWIGLU output (f16)
    const uint16_t *res16;  // ADD: y = f16(f16(W x) + res)
    float *y32;         // LOGITS: the f16 results as f32
};
void launch_gemv16(int mode, const DraftGemv &p, hipStream_t st);

struct DraftNorm {
    const uint16_t *x16[2];  // f16 input of row i, or
    const float *x32[2];     // f32 input (rounded to f16 first), one of them null
    const uint16_t *w[2];
    uint16_t *out[2];
    int H;
    float eps;
};
void launch_rmsnorm16(const DraftNorm &p, int rows, hipStream_t st);
// out[0, H) = table[*id][0, H) (f16 rows; nothing written for an id out of range)
void launch_gather16(const uint16_t *table, int64_t rows, int H, const int32_t *id, uint16_t *out, hipStream_t st);
void launch_to_f16(const float *x, int64_t n, uint16_t *y, hipStream_t st);

// RoPE of q and this step's k, the append of k and v to the draft cache, and
// attention over every cached step, one launch
struct DraftAttn {
    const uint16_t *qkv;              // [n_heads + 2 n_kv][hd] of this step
    const uint16_t *cos16, *sin16;    // [max_pos][hd/2]
    uint16_t *kcache, *vcache;        // [kDraftMaxSteps][n_kv][hd]
    uint16_t *out;                    // [n_heads][hd]
    int n_heads, n_kv, hd, pos, step; // step: this step's cache slot
    float scale;
};
void launch_draft_attn(const DraftAttn &p, hipStream_t st);

struct DraftTopk {
    const float *logits;  // [V]
    int V, k;
    const int32_t *d2t;   // [V] target ids (null: the ids themselves)
    int32_t *out_draft, *out_target;
    float *out_lp;
    int32_t *next_token;  // the top-1 target id (the next step's embedding row)
    uint64_t *part;       // [64][1 + kDraftMaxTopk] per-slice partials
    int *cnt;             // arrival count, 0 between launches
};
void launch_draft_topk(const DraftTopk &p, hipStream_t st);

struct Draft3Cfg {
    int hidden = 4096, n_heads = 32, n_kv_heads = 8, ffn = 14336, draft_vocab = 32000, target_vocab = 128256;
    float rms_eps = 1e-5f, rope_theta = 500000.f;
    int max_pos = 2048;
    int device = 0;
    int head_dim() const { return hidden / n_heads; }
};

// Tensor kinds of the checkpoint (eagle3.rs:133-150, 363-386)
enum Draft3Tensor : int {
    D3_FC = 0, D3_Q, D3_K, D3_V, D3_O, D3_GATE, D3_UP, D3_DOWN, D3_LM_HEAD,
    D3_IN_NORM, D3_HID_NORM, D3_POST_NORM, D3_NORM, D3_D2T, D3_NUM
};

class Draft3 {
  public:
    explicit Draft3(const Draft3Cfg &c);
    ~Draft3();
    Draft3Cfg cfg;

    // f16 weights [out][in] / norms [hidden]; D3_D2T: int64 [draft_vocab]
    void set_tensor(int kind, const void *host, size_t bytes);
    void get_tensor(int kind, void *host, size_t bytes) const;
    size_t tensor_bytes(int kind) const;
    // seeded synthetic weights (N(0, std) f16 matrices, norms 1 + N(0, 0.1), a
    // permutation-free d2t of distinct target ids)
    void synthesize(uint64_t seed, float std);
    bool ready() const;

    // forward_hidden + apply_norm_lm_head of one step from host inputs:
    // hidden_in f32 [3 hidden] (first step: fc applied) or [hidden]; input_emb
    // f32 [hidden]; appends to the draft's cache (reset() clears it)
    void step_host(const float *hidden_in, size_t n_in, const float *input_emb, int position, float *out_hidden,
                   float *out_logits);
    void reset() { steps = 0; }

    // One round of run_eagle3 (eagle3.rs:598-673) against `target`: the hidden
    // states of `layers` for the committed token, then `depth` steps, top_k[s]
    // candidates at step s; outputs target ids, draft ids and log-probs,
    // [depth][kDraftMaxTopk] each.
    void round(Model &target, Decoder &dec, const uint32_t layers[3], int depth, const int *top_k, int32_t *ids,
               int32_t *draft_ids, float *log_probs);

  private:
    void step_device(int position, bool first, hipStream_t st, int k, int32_t *ids, int32_t *dids, float *lps);
    size_t off[D3_NUM] = {}, len[D3_NUM] = {};
    bool have[D3_NUM] = {};
    uint16_t *w = nullptr;     // every f16 tensor, one allocation (Q, K, V adjacent; GATE, UP adjacent)
    int32_t *d2t = nullptr;    // [draft_vocab]
    std::vector<int64_t> d2t_host;
    uint16_t *cos16 = nullptr, *sin16 = nullptr;
    uint16_t *kc = nullptr, *vc = nullptr;
    // work: x3 [3H], hid[2] [H] (this step's input / output), proj [H], comb [2H],
    // qkv [(nh + 2 nkv) hd], att [nh hd], after [H], xn [H], act [ffn], xf [H]
    uint16_t *x3 = nullptr, *hid[2] = {nullptr, nullptr}, *proj = nullptr, *comb = nullptr, *qkv = nullptr,
             *att = nullptr, *after = nullptr, *xn = nullptr, *act = nullptr, *xf = nullptr;
    float *emb = nullptr, *logits = nullptr, *hin32 = nullptr;
    int32_t *tok = nullptr;                         // the current step's token id
    uint64_t *tk_part = nullptr;                    // top-k slice partials
    int *tk_cnt = nullptr;                          // top-k arrival count
    int32_t *o_ids = nullptr, *o_dids = nullptr;    // [kDraftMaxSteps][kDraftMaxTopk], in one block with o_lp
    float *o_lp = nullptr;
    int32_t *pin = nullptr;                         // pinned: the three output arrays, then the root token
    int cur = 0;  // which hid[] holds the current step's input
    int steps = 0;
    hipStream_t own = nullptr;
};

// ---- EAGLE-2 (EagleDraftCandle, eagle.rs:306-428) ----------------------------------
struct Draft2Cfg {
    int hidden = 4096, n_heads = 32, n_kv_heads = 8, ffn = 14336, vocab = 128256;
    float rms_eps = 1e-5f, rope_theta = 500000.f;
    int max_pos = 2048;
    int device = 0;
    int head_dim() const { return hidden / n_heads; }
};

// Tensor kinds of the checkpoint (eagle.rs:126-131, 279-286, 349-361)
enum Draft2Tensor : int {
    D2_EMBED = 0, D2_FC, D2_Q, D2_K, D2_V, D2_O, D2_GATE, D2_UP, D2_DOWN, D2_POST_NORM, D2_NUM
};

class Draft2 {
  public:
    explicit Draft2(const Draft2Cfg &c);
    ~Draft2();
    Draft2Cfg cfg;

    // f16 weights [out][in] (embed_tokens [vocab][hidden]) / post_attention_layernorm [hidden]
    void set_tensor(int kind, const void *host, size_t bytes);
    void get_tensor(int kind, void *host, size_t bytes) const;
    size_t tensor_bytes(int kind) const;
    void synthesize(uint64_t seed, float std);
    bool ready() const;

    // EagleDraftCandle::forward (eagle.rs:390-427) of one position:
    // target_hidden f32 [hidden] (the target's final-norm hidden state, or the
    // previous step's output), the token id, the RoPE position; appends to the
    // draft's cache (reset() clears it); out f32 [hidden] (f16 values)
    void step_host(const float *target_hidden, uint32_t token, int position, float *out);
    void reset() { steps = 0; }

    // The draft half of one run_eagle iteration (eagle.rs:519-575) against
    // `target`: the committed token's final-norm hidden state (host f32),
    // then `depth` steps, each a draft forward, the target's lm_head on its
    // output, top_k[s] ids by value (index ascending on ties) with their
    // log-probs; the top-1 id and the step's output feed the next step.
    // Outputs [depth][kDraftMaxTopk].
    void round(Model &target, Decoder &dec, const float *target_hidden, int depth, const int *top_k, int32_t *ids,
               float *log_probs);

  private:
    void step_device(int position, hipStream_t st);
    size_t off[D2_NUM] = {}, len[D2_NUM] = {};
    bool have[D2_NUM] = {};
    uint16_t *w = nullptr;  // every f16 tensor (Q, K, V adjacent; GATE, UP adjacent)
    uint16_t *cos16 = nullptr, *sin16 = nullptr, *kc = nullptr, *vc = nullptr;
    // work: comb [2H] = [input hidden | token embedding], xs [H] (fc), qkv,
    // att [nh hd], after [H], xn [H], act [ffn]; the step's output goes to
    // comb[0, H) (the next step's input) and out32 [H]
    uint16_t *comb = nullptr, *xs = nullptr, *qkv = nullptr, *att = nullptr, *after = nullptr, *xn = nullptr,
             *act = nullptr, *xp = nullptr;
    float *hin32 = nullptr, *out32 = nullptr, *logits = nullptr;
    int32_t *tok = nullptr, *o_ids = nullptr, *o_dids = nullptr;  // o_ids | o_dids | o_lp: one block
    float *o_lp = nullptr;
    int32_t *pin = nullptr;  // pinned: the three output arrays, then the root token
    uint64_t *tk_part = nullptr;
    int *tk_cnt = nullptr;
    int steps = 0;
    hipStream_t own = nullptr;
};

}  // namespace sd
