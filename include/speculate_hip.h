/*
 * speculate_hip.h -- C ABI of the MI355X (gfx950) target-verify library.
 *
 * The drop-in point is the reference's decoder boundary: the `Decoder` and
 * `TreeDecoder` traits (crates/speculate/src/model/mod.rs:39-108, :118-236) as
 * implemented by `LlamaQuantDecoder` (crates/speculate/src/model/quantized_llama.rs)
 * and `Qwen2QuantDecoder` (crates/speculate/src/model/quantized_qwen2.rs).  One
 * `sd_model` handle is one such decoder: quantised weights, fp16 KV cache,
 * token history and the cached next-token logits, all resident on one GPU.
 * Paths cited below are relative to the reference checkout.
 *
 * Conventions
 *  - Every entry point that can fail returns an sd_status; on failure the
 *    decoder state is unchanged (model/mod.rs:35-38) and sd_last_error()
 *    returns a thread-local message.
 *  - Output buffers are owned by the caller (host memory); pass NULL to skip an
 *    output.  Logits are row-major [rows][vocab] f32, hidden states [rows][hidden] f32.
 *  - A draft tree is passed as two arrays of n entries, node tokens and parent
 *    indices in BFS order (parents[0] is ignored; parents[i] < i), exactly the
 *    parent table of DraftTree::from_parent_table (tree.rs:52-74).
 *  - A handle is not thread-safe; it may move between threads.  Every call
 *    sets its device and uses the handle's own stream.
 */
#ifndef SPECULATE_HIP_H
#define SPECULATE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes, one per reference Error variant (crates/speculate/src/error.rs:10-50). */
typedef enum sd_status {
    SD_OK = 0,
    SD_ERR_SAMPLING = 1,    /* Error::Sampling: empty history/tokens, tree root mismatch, bad tree */
    SD_ERR_ROLLBACK = 2,    /* Error::CacheRollback: rollback past the history */
    SD_ERR_BACKEND = 3,     /* Error::Candle: device/runtime failure, truncate past the cache */
    SD_ERR_ARG = 4,         /* invalid argument (sizes, ids, capacity) */
    SD_ERR_UNSUPPORTED = 5  /* Error::UnsupportedMethod / unsupported shape or format */
} sd_status;

/* Tensor formats: the GGML type ids of the GGUF blocks. */
enum { SD_F32 = 0, SD_Q8_0 = 8, SD_Q4_K = 12, SD_Q5_K = 13, SD_Q6_K = 14 };

/* Tensor kinds.  The GGUF names follow quantized_llama_local.rs:242-281 and
 * quantized_qwen2_local.rs:232-275 ("blk.{i}." prefix for per-layer tensors). */
enum {
    SD_TOK_EMBD = 0,    /* token_embd.weight   [vocab][hidden]  (layer -1) */
    SD_OUTPUT = 1,      /* output.weight       [vocab][hidden]  (layer -1) */
    SD_OUTPUT_NORM = 2, /* output_norm.weight  [hidden] F32     (layer -1) */
    SD_ATTN_Q = 3,      /* attn_q.weight       [q_dim][hidden] */
    SD_ATTN_K = 4,      /* attn_k.weight       [kv_dim][hidden] */
    SD_ATTN_V = 5,      /* attn_v.weight       [kv_dim][hidden] */
    SD_ATTN_OUTPUT = 6, /* attn_output.weight  [hidden][q_dim] */
    SD_FFN_GATE = 7,    /* ffn_gate.weight     [ffn][hidden] */
    SD_FFN_UP = 8,      /* ffn_up.weight       [ffn][hidden] */
    SD_FFN_DOWN = 9,    /* ffn_down.weight     [hidden][ffn] */
    SD_ATTN_NORM = 10,  /* attn_norm.weight    [hidden] F32 */
    SD_FFN_NORM = 11,   /* ffn_norm.weight     [hidden] F32 */
    SD_ATTN_Q_BIAS = 12,/* attn_q.bias         [q_dim] F32   (qwen2 only) */
    SD_ATTN_K_BIAS = 13,/* attn_k.bias         [kv_dim] F32  (qwen2 only) */
    SD_ATTN_V_BIAS = 14 /* attn_v.bias         [kv_dim] F32  (qwen2 only) */
};

/* Architectures: llama = interleaved rope_i, no bias (quantized_llama_local.rs);
 * qwen2 = half-rotation rope, QKV bias (quantized_qwen2_local.rs). */
enum { SD_ARCH_LLAMA = 0, SD_ARCH_QWEN2 = 1 };

/* Synthetic quantisation mixes for sd_model_synthesize. */
enum {
    SD_MIX_Q4_K = 0,     /* every matrix Q4_K */
    SD_MIX_Q4_K_M = 1,   /* Q6_K on attn_v / ffn_down where llama.cpp's use_more_bits holds, Q4_K elsewhere */
    SD_MIX_Q5K_Q80 = 2,  /* attention Q5_K, FFN / embedding / lm_head Q8_0 */
    SD_MIX_Q6_K = 3, SD_MIX_Q5_K = 4, SD_MIX_Q8_0 = 5
};

/* Model hyper-parameters: the GGUF metadata read at quantized_llama_local.rs:229-238
 * (llama.*) / quantized_qwen2_local.rs:220-228 (qwen2.*). */
typedef struct sd_config {
    int32_t arch;
    int32_t n_layers;     /* block_count */
    int32_t hidden;       /* embedding_length */
    int32_t n_heads;      /* attention.head_count */
    int32_t n_kv_heads;   /* attention.head_count_kv */
    int32_t head_dim;     /* embedding_length / head_count (= rope.dimension_count) */
    int32_t ffn;          /* feed_forward_length */
    int32_t vocab;
    float rope_theta;     /* rope.freq_base */
    float rms_eps;        /* attention.layer_norm_rms_epsilon */
    int32_t ctx_len;      /* KV capacity in positions (context_length) */
    int32_t max_batch;    /* rows of one forward pass (<= 128); longer observes are chunked */
    int32_t tied_output;  /* 1: lm_head reuses token_embd (quantized_llama_local.rs:249-252) */
    int32_t device;       /* HIP device ordinal */
} sd_config;

typedef struct sd_model sd_model;

/* ---- lifecycle and weights ------------------------------------------------ */

/* Allocates the handle, KV cache and work buffers; weights start unset.
 * Replaces LlamaQuantDecoder::from_gguf's allocation (quantized_llama.rs:57-98). */
sd_status sd_model_create(const sd_config *cfg, sd_model **out);
void sd_model_destroy(sd_model *m);

/* Uploads one tensor given in its GGUF byte layout (`layer` = -1 for the
 * global tensors).  Replaces the `ct.tensor(reader, name, device)` loads at
 * quantized_llama_local.rs:242-281. */
sd_status sd_model_set_tensor(sd_model *m, int32_t layer, int32_t kind, int32_t fmt, const void *data, size_t bytes);
/* Downloads one tensor in its GGUF byte layout. */
sd_status sd_model_get_tensor(sd_model *m, int32_t layer, int32_t kind, void *out, size_t bytes);
sd_status sd_model_tensor_info(sd_model *m, int32_t layer, int32_t kind, int32_t *fmt, int32_t *rows, int32_t *cols,
                               size_t *gguf_bytes);
/* Generates every tensor on the GPU from `seed`: matrices N(0, std)-like values
 * quantised with `mix`, norms 1.0, biases N(0, std)-like F32. */
sd_status sd_model_synthesize(sd_model *m, int32_t mix, uint64_t seed, float std);
/* Exact f32 dequantisation of one tensor (QTensor::dequantize,
 * quantized_llama_local.rs:242-243): [rows][cols]. */
sd_status sd_model_dequant_tensor(sd_model *m, int32_t layer, int32_t kind, float *out);
/* One fused dequant-matmul, y[rows][N] = x[rows][K] . W^T, x rounded to fp16
 * (QMatMul::forward, quantized_llama_local.rs:47-49, 73-90, 135, 317). */
sd_status sd_model_qmatmul(sd_model *m, int32_t layer, int32_t kind, const float *x, size_t rows, float *y);

const char *sd_last_error(void);

/* ---- Decoder (model/mod.rs:39-108) ------------------------------------------ */
size_t sd_vocab_size(const sd_model *m);                      /* Decoder::vocab_size */
size_t sd_history_len(const sd_model *m);                     /* Decoder::history_len */
size_t sd_history(const sd_model *m, uint32_t *out, size_t cap); /* Decoder::history (copies min(cap, len)) */
void sd_reset(sd_model *m);                                   /* Decoder::reset, quantized_llama.rs:512-517 */
/* Decoder::observe (quantized_llama.rs:519-526): forward + cache the next-token logits. */
sd_status sd_observe(sd_model *m, const uint32_t *ids, size_t n);
/* Decoder::next_logits (quantized_llama.rs:528-551): out [vocab]. */
sd_status sd_next_logits(sd_model *m, float *out);
/* Decoder::batched_logits (quantized_llama.rs:553-583): out [(k+1)][vocab]; history += drafts.
 * out NULL: the rows stay on the device (sd_last_argmax, the acceptance entry
 * points) and the call returns once the forward is queued. */
sd_status sd_batched_logits(sd_model *m, const uint32_t *drafts, size_t k, float *out);
/* Decoder::rollback_to (quantized_llama.rs:585-599). */
sd_status sd_rollback_to(sd_model *m, size_t len);
/* Decoder::eos_token_ids (quantized_llama.rs:500-502): caller-supplied at construction in the reference. */
sd_status sd_set_eos_token_ids(sd_model *m, const uint32_t *ids, size_t n);
size_t sd_eos_token_ids(const sd_model *m, uint32_t *out, size_t cap);

/* ---- TreeDecoder (model/mod.rs:118-236) -------------------------------------- */
/* TreeDecoder::tree_logits_keep_kv (quantized_llama.rs:341-394): out_logits [n][vocab],
 * out_hidden [n][hidden] (final-norm hidden); cache left at prefix + n. */
sd_status sd_tree_logits_keep_kv(sd_model *m, const uint32_t *tokens, const uint32_t *parents, size_t n,
                                 float *out_logits, float *out_hidden);
/* TreeDecoder::tree_logits: the tree pass, then the cache restored by an M=1 pass of the
 * root (which refreshes the cached next-token row). Llama handles (quantized_llama.rs:262-325)
 * return that M=1 row as row 0; Qwen2 handles (quantized_qwen2.rs:184-237) keep the tree
 * pass's row 0 and discard the M=1 row, as the reference does. */
sd_status sd_tree_logits(sd_model *m, const uint32_t *tokens, const uint32_t *parents, size_t n, float *out_logits);
/* TreeDecoder::commit_tree_path (quantized_llama.rs:409-440): keep [0..P) ++ [P + accepted[j]]. */
sd_status sd_commit_tree_path(sd_model *m, const uint32_t *tokens, const uint32_t *parents, size_t n,
                              const uint32_t *accepted, size_t n_accepted);
/* TreeDecoder::last_hidden_state (quantized_llama.rs:193-214): out [hidden]. */
sd_status sd_last_hidden_state(sd_model *m, float *out);
/* TreeDecoder::observe_returning_last_hidden (quantized_llama.rs:174-191): out [hidden]. */
sd_status sd_observe_returning_last_hidden(sd_model *m, const uint32_t *ids, size_t n, float *out);
/* TreeDecoder::last_hidden_states_multi (quantized_llama.rs:221-250):
 * out_final [hidden], out_layers [n_layers_requested][hidden].  Layers may repeat;
 * at most max(n_layers, 16) of them (SD_ERR_ARG beyond). */
sd_status sd_last_hidden_states_multi(sd_model *m, const uint32_t *layers, size_t n_layers, float *out_final,
                                      float *out_layers);
/* TreeDecoder::apply_lm_head (quantized_llama.rs:112-122): hidden [rows][hidden] -> out [rows][vocab].
 * A &self method in the reference (model/mod.rs:148): it runs on buffers of its
 * own and leaves the last verify pass (its logits rows, sd_last_argmax, device
 * acceptance) and the decoder state as they were.  embed_tokens likewise. */
sd_status sd_apply_lm_head(sd_model *m, const float *hidden, size_t rows, float *out);
/* TreeDecoder::embed_tokens (quantized_llama.rs:258-260 via ModelWeights::embed_tokens): out [n][hidden]. */
sd_status sd_embed_tokens(sd_model *m, const uint32_t *ids, size_t n, float *out);
size_t sd_num_hidden_layers(const sd_model *m);               /* TreeDecoder::num_hidden_layers */
size_t sd_hidden_size(const sd_model *m);                     /* LlamaQuantDecoder::hidden_size */

/* ---- device acceptance (the logits never leave HBM) ------------------------- */
/* batched_logits + the greedy walk of vanilla.rs:178-210 at temperature 0:
 * commits = drafts[..a] ++ [argmax(row a)], a = accepted drafts.  State as
 * after sd_batched_logits; the caller re-anchors with rollback_to + observe
 * (vanilla.rs:219-223).  commits has room for k+1 entries. */
sd_status sd_verify_greedy_linear(sd_model *m, const uint32_t *drafts, size_t k, uint32_t *commits,
                                  size_t *n_commit, size_t *n_accepted);
/* tree_logits_keep_kv + the greedy longest-path walk of eagle.rs:605-661
 * (eagle3.rs:714-756) + the commit composition of eagle.rs:664-732
 * (eagle3.rs:758-782):
 *  - path = accepted node indices from the root (room for n), bonus = argmax
 *    of the deepest accepted row;
 *  - committed (room for n; NULL to skip) = the path's tokens (root excluded)
 *    followed by the bonus, cut after the first token of the decoder's EOS set
 *    (sd_set_eos_token_ids); stop = 1 when that set was hit (the caller's
 *    loop ends after this round);
 *  - keep_len: commit path[0 .. keep_len) (plus bonus_node when >= 0) with
 *    sd_commit_tree_path.  An EOS among the path's tokens keeps the root and
 *    the path up to the EOS node, bonus_node = -1 and no bonus forward
 *    follows; otherwise keep_len = path_len and bonus_node = the first child
 *    of the deepest node carrying the bonus token or -1 (eagle.rs:700-709;
 *    always -1 when strict), and the caller observes the bonus when it is -1.
 * strict != 0 takes row 0 from next_logits (EagleRunConfig::strict_root_gemv). */
sd_status sd_verify_greedy_tree(sd_model *m, const uint32_t *tokens, const uint32_t *parents, size_t n,
                                int32_t strict, uint32_t *path, size_t *path_len, uint32_t *bonus,
                                int32_t *bonus_node, uint32_t *committed, size_t *n_committed, size_t *keep_len,
                                int32_t *stop);
/* First-max argmax of each row of the last verify pass (eagle.rs:626-637 fold). */
sd_status sd_last_argmax(sd_model *m, int32_t *out, size_t n);

/* batched_logits + the rejection-sampling walk of run_vanilla_sd
 * (methods/vanilla.rs:178-210) on the device: for draft i, p = softmax of row i
 * at `temperature` (sampling/tokens.rs:15-55), q = q_rows[i][drafts[i]];
 * accept iff q <= 0 or uniforms[used++] <= min(1, p/q) (vanilla.rs:59-73); on
 * the first rejection one token is drawn with uniforms[used++] from
 * max(0, p - q_rows[i]) renormalised (vanilla.rs:83-106, tokens.rs:99-120)
 * and the walk stops; after k accepted drafts the bonus is drawn from row k.
 * max_commit (0 = none) stops after that many accepted drafts with no final
 * draw (the max_new_tokens checks of vanilla.rs:190, 206).  q_rows [k][vocab]
 * and uniforms (>= k + 1 values) are host arrays; commits has room for k + 1.
 * State afterwards is that of sd_batched_logits; the caller re-anchors with
 * sd_rollback_to(len + n_accepted) + sd_observe(commits + n_accepted)
 * (vanilla.rs:219-223).  SD_ERR_SAMPLING for the reference's softmax /
 * adjusted-distribution errors and invalid temperatures. */
sd_status sd_verify_rejection_linear(sd_model *m, const uint32_t *drafts, size_t k, const float *q_rows,
                                     const float *uniforms, size_t n_uniforms, float temperature, size_t max_commit,
                                     uint32_t *commits, size_t *n_commit, size_t *n_accepted, size_t *n_used);
/* tree_logits_keep_kv + rejection sampling over the tree.  The reference has no
 * tree rejection rule (run_eagle / run_eagle3 ignore the temperature,
 * eagle.rs:739-740, eagle3.rs:789); this one reduces to the linear walk above
 * on a chain: the children of a node are tested in BFS order with the rule of
 * vanilla.rs:59-73 against the node's current distribution p (softmax of its
 * row) and its current draft distribution q; a rejection replaces p by
 * max(0, p - q) renormalised before the next sibling is tested; if no child is
 * accepted the final token is drawn from the current p, after a leaf from the
 * leaf's row.  The committed token follows the target distribution only when
 * the siblings were drawn as `siblings` states:
 *  - siblings = 0: i.i.d. draws from q_rows[q_row_of[node]] (with
 *    replacement); q stays that row for every sibling;
 *  - siblings = 1: draws without replacement from that row (distinct
 *    tokens); after each rejected token x, q(x) is set to 0 and q
 *    renormalised over the remaining mass before the next sibling.
 * Deterministic top-k siblings meet neither precondition.  At most 16
 * children per node (SD_ERR_UNSUPPORTED beyond).  q_rows has q_rows_n rows of q_vocab entries: q_vocab = vocab
 * (target ids) or the draft vocabulary of sd_set_d2t (target id x reads entry
 * t2d(x), 0 where unreachable).  use_t2d masks target entries unreachable
 * through d2t to -inf first (mask_target_logits, eagle3.rs:498-513).
 * uniforms: >= n values.  path receives the accepted node indices from the
 * root (room for n), token the final draw or -1 (max_commit reached). */
sd_status sd_verify_rejection_tree(sd_model *m, const uint32_t *tokens, const uint32_t *parents, size_t n,
                                   const float *q_rows, size_t q_rows_n, size_t q_vocab, const int32_t *q_row_of,
                                   const float *uniforms, size_t n_uniforms, float temperature, int32_t use_t2d,
                                   int32_t siblings, size_t max_commit, uint32_t *path, size_t *path_len,
                                   int32_t *token, size_t *n_used);
/* The two rejection verifies above with the draft rows already in device
 * memory (q_rows_dev: [k][vocab] or [q_rows_n][q_vocab] f32, device memory of
 * this model's GPU, e.g. written there by the draft model), so that nothing
 * of them crosses PCIe.  The rows must be complete before the call (the
 * library reads them on its own stream).  SD_ERR_ARG for a pointer that is
 * not device memory of this GPU.  No counterpart in the reference: it is the
 * same walk as sd_verify_rejection_linear (vanilla.rs:178-210) /
 * sd_verify_rejection_tree, for callers whose draft side runs on the GPU. */
sd_status sd_verify_rejection_linear_device_q(sd_model *m, const uint32_t *drafts, size_t k, const float *q_rows_dev,
                                              const float *uniforms, size_t n_uniforms, float temperature,
                                              size_t max_commit, uint32_t *commits, size_t *n_commit,
                                              size_t *n_accepted, size_t *n_used);
sd_status sd_verify_rejection_tree_device_q(sd_model *m, const uint32_t *tokens, const uint32_t *parents, size_t n,
                                            const float *q_rows_dev, size_t q_rows_n, size_t q_vocab,
                                            const int32_t *q_row_of, const float *uniforms, size_t n_uniforms,
                                            float temperature, int32_t use_t2d, int32_t siblings, size_t max_commit,
                                            uint32_t *path, size_t *path_len, int32_t *token, size_t *n_used);
/* EAGLE-3 vocabulary map (Eagle3DraftCandle's d2t, eagle3.rs:377-397): d2t[draft id]
 * = absolute target id; entries outside [0, vocab) are skipped; the inverse
 * keeps the last draft id of a target id (HashMap::insert). */
sd_status sd_set_d2t(sd_model *m, const int64_t *d2t, size_t n);
/* draft_to_target_token (eagle3.rs:476-484): SD_ERR_SAMPLING for an id past the table. */
sd_status sd_draft_to_target(sd_model *m, const uint32_t *draft_ids, size_t n, uint32_t *out);
/* t2d_mask (eagle3.rs:495-497): out[i] = 1 iff target id i is reachable; returns
 * the mask length (vocab), 0 without a d2t table; copies min(cap, vocab). */
size_t sd_t2d_mask(const sd_model *m, uint8_t *out, size_t cap);

/* ---- synthetic state and measurement ---------------------------------------- */
/* Sets history = ids and fills KV rows [0, n) with seeded N(0,1)-like fp16
 * values; the next-token logits cache is invalid afterwards. */
sd_status sd_prime_synthetic(sd_model *m, const uint32_t *ids, size_t n, uint64_t kv_seed);
/* Enables (1) / disables (0) HIP-event timing, on the handle's stream, of every
 * quantised matmul launch and of every layer's attention. */
sd_status sd_profile_enable(sd_model *m, int32_t on);
/* Reads and clears the timed launches: class ids (0 qkv, 1 wo, 2 gate_up,
 * 3 down, 4 lm_head, 5 attn), algorithmic bytes (weight blocks for the
 * matmuls, K and V rows for attention) and milliseconds.  Returns the number of
 * entries written. */
size_t sd_profile_read(sd_model *m, int32_t *cls, double *bytes, float *ms, size_t cap);
sd_status sd_synchronize(sd_model *m);
/* sd_model_qmatmul without any allocation, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  No counterpart in the reference.  x_dev [rows][K]
 * f32 and y_dev [rows][N] f32 are device buffers owned by the caller; the
 * fp16 activations are staged in a scratch array that every GPU the library
 * runs on holds once, 4 MiB (rows * K * 2 bytes must fit: SD_ERR_ARG beyond;
 * rows <= 128).  The call enqueues on `stream` (a hipStream_t; NULL = the
 * handle's own stream) and returns without waiting.  All calls on one GPU
 * share its scratch: calls that overlap on one GPU (other streams, other
 * threads, other handles on that GPU) race, so serialise them. */
sd_status sd_model_qmatmul_noalloc(sd_model *m, int32_t layer, int32_t kind, const float *x_dev, size_t rows,
                                   float *y_dev, void *stream);

/* Microbenchmark of one dequant-matmul launch of layer `layer`: kind is a
 * matrix kind, SD_BENCH_QKV (fused Q/K/V) or SD_BENCH_GATE_UP (fused gate/up +
 * SiLU), at `rows` activation rows; *us = mean microseconds per launch over
 * `iters` back-to-back launches timed with HIP events, *bytes = algorithmic
 * bytes per launch (weight blocks + activations in + outputs).  layer =
 * SD_BENCH_ALL_LAYERS cycles the launches over every layer's matrix, so each
 * launch streams weights the previous ones did not leave in the caches (the
 * situation inside a forward pass). */
enum { SD_BENCH_QKV = 100, SD_BENCH_GATE_UP = 101, SD_BENCH_ALL_LAYERS = -2 };
sd_status sd_bench_qmatmul(sd_model *m, int32_t layer, int32_t kind, size_t rows, int32_t iters, double *us,
                           double *bytes);
/* Copies n fp16 cache rows [pos0, pos0+n) of one (layer, K=0/V=1, kv head):
 * out [n][head_dim] (checks of the in-place KV layout). */
sd_status sd_read_kv_rows(sd_model *m, int32_t layer, int32_t which, int32_t head, size_t pos0, size_t n,
                          uint16_t *out);
/* Number of positions currently held in the KV cache. */
size_t sd_cache_len(const sd_model *m);

/* ---- device weight layout (host only; no GPU needed) ---------------------------- */
/* The library keeps quantised matrices in a tile-interleaved order: each
 * 16-row x 256-column tile block is rearranged so that every load of the
 * matmul kernel's MFMA lane mapping reads contiguous bytes (same byte count as
 * GGUF).  sd_model_set_tensor repacks on the device; these do it on the host,
 * e.g. for a loader that streams a GGUF file straight into the device layout.
 * rows must be a multiple of 16 and K of 256.  GGUF: row-major blocks as in
 * the file; tiles: rows/16 x K/256 tile blocks, tile-major. */
sd_status sd_repack_gguf(int32_t fmt, const void *gguf, size_t rows, size_t K, void *out);
sd_status sd_unpack_tiles(int32_t fmt, const void *tiles, size_t rows, size_t K, void *gguf_out);
/* The four 32-bit words (two fp16 codes each, slots 0-1, 2-3, 4-5, 6-7) that
 * lane `lane` of the matmul builds for K-chunk `chunk` from one tile block: a
 * layout self-check hook; codes are 1024 + q (0x6400 | q) for slots 0-3 and
 * 64 + q for slots 4-7 (1024 + q + 128 throughout for Q8_0). */
sd_status sd_lane_codes(int32_t fmt, const void *tile_block, int32_t lane, int32_t chunk, uint32_t *out);

/* ---- GGUF files (parsing is host only; sd_model_load_gguf uploads) -------------- */
/* An opened .gguf file: header, metadata and tensor directory, read as
 * gguf_file::Content::read (candle-core 0.8.4) does at quantized_llama.rs:63-65
 * / quantized_qwen2.rs:61-63 (GGUF v1-v3; general.alignment, default 32).  The
 * file stays memory-mapped until sd_gguf_close.  A malformed file is
 * SD_ERR_BACKEND (Error::Candle), never an out-of-range read. */
typedef struct sd_gguf sd_gguf;
sd_status sd_gguf_open(const char *path, sd_gguf **out);
void sd_gguf_close(sd_gguf *g);
/* The hyper-parameters ModelWeights::from_gguf reads
 * (quantized_llama_local.rs:222-240, quantized_qwen2_local.rs:215-230): arch
 * SD_ARCH_LLAMA / SD_ARCH_QWEN2 picks the key prefix ("llama." / "qwen2.", the
 * decoder type the caller builds), -1 takes it from general.architecture.
 * Missing keys fail in the reference's order ("cannot find <key> in GGUF
 * metadata"); rope.freq_base defaults to 10000; head_dim = embedding_length /
 * head_count; ffn and vocab are the rows of blk.0.ffn_gate.weight and
 * token_embd.weight; tied_output = 1 when output.weight is absent (the
 * fallback at quantized_llama_local.rs:248-252).  ctx_len is set to
 * context_length, max_batch to 128, device to 0: the caller may change these
 * three before sd_model_create. */
sd_status sd_gguf_config(const sd_gguf *g, int32_t arch, sd_config *cfg);
/* File layout: GGUF version, alignment and the absolute offset of the data section. */
sd_status sd_gguf_layout(const sd_gguf *g, uint32_t *version, uint64_t *alignment, uint64_t *data_offset);
size_t sd_gguf_tensor_count(const sd_gguf *g);
/* One tensor-directory entry: GGML type, dims (ne[0] the contiguous one; the
 * unused ones are 1), offset from the data section.  SD_ERR_BACKEND "cannot
 * find tensor info for <name>" if absent (Content::tensor). */
sd_status sd_gguf_tensor_info(const sd_gguf *g, const char *name, int32_t *type, int32_t *n_dims, uint64_t *ne,
                              uint64_t *offset);
/* Uploads every tensor ModelWeights::from_gguf loads
 * (quantized_llama_local.rs:242-281, quantized_qwen2_local.rs:232-283), in
 * its order; F16/BF16 norms and biases are widened to F32 as
 * RmsNorm::from_qtensor / dequantize do.  All tensors are checked (present,
 * shape, Q4_K/Q5_K/Q6_K/Q8_0 matrices, data inside the file) before the first
 * upload; the model must have been created from this file's config (ctx_len,
 * max_batch and device aside), else SD_ERR_ARG. */
sd_status sd_model_load_gguf(sd_model *m, const sd_gguf *g);

/* ---- draft-tree builders (host only; no GPU needed) ---------------------------- */
/* build_cartesian_tree (methods/medusa.rs:172-193): step d has branching[d]
 * candidate tokens, stored back to back in cand[]; layer d+1 hangs every
 * candidate of step d under every node of layer d, in BFS order.  *n receives
 * the node count 1 + b0 + b0*b1 + ...; with tokens or parents NULL only the
 * size is returned.  SD_ERR_ARG if the tree exceeds cap. */
sd_status sd_tree_cartesian(uint32_t root, const uint32_t *cand, const uint32_t *branching, size_t depth,
                            uint32_t *tokens, uint32_t *parents, size_t cap, size_t *n);
/* prune_cartesian_tree (methods/eagle.rs:763-845): keeps the max_total - 1
 * non-root nodes with the highest summed per-step log-prob (log_probs holds
 * branching[d] values for step d, back to back; equal scores keep BFS order)
 * plus their ancestors, re-emitted stably by depth.  A tree of at most
 * max_total nodes is returned unchanged.  out_* need room for n entries: the
 * ancestor closure can exceed max_total when log-probs are not all <= 0. */
sd_status sd_tree_prune(const uint32_t *tokens, const uint32_t *parents, size_t n, const float *log_probs,
                        const uint32_t *branching, size_t depth, size_t max_total, uint32_t *out_tokens,
                        uint32_t *out_parents, size_t *n_out);

/* ---- EAGLE-3 draft (the draft side feeding the tree) ------------------------- */
/* Eagle3DraftCandle (crates/speculate/src/methods/eagle3.rs:307-516) on the
 * device: the f16 midlayer, norm + lm_head, the per-step top-k, log-probs and
 * d2t of run_eagle3 (:598-673).  Tensors are the checkpoint's (f16, row-major
 * [out][in]); d2t is int64 [draft_vocab]. */
typedef struct sd_draft3 sd_draft3;
typedef struct {
    int32_t hidden, n_heads, n_kv_heads, ffn, draft_vocab, target_vocab;
    float rms_eps, rope_theta;
    int32_t max_pos; /* rows of the RoPE tables (Eagle3DraftConfig::max_position_embeddings) */
    int32_t device;
} sd_draft3_config;
enum {
    SD_D3_FC = 0, SD_D3_Q, SD_D3_K, SD_D3_V, SD_D3_O, SD_D3_GATE, SD_D3_UP, SD_D3_DOWN, SD_D3_LM_HEAD,
    SD_D3_INPUT_NORM, SD_D3_HIDDEN_NORM, SD_D3_POST_NORM, SD_D3_NORM, SD_D3_D2T
};
sd_status sd_draft3_create(const sd_draft3_config *cfg, sd_draft3 **out);
void sd_draft3_destroy(sd_draft3 *d);
/* bytes of one tensor kind (0 for a bad handle or kind) */
size_t sd_draft3_tensor_bytes(const sd_draft3 *d, int32_t kind);
/* Eagle3DraftCandle::from_var_builder (:353-410): one tensor at a time */
sd_status sd_draft3_set_tensor(sd_draft3 *d, int32_t kind, const void *data, size_t bytes);
sd_status sd_draft3_get_tensor(const sd_draft3 *d, int32_t kind, void *data, size_t bytes);
/* seeded synthetic weights (N(0, std) f16 matrices, norms 1 + N(0, 0.1), d2t
 * distinct target ids): benchmarks and tests */
sd_status sd_draft3_synthesize(sd_draft3 *d, uint64_t seed, float weight_std);
/* Eagle3DraftCandle::reset (:416-418): clears the draft's own KV cache */
sd_status sd_draft3_reset(sd_draft3 *d);
/* forward_hidden (:433-450) + apply_norm_lm_head (:451-454) of one step:
 * hidden_in f32 [n_in] with n_in = 3 * hidden (fc applied) or hidden (the
 * previous step's output), input_emb f32 [hidden]; out_hidden [hidden] (the
 * pre-norm midlayer output, f16 values), out_logits [draft_vocab] (f16 values)
 * or NULL.  Appends the step to the draft's cache (at most 16 steps between
 * resets). */
sd_status sd_draft3_forward(sd_draft3 *d, const float *hidden_in, size_t n_in, const float *input_emb,
                            size_t position, float *out_hidden, float *out_logits);
/* One draft round of run_eagle3 (:598-673) against the target m, on the
 * device with no host round trip between steps: the hidden states after
 * `layers` (3 of them) of m's last committed token
 * (TreeDecoder::last_hidden_states_multi), then `depth` (<= 16) steps, each
 * embedding the current token through m's token table, running the midlayer
 * and norm + lm_head, and taking the top top_k[s] (<= 8) draft ids by value
 * (index ascending on ties, medusa.rs:477-487) with their log-probs
 * l - logsumexp(l) and their d2t target ids; the top-1 target id is the next
 * step's token.  Outputs [depth][8] each (entries past top_k[s] unset).
 * The decoder's history and cache are as before the call.  Positions run
 * from the history length; they must stay below max_pos (SD_ERR_ARG). */
sd_status sd_draft3_round(sd_draft3 *d, sd_model *m, const uint32_t *layers, size_t depth, const int32_t *top_k,
                          int32_t *target_ids, int32_t *draft_ids, float *log_probs);

/* EagleDraftCandle (crates/speculate/src/methods/eagle.rs:306-428), the
 * EAGLE-2 draft, on the device: its own token table, fc over [target hidden,
 * token embedding], one Llama block without input norm, f16 throughout; its
 * logits come from the target's lm_head (apply_lm_head). */
typedef struct sd_draft2 sd_draft2;
typedef struct {
    int32_t hidden, n_heads, n_kv_heads, ffn, vocab; /* vocab: the target's (<= 262144) */
    float rms_eps, rope_theta;
    int32_t max_pos; /* rows of the RoPE tables (EagleDraftConfig::max_position_embeddings) */
    int32_t device;
} sd_draft2_config;
enum {
    SD_D2_EMBED = 0, SD_D2_FC, SD_D2_Q, SD_D2_K, SD_D2_V, SD_D2_O, SD_D2_GATE, SD_D2_UP, SD_D2_DOWN,
    SD_D2_POST_NORM
};
sd_status sd_draft2_create(const sd_draft2_config *cfg, sd_draft2 **out);
void sd_draft2_destroy(sd_draft2 *d);
/* bytes of one tensor kind (0 for a bad handle or kind) */
size_t sd_draft2_tensor_bytes(const sd_draft2 *d, int32_t kind);
/* EagleDraftCandle::from_var_builder (:343-371): f16 row-major tensors
 * ([out][in]; embed_tokens [vocab][hidden]; post_attention_layernorm [hidden]) */
sd_status sd_draft2_set_tensor(sd_draft2 *d, int32_t kind, const void *data, size_t bytes);
sd_status sd_draft2_get_tensor(const sd_draft2 *d, int32_t kind, void *data, size_t bytes);
/* seeded synthetic weights (N(0, std) f16 matrices and table, norm 1 + N(0, 0.1)) */
sd_status sd_draft2_synthesize(sd_draft2 *d, uint64_t seed, float weight_std);
/* EagleDraftCandle::reset (:373-375): clears the draft's own KV cache */
sd_status sd_draft2_reset(sd_draft2 *d);
/* EagleDraftCandle::forward (:390-427) of one position: target_hidden f32
 * [hidden] (the target's final-norm hidden state or the previous step's
 * output), token < vocab, the RoPE position (< max_pos); out f32 [hidden]
 * (f16 values).  Appends the step to the draft's cache (at most 16 steps
 * between resets). */
sd_status sd_draft2_forward(sd_draft2 *d, const float *target_hidden, size_t n, uint32_t token, size_t position,
                            float *out_hidden);
/* The draft half of one run_eagle iteration (:519-575) against the target m,
 * on the device: `depth` (<= 16) steps from target_hidden (f32 [hidden], the
 * committed token's final-norm hidden state, as observe_returning_last_hidden
 * returns it) and m's last committed token, each a draft forward, m's lm_head
 * on its output, and the top top_k[s] (<= 8) ids by value (index ascending on
 * ties) with their log-probs l - logsumexp(l); the top-1 id and the step's
 * output feed the next step.  Outputs [depth][8] (entries past top_k[s]
 * unset).  m's history and cache are untouched; positions run from the
 * history length and must stay below max_pos (SD_ERR_ARG). */
sd_status sd_draft2_round(sd_draft2 *d, sd_model *m, const float *target_hidden, size_t depth, const int32_t *top_k,
                          int32_t *ids, float *log_probs);

#ifdef __cplusplus
}
#endif
#endif /* SPECULATE_HIP_H */
