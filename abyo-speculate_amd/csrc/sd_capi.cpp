// extern "C" boundary (include/speculate_hip.h) over Model / Decoder.
#include <cstring>
#include <memory>
#include <string>

#include "speculate_hip.h"
#include "sd_model.hpp"
#include "sd_common.hpp"
#include "sd_draft.hpp"
#include "sd_gguf.hpp"
#include "sd_qcodes.hpp"
#include "sd_tiles.hpp"

struct sd_model {
    std::unique_ptr<sd::Model> model;
    std::unique_ptr<sd::Decoder> dec;
};

struct sd_gguf {
    std::unique_ptr<sd::GgufFile> file;
};

struct sd_draft2 {
    std::unique_ptr<sd::Draft2> d;
};
struct sd_draft3 {
    std::unique_ptr<sd::Draft3> d;
};

static thread_local std::string g_err;

template <typename F> static sd_status guard(F &&f) {
    try {
        f();
        return SD_OK;
    } catch (const sd::SamplingError &e) {
        g_err = e.what();
        return SD_ERR_SAMPLING;
    } catch (const sd::RollbackError &e) {
        g_err = e.what();
        return SD_ERR_ROLLBACK;
    } catch (const sd::ArgError &e) {
        g_err = e.what();
        return SD_ERR_ARG;
    } catch (const sd::UnsupportedError &e) {
        g_err = e.what();
        return SD_ERR_UNSUPPORTED;
    } catch (const sd::BackendError &e) {
        g_err = e.what();
        return SD_ERR_BACKEND;
    } catch (const std::exception &e) {
        g_err = e.what();
        return SD_ERR_BACKEND;
    }
}

static void need(const sd_model *m) {
    if (!m || !m->model) throw sd::ArgError("null model handle");
}
static void need_weights(const sd_model *m) {
    need(m);
    if (!m->model->weights_ready()) throw sd::ArgError("model weights are not fully set");
}
static void setdev(sd_model *m) { SD_HIP_CHECK(hipSetDevice(m->model->cfg.device)); }

extern "C" {

const char *sd_last_error(void) { return g_err.c_str(); }

sd_status sd_model_create(const sd_config *cfg, sd_model **out) {
    return guard([&] {
        if (!cfg || !out) throw sd::ArgError("null argument");
        *out = nullptr;
        sd::ModelCfg c;
        c.arch = cfg->arch;
        if (c.arch != SD_ARCH_LLAMA && c.arch != SD_ARCH_QWEN2) throw sd::ArgError("unknown arch");
        c.n_layers = cfg->n_layers;
        c.hidden = cfg->hidden;
        c.n_heads = cfg->n_heads;
        c.n_kv_heads = cfg->n_kv_heads;
        c.head_dim = cfg->head_dim;
        c.ffn = cfg->ffn;
        c.vocab = cfg->vocab;
        c.rope_theta = cfg->rope_theta;
        c.rms_eps = cfg->rms_eps;
        c.ctx_len = cfg->ctx_len;
        c.max_batch = cfg->max_batch;
        c.tied_output = cfg->tied_output;
        c.device = cfg->device;
        if (c.hidden != c.n_heads * c.head_dim) throw sd::UnsupportedError("hidden must equal n_heads * head_dim");
        auto h = std::make_unique<sd_model>();
        h->model = std::make_unique<sd::Model>(c);
        h->dec = std::make_unique<sd::Decoder>(h->model.get());
        // set-up of the allocation-free entry points: this device's scratch
        // address, resolved while the device is current (Model set it)
        sd::noalloc_scratch(c.device);
        *out = h.release();
    });
}

void sd_model_destroy(sd_model *m) { delete m; }

sd_status sd_model_set_tensor(sd_model *m, int32_t layer, int32_t kind, int32_t fmt, const void *data, size_t bytes) {
    return guard([&] {
        need(m);
        if (!data) throw sd::ArgError("null data");
        m->model->set_tensor(layer, kind, fmt, data, bytes);
        m->dec->last_valid = false;
    });
}

sd_status sd_model_get_tensor(sd_model *m, int32_t layer, int32_t kind, void *out, size_t bytes) {
    return guard([&] {
        need(m);
        if (!out) throw sd::ArgError("null output");
        m->model->get_tensor(layer, kind, out, bytes);
    });
}

sd_status sd_model_tensor_info(sd_model *m, int32_t layer, int32_t kind, int32_t *fmt, int32_t *rows, int32_t *cols,
                               size_t *gguf_bytes) {
    return guard([&] {
        need(m);
        int f, r, k;
        size_t b;
        m->model->tensor_info(layer, kind, &f, &r, &k, &b);
        if (fmt) *fmt = f;
        if (rows) *rows = r;
        if (cols) *cols = k;
        if (gguf_bytes) *gguf_bytes = b;
    });
}

sd_status sd_model_synthesize(sd_model *m, int32_t mix, uint64_t seed, float stdv) {
    return guard([&] {
        need(m);
        m->model->synthesize(mix, seed, stdv);
        m->dec->last_valid = false;
    });
}

sd_status sd_gguf_open(const char *path, sd_gguf **out) {
    return guard([&] {
        if (!path || !out) throw sd::ArgError("null argument");
        *out = nullptr;
        auto g = std::make_unique<sd_gguf>();
        g->file = std::make_unique<sd::GgufFile>(path);
        *out = g.release();
    });
}

void sd_gguf_close(sd_gguf *g) { delete g; }

static const sd::GgufFile &gfile(const sd_gguf *g) {
    if (!g || !g->file) throw sd::ArgError("null gguf handle");
    return *g->file;
}

sd_status sd_gguf_config(const sd_gguf *g, int32_t arch, sd_config *cfg) {
    return guard([&] {
        if (!cfg) throw sd::ArgError("null argument");
        const sd::ModelCfg c = gfile(g).config(arch);
        sd_config o;
        o.arch = c.arch;
        o.n_layers = c.n_layers;
        o.hidden = c.hidden;
        o.n_heads = c.n_heads;
        o.n_kv_heads = c.n_kv_heads;
        o.head_dim = c.head_dim;
        o.ffn = c.ffn;
        o.vocab = c.vocab;
        o.rope_theta = c.rope_theta;
        o.rms_eps = c.rms_eps;
        o.ctx_len = c.ctx_len;
        o.max_batch = c.max_batch;
        o.tied_output = c.tied_output;
        o.device = c.device;
        *cfg = o;
    });
}

sd_status sd_gguf_layout(const sd_gguf *g, uint32_t *version, uint64_t *alignment, uint64_t *data_offset) {
    return guard([&] {
        const sd::GgufFile &f = gfile(g);
        if (version) *version = f.version;
        if (alignment) *alignment = f.alignment;
        if (data_offset) *data_offset = f.data_start;
    });
}

size_t sd_gguf_tensor_count(const sd_gguf *g) { return g && g->file ? g->file->tensors.size() : 0; }

sd_status sd_gguf_tensor_info(const sd_gguf *g, const char *name, int32_t *type, int32_t *n_dims, uint64_t *ne,
                              uint64_t *offset) {
    return guard([&] {
        if (!name) throw sd::ArgError("null name");
        const sd::GgufTensor &t = gfile(g).tensor(name);
        if (type) *type = (int32_t)t.type;
        if (n_dims) *n_dims = (int32_t)t.n_dims;
        if (ne)
            for (int d = 0; d < 4; d++) ne[d] = t.ne[d];
        if (offset) *offset = t.offset;
    });
}

sd_status sd_model_load_gguf(sd_model *m, const sd_gguf *g) {
    return guard([&] {
        need(m);
        const sd::GgufFile &f = gfile(g);
        f.load(*m->model);
        m->dec->last_valid = false;
    });
}

sd_status sd_model_dequant_tensor(sd_model *m, int32_t layer, int32_t kind, float *out) {
    return guard([&] {
        need(m);
        if (!out) throw sd::ArgError("null output");
        m->model->dequant_tensor(layer, kind, out);
    });
}

sd_status sd_model_qmatmul(sd_model *m, int32_t layer, int32_t kind, const float *x, size_t rows, float *y) {
    return guard([&] {
        need(m);
        if (!x || !y) throw sd::ArgError("null argument");
        m->model->qmatmul(layer, kind, x, (int)rows, y);
    });
}

sd_status sd_model_qmatmul_noalloc(sd_model *m, int32_t layer, int32_t kind, const float *x_dev, size_t rows,
                                   float *y_dev, void *stream) {
    return guard([&] {
        need(m);
        if (!x_dev || !y_dev) throw sd::ArgError("null argument");
        if (rows < 1 || rows > 128) throw sd::ArgError("rows must be in [1, 128]");
        setdev(m);
        // resolved at sd_model_create for this device; a kept pointer, no allocation
        void *scr = sd::noalloc_scratch(m->model->cfg.device);
        m->model->qmatmul_into(layer, kind, x_dev, (int)rows, y_dev, (hipStream_t)stream, scr,
                               sd::kNoAllocScratchBytes);
    });
}

sd_status sd_bench_qmatmul(sd_model *m, int32_t layer, int32_t kind, size_t rows, int32_t iters, double *us,
                           double *bytes) {
    return guard([&] {
        need_weights(m);
        if (!us) throw sd::ArgError("null argument");
        *us = m->model->bench_qmatmul(layer, kind, (int)rows, iters, bytes);
    });
}

size_t sd_vocab_size(const sd_model *m) { return m && m->model ? (size_t)m->model->cfg.vocab : 0; }
size_t sd_history_len(const sd_model *m) { return m && m->dec ? m->dec->history.size() : 0; }
size_t sd_history(const sd_model *m, uint32_t *out, size_t cap) {
    if (!m || !m->dec) return 0;
    const size_t n = std::min(cap, m->dec->history.size());
    if (out && n) std::memcpy(out, m->dec->history.data(), n * 4);
    return n;
}
void sd_reset(sd_model *m) {
    if (m && m->dec) m->dec->reset();
}
size_t sd_num_hidden_layers(const sd_model *m) { return m && m->model ? (size_t)m->model->cfg.n_layers : 0; }
size_t sd_hidden_size(const sd_model *m) { return m && m->model ? (size_t)m->model->cfg.hidden : 0; }

sd_status sd_observe(sd_model *m, const uint32_t *ids, size_t n) {
    return guard([&] {
        need_weights(m);
        if (n && !ids) throw sd::ArgError("null ids");
        setdev(m);
        m->dec->observe(ids, n);
    });
}

sd_status sd_next_logits(sd_model *m, float *out) {
    return guard([&] {
        need_weights(m);
        setdev(m);
        m->dec->next_logits(out);
    });
}

sd_status sd_batched_logits(sd_model *m, const uint32_t *drafts, size_t k, float *out) {
    return guard([&] {
        need_weights(m);
        if (k && !drafts) throw sd::ArgError("null drafts");
        setdev(m);
        m->dec->batched_logits(drafts, k, out);
    });
}

sd_status sd_rollback_to(sd_model *m, size_t len) {
    return guard([&] {
        need(m);
        m->dec->rollback_to(len);
    });
}

sd_status sd_set_eos_token_ids(sd_model *m, const uint32_t *ids, size_t n) {
    return guard([&] {
        need(m);
        if (n && !ids) throw sd::ArgError("null ids");
        m->dec->eos.assign(ids, ids + n);
    });
}

size_t sd_eos_token_ids(const sd_model *m, uint32_t *out, size_t cap) {
    if (!m || !m->dec) return 0;
    const size_t n = std::min(cap, m->dec->eos.size());
    if (out && n) std::memcpy(out, m->dec->eos.data(), n * 4);
    return m->dec->eos.size();
}

sd_status sd_tree_logits_keep_kv(sd_model *m, const uint32_t *tokens, const uint32_t *parents, size_t n,
                                 float *out_logits, float *out_hidden) {
    return guard([&] {
        need_weights(m);
        if (!tokens || !parents) throw sd::ArgError("null tree");
        setdev(m);
        m->dec->tree_logits_keep_kv(tokens, parents, n, out_logits, out_hidden);
    });
}

sd_status sd_tree_logits(sd_model *m, const uint32_t *tokens, const uint32_t *parents, size_t n, float *out_logits) {
    return guard([&] {
        need_weights(m);
        if (!tokens || !parents) throw sd::ArgError("null tree");
        setdev(m);
        m->dec->tree_logits(tokens, parents, n, out_logits);
    });
}

sd_status sd_commit_tree_path(sd_model *m, const uint32_t *tokens, const uint32_t *parents, size_t n,
                              const uint32_t *accepted, size_t n_accepted) {
    return guard([&] {
        need_weights(m);
        if (!tokens || !parents || (n_accepted && !accepted)) throw sd::ArgError("null argument");
        setdev(m);
        m->dec->commit_tree_path(tokens, parents, n, accepted, n_accepted);
    });
}

sd_status sd_last_hidden_state(sd_model *m, float *out) {
    return guard([&] {
        need_weights(m);
        setdev(m);
        m->dec->last_hidden_state(out);
    });
}

sd_status sd_observe_returning_last_hidden(sd_model *m, const uint32_t *ids, size_t n, float *out) {
    return guard([&] {
        need_weights(m);
        if (n && !ids) throw sd::ArgError("null ids");
        setdev(m);
        m->dec->observe_returning_last_hidden(ids, n, out);
    });
}

sd_status sd_last_hidden_states_multi(sd_model *m, const uint32_t *layers, size_t n_layers, float *out_final,
                                      float *out_layers) {
    return guard([&] {
        need_weights(m);
        if (n_layers && !layers) throw sd::ArgError("null layers");
        setdev(m);
        m->dec->last_hidden_states_multi(layers, n_layers, out_final, out_layers);
    });
}

sd_status sd_apply_lm_head(sd_model *m, const float *hidden, size_t rows, float *out) {
    return guard([&] {
        need_weights(m);
        if (!hidden || !out) throw sd::ArgError("null argument");
        setdev(m);
        m->model->lm_head_rows(hidden, (int)rows, out);
    });
}

sd_status sd_embed_tokens(sd_model *m, const uint32_t *ids, size_t n, float *out) {
    return guard([&] {
        need_weights(m);
        if (!ids || !out) throw sd::ArgError("null argument");
        setdev(m);
        std::vector<int> v(ids, ids + n);
        for (size_t i = 0; i < n; i++)
            if (ids[i] >= (uint32_t)m->model->cfg.vocab) throw sd::ArgError("token id out of range");
        m->model->embed_rows(v.data(), (int)n, out);
    });
}

sd_status sd_verify_greedy_linear(sd_model *m, const uint32_t *drafts, size_t k, uint32_t *commits,
                                  size_t *n_commit, size_t *n_accepted) {
    return guard([&] {
        need_weights(m);
        if ((k && !drafts) || !commits || !n_commit || !n_accepted) throw sd::ArgError("null argument");
        setdev(m);
        m->dec->verify_greedy_linear(drafts, k, commits, n_commit, n_accepted);
    });
}

sd_status sd_verify_greedy_tree(sd_model *m, const uint32_t *tokens, const uint32_t *parents, size_t n,
                                int32_t strict, uint32_t *path, size_t *path_len, uint32_t *bonus,
                                int32_t *bonus_node, uint32_t *committed, size_t *n_committed, size_t *keep_len,
                                int32_t *stop) {
    return guard([&] {
        need_weights(m);
        if (!tokens || !parents || !path || !path_len || !bonus || !bonus_node || !n_committed || !keep_len || !stop)
            throw sd::ArgError("null argument");
        setdev(m);
        m->dec->verify_greedy_tree(tokens, parents, n, strict, path, path_len, bonus, bonus_node, committed,
                                   n_committed, keep_len, stop);
    });
}

sd_status sd_verify_rejection_linear(sd_model *m, const uint32_t *drafts, size_t k, const float *q_rows,
                                     const float *uniforms, size_t n_uniforms, float temperature, size_t max_commit,
                                     uint32_t *commits, size_t *n_commit, size_t *n_accepted, size_t *n_used) {
    return guard([&] {
        need_weights(m);
        if ((k && (!drafts || !q_rows)) || !uniforms || !commits || !n_commit || !n_accepted || !n_used)
            throw sd::ArgError("null argument");
        setdev(m);
        m->dec->verify_rejection_linear(drafts, k, q_rows, uniforms, n_uniforms, temperature, max_commit, commits,
                                        n_commit, n_accepted, n_used);
    });
}

sd_status sd_verify_rejection_linear_device_q(sd_model *m, const uint32_t *drafts, size_t k, const float *q_rows_dev,
                                              const float *uniforms, size_t n_uniforms, float temperature,
                                              size_t max_commit, uint32_t *commits, size_t *n_commit,
                                              size_t *n_accepted, size_t *n_used) {
    return guard([&] {
        need_weights(m);
        if ((k && (!drafts || !q_rows_dev)) || !uniforms || !commits || !n_commit || !n_accepted || !n_used)
            throw sd::ArgError("null argument");
        setdev(m);
        m->dec->verify_rejection_linear(drafts, k, q_rows_dev, uniforms, n_uniforms, temperature, max_commit, commits,
                                        n_commit, n_accepted, n_used, true);
    });
}

sd_status sd_verify_rejection_tree(sd_model *m, const uint32_t *tokens, const uint32_t *parents, size_t n,
                                   const float *q_rows, size_t q_rows_n, size_t q_vocab, const int32_t *q_row_of,
                                   const float *uniforms, size_t n_uniforms, float temperature, int32_t use_t2d,
                                   int32_t siblings, size_t max_commit, uint32_t *path, size_t *path_len,
                                   int32_t *token, size_t *n_used) {
    return guard([&] {
        need_weights(m);
        if (!tokens || !parents || !q_row_of || !uniforms || !path || !path_len || !token || !n_used ||
            (q_rows_n && !q_rows))
            throw sd::ArgError("null argument");
        setdev(m);
        m->dec->verify_rejection_tree(tokens, parents, n, q_rows, q_rows_n, q_vocab, q_row_of, uniforms, n_uniforms,
                                      temperature, use_t2d, siblings, max_commit, path, path_len, token, n_used);
    });
}

sd_status sd_verify_rejection_tree_device_q(sd_model *m, const uint32_t *tokens, const uint32_t *parents, size_t n,
                                            const float *q_rows_dev, size_t q_rows_n, size_t q_vocab,
                                            const int32_t *q_row_of, const float *uniforms, size_t n_uniforms,
                                            float temperature, int32_t use_t2d, int32_t siblings, size_t max_commit,
                                            uint32_t *path, size_t *path_len, int32_t *token, size_t *n_used) {
    return guard([&] {
        need_weights(m);
        if (!tokens || !parents || !q_row_of || !uniforms || !path || !path_len || !token || !n_used ||
            (q_rows_n && !q_rows_dev))
            throw sd::ArgError("null argument");
        setdev(m);
        m->dec->verify_rejection_tree(tokens, parents, n, q_rows_dev, q_rows_n, q_vocab, q_row_of, uniforms,
                                      n_uniforms, temperature, use_t2d, siblings, max_commit, path, path_len, token,
                                      n_used, true);
    });
}

sd_status sd_set_d2t(sd_model *m, const int64_t *d2t, size_t n) {
    return guard([&] {
        need(m);
        if (!d2t) throw sd::ArgError("null d2t");
        setdev(m);
        m->dec->set_d2t(d2t, n);
    });
}

sd_status sd_draft_to_target(sd_model *m, const uint32_t *draft_ids, size_t n, uint32_t *out) {
    return guard([&] {
        need(m);
        if ((n && (!draft_ids || !out))) throw sd::ArgError("null argument");
        const auto &d2t = m->dec->d2t_host;
        if (d2t.empty()) throw sd::ArgError("no d2t table (sd_set_d2t)");
        for (size_t i = 0; i < n; i++)
            if (draft_ids[i] >= d2t.size())
                throw sd::SamplingError("draft id " + std::to_string(draft_ids[i]) + " out of range (" +
                                        std::to_string(d2t.size()) + ")");
        for (size_t i = 0; i < n; i++) out[i] = (uint32_t)d2t[draft_ids[i]];
    });
}

size_t sd_t2d_mask(const sd_model *m, uint8_t *out, size_t cap) {
    if (!m || !m->dec || m->dec->t2d_host.empty()) return 0;
    const auto &inv = m->dec->t2d_host;
    const size_t n = std::min(cap, inv.size());
    for (size_t i = 0; i < n && out; i++) out[i] = inv[i] >= 0 ? 1 : 0;
    return inv.size();
}

sd_status sd_last_argmax(sd_model *m, int32_t *out, size_t n) {
    return guard([&] {
        need(m);
        if (!out) throw sd::ArgError("null output");
        setdev(m);
        m->dec->argmax_rows(out, n);
    });
}

sd_status sd_prime_synthetic(sd_model *m, const uint32_t *ids, size_t n, uint64_t kv_seed) {
    return guard([&] {
        need(m);
        if (!ids) throw sd::ArgError("null ids");
        setdev(m);
        m->dec->prime_synthetic(ids, n, kv_seed);
    });
}

sd_status sd_profile_enable(sd_model *m, int32_t on) {
    return guard([&] {
        need(m);
        m->model->prof_on = on != 0;
    });
}

size_t sd_profile_read(sd_model *m, int32_t *cls, double *bytes, float *ms, size_t cap) {
    if (!m || !m->model) return 0;
    auto &P = m->model->prof;
    (void)hipSetDevice(m->model->cfg.device);
    (void)hipStreamSynchronize(m->model->st);
    size_t n = 0;
    for (auto &e : P) {
        if (n >= cap) break;
        float t = 0.f;
        (void)hipEventElapsedTime(&t, m->model->ev_pool[e.ev], m->model->ev_pool[e.ev + 1]);
        if (cls) cls[n] = e.cls;
        if (bytes) bytes[n] = e.bytes;
        if (ms) ms[n] = t;
        n++;
    }
    m->model->prof_reset();
    return n;
}

sd_status sd_synchronize(sd_model *m) {
    return guard([&] {
        need(m);
        setdev(m);
        m->model->sync();
    });
}

sd_status sd_read_kv_rows(sd_model *m, int32_t layer, int32_t which, int32_t head, size_t pos0, size_t n,
                          uint16_t *out) {
    return guard([&] {
        need(m);
        const sd::ModelCfg &c = m->model->cfg;
        if (!out) throw sd::ArgError("null output");
        if (layer < 0 || layer >= c.n_layers || which < 0 || which > 1 || head < 0 || head >= c.n_kv_heads)
            throw sd::ArgError("kv row selector out of range");
        if (pos0 + n > (size_t)m->model->cap) throw sd::ArgError("kv rows out of range");
        setdev(m);
        const uint16_t *base = m->model->kv + (((int64_t)layer * 2 + which) * c.n_kv_heads + head) * m->model->cap *
                                                  c.head_dim;
        // copy the whole 32-position blocks covering the rows, then gather the
        // rows out of the blocked layout (sd_common.hpp: kv_k_off / kv_v_off)
        const int64_t b0 = (int64_t)pos0 / 32, b1 = ((int64_t)(pos0 + n) + 31) / 32;
        std::vector<uint16_t> blk((size_t)(b1 - b0) * 32 * c.head_dim);
        m->model->sync();
        if (!blk.empty())
            SD_HIP_CHECK(hipMemcpy(blk.data(), base + b0 * 32 * c.head_dim, blk.size() * 2, hipMemcpyDeviceToHost));
        const int64_t off0 = b0 * 32 * c.head_dim;
        for (size_t j = 0; j < n; j++)
            for (int d = 0; d < c.head_dim; d++)
                out[j * c.head_dim + d] = blk[sd::kv_off(which, (int64_t)(pos0 + j), d, c.head_dim) - off0];
    });
}

size_t sd_cache_len(const sd_model *m) { return m && m->dec ? (size_t)m->dec->cache_len : 0; }

static int64_t quant_rows_check(int32_t fmt, size_t rows, size_t K) {
    if (fmt != SD_Q4_K && fmt != SD_Q5_K && fmt != SD_Q6_K && fmt != SD_Q8_0)
        throw sd::UnsupportedError("format must be Q4_K, Q5_K, Q6_K or Q8_0");
    if (rows == 0 || rows % 16 || K == 0 || K % 256) throw sd::ArgError("rows must be a multiple of 16 and K of 256");
    return (int64_t)(K / 256);
}

sd_status sd_repack_gguf(int32_t fmt, const void *gguf, size_t rows, size_t K, void *out) {
    return guard([&] {
        if (!gguf || !out) throw sd::ArgError("null argument");
        const int64_t nsb = quant_rows_check(fmt, rows, K);
        const int sbb = sd::fmt_sb_bytes(fmt), tbb = sd::tile_block_bytes(fmt);
        const uint8_t *src = (const uint8_t *)gguf;
        uint8_t *dst = (uint8_t *)out;
        for (size_t r = 0; r < rows; r++)
            for (int64_t sb = 0; sb < nsb; sb++)
                sd::pack_sb(fmt, src + ((int64_t)r * nsb + sb) * sbb, dst + ((int64_t)(r >> 4) * nsb + sb) * tbb,
                            (int)(r & 15));
    });
}

sd_status sd_unpack_tiles(int32_t fmt, const void *tiles, size_t rows, size_t K, void *gguf_out) {
    return guard([&] {
        if (!tiles || !gguf_out) throw sd::ArgError("null argument");
        const int64_t nsb = quant_rows_check(fmt, rows, K);
        const int sbb = sd::fmt_sb_bytes(fmt), tbb = sd::tile_block_bytes(fmt);
        const uint8_t *src = (const uint8_t *)tiles;
        uint8_t *dst = (uint8_t *)gguf_out;
        for (size_t r = 0; r < rows; r++)
            for (int64_t sb = 0; sb < nsb; sb++)
                sd::unpack_sb(fmt, src + ((int64_t)(r >> 4) * nsb + sb) * tbb, (int)(r & 15),
                              dst + ((int64_t)r * nsb + sb) * sbb);
    });
}

sd_status sd_lane_codes(int32_t fmt, const void *tile_block, int32_t lane, int32_t chunk, uint32_t *out) {
    return guard([&] {
        if (!tile_block || !out) throw sd::ArgError("null argument");
        if (lane < 0 || lane > 63 || chunk < 0 || chunk > 7) throw sd::ArgError("lane in [0, 64), chunk in [0, 8)");
        const uint8_t *tb = (const uint8_t *)tile_block;
        auto v4 = [&](int off) {
            sd::uintx4 v;
            std::memcpy(&v, tb + off, 16);
            return v;
        };
        const int g = lane >> 4;
        if (fmt == SD_Q4_K) {
            sd::LaneQ4K d;
            d.hdr = v4(d.off_hdr(lane));
            d.q0 = v4(d.off_q0(lane));
            d.q1 = v4(d.off_q1(lane));
            d.codes(g, chunk, out);
        } else if (fmt == SD_Q5_K) {
            sd::LaneQ5K d;
            d.hdr = v4(d.off_hdr(lane));
            std::memcpy(&d.qh, tb + d.off_qh(lane), 8);
            d.q0 = v4(d.off_q0(lane));
            d.q1 = v4(d.off_q1(lane));
            d.codes(g, chunk, out);
        } else if (fmt == SD_Q6_K) {
            sd::LaneQ6K d;
            d.n0 = v4(d.off_n0(lane));
            d.n1 = v4(d.off_n1(lane));
            d.hb = v4(d.off_hb(lane));
            d.codes(g, chunk, out);
        } else if (fmt == SD_Q8_0) {
            sd::LaneQ80 d;
            d.a0 = v4(d.off_part(lane, 0));
            d.a1 = v4(d.off_part(lane, 1));
            d.b0 = v4(d.off_part(lane, 2));
            d.b1 = v4(d.off_part(lane, 3));
            d.codes(g, chunk, out);
        } else {
            throw sd::UnsupportedError("format must be Q4_K, Q5_K, Q6_K or Q8_0");
        }
    });
}

sd_status sd_tree_cartesian(uint32_t root, const uint32_t *cand, const uint32_t *branching, size_t depth,
                            uint32_t *tokens, uint32_t *parents, size_t cap, size_t *n) {
    return guard([&] {
        if (!n || (depth && (!cand || !branching))) throw sd::ArgError("null argument");
        const size_t need = sd::cartesian_size(branching, depth);
        *n = need;
        if (!tokens || !parents) return;  // size query
        if (need > cap) throw sd::ArgError("output capacity smaller than the Cartesian tree");
        const sd::DraftTreeC t = sd::cartesian_tree(root, cand, branching, depth);
        std::memcpy(tokens, t.tokens.data(), need * 4);
        std::memcpy(parents, t.parents.data(), need * 4);
    });
}

sd_status sd_tree_prune(const uint32_t *tokens, const uint32_t *parents, size_t n, const float *log_probs,
                        const uint32_t *branching, size_t depth, size_t max_total, uint32_t *out_tokens,
                        uint32_t *out_parents, size_t *n_out) {
    return guard([&] {
        if (!tokens || !parents || !out_tokens || !out_parents || !n_out || (depth && (!log_probs || !branching)))
            throw sd::ArgError("null argument");
        const sd::DraftTreeC full = sd::DraftTreeC::from_arrays(tokens, parents, n);
        const sd::DraftTreeC t = sd::prune_cartesian(full, log_probs, branching, depth, max_total);
        std::memcpy(out_tokens, t.tokens.data(), t.size() * 4);
        std::memcpy(out_parents, t.parents.data(), t.size() * 4);
        *n_out = t.size();
    });
}


/* ---- EAGLE-3 draft (crates/speculate/src/methods/eagle3.rs) ---- */
static void need3(const sd_draft3 *d) {
    if (!d || !d->d) throw sd::ArgError("null draft handle");
}

sd_status sd_draft3_create(const sd_draft3_config *cfg, sd_draft3 **out) {
    return guard([&] {
        if (!cfg || !out) throw sd::ArgError("null argument");
        *out = nullptr;
        sd::Draft3Cfg c;
        c.hidden = cfg->hidden;
        c.n_heads = cfg->n_heads;
        c.n_kv_heads = cfg->n_kv_heads;
        c.ffn = cfg->ffn;
        c.draft_vocab = cfg->draft_vocab;
        c.target_vocab = cfg->target_vocab;
        c.rms_eps = cfg->rms_eps;
        c.rope_theta = cfg->rope_theta;
        c.max_pos = cfg->max_pos;
        c.device = cfg->device;
        auto h = std::make_unique<sd_draft3>();
        h->d = std::make_unique<sd::Draft3>(c);
        *out = h.release();
    });
}

void sd_draft3_destroy(sd_draft3 *d) { delete d; }

size_t sd_draft3_tensor_bytes(const sd_draft3 *d, int32_t kind) {
    if (!d || !d->d || kind < 0 || kind >= sd::D3_NUM) return 0;
    return d->d->tensor_bytes(kind);
}

sd_status sd_draft3_set_tensor(sd_draft3 *d, int32_t kind, const void *data, size_t bytes) {
    return guard([&] {
        need3(d);
        d->d->set_tensor(kind, data, bytes);
    });
}

sd_status sd_draft3_get_tensor(const sd_draft3 *d, int32_t kind, void *data, size_t bytes) {
    return guard([&] {
        need3(d);
        if (!data) throw sd::ArgError("null data");
        d->d->get_tensor(kind, data, bytes);
    });
}

sd_status sd_draft3_synthesize(sd_draft3 *d, uint64_t seed, float weight_std) {
    return guard([&] {
        need3(d);
        d->d->synthesize(seed, weight_std);
    });
}

sd_status sd_draft3_reset(sd_draft3 *d) {
    return guard([&] {
        need3(d);
        d->d->reset();
    });
}

sd_status sd_draft3_forward(sd_draft3 *d, const float *hidden_in, size_t n_in, const float *input_emb,
                            size_t position, float *out_hidden, float *out_logits) {
    return guard([&] {
        need3(d);
        if (!hidden_in || !input_emb) throw sd::ArgError("null argument");
        if (position > (size_t)INT32_MAX) throw sd::ArgError("position out of range");
        d->d->step_host(hidden_in, n_in, input_emb, (int)position, out_hidden, out_logits);
    });
}

sd_status sd_draft3_round(sd_draft3 *d, sd_model *m, const uint32_t *layers, size_t depth, const int32_t *top_k,
                          int32_t *target_ids, int32_t *draft_ids, float *log_probs) {
    return guard([&] {
        need3(d);
        need_weights(m);
        if (!layers || !top_k || !target_ids || !draft_ids || !log_probs) throw sd::ArgError("null argument");
        if (depth < 1 || depth > (size_t)sd::kDraftMaxSteps) throw sd::ArgError("draft depth out of range");
        setdev(m);
        d->d->round(*m->model, *m->dec, layers, (int)depth, top_k, target_ids, draft_ids, log_probs);
    });
}


/* ---- EAGLE-2 draft (crates/speculate/src/methods/eagle.rs) ---- */
static void need2(const sd_draft2 *d) {
    if (!d || !d->d) throw sd::ArgError("null draft handle");
}

sd_status sd_draft2_create(const sd_draft2_config *cfg, sd_draft2 **out) {
    return guard([&] {
        if (!cfg || !out) throw sd::ArgError("null argument");
        *out = nullptr;
        sd::Draft2Cfg c;
        c.hidden = cfg->hidden;
        c.n_heads = cfg->n_heads;
        c.n_kv_heads = cfg->n_kv_heads;
        c.ffn = cfg->ffn;
        c.vocab = cfg->vocab;
        c.rms_eps = cfg->rms_eps;
        c.rope_theta = cfg->rope_theta;
        c.max_pos = cfg->max_pos;
        c.device = cfg->device;
        auto h = std::make_unique<sd_draft2>();
        h->d = std::make_unique<sd::Draft2>(c);
        *out = h.release();
    });
}

void sd_draft2_destroy(sd_draft2 *d) { delete d; }

size_t sd_draft2_tensor_bytes(const sd_draft2 *d, int32_t kind) {
    if (!d || !d->d || kind < 0 || kind >= sd::D2_NUM) return 0;
    return d->d->tensor_bytes(kind);
}

sd_status sd_draft2_set_tensor(sd_draft2 *d, int32_t kind, const void *data, size_t bytes) {
    return guard([&] {
        need2(d);
        d->d->set_tensor(kind, data, bytes);
    });
}

sd_status sd_draft2_get_tensor(const sd_draft2 *d, int32_t kind, void *data, size_t bytes) {
    return guard([&] {
        need2(d);
        if (!data) throw sd::ArgError("null data");
        d->d->get_tensor(kind, data, bytes);
    });
}

sd_status sd_draft2_synthesize(sd_draft2 *d, uint64_t seed, float weight_std) {
    return guard([&] {
        need2(d);
        d->d->synthesize(seed, weight_std);
    });
}

sd_status sd_draft2_reset(sd_draft2 *d) {
    return guard([&] {
        need2(d);
        d->d->reset();
    });
}

sd_status sd_draft2_forward(sd_draft2 *d, const float *target_hidden, size_t n, uint32_t token, size_t position,
                            float *out_hidden) {
    return guard([&] {
        need2(d);
        if (!target_hidden) throw sd::ArgError("null argument");
        if (n != (size_t)d->d->cfg.hidden) throw sd::ArgError("target_hidden must be hidden wide");
        if (position > (size_t)INT32_MAX) throw sd::ArgError("position out of range");
        d->d->step_host(target_hidden, token, (int)position, out_hidden);
    });
}

sd_status sd_draft2_round(sd_draft2 *d, sd_model *m, const float *target_hidden, size_t depth, const int32_t *top_k,
                          int32_t *ids, float *log_probs) {
    return guard([&] {
        need2(d);
        need_weights(m);
        if (!target_hidden || !top_k || !ids || !log_probs) throw sd::ArgError("null argument");
        if (depth < 1 || depth > (size_t)sd::kDraftMaxSteps) throw sd::ArgError("draft depth out of range");
        setdev(m);
        d->d->round(*m->model, *m->dec, target_hidden, (int)depth, top_k, ids, log_probs);
    });
}

}  // extern "C"
