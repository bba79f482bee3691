// Host runtime of the target-verify path.  See sd_model.hpp.
#include "sd_model.hpp"

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>

#include "sd_common.hpp"

namespace sd {

static const bool kIsF32Kind[K_NUM] = {false, false, true, false, false, false, false,
                                       false, false, false, true, true, true, true, true};

bool kind_is_f32(int kind) { return kind >= 0 && kind < K_NUM && kIsF32Kind[kind]; }

void tensor_shape(const ModelCfg &c, int kind, int &rows, int &K) {
    const int H = c.hidden, F = c.ffn;
    switch (kind) {
    case K_TOK_EMBD: case K_OUTPUT: rows = c.vocab; K = H; break;
    case K_OUTPUT_NORM: case K_ATTN_NORM: case K_FFN_NORM: rows = 1; K = H; break;
    case K_ATTN_Q: rows = c.q_dim(); K = H; break;
    case K_ATTN_K: case K_ATTN_V: rows = c.kv_dim(); K = H; break;
    case K_ATTN_O: rows = H; K = c.q_dim(); break;
    case K_FFN_GATE: case K_FFN_UP: rows = F; K = H; break;
    case K_FFN_DOWN: rows = H; K = F; break;
    case K_BQ: rows = 1; K = c.q_dim(); break;
    case K_BK: case K_BV: rows = 1; K = c.kv_dim(); break;
    default: throw ArgError("unknown tensor kind");
    }
}

static int64_t gguf_row_bytes(int fmt, int64_t K) {
    if (fmt == F32) return 4 * K;
    return K / fmt_block_elems(fmt) * fmt_block_bytes(fmt);
}

// Zeroed device allocation.  The fill runs on the null stream, which does not
// order against the model's non-blocking stream, so wait for it here.
template <typename T> static T *dalloc(size_t n) {
    void *p = nullptr;
    SD_HIP_CHECK(hipMalloc(&p, n * sizeof(T) + 256));
    SD_HIP_CHECK(hipMemset(p, 0, n * sizeof(T) + 256));
    SD_HIP_CHECK(hipDeviceSynchronize());
    return (T *)p;
}

Model::Model(const ModelCfg &c) : cfg(c) {
    if (c.n_layers <= 0 || c.hidden <= 0 || c.n_heads <= 0 || c.n_kv_heads <= 0 || c.head_dim <= 0 || c.ffn <= 0 ||
        c.vocab <= 0 || c.ctx_len <= 0)
        throw ArgError("config: all sizes must be positive");
    if (c.n_heads % c.n_kv_heads) throw ArgError("config: n_heads must be a multiple of n_kv_heads");
    if (c.head_dim != 64 && c.head_dim != 128) throw UnsupportedError("config: head_dim must be 64 or 128");
    if (c.hidden % 256 || c.ffn % 256 || c.q_dim() % 256) throw UnsupportedError("config: hidden/ffn/q_dim must be multiples of 256");
    if (c.kv_dim() % 32 || c.vocab % 32) throw UnsupportedError("config: kv_dim and vocab must be multiples of 32");
    if (c.max_batch < 1 || c.max_batch > 128) throw ArgError("config: max_batch must be in [1, 128]");
    SD_HIP_CHECK(hipSetDevice(c.device));
    SD_HIP_CHECK(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
    lw.resize(c.n_layers);
    alloc_buffers();
}

Model::~Model() {
    hipSetDevice(cfg.device);
    if (st) hipStreamSynchronize(st);
    auto F = [](void *p) {
        if (p) hipFree(p);
    };
    for (auto &L : lw)
        for (auto &t : L) F(t.d);
    for (auto &t : gw) {
        F(t.d);
        F(t.gguf);
    }
    for (void *p : {(void *)kv, (void *)cos_t, (void *)sin_t, (void *)h, (void *)qkv, (void *)logits,
                    (void *)hidden_out, (void *)last_row, (void *)part_o, (void *)part_ml, (void *)amax_v,
                    (void *)collect_buf, (void *)amax_i, (void *)argmax, (void *)d_ids,
                    (void *)d_src, (void *)xp, (void *)ap, (void *)act, (void *)q16,
                    (void *)acc_m, (void *)acc_s, (void *)acc_q, (void *)acc_am, (void *)acc_tree,
                    (void *)acc_out, (void *)t2d_inv, (void *)qg_part, (void *)aux_h, (void *)aux_x, (void *)aux_y,
                    (void *)aux_ids, (void *)ssq, (void *)split_cnt, (void *)acc_part, (void *)acc_cnt,
                    (void *)acc_prob, (void *)acc_lin, (void *)qa_flags})
        F(p);
    if (qa_status) hipHostFree(qa_status);
    if (h_stage) hipHostFree(h_stage);
    if (acc_stage) hipHostFree(acc_stage);
    if (stage_ev) hipEventDestroy(stage_ev);
    for (hipEvent_t e : ev_pool) hipEventDestroy(e);
    if (st) hipStreamDestroy(st);
}

void Model::alloc_buffers() {
    const ModelCfg &c = cfg;
    const int Mx = c.max_batch, Mp = 128 + 16;  // padded rows (16-token MFMA tiles + last-row slack)
    cap = ((int64_t)c.ctx_len + 128 + 31) / 32 * 32;  // whole 32-position blocks of the V layout
    kv = dalloc<uint16_t>((size_t)c.n_layers * 2 * c.n_kv_heads * cap * c.head_dim);
    // RoPE tables (quantized_llama_local.rs:189-205): host f32 powf/cosf/sinf
    {
        const int half = c.head_dim / 2;
        std::vector<float> theta(half), ct((size_t)cap * half), stt((size_t)cap * half);
        for (int i = 0; i < half; i++) theta[i] = 1.0f / powf(c.rope_theta, (float)(2 * i) / (float)c.head_dim);
        for (int64_t t = 0; t < cap; t++)
            for (int i = 0; i < half; i++) {
                const float a = (float)t * theta[i];
                ct[t * half + i] = cosf(a);
                stt[t * half + i] = sinf(a);
            }
        cos_t = dalloc<float>(ct.size());
        sin_t = dalloc<float>(stt.size());
        SD_HIP_CHECK(hipMemcpy(cos_t, ct.data(), ct.size() * 4, hipMemcpyHostToDevice));
        SD_HIP_CHECK(hipMemcpy(sin_t, stt.data(), stt.size() * 4, hipMemcpyHostToDevice));
    }
    const int qkvd = c.q_dim() + 2 * c.kv_dim();
    xp_ld = std::max(c.hidden, c.q_dim());
    ap_ld = c.q_dim();
    act_ld = c.ffn;
    h = dalloc<float>((size_t)Mx * c.hidden);
    qkv = dalloc<float>((size_t)Mx * qkvd);
    xp = dalloc<uint16_t>((size_t)Mp * xp_ld);
    ap = dalloc<uint16_t>((size_t)Mp * ap_ld);
    act = dalloc<uint16_t>((size_t)Mp * act_ld);
    q16 = dalloc<uint16_t>((size_t)c.n_heads * Mx * c.head_dim);
    nsplit_max = attn_max_splits(c.n_kv_heads);
    part_o = dalloc<float>((size_t)nsplit_max * c.n_heads * Mx * c.head_dim);
    part_ml = dalloc<float>((size_t)nsplit_max * c.n_heads * Mx * 2);
    split_cnt = dalloc<int>(c.n_heads);  // n_kv x (query tiles <= n_rep up to 16 rows), zero
    qa_flags = dalloc<unsigned>(kQaFlags);
    SD_HIP_CHECK(hipHostMalloc((void **)&qa_status, sizeof(int), hipHostMallocMapped | hipHostMallocCoherent));
    *(volatile int *)qa_status = 0;
    SD_HIP_CHECK(hipHostGetDevicePointer((void **)&qa_status_dev, qa_status, 0));
    SD_HIP_CHECK(hipDeviceGetAttribute(&n_cus, hipDeviceAttributeMultiprocessorCount, c.device));
    const char *unfused = std::getenv("SD_ATTN_UNFUSED");
    fused_qkv_attn = !(unfused && unfused[0] == '1');
    logits = dalloc<float>((size_t)Mx * c.vocab);
    hidden_out = dalloc<float>((size_t)Mx * c.hidden);
    last_row = dalloc<float>((size_t)c.vocab);
    amax_ld = c.vocab / 16;
    amax_v = dalloc<float>((size_t)Mx * amax_ld);
    amax_i = dalloc<int>((size_t)Mx * amax_ld);
    argmax = dalloc<int>(Mx);
    // rows of last_hidden_states_multi: one per requested layer, repeats allowed
    collect_cap = std::max(c.n_layers, 16);
    collect_buf = dalloc<float>((size_t)collect_cap * c.hidden);
    // ids | pos | (unused) | mask in one block laid out as the pinned staging
    // buffer, so that one copy uploads a forward's inputs
    d_ids = dalloc<int>((size_t)3 * Mx + (Mx & 1) + (size_t)4 * Mx);
    d_pos = d_ids + Mx;
    d_mask = (uint64_t *)(d_ids + 3 * Mx + (Mx & 1));
    d_src = dalloc<int>(Mx);
    qg_part_cap = std::max<int64_t>((int64_t)8 * Mx * std::max(qkvd, c.hidden), (int64_t)2 * Mx * 2 * c.ffn);
    qg_part = dalloc<float>((size_t)qg_part_cap);
    ssq = dalloc<float>((size_t)16 * (c.hidden / 16));
    acc_m = dalloc<float>(Mx);
    acc_s = dalloc<float>(Mx);
    acc_am = dalloc<int>(Mx);
    // parents | tokens | q_row_of | uniforms | children per node | the children's tokens [n][16] | the
    // nodes of each precomputed pass (<= 17 n) of one walk
    acc_tree = dalloc<int>((size_t)kAccTreeInts * Mx);
    acc_out = dalloc<int>((size_t)Mx + 4);
    acc_part = dalloc<uint64_t>((size_t)Mx * 2 * kRowStatsMaxSlices);
    acc_cnt = dalloc<int>(Mx);
    aux_h = dalloc<float>((size_t)kAuxRows * c.hidden);
    aux_x = dalloc<uint16_t>((size_t)(kAuxRows + 16) * c.hidden);
    aux_y = dalloc<float>((size_t)kAuxRows * c.vocab);
    aux_ids = dalloc<int>(kAuxRows);
    h_stage_bytes = (size_t)Mx * (3 * sizeof(int) + 2 * sizeof(uint64_t)) + 256;
    SD_HIP_CHECK(hipHostMalloc((void **)&h_stage, h_stage_bytes, hipHostMallocDefault));
    SD_HIP_CHECK(hipHostMalloc((void **)&acc_stage, ((size_t)(kAccTreeInts + 1) * Mx + 8) * sizeof(int),
                               hipHostMallocDefault));
    SD_HIP_CHECK(hipEventCreateWithFlags(&stage_ev, hipEventDisableTiming));
}

void Model::stage_wait() { SD_HIP_CHECK(hipEventSynchronize(stage_ev)); }

void Model::check_status() {
    if (*(volatile int *)qa_status == 0) return;
    // the launch's outputs are undefined and its counters may be left mid-count
    SD_HIP_CHECK(hipStreamSynchronize(st));
    SD_HIP_CHECK(hipMemsetAsync(split_cnt, 0, (size_t)cfg.n_heads * sizeof(int), st));
    SD_HIP_CHECK(hipStreamSynchronize(st));
    *(volatile int *)qa_status = 0;
    throw BackendError("fused Q/K/V + attention launch: the attention gave up waiting for the matmul");
}

void Model::sync() {
    SD_HIP_CHECK(hipStreamSynchronize(st));
    check_status();
}
void Model::stage_done() { SD_HIP_CHECK(hipEventRecord(stage_ev, st)); }

bool Model::weights_ready() const {
    static const int need[] = {K_ATTN_Q, K_ATTN_K, K_ATTN_V, K_ATTN_O, K_FFN_GATE, K_FFN_UP, K_FFN_DOWN,
                               K_ATTN_NORM, K_FFN_NORM};
    if (!gw[K_TOK_EMBD].set() || !gw[K_OUTPUT_NORM].set()) return false;
    if (!cfg.tied_output && !gw[K_OUTPUT].set()) return false;
    for (auto &L : lw) {
        for (int k : need)
            if (!L[k].set()) return false;
        if (cfg.arch == 1 && (!L[K_BQ].set() || !L[K_BK].set() || !L[K_BV].set())) return false;
    }
    return true;
}

static void check_fmt(int kind, int fmt, int K) {
    if (kIsF32Kind[kind]) {
        if (fmt != F32) throw ArgError("norm/bias tensors must be F32");
        return;
    }
    if (fmt != Q4_K && fmt != Q5_K && fmt != Q6_K && fmt != Q8_0)
        throw UnsupportedError("matrix tensors must be Q4_K, Q5_K, Q6_K or Q8_0");
    if (K % 256) throw UnsupportedError("K must be a multiple of 256");
}

static DevTensor &slot(Model &m, int layer, int kind) {
    if (kind < 0 || kind >= K_NUM) throw ArgError("unknown tensor kind");
    if (layer < -1 || layer >= m.cfg.n_layers) throw ArgError("layer out of range");
    const bool global = kind <= K_OUTPUT_NORM;
    if (global != (layer == -1)) throw ArgError("global tensors use layer -1, per-layer tensors 0..n_layers-1");
    if (kind >= K_BQ && m.cfg.arch != 1) throw ArgError("QKV bias tensors exist only for qwen2");
    return global ? m.gw[kind] : m.lw[layer][kind];
}

void Model::set_tensor(int layer, int kind, int fmt, const void *host, size_t bytes) {
    fwd_count++;
    DevTensor &t = slot(*this, layer, kind);
    int rows, K;
    tensor_shape(cfg, kind, rows, K);
    check_fmt(kind, fmt, K);
    const size_t want = (size_t)rows * gguf_row_bytes(fmt, K);
    if (bytes != want) throw ArgError("tensor byte size does not match its shape and format");
    SD_HIP_CHECK(hipSetDevice(cfg.device));
    if (t.d) {
        SD_HIP_CHECK(hipFree(t.d));
        t.d = nullptr;
    }
    if (t.gguf) {
        SD_HIP_CHECK(hipFree(t.gguf));
        t.gguf = nullptr;
    }
    if ((size_t)dev_tensor_bytes(fmt, rows, K) >= ((size_t)1 << 31))
        throw UnsupportedError("a matrix must be smaller than 2 GiB (32-bit buffer offsets)");
    if (fmt != F32 && rows % 16) throw UnsupportedError("quantised matrices need a multiple of 16 rows");
    t.fmt = fmt;
    t.rows = rows;
    t.K = K;
    t.bytes = (size_t)dev_tensor_bytes(fmt, rows, K);
    t.d = dalloc<uint8_t>(t.bytes);
    if (fmt == F32) {
        SD_HIP_CHECK(hipMemcpy(t.d, host, bytes, hipMemcpyHostToDevice));
    } else {
        uint8_t *tmp = dalloc<uint8_t>(bytes);
        SD_HIP_CHECK(hipMemcpy(tmp, host, bytes, hipMemcpyHostToDevice));
        launch_gguf_to_dev(fmt, tmp, t.d, rows, K, st);
        SD_HIP_CHECK(hipStreamSynchronize(st));
        if (kind == K_TOK_EMBD) t.gguf = tmp;
        else SD_HIP_CHECK(hipFree(tmp));
    }
}

void Model::tensor_info(int layer, int kind, int *fmt, int *rows, int *K, size_t *gbytes) {
    DevTensor &t = slot(*this, layer, kind);
    if (!t.set()) throw ArgError("tensor not set");
    *fmt = t.fmt;
    *rows = t.rows;
    *K = t.K;
    *gbytes = (size_t)t.rows * gguf_row_bytes(t.fmt, t.K);
}

void Model::get_tensor(int layer, int kind, void *host, size_t bytes) {
    DevTensor &t = slot(*this, layer, kind);
    if (!t.set()) throw ArgError("tensor not set");
    const size_t g = (size_t)t.rows * gguf_row_bytes(t.fmt, t.K);
    if (bytes != g) throw ArgError("buffer size does not match the tensor");
    SD_HIP_CHECK(hipSetDevice(cfg.device));
    if (t.fmt == F32) {
        SD_HIP_CHECK(hipStreamSynchronize(st));  // the model's stream does not order with this copy
        SD_HIP_CHECK(hipMemcpy(host, t.d, g, hipMemcpyDeviceToHost));
    } else {
        uint8_t *tmp = dalloc<uint8_t>(g);
        launch_dev_to_gguf(t.fmt, t.d, tmp, t.rows, t.K, st);
        SD_HIP_CHECK(hipStreamSynchronize(st));
        SD_HIP_CHECK(hipMemcpy(host, tmp, g, hipMemcpyDeviceToHost));
        SD_HIP_CHECK(hipFree(tmp));
    }
}

void Model::dequant_tensor(int layer, int kind, float *host) {
    DevTensor &t = slot(*this, layer, kind);
    if (!t.set()) throw ArgError("tensor not set");
    SD_HIP_CHECK(hipSetDevice(cfg.device));
    const size_t n = (size_t)t.rows * t.K;
    if (t.fmt == F32) {
        SD_HIP_CHECK(hipStreamSynchronize(st));  // the model's stream does not order with this copy
        SD_HIP_CHECK(hipMemcpy(host, t.d, n * 4, hipMemcpyDeviceToHost));
        return;
    }
    float *y = dalloc<float>(n);
    launch_dequant_dev(t.fmt, t.d, t.rows, t.K, y, st);
    SD_HIP_CHECK(hipStreamSynchronize(st));
    SD_HIP_CHECK(hipMemcpy(host, y, n * 4, hipMemcpyDeviceToHost));
    SD_HIP_CHECK(hipFree(y));
}

// Q4_K_M mix (llama.cpp's use_more_bits rule for attn_v / ffn_down) and the others
static int mix_fmt(int mix, int n_layers, int layer, int kind) {
    if (kIsF32Kind[kind]) return F32;
    if (mix == 0) return Q4_K;
    if (mix == 1) {
        const int n = n_layers, i = layer;
        const bool more = i < n / 8 || i >= 7 * n / 8 || (i - n / 8) % 3 == 2;
        if ((kind == K_ATTN_V || kind == K_FFN_DOWN) && more) return Q6_K;
        return Q4_K;
    }
    if (mix == 2) {
        if (kind == K_ATTN_Q || kind == K_ATTN_K || kind == K_ATTN_V || kind == K_ATTN_O) return Q5_K;
        return Q8_0;
    }
    if (mix == 3) return Q6_K;
    if (mix == 4) return Q5_K;
    if (mix == 5) return Q8_0;
    throw ArgError("unknown quantisation mix");
}

void Model::synthesize(int mix, uint64_t seed, float stdv) {
    fwd_count++;
    SD_HIP_CHECK(hipSetDevice(cfg.device));
    const float mult = (float)((double)stdv * std::sqrt(3.0) / 65536.0);
    auto make = [&](int layer, int kind) {
        DevTensor &t = slot(*this, layer, kind);
        int rows, K;
        tensor_shape(cfg, kind, rows, K);
        const int fmt = mix_fmt(mix, cfg.n_layers, layer, kind);
        if ((size_t)dev_tensor_bytes(fmt, rows, K) >= ((size_t)1 << 31))
            throw UnsupportedError("a matrix must be smaller than 2 GiB (32-bit buffer offsets)");
        if (fmt != F32 && rows % 16) throw UnsupportedError("quantised matrices need a multiple of 16 rows");
        if (t.d) SD_HIP_CHECK(hipFree(t.d));
        if (t.gguf) SD_HIP_CHECK(hipFree(t.gguf));
        t.d = t.gguf = nullptr;
        t.fmt = fmt;
        t.rows = rows;
        t.K = K;
        t.bytes = (size_t)dev_tensor_bytes(fmt, rows, K);
        t.d = dalloc<uint8_t>(t.bytes);
        const uint64_t ts = tensor_seed(seed, layer, kind);
        if (kind == K_OUTPUT_NORM || kind == K_ATTN_NORM || kind == K_FFN_NORM) {
            launch_fill_f32((float *)t.d, (int64_t)rows * K, 1.0f, st);
        } else if (fmt == F32) {
            launch_synth_f32((float *)t.d, (int64_t)rows * K, ts, mult, st);
        } else {
            const size_t g = (size_t)rows * gguf_row_bytes(fmt, K);
            uint8_t *tmp = dalloc<uint8_t>(g);
            launch_synth_quant(fmt, tmp, rows, K, ts, mult, st);
            launch_gguf_to_dev(fmt, tmp, t.d, rows, K, st);
            SD_HIP_CHECK(hipStreamSynchronize(st));
            if (kind == K_TOK_EMBD) t.gguf = tmp;
            else SD_HIP_CHECK(hipFree(tmp));
        }
    };
    make(-1, K_TOK_EMBD);
    make(-1, K_OUTPUT_NORM);
    if (!cfg.tied_output) make(-1, K_OUTPUT);
    for (int l = 0; l < cfg.n_layers; l++) {
        for (int k = K_ATTN_Q; k <= K_FFN_NORM; k++) make(l, k);
        if (cfg.arch == 1)
            for (int k = K_BQ; k <= K_BV; k++) make(l, k);
    }
    SD_HIP_CHECK(hipStreamSynchronize(st));
}

void Model::fill_kv_synthetic(int P, uint64_t seed) {
    fwd_count++;
    if (P < 0 || P > cfg.ctx_len) throw ArgError("prefix longer than the KV capacity");
    const float mult = (float)(std::sqrt(3.0) / 65536.0);
    launch_fill_kv(kv, cfg.n_layers, cfg.n_kv_heads, cap, cfg.head_dim, P, seed, mult, st);
    SD_HIP_CHECK(hipStreamSynchronize(st));
}

void Model::prof_reset() { prof.clear(); }

int Model::prof_events() {
    const size_t need = 2 * (prof.size() + 1);
    while (ev_pool.size() < need) {
        hipEvent_t e;
        SD_HIP_CHECK(hipEventCreate(&e));
        ev_pool.push_back(e);
    }
    return (int)(2 * prof.size());
}

int Model::prof_begin() {
    const int ev = prof_events();
    SD_HIP_CHECK(hipEventRecord(ev_pool[ev], st));
    return ev;
}

void Model::prof_end(int ev, int cls, double bytes) {
    SD_HIP_CHECK(hipEventRecord(ev_pool[ev + 1], st));
    prof.push_back(ProfEntry{cls, bytes, ev});
}

// Algorithmic bytes of one dequant-matmul launch: the weight blocks (given),
// the fp16 activations read once, and the output written once (read too when
// the epilogue adds the residual).
static double gemm_bytes(const GemmParams &p, double wbytes) {
    const double x = 2.0 * p.M * p.K;
    double y = 0.0;
    if (p.mode == GM_SWIGLU) {
        y = 2.0 * p.M * p.seg[0].rows;
    } else {
        for (int i = 0; i < p.nseg; i++) y += 4.0 * p.M * p.seg[i].rows * (p.mode == GM_RESID ? 2 : 1);
    }
    return wbytes + x + y;
}

void Model::run_gemm(GemmParams &p, int cls, double bytes) {
    bytes = gemm_bytes(p, bytes);
    if (prof_on) {
        // the events carry the dispatch's own start / end timestamps
        const int ev = prof_events();
        launch_qgemm(p, st, LaunchTiming{ev_pool[ev], ev_pool[ev + 1]});
        prof.push_back(ProfEntry{cls, bytes, ev});
    } else {
        launch_qgemm(p, st);
    }
}

static double wbytes(const DevTensor &t) { return (double)t.rows * gguf_row_bytes(t.fmt, t.K); }
static double gemm_bytes(const GemmParams &p, double wbytes);

static GemmSeg seg_of(const DevTensor &t, int tile0, float *out, int ldo, int col0, const float *bias) {
    GemmSeg s;
    s.w = t.d;
    s.fmt = t.fmt;
    s.rows = t.rows;
    s.tile0 = tile0;
    s.out = out;
    s.ldo = ldo;
    s.col0 = col0;
    s.bias = bias;
    return s;
}

void Model::qmatmul(int layer, int kind, const float *x, int M, float *y) {
    DevTensor &t = slot(*this, layer, kind);
    if (!t.set() || t.fmt == F32) throw ArgError("qmatmul needs a quantised matrix tensor");
    if (M < 1 || M > cfg.max_batch) throw ArgError("M out of range");
    SD_HIP_CHECK(hipSetDevice(cfg.device));
    float *dx = dalloc<float>((size_t)M * t.K);
    float *dy = dalloc<float>((size_t)M * t.rows);
    uint16_t *dxp = dalloc<uint16_t>((size_t)(128 + 16) * t.K);
    SD_HIP_CHECK(hipMemcpy(dx, x, (size_t)M * t.K * 4, hipMemcpyHostToDevice));
    launch_to_frag16(dx, M, t.K, dxp, t.K, st);
    GemmParams p{};
    gemm_workspace(p);
    p.seg[0] = seg_of(t, 0, dy, t.rows, 0, nullptr);
    p.nseg = 1;
    p.ntiles = t.rows / 16;
    p.xp = dxp;
    p.K = t.K;
    p.M = M;
    p.mode = GM_STORE;
    launch_qgemm(p, st);
    SD_HIP_CHECK(hipStreamSynchronize(st));
    SD_HIP_CHECK(hipMemcpy(y, dy, (size_t)M * t.rows * 4, hipMemcpyDeviceToHost));
    hipFree(dx);
    hipFree(dy);
    hipFree(dxp);
}

void Model::qmatmul_into(int layer, int kind, const float *x_dev, int M, float *y_dev, hipStream_t stream,
                         void *staging, size_t staging_bytes) {
    DevTensor &t = slot(*this, layer, kind);
    if (!t.set() || t.fmt == F32) throw ArgError("qmatmul needs a quantised matrix tensor");
    if (M < 1 || M > 128) throw ArgError("rows must be in [1, 128]");
    if ((size_t)M * t.K * 2 > staging_bytes)
        throw ArgError("rows * K * 2 = " + std::to_string((size_t)M * t.K * 2) + " bytes of staged activations exceed the " +
                       std::to_string(staging_bytes) + "-byte scratch");
    hipStream_t s = stream ? stream : st;
    launch_to_frag16(x_dev, M, t.K, (uint16_t *)staging, t.K, s);
    GemmParams p{};  // allow_split = 0: no split-K partials
    p.seg[0] = seg_of(t, 0, y_dev, t.rows, 0, nullptr);
    p.nseg = 1;
    p.ntiles = t.rows / 16;
    p.xp = (const uint16_t *)staging;
    p.K = t.K;
    p.M = M;
    p.mode = GM_STORE;
    launch_qgemm(p, s);
    SD_HIP_CHECK(hipGetLastError());
}

// Times `iters` back-to-back launches of one dequant-matmul with HIP events on
// the model's stream (activations: whatever the work buffers hold).  kind is a
// matrix kind, or BENCH_QKV / BENCH_GATE_UP for the fused launches of a layer.
double Model::bench_qmatmul(int layer, int kind, int M, int iters, double *bytes_out) {
    if (M < 1 || M > cfg.max_batch) throw ArgError("M out of range");
    if (layer < BENCH_ALL_LAYERS || layer >= cfg.n_layers) throw ArgError("layer out of range");
    if ((kind == BENCH_QKV || kind == BENCH_GATE_UP) && layer == -1) throw ArgError("fused launches need a layer");
    if (layer == BENCH_ALL_LAYERS && !(kind == BENCH_QKV || kind == BENCH_GATE_UP || kind == K_ATTN_Q ||
                                       kind == K_ATTN_K || kind == K_ATTN_V || kind == K_ATTN_O || kind == K_FFN_GATE ||
                                       kind == K_FFN_UP || kind == K_FFN_DOWN))
        throw ArgError("cycling over the layers needs a per-layer matrix");
    if (iters < 1) throw ArgError("iters must be positive");
    SD_HIP_CHECK(hipSetDevice(cfg.device));
    // one launch description per layer when cycling (each launch then reads
    // weights that the previous launches have not left in the caches)
    std::vector<GemmParams> ps;
    double bytes = 0.0;
    const int l0 = layer == BENCH_ALL_LAYERS ? 0 : layer;
    const int l1 = layer == BENCH_ALL_LAYERS ? cfg.n_layers : layer + 1;
    for (int l = l0; l < l1; l++) {
        double b = 0.0;
        ps.push_back(bench_params(l, kind, M, &b));
        bytes += b;
    }
    if (bytes_out) *bytes_out = bytes / (double)ps.size();
    hipEvent_t a, b;
    SD_HIP_CHECK(hipEventCreate(&a));
    SD_HIP_CHECK(hipEventCreate(&b));
    for (auto &p : ps) launch_qgemm(p, st);  // warm
    SD_HIP_CHECK(hipEventRecord(a, st));
    for (int i = 0; i < iters; i++) launch_qgemm(ps[i % ps.size()], st);
    SD_HIP_CHECK(hipEventRecord(b, st));
    SD_HIP_CHECK(hipEventSynchronize(b));
    float ms = 0.f;
    SD_HIP_CHECK(hipEventElapsedTime(&ms, a, b));
    hipEventDestroy(a);
    hipEventDestroy(b);
    return (double)ms * 1e3 / iters;
}

GemmParams Model::bench_params(int layer, int kind, int M, double *bytes_out) {
    auto &L = lw[layer < 0 ? 0 : layer];
    GemmParams p{};
    gemm_workspace(p);
    p.xp = xp;
    p.M = M;
    double wb = 0.0;
    if (kind == BENCH_QKV) {
        int t0 = 0;
        const int QD = cfg.q_dim(), KVD = cfg.kv_dim(), QKVD = QD + 2 * KVD;
        p.seg[0] = seg_of(L[K_ATTN_Q], t0, qkv, QKVD, 0, nullptr);
        t0 += L[K_ATTN_Q].rows / 16;
        p.seg[1] = seg_of(L[K_ATTN_K], t0, qkv, QKVD, QD, nullptr);
        t0 += L[K_ATTN_K].rows / 16;
        p.seg[2] = seg_of(L[K_ATTN_V], t0, qkv, QKVD, QD + KVD, nullptr);
        t0 += L[K_ATTN_V].rows / 16;
        p.nseg = 3;
        p.ntiles = t0;
        p.K = cfg.hidden;
        p.mode = GM_STORE;
        wb = wbytes(L[K_ATTN_Q]) + wbytes(L[K_ATTN_K]) + wbytes(L[K_ATTN_V]);
    } else if (kind == BENCH_GATE_UP) {
        p.seg[0] = seg_of(L[K_FFN_GATE], 0, nullptr, 0, 0, nullptr);
        p.seg[1] = seg_of(L[K_FFN_UP], 0, nullptr, 0, 0, nullptr);
        p.nseg = 2;
        p.ntiles = L[K_FFN_GATE].rows / 16 * 2;
        p.K = cfg.hidden;
        p.mode = GM_SWIGLU;
        p.act = act;
        p.act_ld = act_ld;
        wb = wbytes(L[K_FFN_GATE]) + wbytes(L[K_FFN_UP]);
    } else {
        DevTensor &t = slot(*this, layer, kind);
        if (!t.set() || t.fmt == F32) throw ArgError("bench_qmatmul needs a quantised matrix");
        if ((size_t)M * t.rows > (size_t)cfg.max_batch * cfg.vocab) throw ArgError("output too large");
        p.seg[0] = seg_of(t, 0, logits, t.rows, 0, nullptr);
        p.nseg = 1;
        p.ntiles = t.rows / 16;
        p.K = t.K;
        p.mode = GM_STORE;
        wb = wbytes(t);
    }
    if (p.K > xp_ld && kind != K_FFN_DOWN) throw ArgError("activation buffer too narrow");
    if (kind == K_FFN_DOWN) p.xp = act;
    if (bytes_out) *bytes_out = gemm_bytes(p, wb);
    return p;
}

void Model::forward(const int *ids, const int *pos, const uint64_t *mask, int mask_words, int M, int P,
                    int logits_mode, bool want_hidden, const std::vector<int> &collect, float *collect_out) {
    fwd_count++;
    const ModelCfg &c = cfg;
    if (M < 1 || M > c.max_batch) throw ArgError("forward: M out of range");
    if (P + M > c.ctx_len) throw ArgError("forward: KV capacity exceeded");
    if (mask_words < 1 || mask_words > 2) throw ArgError("forward: mask words");
    SD_HIP_CHECK(hipSetDevice(c.device));
    check_status();  // a fused launch of an earlier forward that gave up
    // fault injection for tests (SD_ATTN_WAIT_TEST=<reads>): the fused
    // launch's attention waits for a number no producer writes, gives up
    // after that many reads, and the step ends in BackendError
    const char *wtest = std::getenv("SD_ATTN_WAIT_TEST");
    const int fault_polls = wtest ? std::max(1, std::atoi(wtest)) : 0;
    // stage ids | pos | mask in pinned memory with the device block's layout,
    // then one H2D copy
    stage_wait();
    std::memcpy(h_stage, ids, M * sizeof(int));
    std::memcpy(h_stage + c.max_batch, pos, M * sizeof(int));
    const size_t mask_at = (size_t)3 * c.max_batch + (c.max_batch & 1);
    std::memcpy(h_stage + mask_at, mask, (size_t)M * mask_words * sizeof(uint64_t));
    SD_HIP_CHECK(hipMemcpyAsync(d_ids, h_stage, mask_at * sizeof(int) + (size_t)M * mask_words * sizeof(uint64_t),
                                hipMemcpyHostToDevice, st));
    stage_done();

    const int H = c.hidden, QD = c.q_dim(), KVD = c.kv_dim(), QKVD = QD + 2 * KVD;
    launch_embed(gw[K_TOK_EMBD].fmt, embed_table(), H, d_ids, M, h, st);
    const AttnSplit split = attn_split(P, M, c.n_kv_heads, c.n_heads / c.n_kv_heads);
    if (split.nsplit > nsplit_max) throw BackendError("attention split count exceeds workspace");
    // M > 16 matmuls may leave K-slice partial sums in qg_part for the next
    // kernel to add (rope for QKV, the following RMSNorm for the residual
    // matmuls); not while per-layer hidden states are collected
    const int split_ok = collect.empty() ? 1 : 0;
    int pend = 1;  // K slices of the last residual matmul not yet added to h
    // Up to 16 rows the RMSNorms and RoPE live in the matmul epilogues: the
    // residual matmuls (wo, ffn_down) also write u = fp16(h * w_next_norm)
    // and per-tile sums of h^2, the next matmul scales its outputs by
    // 1/rms, and the fused Q/K/V launch rotates q, k and appends k, v to the
    // cache.  Nine launches per layer become five (four with one key split).
    const bool fused = M <= 16 && H % 256 == 0 && H / 16 <= 256 && (c.head_dim == 64 || c.head_dim == 128);
    const int np = H / 16;
    if (fused) launch_norm_u(h, (const float *)lw[0][K_ATTN_NORM].d, M, H, xp, xp_ld, ssq, st);
    // 17..64 rows: each RMSNorm is split the same way around its matmul: the
    // residual finaliser writes u = fp16(h * w) and sums of h^2 per column
    // block from many workgroups per row, and the matmul (or, after K slices,
    // the RoPE finaliser) scales by 1/rms
    const bool spread = !fused && M > 16 && M <= 64;
    const int sp_parts = resid_u_parts(H);
    // K and V rows read once per layer by the attention: [0, P + M) of every KV head
    const double kv_bytes = 2.0 * c.n_kv_heads * (double)(P + M) * c.head_dim * 2.0;
    // up to 16 rows, with the epilogues fused, the attention's workgroups join
    // the Q/K/V launch where its shape allows (qkv_attention_fits)
    auto qa_fits = [&](const GemmParams &g, const AttnParams &at) {
        return fused && fused_qkv_attn && qkv_attention_fits(g, at, n_cus);
    };
    for (int l = 0; l < c.n_layers; l++) {
        auto &L = lw[l];
        if (spread)
            launch_resid_u(h, (const float *)L[K_ATTN_NORM].d, M, H, qg_part, pend, xp, xp_ld, ssq, st);
        else if (!fused)
            launch_rmsnorm(h, (const float *)L[K_ATTN_NORM].d, M, H, c.rms_eps, xp, xp_ld, nullptr, st, qg_part, pend);
        int nks_qkv;
        bool qa_launched = false;
        AttnParams a{};
        a.q16 = q16;
        a.kc = kc(l);
        a.vc = vc(l);
        a.cap = cap;
        a.mask = d_mask;
        a.mask_words = mask_words;
        a.P = P;
        a.M = M;
        a.n_heads = c.n_heads;
        a.n_kv = c.n_kv_heads;
        a.n_rep = c.n_heads / c.n_kv_heads;
        a.hd = c.head_dim;
        a.keys_per_wave = split.keys_per_wave;
        a.nsplit = split.nsplit;
        a.scale = (float)(1.0 / std::sqrt((double)c.head_dim));
        a.part_o = part_o;
        a.part_ml = part_ml;
        a.split_cnt = split_cnt;
        a.split_cnt_len = c.n_heads;
        a.out16 = ap;
        a.out_ld = ap_ld;
        {
            GemmParams p{};
            gemm_workspace(p);
            const bool bias = c.arch == 1;
            int t0 = 0;
            p.seg[0] = seg_of(L[K_ATTN_Q], t0, qkv, QKVD, 0, bias ? (const float *)L[K_BQ].d : nullptr);
            t0 += L[K_ATTN_Q].rows / 16;
            p.seg[1] = seg_of(L[K_ATTN_K], t0, qkv, QKVD, QD, bias ? (const float *)L[K_BK].d : nullptr);
            t0 += L[K_ATTN_K].rows / 16;
            p.seg[2] = seg_of(L[K_ATTN_V], t0, qkv, QKVD, QD + KVD, bias ? (const float *)L[K_BV].d : nullptr);
            t0 += L[K_ATTN_V].rows / 16;
            p.nseg = 3;
            p.ntiles = t0;
            p.xp = xp;
            p.K = H;
            p.M = M;
            p.mode = GM_STORE;
            p.allow_split = split_ok;
            if (spread) {
                p.norm_ssq = ssq;
                p.norm_parts = sp_parts;
                p.norm_eps = c.rms_eps;
            }
            if (fused) {
                p.norm_ssq = ssq;
                p.norm_parts = np;
                p.norm_eps = c.rms_eps;
                RopeOut &R = p.rope;
                R.pos = d_pos;
                R.cos_t = cos_t;
                R.sin_t = sin_t;
                R.q16 = q16;
                R.kc = kc(l);
                R.vc = vc(l);
                R.cap = cap;
                R.P = P;
                R.n_heads = c.n_heads;
                R.n_kv = c.n_kv_heads;
                R.hd = c.head_dim;
                R.interleaved = c.arch == 0;
            }
            const double wqkv = wbytes(L[K_ATTN_Q]) + wbytes(L[K_ATTN_K]) + wbytes(L[K_ATTN_V]);
            if (qa_fits(p, a)) {
                // the attention's workgroups ride in the Q/K/V launch
                nks_qkv = 1;
                qa_launched = true;
                // a launch number per launch, never 0 (the flags' initial value)
                if (++qa_epoch >= 0x80000000u) qa_epoch = 1;
                const QkvAttnSync sy{qa_flags, kQaFlags, qa_epoch, qa_status_dev, fault_polls};
                if (prof_on) {
                    const int ev = prof_events();
                    launch_qkv_attention(p, a, sy, n_cus, st, LaunchTiming{ev_pool[ev], ev_pool[ev + 1]});
                    prof.push_back(ProfEntry{PC_QKV_ATTN, gemm_bytes(p, wqkv) + kv_bytes, ev});
                } else {
                    launch_qkv_attention(p, a, sy, n_cus, st);
                }
            } else {
                run_gemm(p, PC_QKV, wqkv);
                nks_qkv = qgemm_slices(p);
            }
        }
        {
            RopeKvParams r{};
            r.qkv = qkv;
            r.ld_qkv = QKVD;
            r.pos = d_pos;
            r.cos_t = cos_t;
            r.sin_t = sin_t;
            r.q16 = q16;
            r.kc = kc(l);
            r.vc = vc(l);
            r.cap = cap;
            r.P = P;
            r.M = M;
            r.n_heads = c.n_heads;
            r.n_kv = c.n_kv_heads;
            r.hd = c.head_dim;
            r.interleaved = c.arch == 0;
            r.part = qg_part;
            r.nks = nks_qkv;
            if (c.arch == 1) {
                r.bq = (const float *)L[K_BQ].d;
                r.bk = (const float *)L[K_BK].d;
                r.bv = (const float *)L[K_BV].d;
            }
            if (spread) {
                r.norm_ssq = ssq;
                r.norm_parts = sp_parts;
                r.norm_K = H;
                r.norm_eps = c.rms_eps;
            }
            if (!fused) launch_rope_kv(r, st);
            if (!qa_launched) {
                if (prof_on) {
                    const int ev = prof_begin();
                    launch_attention(a, st);
                    prof_end(ev, PC_ATTN, kv_bytes);
                } else {
                    launch_attention(a, st);
                }
            }
        }
        {
            GemmParams p{};
            gemm_workspace(p);
            p.seg[0] = seg_of(L[K_ATTN_O], 0, h, H, 0, nullptr);
            p.nseg = 1;
            p.ntiles = L[K_ATTN_O].rows / 16;
            p.xp = ap;
            p.K = QD;
            p.M = M;
            p.mode = GM_RESID;
            p.allow_split = split_ok;
            if (fused) {
                p.next_w = (const float *)L[K_FFN_NORM].d;
                p.next_u = xp;
                p.next_ld = xp_ld;
                p.next_ssq = ssq;
            }
            run_gemm(p, PC_WO, wbytes(L[K_ATTN_O]));
            pend = qgemm_slices(p);
        }
        if (spread)
            launch_resid_u(h, (const float *)L[K_FFN_NORM].d, M, H, qg_part, pend, xp, xp_ld, ssq, st);
        else if (!fused)
            launch_rmsnorm(h, (const float *)L[K_FFN_NORM].d, M, H, c.rms_eps, xp, xp_ld, nullptr, st, qg_part, pend);
        {
            GemmParams p{};
            gemm_workspace(p);
            p.seg[0] = seg_of(L[K_FFN_GATE], 0, nullptr, 0, 0, nullptr);
            p.seg[1] = seg_of(L[K_FFN_UP], 0, nullptr, 0, 0, nullptr);
            p.nseg = 2;
            p.ntiles = L[K_FFN_GATE].rows / 16 * 2;
            p.xp = xp;
            p.K = H;
            p.M = M;
            p.mode = GM_SWIGLU;
            p.act = act;
            p.act_ld = act_ld;
            if (fused || spread) {
                p.norm_ssq = ssq;
                p.norm_parts = fused ? np : sp_parts;
                p.norm_eps = c.rms_eps;
            }
            if (L[K_FFN_GATE].fmt != L[K_FFN_UP].fmt) throw UnsupportedError("ffn_gate and ffn_up must share a format");
            run_gemm(p, PC_GATE_UP, wbytes(L[K_FFN_GATE]) + wbytes(L[K_FFN_UP]));
        }
        {
            GemmParams p{};
            gemm_workspace(p);
            p.seg[0] = seg_of(L[K_FFN_DOWN], 0, h, H, 0, nullptr);
            p.nseg = 1;
            p.ntiles = L[K_FFN_DOWN].rows / 16;
            p.xp = act;
            p.K = c.ffn;
            p.M = M;
            p.mode = GM_RESID;
            p.allow_split = split_ok;
            if (fused) {
                p.next_w = (const float *)(l + 1 < c.n_layers ? lw[l + 1][K_ATTN_NORM] : gw[K_OUTPUT_NORM]).d;
                p.next_u = xp;
                p.next_ld = xp_ld;
                p.next_ssq = ssq;
            }
            run_gemm(p, PC_DOWN, wbytes(L[K_FFN_DOWN]));
            pend = qgemm_slices(p);
        }
        for (size_t ci = 0; ci < collect.size(); ci++)
            if (collect[ci] == l)
                SD_HIP_CHECK(hipMemcpyAsync(collect_buf + ci * H, h + (size_t)(M - 1) * H, H * 4,
                                            hipMemcpyDeviceToDevice, st));
    }
    // the lm_head over all rows reads u and scales; other requests normalise here
    const bool spread_head = spread && logits_mode == 2;
    if (spread_head) {
        launch_resid_u(h, (const float *)gw[K_OUTPUT_NORM].d, M, H, qg_part, pend, xp, xp_ld, ssq, st);
        if (want_hidden)  // h is complete: the final-norm hidden rows only
            launch_rmsnorm(h, (const float *)gw[K_OUTPUT_NORM].d, M, H, c.rms_eps, nullptr, 0, hidden_out, st);
    } else if (!fused) {
        launch_rmsnorm(h, (const float *)gw[K_OUTPUT_NORM].d, M, H, c.rms_eps, xp, xp_ld,
                       want_hidden ? hidden_out : nullptr, st, qg_part, pend);
    } else if (want_hidden) {  // the final-norm hidden rows only; the lm_head input is already in xp
        launch_rmsnorm(h, (const float *)gw[K_OUTPUT_NORM].d, M, H, c.rms_eps, nullptr, 0, hidden_out, st);
    }
    logits_rows_last = 0;
    if (logits_mode != 0) {
        const DevTensor &W = c.tied_output ? gw[K_TOK_EMBD] : gw[K_OUTPUT];
        const int rows = logits_mode == 1 ? 1 : M;
        GemmParams p{};
        gemm_workspace(p);
        p.seg[0] = seg_of(W, 0, logits, c.vocab, 0, nullptr);
        p.nseg = 1;
        p.ntiles = W.rows / 16;
        p.xp = xp + (logits_mode == 1 ? (size_t)(M - 1) * xp_ld : 0);
        p.K = H;
        p.M = rows;
        p.mode = GM_LOGITS;
        p.amax_v = amax_v;
        p.amax_i = amax_i;
        if (fused) {
            p.norm_ssq = ssq + (logits_mode == 1 ? (size_t)(M - 1) * np : 0);
            p.norm_parts = np;
            p.norm_eps = c.rms_eps;
        } else if (spread_head) {
            p.norm_ssq = ssq;
            p.norm_parts = sp_parts;
            p.norm_eps = c.rms_eps;
        }
        if (xp_ld != H) throw UnsupportedError("lm_head needs hidden == q_dim activations stride");
        p.amax_ld = qgemm_workgroups(p);
        if (p.amax_ld > amax_ld) throw BackendError("argmax workspace too small");
        run_gemm(p, PC_LM_HEAD, wbytes(W));
        launch_argmax_reduce(amax_v, amax_i, p.amax_ld, rows, argmax, st);
        logits_rows_last = rows;
    }
    if (!collect.empty() && collect_out) {
        SD_HIP_CHECK(hipMemcpyAsync(collect_out, collect_buf, collect.size() * H * 4, hipMemcpyDeviceToHost, st));
    }
}

// apply_lm_head and embed_tokens take &self in the reference
// (model/mod.rs:148, 182): they run on buffers of their own (aux_*), in
// chunks of kAuxRows rows, and leave the verify pass's logits, argmax rows,
// hidden states and inputs as they were.  Chunks of <= 16 rows run the M <= 16
// matmul, whose rows do not depend on the chunking.
void Model::lm_head_rows(const float *hidden_host, int rows, float *out_host) {
    const ModelCfg &c = cfg;
    SD_HIP_CHECK(hipSetDevice(c.device));
    const DevTensor &W = c.tied_output ? gw[K_TOK_EMBD] : gw[K_OUTPUT];
    for (int r0 = 0; r0 < rows; r0 += kAuxRows) {
        const int n = std::min(kAuxRows, rows - r0);
        SD_HIP_CHECK(hipMemcpyAsync(aux_h, hidden_host + (size_t)r0 * c.hidden, (size_t)n * c.hidden * 4,
                                    hipMemcpyHostToDevice, st));
        launch_to_frag16(aux_h, n, c.hidden, aux_x, c.hidden, st);
        GemmParams p{};
        p.seg[0] = seg_of(W, 0, aux_y, c.vocab, 0, nullptr);
        p.nseg = 1;
        p.ntiles = W.rows / 16;
        p.xp = aux_x;
        p.K = c.hidden;
        p.M = n;
        p.mode = GM_STORE;
        launch_qgemm(p, st);
        SD_HIP_CHECK(hipMemcpyAsync(out_host + (size_t)r0 * c.vocab, aux_y, (size_t)n * c.vocab * 4,
                                    hipMemcpyDeviceToHost, st));
        sync();
    }
}

void Model::lm_head_device(const uint16_t *xp, int M, float *out, hipStream_t s) {
    if (M < 1 || M > 16) throw ArgError("lm_head_device: 1 to 16 rows");
    const DevTensor &W = cfg.tied_output ? gw[K_TOK_EMBD] : gw[K_OUTPUT];
    GemmParams p{};
    p.seg[0] = seg_of(W, 0, out, cfg.vocab, 0, nullptr);
    p.nseg = 1;
    p.ntiles = W.rows / 16;
    p.xp = xp;
    p.K = cfg.hidden;
    p.M = M;
    p.mode = GM_STORE;
    launch_qgemm(p, s);
}

void Model::embed_rows(const int *ids, int n, float *out_host) {
    const ModelCfg &c = cfg;
    SD_HIP_CHECK(hipSetDevice(c.device));
    for (int i = 0; i < n; i++)
        if (ids[i] < 0 || ids[i] >= c.vocab) throw ArgError("token id out of range");
    for (int r0 = 0; r0 < n; r0 += kAuxRows) {
        const int k = std::min(kAuxRows, n - r0);
        SD_HIP_CHECK(hipMemcpyAsync(aux_ids, ids + r0, k * sizeof(int), hipMemcpyHostToDevice, st));
        launch_embed(gw[K_TOK_EMBD].fmt, embed_table(), c.hidden, aux_ids, k, aux_h, st);
        SD_HIP_CHECK(hipMemcpyAsync(out_host + (size_t)r0 * c.hidden, aux_h, (size_t)k * c.hidden * 4,
                                    hipMemcpyDeviceToHost, st));
        sync();
    }
}

void Model::compact_tail(int P, const std::vector<int> &src) {
    fwd_count++;
    const int n = (int)src.size();
    if (n == 0) return;
    SD_HIP_CHECK(hipSetDevice(cfg.device));
    stage_wait();
    std::memcpy(h_stage, src.data(), n * sizeof(int));
    SD_HIP_CHECK(hipMemcpyAsync(d_src, h_stage, n * sizeof(int), hipMemcpyHostToDevice, st));
    stage_done();
    launch_keep_kv_tail(kv, cfg.n_layers * 2 * cfg.n_kv_heads, cap * cfg.head_dim, cfg.n_kv_heads, cfg.head_dim, P, d_src,
                        n, st);
}

// ===========================================================================
// DraftTree (tree.rs)
// ===========================================================================
DraftTreeC DraftTreeC::from_arrays(const uint32_t *tokens, const uint32_t *parents, size_t n) {
    if (n == 0) throw SamplingError("DraftTree must have at least a root");
    DraftTreeC t;
    t.tokens.assign(tokens, tokens + n);
    t.parents.assign(n, 0);
    for (size_t i = 1; i < n; i++) {
        if (parents[i] >= i)
            throw SamplingError("node " + std::to_string(i) + " has parent index " + std::to_string(parents[i]) +
                                ", which is not strictly smaller");
        t.parents[i] = parents[i];
    }
    return t;
}

int DraftTreeC::depth_of(size_t i) const {
    int d = 0;
    while (i != 0) {
        i = parents[i];
        d++;
    }
    return d;
}

bool DraftTreeC::is_ancestor_of(size_t a, size_t n) const {
    size_t cur = n;
    if (cur == a) return true;
    while (cur != 0) {
        cur = parents[cur];
        if (cur == a) return true;
    }
    return a == 0;
}

std::vector<std::vector<size_t>> DraftTreeC::paths() const {
    std::vector<bool> leaf(size(), true);
    for (size_t i = 1; i < size(); i++) leaf[parents[i]] = false;
    std::vector<std::vector<size_t>> out;
    for (size_t i = 0; i < size(); i++) {
        if (!leaf[i]) continue;
        std::vector<size_t> chain{i};
        size_t c = i;
        while (c != 0) {
            c = parents[c];
            chain.push_back(c);
        }
        std::reverse(chain.begin(), chain.end());
        out.push_back(chain);
    }
    return out;
}

void DraftTreeC::masks(std::vector<uint64_t> &words, int &nw) const {
    const size_t n = size();
    nw = (int)((n + 63) / 64);
    words.assign(n * nw, 0ull);
    for (size_t i = 0; i < n; i++) {
        size_t c = i;
        while (true) {
            words[i * nw + c / 64] |= 1ull << (c % 64);
            if (c == 0) break;
            c = parents[c];
        }
    }
}

// ===========================================================================
// Decoder (quantized_llama.rs)
// ===========================================================================
static void causal_masks(int M, std::vector<uint64_t> &w, int &nw) {
    nw = (M + 63) / 64;
    w.assign((size_t)M * nw, 0ull);
    for (int i = 0; i < M; i++)
        for (int j = 0; j <= i; j++) w[(size_t)i * nw + j / 64] |= 1ull << (j % 64);
}

void Decoder::reset() {
    history.clear();
    cache_len = 0;
    last_valid = false;
    collect_hist = 0;
}

void Decoder::truncate(size_t len) {
    // ModelWeights::truncate_kv_cache_to (quantized_llama_local.rs:162-175, 441-446)
    if ((int)len > cache_len) throw BackendError("truncate_kv_cache_to(" + std::to_string(len) + ") exceeds " +
                                                 std::to_string(cache_len));
    cache_len = (int)len;
}

// forward_advance_logits (quantized_llama.rs:137-158): forward `tokens` at the
// cache end; caches the last row's logits.  Chunks longer inputs by max_batch.
void Decoder::forward_advance(const uint32_t *tokens, size_t n, bool all_rows) {
    if (n == 0) throw SamplingError("forward_advance with empty tokens");
    Model &m = *model;
    const int V = m.cfg.vocab;
    for (size_t i = 0; i < n; i++)
        if (tokens[i] >= (uint32_t)V) throw ArgError("token id out of range");
    if (all_rows && n > (size_t)m.cfg.max_batch) throw ArgError("too many rows for one verify pass");
    if (cache_len + n > (size_t)m.cfg.ctx_len) throw ArgError("KV capacity exceeded");
    size_t done = 0;
    std::vector<int> ids, pos;
    std::vector<uint64_t> mw;
    int nw;
    while (done < n) {
        const int M = (int)std::min<size_t>(m.cfg.max_batch, n - done);
        const bool last_chunk = done + M == n;
        ids.assign(tokens + done, tokens + done + M);
        pos.resize(M);
        for (int i = 0; i < M; i++) pos[i] = cache_len + i;
        causal_masks(M, mw, nw);
        const bool keep = n == 1 && !collect_keep.empty();
        m.forward(ids.data(), pos.data(), mw.data(), nw, M, cache_len, last_chunk ? (all_rows ? 2 : 1) : 0, false,
                  keep ? collect_keep : std::vector<int>{}, nullptr);
        cache_len += M;
        done += M;
    }
    const int rows = m.logits_rows_last;
    SD_HIP_CHECK(hipMemcpyAsync(m.last_row, m.logits + (size_t)(rows - 1) * V, (size_t)V * 4,
                                hipMemcpyDeviceToDevice, m.st));
    last_valid = true;
}

void Decoder::observe(const uint32_t *ids, size_t n) {
    if (n == 0) return;
    forward_advance(ids, n, false);
    history.insert(history.end(), ids, ids + n);
    if (n == 1 && !collect_keep.empty()) {
        collect_hist = history.size();
        collect_fwd = model->fwd_count;
    }
    model->sync();
}

void Decoder::next_logits(float *out) {
    if (history.empty()) throw SamplingError("next_logits called with empty history");
    Model &m = *model;
    if (!last_valid) {
        const uint32_t last = history.back();
        truncate(history.size() - 1);
        forward_advance(&last, 1, false);
    }
    if (out) SD_HIP_CHECK(hipMemcpyAsync(out, m.last_row, (size_t)m.cfg.vocab * 4, hipMemcpyDeviceToHost, m.st));
    m.sync();
}

void Decoder::batched_logits(const uint32_t *drafts, size_t k, float *out) {
    if (k == 0) {
        next_logits(out);
        return;
    }
    if (history.empty()) throw SamplingError("batched_logits with empty history");
    Model &m = *model;
    if (k + 1 > (size_t)m.cfg.max_batch) throw ArgError("too many draft tokens for one verify pass");
    for (size_t i = 0; i < k; i++)
        if (drafts[i] >= (uint32_t)m.cfg.vocab) throw ArgError("token id out of range");
    // every check forward_advance makes, before the cache is touched: a
    // failed call leaves the decoder as it was
    if (history.size() - 1 + k + 1 > (size_t)m.cfg.ctx_len) throw ArgError("KV capacity exceeded");
    const uint32_t last = history.back();
    truncate(history.size() - 1);
    std::vector<uint32_t> comb;
    comb.push_back(last);
    comb.insert(comb.end(), drafts, drafts + k);
    forward_advance(comb.data(), comb.size(), true);
    history.insert(history.end(), drafts, drafts + k);
    if (out) {
        SD_HIP_CHECK(hipMemcpyAsync(out, m.logits, (k + 1) * (size_t)m.cfg.vocab * 4, hipMemcpyDeviceToHost, m.st));
        m.sync();
    }
    // without `out` the rows stay on the device for the caller's own kernels,
    // queued behind the forward on the same stream (the device-acceptance
    // entry points, which synchronise once at their end)
}

void Decoder::rollback_to(size_t len) {
    if (len > history.size())
        throw RollbackError("rollback target " + std::to_string(len) + " > history length " +
                            std::to_string(history.size()));
    history.resize(len);
    last_valid = false;
    truncate(len);
}

void Decoder::tree_forward(const uint32_t *tokens, const uint32_t *parents, size_t n, bool want_hidden,
                           int &prefix) {
    Model &m = *model;
    const DraftTreeC t = DraftTreeC::from_arrays(tokens, parents, n);
    const uint32_t last = history.back();
    if (t.tokens[0] != last)
        throw SamplingError("tree root (" + std::to_string(t.tokens[0]) + ") must equal last committed token (" +
                            std::to_string(last) + ")");
    if (n > (size_t)m.cfg.max_batch) throw ArgError("tree larger than max_batch");
    for (size_t i = 0; i < n; i++)
        if (tokens[i] >= (uint32_t)m.cfg.vocab) throw ArgError("token id out of range");
    prefix = cache_len - 1;
    if (prefix + (int)n > m.cfg.ctx_len) throw ArgError("KV capacity exceeded");
    truncate(prefix);
    std::vector<int> ids(tokens, tokens + n), pos(n);
    for (size_t i = 0; i < n; i++) pos[i] = prefix + t.depth_of(i);
    std::vector<uint64_t> mw;
    int nw;
    t.masks(mw, nw);
    m.forward(ids.data(), pos.data(), mw.data(), nw, (int)n, prefix, 2, want_hidden, {}, nullptr);
}

void Decoder::tree_logits_keep_kv(const uint32_t *tokens, const uint32_t *parents, size_t n, float *out_logits,
                                  float *out_hidden) {
    last_valid = false;
    if (history.empty()) throw SamplingError("tree_logits with empty history");
    Model &m = *model;
    int prefix;
    tree_forward(tokens, parents, n, true, prefix);
    cache_len = prefix + (int)n;
    if (out_logits)
        SD_HIP_CHECK(hipMemcpyAsync(out_logits, m.logits, n * (size_t)m.cfg.vocab * 4, hipMemcpyDeviceToHost, m.st));
    if (out_hidden)
        SD_HIP_CHECK(
            hipMemcpyAsync(out_hidden, m.hidden_out, n * (size_t)m.cfg.hidden * 4, hipMemcpyDeviceToHost, m.st));
    m.sync();
}

void Decoder::tree_logits(const uint32_t *tokens, const uint32_t *parents, size_t n, float *out_logits) {
    if (history.empty()) throw SamplingError("tree_logits with empty history");
    Model &m = *model;
    const uint32_t last = history.back();
    int prefix;
    tree_forward(tokens, parents, n, false, prefix);
    if (out_logits)
        SD_HIP_CHECK(hipMemcpyAsync(out_logits, m.logits, n * (size_t)m.cfg.vocab * 4, hipMemcpyDeviceToHost, m.st));
    m.sync();
    truncate(prefix);
    forward_advance(&last, 1, false);  // restores the cache and the cached next-token row
    // Llama replaces row 0 by the one-token pass's row (quantized_llama.rs:306-322); Qwen2 discards that
    // row and keeps the tree pass's row 0 (quantized_qwen2.rs:227-234).
    if (out_logits && m.cfg.arch == 0)
        SD_HIP_CHECK(hipMemcpyAsync(out_logits, m.last_row, (size_t)m.cfg.vocab * 4, hipMemcpyDeviceToHost, m.st));
    m.sync();
}

void Decoder::commit_tree_path(const uint32_t *tokens, const uint32_t *parents, size_t n, const uint32_t *acc,
                               size_t n_acc) {
    last_valid = false;
    if (history.empty()) throw SamplingError("commit_tree_path with empty history");
    const DraftTreeC t = DraftTreeC::from_arrays(tokens, parents, n);
    const int prefix = (int)history.size() - 1;
    // keep = [0..prefix) ++ [prefix + ti]; every index must exist in the cache
    std::vector<int> src(n_acc);
    for (size_t j = 0; j < n_acc; j++) {
        if (acc[j] >= n || prefix + (int)acc[j] >= cache_len)
            throw BackendError("commit_tree_path: accepted index out of range of the tree / cache");
        src[j] = (int)acc[j];
    }
    if (n_acc == 0) {
        // keep_kv_indices(&[0..prefix)) keeps the prefix only
        cache_len = prefix;
    } else {
        model->compact_tail(prefix, src);
        cache_len = prefix + (int)n_acc;
    }
    for (size_t j = 1; j < n_acc; j++) history.push_back(t.tokens[acc[j]]);
    model->sync();
}

void Decoder::last_hidden_state(float *out) {
    if (history.empty()) throw SamplingError("last_hidden_state with empty history");
    Model &m = *model;
    const uint32_t last = history.back();
    truncate(history.size() - 1);
    int id = (int)last, pos = cache_len;
    uint64_t mk = 1;
    m.forward(&id, &pos, &mk, 1, 1, cache_len, 0, true, {}, nullptr);
    cache_len += 1;
    if (out) SD_HIP_CHECK(hipMemcpyAsync(out, m.hidden_out, (size_t)m.cfg.hidden * 4, hipMemcpyDeviceToHost, m.st));
    m.sync();
}

void Decoder::observe_returning_last_hidden(const uint32_t *ids, size_t n, float *out) {
    if (n == 0) throw SamplingError("observe_returning_last_hidden with empty ids");
    Model &m = *model;
    if (cache_len + n > (size_t)m.cfg.ctx_len) throw ArgError("KV capacity exceeded");
    for (size_t i = 0; i < n; i++)
        if (ids[i] >= (uint32_t)m.cfg.vocab) throw ArgError("token id out of range");
    size_t done = 0;
    std::vector<int> tk, pos;
    std::vector<uint64_t> mw;
    int nw;
    int lastM = 1;
    while (done < n) {
        const int M = (int)std::min<size_t>(m.cfg.max_batch, n - done);
        tk.assign(ids + done, ids + done + M);
        pos.resize(M);
        for (int i = 0; i < M; i++) pos[i] = cache_len + i;
        causal_masks(M, mw, nw);
        m.forward(tk.data(), pos.data(), mw.data(), nw, M, cache_len, 0, done + M == n, {}, nullptr);
        cache_len += M;
        done += M;
        lastM = M;
    }
    history.insert(history.end(), ids, ids + n);
    if (out)
        SD_HIP_CHECK(hipMemcpyAsync(out, m.hidden_out + (size_t)(lastM - 1) * m.cfg.hidden, (size_t)m.cfg.hidden * 4,
                                    hipMemcpyDeviceToHost, m.st));
    m.sync();
}

void Decoder::last_hidden_states_multi(const uint32_t *layers, size_t nl, float *out_final, float *out_layers) {
    if (history.empty()) throw SamplingError("last_hidden_states_multi with empty history");
    Model &m = *model;
    if (nl > (size_t)m.collect_cap) throw ArgError("too many collected layers");
    std::vector<int> col(nl);
    for (size_t i = 0; i < nl; i++) {
        if (layers[i] >= (uint32_t)m.cfg.n_layers)
            throw BackendError("collect_layers[" + std::to_string(i) + "] = " + std::to_string(layers[i]) +
                               " out of range (n_layers=" + std::to_string(m.cfg.n_layers) + ")");
        col[i] = (int)layers[i];
    }
    const uint32_t last = history.back();
    truncate(history.size() - 1);
    int id = (int)last, pos = cache_len;
    uint64_t mk = 1;
    std::vector<float> tmp(nl * (size_t)m.cfg.hidden);
    m.forward(&id, &pos, &mk, 1, 1, cache_len, 0, true, col, tmp.data());
    cache_len += 1;
    collect_keep = col;
    collect_hist = history.size();
    collect_fwd = m.fwd_count;
    if (out_final)
        SD_HIP_CHECK(hipMemcpyAsync(out_final, m.hidden_out, (size_t)m.cfg.hidden * 4, hipMemcpyDeviceToHost, m.st));
    m.sync();
    if (out_layers) std::memcpy(out_layers, tmp.data(), tmp.size() * 4);
}

// last_hidden_states_multi with the rows left on the device: [nl][hidden] f32
// in collect_buf, ready on the model's stream (the caller does not wait)
const float *Decoder::collect_hidden_device(const uint32_t *layers, size_t nl) {
    if (history.empty()) throw SamplingError("last_hidden_states_multi with empty history");
    Model &m = *model;
    if (nl > (size_t)m.collect_cap) throw ArgError("too many collected layers");
    std::vector<int> col(nl);
    for (size_t i = 0; i < nl; i++) {
        if (layers[i] >= (uint32_t)m.cfg.n_layers)
            throw BackendError("collect_layers[" + std::to_string(i) + "] = " + std::to_string(layers[i]) +
                               " out of range (n_layers=" + std::to_string(m.cfg.n_layers) + ")");
        col[i] = (int)layers[i];
    }
    // the rows of this token from the one-token forward that appended it
    // (observe) or from the last collection: the same M=1 forward at the same
    // position over the same cache, so the same values
    if (collect_hist == history.size() && collect_fwd == m.fwd_count && collect_keep == col &&
        cache_len == (int)history.size())
        return m.collect_buf;
    const uint32_t last = history.back();
    truncate(history.size() - 1);
    int id = (int)last, pos = cache_len;
    uint64_t mk = 1;
    m.forward(&id, &pos, &mk, 1, 1, cache_len, 0, true, col, nullptr);
    cache_len += 1;
    collect_keep = col;
    collect_hist = history.size();
    collect_fwd = m.fwd_count;
    return m.collect_buf;
}

// ---- device acceptance -----------------------------------------------------
void Decoder::argmax_rows(int32_t *out, size_t n) {
    Model &m = *model;
    if (n > (size_t)m.logits_rows_last) throw ArgError("fewer rows in the last verify pass");
    // through the pinned output region of the acceptance staging block (a
    // direct copy; a pageable destination goes through the runtime's own
    // staging buffer first)
    int *pin = m.acc_stage + (size_t)kAccTreeInts * m.cfg.max_batch;
    SD_HIP_CHECK(hipMemcpyAsync(pin, m.argmax, n * 4, hipMemcpyDeviceToHost, m.st));
    m.sync();
    std::memcpy(out, pin, n * 4);
}

// batched_logits + greedy acceptance with the logits kept in HBM:
// accept drafts while draft[i] == argmax(row i); the first mismatch (or the
// bonus row k) contributes argmax of that row (vanilla.rs:178-210 at T=0,
// equivalently the first-max fold of eagle.rs:626-637).
void Decoder::verify_greedy_linear(const uint32_t *drafts, size_t k, uint32_t *commits, size_t *n_commit,
                                   size_t *n_accepted) {
    batched_logits(drafts, k, nullptr);
    std::vector<int32_t> am(k + 1);
    if (k == 0) {
        launch_argmax_rows(model->last_row, model->cfg.vocab, model->cfg.vocab, 1, model->argmax, model->st);
        model->logits_rows_last = 1;
    }
    argmax_rows(am.data(), k + 1);
    size_t a = 0;
    while (a < k && (uint32_t)am[a] == drafts[a]) a++;
    for (size_t i = 0; i < a; i++) commits[i] = drafts[i];
    commits[a] = (uint32_t)am[a];
    *n_commit = a + 1;
    *n_accepted = a;
}

// tree_logits_keep_kv + greedy longest accepted path (eagle.rs:605-661):
// paths in ascending leaf order, a strictly longer count replaces the best
// (ties keep the earliest leaf); bonus = argmax of the deepest accepted node;
// bonus_node = first child of that node carrying the bonus token (eagle.rs:700-709),
// -1 if none or in strict mode.
void Decoder::verify_greedy_tree(const uint32_t *tokens, const uint32_t *parents, size_t n, int strict,
                                 uint32_t *path, size_t *path_len, uint32_t *bonus, int32_t *bonus_node,
                                 uint32_t *committed, size_t *n_committed, size_t *keep_len, int32_t *stop) {
    if (history.empty()) throw SamplingError("tree_logits with empty history");
    Model &m = *model;
    int32_t root_am = -1;
    if (strict) {
        next_logits(nullptr);
        launch_argmax_rows(m.last_row, m.cfg.vocab, m.cfg.vocab, 1, m.argmax, m.st);
        int *pin = m.acc_stage + (size_t)kAccTreeInts * m.cfg.max_batch;  // pinned (see argmax_rows)
        SD_HIP_CHECK(hipMemcpyAsync(pin, m.argmax, 4, hipMemcpyDeviceToHost, m.st));
        m.sync();
        root_am = pin[0];
    }
    tree_logits_keep_kv(tokens, parents, n, nullptr, nullptr);
    std::vector<int32_t> am(n);
    argmax_rows(am.data(), n);
    if (strict) am[0] = root_am;
    const DraftTreeC t = DraftTreeC::from_arrays(tokens, parents, n);
    std::vector<size_t> best{0};
    for (const auto &p : t.paths()) {
        size_t acc = 0;
        for (size_t w = 0; w + 1 < p.size(); w++) {
            if ((uint32_t)am[p[w]] == t.tokens[p[w + 1]]) acc++;
            else break;
        }
        if (acc + 1 > best.size()) best.assign(p.begin(), p.begin() + acc + 1);
    }
    for (size_t i = 0; i < best.size(); i++) path[i] = (uint32_t)best[i];
    *path_len = best.size();
    const size_t deepest = best.back();
    *bonus = (uint32_t)am[deepest];
    // Commit composition (eagle.rs:664-732, eagle3.rs:758-782): committed =
    // the path's tokens and the bonus, cut after the first EOS (stop); an EOS
    // among the path's tokens keeps the path up to that node and takes no
    // bonus forward, otherwise the whole path is kept and the bonus joins it
    // when a child of the deepest node carries it (not in strict mode).
    auto is_eos = [&](uint32_t x) { return std::find(eos.begin(), eos.end(), x) != eos.end(); };
    std::vector<uint32_t> com;
    for (size_t i = 1; i < best.size(); i++) com.push_back(t.tokens[best[i]]);
    size_t eos_in_path = com.size();
    for (size_t i = 0; i < com.size(); i++)
        if (is_eos(com[i])) {
            eos_in_path = i;
            break;
        }
    com.push_back(*bonus);
    size_t cut = com.size();
    for (size_t i = 0; i < com.size(); i++)
        if (is_eos(com[i])) {
            cut = i + 1;
            break;
        }
    *stop = cut < com.size() || is_eos(com.back()) ? 1 : 0;
    com.resize(cut);
    if (committed) std::copy(com.begin(), com.end(), committed);
    *n_committed = com.size();
    *bonus_node = -1;
    if (eos_in_path < best.size() - 1) {
        *keep_len = eos_in_path + 2;  // root + the path through the EOS node
    } else {
        *keep_len = best.size();
        if (!strict)
            for (size_t c = 1; c < n; c++)
                if (t.parents[c] == deepest && t.tokens[c] == *bonus) {
                    *bonus_node = (int32_t)c;
                    break;
                }
    }
}

// ---- rejection sampling ------------------------------------------------------
// EAGLE-3's d2t table (eagle3.rs:377-397): draft id -> absolute target id;
// entries outside [0, vocab) are ignored; the inverse keeps the last writer.
void Decoder::set_d2t(const int64_t *d2t, size_t n) {
    Model &m = *model;
    if (n == 0 || n > (size_t)INT32_MAX) throw ArgError("d2t: size out of range");
    std::vector<int32_t> inv((size_t)m.cfg.vocab, -1);
    for (size_t i = 0; i < n; i++)
        if (d2t[i] >= 0 && d2t[i] < m.cfg.vocab) inv[(size_t)d2t[i]] = (int32_t)i;
    SD_HIP_CHECK(hipSetDevice(m.cfg.device));
    if (!m.t2d_inv) SD_HIP_CHECK(hipMalloc((void **)&m.t2d_inv, (size_t)m.cfg.vocab * sizeof(int) + 256));
    SD_HIP_CHECK(hipMemcpyAsync(m.t2d_inv, inv.data(), inv.size() * sizeof(int), hipMemcpyHostToDevice, m.st));
    m.sync();
    d2t_host.assign(d2t, d2t + n);
    t2d_host = std::move(inv);
    m.d2t_draft_vocab = (int)n;
}

// Draft rows the caller already holds in device memory: they must be device
// (or device-accessible managed) memory of this model's GPU.
static void check_device_rows(const Model &m, const float *q, size_t n) {
    if (n == 0) return;
    if (!q) throw ArgError("draft rows: null device pointer");
    hipPointerAttribute_t at{};
    if (hipPointerGetAttributes(&at, q) != hipSuccess) {
        (void)hipGetLastError();
        throw ArgError("draft rows: not a device allocation");
    }
    if (at.type != hipMemoryTypeDevice && at.type != hipMemoryTypeManaged)
        throw ArgError("draft rows: not device memory");
    if (at.device != m.cfg.device) throw ArgError("draft rows: memory of another device");
}

void Decoder::accept_walk(const int *parents, const int *tokens, int n, const float *q_rows, bool q_on_device,
                          size_t q_rows_n, size_t q_vocab, const int *q_row_of, const float *uniforms,
                          float temperature, int use_t2d, int wor, size_t max_commit, std::vector<int> &path, int &fin,
                          size_t &used) {
    Model &m = *model;
    const ModelCfg &c = m.cfg;
    if (m.logits_rows_last < n) throw BackendError("acceptance: fewer logits rows than tree nodes");
    const size_t qn = q_rows_n * q_vocab;
    if (!q_on_device && qn > m.acc_q_cap) {
        if (m.acc_q) SD_HIP_CHECK(hipFree(m.acc_q));
        m.acc_q = nullptr;
        m.acc_q_cap = 0;
        SD_HIP_CHECK(hipMalloc((void **)&m.acc_q, qn * sizeof(float) + 256));
        m.acc_q_cap = qn;
    }
    const size_t pn = (size_t)n * c.vocab;
    if (pn > m.acc_prob_cap) {
        if (m.acc_prob) SD_HIP_CHECK(hipFree(m.acc_prob));
        m.acc_prob = nullptr;
        m.acc_prob_cap = 0;
        SD_HIP_CHECK(hipMalloc((void **)&m.acc_prob, pn * sizeof(float) + 256));
        m.acc_prob_cap = pn;
    }
    // parents | tokens | q_row_of | uniforms | children per node | children's
    // tokens in BFS order through the pinned acceptance stage in one copy (the
    // previous walk synchronised before returning, so the stage is free), the
    // draft rows in another unless on the device
    int *in = m.acc_stage;
    std::memcpy(in, parents, n * sizeof(int));
    std::memcpy(in + n, tokens, n * sizeof(int));
    std::memcpy(in + 2 * n, q_row_of, n * sizeof(int));
    std::memcpy(in + 3 * n, uniforms, n * sizeof(float));
    int *nchild = in + 4 * n, *kids = in + 5 * n;
    std::fill(nchild, nchild + n, 0);
    std::fill(kids, kids + (size_t)n * kAcceptMaxChildren, 0);
    for (int i = 1; i < n; i++) {
        const int p = parents[i];
        if (nchild[p] >= kAcceptMaxChildren) throw UnsupportedError("rejection walk: at most 16 children per node");
        kids[(size_t)p * kAcceptMaxChildren + nchild[p]++] = tokens[i];
    }
    const int kmax = *std::max_element(nchild, nchild + n);
    // the nodes each precomputed pass k covers (those with at least k
    // children) as records: node, children, draft row, child k's token, its
    // index into the draft row (through the t2d map for draft-vocabulary
    // rows; -1: none) and whether the t2d mask removes it from the target row
    const bool qmap = q_vocab != (size_t)c.vocab;
    int *lists = kids + (size_t)n * kAcceptMaxChildren;
    int counts[kAcceptMaxChildren + 1];
    const int *dlists[kAcceptMaxChildren + 1];
    size_t off = 0;
    for (int k = 0; k <= kmax; k++) {
        counts[k] = 0;
        dlists[k] = m.acc_tree + (lists - in) + off;
        for (int i = 0; i < n; i++) {
            if (nchild[i] < k) continue;
            int *rc = lists + off + (size_t)kTreeRec * counts[k]++;
            const int tk = k < nchild[i] ? kids[(size_t)i * kAcceptMaxChildren + k] : 0;
            const int dk = k < nchild[i] ? (qmap ? t2d_host[tk] : tk) : -1;
            rc[0] = i;
            rc[1] = nchild[i];
            rc[2] = q_row_of[i];
            rc[3] = tk;
            rc[4] = dk;
            rc[5] = use_t2d && t2d_host[tk] < 0 ? 1 : 0;
            rc[6] = rc[7] = 0;
        }
        off += (size_t)kTreeRec * counts[k];
    }
    SD_HIP_CHECK(hipMemcpyAsync(m.acc_tree, in, ((size_t)(lists - in) + off) * sizeof(int), hipMemcpyHostToDevice,
                                m.st));
    if (qn && !q_on_device)
        SD_HIP_CHECK(hipMemcpyAsync(m.acc_q, q_rows, qn * sizeof(float), hipMemcpyHostToDevice, m.st));
    const bool greedy = temperature == 0.f;
    const float inv_t = greedy ? 1.f : 1.0f / temperature;
    const int *mask = use_t2d ? m.t2d_inv : nullptr;
    launch_row_stats(m.logits, c.vocab, c.vocab, n, inv_t, mask, m.acc_part, m.acc_cnt, m.acc_m, m.acc_s, m.acc_am,
                     m.st);
    AcceptParams a{};
    a.prob = m.acc_prob;
    a.V = c.vocab;
    a.n = n;
    a.parents = m.acc_tree;
    a.tokens = m.acc_tree + n;
    a.q_row_of = m.acc_tree + 2 * n;
    a.row_m = m.acc_m;
    a.row_s = m.acc_s;
    a.row_am = m.acc_am;
    a.inv_t = inv_t;
    a.greedy = greedy ? 1 : 0;
    a.t2d_inv = mask;
    a.q = q_on_device ? q_rows : m.acc_q;
    a.q_ld = (int64_t)q_vocab;
    a.q_map = q_vocab == (size_t)c.vocab ? nullptr : m.t2d_inv;
    a.uniforms = (const float *)(m.acc_tree + 3 * n);
    a.max_commit = (int)max_commit;
    a.wor = wor;
    a.out_path = m.acc_out + 4;
    a.out_info = m.acc_out;
    // every pass the walk can make (per node, one per possible rejection and
    // the final draw), computed across the GPU first; the walk reads them
    a.nchild = m.acc_tree + 4 * n;
    a.kids = m.acc_tree + 5 * n;
    const int ntl = (c.vocab + 255) / 256;
    const size_t ln = tree_tiles_floats(n, c.vocab, kmax);
    if (ln > m.acc_lin_cap) {
        if (m.acc_lin) SD_HIP_CHECK(hipFree(m.acc_lin));
        m.acc_lin = nullptr;
        m.acc_lin_cap = 0;
        SD_HIP_CHECK(hipMalloc((void **)&m.acc_lin, ln * sizeof(float) + 256));
        m.acc_lin_cap = ln;
    }
    a.tiles = m.acc_lin;
    a.test = a.tiles + (size_t)(kmax + 1) * n * ntl;
    a.logits = m.logits;
    a.logits_ld = c.vocab;
    launch_tree_tiles(a, kmax, dlists, counts, m.st);
    launch_accept_walk(a, m.st);
    int *out = m.acc_stage + (size_t)kAccTreeInts * c.max_batch;
    SD_HIP_CHECK(hipMemcpyAsync(out, m.acc_out, ((size_t)n + 4) * sizeof(int), hipMemcpyDeviceToHost, m.st));
    m.sync();
    const int status = out[3];
    if (status == ACC_ERR_SOFTMAX) throw SamplingError("softmax produced a non-positive or non-finite sum");
    if (status == ACC_ERR_ADJUSTED) throw SamplingError("adjusted distribution has non-positive mass");
    if (status != ACC_OK) throw SamplingError("acceptance walk: too many rejections at one node");
    const int plen = out[0];
    if (plen < 1 || plen > n) throw BackendError("acceptance walk: bad path length");
    path.assign(out + 4, out + 4 + plen);
    fin = out[1];
    used = (size_t)out[2];
}

static void check_temperature(float t) {
    // softmax_with_temperature rejects these (tokens.rs:19-23)
    if (!std::isfinite(t) || t < 0.f) throw SamplingError("invalid temperature");
}

void Decoder::verify_rejection_linear(const uint32_t *drafts, size_t k, const float *q_rows, const float *uniforms,
                                      size_t n_uniforms, float temperature, size_t max_commit, uint32_t *commits,
                                      size_t *n_commit, size_t *n_accepted, size_t *n_used, bool q_on_device) {
    Model &m = *model;
    check_temperature(temperature);
    if (n_uniforms < k + 1) throw ArgError("rejection verify needs k + 1 uniforms");
    if (k + 1 > (size_t)m.cfg.max_batch) throw ArgError("too many draft tokens for one verify pass");
    if (q_on_device) check_device_rows(m, q_rows, k * (size_t)m.cfg.vocab);
    if (history.empty()) throw SamplingError("batched_logits with empty history");
    const uint32_t last = history.back();
    batched_logits(drafts, k, nullptr);
    if (k == 0) {
        // next_logits left the row in last_row; the walk reads logits row 0
        SD_HIP_CHECK(hipMemcpyAsync(m.logits, m.last_row, (size_t)m.cfg.vocab * 4, hipMemcpyDeviceToDevice, m.st));
        m.logits_rows_last = 1;
    }
    const int n = (int)k + 1;
    std::vector<int> parents(n), tokens(n), qrow(n);
    for (int i = 0; i < n; i++) {
        parents[i] = i - 1;
        tokens[i] = (int)(i == 0 ? last : drafts[i - 1]);
        qrow[i] = i < (int)k ? i : -1;
    }
    parents[0] = 0;
    std::vector<int> path;
    int fin;
    size_t used;
    accept_walk(parents.data(), tokens.data(), n, q_rows, q_on_device, k, m.cfg.vocab, qrow.data(), uniforms,
                temperature, 0, 0, max_commit, path, fin, used);
    size_t nc = 0;
    for (size_t i = 1; i < path.size(); i++) commits[nc++] = (uint32_t)tokens[path[i]];
    if (fin >= 0) commits[nc++] = (uint32_t)fin;
    *n_commit = nc;
    *n_accepted = path.size() - 1;
    *n_used = used;
}

void Decoder::verify_rejection_tree(const uint32_t *tokens, const uint32_t *parents, size_t n, const float *q_rows,
                                    size_t q_rows_n, size_t q_vocab, const int32_t *q_row_of,
                                    const float *uniforms, size_t n_uniforms, float temperature, int use_t2d,
                                    int siblings, size_t max_commit, uint32_t *path, size_t *path_len,
                                    int32_t *token, size_t *n_used, bool q_on_device) {
    Model &m = *model;
    check_temperature(temperature);
    if (siblings != 0 && siblings != 1) throw ArgError("sibling rule must be 0 (i.i.d.) or 1 (without replacement)");
    if (history.empty()) throw SamplingError("tree_logits with empty history");
    const DraftTreeC t = DraftTreeC::from_arrays(tokens, parents, n);
    if (n_uniforms < n) throw ArgError("rejection verify needs one uniform per tree node");
    if (q_vocab != (size_t)m.cfg.vocab && (q_vocab != (size_t)m.d2t_draft_vocab || !m.t2d_inv))
        throw ArgError("draft rows must span the target vocabulary, or the d2t draft vocabulary after sd_set_d2t");
    if (use_t2d && !m.t2d_inv) throw ArgError("t2d masking needs sd_set_d2t");
    if (q_on_device) check_device_rows(m, q_rows, q_rows_n * q_vocab);
    std::vector<bool> has_child(n, false);
    std::vector<int> nchild(n, 0);
    for (size_t i = 1; i < n; i++) {
        has_child[t.parents[i]] = true;
        if (++nchild[t.parents[i]] > kAcceptMaxChildren)
            throw UnsupportedError("rejection walk: at most 16 children per node");
    }
    for (size_t i = 0; i < n; i++) {
        if (has_child[i] && (q_row_of[i] < 0 || (size_t)q_row_of[i] >= q_rows_n))
            throw ArgError("every node with children needs a draft row");
    }
    tree_logits_keep_kv(tokens, parents, n, nullptr, nullptr);
    std::vector<int> par(n), tok(n), qr(n);
    for (size_t i = 0; i < n; i++) {
        par[i] = (int)t.parents[i];
        tok[i] = (int)tokens[i];
        qr[i] = has_child[i] ? q_row_of[i] : -1;
    }
    std::vector<int> p;
    int fin;
    size_t used;
    accept_walk(par.data(), tok.data(), (int)n, q_rows, q_on_device, q_rows_n, q_vocab, qr.data(), uniforms,
                temperature, use_t2d,
                siblings, max_commit, p, fin, used);
    for (size_t i = 0; i < p.size(); i++) path[i] = (uint32_t)p[i];
    *path_len = p.size();
    *token = fin;
    *n_used = used;
}

void Decoder::prime_synthetic(const uint32_t *ids, size_t n, uint64_t kv_seed) {
    Model &m = *model;
    if (n == 0 || n > (size_t)m.cfg.ctx_len) throw ArgError("prefix length out of range");
    for (size_t i = 0; i < n; i++)
        if (ids[i] >= (uint32_t)m.cfg.vocab) throw ArgError("token id out of range");
    m.fill_kv_synthetic((int)n, kv_seed);
    history.assign(ids, ids + n);
    cache_len = (int)n;
    last_valid = false;
}

}  // namespace sd
