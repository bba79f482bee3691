// EAGLE-3 draft on the device: buffers, synthetic weights, one draft step and
// one draft round against a target model (kernels in sd_draft.hip).
//
// Restates crates/speculate/src/methods/eagle3.rs: Midlayer::load's RoPE
// tables (:153-182), Midlayer::forward (:196-299), forward_hidden (:433-450),
// apply_norm_lm_head (:451-454) and the draft loop of run_eagle3 (:598-673).
#include "sd_draft.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <numeric>
#include <random>

#include "sd_common.hpp"
#include "sd_kernels_elem.hpp"
#include "sd_model.hpp"

namespace sd {

#define SD_D3_CHECK(x)                                                                            \
    do {                                                                                          \
        const hipError_t e_ = (x);                                                                \
        if (e_ != hipSuccess) throw BackendError(std::string("draft: ") + hipGetErrorString(e_)); \
    } while (0)

static uint16_t f32_to_f16_bits(float v) {
    const _Float16 h = (_Float16)v;
    uint16_t b;
    std::memcpy(&b, &h, 2);
    return b;
}
static float f16_bits_to_f32(uint16_t b) {
    _Float16 h;
    std::memcpy(&h, &b, 2);
    return (float)h;
}

template <typename T> static T *dmalloc(size_t n) {
    void *p = nullptr;
    SD_D3_CHECK(hipMalloc(&p, n * sizeof(T) + 256));
    SD_D3_CHECK(hipMemset(p, 0, n * sizeof(T) + 256));
    // the fill runs on the null stream, which the draft's non-blocking stream
    // does not wait for: without this, the zeros could land after a kernel
    // on that stream has written the buffer
    SD_D3_CHECK(hipDeviceSynchronize());
    return (T *)p;
}

// RoPE tables of Midlayer::load / DraftAttention::load (eagle3.rs:153-182,
// eagle.rs:134-157): inv_freq in f32, t and inv_freq cast to f16, their
// product rounded to f16, cos / sin of it rounded to f16; [max_pos][hd/2]
static void rope_tables(int hd, int max_pos, float theta, uint16_t **cos16, uint16_t **sin16) {
    const int half = hd / 2;
    std::vector<uint16_t> cs((size_t)max_pos * half), sn((size_t)max_pos * half);
    for (int j = 0; j < half; j++) {
        const float inv = 1.0f / std::pow(theta, (float)(2 * j) / (float)hd);
        const float inv16 = f16_bits_to_f32(f32_to_f16_bits(inv));
        for (int t = 0; t < max_pos; t++) {
            const float t16 = f16_bits_to_f32(f32_to_f16_bits((float)t));
            const float fr = f16_bits_to_f32(f32_to_f16_bits(t16 * inv16));
            cs[(size_t)t * half + j] = f32_to_f16_bits(std::cos(fr));
            sn[(size_t)t * half + j] = f32_to_f16_bits(std::sin(fr));
        }
    }
    *cos16 = dmalloc<uint16_t>(cs.size());
    *sin16 = dmalloc<uint16_t>(sn.size());
    SD_D3_CHECK(hipMemcpy(*cos16, cs.data(), cs.size() * 2, hipMemcpyHostToDevice));
    SD_D3_CHECK(hipMemcpy(*sin16, sn.data(), sn.size() * 2, hipMemcpyHostToDevice));
}

// seeded N(0, std)-like f16 values (synth_value: a sum of four uniform 16-bit
// values, standard deviation 65536 / sqrt(3) before the multiplier)
static void synth_f16(uint16_t *dst, size_t n, uint64_t seed, float std_, hipStream_t st) {
    constexpr size_t kChunk = (size_t)1 << 24;
    const float mult = (float)((double)std_ * std::sqrt(3.0) / 65536.0);
    float *tmp = dmalloc<float>(std::min(kChunk, n));
    for (size_t c0 = 0; c0 < n; c0 += kChunk) {
        const size_t k = std::min(kChunk, n - c0);
        launch_synth_f32(tmp, (int64_t)k, seed + c0 / kChunk, mult, st);
        launch_to_f16(tmp, (int64_t)k, dst + c0, st);
    }
    SD_D3_CHECK(hipStreamSynchronize(st));
    SD_D3_CHECK(hipFree(tmp));
}

static size_t numel(const Draft3Cfg &c, int kind) {
    const size_t H = c.hidden, hd = c.head_dim(), nh = c.n_heads, nkv = c.n_kv_heads, F = c.ffn;
    switch (kind) {
    case D3_FC: return H * 3 * H;
    case D3_Q: return nh * hd * 2 * H;
    case D3_K: case D3_V: return nkv * hd * 2 * H;
    case D3_O: return H * nh * hd;
    case D3_GATE: case D3_UP: return F * H;
    case D3_DOWN: return H * F;
    case D3_LM_HEAD: return (size_t)c.draft_vocab * H;
    case D3_IN_NORM: case D3_HID_NORM: case D3_POST_NORM: case D3_NORM: return H;
    case D3_D2T: return (size_t)c.draft_vocab;
    default: throw ArgError("draft tensor kind out of range");
    }
}

Draft3::Draft3(const Draft3Cfg &c) : cfg(c) {
    if (c.hidden < 256 || c.n_heads < 1 || c.n_kv_heads < 1 || c.n_heads % c.n_kv_heads || c.hidden % c.n_heads)
        throw ArgError("draft config: head layout");
    const int hd = c.head_dim();
    if (hd % 2 || hd > 256) throw ArgError("draft config: head_dim must be even and <= 256");
    if (c.hidden % 8 || c.ffn % 8 || c.ffn < 8 || 3 * c.hidden > kDraftMaxK || c.ffn > kDraftMaxK)
        throw ArgError("draft config: widths must be multiples of 8, at most 32768 inputs per product");
    if (c.draft_vocab < kDraftMaxTopk || c.draft_vocab > 65536 || c.target_vocab < 1 || c.max_pos < 1)
        throw ArgError("draft config: sizes (draft_vocab 8 .. 65536)");
    SD_D3_CHECK(hipSetDevice(c.device));
    SD_D3_CHECK(hipStreamCreateWithFlags(&own, hipStreamNonBlocking));
    size_t at = 0;
    for (int k = 0; k < D3_D2T; k++) {
        off[k] = at;
        len[k] = numel(c, k);
        at += len[k];  // Q, K, V and GATE, UP stay adjacent: each size is a multiple of 8 elements
    }
    w = dmalloc<uint16_t>(at);
    len[D3_D2T] = numel(c, D3_D2T);
    d2t = dmalloc<int32_t>(len[D3_D2T]);
    rope_tables(hd, c.max_pos, c.rope_theta, &cos16, &sin16);
    const size_t H = c.hidden, nkv = c.n_kv_heads, nh = c.n_heads;
    kc = dmalloc<uint16_t>((size_t)kDraftMaxSteps * nkv * hd);
    vc = dmalloc<uint16_t>((size_t)kDraftMaxSteps * nkv * hd);
    x3 = dmalloc<uint16_t>(3 * H);
    hid[0] = dmalloc<uint16_t>(H);
    hid[1] = dmalloc<uint16_t>(H);
    proj = dmalloc<uint16_t>(H);
    comb = dmalloc<uint16_t>(2 * H);
    qkv = dmalloc<uint16_t>((nh + 2 * nkv) * hd);
    att = dmalloc<uint16_t>(nh * hd);
    after = dmalloc<uint16_t>(H);
    xn = dmalloc<uint16_t>(H);
    act = dmalloc<uint16_t>(c.ffn);
    xf = dmalloc<uint16_t>(H);
    emb = dmalloc<float>(H);
    hin32 = dmalloc<float>(3 * H);
    logits = dmalloc<float>(c.draft_vocab);
    tok = dmalloc<int32_t>(1);
    tk_part = dmalloc<uint64_t>((size_t)64 * (1 + kDraftMaxTopk));
    tk_cnt = dmalloc<int>(1);
    // the round's outputs, ids | draft ids | log-probs, in one block that a
    // single copy brings back into pinned memory
    o_ids = dmalloc<int32_t>(3 * kDraftOut);
    o_dids = o_ids + kDraftOut;
    o_lp = (float *)(o_ids + 2 * kDraftOut);
    SD_D3_CHECK(hipHostMalloc((void **)&pin, (3 * kDraftOut + 4) * sizeof(int32_t), hipHostMallocDefault));
    SD_D3_CHECK(hipDeviceSynchronize());
}

Draft3::~Draft3() {
    hipSetDevice(cfg.device);
    if (own) hipStreamSynchronize(own);
    for (void *p : {(void *)w, (void *)d2t, (void *)cos16, (void *)sin16, (void *)kc, (void *)vc, (void *)x3,
                    (void *)hid[0], (void *)hid[1], (void *)proj, (void *)comb, (void *)qkv, (void *)att,
                    (void *)after, (void *)xn, (void *)act, (void *)xf, (void *)emb, (void *)hin32, (void *)logits,
                    (void *)tok, (void *)tk_part, (void *)tk_cnt, (void *)o_ids})
        if (p) hipFree(p);
    if (pin) hipHostFree(pin);
    if (own) hipStreamDestroy(own);
}

size_t Draft3::tensor_bytes(int kind) const {
    if (kind < 0 || kind >= D3_NUM) throw ArgError("draft tensor kind out of range");
    return kind == D3_D2T ? len[kind] * 8 : len[kind] * 2;
}

bool Draft3::ready() const {
    for (int k = 0; k < D3_NUM; k++)
        if (!have[k]) return false;
    return true;
}

void Draft3::set_tensor(int kind, const void *host, size_t bytes) {
    if (bytes != tensor_bytes(kind)) throw ArgError("draft tensor: byte size does not match the config");
    if (!host) throw ArgError("draft tensor: null data");
    SD_D3_CHECK(hipSetDevice(cfg.device));
    SD_D3_CHECK(hipStreamSynchronize(own));  // kernels still reading the old tensor
    if (kind == D3_D2T) {
        const int64_t *src = (const int64_t *)host;
        std::vector<int32_t> t(len[kind]);
        for (size_t i = 0; i < t.size(); i++) {
            // draft_to_target_token: `*v as u32` (eagle3.rs:476-485); ids past the
            // target vocabulary are rejected when the round uses them
            t[i] = (int32_t)(uint32_t)src[i];
        }
        d2t_host.assign(src, src + len[kind]);
        SD_D3_CHECK(hipMemcpy(d2t, t.data(), t.size() * 4, hipMemcpyHostToDevice));
    } else {
        SD_D3_CHECK(hipMemcpy(w + off[kind], host, bytes, hipMemcpyHostToDevice));
    }
    have[kind] = true;
}

void Draft3::get_tensor(int kind, void *host, size_t bytes) const {
    if (bytes != tensor_bytes(kind)) throw ArgError("draft tensor: byte size does not match the config");
    if (!have[kind]) throw ArgError("draft tensor not set");
    SD_D3_CHECK(hipSetDevice(cfg.device));
    SD_D3_CHECK(hipStreamSynchronize(own));
    if (kind == D3_D2T) std::memcpy(host, d2t_host.data(), bytes);
    else SD_D3_CHECK(hipMemcpy(host, w + off[kind], bytes, hipMemcpyDeviceToHost));
}

void Draft3::synthesize(uint64_t seed, float std_) {
    SD_D3_CHECK(hipSetDevice(cfg.device));
    for (int k = D3_FC; k <= D3_LM_HEAD; k++) {
        synth_f16(w + off[k], len[k], seed * 1315423911ull + (uint64_t)k * 977ull, std_, own);
        have[k] = true;
    }
    // the draft's stream does not order with the synchronous copies of
    // get_tensor / set_tensor: the tensors are complete when this returns
    SD_D3_CHECK(hipStreamSynchronize(own));
    // norms 1 + N(0, 0.1) and d2t = distinct target ids, from a host generator
    std::mt19937_64 rng(seed ^ 0x9E3779B97F4A7C15ull);
    std::normal_distribution<float> nd(0.f, 0.1f);
    std::vector<uint16_t> nw(cfg.hidden);
    for (int k = D3_IN_NORM; k <= D3_NORM; k++) {
        for (auto &v : nw) v = f32_to_f16_bits(1.0f + nd(rng));
        set_tensor(k, nw.data(), nw.size() * 2);
    }
    std::vector<int64_t> ids(cfg.target_vocab);
    std::iota(ids.begin(), ids.end(), 0);
    for (int i = 0; i < cfg.draft_vocab && i < cfg.target_vocab; i++) {
        std::uniform_int_distribution<int64_t> u(i, cfg.target_vocab - 1);
        std::swap(ids[i], ids[u(rng)]);
    }
    ids.resize(cfg.draft_vocab, 0);
    set_tensor(D3_D2T, ids.data(), ids.size() * 8);
}

// one step from proj (this step's projected input, f16) and emb (f32 input
// embedding); writes the step's midlayer output into hid[cur ^ 1]
void Draft3::step_device(int position, bool first, hipStream_t st, int k, int32_t *ids, int32_t *dids, float *lps) {
    if (steps >= kDraftMaxSteps) throw ArgError("draft round longer than the draft cache");
    if (position < 0 || position >= cfg.max_pos) throw ArgError("draft position past the RoPE tables (max_pos)");
    const Draft3Cfg &c = cfg;
    const int H = c.hidden, hd = c.head_dim(), nh = c.n_heads, nkv = c.n_kv_heads;
    uint16_t *in_h = hid[cur], *out_h = hid[cur ^ 1];
    if (first) {
        // forward_hidden: fc over the [low, mid, high] concat
        DraftGemv g{};
        g.w = w + off[D3_FC];
        g.x = x3;
        g.N = H;
        g.K = 3 * H;
        g.y16 = in_h;
        launch_gemv16(DG_STORE, g, st);
    }
    DraftNorm n{};
    n.x32[0] = emb;
    n.w[0] = w + off[D3_IN_NORM];
    n.out[0] = comb;
    n.x16[1] = in_h;
    n.w[1] = w + off[D3_HID_NORM];
    n.out[1] = comb + H;
    n.H = H;
    n.eps = c.rms_eps;
    launch_rmsnorm16(n, 2, st);
    DraftGemv g{};
    g.w = w + off[D3_Q];  // Q, K, V adjacent: one [(nh + 2 nkv) hd][2H] product
    g.x = comb;
    g.N = (nh + 2 * nkv) * hd;
    g.K = 2 * H;
    g.y16 = qkv;
    launch_gemv16(DG_STORE, g, st);
    DraftAttn a{};
    a.qkv = qkv;
    a.cos16 = cos16;
    a.sin16 = sin16;
    a.kcache = kc;
    a.vcache = vc;
    a.out = att;
    a.n_heads = nh;
    a.n_kv = nkv;
    a.hd = hd;
    a.pos = position;
    a.step = steps;
    a.scale = (float)(1.0 / std::sqrt((double)hd));
    launch_draft_attn(a, st);
    g = DraftGemv{};
    g.w = w + off[D3_O];
    g.x = att;
    g.N = H;
    g.K = nh * hd;
    g.y16 = after;
    g.res16 = in_h;  // attn_out + projected_features
    launch_gemv16(DG_ADD, g, st);
    DraftNorm n1{};
    n1.x16[0] = after;
    n1.w[0] = w + off[D3_POST_NORM];
    n1.out[0] = xn;
    n1.H = H;
    n1.eps = c.rms_eps;
    launch_rmsnorm16(n1, 1, st);
    g = DraftGemv{};
    g.w = w + off[D3_GATE];  // GATE, UP adjacent
    g.x = xn;
    g.N = c.ffn;
    g.K = H;
    g.y16 = act;
    launch_gemv16(DG_SWIGLU, g, st);
    g = DraftGemv{};
    g.w = w + off[D3_DOWN];
    g.x = act;
    g.N = H;
    g.K = c.ffn;
    g.y16 = out_h;
    g.res16 = after;
    launch_gemv16(DG_ADD, g, st);
    DraftNorm n2{};
    n2.x16[0] = out_h;
    n2.w[0] = w + off[D3_NORM];
    n2.out[0] = xf;
    n2.H = H;
    n2.eps = c.rms_eps;
    launch_rmsnorm16(n2, 1, st);
    g = DraftGemv{};
    g.w = w + off[D3_LM_HEAD];
    g.x = xf;
    g.N = c.draft_vocab;
    g.K = H;
    g.y32 = logits;
    launch_gemv16(DG_LOGITS, g, st);
    if (k > 0) {
        DraftTopk t{};
        t.logits = logits;
        t.V = c.draft_vocab;
        t.k = k;
        t.d2t = d2t;
        t.out_draft = dids;
        t.out_target = ids;
        t.out_lp = lps;
        t.next_token = tok;
        t.part = tk_part;
        t.cnt = tk_cnt;
        launch_draft_topk(t, st);
    }
    steps++;
    cur ^= 1;
}

void Draft3::step_host(const float *hidden_in, size_t n_in, const float *input_emb, int position, float *out_hidden,
                       float *out_logits) {
    if (!ready()) throw ArgError("draft weights are not fully set");
    const size_t H = cfg.hidden;
    if (n_in != H && n_in != 3 * H) throw ArgError("draft hidden input must be hidden or 3 * hidden wide");
    if (steps >= kDraftMaxSteps) throw ArgError("draft round longer than the draft cache");
    if (position < 0 || position >= cfg.max_pos) throw ArgError("draft position past the RoPE tables (max_pos)");
    SD_D3_CHECK(hipSetDevice(cfg.device));
    SD_D3_CHECK(hipMemcpyAsync(hin32, hidden_in, n_in * 4, hipMemcpyHostToDevice, own));
    SD_D3_CHECK(hipMemcpyAsync(emb, input_emb, H * 4, hipMemcpyHostToDevice, own));
    const bool first = n_in == 3 * H;
    launch_to_f16(hin32, (int64_t)n_in, first ? x3 : hid[cur], own);
    step_device(position, first, own, 0, nullptr, nullptr, nullptr);
    std::vector<uint16_t> h16(H);
    SD_D3_CHECK(hipMemcpyAsync(h16.data(), hid[cur], H * 2, hipMemcpyDeviceToHost, own));
    if (out_logits)
        SD_D3_CHECK(hipMemcpyAsync(out_logits, logits, (size_t)cfg.draft_vocab * 4, hipMemcpyDeviceToHost, own));
    SD_D3_CHECK(hipStreamSynchronize(own));
    if (out_hidden)
        for (size_t i = 0; i < H; i++) out_hidden[i] = f16_bits_to_f32(h16[i]);
}

void Draft3::round(Model &target, Decoder &dec, const uint32_t layers[3], int depth, const int *top_k, int32_t *ids,
                   int32_t *draft_ids, float *log_probs) {
    if (!ready()) throw ArgError("draft weights are not fully set");
    if (depth < 1 || depth > kDraftMaxSteps) throw ArgError("draft depth out of range");
    for (int s = 0; s < depth; s++)
        if (top_k[s] < 1 || top_k[s] > kDraftMaxTopk) throw ArgError("draft top_k out of range");
    if (target.cfg.device != cfg.device) throw ArgError("draft and target on different devices");
    if (target.cfg.hidden != cfg.hidden) throw ArgError("draft and target hidden sizes differ");
    if (target.cfg.vocab != cfg.target_vocab) throw ArgError("draft target vocabulary differs from the target's");
    for (size_t i = 0; i < d2t_host.size(); i++)
        if (d2t_host[i] < 0 || d2t_host[i] >= cfg.target_vocab)
            throw ArgError("d2t maps a draft id outside the target vocabulary");
    const size_t hl = dec.history.size();
    if (hl == 0) throw SamplingError("EAGLE-3 requires non-empty prompt");
    if ((int64_t)hl + depth - 1 >= cfg.max_pos) throw ArgError("draft positions past the RoPE tables (max_pos)");
    SD_D3_CHECK(hipSetDevice(cfg.device));
    hipStream_t st = target.st;
    // 1. the committed token's hidden states after the three layers, left on
    //    the device (TreeDecoder::last_hidden_states_multi), as f16 [low, mid, high]
    const float *h3 = dec.collect_hidden_device(layers, 3);
    launch_to_f16(h3, 3 * (int64_t)cfg.hidden, x3, st);
    pin[3 * kDraftOut] = (int32_t)dec.history.back();
    SD_D3_CHECK(hipMemcpyAsync(tok, pin + 3 * kDraftOut, 4, hipMemcpyHostToDevice, st));
    // 2. depth steps: the embedding of the current token, the midlayer, norm +
    //    lm_head, top-k; the top-1 target id is the next step's token
    reset();
    for (int s = 0; s < depth; s++) {
        launch_embed(target.gw[K_TOK_EMBD].fmt, target.embed_table(), cfg.hidden, tok, 1, emb, st);
        step_device((int)hl + s, s == 0, st, top_k[s], o_ids + s * kDraftMaxTopk, o_dids + s * kDraftMaxTopk,
                    o_lp + s * kDraftMaxTopk);
    }
    const size_t n = (size_t)depth * kDraftMaxTopk;
    SD_D3_CHECK(hipMemcpyAsync(pin, o_ids, 3 * kDraftOut * 4, hipMemcpyDeviceToHost, st));
    SD_D3_CHECK(hipStreamSynchronize(st));
    std::memcpy(ids, pin, n * 4);
    std::memcpy(draft_ids, pin + kDraftOut, n * 4);
    std::memcpy(log_probs, pin + 2 * kDraftOut, n * 4);
}

// ===== EAGLE-2 (EagleDraftCandle, crates/speculate/src/methods/eagle.rs) =====

static size_t numel2(const Draft2Cfg &c, int kind) {
    const size_t H = c.hidden, hd = c.head_dim(), nh = c.n_heads, nkv = c.n_kv_heads, F = c.ffn;
    switch (kind) {
    case D2_EMBED: return (size_t)c.vocab * H;
    case D2_FC: return H * 2 * H;
    case D2_Q: return nh * hd * H;
    case D2_K: case D2_V: return nkv * hd * H;
    case D2_O: return H * nh * hd;
    case D2_GATE: case D2_UP: return F * H;
    case D2_DOWN: return H * F;
    case D2_POST_NORM: return H;
    default: throw ArgError("draft tensor kind out of range");
    }
}

Draft2::Draft2(const Draft2Cfg &c) : cfg(c) {
    if (c.hidden < 256 || c.n_heads < 1 || c.n_kv_heads < 1 || c.n_heads % c.n_kv_heads || c.hidden % c.n_heads)
        throw ArgError("draft config: head layout");
    const int hd = c.head_dim();
    if (hd % 2 || hd > 256) throw ArgError("draft config: head_dim must be even and <= 256");
    if (c.hidden % 8 || c.ffn % 8 || c.ffn < 8 || 2 * c.hidden > kDraftMaxK || c.ffn > kDraftMaxK)
        throw ArgError("draft config: widths must be multiples of 8, at most 32768 inputs per product");
    if (c.vocab < kDraftMaxTopk || c.vocab > 262144 || c.max_pos < 1)
        throw ArgError("draft config: sizes (vocab 8 .. 262144)");
    SD_D3_CHECK(hipSetDevice(c.device));
    SD_D3_CHECK(hipStreamCreateWithFlags(&own, hipStreamNonBlocking));
    size_t at = 0;
    for (int k = 0; k < D2_NUM; k++) {
        off[k] = at;
        len[k] = numel2(c, k);
        at += len[k];  // Q, K, V and GATE, UP stay adjacent: each size is a multiple of 8 elements
    }
    w = dmalloc<uint16_t>(at);
    rope_tables(hd, c.max_pos, c.rope_theta, &cos16, &sin16);
    const size_t H = c.hidden, nkv = c.n_kv_heads, nh = c.n_heads;
    kc = dmalloc<uint16_t>((size_t)kDraftMaxSteps * nkv * hd);
    vc = dmalloc<uint16_t>((size_t)kDraftMaxSteps * nkv * hd);
    comb = dmalloc<uint16_t>(2 * H);
    xs = dmalloc<uint16_t>(H);
    qkv = dmalloc<uint16_t>((nh + 2 * nkv) * hd);
    att = dmalloc<uint16_t>(nh * hd);
    after = dmalloc<uint16_t>(H);
    xn = dmalloc<uint16_t>(H);
    act = dmalloc<uint16_t>(c.ffn);
    xp = dmalloc<uint16_t>(16 * H);
    hin32 = dmalloc<float>(H);
    out32 = dmalloc<float>(H);
    logits = dmalloc<float>(c.vocab);
    tok = dmalloc<int32_t>(1);
    // the round's outputs, ids | draft ids | log-probs, in one block that a
    // single copy brings back into pinned memory
    o_ids = dmalloc<int32_t>(3 * kDraftOut);
    o_dids = o_ids + kDraftOut;
    o_lp = (float *)(o_ids + 2 * kDraftOut);
    SD_D3_CHECK(hipHostMalloc((void **)&pin, (3 * kDraftOut + 4) * sizeof(int32_t), hipHostMallocDefault));
    tk_part = dmalloc<uint64_t>((size_t)256 * (1 + kDraftMaxTopk));
    tk_cnt = dmalloc<int>(1);
    SD_D3_CHECK(hipDeviceSynchronize());
}

Draft2::~Draft2() {
    hipSetDevice(cfg.device);
    if (own) hipStreamSynchronize(own);
    for (void *p : {(void *)w, (void *)cos16, (void *)sin16, (void *)kc, (void *)vc, (void *)comb, (void *)xs,
                    (void *)qkv, (void *)att, (void *)after, (void *)xn, (void *)act, (void *)xp, (void *)hin32,
                    (void *)out32, (void *)logits, (void *)tok, (void *)o_ids, (void *)tk_part, (void *)tk_cnt})
        if (p) hipFree(p);
    if (pin) hipHostFree(pin);
    if (own) hipStreamDestroy(own);
}

size_t Draft2::tensor_bytes(int kind) const {
    if (kind < 0 || kind >= D2_NUM) throw ArgError("draft tensor kind out of range");
    return len[kind] * 2;
}

bool Draft2::ready() const {
    for (int k = 0; k < D2_NUM; k++)
        if (!have[k]) return false;
    return true;
}

void Draft2::set_tensor(int kind, const void *host, size_t bytes) {
    if (bytes != tensor_bytes(kind)) throw ArgError("draft tensor: byte size does not match the config");
    if (!host) throw ArgError("draft tensor: null data");
    SD_D3_CHECK(hipSetDevice(cfg.device));
    SD_D3_CHECK(hipStreamSynchronize(own));  // kernels still reading the old tensor
    SD_D3_CHECK(hipMemcpy(w + off[kind], host, bytes, hipMemcpyHostToDevice));
    have[kind] = true;
}

void Draft2::get_tensor(int kind, void *host, size_t bytes) const {
    if (bytes != tensor_bytes(kind)) throw ArgError("draft tensor: byte size does not match the config");
    if (!have[kind]) throw ArgError("draft tensor not set");
    SD_D3_CHECK(hipSetDevice(cfg.device));
    SD_D3_CHECK(hipStreamSynchronize(own));
    SD_D3_CHECK(hipMemcpy(host, w + off[kind], bytes, hipMemcpyDeviceToHost));
}

void Draft2::synthesize(uint64_t seed, float std_) {
    SD_D3_CHECK(hipSetDevice(cfg.device));
    for (int k = D2_EMBED; k <= D2_DOWN; k++) {
        synth_f16(w + off[k], len[k], seed * 2654435761ull + (uint64_t)k * 7919ull, std_, own);
        have[k] = true;
    }
    // the draft's stream does not order with the synchronous copies of
    // get_tensor / set_tensor: the tensors are complete when this returns
    SD_D3_CHECK(hipStreamSynchronize(own));
    std::mt19937_64 rng(seed ^ 0xC2B2AE3D27D4EB4Full);
    std::normal_distribution<float> nd(0.f, 0.1f);
    std::vector<uint16_t> nw(cfg.hidden);
    for (auto &v : nw) v = f32_to_f16_bits(1.0f + nd(rng));
    set_tensor(D2_POST_NORM, nw.data(), nw.size() * 2);
}

// one step: comb = [input hidden | embedding of *tok] (both f16) in place;
// writes the step's output to comb[0, H) and out32
void Draft2::step_device(int position, hipStream_t st) {
    if (steps >= kDraftMaxSteps) throw ArgError("draft round longer than the draft cache");
    if (position < 0 || position >= cfg.max_pos) throw ArgError("draft position past the RoPE tables (max_pos)");
    const Draft2Cfg &c = cfg;
    const int H = c.hidden, hd = c.head_dim(), nh = c.n_heads, nkv = c.n_kv_heads;
    launch_gather16(w + off[D2_EMBED], c.vocab, H, tok, comb + H, st);
    DraftGemv g{};
    g.w = w + off[D2_FC];  // fc over cat(target_hidden, token_emb)
    g.x = comb;
    g.N = H;
    g.K = 2 * H;
    g.y16 = xs;
    launch_gemv16(DG_STORE, g, st);
    g = DraftGemv{};
    g.w = w + off[D2_Q];  // no input norm (eagle.rs:413-418)
    g.x = xs;
    g.N = (nh + 2 * nkv) * hd;
    g.K = H;
    g.y16 = qkv;
    launch_gemv16(DG_STORE, g, st);
    DraftAttn a{};
    a.qkv = qkv;
    a.cos16 = cos16;
    a.sin16 = sin16;
    a.kcache = kc;
    a.vcache = vc;
    a.out = att;
    a.n_heads = nh;
    a.n_kv = nkv;
    a.hd = hd;
    a.pos = position;
    a.step = steps;
    a.scale = (float)(1.0 / std::sqrt((double)hd));
    launch_draft_attn(a, st);
    g = DraftGemv{};
    g.w = w + off[D2_O];
    g.x = att;
    g.N = H;
    g.K = nh * hd;
    g.y16 = after;
    g.res16 = xs;  // attn + res
    launch_gemv16(DG_ADD, g, st);
    DraftNorm n{};
    n.x16[0] = after;
    n.w[0] = w + off[D2_POST_NORM];
    n.out[0] = xn;
    n.H = H;
    n.eps = c.rms_eps;
    launch_rmsnorm16(n, 1, st);
    g = DraftGemv{};
    g.w = w + off[D2_GATE];  // GATE, UP adjacent
    g.x = xn;
    g.N = c.ffn;
    g.K = H;
    g.y16 = act;
    launch_gemv16(DG_SWIGLU, g, st);
    g = DraftGemv{};
    g.w = w + off[D2_DOWN];
    g.x = act;
    g.N = H;
    g.K = c.ffn;
    g.y16 = comb;  // m + res: the next step's input hidden
    g.res16 = after;
    g.y32 = out32;
    launch_gemv16(DG_ADD, g, st);
    steps++;
}

void Draft2::step_host(const float *target_hidden, uint32_t token, int position, float *out) {
    if (!ready()) throw ArgError("draft weights are not fully set");
    if (token >= (uint32_t)cfg.vocab) throw ArgError("token id out of range");
    if (steps >= kDraftMaxSteps) throw ArgError("draft round longer than the draft cache");
    if (position < 0 || position >= cfg.max_pos) throw ArgError("draft position past the RoPE tables (max_pos)");
    SD_D3_CHECK(hipSetDevice(cfg.device));
    const int32_t t = (int32_t)token;
    SD_D3_CHECK(hipMemcpyAsync(hin32, target_hidden, (size_t)cfg.hidden * 4, hipMemcpyHostToDevice, own));
    SD_D3_CHECK(hipMemcpyAsync(tok, &t, 4, hipMemcpyHostToDevice, own));
    launch_to_f16(hin32, cfg.hidden, comb, own);
    step_device(position, own);
    if (out) SD_D3_CHECK(hipMemcpyAsync(out, out32, (size_t)cfg.hidden * 4, hipMemcpyDeviceToHost, own));
    SD_D3_CHECK(hipStreamSynchronize(own));
}

void Draft2::round(Model &target, Decoder &dec, const float *target_hidden, int depth, const int *top_k, int32_t *ids,
                   float *log_probs) {
    if (!ready()) throw ArgError("draft weights are not fully set");
    if (depth < 1 || depth > kDraftMaxSteps) throw ArgError("draft depth out of range");
    for (int s = 0; s < depth; s++)
        if (top_k[s] < 1 || top_k[s] > kDraftMaxTopk) throw ArgError("draft top_k out of range");
    if (target.cfg.device != cfg.device) throw ArgError("draft and target on different devices");
    if (target.cfg.hidden != cfg.hidden) throw ArgError("draft and target hidden sizes differ");
    if (target.cfg.vocab != cfg.vocab) throw ArgError("draft vocabulary differs from the target's");
    const size_t hl = dec.history.size();
    if (hl == 0) throw SamplingError("EAGLE requires non-empty prompt");
    if ((int64_t)hl + depth - 1 >= cfg.max_pos) throw ArgError("draft positions past the RoPE tables (max_pos)");
    SD_D3_CHECK(hipSetDevice(cfg.device));
    hipStream_t st = target.st;
    const int H = cfg.hidden;
    pin[3 * kDraftOut] = (int32_t)dec.history.back();
    SD_D3_CHECK(hipMemcpyAsync(hin32, target_hidden, (size_t)H * 4, hipMemcpyHostToDevice, st));
    SD_D3_CHECK(hipMemcpyAsync(tok, pin + 3 * kDraftOut, 4, hipMemcpyHostToDevice, st));
    launch_to_f16(hin32, H, comb, st);
    reset();
    for (int s = 0; s < depth; s++) {
        step_device((int)hl + s, st);
        // apply_lm_head: the target's lm_head on the f16 output (exact in the
        // matmul's fp16 input)
        launch_to_frag16(out32, 1, H, xp, H, st);
        target.lm_head_device(xp, 1, logits, st);
        DraftTopk t{};
        t.logits = logits;
        t.V = cfg.vocab;
        t.k = top_k[s];
        t.d2t = nullptr;
        t.out_draft = o_dids + s * kDraftMaxTopk;
        t.out_target = o_ids + s * kDraftMaxTopk;
        t.out_lp = o_lp + s * kDraftMaxTopk;
        t.next_token = tok;
        t.part = tk_part;
        t.cnt = tk_cnt;
        launch_draft_topk(t, st);
    }
    const size_t n = (size_t)depth * kDraftMaxTopk;
    SD_D3_CHECK(hipMemcpyAsync(pin, o_ids, 3 * kDraftOut * 4, hipMemcpyDeviceToHost, st));
    SD_D3_CHECK(hipStreamSynchronize(st));
    std::memcpy(ids, pin, n * 4);
    std::memcpy(log_probs, pin + 2 * kDraftOut, n * 4);
}

}  // namespace sd
