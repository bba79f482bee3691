// GGUF reader and model loader.  See sd_gguf.hpp.
//
// File layout (GGUF v1-v3, little endian), as gguf_file::Content::read of
// candle-core 0.8.4 parses it:
//   u32 magic "GGUF", u32 version,
//   tensor count, metadata count        (u32 in v1, u64 from v2),
//   metadata: string key, u32 value type, value
//             (strings and array lengths: u32 length in v1, u64 from v2;
//              arrays: u32 element type, length, elements),
//   tensor directory: string name, u32 n_dims, n_dims sizes (u32 in v1,
//             u64 from v2; the first is the contiguous one), u32 GGML type,
//             u64 offset into the data section,
//   padding to general.alignment (default 32), the data section.
// The parser treats the file as untrusted: every read is bounds-checked and
// a malformed file is an error, never an out-of-range access.
#include "sd_gguf.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cmath>
#include <cstring>
#include <vector>

namespace sd {

namespace {

constexpr uint32_t kMagic = 0x46554747u;  // "GGUF" read as a little-endian u32
constexpr int kMaxNesting = 8;

struct Cursor {
    const uint8_t *p;
    size_t n;
    size_t at = 0;
    void need(uint64_t k) const {
        if (k > n - at) throw BackendError("gguf: unexpected end of file");
    }
    template <typename T> T get() {
        need(sizeof(T));
        T v;
        std::memcpy(&v, p + at, sizeof(T));
        at += sizeof(T);
        return v;
    }
    uint64_t len(uint32_t ver) { return ver == 1 ? get<uint32_t>() : get<uint64_t>(); }
    std::string str(uint32_t ver) {
        const uint64_t k = len(ver);
        need(k);
        std::string s((const char *)p + at, (size_t)k);
        at += (size_t)k;
        return s;
    }
    void skip(uint64_t k) {
        need(k);
        at += (size_t)k;
    }
};

size_t scalar_size(uint32_t t) {
    switch (t) {
    case GV_U8: case GV_I8: case GV_BOOL: return 1;
    case GV_U16: case GV_I16: return 2;
    case GV_U32: case GV_I32: case GV_F32: return 4;
    case GV_U64: case GV_I64: case GV_F64: return 8;
    default: return 0;
    }
}

// cnt elements of a fixed-size type; bools must be 0 or 1
void skip_scalars(Cursor &c, uint32_t t, uint64_t cnt, size_t s) {
    if (cnt > (c.n - c.at) / s) throw BackendError("gguf: unexpected end of file");
    if (t == GV_BOOL)
        for (uint64_t i = 0; i < cnt; i++)
            if (c.p[c.at + i] > 1) throw BackendError("gguf: bool value " + std::to_string(c.p[c.at + i]));
    c.skip(cnt * s);
}

void skip_value(Cursor &c, uint32_t t, uint32_t ver, int depth) {
    if (const size_t s = scalar_size(t)) {
        c.skip(s);
    } else if (t == GV_STRING) {
        c.skip(c.len(ver));
    } else if (t == GV_ARRAY) {
        if (depth >= kMaxNesting) throw BackendError("gguf: arrays nested too deeply");
        const uint32_t et = c.get<uint32_t>();
        const uint64_t cnt = c.len(ver);
        if (const size_t s = scalar_size(et)) {
            skip_scalars(c, et, cnt, s);
        } else {
            // every string or array element takes at least 4 bytes, so the end
            // of the file bounds this loop
            for (uint64_t i = 0; i < cnt; i++) skip_value(c, et, ver, depth + 1);
        }
    } else {
        throw BackendError("gguf: unknown metadata value type " + std::to_string(t));
    }
}

GgufValue read_value(Cursor &c, uint32_t t, uint32_t ver) {
    GgufValue v;
    v.type = t;
    switch (t) {
    case GV_U8: v.u = c.get<uint8_t>(); break;
    case GV_I8: v.i = c.get<int8_t>(); break;
    case GV_U16: v.u = c.get<uint16_t>(); break;
    case GV_I16: v.i = c.get<int16_t>(); break;
    case GV_U32: v.u = c.get<uint32_t>(); break;
    case GV_I32: v.i = c.get<int32_t>(); break;
    case GV_U64: v.u = c.get<uint64_t>(); break;
    case GV_I64: v.i = c.get<int64_t>(); break;
    case GV_F32: v.f = c.get<float>(); break;
    case GV_F64: v.f = c.get<double>(); break;
    case GV_BOOL: {
        const uint8_t b = c.get<uint8_t>();
        if (b > 1) throw BackendError("gguf: bool value " + std::to_string(b));
        v.u = b;
        break;
    }
    case GV_STRING: v.s = c.str(ver); break;
    case GV_ARRAY: {
        v.elem_type = c.get<uint32_t>();
        v.count = c.len(ver);
        const size_t s = scalar_size(v.elem_type);
        if (s) {
            skip_scalars(c, v.elem_type, v.count, s);
        } else if (v.elem_type == GV_STRING || v.elem_type == GV_ARRAY) {
            for (uint64_t i = 0; i < v.count; i++) skip_value(c, v.elem_type, ver, 1);
        } else {
            throw BackendError("gguf: unknown metadata value type " + std::to_string(v.elem_type));
        }
        break;
    }
    default: throw BackendError("gguf: unknown metadata value type " + std::to_string(t));
    }
    return v;
}

// (elements per block, bytes per block) of the GGML types candle-core 0.8.4 knows
bool ggml_block(uint32_t t, uint64_t &elems, uint64_t &bytes) {
    switch (t) {
    case GT_F32: elems = 1; bytes = 4; return true;
    case GT_F16: case GT_BF16: elems = 1; bytes = 2; return true;
    case GT_Q4_0: elems = 32; bytes = 18; return true;
    case GT_Q4_1: elems = 32; bytes = 20; return true;
    case GT_Q5_0: elems = 32; bytes = 22; return true;
    case GT_Q5_1: elems = 32; bytes = 24; return true;
    case GT_Q8_0: elems = 32; bytes = 34; return true;
    case GT_Q8_1: elems = 32; bytes = 36; return true;
    case GT_Q2_K: elems = 256; bytes = 84; return true;
    case GT_Q3_K: elems = 256; bytes = 110; return true;
    case GT_Q4_K: elems = 256; bytes = 144; return true;
    case GT_Q5_K: elems = 256; bytes = 176; return true;
    case GT_Q6_K: elems = 256; bytes = 210; return true;
    case GT_Q8_K: elems = 256; bytes = 292; return true;
    default: return false;
    }
}

float f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 31u, f = h & 1023u;
    uint32_t bits;
    if (e == 0) {
        const float mag = std::ldexp((float)f, -24);  // zero or subnormal, exact
        std::memcpy(&bits, &mag, 4);
        bits |= sign;
    } else if (e == 31) {
        bits = sign | 0x7f800000u | (f << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (f << 13);
    }
    float v;
    std::memcpy(&v, &bits, 4);
    return v;
}

float bf16_to_f32(uint16_t h) {
    const uint32_t bits = (uint32_t)h << 16;
    float v;
    std::memcpy(&v, &bits, 4);
    return v;
}

int to_int(uint32_t v, const std::string &key) {
    if (v > 0x7fffffffu) throw UnsupportedError(key + " = " + std::to_string(v) + " is out of range");
    return (int)v;
}

}  // namespace

GgufFile::GgufFile(const std::string &path) {
    const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) throw BackendError("open gguf: " + path + ": " + std::strerror(errno));
    struct stat sb;
    if (::fstat(fd, &sb) != 0) {
        const int e = errno;
        ::close(fd);
        throw BackendError("open gguf: " + path + ": " + std::strerror(e));
    }
    size_ = (size_t)sb.st_size;
    if (size_ == 0) {
        ::close(fd);
        throw BackendError("gguf: unexpected end of file");
    }
    void *p = ::mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (p == MAP_FAILED) throw BackendError("gguf: mmap failed for " + path);
    base_ = (const uint8_t *)p;
    try {
        Cursor c{base_, size_};
        const uint32_t magic = c.get<uint32_t>();
        if (magic != kMagic) {
            char buf[64];
            std::snprintf(buf, sizeof buf, "gguf: unknown magic 0x%08x", magic);
            throw BackendError(buf);
        }
        version = c.get<uint32_t>();
        if (version < 1 || version > 3) throw BackendError("gguf: unsupported version " + std::to_string(version));
        const uint64_t n_tensors = c.len(version);
        const uint64_t n_kv = c.len(version);
        for (uint64_t i = 0; i < n_kv; i++) {
            std::string key = c.str(version);
            const uint32_t t = c.get<uint32_t>();
            md[std::move(key)] = read_value(c, t, version);
        }
        for (uint64_t i = 0; i < n_tensors; i++) {
            std::string name = c.str(version);
            GgufTensor t;
            t.n_dims = c.get<uint32_t>();
            if (t.n_dims > 4) throw BackendError("gguf: tensor " + name + " has " + std::to_string(t.n_dims) + " dims");
            uint64_t elems = 1;
            for (uint32_t d = 0; d < t.n_dims; d++) {
                t.ne[d] = version == 1 ? c.get<uint32_t>() : c.get<uint64_t>();
                if (t.ne[d] != 0 && elems > (uint64_t(1) << 62) / t.ne[d])
                    throw BackendError("gguf: tensor " + name + " is too large");
                elems *= t.ne[d];
            }
            t.type = c.get<uint32_t>();
            t.offset = c.get<uint64_t>();
            uint64_t be, bb;
            if (!ggml_block(t.type, be, bb))
                throw BackendError("gguf: unknown dtype " + std::to_string(t.type) + " for tensor " + name);
            if (t.ne[0] % be) throw BackendError("gguf: tensor " + name + ": rows are not whole blocks");
            t.bytes = elems / be * bb;
            tensors[std::move(name)] = t;
        }
        alignment = 32;
        if (const GgufValue *a = find("general.alignment")) {
            if (a->type == GV_U8 || a->type == GV_U16 || a->type == GV_U32) alignment = a->u;
            else if ((a->type == GV_I8 || a->type == GV_I16 || a->type == GV_I32) && a->i >= 0) alignment = (uint64_t)a->i;
        }
        if (alignment == 0) throw BackendError("gguf: general.alignment is 0");
        data_start = (c.at + alignment - 1) / alignment * alignment;
    } catch (...) {
        ::munmap((void *)base_, size_);
        base_ = nullptr;
        throw;
    }
}

GgufFile::~GgufFile() {
    if (base_) ::munmap((void *)base_, size_);
}

const GgufValue *GgufFile::find(const std::string &key) const {
    const auto it = md.find(key);
    return it == md.end() ? nullptr : &it->second;
}

uint32_t GgufFile::md_u32(const std::string &key) const {
    const GgufValue *v = find(key);
    if (!v) throw BackendError("cannot find " + key + " in GGUF metadata");
    if (v->type != GV_U32) throw BackendError("not a u32: " + key);
    return (uint32_t)v->u;
}

float GgufFile::md_f32(const std::string &key) const {
    const GgufValue *v = find(key);
    if (!v) throw BackendError("cannot find " + key + " in GGUF metadata");
    if (v->type != GV_F32) throw BackendError("not a f32: " + key);
    return (float)v->f;
}

const GgufTensor &GgufFile::tensor(const std::string &name) const {
    const auto it = tensors.find(name);
    if (it == tensors.end()) throw BackendError("cannot find tensor info for " + name);
    return it->second;
}

// quantized_llama_local.rs:222-240 / quantized_qwen2_local.rs:215-230: the
// same keys in the same order (so the first missing one is the one named);
// the FFN width and the vocabulary come from the tensor shapes the forward
// multiplies with.
ModelCfg GgufFile::config(int arch) const {
    if (arch < 0) {
        const GgufValue *a = find("general.architecture");
        if (!a) throw BackendError("cannot find general.architecture in GGUF metadata");
        if (a->type != GV_STRING) throw BackendError("not a string: general.architecture");
        if (a->s == "llama") arch = 0;
        else if (a->s == "qwen2") arch = 1;
        else throw UnsupportedError("gguf: architecture '" + a->s + "' (llama and qwen2 load)");
    }
    if (arch != 0 && arch != 1) throw ArgError("unknown arch");
    const std::string p = arch == 0 ? "llama." : "qwen2.";
    ModelCfg c;
    c.arch = arch;
    c.n_heads = to_int(md_u32(p + "attention.head_count"), p + "attention.head_count");
    c.n_kv_heads = to_int(md_u32(p + "attention.head_count_kv"), p + "attention.head_count_kv");
    c.hidden = to_int(md_u32(p + "embedding_length"), p + "embedding_length");
    c.ctx_len = to_int(md_u32(p + "context_length"), p + "context_length");
    c.n_layers = to_int(md_u32(p + "block_count"), p + "block_count");
    uint32_t rope_dim = 0;
    if (arch == 0) rope_dim = md_u32("llama.rope.dimension_count");
    c.rms_eps = md_f32(p + "attention.layer_norm_rms_epsilon");
    c.rope_theta = 10000.f;  // .and_then(to_f32).unwrap_or(10000)
    if (const GgufValue *v = find(p + "rope.freq_base"))
        if (v->type == GV_F32) c.rope_theta = (float)v->f;
    if (c.n_heads == 0) throw BackendError(p + "attention.head_count is 0");
    c.head_dim = c.hidden / c.n_heads;
    if (arch == 0 && rope_dim != (uint32_t)c.head_dim)
        throw UnsupportedError("llama.rope.dimension_count " + std::to_string(rope_dim) + " != head_dim " +
                               std::to_string(c.head_dim) + " (partial rotary embedding)");
    const GgufTensor &gate = tensor("blk.0.ffn_gate.weight");
    const GgufTensor &embd = tensor("token_embd.weight");
    if (gate.ne[1] > 0x7fffffffu || embd.ne[1] > 0x7fffffffu) throw UnsupportedError("gguf: tensor too large");
    c.ffn = (int)gate.ne[1];
    c.vocab = (int)embd.ne[1];
    c.tied_output = tensors.count("output.weight") ? 0 : 1;
    c.max_batch = 128;
    c.device = 0;
    return c;
}

void GgufFile::load(Model &m) const {
    const ModelCfg f = config(m.cfg.arch);
    const ModelCfg &c = m.cfg;
    if (f.n_layers != c.n_layers || f.hidden != c.hidden || f.n_heads != c.n_heads || f.n_kv_heads != c.n_kv_heads ||
        f.head_dim != c.head_dim || f.ffn != c.ffn || f.vocab != c.vocab || f.tied_output != c.tied_output ||
        f.rope_theta != c.rope_theta || f.rms_eps != c.rms_eps)
        throw ArgError("the model's config is not the GGUF file's (build it from the file's config)");

    struct Item {
        std::string name;
        int layer, kind;
        const GgufTensor *t;
    };
    std::vector<Item> items;
    auto add = [&](const std::string &name, int layer, int kind) { items.push_back({name, layer, kind, &tensor(name)}); };
    // the order of ModelWeights::from_gguf, so a missing tensor is reported as there
    add("token_embd.weight", -1, K_TOK_EMBD);
    add("output_norm.weight", -1, K_OUTPUT_NORM);
    if (!c.tied_output) add("output.weight", -1, K_OUTPUT);
    for (int i = 0; i < c.n_layers; i++) {
        const std::string b = "blk." + std::to_string(i) + ".";
        add(b + "attn_q.weight", i, K_ATTN_Q);
        add(b + "attn_k.weight", i, K_ATTN_K);
        add(b + "attn_v.weight", i, K_ATTN_V);
        if (c.arch == 1) {
            add(b + "attn_q.bias", i, K_BQ);
            add(b + "attn_k.bias", i, K_BK);
            add(b + "attn_v.bias", i, K_BV);
        }
        add(b + "attn_output.weight", i, K_ATTN_O);
        add(b + "ffn_gate.weight", i, K_FFN_GATE);
        add(b + "ffn_down.weight", i, K_FFN_DOWN);
        add(b + "ffn_up.weight", i, K_FFN_UP);
        add(b + "attn_norm.weight", i, K_ATTN_NORM);
        add(b + "ffn_norm.weight", i, K_FFN_NORM);
    }
    // every check before the first upload
    for (const Item &it : items) {
        const GgufTensor &t = *it.t;
        int rows, K;
        tensor_shape(c, it.kind, rows, K);
        const bool vec = kind_is_f32(it.kind);
        const bool shape_ok = vec ? (t.ne[0] == (uint64_t)K && t.ne[1] == 1 && t.ne[2] == 1 && t.ne[3] == 1)
                                  : (t.ne[0] == (uint64_t)K && t.ne[1] == (uint64_t)rows && t.ne[2] == 1 && t.ne[3] == 1);
        if (!shape_ok)
            throw BackendError(it.name + ": shape [" + std::to_string(t.ne[1]) + ", " + std::to_string(t.ne[0]) +
                               "] in the file, [" + std::to_string(rows) + ", " + std::to_string(K) + "] expected");
        if (vec && t.type != GT_F32 && t.type != GT_F16 && t.type != GT_BF16)
            throw UnsupportedError(it.name + ": GGML type " + std::to_string(t.type) + " (vectors load from F32, F16, BF16)");
        if (!vec && t.type != GT_Q4_K && t.type != GT_Q5_K && t.type != GT_Q6_K && t.type != GT_Q8_0)
            throw UnsupportedError(it.name + ": GGML type " + std::to_string(t.type) +
                                   " (matrices load from Q4_K, Q5_K, Q6_K, Q8_0)");
        if (data_start > size_ || t.offset > size_ - data_start || t.bytes > size_ - data_start - t.offset)
            throw BackendError(it.name + ": tensor data past the end of the file");
    }
    std::vector<float> conv;
    for (const Item &it : items) {
        const GgufTensor &t = *it.t;
        const uint8_t *src = bytes_of(t);
        if (t.type == GT_F16 || t.type == GT_BF16) {
            conv.resize((size_t)t.ne[0]);
            for (size_t j = 0; j < conv.size(); j++) {
                uint16_t h;
                std::memcpy(&h, src + 2 * j, 2);
                conv[j] = t.type == GT_F16 ? f16_to_f32(h) : bf16_to_f32(h);
            }
            m.set_tensor(it.layer, it.kind, F32, conv.data(), conv.size() * 4);
        } else {
            // GGML type ids are the model's format ids
            m.set_tensor(it.layer, it.kind, (int)t.type, src, (size_t)t.bytes);
        }
    }
}

}  // namespace sd
