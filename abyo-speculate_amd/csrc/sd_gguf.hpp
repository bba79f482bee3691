// GGUF files: the header, metadata and tensor directory (what
// candle-core 0.8.4's gguf_file::Content::read keeps), the hyper-parameters
// ModelWeights::from_gguf reads from the metadata, and the upload of every
// tensor it loads.  References: crates/speculate/src/model/
// quantized_llama_local.rs:217-308 and quantized_qwen2_local.rs:210-305
// (which keys, which tensor names, the tied-output fallback), and the GGUF
// v1-v3 layout that Content::read parses.
#pragma once
#include <stdint.h>

#include <string>
#include <unordered_map>

#include "sd_model.hpp"

namespace sd {

// GGUF metadata value types
enum GgufType : uint32_t {
    GV_U8 = 0, GV_I8 = 1, GV_U16 = 2, GV_I16 = 3, GV_U32 = 4, GV_I32 = 5, GV_F32 = 6, GV_BOOL = 7,
    GV_STRING = 8, GV_ARRAY = 9, GV_U64 = 10, GV_I64 = 11, GV_F64 = 12
};

// GGML tensor types that may appear in a directory (the set candle-core 0.8.4
// knows); only F32/F16/BF16 vectors and Q4_K/Q5_K/Q6_K/Q8_0 matrices load.
enum GgmlType : uint32_t {
    GT_F32 = 0, GT_F16 = 1, GT_Q4_0 = 2, GT_Q4_1 = 3, GT_Q5_0 = 6, GT_Q5_1 = 7, GT_Q8_0 = 8, GT_Q8_1 = 9,
    GT_Q2_K = 10, GT_Q3_K = 11, GT_Q4_K = 12, GT_Q5_K = 13, GT_Q6_K = 14, GT_Q8_K = 15, GT_BF16 = 30
};

struct GgufValue {
    uint32_t type = 0;
    uint64_t u = 0;          // unsigned integers, bool
    int64_t i = 0;           // signed integers
    double f = 0.0;          // F32 / F64
    std::string s;           // STRING
    uint32_t elem_type = 0;  // ARRAY: element type and count (elements are
    uint64_t count = 0;      //   skipped; no loaded tensor depends on them)
};

struct GgufTensor {
    uint32_t type = 0;
    uint32_t n_dims = 0;
    uint64_t ne[4] = {1, 1, 1, 1};  // GGUF order: ne[0] is the contiguous dimension
    uint64_t offset = 0;            // from the start of the data section
    uint64_t bytes = 0;
};

class GgufFile {
  public:
    explicit GgufFile(const std::string &path);
    ~GgufFile();
    GgufFile(const GgufFile &) = delete;
    GgufFile &operator=(const GgufFile &) = delete;

    uint32_t version = 0;
    uint64_t alignment = 32;
    uint64_t data_start = 0;  // absolute file offset of the data section
    std::unordered_map<std::string, GgufValue> md;
    std::unordered_map<std::string, GgufTensor> tensors;

    const GgufValue *find(const std::string &key) const;
    uint32_t md_u32(const std::string &key) const;  // md_get(key)?.to_u32()?
    float md_f32(const std::string &key) const;     // md_get(key)?.to_f32()?
    const GgufTensor &tensor(const std::string &name) const;
    const uint8_t *bytes_of(const GgufTensor &t) const { return base_ + data_start + t.offset; }

    // arch: 0 llama, 1 qwen2 (the key prefix of the decoder type being
    // built), -1 from general.architecture.  ctx_len = context_length,
    // max_batch = 128, device = 0.
    ModelCfg config(int arch) const;
    // Checks every tensor the model needs (presence, type, shape) and only
    // then uploads them; the model's config must be this file's.
    void load(Model &m) const;

  private:
    const uint8_t *base_ = nullptr;
    size_t size_ = 0;
};

}  // namespace sd
