// Host-side launchers of the HIP kernels (one translation unit per kernel family).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdexcept>
#include <string>

namespace sd {

struct BackendError : std::runtime_error {
    explicit BackendError(const std::string &m) : std::runtime_error(m) {}
};

// ---- sd_noalloc.hip: scratch of the allocation-free entry points ----
// Device address of this GPU's file-scope scratch array (kNoAllocScratchBytes),
// resolved with hipGetSymbolAddress on the first call for `device`, which must
// be the current device; later calls return the kept address.
constexpr size_t kNoAllocScratchBytes = (size_t)4 << 20;
void *noalloc_scratch(int device);

// ---- sd_synth.hip ----
void launch_synth_quant(int fmt, uint8_t *out, int64_t rows, int64_t K, uint64_t seed, float mult, hipStream_t st);
void launch_synth_f32(float *out, int64_t n, uint64_t seed, float mult, hipStream_t st);
void launch_fill_f32(float *out, int64_t n, float v, hipStream_t st);
void launch_fill_kv(uint16_t *kv, int L, int n_kv, int64_t cap, int hd, int P, uint64_t seed, float mult,
                    hipStream_t st);
// GGUF block bytes -> f32, exact (input must be in GGUF layout)
void launch_dequant(int fmt, const uint8_t *w, int64_t n_elems, float *y, hipStream_t st);

// ---- sd_layout.hip: GGUF rows <-> tile-interleaved device layout ----
void launch_gguf_to_dev(int fmt, const uint8_t *src, uint8_t *dst, int64_t rows, int64_t K, hipStream_t st);
void launch_dev_to_gguf(int fmt, const uint8_t *src, uint8_t *dst, int64_t rows, int64_t K, hipStream_t st);

// ---- sd_qgemm.hip: fused dequant-matmul on MFMA ----
enum GemmMode : int { GM_STORE = 0, GM_RESID = 1, GM_SWIGLU = 2, GM_LOGITS = 3 };

struct GemmSeg {
    const uint8_t *w;  // tile-interleaved device layout (sd_layout.hip)
    int fmt;
    int rows;          // multiple of 16
    int tile0;         // first 16-row tile of this segment in the launch
    float *out;        // GM_STORE/GM_RESID/GM_LOGITS: out[m*ldo + col0 + n]
    int ldo;
    int col0;
    const float *bias; // optional per-row bias (GM_STORE)
};

// RoPE and KV append in the epilogue of the fused Q/K/V launch (M <= 16):
// the launch's columns are q (n_heads heads) | k (n_kv) | v (n_kv), hd each.
// Rotated q goes to q16[head][M][hd] (fp16), rotated k and v to the layer's
// cache streams at position P + m (blocked layout, kv_k_off / kv_v_off).
struct RopeOut {
    const int *pos;              // [M] absolute positions
    const float *cos_t, *sin_t;  // [ctx][hd/2]
    uint16_t *q16;
    uint16_t *kc, *vc;
    int64_t cap;
    int P, n_heads, n_kv, hd;
    int interleaved;             // 1: pairs (2i, 2i+1); 0: pairs (i, i + hd/2)
};

struct GemmParams {
    GemmSeg seg[4];
    int nseg;
    int ntiles;              // total 16-row tiles (sum over segments)
    const uint16_t *xp;      // fp16 activations, fragment layout, [Mpad][K]
    int K;
    int M;
    int mode;
    uint16_t *act;           // GM_SWIGLU: fp16 fragment-layout output [Mpad][act_ld]
    int act_ld;
    float *amax_v;           // GM_LOGITS: per (token, workgroup) argmax partials
    int *amax_i;
    int amax_ld;             // = number of workgroups
    // M > 16 only: with allow_split (GM_STORE / GM_RESID) the launch may split
    // K into qgemm_slices(p) slices and then writes partial sums
    // part[ks][M][ntiles * 16] instead of the output; the caller adds them.
    int allow_split;
    float *part;
    int64_t part_cap;        // floats
    // ---- M <= 16 fused RMSNorm (RmsNorm::forward applied around the matmul) ----
    // Input side (norm_ssq set): the activations are u = fp16(h * w_norm) and
    // every output of token m is scaled by 1 / sqrt(S_m / K + norm_eps), with
    // S_m = sum over t < norm_parts of norm_ssq[m * norm_parts + t] (sum of h^2).
    const float *norm_ssq;
    int norm_parts;
    float norm_eps;
    // Output side (GM_RESID, next_w set): with the new residual row h also
    // next_u[m][frag(n)] = fp16(h[n] * next_w[n]) and, for each 16-row tile,
    // next_ssq[m * ntiles + tile] = sum of h^2 over the tile: the input of the
    // next normalised matmul.
    const float *next_w;
    uint16_t *next_u;
    int next_ld;
    float *next_ssq;
    // GM_STORE with rope.q16 set: RoPE + KV append instead of storing the output
    RopeOut rope;
};

// Optional timing of one launch: with both events set the kernel goes through
// hipExtLaunchKernel, which stamps the events with the dispatch's own start and
// end (the kernel's duration, without the queue gaps around it).
struct LaunchTiming {
    hipEvent_t start = nullptr, stop = nullptr;
};

// Launches y = x . W^T over all segments.  Chooses the tile shape from M.
// Returns the number of workgroups launched (GM_LOGITS partial count).
int launch_qgemm(const GemmParams &p, hipStream_t st, const LaunchTiming &tm = LaunchTiming{});
int qgemm_workgroups(const GemmParams &p);
int qgemm_slices(const GemmParams &p);  // 1 when the output is written directly

}  // namespace sd
