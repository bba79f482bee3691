// EAGLE-3 draft side on the device: the kernels of one draft step.
//
// Restates crates/speculate/src/methods/eagle3.rs: Midlayer::forward
// (:196-299), forward_hidden (:433-450), apply_norm_lm_head (:451-454) and the
// per-step top-k / log-probs / d2t of run_eagle3 (:634-673).  The draft's
// tensors are f16 as the reference runs them: every op reads f16 values,
// computes in f32 and rounds its result to f16 at the points candle does
// (after each matmul, norm, add, activation; RoPE in f16 arithmetic, every
// multiply and add rounded).
//
// Weights are row-major [out][in] f16 (the checkpoint's Linear layout); the
// matrix-vector products stream them once from HBM: a lane reads 16 bytes (8
// weights) of a row per load and a wave covers 512 inputs of 8 rows per step.
#include <math.h>

#include "sd_buffer.hpp"
#include "sd_common.hpp"
#include "sd_draft.hpp"

namespace sd {

#pragma clang fp contract(off)

__device__ __forceinline__ float r16(float v) { return (float)(_Float16)v; }

typedef _Float16 half2v_t __attribute__((ext_vector_type(2)));

// ---- y = W x: f16 weights [N][K], f16 x [K] ------------------------------------
// A workgroup owns 8 rows (SwiGLU: 4 features as gate / up row pairs); its 4
// waves split K into 512-input chunks (wave w takes chunks w, w + 4, ...),
// two chunks in flight per wave: 16 loads of 16 bytes per lane, and the x
// slices of the same chunks read through the cache.  Per-wave sums meet in
// LDS and are added in a fixed order.
constexpr int kGvWaves = 4, kGvRows = 8, kGvChunk = 512;
template <int MODE>
__global__ __launch_bounds__(64 * kGvWaves) void k_gemv16(DraftGemv p) {
    warm_kernargs<sizeof(DraftGemv)>();
    __shared__ float red[kGvWaves][kGvRows];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int row[kGvRows];
    const int base = blockIdx.x * kGvRows;
#pragma unroll
    for (int r = 0; r < kGvRows; r++) {
        if (MODE == DG_SWIGLU) row[r] = (base / 2 + r / 2) + (r & 1) * p.N;  // N = features
        else row[r] = base + r;
    }
    const int nrows = MODE == DG_SWIGLU ? 2 * p.N : p.N;
    const rsrc_t wr = make_rsrc(p.w, (uint32_t)((int64_t)nrows * p.K * 2));
    const rsrc_t xr = make_rsrc(p.x, (uint32_t)p.K * 2);
    float acc[kGvRows];
#pragma unroll
    for (int r = 0; r < kGvRows; r++) acc[r] = 0.f;
    const int nchunk = (p.K + kGvChunk - 1) / kGvChunk;
    for (int c0 = wave; c0 < nchunk; c0 += 2 * kGvWaves) {
        uintx4 wv[2][kGvRows], xv[2];
#pragma unroll
        for (int s = 0; s < 2; s++) {
            const int k = (c0 + s * kGvWaves) * kGvChunk + lane * 8;
            const bool kin = k < p.K;
            xv[s] = bld16(xr, kin ? (uint32_t)k * 2 : 0x80000000u, 0);
#pragma unroll
            for (int r = 0; r < kGvRows; r++) {
                const bool ok = kin && row[r] < nrows;
                wv[s][r] = bld16(wr, ok ? (uint32_t)(((int64_t)row[r] * p.K + k) * 2) : 0x80000000u, 0);
            }
        }
        // out-of-range loads read zeros, which add nothing
#pragma unroll
        for (int s = 0; s < 2; s++)
#pragma unroll
            for (int r = 0; r < kGvRows; r++)
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    // element to a scalar first: a bit_cast of a vector element
                    // expression reads element 0 whatever the index
                    const uint32_t wj = wv[s][r][j], xj = xv[s][j];
                    acc[r] = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2v_t, wj), __builtin_bit_cast(half2v_t, xj),
                                                    acc[r], false);
                }
    }
#pragma unroll
    for (int r = 0; r < kGvRows; r++) {
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) acc[r] += __shfl_xor(acc[r], o);
    }
    if (lane == 0)
#pragma unroll
        for (int r = 0; r < kGvRows; r++) red[wave][r] = acc[r];
    __syncthreads();
    if (threadIdx.x >= kGvRows) return;
    const int r = threadIdx.x;
    const float v = r16((red[0][r] + red[1][r]) + (red[2][r] + red[3][r]));
    if constexpr (MODE == DG_SWIGLU) {
        // thread 2f: gate and up of feature base/2 + f (up in the odd slot)
        if (r & 1) return;
        const int feat = base / 2 + r / 2;
        if (feat >= p.N) return;
        const float u = r16((red[0][r + 1] + red[1][r + 1]) + (red[2][r + 1] + red[3][r + 1]));
        const float sg = r16(v / (1.0f + expf(-v)));
        p.y16[feat] = f2h(sg * u);
        return;
    }
    const int n = base + r;
    if (n >= p.N) return;
    if constexpr (MODE == DG_STORE) {
        p.y16[n] = f2h(v);
    } else if constexpr (MODE == DG_ADD) {
        const uint16_t y = f2h(v + h2f(p.res16[n]));
        p.y16[n] = y;
        if (p.y32) p.y32[n] = h2f(y);  // the same f16 value widened, when asked for
    } else {
        p.y32[n] = v;  // DG_LOGITS: the f16 logit widened
    }
}

void launch_gemv16(int mode, const DraftGemv &p, hipStream_t st) {
    if (p.K % 8 || p.K < 8 || p.K > kDraftMaxK) throw BackendError("draft gemv: K must be a multiple of 8");
    const int rows = mode == DG_SWIGLU ? 2 * p.N : p.N;
    // weight offsets stay below 2^31 bytes, so the out-of-range sentinel 2^31
    // lies past the buffer resource's size
    if ((int64_t)rows * p.K * 2 >= ((int64_t)1 << 31)) throw BackendError("draft gemv: weight matrix over 2 GiB");
    const dim3 grid((rows + kGvRows - 1) / kGvRows), block(64 * kGvWaves);
    switch (mode) {
    case DG_STORE: hipLaunchKernelGGL(k_gemv16<DG_STORE>, grid, block, 0, st, p); break;
    case DG_ADD: hipLaunchKernelGGL(k_gemv16<DG_ADD>, grid, block, 0, st, p); break;
    case DG_SWIGLU: hipLaunchKernelGGL(k_gemv16<DG_SWIGLU>, grid, block, 0, st, p); break;
    case DG_LOGITS: hipLaunchKernelGGL(k_gemv16<DG_LOGITS>, grid, block, 0, st, p); break;
    default: throw BackendError("draft gemv: mode");
    }
}

// ---- RMSNorm of up to two rows (f16 or f32 in, f16 out) ----------------------
// row i: out[i] = f16(x / sqrt(mean(x^2) + eps) * w), x = f16 of the input
// (the reference casts an f32 input to the draft's dtype first).  1024
// threads, each holding up to kNormPer elements, loaded in one batch.
constexpr int kNormT = 1024;
template <int PER>  // elements per thread: H <= 1024 PER
__global__ __launch_bounds__(kNormT) void k_rmsnorm16(DraftNorm p) {
    warm_kernargs<sizeof(DraftNorm)>();
    const int r = blockIdx.x;
    const uint16_t *x16 = p.x16[r];
    const float *x32 = p.x32[r];
    const uint16_t *w = p.w[r];
    uint16_t *out = p.out[r];
    __shared__ float red[kNormT / 64];
    float v[PER];
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int i = threadIdx.x + j * kNormT;
        const int ic = i < p.H ? i : 0;
        const float a = x32 ? r16(x32[ic]) : h2f(x16[ic]);
        v[j] = i < p.H ? a : 0.f;
    }
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < PER; j++) s += v[j] * v[j];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    float ms = 0.f;
#pragma unroll
    for (int k = 0; k < kNormT / 64; k++) ms += red[k];
    ms /= (float)p.H;
    const float inv = 1.0f / sqrtf(ms + p.eps);
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int i = threadIdx.x + j * kNormT;
        if (i < p.H) out[i] = f2h(v[j] * inv * h2f(w[i]));
    }
}

void launch_rmsnorm16(const DraftNorm &p, int rows, hipStream_t st) {
    if (rows < 1 || rows > 2) throw BackendError("draft norm rows");
    const int per = (p.H + kNormT - 1) / kNormT;
    const dim3 g(rows), b(kNormT);
    if (p.H < 1) throw BackendError("draft norm width");
    else if (per <= 4) hipLaunchKernelGGL(k_rmsnorm16<4>, g, b, 0, st, p);
    else if (per <= 8) hipLaunchKernelGGL(k_rmsnorm16<8>, g, b, 0, st, p);
    else if (per <= 16) hipLaunchKernelGGL(k_rmsnorm16<16>, g, b, 0, st, p);
    else if (per <= 32) hipLaunchKernelGGL(k_rmsnorm16<32>, g, b, 0, st, p);
    else throw BackendError("draft norm width");
}

// ---- one row of an f16 table, the row id on the device ------------------------------
__global__ void k_gather16(const uint16_t *table, int64_t rows, int H, const int32_t *id, uint16_t *out) {
    const int i = (blockIdx.x * blockDim.x + threadIdx.x) * 8;
    const int64_t r = *id;
    if (i >= H || r < 0 || r >= rows) return;
    *(uintx4 *)(out + i) = *(const uintx4 *)(table + r * H + i);
}
void launch_gather16(const uint16_t *table, int64_t rows, int H, const int32_t *id, uint16_t *out, hipStream_t st) {
    if (H % 8) throw BackendError("draft gather: width must be a multiple of 8");
    hipLaunchKernelGGL(k_gather16, dim3((H / 8 + 255) / 256), dim3(256), 0, st, table, rows, H, id, out);
}

// ---- f32 -> f16 ------------------------------------------------------------------
__global__ void k_to_f16(const float *x, int64_t n, uint16_t *y) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) y[i] = f2h(x[i]);
}
void launch_to_f16(const float *x, int64_t n, uint16_t *y, hipStream_t st) {
    hipLaunchKernelGGL(k_to_f16, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, x, n, y);
}

// ---- RoPE, the draft cache append and attention, one wave per query head ----
// q and this step's k rotated by the half-rotation RoPE at `pos` in f16
// arithmetic (y1 = x1 c - x2 s, y2 = x1 s + x2 c, every product and sum
// rounded), scores f16(f16(q . k_j) * scale) over the cached steps and this
// one, softmax in f32 rounded to f16, out = f16(sum_j p_j v_j).  Every wave of
// a kv head rotates that head's k itself; the first of them appends k and v to
// slot `step` of the caches, which later steps read.  A lane holds the
// rotation pairs (i, i + hd/2) for i = lane and lane + 64.
constexpr int kAttnPairs = 2;  // head_dim up to 256
__global__ __launch_bounds__(64) void k_draft_attn(DraftAttn p) {
    warm_kernargs<sizeof(DraftAttn)>();
    const int h = blockIdx.x, lane = threadIdx.x;
    const int rep = p.n_heads / p.n_kv, kv = h / rep;
    const int hd = p.hd, half = hd / 2, T = p.step + 1;
    const uint16_t *cs = p.cos16 + (int64_t)p.pos * half, *sn = p.sin16 + (int64_t)p.pos * half;
    const uint16_t *qg = p.qkv + (int64_t)h * hd;
    const uint16_t *kg = p.qkv + (int64_t)(p.n_heads + kv) * hd;
    const uint16_t *vg = p.qkv + (int64_t)(p.n_heads + p.n_kv + kv) * hd;
    _Float16 q1[kAttnPairs], q2[kAttnPairs], k1[kAttnPairs], k2[kAttnPairs];
    float v1[kAttnPairs], v2[kAttnPairs];
#pragma unroll
    for (int e = 0; e < kAttnPairs; e++) {
        const int i = lane + 64 * e;
        const int ic = i < half ? i : 0;
        const _Float16 c = __builtin_bit_cast(_Float16, cs[ic]), sv = __builtin_bit_cast(_Float16, sn[ic]);
        const _Float16 x1 = __builtin_bit_cast(_Float16, qg[ic]), x2 = __builtin_bit_cast(_Float16, qg[ic + half]);
        const _Float16 a1 = __builtin_bit_cast(_Float16, kg[ic]), a2 = __builtin_bit_cast(_Float16, kg[ic + half]);
        const _Float16 qa = x1 * c, qb = x2 * sv, qc = x1 * sv, qd = x2 * c;
        const _Float16 ka = a1 * c, kb = a2 * sv, kc = a1 * sv, kd = a2 * c;
        const bool in = i < half;
        q1[e] = in ? (_Float16)(qa - qb) : (_Float16)0;
        q2[e] = in ? (_Float16)(qc + qd) : (_Float16)0;
        k1[e] = in ? (_Float16)(ka - kb) : (_Float16)0;
        k2[e] = in ? (_Float16)(kc + kd) : (_Float16)0;
        v1[e] = in ? h2f(vg[ic]) : 0.f;
        v2[e] = in ? h2f(vg[ic + half]) : 0.f;
    }
    if (h % rep == 0) {
        uint16_t *kd = p.kcache + ((int64_t)p.step * p.n_kv + kv) * hd;
        uint16_t *vd = p.vcache + ((int64_t)p.step * p.n_kv + kv) * hd;
#pragma unroll
        for (int e = 0; e < kAttnPairs; e++) {
            const int i = lane + 64 * e;
            if (i < half) {
                kd[i] = __builtin_bit_cast(uint16_t, k1[e]);
                kd[i + half] = __builtin_bit_cast(uint16_t, k2[e]);
                vd[i] = vg[i];
                vd[i + half] = vg[i + half];
            }
        }
    }
    // scores: the cached steps' keys loaded in one batch (clamped to slot 0
    // past the cached ones, every load issued), this step's from registers
    float sc[kDraftMaxSteps];
#pragma unroll
    for (int j = 0; j < kDraftMaxSteps; j++) {
        const int jc = j < T - 1 ? j : 0;
        const uint16_t *kj = p.kcache + ((int64_t)jc * p.n_kv + kv) * hd;
        float a = 0.f, b = 0.f;
#pragma unroll
        for (int e = 0; e < kAttnPairs; e++) {
            const int i = lane + 64 * e;
            const int ic = i < half ? i : 0;
            const float c1 = h2f(kj[ic]), c2 = h2f(kj[ic + half]);
            if (i < half) {
                a += (float)q1[e] * c1 + (float)q2[e] * c2;
                b += (float)q1[e] * (float)k1[e] + (float)q2[e] * (float)k2[e];
            }
        }
        sc[j] = j < T - 1 ? a : (j == T - 1 ? b : 0.f);
    }
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < kDraftMaxSteps; j++) {
        float a = sc[j];
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) a += __shfl_xor(a, o);
        sc[j] = r16(r16(a) * p.scale);
        if (j < T) mx = fmaxf(mx, sc[j]);
    }
    float sum = 0.f;
#pragma unroll
    for (int j = 0; j < kDraftMaxSteps; j++) {
        sc[j] = j < T ? expf(sc[j] - mx) : 0.f;
        sum += sc[j];
    }
    float o1[kAttnPairs] = {}, o2[kAttnPairs] = {};
#pragma unroll
    for (int j = 0; j < kDraftMaxSteps; j++) {
        const float pj = r16(sc[j] / sum);
        const int jc = j < T - 1 ? j : 0;
        const uint16_t *vj = p.vcache + ((int64_t)jc * p.n_kv + kv) * hd;
#pragma unroll
        for (int e = 0; e < kAttnPairs; e++) {
            const int i = lane + 64 * e;
            const int ic = i < half ? i : 0;
            const float c1 = h2f(vj[ic]), c2 = h2f(vj[ic + half]);
            const float a = j < T - 1 ? c1 : v1[e], b = j < T - 1 ? c2 : v2[e];
            if (j < T) {
                o1[e] += pj * a;
                o2[e] += pj * b;
            }
        }
    }
#pragma unroll
    for (int e = 0; e < kAttnPairs; e++) {
        const int i = lane + 64 * e;
        if (i < half) {
            p.out[(int64_t)h * hd + i] = f2h(o1[e]);
            p.out[(int64_t)h * hd + i + half] = f2h(o2[e]);
        }
    }
}
void launch_draft_attn(const DraftAttn &p, hipStream_t st) {
    if (p.step < 0 || p.step >= kDraftMaxSteps) throw BackendError("draft attention: steps out of range");
    if (p.hd % 2 || p.hd > 128 * kAttnPairs || p.n_heads % p.n_kv) throw BackendError("draft attention: head layout");
    hipLaunchKernelGGL(k_draft_attn, dim3(p.n_heads), dim3(64), 0, st, p);
}

// ---- top-k, log-probs and the next step's token --------------------------------
// Slices of kTkSlice logits, one workgroup each: the slice's max m (NaN
// skipped, as f32::max folds), its sum s of exp(l - m) over the entries above
// -inf, and its top k by (value descending, index ascending)
// (medusa.rs:477-487; NaN after every number, NaNs by index), found in k
// selection rounds (each takes the first item of the order after the previous
// winner).  The last workgroup to finish merges the slices in slice order:
// M = max m, S = sum over slices of s exp(m - M) (NaN when every logit is
// -inf, as the reference's sum of exp(-inf - -inf) is), lse = ln S + M, and
// the top k of the slices' candidates.  Outputs the draft ids, l_i - lse, the
// target ids through d2t, and the top-1 target id as the next step's token.
constexpr int kTkT = 256, kTkPer = 4, kTkSlice = kTkT * kTkPer, kTkMaxSlices = 256, kTkLaneSlices = kTkMaxSlices / 64;
static_assert(kTkSlice * kTkMaxSlices >= 262144, "draft top-k slices");
__device__ __forceinline__ bool tk_before(float v1, int i1, float v2, int i2) {
    const bool n1 = v1 != v1, n2 = v2 != v2;
    if (n1 || n2) return n1 == n2 ? i1 < i2 : n2;
    return v1 > v2 || (v1 == v2 && i1 < i2);
}
__device__ __forceinline__ void tk_wave_best(float &bv, int &bi) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o);
        const int oi = __shfl_xor(bi, o);
        if (tk_before(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
        }
    }
}
__device__ __forceinline__ void tk_st64(uint64_t *p, float a, uint32_t b) {
    __hip_atomic_store(p, (uint64_t)__float_as_uint(a) | ((uint64_t)b << 32), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void tk_ld64(const uint64_t *p, float &a, int &b) {
    const uint64_t u = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    a = __uint_as_float((uint32_t)u);
    b = (int)(uint32_t)(u >> 32);
}
constexpr int kTkNone = 0x7fffffff;
__global__ __launch_bounds__(kTkT) void k_draft_topk(DraftTopk p) {
    warm_kernargs<sizeof(DraftTopk)>();
    __shared__ float sv[2][kTkT / 64], red[kTkT / 64], wv[kDraftMaxTopk];
    __shared__ int si[2][kTkT / 64], wi[kDraftMaxTopk];
    __shared__ int s_last;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, sl = blockIdx.x, nsl = gridDim.x;
    float v[kTkPer];
    int xi[kTkPer];
#pragma unroll
    for (int j = 0; j < kTkPer; j++) {
        xi[j] = sl * kTkSlice + t + j * kTkT;
        v[j] = p.logits[xi[j] < p.V ? xi[j] : 0];
    }
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < kTkPer; j++)
        if (xi[j] < p.V && v[j] == v[j]) mx = fmaxf(mx, v[j]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < kTkPer; j++)
        if (xi[j] < p.V && v[j] != -INFINITY) s += expf(v[j] - mx);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
    if (lane == 0) red[wave] = s;
    float lv = 0.f;
    int li = -1;
    for (int r = 0; r < p.k; r++) {
        float bv = NAN;
        int bi = kTkNone;
#pragma unroll
        for (int j = 0; j < kTkPer; j++) {
            const bool elig = xi[j] < p.V && (li < 0 || tk_before(lv, li, v[j], xi[j]));
            if (elig && tk_before(v[j], xi[j], bv, bi)) {
                bv = v[j];
                bi = xi[j];
            }
        }
        tk_wave_best(bv, bi);
        if (lane == 0) {
            sv[r & 1][wave] = bv;
            si[r & 1][wave] = bi;
        }
        __syncthreads();
        bv = sv[r & 1][0];
        bi = si[r & 1][0];
#pragma unroll
        for (int w = 1; w < kTkT / 64; w++)
            if (tk_before(sv[r & 1][w], si[r & 1][w], bv, bi)) {
                bv = sv[r & 1][w];
                bi = si[r & 1][w];
            }
        lv = bv;
        li = bi;
        if (t == 0) {
            wv[r] = bv;
            wi[r] = bi;
        }
    }
    if (t == 0) {
        uint64_t *pp = p.part + (int64_t)sl * (1 + kDraftMaxTopk);
        tk_st64(pp, mx, __float_as_uint((red[0] + red[1]) + (red[2] + red[3])));
        for (int r = 0; r < p.k; r++) tk_st64(pp + 1 + r, wv[r], (uint32_t)wi[r]);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the partials are stored before the count
        const int last = __hip_atomic_fetch_add(p.cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == nsl - 1;
        if (last) __hip_atomic_store(p.cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = last;
    }
    __syncthreads();
    if (!s_last || wave != 0) return;
    // the merge, one wave: lane l holds slices l, l + 64, ... (kTkLaneSlices of them)
    float cv[kTkLaneSlices * kDraftMaxTopk];
    int ci[kTkLaneSlices * kDraftMaxTopk];
    float m_l[kTkLaneSlices], s_l[kTkLaneSlices];
#pragma unroll
    for (int q = 0; q < kTkLaneSlices; q++) {
        const int w = lane + 64 * q;
        m_l[q] = -INFINITY;
        s_l[q] = 0.f;
        if (w < nsl) {
            int sb;
            tk_ld64(p.part + (int64_t)w * (1 + kDraftMaxTopk), m_l[q], sb);
            s_l[q] = __int_as_float(sb);
        }
#pragma unroll
        for (int r = 0; r < kDraftMaxTopk; r++) {
            float a = NAN;
            int b = kTkNone;
            if (w < nsl && r < p.k) tk_ld64(p.part + (int64_t)w * (1 + kDraftMaxTopk) + 1 + r, a, b);
            cv[q * kDraftMaxTopk + r] = a;
            ci[q * kDraftMaxTopk + r] = (b < 0 || b >= p.V) ? kTkNone : b;
        }
    }
    float M = -INFINITY;
#pragma unroll
    for (int q = 0; q < kTkLaneSlices; q++) M = fmaxf(M, m_l[q]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) M = fmaxf(M, __shfl_xor(M, o));
    float S = 0.f;  // in slice order, the same on every lane
    for (int w = 0; w < nsl; w++) {
        float mw = 0.f, sw = 0.f;
#pragma unroll
        for (int q = 0; q < kTkLaneSlices; q++)
            if (w >> 6 == q) {
                mw = __shfl(m_l[q], w & 63);
                sw = __shfl(s_l[q], w & 63);
            }
        if (mw != -INFINITY) S += sw * expf(mw - M);
    }
    if (M == -INFINITY) S = NAN;
    const float lse = logf(S) + M;
    float lv2 = 0.f;
    int li2 = -1;
    for (int r = 0; r < p.k; r++) {
        float bv = NAN;
        int bi = kTkNone;
#pragma unroll
        for (int j = 0; j < kTkLaneSlices * kDraftMaxTopk; j++) {
            const bool elig = ci[j] != kTkNone && (li2 < 0 || tk_before(lv2, li2, cv[j], ci[j]));
            if (elig && tk_before(cv[j], ci[j], bv, bi)) {
                bv = cv[j];
                bi = ci[j];
            }
        }
        tk_wave_best(bv, bi);
        lv2 = bv;
        li2 = bi;
        if (lane == 0) {
            const bool ok = bi >= 0 && bi < p.V;
            const int tgt = ok ? (p.d2t ? p.d2t[bi] : bi) : -1;
            p.out_draft[r] = ok ? bi : -1;
            p.out_lp[r] = ok ? bv - lse : NAN;
            p.out_target[r] = tgt;
            if (r == 0) *p.next_token = ok ? tgt : 0;
        }
    }
}
void launch_draft_topk(const DraftTopk &p, hipStream_t st) {
    if (p.k < 1 || p.k > kDraftMaxTopk || p.k > p.V) throw BackendError("draft top-k: k out of range");
    const int nsl = (p.V + kTkSlice - 1) / kTkSlice;
    if (nsl > kTkMaxSlices || !p.part || !p.cnt) throw BackendError("draft top-k: vocabulary over 262144 or no scratch");
    hipLaunchKernelGGL(k_draft_topk, dim3(nsl), dim3(kTkT), 0, st, p);
}

}  // namespace sd
