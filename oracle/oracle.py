"""CPU oracle for the target-verify path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg
may import this module, and only to check results against (or as the timed CPU
baseline).  The product (``abyo-speculate_amd/``) never imports it.

It restates, op by op, the reference's quantized target forward and the
decoder / tree / acceptance semantics around it (paths relative to the
reference checkout):

* forward: ``crates/speculate/src/model/quantized_llama_local.rs`` (whole file)
  and ``quantized_qwen2_local.rs:69-139,181-197,345-395`` -- embedding gather
  of the dequantised table, per layer RMSNorm -> Q/K/V QMatMul (+bias for Qwen2)
  -> RoPE (interleaved ``rope_i`` for Llama, half rotation ``rope`` for Qwen2)
  -> KV append -> GQA softmax(QK^T/sqrt(hd) + bias) V -> wo -> residual ->
  RMSNorm -> SwiGLU MLP -> residual; final RMSNorm; lm_head.
  KV entries are stored as fp16 (the build's cache dtype); all else is f32
  with f64 accumulation in the matmuls / reductions.
* decoder state machine: ``model/quantized_llama.rs:137-167,262-440,519-599``.
* tree utilities: ``tree.rs:52-281``; Cartesian builder ``methods/medusa.rs:172-193``;
  pruning ``methods/eagle.rs:763-845``; top-k ``methods/medusa.rs:477-487``.
* acceptance: greedy tree walk ``methods/eagle.rs:618-661`` (same in
  ``eagle3.rs:714-756``), Leviathan ``methods/vanilla.rs:59-106,178-210``,
  sampling ``sampling/tokens.rs:15-120`` (the last four through the C
  library, which folds sequentially in f32 with libm ``expf``), d2t/t2d
  ``methods/eagle3.rs:377-397,476-513``.

Which checks pin each function is recorded in the tests (``tests/test_oracle_*``).
"""
from __future__ import annotations

import ctypes
import math
import os
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle.so")

# GGML type ids used as format ids throughout.
F32, Q8_0, Q4_K, Q5_K, Q6_K = 0, 8, 12, 13, 14
BLOCK_BYTES = {Q4_K: 144, Q5_K: 176, Q6_K: 210, Q8_0: 34}
BLOCK_ELEMS = {Q4_K: 256, Q5_K: 256, Q6_K: 256, Q8_0: 32}
FMT_NAMES = {F32: "F32", Q8_0: "Q8_0", Q4_K: "Q4_K", Q5_K: "Q5_K", Q6_K: "Q6_K"}

_lib = None


def lib():
    """Load liboracle.so (built by __graft_entry__.build() / oracle/build_oracle.py)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle library missing: {LIB_PATH} (run __graft_entry__.build())")
        L = ctypes.CDLL(LIB_PATH)
        P = ctypes.c_void_p
        i64 = ctypes.c_int64
        L.or_f16_to_f32.restype = ctypes.c_float
        L.or_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.or_f32_to_f16.restype = ctypes.c_uint16
        L.or_f32_to_f16.argtypes = [ctypes.c_float]
        for n in ("or_f32_to_f16_array", "or_f16_to_f32_array"):
            getattr(L, n).argtypes = [P, i64, P]
        L.or_get_scale_min_k4.argtypes = [ctypes.c_int, P, P, P]
        L.or_dequant.argtypes = [ctypes.c_int, P, i64, P]
        L.or_dequant.restype = ctypes.c_int
        L.or_dequant_rows.argtypes = [ctypes.c_int, P, i64, i64, i64, P]
        L.or_dequant_rows.restype = ctypes.c_int
        L.or_qmatmul.argtypes = [ctypes.c_int, P, i64, i64, P, i64, P]
        L.or_qmatmul.restype = ctypes.c_int
        L.or_quantize.argtypes = [ctypes.c_int, P, i64, P]
        L.or_quantize.restype = ctypes.c_int
        L.or_mix64.argtypes = [ctypes.c_uint64]
        L.or_mix64.restype = ctypes.c_uint64
        L.or_synth_value.argtypes = [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_float]
        L.or_synth_value.restype = ctypes.c_float
        L.or_synth_f32.argtypes = [ctypes.c_uint64, i64, ctypes.c_float, P]
        L.or_synth_quant.argtypes = [ctypes.c_int, ctypes.c_uint64, i64, i64, ctypes.c_float, P]
        L.or_synth_quant.restype = ctypes.c_int
        L.or_argmax_fold.argtypes = [P, i64]
        L.or_argmax_fold.restype = i64
        L.or_softmax_t.argtypes = [P, i64, ctypes.c_float, P]
        L.or_softmax_t.restype = ctypes.c_int
        L.or_sample_u.argtypes = [P, i64, ctypes.c_float]
        L.or_sample_u.restype = i64
        L.or_rejection_step.argtypes = [ctypes.c_float, ctypes.c_float, ctypes.c_float]
        L.or_rejection_step.restype = ctypes.c_int
        L.or_adjusted.argtypes = [P, P, i64, P]
        L.or_adjusted.restype = ctypes.c_int
        L.or_rope_tables.argtypes = [i64, ctypes.c_float, i64, P, P]
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


# ---------------------------------------------------------------------------
# fp16, blocks
# ---------------------------------------------------------------------------
def f32_to_f16_bits(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().or_f32_to_f16_array(_p(x), x.size, _p(out))
    return out


def f16_bits_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().or_f16_to_f32_array(_p(h), h.size, _p(out))
    return out


def round_f16(x) -> np.ndarray:
    """f32 -> nearest binary16 -> f32 (the KV cache's storage rounding)."""
    return f16_bits_to_f32(f32_to_f16_bits(x))


def row_bytes(fmt: int, K: int) -> int:
    if fmt == F32:
        return 4 * K
    assert K % BLOCK_ELEMS[fmt] == 0, (fmt, K)
    return K // BLOCK_ELEMS[fmt] * BLOCK_BYTES[fmt]


def dequant(fmt: int, blocks: np.ndarray, n_elems: int) -> np.ndarray:
    """Dequantise a flat block buffer to f32 (bit-exact restatement)."""
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    nb = n_elems // BLOCK_ELEMS[fmt]
    assert blocks.size >= nb * BLOCK_BYTES[fmt]
    out = np.empty(n_elems, np.float32)
    rc = lib().or_dequant(fmt, _p(blocks), nb, _p(out))
    assert rc == 0
    return out


def dequant_matrix(fmt: int, blocks: np.ndarray, N: int, K: int) -> np.ndarray:
    if fmt == F32:
        return np.frombuffer(np.ascontiguousarray(blocks).tobytes(), np.float32).reshape(N, K).copy()
    out = np.empty((N, K), np.float32)
    rc = lib().or_dequant_rows(fmt, _p(np.ascontiguousarray(blocks)), K, 0, N, _p(out))
    assert rc == 0
    return out


def quantize(fmt: int, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    nb = x.size // BLOCK_ELEMS[fmt]
    out = np.zeros(nb * BLOCK_BYTES[fmt], np.uint8)
    assert lib().or_quantize(fmt, _p(x), nb, _p(out)) == 0
    return out


def get_scale_min_k4(j: int, scales12: bytes) -> Tuple[int, int]:
    q = np.frombuffer(bytes(scales12), np.uint8).copy()
    d = np.zeros(1, np.uint8)
    m = np.zeros(1, np.uint8)
    lib().or_get_scale_min_k4(j, _p(q), _p(d), _p(m))
    return int(d[0]), int(m[0])


# ---------------------------------------------------------------------------
# Synthetic model (seeded; identical to the product's GPU generator)
# ---------------------------------------------------------------------------
GOLDEN = 0x9E3779B97F4A7C15
MASK64 = (1 << 64) - 1

# tensor kinds (global ones use layer = -1)
K_TOK_EMBD, K_OUTPUT, K_OUTPUT_NORM = 0, 1, 2
K_ATTN_Q, K_ATTN_K, K_ATTN_V, K_ATTN_O = 3, 4, 5, 6
K_FFN_GATE, K_FFN_UP, K_FFN_DOWN = 7, 8, 9
K_ATTN_NORM, K_FFN_NORM = 10, 11
K_BQ, K_BK, K_BV = 12, 13, 14
K_KV_FILL = 15


def mix64(z: int) -> int:
    z &= MASK64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & MASK64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & MASK64
    return z ^ (z >> 31)


def tensor_seed(model_seed: int, layer: int, kind: int) -> int:
    """Seed of one tensor: mix64(model_seed ^ ((layer+1) << 8 | kind) * C)."""
    tag = (((layer + 1) << 8) | kind) * 0xD1B54A32D192ED03
    return mix64((model_seed ^ tag) & MASK64)


def synth_mult(std: float) -> float:
    return float(np.float32(std * math.sqrt(3.0) / 65536.0))


def synth_f32(seed: int, n: int, std: float) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().or_synth_f32(seed, n, synth_mult(std), _p(out))
    return out


def synth_quant(fmt: int, seed: int, rows: int, K: int, std: float) -> np.ndarray:
    out = np.zeros(rows * row_bytes(fmt, K), np.uint8)
    assert lib().or_synth_quant(fmt, seed, rows, K, synth_mult(std), _p(out)) == 0
    return out


def use_more_bits(i: int, n: int) -> bool:
    """llama.cpp's Q4_K_M rule for attn_v / ffn_down (external; 16 of 32 layers)."""
    return i < n // 8 or i >= 7 * n // 8 or (i - n // 8) % 3 == 2


@dataclass
class ModelConfig:
    arch: str = "llama"  # "llama" (rope_i, no bias) | "qwen2" (rope, QKV bias)
    n_layers: int = 4
    hidden: int = 512
    n_heads: int = 8
    n_kv_heads: int = 8
    head_dim: int = 64
    ffn: int = 1536
    vocab: int = 32000
    rope_theta: float = 10000.0
    rms_eps: float = 1e-5
    ctx_len: int = 4096
    mix: str = "q4_k"  # "q4_k" | "q4_k_m" | "q5k_q80"
    seed: int = 0x5EED0001
    weight_std: float = 0.02
    tied_output: bool = False

    @property
    def q_dim(self):
        return self.n_heads * self.head_dim

    @property
    def kv_dim(self):
        return self.n_kv_heads * self.head_dim

    def fmt(self, layer: int, kind: int) -> int:
        if kind in (K_OUTPUT_NORM, K_ATTN_NORM, K_FFN_NORM, K_BQ, K_BK, K_BV):
            return F32
        if self.mix == "q4_k":
            return Q4_K
        if self.mix == "q4_k_m":
            if kind in (K_ATTN_V, K_FFN_DOWN) and use_more_bits(layer, self.n_layers):
                return Q6_K
            return Q4_K
        if self.mix == "q5k_q80":
            if kind in (K_ATTN_Q, K_ATTN_K, K_ATTN_V, K_ATTN_O):
                return Q5_K
            return Q8_0
        single = {"q6_k": Q6_K, "q5_k": Q5_K, "q8_0": Q8_0}
        if self.mix in single:
            return single[self.mix]
        raise ValueError(self.mix)

    def shape(self, kind: int) -> Tuple[int, int]:
        H, F = self.hidden, self.ffn
        return {
            K_TOK_EMBD: (self.vocab, H), K_OUTPUT: (self.vocab, H), K_OUTPUT_NORM: (1, H),
            K_ATTN_Q: (self.q_dim, H), K_ATTN_K: (self.kv_dim, H), K_ATTN_V: (self.kv_dim, H),
            K_ATTN_O: (H, self.q_dim), K_FFN_GATE: (F, H), K_FFN_UP: (F, H), K_FFN_DOWN: (H, F),
            K_ATTN_NORM: (1, H), K_FFN_NORM: (1, H),
            K_BQ: (1, self.q_dim), K_BK: (1, self.kv_dim), K_BV: (1, self.kv_dim),
        }[kind]

    def layer_kinds(self) -> List[int]:
        ks = [K_ATTN_Q, K_ATTN_K, K_ATTN_V, K_ATTN_O, K_FFN_GATE, K_FFN_UP, K_FFN_DOWN, K_ATTN_NORM, K_FFN_NORM]
        if self.arch == "qwen2":
            ks += [K_BQ, K_BK, K_BV]
        return ks


def synth_tensor(cfg: ModelConfig, layer: int, kind: int) -> Tuple[int, np.ndarray]:
    """(fmt, raw bytes) of one synthetic tensor."""
    rows, K = cfg.shape(kind)
    fmt = cfg.fmt(layer, kind)
    if kind in (K_OUTPUT_NORM, K_ATTN_NORM, K_FFN_NORM):
        return F32, np.ones(K, np.float32).view(np.uint8)
    seed = tensor_seed(cfg.seed, layer, kind)
    if fmt == F32:
        return F32, synth_f32(seed, rows * K, cfg.weight_std).view(np.uint8)
    return fmt, synth_quant(fmt, seed, rows, K, cfg.weight_std)


# ---------------------------------------------------------------------------
# Forward (numpy restatement of quantized_llama_local.rs)
# ---------------------------------------------------------------------------
def rope_tables(dim: int, base: float, ctx: int) -> Tuple[np.ndarray, np.ndarray]:
    h = dim // 2
    c = np.empty((ctx, h), np.float32)
    s = np.empty((ctx, h), np.float32)
    lib().or_rope_tables(dim, base, ctx, _p(c), _p(s))
    return c, s


def rope_interleaved(x: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """candle rope_i: pairs (2i, 2i+1).  x [..., T, d], cos/sin [T, d/2]."""
    a, b = x[..., 0::2], x[..., 1::2]
    out = np.empty_like(x)
    out[..., 0::2] = a * cos - b * sin
    out[..., 1::2] = a * sin + b * cos
    return out


def rope_half(x: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """candle rope: pairs (i, i + d/2)."""
    h = x.shape[-1] // 2
    a, b = x[..., :h], x[..., h:]
    out = np.empty_like(x)
    out[..., :h] = a * cos - b * sin
    out[..., h:] = a * sin + b * cos
    return out


def rms_norm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x64 = x.astype(np.float64)
    ms = (x64 * x64).mean(axis=-1, keepdims=True)
    return (x64 / np.sqrt(ms + eps) * w.astype(np.float64)).astype(np.float32)


def silu(x: np.ndarray) -> np.ndarray:
    x64 = x.astype(np.float64)
    return (x64 / (1.0 + np.exp(-x64))).astype(np.float32)


def matmul_t(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    """x [M,K] . w[N,K]^T with f64 accumulation (row chunks bound the f64 copy)."""
    x64 = x.astype(np.float64)
    out = np.empty((x.shape[0], w.shape[0]), np.float32)
    step = max(1, (1 << 24) // max(1, w.shape[1]))
    for r0 in range(0, w.shape[0], step):
        out[:, r0:r0 + step] = (x64 @ w[r0:r0 + step].astype(np.float64).T).astype(np.float32)
    return out


def attend(q: np.ndarray, k_all: np.ndarray, v_all: np.ndarray, mask: np.ndarray, scale: float) -> np.ndarray:
    """LayerWeights::run_attn's core (quantized_llama_local.rs:116-129):
    softmax(q k^T * scale + bias) v with GQA through repeat_kv (query head h
    reads KV head h // n_rep: repeat_kv concatenates n_rep copies along the
    sequence axis and reshapes, candle-transformers utils, restated at
    llama_local.rs:171-177).  q [n_heads, M, hd], k_all/v_all [n_kv, T, hd],
    mask [M, T] bool (True = visible; the additive bias is 0 / -inf).
    f64 throughout; returns [M, n_heads, hd] f32."""
    n_heads, M, hd = q.shape
    n_kv = k_all.shape[0]
    n_rep = n_heads // n_kv
    y = np.empty((M, n_heads, hd), np.float32)
    K = k_all.astype(np.float64)
    V = v_all.astype(np.float64)
    for h in range(n_heads):
        kv = h // n_rep
        s = (q[h].astype(np.float64) @ K[kv].T) * float(scale)
        s = np.where(mask, s, -np.inf)
        s = s - s.max(axis=1, keepdims=True)
        p = np.exp(s)
        p = p / p.sum(axis=1, keepdims=True)
        y[:, h, :] = (p @ V[kv]).astype(np.float32)
    return y


class OracleModel:
    """Dequantised weights + fp16 KV cache + the forward of quantized_llama_local.rs."""

    def __init__(self, cfg: ModelConfig, tensors: Optional[Dict[Tuple[int, int], Tuple[int, np.ndarray]]] = None):
        self.cfg = cfg
        self.raw: Dict[Tuple[int, int], Tuple[int, np.ndarray]] = {}
        if tensors is None:
            tensors = {}
            kinds = [(-1, K_TOK_EMBD), (-1, K_OUTPUT_NORM)] + ([] if cfg.tied_output else [(-1, K_OUTPUT)])
            for li in range(cfg.n_layers):
                kinds += [(li, k) for k in cfg.layer_kinds()]
            for (li, k) in kinds:
                tensors[(li, k)] = synth_tensor(cfg, li, k)
        self.raw = tensors
        self.w: Dict[Tuple[int, int], np.ndarray] = {}
        for (li, k), (fmt, data) in tensors.items():
            rows, K = cfg.shape(k)
            self.w[(li, k)] = dequant_matrix(fmt, data, rows, K) if fmt != F32 else \
                np.frombuffer(data.tobytes(), np.float32).reshape(rows, K).copy()
        if cfg.tied_output:
            self.w[(-1, K_OUTPUT)] = self.w[(-1, K_TOK_EMBD)]
        self.cos, self.sin = rope_tables(cfg.head_dim, cfg.rope_theta, cfg.ctx_len)
        # per layer fp16-valued K, V: [n_kv, T, hd] float32 holding fp16 values
        self.k_cache: List[Optional[np.ndarray]] = [None] * cfg.n_layers
        self.v_cache: List[Optional[np.ndarray]] = [None] * cfg.n_layers

    # -- cache ops (quantized_llama_local.rs:162-186, 434-463) --
    def cache_len(self) -> int:
        k = self.k_cache[0]
        return 0 if k is None else k.shape[1]

    def clear_kv_cache(self):
        self.k_cache = [None] * self.cfg.n_layers
        self.v_cache = [None] * self.cfg.n_layers

    def truncate_kv_cache_to(self, n: int):
        for li in range(self.cfg.n_layers):
            k = self.k_cache[li]
            if k is None:
                continue
            cur = k.shape[1]
            if n > cur:
                raise RuntimeError(f"truncate_kv_cache_to({n}) exceeds {cur}")
            if n == 0:
                self.k_cache[li] = self.v_cache[li] = None
            elif n < cur:
                self.k_cache[li] = k[:, :n].copy()
                self.v_cache[li] = self.v_cache[li][:, :n].copy()

    def keep_kv_indices(self, idx: Sequence[int]):
        if len(idx) == 0:
            self.clear_kv_cache()
            return
        ix = np.asarray(idx, np.int64)
        for li in range(self.cfg.n_layers):
            if self.k_cache[li] is not None:
                self.k_cache[li] = self.k_cache[li][:, ix].copy()
                self.v_cache[li] = self.v_cache[li][:, ix].copy()

    # -- forward --
    def embed(self, ids: Sequence[int]) -> np.ndarray:
        return self.w[(-1, K_TOK_EMBD)][np.asarray(ids, np.int64)].copy()

    def forward(self, ids: Sequence[int], positions: Sequence[int], mask: np.ndarray,
                collect_layers: Sequence[int] = ()) -> Tuple[np.ndarray, List[np.ndarray]]:
        """Hidden states after the final norm, [M, H]; mask [M, P+M] bool (True = visible).

        Appends the M new K/V rows (fp16) to every layer's cache, as run_attn does.
        """
        cfg = self.cfg
        M = len(ids)
        pos = np.asarray(positions, np.int64)
        cos, sin = self.cos[pos], self.sin[pos]
        rope = rope_interleaved if cfg.arch == "llama" else rope_half
        x = self.embed(ids)
        collected: Dict[int, np.ndarray] = {}
        scale = np.float32(1.0 / math.sqrt(cfg.head_dim))
        for li in range(cfg.n_layers):
            W = lambda k: self.w[(li, k)]
            xn = rms_norm(x, W(K_ATTN_NORM)[0], cfg.rms_eps)
            q = matmul_t(xn, W(K_ATTN_Q))
            k = matmul_t(xn, W(K_ATTN_K))
            v = matmul_t(xn, W(K_ATTN_V))
            if cfg.arch == "qwen2":
                q = q + W(K_BQ)[0]
                k = k + W(K_BK)[0]
                v = v + W(K_BV)[0]
            q = q.reshape(M, cfg.n_heads, cfg.head_dim).transpose(1, 0, 2)
            k = k.reshape(M, cfg.n_kv_heads, cfg.head_dim).transpose(1, 0, 2)
            v = v.reshape(M, cfg.n_kv_heads, cfg.head_dim).transpose(1, 0, 2)
            q = rope(q, cos, sin)
            k = rope(k, cos, sin)
            k16, v16 = round_f16(k), round_f16(v)
            if self.k_cache[li] is None:
                self.k_cache[li], self.v_cache[li] = k16, v16
            else:
                self.k_cache[li] = np.concatenate([self.k_cache[li], k16], axis=1)
                self.v_cache[li] = np.concatenate([self.v_cache[li], v16], axis=1)
            T = self.k_cache[li].shape[1]
            assert mask.shape == (M, T), (mask.shape, M, T)
            y = attend(q, self.k_cache[li], self.v_cache[li], mask, scale)
            attn = matmul_t(y.reshape(M, cfg.q_dim), W(K_ATTN_O))
            x = (attn + x).astype(np.float32)
            xn = rms_norm(x, W(K_FFN_NORM)[0], cfg.rms_eps)
            g = matmul_t(xn, W(K_FFN_GATE))
            u = matmul_t(xn, W(K_FFN_UP))
            act = (silu(g).astype(np.float64) * u).astype(np.float32)
            x = (matmul_t(act, W(K_FFN_DOWN)) + x).astype(np.float32)
            if li in collect_layers:
                collected[li] = x.copy()
        final = rms_norm(x, self.w[(-1, K_OUTPUT_NORM)][0], cfg.rms_eps)
        return final, [collected[l] for l in collect_layers]

    def lm_head(self, hidden: np.ndarray) -> np.ndarray:
        return matmul_t(hidden, self.w[(-1, K_OUTPUT)])


def causal_mask(prev_len: int, M: int) -> np.ndarray:
    """causal_bias (quantized_llama_local.rs:332-350) as a bool mask [M, prev+M]."""
    m = np.ones((M, prev_len + M), bool)
    for i in range(M):
        m[i, prev_len + i + 1:] = False
    return m


# ---------------------------------------------------------------------------
# DraftTree (tree.rs) and builders
# ---------------------------------------------------------------------------
class DraftTree:
    def __init__(self, tokens: List[int], parents: List[int]):
        self._tokens = list(tokens)
        self._parents = list(parents)

    @staticmethod
    def from_parent_table(nodes: Sequence[Tuple[int, int]]) -> "DraftTree":
        if len(nodes) == 0:
            raise ValueError("DraftTree must have at least a root")
        toks, pars = [int(nodes[0][1])], [0]
        for i, (p, t) in enumerate(nodes):
            if i == 0:
                continue
            if p >= i:
                raise ValueError(f"node {i} has parent index {p}, which is not strictly smaller")
            toks.append(int(t))
            pars.append(int(p))
        return DraftTree(toks, pars)

    @staticmethod
    def linear(root: int, tail: Sequence[int]) -> "DraftTree":
        return DraftTree([root] + list(tail), [0] + list(range(len(tail))))

    def __len__(self):
        return len(self._tokens)

    def token_at(self, i):
        return self._tokens[i]

    def tokens(self):
        return list(self._tokens)

    def parent_of(self, i):
        return self._parents[i]

    def parents(self):
        return list(self._parents)

    def ancestors(self, i):
        out = [i]
        while i != 0:
            i = self._parents[i]
            out.append(i)
        return out

    def depth_of(self, i):
        d = 0
        while i != 0:
            i = self._parents[i]
            d += 1
        return d

    def position_ids(self, prefix_len):
        return [prefix_len + self.depth_of(i) for i in range(len(self))]

    def is_ancestor_of(self, a, n):
        cur = n
        if cur == a:
            return True
        while cur != 0:
            cur = self._parents[cur]
            if cur == a:
                return True
        return a == 0

    def attention_mask_bool(self):
        n = len(self)
        m = [[False] * n for _ in range(n)]
        for i in range(n):
            for j in self.ancestors(i):
                m[i][j] = True
        return m

    def full_attention_bias(self, prefix_len: int) -> np.ndarray:
        n = len(self)
        b = np.zeros((n, prefix_len + n), np.float32)
        for i in range(n):
            for j in range(n):
                if not self.is_ancestor_of(j, i):
                    b[i, prefix_len + j] = -np.inf
        return b

    def paths(self):
        is_leaf = [True] * len(self)
        for p in self._parents[1:]:
            is_leaf[p] = False
        out = []
        for i, leaf in enumerate(is_leaf):
            if leaf:
                c = self.ancestors(i)
                c.reverse()
                out.append(c)
        return out

    def path_to(self, t):
        c = self.ancestors(t)
        c.reverse()
        return c


def build_cartesian_tree(root: int, head_top_k: Sequence[Sequence[int]]) -> DraftTree:
    nodes = [(0, root)]
    prev = [0]
    for cands in head_top_k:
        nxt = []
        for p in prev:
            for c in cands:
                nxt.append(len(nodes))
                nodes.append((p, c))
        prev = nxt
    return DraftTree.from_parent_table(nodes)


def prune_cartesian_tree(full: DraftTree, per_step_log_probs: Sequence[Sequence[float]], max_total: int) -> DraftTree:
    n = len(full)
    if n <= max_total:
        return DraftTree(full.tokens(), full.parents())
    children = [[] for _ in range(n)]
    for i in range(1, n):
        children[full.parent_of(i)].append(i)
    cand = [0] * n
    for sib in children:
        for r, c in enumerate(sib):
            cand[c] = r
    scores = []
    for i in range(1, n):
        d = full.depth_of(i)
        s = np.float32(0.0)
        cur = i
        for dd in range(d - 1, -1, -1):
            s = np.float32(s + np.float32(per_step_log_probs[dd][cand[cur]]))
            cur = full.parent_of(cur)
        scores.append((i, float(s)))
    # stable sort, descending by score (Rust sort_by is stable)
    scores.sort(key=lambda t: -t[1])
    want = min(max(max_total - 1, 0), len(scores))
    keep = [False] * n
    keep[0] = True
    for (i, _) in scores[:want]:
        keep[i] = True
    for i in range(n - 1, 0, -1):
        if keep[i]:
            keep[full.parent_of(i)] = True
    order = [i for i in range(n) if keep[i]]
    order.sort(key=lambda i: full.depth_of(i))  # stable
    new_index = {old: k for k, old in enumerate(order)}
    entries = []
    for old in order:
        po = 0 if old == 0 else full.parent_of(old)
        entries.append((new_index[po], full.token_at(old)))
    return DraftTree.from_parent_table(entries)


def top_k_indices(logits: Sequence[float], k: int) -> List[int]:
    k = min(k, len(logits))
    idx = list(range(len(logits)))
    idx.sort(key=lambda i: (-float(logits[i]), i))
    return idx[:k]


def ancestor_masks(tree: DraftTree) -> np.ndarray:
    """Per-node ancestor-or-self bitmask words: [n, ceil(n/64)] uint64."""
    n = len(tree)
    nw = (n + 63) // 64
    out = np.zeros((n, nw), np.uint64)
    for i in range(n):
        for j in tree.ancestors(i):
            out[i, j // 64] |= np.uint64(1 << (j % 64))
    return out


# ---------------------------------------------------------------------------
# Acceptance
# ---------------------------------------------------------------------------
def argmax_fold(row: np.ndarray) -> int:
    r = np.ascontiguousarray(row, np.float32)
    return int(lib().or_argmax_fold(_p(r), r.size))


def softmax_t(logits: np.ndarray, t: float) -> np.ndarray:
    l = np.ascontiguousarray(logits, np.float32)
    out = np.empty_like(l)
    if lib().or_softmax_t(_p(l), l.size, t, _p(out)) != 0:
        raise ValueError("softmax_with_temperature error")
    return out


def sample_u(probs: np.ndarray, u: float) -> int:
    p = np.ascontiguousarray(probs, np.float32)
    r = int(lib().or_sample_u(_p(p), p.size, u))
    if r < 0:
        raise ValueError("sample_from_distribution error")
    return r


def rejection_step(q: float, p: float, u: float) -> bool:
    return bool(lib().or_rejection_step(q, p, u))


def adjusted_distribution(p: np.ndarray, q: np.ndarray) -> np.ndarray:
    p = np.ascontiguousarray(p, np.float32)
    q = np.ascontiguousarray(q, np.float32)
    if p.size != q.size:
        raise ValueError("vocab size mismatch")
    out = np.empty_like(p)
    if lib().or_adjusted(_p(p), _p(q), p.size, _p(out)) != 0:
        raise ValueError("adjusted distribution has non-positive mass")
    return out


def greedy_tree_accept(tree: DraftTree, logits: Sequence[np.ndarray], argmaxes: Optional[Sequence[int]] = None):
    """eagle.rs:618-661 -> (best_path node indices, bonus token)."""
    am = list(argmaxes) if argmaxes is not None else [argmax_fold(r) for r in logits]
    best = [0]
    for path in tree.paths():
        acc = 0
        for a, b in zip(path[:-1], path[1:]):
            if am[a] == tree.token_at(b):
                acc += 1
            else:
                break
        if acc + 1 > len(best):
            best = path[:acc + 1]
    return best, am[best[-1]]


def bonus_in_tree(tree: DraftTree, deepest: int, bonus: int) -> Optional[int]:
    """eagle.rs:700-709: first child of `deepest` carrying the bonus token."""
    for n in range(1, len(tree)):
        if tree.parent_of(n) == deepest and tree.token_at(n) == bonus:
            return n
    return None


def greedy_tree_commit(tree: DraftTree, best: Sequence[int], bonus: int, eos: Sequence[int], strict: bool = False):
    """Commit composition of run_eagle (eagle.rs:664-732; eagle3.rs:758-782
    is the same without the bonus-in-tree shortcut, i.e. strict here).

    -> (committed tokens, stop, kept node indices for commit_tree_path,
    bonus node or None).  committed = path tokens (root excluded) + bonus,
    cut after the first EOS; an EOS among the path tokens keeps the root and
    the path through that node (no bonus forward follows); otherwise the
    whole path is kept, plus the first child of the deepest node carrying the
    bonus token when not strict.
    """
    eos_set = set(int(e) for e in eos)
    path_tokens = [tree.token_at(i) for i in best[1:]]
    committed = path_tokens + [bonus]
    eos_pos = next((i for i, t in enumerate(committed) if t in eos_set), None)
    stop = eos_pos is not None
    if eos_pos is not None:
        committed = committed[:eos_pos + 1]
    path_eos = next((i for i, t in enumerate(path_tokens) if t in eos_set), None)
    if path_eos is not None:
        return committed, stop, list(best[:path_eos + 2]), None
    bn = None if strict else bonus_in_tree(tree, best[-1], bonus)
    return committed, stop, list(best) + ([bn] if bn is not None else []), bn


def greedy_linear_accept(drafts: Sequence[int], argmaxes: Sequence[int]) -> Tuple[int, int]:
    """Greedy verify of a k-token chain: (#accepted, bonus = argmax of row #accepted)."""
    a = 0
    while a < len(drafts) and argmaxes[a] == drafts[a]:
        a += 1
    return a, argmaxes[a]


def rejection_linear_accept(target_rows: Sequence[np.ndarray], q_rows: Sequence[np.ndarray],
                            drafts: Sequence[int], uniforms: Sequence[float], temperature: float,
                            max_commit: Optional[int] = None):
    """vanilla.rs:178-210 with explicit uniforms consumed in the reference's order.

    Returns (commits, n_accepted, uniforms_used).  uniforms[i] drives draft i's
    test; the resample/bonus draw takes the next unused uniform.
    """
    k = len(drafts)
    commits: List[int] = []
    used = 0
    rejected = False
    for i in range(k):
        p_probs = softmax_t(target_rows[i], temperature)
        q_probs = q_rows[i]
        tok = drafts[i]
        u = uniforms[used]
        used += 1
        if rejection_step(float(q_probs[tok]), float(p_probs[tok]), u):
            commits.append(tok)
            if max_commit is not None and len(commits) >= max_commit:
                break
        else:
            adj = adjusted_distribution(p_probs, q_probs)
            commits.append(sample_u(adj, uniforms[used]))
            used += 1
            rejected = True
            break
    n_acc = len(commits) - (1 if rejected else 0)
    if not rejected and len(commits) == k and (max_commit is None or len(commits) < max_commit):
        commits.append(sample_u(softmax_t(target_rows[k], temperature), uniforms[used]))
        used += 1
    return commits, n_acc, used


def rejection_tree_accept(tree: "DraftTree", target_rows: Sequence[np.ndarray], q_rows: Sequence[np.ndarray],
                          q_row_of: Sequence[int], uniforms: Sequence[float], temperature: float,
                          t2d_mask: Optional[np.ndarray] = None, max_commit: Optional[int] = None,
                          without_replacement: bool = False):
    """Tree rejection walk (a build extension: the reference has no tree rule,
    eagle.rs:739-740 and eagle3.rs:789 ignore the temperature), made of the
    reference's own steps: at the current node, children are tested in BFS
    order with modified_rejection_step (vanilla.rs:59-73) against the node's
    current distribution p (softmax_with_temperature of its row, tokens.rs:15-55)
    and its draft row q = q_rows[q_row_of[node]] (target vocabulary); each
    rejection sets p = adjusted_distribution(p, q) (vanilla.rs:83-106); the first
    accepted child is descended into; with no child left the final token is
    sample_from_distribution(p) (tokens.rs:99-120).  On a chain this is exactly
    rejection_linear_accept.  t2d_mask (eagle3.rs:498-513) sets unreachable
    target logits to -inf first.

    Sibling rule: with i.i.d. siblings q stays the node's draft row; with
    ``without_replacement`` (siblings drawn without replacement from q) the
    sibling tested after rejections x_0..x_{r-1} sees q_r(y) = q(y) / R_r off
    the rejected tokens and 0 on them, R_0 = 1, R_{r+1} = R_r - q(x_r) in f32
    (0 everywhere once R_r <= 0), and each rejection adjusts p against that q_r.

    Returns (path node indices, final token or None, uniforms used).
    """
    n = len(tree)
    children = [[] for _ in range(n)]
    for c in range(1, n):
        children[tree.parent_of(c)].append(c)
    used = 0
    node = 0
    path = [0]
    while True:
        if max_commit is not None and max_commit > 0 and len(path) - 1 >= max_commit:
            return path, None, used
        row = np.array(target_rows[node], np.float32)
        if t2d_mask is not None:
            row[~t2d_mask] = -np.inf
        p = softmax_t(row, temperature)
        accepted = None
        R = np.float32(1.0)
        rejected: List[int] = []
        for c in children[node]:
            q0 = np.asarray(q_rows[q_row_of[node]], np.float32)
            q = q0
            if without_replacement:
                q = (q0 / R).astype(np.float32) if R > 0 else np.zeros_like(q0)
                q[rejected] = 0.0
            tok = tree.token_at(c)
            u = uniforms[used]
            used += 1
            if rejection_step(float(q[tok]), float(p[tok]), u):
                accepted = c
                break
            p = adjusted_distribution(p, q)
            rejected.append(tok)
            R = np.float32(R - q0[tok])
        if accepted is not None:
            path.append(accepted)
            node = accepted
            continue
        tok = sample_u(p, uniforms[used])
        used += 1
        return path, tok, used


def d2t_maps(d2t: Sequence[int], target_vocab: int):
    """eagle3.rs:386-397 -> (target_to_draft dict, t2d mask)."""
    t2d = np.zeros(target_vocab, bool)
    inv = {}
    for di, ti in enumerate(d2t):
        if ti >= 0 and ti < target_vocab:
            inv[int(ti)] = di
            t2d[int(ti)] = True
    return inv, t2d


# ---------------------------------------------------------------------------
# Decoder state machine (quantized_llama.rs)
# ---------------------------------------------------------------------------
class SamplingError(Exception):
    pass


class RollbackError(Exception):
    pass


class OracleDecoder:
    """LlamaQuantDecoder's contract over OracleModel."""

    def __init__(self, model: OracleModel):
        self.m = model
        self.history: List[int] = []
        self.cache_len = 0
        self.last_logits: Optional[np.ndarray] = None

    def reset(self):
        self.history = []
        self.m.clear_kv_cache()
        self.cache_len = 0
        self.last_logits = None

    def _forward_advance(self, tokens: Sequence[int]) -> np.ndarray:
        if len(tokens) == 0:
            raise SamplingError("forward_advance with empty tokens")
        M = len(tokens)
        P = self.cache_len
        mask = causal_mask(P, M)
        hidden, _ = self.m.forward(tokens, list(range(P, P + M)), mask)
        logits = self.m.lm_head(hidden)
        self.cache_len += M
        self.last_logits = logits[-1].copy()
        self._last_hidden = hidden
        return logits

    def observe(self, ids: Sequence[int]):
        if len(ids) == 0:
            return
        self._forward_advance(ids)
        self.history += list(ids)

    def next_logits(self) -> np.ndarray:
        if not self.history:
            raise SamplingError("next_logits called with empty history")
        if self.last_logits is not None:
            return self.last_logits.copy()
        last = self.history[-1]
        t = len(self.history) - 1
        self.m.truncate_kv_cache_to(t)
        self.cache_len = t
        return self._forward_advance([last])[-1].copy()

    def batched_logits(self, drafts: Sequence[int]) -> np.ndarray:
        if len(drafts) == 0:
            return self.next_logits()[None, :]
        if not self.history:
            raise SamplingError("batched_logits with empty history")
        last = self.history[-1]
        t = len(self.history) - 1
        self.m.truncate_kv_cache_to(t)
        self.cache_len = t
        logits = self._forward_advance([last] + list(drafts))
        self.history += list(drafts)
        return logits

    def rollback_to(self, n: int):
        if n > len(self.history):
            raise RollbackError(f"rollback target {n} > history length {len(self.history)}")
        self.history = self.history[:n]
        self.last_logits = None
        self.m.truncate_kv_cache_to(n)
        self.cache_len = n

    def _tree_forward(self, tree: DraftTree):
        last = self.history[-1]
        if tree.token_at(0) != last:
            raise SamplingError(f"tree root ({tree.token_at(0)}) must equal last committed token ({last})")
        prefix = self.cache_len - 1
        self.m.truncate_kv_cache_to(prefix)
        self.cache_len = prefix
        n = len(tree)
        mask = np.ones((n, prefix + n), bool)
        am = tree.attention_mask_bool()
        mask[:, prefix:] = np.asarray(am, bool)
        hidden, _ = self.m.forward(tree.tokens(), tree.position_ids(prefix), mask)
        logits = self.m.lm_head(hidden)
        return prefix, hidden, logits

    def tree_logits_keep_kv(self, tree: DraftTree):
        self.last_logits = None
        if not self.history:
            raise SamplingError("tree_logits with empty history")
        prefix, hidden, logits = self._tree_forward(tree)
        self.cache_len = prefix + len(tree)
        return logits, hidden

    def tree_logits(self, tree: DraftTree) -> np.ndarray:
        """Strict tree verify: tree pass, cache restored to P, then a one-token
        pass of the root (which also refreshes last_logits).

        Llama (quantized_llama.rs:262-325): row 0 is replaced by the restoring
        pass's row. Qwen2 (quantized_qwen2.rs:184-237): the restoring pass's
        row is discarded and row 0 stays the tree pass's row.
        """
        if not self.history:
            raise SamplingError("tree_logits with empty history")
        last = self.history[-1]
        prefix, _, logits = self._tree_forward(tree)
        logits = logits.copy()
        self.m.truncate_kv_cache_to(prefix)
        self.cache_len = prefix
        restore = self._forward_advance([last])
        if self.m.cfg.arch == "llama":
            logits[0] = restore[-1]
        return logits

    def commit_tree_path(self, tree: DraftTree, accepted: Sequence[int]):
        self.last_logits = None
        if not self.history:
            raise SamplingError("commit_tree_path with empty history")
        prefix = len(self.history) - 1
        keep = list(range(prefix)) + [prefix + ti for ti in accepted]
        self.m.keep_kv_indices(keep)
        self.cache_len = len(keep)
        for ti in accepted[1:]:
            self.history.append(tree.token_at(ti))
