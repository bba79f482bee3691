"""CPU baseline of the verify step -- test and measurement infrastructure only.

Python side of oracle/cpu_q8k.c: the CPU algorithm candle runs for the
reference's quantised matmul (activations quantised per row to Q8_K, integer
block dot products scaled in f32, threads over output rows, AVX2), composed
into the layers of quantized_llama_local.rs:363-409 (RMSNorm -> Q/K/V ->
interleaved RoPE -> KV append -> attention -> wo + residual -> RMSNorm ->
gate/up -> SwiGLU -> down + residual) and the final RMSNorm + lm_head, so that a
bounded sample of whole layers can be timed on the host and scaled to one
verify step.  Only bench.py's cpu_baseline leg and tests/ use it.
"""
from __future__ import annotations

import ctypes
import os
import time

import numpy as np

import oracle as O

Q8K = np.dtype([("d", np.float32), ("qs", np.int8, 256), ("bsums", np.int16, 16)])
assert Q8K.itemsize == 292

_ready = False


def _lib():
    global _ready
    L = O.lib()
    if not _ready:
        P, i64 = ctypes.c_void_p, ctypes.c_int64
        L.or_quantize_row_q8k.argtypes = [P, i64, P]
        L.or_dot_q8k.argtypes = [ctypes.c_int, P, P, i64, ctypes.c_int]
        L.or_dot_q8k.restype = ctypes.c_float
        L.or_cpu_qmatmul_q8k.argtypes = [ctypes.c_int, P, i64, i64, P, i64, P, P, ctypes.c_int]
        L.or_cpu_qmatmul_q8k.restype = ctypes.c_int
        L.or_cpu_attention.argtypes = [P, P, P, i64, i64, ctypes.c_int, ctypes.c_int, ctypes.c_int, P]
        L.or_cpu_attention.restype = ctypes.c_int
        _ready = True
    return L


def quantize_q8k(x: np.ndarray) -> np.ndarray:
    """ggml's quantize_row_q8_K of one row (len a multiple of 256)."""
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(x.size // 256, Q8K)
    _lib().or_quantize_row_q8k(O._p(x), x.size, out.ctypes.data_as(ctypes.c_void_p))
    return out


def dot_q8k(fmt: int, wrow: np.ndarray, xq: np.ndarray, simd: bool = True) -> float:
    wrow = np.ascontiguousarray(wrow, np.uint8)
    return float(_lib().or_dot_q8k(fmt, O._p(wrow), xq.ctypes.data_as(ctypes.c_void_p), xq.size, 1 if simd else 0))


def qmatmul_q8k(fmt: int, raw: np.ndarray, N: int, K: int, x: np.ndarray, simd: bool = True,
                out: np.ndarray | None = None) -> np.ndarray:
    """y[m][n] = dot(W row n, Q8_K(x row m)), threads over n."""
    x = np.ascontiguousarray(x, np.float32)
    M = x.shape[0]
    y = np.empty((M, N), np.float32) if out is None else out
    xq = np.empty(M * (K // 256), Q8K)
    rc = _lib().or_cpu_qmatmul_q8k(fmt, O._p(raw), N, K, O._p(x), M, O._p(y), xq.ctypes.data_as(ctypes.c_void_p),
                                   1 if simd else 0)
    if rc:
        raise ValueError("unsupported format for the Q8_K path")
    return y


def attention(q: np.ndarray, kc: np.ndarray, vc: np.ndarray, P: int) -> np.ndarray:
    """q [M][n_heads][hd], kc/vc [n_kv][P + M][hd] -> [M][n_heads][hd]; query i
    sees keys < P + i + 1."""
    M, nh, hd = q.shape
    nkv = kc.shape[0]
    out = np.empty_like(q)
    _lib().or_cpu_attention(O._p(np.ascontiguousarray(q)), O._p(kc), O._p(vc), M, P, nh, nkv, hd, O._p(out))
    return out


def _rmsnorm(x, w, eps):
    return (x / np.sqrt(np.mean(x.astype(np.float32) ** 2, axis=-1, keepdims=True) + eps) * w).astype(np.float32)


def _rope_i(x, cos, sin):
    """interleaved pairs (2i, 2i+1), rope_i; x [M][heads][hd], cos/sin [M][hd/2]"""
    a, b = x[..., 0::2], x[..., 1::2]
    c, s = cos[:, None, :], sin[:, None, :]
    out = np.empty_like(x)
    out[..., 0::2] = a * c - b * s
    out[..., 1::2] = a * s + b * c
    return out


class CpuLayer:
    """One decoder layer's weights (GGUF blocks of the oracle's synthetic model)
    and an f32 KV cache of P rows, run for M new rows."""

    def __init__(self, cfg: "O.ModelConfig", layer: int, P: int, M: int, rng: np.random.Generator):
        self.cfg, self.P, self.M = cfg, P, M
        self.w = {}
        for kind in (O.K_ATTN_Q, O.K_ATTN_K, O.K_ATTN_V, O.K_ATTN_O, O.K_FFN_GATE, O.K_FFN_UP, O.K_FFN_DOWN):
            fmt, raw = O.synth_tensor(cfg, layer, kind)
            N, K = cfg.shape(kind)
            self.w[kind] = (fmt, np.ascontiguousarray(raw), N, K)
        H, hd = cfg.hidden, cfg.head_dim
        self.norm1 = np.ones(H, np.float32)
        self.norm2 = np.ones(H, np.float32)
        T = P + M
        self.kc = (rng.standard_normal((cfg.n_kv_heads, T, hd)) * 0.5).astype(np.float32)
        self.vc = (rng.standard_normal((cfg.n_kv_heads, T, hd)) * 0.5).astype(np.float32)
        ang = np.arange(P, T)[:, None] / (cfg.rope_theta ** (np.arange(0, hd, 2) / hd))[None, :]
        self.cos, self.sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)

    def _mm(self, kind, x):
        fmt, raw, N, K = self.w[kind]
        return qmatmul_q8k(fmt, raw, N, K, x)

    def forward(self, h: np.ndarray) -> np.ndarray:
        c, M, P = self.cfg, self.M, self.P
        hd = c.head_dim
        x = _rmsnorm(h, self.norm1, c.rms_eps)
        q = self._mm(O.K_ATTN_Q, x).reshape(M, c.n_heads, hd)
        k = self._mm(O.K_ATTN_K, x).reshape(M, c.n_kv_heads, hd)
        v = self._mm(O.K_ATTN_V, x).reshape(M, c.n_kv_heads, hd)
        q = _rope_i(q, self.cos, self.sin)
        k = _rope_i(k, self.cos, self.sin)
        self.kc[:, P:P + M] = k.transpose(1, 0, 2)
        self.vc[:, P:P + M] = v.transpose(1, 0, 2)
        a = attention(q, self.kc, self.vc, P).reshape(M, c.n_heads * hd)
        h = h + self._mm(O.K_ATTN_O, a)
        x = _rmsnorm(h, self.norm2, c.rms_eps)
        g = self._mm(O.K_FFN_GATE, x)
        u = self._mm(O.K_FFN_UP, x)
        act = (g / (1.0 + np.exp(-g)) * u).astype(np.float32)
        return (h + self._mm(O.K_FFN_DOWN, act)).astype(np.float32)


def time_step_sample(cfg: "O.ModelConfig", P: int, M: int, budget_s: float, log=print) -> dict:
    """Times whole layers (one with the Q6_K attn_v / ffn_down of the Q4_K_M
    mix, one all-Q4_K) and the final norm + lm_head for M rows at P cached
    positions, repeated for about budget_s seconds; returns per-part means and
    the scaled step time."""
    rng = np.random.default_rng(5)
    q6_layer = next(i for i in range(cfg.n_layers) if O.use_more_bits(i, cfg.n_layers))
    q4_layer = next(i for i in range(cfg.n_layers) if not O.use_more_bits(i, cfg.n_layers))
    L6, L4 = CpuLayer(cfg, q6_layer, P, M, rng), CpuLayer(cfg, q4_layer, P, M, rng)
    fmt, raw = O.synth_tensor(cfg, -1, O.K_OUTPUT)
    N, K = cfg.shape(O.K_OUTPUT)
    raw = np.ascontiguousarray(raw)
    h0 = (rng.standard_normal((M, cfg.hidden)) * 0.5).astype(np.float32)
    wn = np.ones(cfg.hidden, np.float32)
    t6 = t4 = tl = 0.0
    reps = 0
    t_start = time.perf_counter()
    while reps < 2 or time.perf_counter() - t_start < budget_s:
        t0 = time.perf_counter()
        h = L6.forward(h0)
        t1 = time.perf_counter()
        h = L4.forward(h)
        t2 = time.perf_counter()
        qmatmul_q8k(fmt, raw, N, K, _rmsnorm(h, wn, cfg.rms_eps))
        t3 = time.perf_counter()
        t6, t4, tl = t6 + t1 - t0, t4 + t2 - t1, tl + t3 - t2
        reps += 1
    t6, t4, tl = t6 / reps, t4 / reps, tl / reps
    n6 = sum(1 for i in range(cfg.n_layers) if O.use_more_bits(i, cfg.n_layers))
    step = n6 * t6 + (cfg.n_layers - n6) * t4 + tl
    return {"reps": reps, "q6_layer_s": t6, "q4_layer_s": t4, "lm_head_s": tl, "n_q6_layers": n6, "step_s": step}


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def threads() -> int:
    return int(os.environ.get("OMP_NUM_THREADS", "0")) or os.cpu_count() or 1
