"""Shared model builders for the tests (oracle and HIP twins of one config)."""
from __future__ import annotations

import numpy as np

import oracle as O

# The tiny random-init Llama decoder: 4 layers, hidden 512, 8/8 heads, head_dim 64,
# SwiGLU FFN 1536, vocab 32000, RoPE theta 10000, Q4_K.
TINY = dict(arch="llama", n_layers=4, hidden=512, n_heads=8, n_kv_heads=8, head_dim=64, ffn=1536,
            vocab=32000, rope_theta=10000.0, rms_eps=1e-5, ctx_len=1024, mix="q4_k", seed=0x5EED0001)

MIX_IDS = {"q4_k": 0, "q4_k_m": 1, "q5k_q80": 2, "q6_k": 3, "q5_k": 4, "q8_0": 5}


def oracle_cfg(**over) -> O.ModelConfig:
    d = dict(TINY)
    d.update(over)
    return O.ModelConfig(**d)


def hip_cfg(hip, ocfg: O.ModelConfig, max_batch: int = 128):
    return hip.Config(arch=0 if ocfg.arch == "llama" else 1, n_layers=ocfg.n_layers, hidden=ocfg.hidden,
                      n_heads=ocfg.n_heads, n_kv_heads=ocfg.n_kv_heads, head_dim=ocfg.head_dim, ffn=ocfg.ffn,
                      vocab=ocfg.vocab, rope_theta=ocfg.rope_theta, rms_eps=ocfg.rms_eps, ctx_len=ocfg.ctx_len,
                      max_batch=max_batch, tied_output=int(ocfg.tied_output))


def fmt_of_mix(mix: str, layer: int, kind: int, n_layers: int) -> int:
    return O.ModelConfig(mix=mix, n_layers=n_layers).fmt(layer, kind)


def all_tensor_keys(cfg: O.ModelConfig):
    keys = [(-1, O.K_TOK_EMBD), (-1, O.K_OUTPUT_NORM)] + ([] if cfg.tied_output else [(-1, O.K_OUTPUT)])
    for li in range(cfg.n_layers):
        keys += [(li, k) for k in cfg.layer_kinds()]
    return keys


def rel_err(a: np.ndarray, b: np.ndarray) -> float:
    """max |a-b| / max |b| (per-array relative error used for logits)."""
    return float(np.max(np.abs(a.astype(np.float64) - b)) / max(np.max(np.abs(b)), 1e-30))
