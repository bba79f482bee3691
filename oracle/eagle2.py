"""EAGLE-2 draft side -- TEST INFRASTRUCTURE ONLY (tests/ use it as the
checker of the device draft; the product never imports it).

A numpy restatement of the reference's EAGLE draft
(crates/speculate/src/methods/eagle.rs):
  * EagleDraftCandle::forward (:390-427) of one position:
    combined = [f16(target_hidden), embed_tokens(token)] (2 * hidden),
    xs = fc(combined); one Llama block without an input norm: q/k/v = xs . W^T,
    RoPE with half rotation (candle_nn::rotary_emb::rope) at `position`, K/V
    appended to the draft's own cache (cleared each round, :531), softmax(q
    k^T / sqrt(hd)) v over every cached step (GQA through repeat_kv),
    o_proj, + xs; post_attention_layernorm; SiLU(gate) * up; down; + the
    attention output;
  * the RoPE tables of DraftAttention::load (:134-157), as Midlayer::load's
    (oracle/eagle3.py rope_tables);
  * one round of run_eagle (:519-575): from the committed token's final-norm
    hidden state and its id, `depth` steps, each the draft forward, the
    target's lm_head on its output (apply_lm_head), top_k_indices (value
    descending, index ascending) with log-probs l - lse (sequential f32); the
    top-1 id and the step's output feed the next step.

The draft's tensors are f16: every op rounds its result to f16 (see
oracle/eagle3.py for the conventions).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, Dict, List, Tuple

import numpy as np

from eagle3 import Eagle3Config, attend, f16, linear, log_probs, rmsnorm, rope_half, rope_tables, top_k_indices


@dataclass
class Eagle2Config:
    hidden: int = 4096
    n_heads: int = 32
    n_kv_heads: int = 8
    ffn: int = 14336
    vocab: int = 128256
    rms_eps: float = 1e-5
    rope_theta: float = 500000.0
    max_pos: int = 2048

    @property
    def head_dim(self) -> int:
        return self.hidden // self.n_heads


# tensor names of the checkpoint (eagle.rs:126-131, 279-286, 349-361)
EMBED, FC, Q, K, V, O, GATE, UP, DOWN, POST_NORM = range(10)


def shapes(c: Eagle2Config) -> Dict[int, Tuple[int, ...]]:
    H, hd = c.hidden, c.head_dim
    return {EMBED: (c.vocab, H), FC: (H, 2 * H), Q: (c.n_heads * hd, H), K: (c.n_kv_heads * hd, H),
            V: (c.n_kv_heads * hd, H), O: (H, c.n_heads * hd), GATE: (c.ffn, H), UP: (c.ffn, H), DOWN: (H, c.ffn),
            POST_NORM: (H,)}


class Eagle2Oracle:
    def __init__(self, cfg: Eagle2Config, tensors: Dict[int, np.ndarray]):
        self.c = cfg
        self.t = {k: f16(v) for k, v in tensors.items()}
        self.cos, self.sin = rope_tables(Eagle3Config(hidden=cfg.hidden, n_heads=cfg.n_heads,
                                                      rope_theta=cfg.rope_theta, max_pos=cfg.max_pos))
        self.reset()

    def reset(self):
        self.kc: List[np.ndarray] = []
        self.vc: List[np.ndarray] = []

    def forward(self, target_hidden: np.ndarray, token: int, position: int) -> np.ndarray:
        c, t = self.c, self.t
        hd, nh, nkv = c.head_dim, c.n_heads, c.n_kv_heads
        comb = np.concatenate([f16(target_hidden), t[EMBED][token]])
        xs = linear(t[FC], comb[None])[0]
        q = linear(t[Q], xs[None])[0].reshape(nh, hd)
        k = linear(t[K], xs[None])[0].reshape(nkv, hd)
        v = linear(t[V], xs[None])[0].reshape(nkv, hd)
        q = rope_half(q, self.cos[position], self.sin[position])
        k = rope_half(k, self.cos[position], self.sin[position])
        self.kc.append(k)
        self.vc.append(v)
        y = attend(q, np.stack(self.kc, axis=1), np.stack(self.vc, axis=1))
        after = f16(linear(t[O], y.reshape(1, -1))[0] + xs)
        xn = rmsnorm(after, t[POST_NORM], c.rms_eps)
        g = linear(t[GATE], xn[None])[0]
        u = linear(t[UP], xn[None])[0]
        act = f16(f16(g / (1.0 + np.exp(-g.astype(np.float32)))) * u)
        return f16(linear(t[DOWN], act[None])[0] + after)

    def round(self, target_hidden: np.ndarray, lm_head: Callable[[np.ndarray], np.ndarray], root_token: int,
              history_len: int, depth: int, top_k: int):
        """-> (per-step top-k ids, per-step log-probs, per-step logits)"""
        self.reset()
        h, cur = target_hidden, root_token
        ids, lps, logits_all = [], [], []
        for step in range(depth):
            out = self.forward(h, cur, history_len + step)
            logits = np.asarray(lm_head(out), np.float32)
            idx = top_k_indices(logits, top_k)
            ids.append(idx)
            lps.append(log_probs(logits, idx))
            logits_all.append(logits)
            h, cur = out, idx[0]
        return ids, lps, logits_all
