"""EAGLE-3 draft side -- TEST INFRASTRUCTURE ONLY (tests/ use it as the
checker of the device draft; the product never imports it).

A numpy restatement of the reference's EAGLE-3 draft
(crates/speculate/src/methods/eagle3.rs):
  * Midlayer::forward (:196-299): th = input_layernorm(input_emb),
    pf = hidden_norm(projected), combined = [th, pf] (2 * hidden);
    q/k/v = combined . W^T; RoPE with half rotation
    (candle_nn::rotary_emb::rope) at `position`; K/V appended to the draft's
    own cache (cleared each round, :628); softmax(q k^T * 1/sqrt(hd)) v
    over every cached step (GQA through repeat_kv); o_proj + projected
    (the pre-norm input); post_attention_layernorm; SiLU(gate) * up; down;
    + the attention output;
  * the RoPE tables of Midlayer::load (:153-182): inv_freq_j =
    1 / theta^(2j / hd) in f32, then t (0 .. max_pos) and inv_freq cast to
    the draft's dtype, freqs = t . inv_freq in that dtype, cos / sin of it;
  * forward_hidden (:433-450): fc (3 * hidden -> hidden) only when the input
    is the concat of the three target layers' hidden states;
  * apply_norm_lm_head (:451-454): lm_head(norm(hidden));
  * one round of run_eagle3 (:598-673): hidden_in = [low, mid, high] of the
    committed token, input_emb = the target's embedding of the current token,
    per step top_k_indices of the draft logits (medusa.rs:477-487: value
    descending, index ascending on ties), log-probs l_i - lse with
    lse = ln(sum exp(l - max)) + max in sequential f32, d2t to target ids, and
    the top-1 target id plus this step's midlayer output feed the next step.

The draft's tensors are f16 (the reference runs the draft in F16): every
candle op takes f16 tensors and rounds its result to f16; matmuls and
reductions accumulate in f32 (here f64 for the products, then rounded), and
the RoPE formula y1 = x1 c - x2 s, y2 = x1 s + x2 c rounds after every
multiply and add as f16 arithmetic does.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, List, Sequence, Tuple

import numpy as np


def f16(x) -> np.ndarray:
    """round to f16, back as f32"""
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)


@dataclass
class Eagle3Config:
    hidden: int = 4096
    n_heads: int = 32
    n_kv_heads: int = 8
    ffn: int = 14336
    draft_vocab: int = 32000
    target_vocab: int = 128256
    rms_eps: float = 1e-5
    rope_theta: float = 500000.0
    max_pos: int = 2048

    @property
    def head_dim(self) -> int:
        return self.hidden // self.n_heads


# tensor names of the checkpoint (eagle3.rs:133-150, 363-386)
FC, Q, K, V, O, GATE, UP, DOWN, LM_HEAD, IN_NORM, HID_NORM, POST_NORM, NORM = range(13)


def shapes(c: Eagle3Config) -> Dict[int, Tuple[int, ...]]:
    H, hd = c.hidden, c.head_dim
    return {FC: (H, 3 * H), Q: (c.n_heads * hd, 2 * H), K: (c.n_kv_heads * hd, 2 * H), V: (c.n_kv_heads * hd, 2 * H),
            O: (H, c.n_heads * hd), GATE: (c.ffn, H), UP: (c.ffn, H), DOWN: (H, c.ffn), LM_HEAD: (c.draft_vocab, H),
            IN_NORM: (H,), HID_NORM: (H,), POST_NORM: (H,), NORM: (H,)}


def rope_tables(c: Eagle3Config) -> Tuple[np.ndarray, np.ndarray]:
    hd = c.head_dim
    inv = (1.0 / np.power(np.float32(c.rope_theta), np.arange(0, hd, 2, dtype=np.float32) / np.float32(hd)))
    inv = f16(inv.astype(np.float32))
    t = f16(np.arange(c.max_pos, dtype=np.float32))
    freqs = f16(t[:, None].astype(np.float64) * inv[None, :].astype(np.float64))
    return f16(np.cos(freqs)), f16(np.sin(freqs))


def linear(W: np.ndarray, x: np.ndarray) -> np.ndarray:
    """x [n][in] . W [out][in]^T, f32 accumulation, f16 result"""
    return f16(np.asarray(x, np.float64) @ np.asarray(W, np.float64).T)


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x32 = np.asarray(x, np.float32)
    ms = np.mean(x32.astype(np.float64) ** 2, axis=-1, keepdims=True)
    return f16(x32 / np.sqrt(ms + eps).astype(np.float32) * np.asarray(w, np.float32))


def rope_half(x: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """x [heads][hd] at one position; cos / sin [hd/2]; f16 arithmetic"""
    h = x.shape[-1] // 2
    x1, x2 = x[..., :h], x[..., h:]
    y1 = f16(f16(x1 * cos) - f16(x2 * sin))
    y2 = f16(f16(x1 * sin) + f16(x2 * cos))
    return np.concatenate([y1, y2], axis=-1)


def default_layers_for(n_layers: int) -> List[int]:
    """eagle3.rs:540-546: [1, n/2 - 1, n - 4], [0, 0, 0] below 4 layers"""
    return [0, 0, 0] if n_layers < 4 else [1, n_layers // 2 - 1, n_layers - 4]


def top_k_indices(logits: np.ndarray, k: int) -> List[int]:
    """medusa.rs:477-487: value descending, index ascending on ties"""
    order = sorted(range(len(logits)), key=lambda i: (-float(logits[i]), i))
    return order[:min(k, len(logits))]


def log_probs(logits: np.ndarray, idx: Sequence[int]) -> List[float]:
    """eagle3.rs:659-661: l_i - (ln(sum exp(l - max)) + max), sequential f32"""
    l32 = np.asarray(logits, np.float32)
    mx = np.float32(-np.inf)
    for v in l32:
        mx = np.float32(max(mx, v)) if not np.isnan(v) else mx
    s = np.float32(0.0)
    for v in l32:
        s = np.float32(s + np.float32(np.exp(np.float32(v - mx))))
    lse = np.float32(np.float32(np.log(s)) + mx)
    return [float(np.float32(l32[i] - lse)) for i in idx]


def attend(q: np.ndarray, Kc: np.ndarray, Vc: np.ndarray) -> np.ndarray:
    """q [n_heads][hd], Kc / Vc [n_kv][T][hd] -> [n_heads][hd]: softmax(q k^T *
    1/sqrt(hd)) v per head, head h reading kv head h // (n_heads / n_kv)
    (candle_transformers::utils::repeat_kv repeats each kv head n_rep times in
    a row), f16 scores, probabilities and outputs (eagle3.rs:260-284)"""
    nh, hd = q.shape
    rep = nh // Kc.shape[0]
    scale = 1.0 / np.sqrt(hd)
    y = np.empty((nh, hd), np.float32)
    for h in range(nh):
        s = f16(Kc[h // rep].astype(np.float64) @ q[h].astype(np.float64))
        s = f16(s * np.float32(scale))
        e = np.exp((s - s.max()).astype(np.float32))
        p = f16(e / e.sum(dtype=np.float32))
        y[h] = f16(p.astype(np.float64) @ Vc[h // rep].astype(np.float64))
    return y


class Eagle3Oracle:
    def __init__(self, cfg: Eagle3Config, tensors: Dict[int, np.ndarray]):
        self.c = cfg
        self.t = {k: f16(v) for k, v in tensors.items()}
        self.cos, self.sin = rope_tables(cfg)
        self.reset()

    def reset(self):
        self.kc: List[np.ndarray] = []  # per step [n_kv][hd]
        self.vc: List[np.ndarray] = []

    def midlayer(self, input_emb: np.ndarray, projected: np.ndarray, position: int) -> np.ndarray:
        c, t = self.c, self.t
        hd, nh, nkv = c.head_dim, c.n_heads, c.n_kv_heads
        th = rmsnorm(input_emb, t[IN_NORM], c.rms_eps)
        pf = rmsnorm(projected, t[HID_NORM], c.rms_eps)
        comb = np.concatenate([th, pf])
        q = linear(t[Q], comb[None])[0].reshape(nh, hd)
        k = linear(t[K], comb[None])[0].reshape(nkv, hd)
        v = linear(t[V], comb[None])[0].reshape(nkv, hd)
        q = rope_half(q, self.cos[position], self.sin[position])
        k = rope_half(k, self.cos[position], self.sin[position])
        self.kc.append(k)
        self.vc.append(v)
        y = attend(q, np.stack(self.kc, axis=1), np.stack(self.vc, axis=1))
        attn_out = linear(t[O], y.reshape(1, -1))[0]
        after = f16(attn_out + projected)
        xn = rmsnorm(after, t[POST_NORM], c.rms_eps)
        g = linear(t[GATE], xn[None])[0]
        u = linear(t[UP], xn[None])[0]
        act = f16(f16(g / (1.0 + np.exp(-g.astype(np.float32)))) * u)
        m = linear(t[DOWN], act[None])[0]
        return f16(m + after)

    def forward_hidden(self, hidden_in: np.ndarray, input_emb: np.ndarray, position: int) -> np.ndarray:
        h = f16(hidden_in)
        projected = linear(self.t[FC], h[None])[0] if h.size == 3 * self.c.hidden else h
        return self.midlayer(f16(input_emb), projected, position)

    def norm_lm_head(self, hidden: np.ndarray) -> np.ndarray:
        return linear(self.t[LM_HEAD], rmsnorm(hidden, self.t[NORM], self.c.rms_eps)[None])[0]

    def round(self, hidden3: np.ndarray, embed, root_token: int, history_len: int, depth: int, top_k: int,
              d2t: np.ndarray):
        """-> (per-step top-k target ids, per-step log-probs, per-step logits)"""
        self.reset()
        hidden_in = hidden3
        cur = root_token
        ids, lps, logits_all = [], [], []
        for step in range(depth):
            out = self.forward_hidden(hidden_in, embed(cur), history_len + step)
            logits = self.norm_lm_head(out)
            idx = top_k_indices(logits, top_k)
            ids.append([int(d2t[i]) for i in idx])
            lps.append(log_probs(logits, idx))
            logits_all.append(logits)
            hidden_in = out
            cur = ids[-1][0]
        return ids, lps, logits_all
