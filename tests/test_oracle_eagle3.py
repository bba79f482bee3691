"""The EAGLE-3 draft oracle (oracle/eagle3.py), pinned by the reference's own
known answers (eagle3.rs:799-833, medusa.rs:846-858) and by what the
mathematics fixes: RoPE at position 0 is the identity and a unit vector
rotates by (cos, sin) into its half partner, one cached key gives back its
value, head h reads kv head h // n_rep, zero projections leave the
residual path alone, fc runs only on the 3 * hidden input, and the
log-probs are a normalised log-softmax."""
import numpy as np
import pytest
from scipy.special import logsumexp

import eagle3 as E

SMALL = E.Eagle3Config(hidden=64, n_heads=4, n_kv_heads=2, ffn=96, draft_vocab=50, target_vocab=80,
                       rope_theta=10000.0, max_pos=64)


def _tensors(c, seed=0, std=0.1):
    rng = np.random.default_rng(seed)
    t = {}
    for k, shp in E.shapes(c).items():
        t[k] = (1.0 + 0.1 * rng.standard_normal(shp)) if len(shp) == 1 else std * rng.standard_normal(shp)
    return {k: E.f16(v) for k, v in t.items()}


def test_config_defaults_and_layers():
    c = E.Eagle3Config()
    assert (c.hidden, c.draft_vocab, c.target_vocab, c.head_dim) == (4096, 32000, 128256, 128)
    assert E.default_layers_for(32) == [1, 15, 28]
    assert E.default_layers_for(3) == [0, 0, 0]


def test_top_k_tie_break_and_clamp():
    assert E.top_k_indices(np.array([0.1, 0.5, 0.5, 0.3, 0.5], np.float32), 3) == [1, 2, 4]
    assert E.top_k_indices(np.array([0.5, 0.4], np.float32), 100) == [0, 1]


def test_rope_tables_and_rotation():
    c = SMALL
    cos, sin = E.rope_tables(c)
    hd, h = c.head_dim, c.head_dim // 2
    assert np.all(cos[0] == 1) and np.all(sin[0] == 0)
    # inv_freq_0 = 1: column 0 holds cos / sin of the (f16) position itself
    pos = np.arange(c.max_pos)
    assert np.allclose(cos[:, 0], np.cos(E.f16(pos)), atol=1e-3)
    assert np.allclose(sin[:, 0], np.sin(E.f16(pos)), atol=1e-3)
    x = E.f16(np.random.default_rng(1).standard_normal((3, hd)))
    assert np.array_equal(E.rope_half(x, cos[0], sin[0]), x)
    # half rotation: e_j -> cos e_j + sin e_{j + hd/2}; e_{j + hd/2} -> -sin e_j + cos e_{j + hd/2}
    p, j = 7, 3
    e = np.zeros((2, hd), np.float32)
    e[0, j] = 1
    e[1, j + h] = 1
    y = E.rope_half(e, cos[p], sin[p])
    assert y[0, j] == cos[p, j] and y[0, j + h] == sin[p, j]
    assert y[1, j] == -sin[p, j] and y[1, j + h] == cos[p, j]
    assert np.count_nonzero(y) == 4
    # a rotation: pair norms kept to f16 precision
    y = E.rope_half(x, cos[p], sin[p])
    n0 = x[:, :h] ** 2 + x[:, h:] ** 2
    n1 = y[:, :h] ** 2 + y[:, h:] ** 2
    assert np.allclose(n0, n1, rtol=5e-3, atol=1e-3)


def test_attention_one_key_returns_value_and_gqa_mapping():
    rng = np.random.default_rng(2)
    nh, nkv, hd = 4, 2, 8
    q = E.f16(rng.standard_normal((nh, hd)))
    K1 = E.f16(rng.standard_normal((nkv, 1, hd)))
    V1 = E.f16(rng.standard_normal((nkv, 1, hd)))
    y = E.attend(q, K1, V1)
    for hh in range(nh):
        assert np.array_equal(y[hh], V1[hh // 2, 0])
    # equal keys: the mean of the values
    K = np.repeat(K1, 3, axis=1)
    V = E.f16(rng.standard_normal((nkv, 3, hd)))
    y = E.attend(q, K, V)
    for hh in range(nh):
        assert np.allclose(y[hh], V[hh // 2].mean(0), atol=2e-3)
    # against the f64 softmax
    K = E.f16(rng.standard_normal((nkv, 5, hd)))
    y = E.attend(q, K, V := E.f16(rng.standard_normal((nkv, 5, hd))))
    for hh in range(nh):
        s = K[hh // 2].astype(np.float64) @ q[hh] / np.sqrt(hd)
        pr = np.exp(s - s.max())
        pr /= pr.sum()
        assert np.allclose(y[hh], pr @ V[hh // 2], atol=1e-2)


def test_zero_projections_keep_the_residual_path():
    c = SMALL
    t = _tensors(c)
    for k in (E.Q, E.K, E.V, E.O, E.GATE, E.UP, E.DOWN):
        t[k] = np.zeros_like(t[k])
    o = E.Eagle3Oracle(c, t)
    rng = np.random.default_rng(3)
    proj = E.f16(rng.standard_normal(c.hidden))
    emb = E.f16(rng.standard_normal(c.hidden))
    # attention and MLP add zero: out = projected (not the embedding)
    assert np.array_equal(o.forward_hidden(proj, emb, 5), proj)
    # a nonzero MLP alone: out = down(silu(gate xn) * up xn) + projected, xn = norm(projected)
    t2 = dict(t)
    t2[E.GATE] = _tensors(c, 4)[E.GATE]
    t2[E.UP] = _tensors(c, 5)[E.UP]
    t2[E.DOWN] = _tensors(c, 6)[E.DOWN]
    o2 = E.Eagle3Oracle(c, t2)
    xn = proj.astype(np.float64) / np.sqrt(np.mean(proj.astype(np.float64) ** 2) + c.rms_eps) * t2[E.POST_NORM]
    g = t2[E.GATE] @ xn
    u = t2[E.UP] @ xn
    ref = t2[E.DOWN] @ (g / (1 + np.exp(-g)) * u) + proj
    got = o2.forward_hidden(proj, emb, 5)
    assert np.allclose(got, ref, rtol=2e-2, atol=2e-2 * np.abs(ref).max())


def test_fc_only_on_the_concatenated_input():
    c = SMALL
    t = _tensors(c)
    rng = np.random.default_rng(7)
    emb = E.f16(rng.standard_normal(c.hidden))
    h3 = E.f16(rng.standard_normal(3 * c.hidden))
    a = E.Eagle3Oracle(c, t).forward_hidden(h3, emb, 0)
    b = E.Eagle3Oracle(c, t).forward_hidden(E.linear(t[E.FC], h3[None])[0], emb, 0)
    assert np.array_equal(a, b)
    bad = dict(t)
    bad[E.FC] = np.full_like(t[E.FC], np.nan)
    h1 = E.f16(rng.standard_normal(c.hidden))
    assert np.all(np.isfinite(E.Eagle3Oracle(c, bad).forward_hidden(h1, emb, 0)))


def test_draft_cache_grows_per_step_and_resets():
    c = SMALL
    o = E.Eagle3Oracle(c, _tensors(c))
    rng = np.random.default_rng(8)
    h = E.f16(rng.standard_normal(3 * c.hidden))
    emb = E.f16(rng.standard_normal(c.hidden))
    out0 = o.forward_hidden(h, emb, 4)
    o.forward_hidden(out0, emb, 5)
    assert len(o.kc) == 2
    o.reset()
    assert np.array_equal(o.forward_hidden(h, emb, 4), out0)


def test_log_probs_are_a_log_softmax():
    rng = np.random.default_rng(9)
    l = (rng.standard_normal(500) * 4).astype(np.float32)
    lp = np.array(E.log_probs(l, range(500)), np.float64)
    assert abs(np.exp(lp).sum() - 1) < 1e-4
    assert np.allclose(lp, l - logsumexp(l.astype(np.float64)), atol=1e-4)


def test_round_feeds_top1_and_previous_output():
    c = SMALL
    t = _tensors(c)
    rng = np.random.default_rng(10)
    table = E.f16(rng.standard_normal((c.target_vocab, c.hidden)))
    d2t = rng.permutation(c.target_vocab)[:c.draft_vocab]
    h3 = E.f16(rng.standard_normal(3 * c.hidden))
    ids, lps, logits = E.Eagle3Oracle(c, t).round(h3, lambda i: table[i], 11, 20, 3, 4, d2t)
    assert [len(s) for s in ids] == [4, 4, 4]
    # step by step by hand
    o = E.Eagle3Oracle(c, t)
    out = o.forward_hidden(h3, table[11], 20)
    assert np.array_equal(o.norm_lm_head(out), logits[0])
    out = o.forward_hidden(out, table[ids[0][0]], 21)
    assert np.array_equal(o.norm_lm_head(out), logits[1])
    for s in range(3):
        assert ids[s] == [int(d2t[i]) for i in E.top_k_indices(logits[s], 4)]
        assert all(lps[s][i] >= lps[s][i + 1] for i in range(3))
