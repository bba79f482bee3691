"""The EAGLE-2 draft oracle (oracle/eagle2.py), pinned by the reference's
known answers (eagle.rs:862-871 config defaults) and by what the mathematics
fixes: no input norm (with the block's projections zero the output is fc's),
fc reads [target hidden, token embedding] in that order, the attention
output is added to fc's output, the cache grows per step and resets, and a
round feeds the top-1 id and the step's output on."""
import numpy as np

import eagle2 as E2
import eagle3 as E3

SMALL = E2.Eagle2Config(hidden=64, n_heads=4, n_kv_heads=2, ffn=96, vocab=80, rope_theta=10000.0, max_pos=64)


def _tensors(c, seed=0, std=0.1):
    rng = np.random.default_rng(seed)
    t = {}
    for k, shp in E2.shapes(c).items():
        t[k] = (1.0 + 0.1 * rng.standard_normal(shp)) if len(shp) == 1 else std * rng.standard_normal(shp)
    return {k: E3.f16(v) for k, v in t.items()}


def test_config_defaults():
    c = E2.Eagle2Config()
    assert (c.hidden, c.vocab, c.n_heads, c.n_kv_heads, c.ffn, c.rope_theta) == (4096, 128256, 32, 8, 14336, 500000.0)
    assert c.head_dim == 128


def test_zero_block_gives_fc_of_hidden_then_embedding():
    c = SMALL
    t = _tensors(c)
    for k in (E2.Q, E2.K, E2.V, E2.O, E2.GATE, E2.UP, E2.DOWN):
        t[k] = np.zeros_like(t[k])
    H = c.hidden
    # fc = [I | 0]: the output is the target hidden (rounded to f16), unnormalised
    fc = np.zeros((H, 2 * H), np.float32)
    fc[:, :H] = np.eye(H)
    t[E2.FC] = fc
    h = E3.f16(np.random.default_rng(1).standard_normal(H) * 3)
    o = E2.Eagle2Oracle(c, t)
    assert np.array_equal(o.forward(h, 5, 0), h)
    # fc = [0 | I]: the embedding row of the token
    fc[:] = 0
    fc[:, H:] = np.eye(H)
    t[E2.FC] = fc
    o = E2.Eagle2Oracle(c, t)
    assert np.array_equal(o.forward(h, 7, 3), t[E2.EMBED][7])


def test_attention_output_adds_to_fc_output():
    c = SMALL
    t = _tensors(c)
    for k in (E2.GATE, E2.UP, E2.DOWN, E2.Q, E2.K):
        t[k] = np.zeros_like(t[k])
    H = c.hidden
    rng = np.random.default_rng(2)
    h = E3.f16(rng.standard_normal(H))
    o = E2.Eagle2Oracle(c, t)
    got = o.forward(h, 3, 9)
    # one cached step: attention returns v; out = o_proj(v) + xs
    xs = t[E2.FC].astype(np.float64) @ np.concatenate([h, t[E2.EMBED][3]]).astype(np.float64)
    v = (t[E2.V].astype(np.float64) @ xs).reshape(c.n_kv_heads, -1)
    rep = c.n_heads // c.n_kv_heads
    y = np.concatenate([v[hh // rep] for hh in range(c.n_heads)])
    ref = t[E2.O].astype(np.float64) @ y + xs
    assert np.allclose(got, ref, rtol=1e-2, atol=1e-2 * np.abs(ref).max())


def test_cache_and_round_feed():
    c = SMALL
    t = _tensors(c)
    rng = np.random.default_rng(3)
    h = E3.f16(rng.standard_normal(c.hidden))
    lm = E3.f16(rng.standard_normal((c.vocab, c.hidden)) * 0.2)
    head = lambda x: (lm.astype(np.float64) @ x.astype(np.float64)).astype(np.float32)
    ids, lps, logits = E2.Eagle2Oracle(c, t).round(h, head, 11, 20, 3, 4)
    o = E2.Eagle2Oracle(c, t)
    out = o.forward(h, 11, 20)
    assert np.array_equal(head(out), logits[0])
    out = o.forward(out, ids[0][0], 21)
    assert np.array_equal(head(out), logits[1])
    assert len(o.kc) == 2
    for s in range(3):
        assert ids[s] == E3.top_k_indices(logits[s], 4)
        assert abs(np.exp(np.array(E3.log_probs(logits[s], range(c.vocab)), np.float64)).sum() - 1) < 1e-4
    o.reset()
    assert np.array_equal(o.forward(h, 11, 20), E2.Eagle2Oracle(c, t).forward(h, 11, 20))
