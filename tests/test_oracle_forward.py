"""Pins of the oracle's forward (oracle.py: rope tables, rope_i / rope,
RMSNorm, SiLU, attention with its GQA head map, the pre-norm residual
structure) and of its decoder state machine, each by what the mathematics or
the reference's own tests fix -- never by retyping the oracle's formula:

* RoPE (quantized_llama_local.rs:94-105, 189-205; quantized_qwen2_local.rs:98-109):
  the table against theta_i = 1 / base^(2i/d) in f64, position 0 is the
  identity, each rotation keeps the norm of its pair, q.k depends only on the
  position difference, and a one-hot input tells the interleaved pairs
  (2i, 2i+1) of rope_i from the half pairs (i, i + d/2) of rope.
* RMSNorm (candle-nn's rms_norm, x / sqrt(mean(x^2) + eps) * w): known
  answers in which eps outside the square root, a sum instead of a mean or a
  missing weight would each give a different value.
* attention (quantized_llama_local.rs:107-136): one visible key returns its V
  row, equal scores the mean of the visible V rows, two keys the closed-form
  logistic weight of exp(delta / sqrt(hd)), masked keys have no influence,
  and query head h reads KV head h // n_rep (repeat_kv).
* the layer structure (quantized_llama_local.rs:363-409): with wo and
  ffn_down zero, every layer is the identity on the residual stream, so the
  final hidden is RMSNorm(embedding) exactly.
* the MLP roles (quantized_llama_local.rs:45-51): a one-feature known answer
  in which silu(gate) * up and silu(up) * gate differ; the roles exchanged
  (a planted mistake) fail it.
* the Qwen2 QKV bias (quantized_qwen2_local.rs:69-109), added before RoPE:
  with zero q/k weights the cached key and the attention weight at position 1
  are the rotated bias's closed forms; the bias added after the rotation (a
  planted mistake) fails it.
* the decoder (quantized_llama.rs; tests/with_qwen2_05b.rs:95-184,
  tests/tree_logits_consistency.rs:74-122): batched rows equal sequential
  observe rows, a linear tree equals the batched pass, tree row 0 equals
  next_logits, strict tree_logits restores the cache; on Qwen2
  (quantized_qwen2.rs:184-237) strict row 0 stays the tree pass's row.
"""
import math

import numpy as np
import pytest

import oracle as O
from _models import oracle_cfg


# ---- RoPE ------------------------------------------------------------------
@pytest.mark.parametrize("dim,base", [(64, 10000.0), (128, 500000.0), (128, 1e6)])
def test_rope_table_closed_form(dim, base):
    ctx = 4096
    c, s = O.rope_tables(dim, base, ctx)
    i = np.arange(dim // 2, dtype=np.float64)
    theta = 1.0 / base ** (2.0 * i / dim)
    t = np.arange(ctx, dtype=np.float64)[:, None]
    # f32 powf / product / cosf: the argument t*theta carries a relative error
    # of a few f32 ulps, i.e. an absolute error up to ~t * theta * 2^-22
    tol = 4e-7 + (t * theta) * 2.0 ** -21
    assert np.all(np.abs(c - np.cos(t * theta)) <= tol)
    assert np.all(np.abs(s - np.sin(t * theta)) <= tol)
    assert np.array_equal(c[0], np.ones(dim // 2, np.float32)) and np.array_equal(s[0], np.zeros(dim // 2, np.float32))


def _tables(dim, base=10000.0, ctx=256):
    return O.rope_tables(dim, base, ctx)


@pytest.mark.parametrize("rope", [O.rope_interleaved, O.rope_half])
def test_rope_position_zero_is_identity_and_norm_kept(rope):
    c, s = _tables(64)
    rng = np.random.default_rng(0)
    x = rng.standard_normal((3, 5, 64)).astype(np.float32)
    y0 = rope(x, c[[0] * 5], s[[0] * 5])
    assert np.array_equal(y0, x)
    pos = [1, 7, 31, 100, 255]
    y = rope(x, c[pos], s[pos])
    np.testing.assert_allclose(np.linalg.norm(y, axis=-1), np.linalg.norm(x, axis=-1), rtol=1e-6)


@pytest.mark.parametrize("rope", [O.rope_interleaved, O.rope_half])
def test_rope_scores_depend_on_relative_position_only(rope):
    c, s = _tables(64, ctx=512)
    rng = np.random.default_rng(1)
    q = rng.standard_normal((1, 1, 64)).astype(np.float32)
    k = rng.standard_normal((1, 1, 64)).astype(np.float32)

    def score(m, n):
        return float(np.sum(rope(q, c[[m]], s[[m]]).astype(np.float64) * rope(k, c[[n]], s[[n]])))

    ref = score(9, 4)
    for m in (20, 133, 300):
        assert abs(score(m, m - 5) - ref) < 2e-4 * (1 + abs(ref))
    assert abs(score(9, 5) - ref) > 1e-3  # a different offset gives a different score


def test_rope_pairing_one_hot():
    """rope_i rotates (2i, 2i+1); rope rotates (i, i + d/2)."""
    d, t, i = 64, 37, 5
    c, s = _tables(d)
    ci, si = float(c[t, i]), float(s[t, i])
    x = np.zeros((1, 1, d), np.float32)
    x[0, 0, 2 * i] = 1.0
    y = O.rope_interleaved(x, c[[t]], s[[t]])[0, 0]
    exp = np.zeros(d, np.float32)
    exp[2 * i], exp[2 * i + 1] = ci, si  # (x0 c - x1 s, x0 s + x1 c) with x0 = 1
    assert np.array_equal(y, exp)
    x = np.zeros((1, 1, d), np.float32)
    x[0, 0, i] = 1.0
    y = O.rope_half(x, c[[t]], s[[t]])[0, 0]
    exp = np.zeros(d, np.float32)
    exp[i], exp[i + d // 2] = ci, si
    assert np.array_equal(y, exp)
    # the second element of a pair: (-s, c)
    x = np.zeros((1, 1, d), np.float32)
    x[0, 0, 2 * i + 1] = 1.0
    y = O.rope_interleaved(x, c[[t]], s[[t]])[0, 0]
    assert y[2 * i] == np.float32(-si) and y[2 * i + 1] == np.float32(ci)


# ---- RMSNorm / SiLU ------------------------------------------------------------
def test_rms_norm_known_answers():
    w = np.array([1.0, 2.0], np.float32)
    # [3, 4]: mean of squares 12.5 -> [3, 4] / sqrt(12.5 + eps) * [1, 2]
    y = O.rms_norm(np.array([[3.0, 4.0]], np.float32), w, 1e-5)[0]
    r = math.sqrt(12.5 + 1e-5)
    np.testing.assert_allclose(y, [3.0 / r, 8.0 / r], rtol=1e-7)
    # constant rows: c / sqrt(c^2 + eps) * w
    y = O.rms_norm(np.full((1, 8), -2.0, np.float32), np.ones(8, np.float32), 1e-5)[0]
    np.testing.assert_allclose(y, np.full(8, -2.0 / math.sqrt(4.0 + 1e-5)), rtol=1e-7)
    # eps inside the root: tiny rows give x / sqrt(eps), not x / (rms + eps)
    y = O.rms_norm(np.full((1, 4), 1e-4, np.float32), np.ones(4, np.float32), 1e-5)[0]
    np.testing.assert_allclose(y, np.full(4, 1e-4 / math.sqrt(1e-8 + 1e-5)), rtol=1e-6)
    assert np.all(O.rms_norm(np.zeros((1, 4), np.float32), np.ones(4, np.float32), 1e-6) == 0)


def test_silu_known_answers():
    x = np.array([0.0, 1.0, -1.0, 30.0, -30.0], np.float32)
    y = O.silu(x)
    np.testing.assert_allclose(y[:3], [0.0, 1 / (1 + math.exp(-1)), -1 / (1 + math.exp(1))], rtol=1e-7)
    assert abs(y[3] - 30.0) < 1e-6 and abs(y[4]) < 1e-11


# ---- attention -------------------------------------------------------------------
def _attn_inputs(rng, n_heads=4, n_kv=2, M=3, T=7, hd=8):
    q = rng.standard_normal((n_heads, M, hd)).astype(np.float32)
    k = rng.standard_normal((n_kv, T, hd)).astype(np.float32)
    v = rng.standard_normal((n_kv, T, hd)).astype(np.float32)
    return q, k, v


def test_attention_single_visible_key_returns_its_value():
    rng = np.random.default_rng(2)
    q, k, v = _attn_inputs(rng, n_heads=2, n_kv=2)
    mask = np.zeros((3, 7), bool)
    mask[0, 4] = mask[1, 0] = mask[2, 6] = True
    y = O.attend(q, k, v, mask, 1 / math.sqrt(8))
    for h in range(2):
        for m, j in ((0, 4), (1, 0), (2, 6)):
            np.testing.assert_allclose(y[m, h], v[h, j], rtol=1e-6)


def test_attention_equal_scores_average_visible_rows():
    rng = np.random.default_rng(3)
    _, k, v = _attn_inputs(rng, n_heads=2, n_kv=2)
    q = np.zeros((2, 3, 8), np.float32)
    mask = np.tril(np.ones((3, 7), bool), k=4)  # causal over a 4-position prefix
    y = O.attend(q, k, v, mask, 1 / math.sqrt(8))
    for h in range(2):
        for m in range(3):
            np.testing.assert_allclose(y[m, h], v[h, :5 + m].astype(np.float64).mean(axis=0), rtol=1e-6, atol=1e-7)


def test_attention_scale_is_inverse_sqrt_head_dim():
    """Two keys whose scores differ by delta: weight = logistic(delta / sqrt(hd))."""
    hd = 64
    q = np.zeros((1, 1, hd), np.float32)
    q[0, 0, 0] = 1.0
    k = np.zeros((1, 2, hd), np.float32)
    k[0, 0, 0] = 3.0  # score 3 before scaling, the other key 0
    v = np.zeros((1, 2, hd), np.float32)
    v[0, 0, 0], v[0, 1, 0] = 1.0, 0.0
    y = O.attend(q, k, v, np.ones((1, 2), bool), 1 / math.sqrt(hd))
    w = 1.0 / (1.0 + math.exp(-3.0 / math.sqrt(hd)))
    assert abs(float(y[0, 0, 0]) - w) < 1e-7


def test_attention_masked_keys_have_no_influence():
    rng = np.random.default_rng(4)
    q, k, v = _attn_inputs(rng)
    mask = rng.random((3, 7)) < 0.6
    mask[:, 0] = True
    y = O.attend(q, k, v, mask, 0.3)
    k2, v2 = k.copy(), v.copy()
    k2[:, ~mask.any(axis=0)] = 1e3
    for m in range(3):
        hidden = ~mask[m]
        kk, vv = k.copy(), v.copy()
        kk[:, hidden], vv[:, hidden] = 50.0, 1e6
        np.testing.assert_allclose(O.attend(q[:, m:m + 1], kk, vv, mask[m:m + 1], 0.3)[0], y[m], rtol=1e-6)


def test_gqa_head_map_is_h_div_n_rep():
    """repeat_kv: query heads 0..n_rep-1 read KV head 0, the next n_rep head 1."""
    rng = np.random.default_rng(5)
    n_heads, n_kv, hd = 8, 2, 8
    q = rng.standard_normal((n_heads, 2, hd)).astype(np.float32)
    k = rng.standard_normal((n_kv, 5, hd)).astype(np.float32)
    v = np.empty((n_kv, 5, hd), np.float32)
    v[0], v[1] = 1.0, -1.0
    y = O.attend(q, k, v, np.ones((2, 5), bool), 0.5)
    for h in range(n_heads):
        np.testing.assert_allclose(y[:, h], 1.0 if h < n_heads // n_kv else -1.0, rtol=1e-6)


# ---- layer structure -------------------------------------------------------------
def _zero_blocks(fmt, rows, K):
    return np.zeros(rows * O.row_bytes(fmt, K), np.uint8)  # d = dmin = 0: every weight is 0


@pytest.mark.parametrize("arch", ["llama", "qwen2"])
def test_zero_residual_branches_make_layers_identity(arch):
    """attn + residual and mlp + residual (pre-norm): with wo = ffn_down = 0
    each layer returns its input, whatever q/k/v and gate/up are."""
    cfg = oracle_cfg(arch=arch, n_layers=2, hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=512, vocab=512,
                     ctx_len=64)
    base = O.OracleModel(cfg)
    tensors = dict(base.raw)
    for li in range(cfg.n_layers):
        for kind in (O.K_ATTN_O, O.K_FFN_DOWN):
            rows, K = cfg.shape(kind)
            fmt = cfg.fmt(li, kind)
            tensors[(li, kind)] = (fmt, _zero_blocks(fmt, rows, K))
    # a non-trivial final norm weight
    tensors[(-1, O.K_OUTPUT_NORM)] = (O.F32, np.linspace(0.5, 1.5, cfg.hidden, dtype=np.float32).view(np.uint8))
    om = O.OracleModel(cfg, tensors)
    ids = [3, 77, 500, 12]
    hid, col = om.forward(ids, list(range(4)), O.causal_mask(0, 4), collect_layers=[0, 1])
    emb = om.embed(ids)
    for c in col:
        assert np.array_equal(c, emb)
    np.testing.assert_allclose(hid, O.rms_norm(emb, om.w[(-1, O.K_OUTPUT_NORM)][0], cfg.rms_eps), rtol=1e-7)


def _q8_0_exact(w):
    """Q8_0 blocks (f16 d, 32 int8) whose weights are the integers of w exactly (d = 1)."""
    w = np.asarray(w)
    rows, K = w.shape
    assert K % 32 == 0 and np.all(np.abs(w) <= 127) and np.all(w == np.round(w))
    blk = np.zeros((rows, K // 32, 34), np.uint8)
    blk[:, :, 0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    blk[:, :, 2:] = w.reshape(rows, K // 32, 32).astype(np.int8).view(np.uint8)
    return O.Q8_0, blk.reshape(-1)


def _f32_tensor(v):
    return O.F32, np.ascontiguousarray(v, np.float32).view(np.uint8)


def _exact_model(cfg, emb, mats):
    """One layer from integer Q8_0 weights: embedding `emb`, the matrices and
    biases in `mats` (keyed by tensor kind), every other matrix and bias zero,
    every norm weight 1."""
    t = {}
    keys = [(-1, O.K_TOK_EMBD), (-1, O.K_OUTPUT_NORM), (-1, O.K_OUTPUT)] + [(0, k) for k in cfg.layer_kinds()]
    for (li, kind) in keys:
        rows, K = cfg.shape(kind)
        if kind in (O.K_OUTPUT_NORM, O.K_ATTN_NORM, O.K_FFN_NORM):
            t[(li, kind)] = _f32_tensor(np.ones(K))
        elif kind in (O.K_BQ, O.K_BK, O.K_BV):
            t[(li, kind)] = _f32_tensor(mats.get(kind, np.zeros(K)))
        elif kind == O.K_TOK_EMBD:
            t[(li, kind)] = _q8_0_exact(emb)
        else:
            t[(li, kind)] = _q8_0_exact(mats.get(kind, np.zeros((rows, K))))
    return O.OracleModel(cfg, t)


def _kat_cfg(arch):
    return oracle_cfg(arch=arch, n_layers=1, hidden=256, n_heads=4, n_kv_heads=4, head_dim=64, ffn=256, vocab=64,
                      ctx_len=16, mix="q8_0")


def _swiglu_kat(swap_roles):
    """quantized_llama_local.rs:45-51 (quantized_qwen2_local.rs:39-45): the MLP is
    ffn_down(silu(ffn_gate(x)) * ffn_up(x)). Attention is off (wo = 0), the
    embedding row is all ones, so the normalised input is r = 1/sqrt(1 + eps)
    in every column; feature 0 has gate weight 2 and up weight -1 on column 0,
    and ffn_down copies feature 0 into column 0 of the residual:
    x[0] = 1 + silu(2r) * (-r), against 1 + silu(-r) * 2r with the roles
    exchanged."""
    cfg = _kat_cfg("llama")
    H, F = cfg.hidden, cfg.ffn
    gate, up, down = np.zeros((F, H)), np.zeros((F, H)), np.zeros((H, F))
    gate[0, 0], up[0, 0], down[0, 0] = 2, -1, 1
    if swap_roles:  # the planted mistake: the two matrices' roles exchanged
        gate, up = up, gate
    om = _exact_model(cfg, np.ones((cfg.vocab, H)), {O.K_FFN_GATE: gate, O.K_FFN_UP: up, O.K_FFN_DOWN: down})
    _, (x1,) = om.forward([5], [0], O.causal_mask(0, 1), collect_layers=[0])
    r = 1.0 / math.sqrt(1.0 + cfg.rms_eps)
    g, u = 2.0 * r, -r
    assert abs(float(x1[0, 0]) - (1.0 + g / (1.0 + math.exp(-g)) * u)) < 2e-6
    assert np.all(x1[0, 1:] == 1.0)


def test_swiglu_gate_and_up_roles():
    _swiglu_kat(swap_roles=False)


def test_swiglu_planted_role_swap_fails():
    with pytest.raises(AssertionError):
        _swiglu_kat(swap_roles=True)


def _qwen2_bias_kat():
    """quantized_qwen2_local.rs:69-109: q = rope(x Wq + bq), k = rope(x Wk + bk),
    v = x Wv + bv -- the bias is added before RoPE. With Wq = Wk = 0 the
    rotated biases are the whole of q and k: bq = bk = 5 e_0 per head, so at
    position 1 (half rotation, theta_0 = 1) k1 = q1 = 5 (cos 1 e_0 + sin 1 e_32)
    while k0 = 5 e_0. Token 1 (all +1) at position 0 and token 2 (all -1) at
    position 1; Wv = Wo = I, so the residual after the layer is the embedding
    plus the attention output: row 0 = 1 + v0, row 1 = -1 + w v1 + (1 - w) v0,
    w = logistic((q1.k1 - q1.k0) / 8), v_t = fp16(xn_t + bv)."""
    cfg = _kat_cfg("qwen2")
    H, hd = cfg.hidden, cfg.head_dim
    emb = np.zeros((cfg.vocab, H))
    emb[1], emb[2] = 1, -1
    bq = np.zeros(H)
    bq[0::hd] = 5.0
    bv = 0.25 * (np.arange(H) % 5) - 0.5
    eye = np.eye(H)
    om = _exact_model(cfg, emb, {O.K_ATTN_V: eye, O.K_ATTN_O: eye, O.K_BQ: bq, O.K_BK: bq, O.K_BV: bv})
    _, (x1,) = om.forward([1, 2], [0, 1], O.causal_mask(0, 2), collect_layers=[0])
    r = 1.0 / math.sqrt(1.0 + cfg.rms_eps)
    f16 = lambda a: np.asarray(a, np.float16).astype(np.float64)
    # the cached key at position 1: 5 (cos 1, sin 1) on the pair (0, 32) of every head
    k1 = np.zeros(hd)
    k1[0], k1[hd // 2] = 5.0 * math.cos(1.0), 5.0 * math.sin(1.0)
    for h in range(cfg.n_kv_heads):
        np.testing.assert_allclose(om.k_cache[0][h, 1], f16(k1), rtol=0, atol=1e-6)
        np.testing.assert_allclose(om.k_cache[0][h, 0], f16(5.0 * np.eye(hd)[0]), rtol=0, atol=1e-6)
    v0, v1 = f16(r + bv), f16(-r + bv)
    s1, s0 = float(k1 @ f16(k1)), float(k1 @ f16(5.0 * np.eye(hd)[0]))
    w = 1.0 / (1.0 + math.exp(-(s1 - s0) / math.sqrt(hd)))
    assert 0.75 < w < 0.85  # 0.5 if the bias were added after the rotation
    np.testing.assert_allclose(x1[0], 1.0 + v0, rtol=0, atol=2e-6)
    np.testing.assert_allclose(x1[1], -1.0 + w * v1 + (1.0 - w) * v0, rtol=0, atol=2e-5)


def test_qwen2_bias_before_rope():
    _qwen2_bias_kat()


def test_qwen2_planted_bias_after_rope_fails(monkeypatch):
    """With Wq = Wk = 0, adding the bias after the rotation gives q = bq and
    k = bk at every position, i.e. the forward with the rotation removed."""
    monkeypatch.setattr(O, "rope_half", lambda x, c, s: x)
    with pytest.raises(AssertionError):
        _qwen2_bias_kat()


def test_causal_mask_matches_causal_bias():
    """causal_bias (quantized_llama_local.rs:332-350): prefix columns visible,
    -inf strictly above the diagonal of the new block."""
    m = O.causal_mask(3, 4)
    assert m.shape == (4, 7) and m[:, :3].all()
    assert np.array_equal(m[:, 3:], np.tril(np.ones((4, 4), bool)))
    assert np.array_equal(np.asarray(O.DraftTree.linear(1, [2, 3, 4]).attention_mask_bool()), m[:, 3:])


# ---- decoder invariants ------------------------------------------------------------
@pytest.fixture(scope="module")
def small():
    return oracle_cfg(n_layers=2, hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=512, vocab=1024, ctx_len=128)


def _dec(cfg):
    return O.OracleDecoder(O.OracleModel(cfg))


def test_batched_rows_equal_sequential_rows(small):
    """tests/with_qwen2_05b.rs:95-139: row i of batched_logits is what
    next_logits gives after observing the drafts one at a time."""
    rng = np.random.default_rng(6)
    prefix = [int(v) for v in rng.integers(0, small.vocab, 9)]
    drafts = [int(v) for v in rng.integers(0, small.vocab, 4)]
    a, b = _dec(small), _dec(small)
    a.observe(prefix)
    b.observe(prefix)
    rows = a.batched_logits(drafts)
    assert a.history == prefix + drafts and a.cache_len == len(prefix) + 4
    seq = [b.next_logits()]
    for d in drafts:
        b.observe([d])
        seq.append(b.next_logits())
    np.testing.assert_allclose(rows, np.stack(seq), rtol=2e-5, atol=2e-5 * np.abs(rows).max())


def test_linear_tree_equals_batched(small):
    """tests/with_qwen2_05b.rs:141-184 and tree_logits_consistency.rs:74-122."""
    rng = np.random.default_rng(7)
    prefix = [int(v) for v in rng.integers(0, small.vocab, 11)]
    drafts = [int(v) for v in rng.integers(0, small.vocab, 5)]
    a, b = _dec(small), _dec(small)
    a.observe(prefix)
    b.observe(prefix)
    rows = a.batched_logits(drafts)
    t_rows, hidden = b.tree_logits_keep_kv(O.DraftTree.linear(prefix[-1], drafts))
    assert b.cache_len == len(prefix) + 5 and b.history == prefix
    np.testing.assert_allclose(t_rows, rows, rtol=2e-5, atol=2e-5 * np.abs(rows).max())
    # the tree's positions are prefix + depth: a sibling at depth 1 sees the
    # same context as the first draft and gets the same row
    c = _dec(small)
    c.observe(prefix)
    tree = O.DraftTree([prefix[-1], drafts[0], drafts[0]], [0, 0, 0])
    tr, _ = c.tree_logits_keep_kv(tree)
    np.testing.assert_allclose(tr[1], tr[2], rtol=1e-6, atol=1e-6 * np.abs(tr).max())
    np.testing.assert_allclose(tr[1], rows[1], rtol=2e-5, atol=2e-5 * np.abs(rows).max())


def test_tree_root_row_and_strict_restore(small):
    rng = np.random.default_rng(8)
    prefix = [int(v) for v in rng.integers(0, small.vocab, 7)]
    a = _dec(small)
    a.observe(prefix)
    nxt = a.next_logits()
    tree = O.build_cartesian_tree(prefix[-1], [[1, 2], [3, 4]])
    rows, _ = a.tree_logits_keep_kv(tree)
    np.testing.assert_allclose(rows[0], nxt, rtol=2e-5, atol=2e-5 * np.abs(nxt).max())
    a.rollback_to(len(prefix))
    strict = a.tree_logits(tree)
    assert a.cache_len == len(prefix) and a.history == prefix
    assert np.array_equal(strict[0], a.next_logits())
    np.testing.assert_allclose(strict[1:], rows[1:], rtol=1e-6, atol=1e-6 * np.abs(rows).max())


def test_qwen2_strict_tree_logits_keeps_the_tree_row(small):
    """Qwen2QuantDecoder::tree_logits (quantized_qwen2.rs:184-237) runs the same
    restoring one-token pass as Llama's but discards its row: row 0 stays the
    tree pass's row, while the restoring pass refreshes next_logits."""
    import dataclasses
    cfg = dataclasses.replace(small, arch="qwen2")
    rng = np.random.default_rng(8)
    prefix = [int(v) for v in rng.integers(0, cfg.vocab, 7)]
    a = _dec(cfg)
    a.observe(prefix)
    tree = O.build_cartesian_tree(prefix[-1], [[1, 2], [3, 4]])
    strict = a.tree_logits(tree)
    assert a.cache_len == len(prefix) and a.history == prefix
    one = a.next_logits()  # the restoring pass's row, cached
    rows, _ = a.tree_logits_keep_kv(tree)
    assert np.array_equal(strict, rows)
    a.rollback_to(len(prefix) - 1)
    a.observe([prefix[-1]])
    assert np.array_equal(one, a.next_logits())


def test_commit_tree_path_equals_observing_the_path(small):
    """commit_tree_path keeps the accepted rows: the next pass equals the one
    after observing the path's tokens directly."""
    rng = np.random.default_rng(9)
    prefix = [int(v) for v in rng.integers(0, small.vocab, 6)]
    tree = O.build_cartesian_tree(prefix[-1], [[10, 11], [12, 13], [14]])
    keep = [0, 2, 5, 9]  # root -> 11 -> 12 -> 14
    assert [tree.parent_of(i) for i in keep[1:]] == keep[:-1]
    a, b = _dec(small), _dec(small)
    a.observe(prefix)
    b.observe(prefix)
    a.tree_logits_keep_kv(tree)
    a.commit_tree_path(tree, keep)
    b.observe([tree.token_at(i) for i in keep[1:]])
    assert a.history == b.history and a.cache_len == b.cache_len
    a.observe([77])
    b.observe([77])
    np.testing.assert_allclose(a.next_logits(), b.next_logits(), rtol=2e-5,
                               atol=2e-5 * np.abs(b.next_logits()).max())
