"""Parity against the oracle at the Qwen2.5-7B widths (hidden 3584, 28 / 4
heads of 128, FFN 18944, vocab 152064, QKV bias, Q5_K attention and Q8_0
FFN / embedding / lm_head), 2 layers:

* every matrix's K1 product at M in {1, 5, 9, 16, 17, 60, 64} against f64 on
  the dequantised weights, and on a row sample against its exact operands;
* the M = 9 linear verify over 2048 cached positions (the rejection-sampling
  workload's forward);
* a 60-node tree over 2048 positions (the Qwen2 tree path, half-rotation
  RoPE in the M > 16 finaliser).

Reference forward: quantized_qwen2_local.rs:345-395.
"""
import numpy as np
import pytest

import oracle as O
from _fullwidth import (QWEN7B, TOL, argmax_agreement, build_pair, load_prefix, oracle_pass, random_tree, rel_rows,
                        tree_mask)
from test_gpu_kernels import operand_weights

pytestmark = pytest.mark.gpu

CTX = 2048 + 256


@pytest.fixture(scope="module")
def pair(hip):
    dec, om = build_pair(hip, QWEN7B, "q5k_q80", 2, CTX)
    yield dec, om
    dec.close()


KINDS = [(0, O.K_ATTN_Q), (0, O.K_ATTN_K), (1, O.K_ATTN_V), (0, O.K_ATTN_O), (0, O.K_FFN_GATE), (1, O.K_FFN_UP),
         (0, O.K_FFN_DOWN), (-1, O.K_OUTPUT)]
MS = (1, 5, 9, 16, 17, 60, 64)


@pytest.mark.parametrize("layer,kind", KINDS)
def test_k1_full_width(hip, pair, layer, kind):
    dec, om = pair
    W = om.w[(layer, kind)]
    fmt, raw = om.raw[(layer, kind)]
    rows, K = W.shape
    rng = np.random.default_rng(2000 + 16 * layer + kind)
    x = rng.standard_normal((64, K)).astype(np.float32)
    ref32 = O.matmul_t(x, W).astype(np.float64)
    pick = np.unique(np.concatenate([np.arange(32), rows - 32 + np.arange(32),
                                     rng.choice(rows, 448, replace=False)]))
    rb = raw.reshape(rows, -1)[pick].reshape(-1)
    x16 = O.round_f16(x).astype(np.float64)
    for M in MS:
        y = dec.qmatmul(layer, kind, x[:M])
        assert y.shape == (M, rows)
        err = float(np.max(rel_rows(y, ref32[:M])))
        assert err < TOL, (M, err)
        Wk = operand_weights(fmt, rb, len(pick), K, M).astype(np.float64)
        ref16 = x16[:M] @ Wk.T
        tight = float(np.max(np.abs(y[:, pick] - ref16)) / np.max(np.abs(ref16)))
        assert tight < 1e-4, (M, tight)


def test_linear_verify_m9_p2048(hip, pair):
    dec, om = pair
    V = QWEN7B["vocab"]
    rng = np.random.default_rng(61)
    hist = [int(v) for v in rng.integers(0, V, 2049)]
    dec.prime_synthetic(hist, 71)
    P = len(hist) - 1
    load_prefix(dec, om, P)
    drafts = [int(v) for v in rng.integers(0, V, 8)]
    ref, _ = oracle_pass(om, [hist[-1]] + drafts, list(range(P, P + 9)), O.causal_mask(P, 9))
    got = dec.batched_logits(drafts)
    err = rel_rows(got, ref)
    assert np.all(err < TOL), err
    argmax_agreement(got, ref)
    assert dec.history() == hist + drafts and dec.cache_len() == P + 9
    dec.rollback_to(P + 1)


def test_tree60_p2048(hip, pair):
    dec, om = pair
    V = QWEN7B["vocab"]
    P = 2048
    rng = np.random.default_rng(81)
    hist = [int(v) for v in rng.integers(0, V, P + 1)]
    dec.prime_synthetic(hist, 91)
    load_prefix(dec, om, P)
    tree = random_tree(hip, rng, hist[-1], V, (4, 3, 2, 2, 1, 1), 60)
    ref, ref_h = oracle_pass(om, tree.tokens(), tree.position_ids(P), tree_mask(tree, P))
    got, got_h = dec.tree_logits_keep_kv((tree.tokens(), tree.parents()))
    err = rel_rows(got, ref)
    assert np.all(err < TOL), (float(err.max()), int(err.argmax()))
    herr = rel_rows(got_h, ref_h)
    assert np.all(herr < TOL), float(herr.max())
    argmax_agreement(got, ref)
    dec.rollback_to(P + 1)


def test_rejection_m9_full_vocab(hip, pair):
    """The rejection walk over 152064-entry rows (the row statistics' slices,
    the walk's tiles) against the oracle's walk, with host and with
    device-resident draft rows (the benchmark's Qwen2.5-7B workload)."""
    from test_gpu_rejection import _check_walk, _draft_rows, _peaked_q
    dec, om = pair
    V, k = QWEN7B["vocab"], 8
    rng = np.random.default_rng(91)
    P = 300
    hist = [int(v) for v in rng.integers(0, V, P + 1)]
    dec.prime_synthetic(hist, 93)
    L = P + 1
    kinds = {"exact": 0, "boundary": 0}
    for trial in range(6):
        q = _draft_rows(rng, k, V)
        drafts = [int(O.sample_u(q[i], float(rng.random()))) for i in range(k)]
        rows = dec.batched_logits(drafts)
        dec.rollback_to(L)
        T = 1.0 if trial < 4 else 0.0
        if trial in (2, 3):
            for i in range(k):
                q[i] = _peaked_q(O.softmax_t(rows[i], T), [drafts[i]], rng)
        u = [float(x) for x in rng.random(k + 1, dtype=np.float32)]
        commits, n_acc, used = dec.verify_rejection_linear(drafts, q, u, T)
        dec.rollback_to(L)
        with hip.DeviceArray(q) as qd:
            assert dec.verify_rejection_linear_device(drafts, qd.ptr, u, T) == (commits, n_acc, used)
        dec.rollback_to(L)
        oc, on, ou = O.rejection_linear_accept(list(rows), list(q), drafts, u, T)
        tree = O.DraftTree.linear(hist[-1], drafts)
        dev_fin = commits[n_acc] if len(commits) > n_acc else None
        ora_fin = oc[on] if len(oc) > on else None
        # the oracle's sequential f32 CDF over 152064 entries drifts by up to
        # V ulps of 1; the device's tree sums are held to the default window
        kind = _check_walk(list(range(n_acc + 1)), dev_fin, list(range(on + 1)), ora_fin, tree, list(rows), list(q),
                           list(range(k)) + [-1], u, T, ora_draw_eps=V * 2.0 ** -24)
        kinds[kind] += 1
        if kind == "exact":
            assert commits == oc and n_acc == on and used == ou
    assert kinds["exact"] >= 2, kinds
