"""Parity against the oracle at the Llama-3-8B widths (hidden 4096, 32 / 8
heads of 128, FFN 14336, vocab 128256, Q4_K_M mix: layer 1 of 2 takes Q6_K on
attn_v / ffn_down), 2 layers, at the benchmark's verify shapes:

* every matrix's K1 product at M in {1, 5, 9, 16, 17, 60, 64} against f64 on
  the dequantised weights (1e-2 contract) and, on a row sample, against its
  exact operands (fp16 activations times the weights the kernel uses);
* the M = 5 linear verify over 512 cached positions;
* the 60-node tree (branching (4,3,2,2,1,1) pruned) over 4096 positions
  (logits and final-norm hidden; the split-K M > 16 matmuls, their RoPE and
  RMSNorm finalisers at 4096 / 14336, the 128256-row lm_head);
* the strict tree row 0 (a 1-row pass of the root) against the oracle;
* the 64-node depth-7 tree over 8192 positions (EAGLE-3 shape).

Logits and hidden rows within 1e-2 relative (fp16 activations, f32
accumulate); first-max argmax equal wherever the oracle's top-2 margin
exceeds twice the row's device/oracle difference, with the near-tie count
asserted rather than skipped.  Reference forward:
quantized_llama_local.rs:363-432.
"""
import numpy as np
import pytest

import oracle as O
from _fullwidth import (LLAMA8B, TOL, argmax_agreement, build_pair, load_prefix, oracle_pass, random_tree, rel_rows,
                        tree_mask)
from test_gpu_kernels import operand_weights

pytestmark = pytest.mark.gpu

CTX = 8192 + 256


@pytest.fixture(scope="module")
def pair(hip):
    dec, om = build_pair(hip, LLAMA8B, "q4_k_m", 2, CTX)
    yield dec, om
    dec.close()


KINDS = [(0, O.K_ATTN_Q), (0, O.K_ATTN_K), (1, O.K_ATTN_V), (0, O.K_ATTN_O), (0, O.K_FFN_GATE), (1, O.K_FFN_UP),
         (0, O.K_FFN_DOWN), (1, O.K_FFN_DOWN), (-1, O.K_OUTPUT)]
MS = (1, 5, 9, 16, 17, 60, 64)


@pytest.mark.parametrize("layer,kind", KINDS)
def test_k1_full_width(hip, pair, layer, kind):
    dec, om = pair
    W = om.w[(layer, kind)]
    fmt, raw = om.raw[(layer, kind)]
    rows, K = W.shape
    rng = np.random.default_rng(1000 + 16 * layer + kind)
    x = rng.standard_normal((64, K)).astype(np.float32)
    ref32 = O.matmul_t(x, W).astype(np.float64)
    # exact operands on a row sample: first / last tiles and random rows
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


def test_linear_verify_m5_p512(hip, pair):
    dec, om = pair
    V = LLAMA8B["vocab"]
    rng = np.random.default_rng(21)
    hist = [int(v) for v in rng.integers(0, V, 513)]
    dec.prime_synthetic(hist, 31)
    P = len(hist) - 1
    load_prefix(dec, om, P)
    drafts = [int(v) for v in rng.integers(0, V, 4)]
    ids = [hist[-1]] + drafts
    ref, _ = oracle_pass(om, ids, list(range(P, P + 5)), O.causal_mask(P, 5))
    got = dec.batched_logits(drafts)
    err = rel_rows(got, ref)
    assert np.all(err < TOL), err
    argmax_agreement(got, ref)
    assert [int(v) for v in dec.last_argmax(5)] == [O.argmax_fold(r) for r in got]
    # greedy acceptance on the device == the oracle's walk over the oracle's
    # rows: a chain whose first two drafts are the target's own argmaxes
    dec.rollback_to(P + 1)
    chain = [O.argmax_fold(ref[0]), 17, 5, 9]
    load_prefix(dec, om, P)
    ref2, _ = oracle_pass(om, [hist[-1]] + chain, list(range(P, P + 5)), O.causal_mask(P, 5))
    chain[1] = O.argmax_fold(ref2[1])
    load_prefix(dec, om, P)
    ref2, _ = oracle_pass(om, [hist[-1]] + chain, list(range(P, P + 5)), O.causal_mask(P, 5))
    rows2 = dec.batched_logits(chain)
    dec.rollback_to(P + 1)
    near = argmax_agreement(rows2, ref2)
    commits, n_acc = dec.verify_greedy_linear(chain)
    # always: the device walk is the walk over the device's own argmaxes
    d_acc, d_bonus = O.greedy_linear_accept(chain, [O.argmax_fold(r) for r in rows2])
    assert n_acc == d_acc and commits == chain[:d_acc] + [d_bonus]
    # and the oracle's walk unless a row it consults is near a tie
    exp_acc, bonus = O.greedy_linear_accept(chain, [O.argmax_fold(r) for r in ref2])
    assert exp_acc >= 2
    if not set(near) & set(range(exp_acc + 1)):
        assert n_acc == exp_acc and commits == chain[:exp_acc] + [bonus]
    dec.rollback_to(P + 1)


def _tree_case(hip, dec, om, P, n, branching, seed):
    V = LLAMA8B["vocab"]
    rng = np.random.default_rng(seed)
    hist = [int(v) for v in rng.integers(0, V, P + 1)]
    dec.prime_synthetic(hist, seed + 1)
    load_prefix(dec, om, P)
    tree = random_tree(hip, rng, hist[-1], V, branching, n)
    assert len(tree) == n
    ref, ref_h = oracle_pass(om, tree.tokens(), tree.position_ids(P), tree_mask(tree, P))
    got, got_h = dec.tree_logits_keep_kv((tree.tokens(), tree.parents()))
    assert dec.cache_len() == P + n
    err = rel_rows(got, ref)
    assert np.all(err < TOL), (float(err.max()), int(err.argmax()))
    herr = rel_rows(got_h, ref_h)
    assert np.all(herr < TOL), float(herr.max())
    near = argmax_agreement(got, ref)
    return hist, tree, ref, near


def test_tree60_p4096(hip, pair):
    dec, om = pair
    P = 4096
    hist, tree, ref, near = _tree_case(hip, dec, om, P, 60, (4, 3, 2, 2, 1, 1), 41)
    # the device walk == the walk over the device's argmaxes, and == the
    # oracle's walk over the oracle rows when no row is near a tie
    dec.rollback_to(P + 1)
    res = dec.verify_greedy_tree((tree.tokens(), tree.parents()), compose=True)
    am_dev = [int(v) for v in dec.last_argmax(len(tree))]
    best, bonus = O.greedy_tree_accept(tree, list(ref), [O.argmax_fold(r) for r in ref])
    dbest, dbonus = O.greedy_tree_accept(tree, None, am_dev)
    assert res.path == dbest and res.bonus == dbonus
    if not set(near) & set(best):
        assert res.path == best and res.bonus == bonus
    # strict: row 0 is a 1-row pass of the root
    dec.rollback_to(P + 1)
    strict = dec.tree_logits((tree.tokens(), tree.parents()))
    assert dec.cache_len() == P + 1
    load_prefix(dec, om, P)
    r0, _ = oracle_pass(om, [hist[-1]], [P], np.ones((1, P + 1), bool))
    assert rel_rows(strict[:1], r0)[0] < TOL
    argmax_agreement(strict[:1], r0, max_near_frac=1.0)


def test_tree64_p8192(hip, pair):
    dec, om = pair
    _, tree, _, _ = _tree_case(hip, dec, om, 8192, 64, (4, 3, 2, 2, 1, 1, 1), 51)
    assert max(tree.depth_of(i) for i in range(len(tree))) >= 5
