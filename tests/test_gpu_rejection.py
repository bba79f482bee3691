"""Device rejection-sampling acceptance (vanilla.rs:178-210, and the tree walk
built from the same steps) against the oracle, through the C ABI.

Both sides read the same logits (the device's own verify rows), so what is
compared is the acceptance arithmetic alone.  The device sums in parallel and
the oracle sequentially in f32 (as the reference does), so results may differ
only where a uniform lies within rounding of a threshold: an accept test with
|u - min(1, p/q)| tiny, or a draw whose target u*sum lies within the
accumulated rounding of a CDF boundary.  Each case is classified by an f64
restatement; away from such boundaries the device must agree with the oracle
exactly, near one it must still pick one of the two tokens that meet there.
"""
import numpy as np
import pytest

import oracle as O
from _models import MIX_IDS, hip_cfg, oracle_cfg

pytestmark = pytest.mark.gpu

DEC_EPS = 1e-5  # accept-test margin below which a decision counts as a boundary case


def _p64(row, T, mask=None):
    r = np.asarray(row, np.float64).copy()
    if mask is not None:
        r[~mask] = -np.inf
    if T == 0:
        p = np.zeros_like(r)
        p[O.argmax_fold(np.where(np.isfinite(r), r, -np.inf).astype(np.float32))] = 1.0
        return p
    e = np.exp((r - r.max()) / T)
    return e / e.sum()


def _walk64(tree, rows, q_rows, q_row_of, u, T, mask=None, max_commit=None):
    """f64 restatement of the walk; returns (path, token, min decision margin,
    draw target, f64 CDF of the drawn distribution)."""
    n = len(tree)
    children = [[] for _ in range(n)]
    for c in range(1, n):
        children[tree.parent_of(c)].append(c)
    used, node, path, margin = 0, 0, [0], np.inf
    while True:
        if max_commit and len(path) - 1 >= max_commit:
            return path, None, margin, None, None
        p = _p64(rows[node], T, mask)
        acc = None
        for c in children[node]:
            q = np.asarray(q_rows[q_row_of[node]], np.float64)
            tok = tree.token_at(c)
            ratio = 1.0 if q[tok] <= 0 else min(1.0, p[tok] / q[tok])
            margin = min(margin, abs(u[used] - ratio))
            ok = q[tok] <= 0 or u[used] <= ratio
            used += 1
            if ok:
                acc = c
                break
            a = np.maximum(p - q, 0.0)
            p = a / a.sum()
        if acc is not None:
            path.append(acc)
            node = acc
            continue
        cdf = np.cumsum(p) / p.sum()
        t = float(u[used])
        tok = int(min(np.searchsorted(cdf, t, side="right"), len(cdf) - 1))
        return path, tok, margin, t, cdf


def _check_walk(dev_path, dev_tok, ora_path, ora_tok, tree, rows, q_rows, q_row_of, u, T, mask=None,
                max_commit=None):
    """Returns 'exact' or 'boundary'; asserts the device result is valid.  A
    draw is near a boundary when its target is within 4 sqrt(V) f32 ulps of
    1 of one (the spread of sequential f32 running sums over V terms)."""
    path64, tok64, margin, t, cdf = _walk64(tree, rows, q_rows, q_row_of, u, T, mask, max_commit)
    draw_eps = 4.0 * np.sqrt(len(rows[0])) * 2.0 ** -24
    if margin < DEC_EPS:
        return "boundary"
    assert dev_path == ora_path == path64
    if tok64 is None:
        assert dev_tok is None and ora_tok is None
        return "exact"
    lo = cdf[tok64 - 1] if tok64 > 0 else 0.0
    near = min(t - lo, cdf[tok64] - t) < draw_eps
    if not near:
        assert dev_tok == ora_tok == tok64, (dev_tok, ora_tok, tok64)
        return "exact"
    # near a boundary: the device token must be one of the two meeting there
    assert dev_tok in (tok64 - 1, tok64, tok64 + 1)
    return "boundary"


def _pair(hip, prefix_len=48, **over):
    ocfg = oracle_cfg(**over)
    hd = hip.HipQuantDecoder(hip_cfg(hip, ocfg))
    hd.synthesize(MIX_IDS[ocfg.mix], ocfg.seed, ocfg.weight_std)
    prefix = [int(v) for v in np.random.default_rng(1).integers(0, ocfg.vocab, prefix_len)]
    hd.observe(prefix)
    return ocfg, hd, prefix


def _draft_rows(rng, k, V, scale=2.0):
    """Draft distributions: softmax of N(0, scale^2) logits (seeded)."""
    out = np.empty((k, V), np.float32)
    for i in range(k):
        out[i] = O.softmax_t(rng.standard_normal(V).astype(np.float32) * scale, 1.0)
    return out


@pytest.mark.parametrize("over,k", [
    (dict(), 4),
    # Qwen2-shaped variant of the mixed-quantisation workload: QKV bias,
    # Q5_K attention, Q8_0 FFN, GQA 2:1, k = 8 (M = 9)
    (dict(arch="qwen2", n_kv_heads=4, mix="q5k_q80", n_layers=2, rms_eps=1e-6, rope_theta=1e6), 8),
])
@pytest.mark.parametrize("T", [0.1, 1.0, 0.0])
def test_rejection_linear_matches_oracle(hip, over, k, T):
    ocfg, hd, prefix = _pair(hip, **over)
    V = ocfg.vocab
    rng = np.random.default_rng(17 + k)
    L = len(prefix)
    kinds = {"exact": 0, "boundary": 0}
    for trial in range(6):
        q = _draft_rows(rng, k, V)
        if trial % 2 == 0:
            drafts = [int(O.sample_u(q[i], float(rng.random()))) for i in range(k)]
        else:
            # drafts that the target likes, so that acceptance runs deep
            rows = hd.batched_logits([int(v) for v in rng.integers(0, V, k)])
            hd.rollback_to(L)
            drafts = [O.argmax_fold(rows[i]) for i in range(k)]
            for i in range(k):
                q[i] = 0.5 * q[i]
                q[i][drafts[i]] += 0.5
        u = [float(x) for x in rng.random(k + 1, dtype=np.float32)]
        rows = hd.batched_logits(drafts)
        hd.rollback_to(L)
        for max_commit in (0, 2):
            commits, n_acc, used = hd.verify_rejection_linear(drafts, q, u, T, max_commit)
            assert hd.history() == prefix + drafts and hd.cache_len() == L + k
            hd.rollback_to(L)
            oc, on, ou = O.rejection_linear_accept(list(rows), list(q), drafts, u, T, max_commit or None)
            tree = O.DraftTree.linear(prefix[-1], drafts)
            dev_fin = commits[n_acc] if len(commits) > n_acc else None
            ora_fin = oc[on] if len(oc) > on else None
            kind = _check_walk(list(range(n_acc + 1)), dev_fin, list(range(on + 1)), ora_fin, tree, list(rows),
                               list(q), list(range(k)) + [-1], u, T, max_commit=max_commit or None)
            kinds[kind] += 1
            if kind == "exact":
                assert commits == oc and n_acc == on and used == ou
    # at T = 1 the tiny model's rows are nearly flat over 32000 tokens, so most
    # draws sit within rounding of a CDF boundary (checked for validity only)
    if T != 1.0:
        assert kinds["exact"] >= 8, kinds


def test_rejection_linear_errors_keep_state(hip):
    ocfg, hd, prefix = _pair(hip, prefix_len=16)
    q = np.full((2, ocfg.vocab), 1.0 / ocfg.vocab, np.float32)
    for T in (-1.0, float("nan"), float("inf")):
        with pytest.raises(hip.SamplingError):
            hd.verify_rejection_linear([1, 2], q, [0.5, 0.5, 0.5], T)
        assert hd.history() == prefix and hd.cache_len() == len(prefix)
    with pytest.raises(hip.ArgError):
        hd.verify_rejection_linear([1, 2], q, [0.5, 0.5], 1.0)  # k + 1 uniforms needed
    assert hd.history() == prefix


def _seeded_d2t(rng, draft_vocab, target_vocab):
    """Seeded injective draft -> target map."""
    return rng.choice(target_vocab, size=draft_vocab, replace=False).astype(np.int64)


@pytest.mark.parametrize("T", [0.1, 1.0])
@pytest.mark.parametrize("use_t2d", [False, True])
def test_rejection_tree_d2t_matches_oracle(hip, T, use_t2d):
    """Tree rejection over a pruned Cartesian tree whose draft rows live in a
    smaller draft vocabulary mapped through a seeded injective d2t table."""
    ocfg, hd, prefix = _pair(hip, prefix_len=40)
    V, Vd = ocfg.vocab, 8000
    rng = np.random.default_rng(123 + int(use_t2d))
    d2t = _seeded_d2t(rng, Vd, V)
    hd.set_d2t(d2t)
    inv, mask = O.d2t_maps(d2t, V)
    assert np.array_equal(hd.t2d_mask(), mask)
    assert hd.draft_to_target([0, 5, Vd - 1]) == [int(d2t[0]), int(d2t[5]), int(d2t[Vd - 1])]
    with pytest.raises(hip.SamplingError):
        hd.draft_to_target([Vd])
    L = len(prefix)
    kinds = {"exact": 0, "boundary": 0}
    for trial in range(3):
        branching = (4, 3, 2, 2, 1, 1, 1)
        cands = [[int(d2t[v]) for v in rng.choice(Vd, b, replace=False)] for b in branching]
        lps = [list(np.sort(np.log(rng.dirichlet(np.ones(b))))[::-1].astype(np.float32)) for b in branching]
        full = hip.tree_cartesian(prefix[-1], cands)
        toks, pars = hip.tree_prune(full, lps, 64)
        tree = O.DraftTree(list(toks), list(pars))
        n = len(tree)
        q_d = _draft_rows(rng, n, Vd)  # one draft row per node, draft vocabulary
        q_row_of = list(range(n))
        u = [float(x) for x in rng.random(n, dtype=np.float32)]
        rows, _ = hd.tree_logits_keep_kv((toks, pars))
        hd.rollback_to(L)
        path, tok, used = hd.verify_rejection_tree((toks, pars), q_d, q_row_of, u, T, use_t2d)
        assert hd.cache_len() == L - 1 + n
        hd.rollback_to(L)
        # the oracle reads target-vocabulary draft rows: scatter through d2t
        q_t = np.zeros((n, V), np.float32)
        for tid, did in inv.items():
            q_t[:, tid] = q_d[:, did]
        opath, otok, oused = O.rejection_tree_accept(tree, list(rows), list(q_t), q_row_of, u, T,
                                                     t2d_mask=mask if use_t2d else None)
        kind = _check_walk(path, tok if tok >= 0 else None, opath, otok, tree, list(rows), list(q_t), q_row_of, u,
                           T, mask=mask if use_t2d else None)
        kinds[kind] += 1
        if kind == "exact":
            assert used == oused
        if use_t2d and tok >= 0:
            assert mask[tok]
    if T != 1.0:
        assert kinds["exact"] >= 2, kinds


def test_rejection_tree_chain_equals_linear(hip):
    """The tree walk on a chain is the linear walk, uniform for uniform."""
    ocfg, hd, prefix = _pair(hip, prefix_len=24)
    V, k = ocfg.vocab, 5
    rng = np.random.default_rng(8)
    L = len(prefix)
    for _ in range(4):
        q = _draft_rows(rng, k, V)
        drafts = [int(O.sample_u(q[i], float(rng.random()))) for i in range(k)]
        u = [float(x) for x in rng.random(k + 1, dtype=np.float32)]
        commits, n_acc, used = hd.verify_rejection_linear(drafts, q, u, 0.1)
        hd.rollback_to(L)
        tree = O.DraftTree.linear(prefix[-1], drafts)
        path, tok, used_t = hd.verify_rejection_tree((tree.tokens(), tree.parents()), q,
                                                     list(range(k)) + [-1], u, 0.1)
        hd.rollback_to(L)
        assert path == list(range(n_acc + 1)) and used_t == used
        assert commits == drafts[:n_acc] + ([tok] if tok >= 0 else [])
