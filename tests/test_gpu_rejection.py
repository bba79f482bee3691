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


def _walk64(tree, rows, q_rows, q_row_of, u, T, mask=None, max_commit=None, flip=frozenset(), wor=False):
    """f64 restatement of the walk; returns (path, token, {uniform index:
    decision margin}, draw target, f64 CDF of the drawn distribution).  The
    accept decisions of the uniforms in `flip` are inverted (the other side
    of a near tie)."""
    n = len(tree)
    children = [[] for _ in range(n)]
    for c in range(1, n):
        children[tree.parent_of(c)].append(c)
    used, node, path, margins = 0, 0, [0], {}
    while True:
        if max_commit and len(path) - 1 >= max_commit:
            return path, None, margins, None, None
        p = _p64(rows[node], T, mask)
        acc = None
        q0 = np.asarray(q_rows[q_row_of[node]], np.float64) if children[node] else None
        R, rejected = 1.0, []
        for c in children[node]:
            q = q0
            if wor:
                q = q0 / R if R > 0 else np.zeros_like(q0)
                q[rejected] = 0.0
            tok = tree.token_at(c)
            ratio = 1.0 if q[tok] <= 0 else min(1.0, p[tok] / q[tok])
            margins[used] = abs(u[used] - ratio)
            ok = q[tok] <= 0 or u[used] <= ratio
            if used in flip:
                ok = not ok
            used += 1
            if ok:
                acc = c
                break
            a = np.maximum(p - q, 0.0)
            p = a / a.sum()
            rejected.append(tok)
            R -= q0[tok]
        if acc is not None:
            path.append(acc)
            node = acc
            continue
        cdf = np.cumsum(p) / p.sum()
        t = float(u[used])
        tok = int(min(np.searchsorted(cdf, t, side="right"), len(cdf) - 1))
        return path, tok, margins, t, cdf


def _draw_ok(tok, tok64, t, cdf, draw_eps):
    """(token valid, drawn away from a CDF boundary).  Near a boundary (the
    target within draw_eps of one) the token may be any token of positive
    mass whose CDF step reaches into [t - draw_eps, t + draw_eps]."""
    if tok64 is None:
        return tok is None, True
    if tok is None:
        return False, True
    lo = cdf[tok64 - 1] if tok64 > 0 else 0.0
    near = min(t - lo, cdf[tok64] - t) < draw_eps
    if not near:
        return tok == tok64, True
    tlo = cdf[tok - 1] if tok > 0 else 0.0
    return bool(cdf[tok] > tlo and tlo <= t + draw_eps and cdf[tok] >= t - draw_eps), False


def _check_walk(dev_path, dev_tok, ora_path, ora_tok, tree, rows, q_rows, q_row_of, u, T, mask=None,
                max_commit=None, wor=False, ora_draw_eps=None):
    """Returns 'exact' or 'boundary' and asserts that the device and the
    oracle results are valid walks.  A decision is a near tie when |u -
    min(1, p/q)| < DEC_EPS: both sides of it are then valid, and device and
    oracle must each follow one of them exactly.  A draw is near a boundary
    when its target is within 4 sqrt(V) f32 ulps of 1 of one (the spread of
    sequential f32 running sums over V terms): the token is then one of the
    two meeting there.  Everything else must agree exactly.  ora_draw_eps
    widens the oracle's window: its sequential f32 running sum over a large
    flat row drifts by up to V f32 ulps of 1 (the reference's own rounding),
    while the device's tree sums stay within the default window."""
    path64, tok64, margins, t, cdf = _walk64(tree, rows, q_rows, q_row_of, u, T, mask, max_commit, wor=wor)
    draw_eps = 4.0 * np.sqrt(len(rows[0])) * 2.0 ** -24
    ora_eps = draw_eps if ora_draw_eps is None else ora_draw_eps
    ties = [i for i, m in margins.items() if m < DEC_EPS]
    if not ties:
        assert dev_path == ora_path == path64, (dev_path, ora_path, path64)
        ok_d, exact_d = _draw_ok(dev_tok, tok64, t, cdf, draw_eps)
        ok_o, exact_o = _draw_ok(ora_tok, tok64, t, cdf, ora_eps)
        assert ok_d and ok_o, (dev_tok, ora_tok, tok64)
        if exact_d and exact_o:
            assert dev_tok == ora_tok == tok64
            return "exact"
        return "boundary"
    # one or more near ties: every combination of their outcomes is valid
    alts = []
    for k in range(1 << len(ties)):
        flip = frozenset(ties[j] for j in range(len(ties)) if (k >> j) & 1)
        alts.append(_walk64(tree, rows, q_rows, q_row_of, u, T, mask, max_commit, flip=flip, wor=wor))
    for path, tok, eps in ((dev_path, dev_tok, draw_eps), (ora_path, ora_tok, ora_eps)):
        assert any(path == a[0] and _draw_ok(tok, a[1], a[3], a[4], eps)[0] for a in alts), (path, tok)
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


def _peaked_q(p, favour, rng, n_keep=6):
    """A draft row that follows the target row p except on its n_keep most
    likely tokens (other than the favour tokens, the drafts), which keep a
    fifth of their mass; the favour tokens take the rest.  After a rejection
    the adjusted distribution max(p - q, 0) is then supported on those n_keep
    tokens only, so the resample lands well inside one of a few wide CDF
    steps even where p itself is nearly flat (T = 1 over a large vocabulary).
    Elsewhere q is p scaled up by a relative margin of 0.3 times the kept
    mass: p - q then stays negative there however either side rounds p (the
    reference's sequential f32 softmax sum over 152064 entries is off by
    ~1e-5 relative; the kept mass is a few 1e-3 or more)."""
    p = np.asarray(p, np.float64)
    q = p.copy()
    order = [int(x) for x in np.argsort(-p, kind="stable") if int(x) not in set(int(f) for f in favour)]
    S = np.array(order[:n_keep])
    pk = float(np.sum(p[S]))
    rest = np.ones(p.size, bool)
    rest[S] = False
    rest[np.asarray(favour)] = False
    q[rest] *= 1.0 + 0.3 * pk
    q[S] *= 0.2
    extra = 1.0 - float(np.sum(q))  # about half the kept mass
    assert extra > 0
    for f in favour:
        q[f] += extra / len(favour)
    return q.astype(np.float32)


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
    for trial in range(10 if T > 0 else 6):
        q = _draft_rows(rng, k, V)
        if trial >= 6:
            # draft rows equal to the target's except on a few tokens, the
            # drafts favoured: rejections resample from a few wide CDF steps
            drafts = [int(v) for v in rng.integers(0, V, k)]
            rows = hd.batched_logits(drafts)
            hd.rollback_to(L)
            for i in range(k):
                q[i] = _peaked_q(O.softmax_t(rows[i], T), [drafts[i]], rng)
        elif trial % 2 == 0:
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
    # at T = 1 the tiny model's rows are nearly flat over 32000 tokens, so a
    # draw from them sits within rounding of a CDF boundary (checked for
    # validity); the peaked draft rows give exact cases at every temperature
    assert kinds["exact"] >= (4 if T == 1.0 else 8), kinds


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
    for trial in range(5 if use_t2d else 3):
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
        if trial >= 3:
            # draft rows that are the masked target rows but for a few tokens,
            # the node's children favoured (exact resamples at any temperature)
            for i in range(n):
                kids = [tree.token_at(c) for c in range(1, n) if tree.parent_of(c) == i]
                r = np.array(rows[i], np.float32)
                r[~mask] = -np.inf
                qt = _peaked_q(O.softmax_t(r, T), kids or [int(d2t[0])], rng) if T > 0 else None
                if qt is not None:
                    q_d[i] = qt[d2t]
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
    # without the t2d mask the 24000 unreachable target tokens keep their
    # nearly flat T = 1 mass, so those draws are checked for validity only
    if T != 1.0 or use_t2d:
        assert kinds["exact"] >= 2, kinds


@pytest.mark.parametrize("T", [1.0, 0.3])
def test_rejection_tree_without_replacement_matches_oracle(hip, T):
    """The without-replacement sibling rule (q zeroed at rejected tokens and
    renormalised) on the device against the oracle, over a tree whose
    siblings are distinct tokens."""
    ocfg, hd, prefix = _pair(hip, prefix_len=40)
    V = ocfg.vocab
    rng = np.random.default_rng(321)
    L = len(prefix)
    kinds = {"exact": 0, "boundary": 0}
    for trial in range(4):
        cands = [[int(v) for v in rng.choice(V, b, replace=False)] for b in (5, 3, 2, 1)]
        tree = O.build_cartesian_tree(prefix[-1], cands)
        n = len(tree)
        rows, _ = hd.tree_logits_keep_kv((tree.tokens(), tree.parents()))
        hd.rollback_to(L)
        q = _draft_rows(rng, n, V)
        if trial % 2:
            for i in range(n):
                kids = [tree.token_at(c) for c in range(1, n) if tree.parent_of(c) == i]
                q[i] = _peaked_q(O.softmax_t(rows[i], T), kids or [0], rng)
        u = [float(x) for x in rng.random(n, dtype=np.float32)]
        path, tok, used = hd.verify_rejection_tree((tree.tokens(), tree.parents()), q, list(range(n)), u, T,
                                                   without_replacement=True)
        hd.rollback_to(L)
        opath, otok, oused = O.rejection_tree_accept(tree, list(rows), list(q), list(range(n)), u, T,
                                                     without_replacement=True)
        kind = _check_walk(path, tok if tok >= 0 else None, opath, otok, tree, list(rows), list(q), list(range(n)),
                           u, T, wor=True)
        kinds[kind] += 1
        if kind == "exact":
            assert used == oused
    assert kinds["exact"] >= 1, kinds


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


QWEN_SMALL = dict(arch="qwen2", n_kv_heads=4, mix="q5k_q80", n_layers=2, rms_eps=1e-6, rope_theta=1e6)


def test_rejection_device_rows_match_host_rows(hip):
    """The device-resident draft-row entry points run the same walk as the
    host-row ones: identical results, uniform for uniform; a host pointer is
    refused before the verify pass touches any state."""
    ocfg, hd, prefix = _pair(hip, **QWEN_SMALL)
    V, k = ocfg.vocab, 8
    rng = np.random.default_rng(5)
    L = len(prefix)
    for T in (1.0, 0.3, 0.0):
        for _ in range(3):
            q = _draft_rows(rng, k, V)
            drafts = [int(O.sample_u(q[i], float(rng.random()))) for i in range(k)]
            u = [float(x) for x in rng.random(k + 1, dtype=np.float32)]
            host = hd.verify_rejection_linear(drafts, q, u, T)
            hd.rollback_to(L)
            with hip.DeviceArray(q) as qd:
                dev = hd.verify_rejection_linear_device(drafts, qd.ptr, u, T)
            hd.rollback_to(L)
            assert dev == host, (T, dev, host)
    # a tree whose draft rows live in a d2t draft vocabulary
    Vd = 8000
    d2t = _seeded_d2t(rng, Vd, V)
    hd.set_d2t(d2t)
    cands = [[int(d2t[v]) for v in rng.choice(Vd, b, replace=False)] for b in (4, 3, 2, 1)]
    toks, pars = hip.tree_prune(hip.tree_cartesian(prefix[-1], cands),
                                [list(np.log(np.full(len(c), 1.0 / len(c))).astype(np.float32)) for c in cands], 24)
    n = len(toks)
    q_d = _draft_rows(rng, n, Vd)
    u = [float(x) for x in rng.random(n, dtype=np.float32)]
    for use_t2d in (False, True):
        host = hd.verify_rejection_tree((toks, pars), q_d, list(range(n)), u, 1.0, use_t2d)
        hd.rollback_to(L)
        with hip.DeviceArray(q_d) as qd:
            dev = hd.verify_rejection_tree_device((toks, pars), qd.ptr, n, Vd, list(range(n)), u, 1.0, use_t2d)
        hd.rollback_to(L)
        assert dev == host, (use_t2d, dev, host)
    q = _draft_rows(rng, 2, V)
    with pytest.raises(hip.ArgError):
        hd.verify_rejection_linear_device([1, 2], q.ctypes.data, [0.5, 0.5, 0.5], 1.0)
    with pytest.raises(hip.ArgError):
        hd.verify_rejection_tree_device((toks, pars), q_d.ctypes.data, n, Vd, list(range(n)), u, 1.0)
    assert hd.history() == prefix and hd.cache_len() == L
