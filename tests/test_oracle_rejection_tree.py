"""The tree rejection walk of the oracle (the rule the device walk follows).

The reference has no tree-level rejection rule (eagle.rs:739-740 and
eagle3.rs:789 ignore the temperature), so this rule is pinned by what the
mathematics fixes rather than by a reference vector:
  * on a chain it is the reference's linear walk (vanilla.rs:178-210), step for
    step and uniform for uniform;
  * with sibling candidates drawn i.i.d. from the node's draft row, the first
    committed token is distributed as the target (multi-candidate speculative
    sampling preserves the target distribution), checked by total variation
    like the reference's own statistical tests (vanilla.rs:478-538);
  * a candidate with zero target mass is never emitted (vanilla.rs:540-570).
A planted mistake in the rule (no adjustment between siblings, or the
adjustment against the wrong row) fails the distribution test.
"""
import numpy as np
import pytest

import oracle as O


def _tv(a, b):
    return 0.5 * float(np.abs(np.asarray(a) - np.asarray(b)).sum())


@pytest.mark.parametrize("seed", range(6))
@pytest.mark.parametrize("temperature", [1.0, 0.7, 0.0])
def test_chain_equals_linear_walk(seed, temperature):
    rng = np.random.default_rng(seed)
    V, k = 12, 4
    rows = [rng.standard_normal(V).astype(np.float32) * 2 for _ in range(k + 1)]
    q = [np.asarray(rng.dirichlet(np.ones(V)), np.float32) for _ in range(k)]
    drafts = [int(O.sample_u(q[i], float(rng.random()))) for i in range(k)]
    for trial in range(20):
        u = [float(x) for x in rng.random(k + 1, dtype=np.float32)]
        for max_commit in (None, 2):
            commits, n_acc, used = O.rejection_linear_accept(rows, q, drafts, u, temperature, max_commit)
            tree = O.DraftTree.linear(7, drafts)
            path, fin, used_t = O.rejection_tree_accept(tree, rows, q, list(range(k)) + [-1], u, temperature,
                                                        max_commit=max_commit)
            assert [tree.token_at(i) for i in path[1:]] + ([fin] if fin is not None else []) == commits
            assert len(path) - 1 == n_acc and used_t == used


def _first_token_distribution(p, q, n_children, trials, rng, rule=O.rejection_tree_accept):
    V = len(p)
    logits = np.log(np.asarray(p, np.float64) + 1e-30).astype(np.float32)
    qv = np.asarray(q, np.float32)
    counts = np.zeros(V)
    for _ in range(trials):
        u = rng.random(n_children + 1 + n_children, dtype=np.float32)
        cands = [int(O.sample_u(qv, float(u[n_children + 1 + j]))) for j in range(n_children)]
        tree = O.DraftTree([99] + cands, [0] * (n_children + 1))
        rows = [logits] + [logits] * n_children
        path, fin, _ = rule(tree, rows, [qv], [0] + [-1] * n_children, [float(x) for x in u[:n_children + 1]], 1.0)
        tok = tree.token_at(path[1]) if len(path) > 1 else fin
        counts[tok] += 1
    return counts / trials


@pytest.mark.parametrize("p,q,nc", [
    ([0.5, 0.3, 0.15, 0.05], [0.25] * 4, 3),
    ([0.7, 0.15, 0.1, 0.05], [0.05, 0.1, 0.15, 0.7], 3),
    ([0.1, 0.2, 0.3, 0.4], [0.4, 0.3, 0.2, 0.1], 2),
    ([0.05, 0.05, 0.6, 0.3], [0.3, 0.3, 0.2, 0.2], 4),
])
def test_multi_candidate_preserves_target(p, q, nc):
    rng = np.random.default_rng(5)
    freq = _first_token_distribution(p, q, nc, 12000, rng)
    assert _tv(freq, p) < 0.03, freq


def _no_adjust_rule(tree, target_rows, q_rows, q_row_of, uniforms, temperature, t2d_mask=None, max_commit=None):
    """A planted mistake: siblings all tested against the unadjusted p."""
    p = O.softmax_t(np.asarray(target_rows[0], np.float32), temperature)
    q = np.asarray(q_rows[0], np.float32)
    used = 0
    for c in range(1, len(tree)):
        u = uniforms[used]
        used += 1
        if O.rejection_step(float(q[tree.token_at(c)]), float(p[tree.token_at(c)]), u):
            return [0, c], None, used
    return [0], O.sample_u(O.adjusted_distribution(p, q), uniforms[used]), used + 1


def test_planted_mistake_is_detected():
    rng = np.random.default_rng(5)
    p, q = [0.7, 0.15, 0.1, 0.05], [0.05, 0.1, 0.15, 0.7]
    freq = _first_token_distribution(p, q, 3, 12000, rng, rule=_no_adjust_rule)
    assert _tv(freq, p) > 0.05


def test_zero_mass_candidates_never_emitted():
    rng = np.random.default_rng(99)
    p = [0.6, 0.4, 0.0, 0.0]
    freq = _first_token_distribution(p, [0.25] * 4, 3, 3000, rng)
    assert freq[2] == 0 and freq[3] == 0


def test_t2d_mask_removes_unreachable_targets():
    rng = np.random.default_rng(3)
    V = 10
    _, mask = O.d2t_maps([0, 3, 5, 9], V)
    row = rng.standard_normal(V).astype(np.float32)
    q = np.zeros(V, np.float32)
    q[[0, 3, 5, 9]] = 0.25
    tree = O.DraftTree([1], [0])
    for _ in range(200):
        _, fin, _ = O.rejection_tree_accept(tree, [row], [q], [-1], [float(rng.random())], 1.0, t2d_mask=mask)
        assert mask[fin]


# ---- siblings drawn without replacement ---------------------------------------------
def _wor_candidates(qv, n, uvals):
    """n distinct tokens drawn sequentially without replacement from q."""
    q = np.asarray(qv, np.float64).copy()
    out = []
    for j in range(n):
        c = np.cumsum(q) / q.sum()
        t = int(min(np.searchsorted(c, float(uvals[j]), side="right"), len(c) - 1))
        while q[t] <= 0:  # drift past the last positive entry
            t -= 1
        out.append(t)
        q[t] = 0.0
    return out


def _first_token_distribution_wor(p, q, n_children, trials, rng, wor=True):
    V = len(p)
    logits = np.log(np.asarray(p, np.float64) + 1e-30).astype(np.float32)
    qv = np.asarray(q, np.float32)
    counts = np.zeros(V)
    for _ in range(trials):
        u = rng.random(n_children + 1, dtype=np.float32)
        cands = _wor_candidates(qv, n_children, rng.random(n_children))
        tree = O.DraftTree([99] + cands, [0] * (n_children + 1))
        rows = [logits] * (n_children + 1)
        path, fin, _ = O.rejection_tree_accept(tree, rows, [qv], [0] + [-1] * n_children, [float(x) for x in u],
                                               1.0, without_replacement=wor)
        tok = tree.token_at(path[1]) if len(path) > 1 else fin
        counts[tok] += 1
    return counts / trials


@pytest.mark.parametrize("p,q,nc", [
    ([0.5, 0.3, 0.15, 0.05], [0.25] * 4, 3),
    ([0.7, 0.15, 0.1, 0.05], [0.05, 0.1, 0.15, 0.7], 3),
    ([0.1, 0.2, 0.3, 0.4], [0.4, 0.3, 0.2, 0.1], 2),
    ([0.05, 0.05, 0.6, 0.2, 0.1], [0.3, 0.3, 0.2, 0.1, 0.1], 4),
])
def test_without_replacement_rule_preserves_target(p, q, nc):
    """Distinct siblings (drawn without replacement from q) with q zeroed at
    each rejected token and renormalised: the committed token follows p."""
    rng = np.random.default_rng(11)
    freq = _first_token_distribution_wor(p, q, nc, 12000, rng)
    assert _tv(freq, p) < 0.03, freq


def test_iid_rule_on_distinct_siblings_is_biased():
    """The i.i.d. rule applied to siblings drawn without replacement (the
    mismatch the sibling flag exists for) moves the distribution off p."""
    rng = np.random.default_rng(11)
    p, q = [0.05, 0.05, 0.6, 0.2, 0.1], [0.3, 0.3, 0.2, 0.1, 0.1]
    freq = _first_token_distribution_wor(p, q, 4, 12000, rng, wor=False)
    assert _tv(freq, p) > 0.05, freq


def test_without_replacement_chain_is_the_linear_walk():
    """One child per node: nothing is ever renormalised, both rules agree."""
    rng = np.random.default_rng(12)
    V, k = 12, 4
    rows = [rng.standard_normal(V).astype(np.float32) * 2 for _ in range(k + 1)]
    q = [np.asarray(rng.dirichlet(np.ones(V)), np.float32) for _ in range(k)]
    drafts = [int(O.sample_u(q[i], float(rng.random()))) for i in range(k)]
    tree = O.DraftTree.linear(7, drafts)
    for _ in range(30):
        u = [float(x) for x in rng.random(k + 1, dtype=np.float32)]
        a = O.rejection_tree_accept(tree, rows, q, list(range(k)) + [-1], u, 1.0)
        b = O.rejection_tree_accept(tree, rows, q, list(range(k)) + [-1], u, 1.0, without_replacement=True)
        assert a == b
