"""Pins the oracle's tree utilities and acceptance rules with the reference's
own unit tests (restated from the Rust sources cited per test) and with
statistical checks of the Leviathan rule."""
import numpy as np
import pytest

import oracle as O
from oracle import DraftTree

# ---- tree.rs:288-482 --------------------------------------------------------
BRANCH = [(0, 100), (0, 11), (0, 12), (1, 23), (1, 24), (2, 35)]


def test_linear_tree_is_a_chain():  # tree.rs:289-299
    t = DraftTree.linear(10, [20, 30, 40])
    assert len(t) == 4 and t.tokens() == [10, 20, 30, 40]
    assert [t.parent_of(i) for i in range(4)] == [0, 0, 1, 2]
    assert t.depth_of(3) == 3
    assert t.paths() == [[0, 1, 2, 3]]


def test_branching_tree_paths():  # tree.rs:301-324
    t = DraftTree.from_parent_table(BRANCH)
    assert len(t) == 6 and t.depth_of(3) == 2 and t.depth_of(5) == 2
    assert sorted(t.paths(), key=lambda p: (len(p), p)) == [[0, 1, 3], [0, 1, 4], [0, 2, 5]]


def test_linear_mask_is_lower_triangular():  # tree.rs:326-337
    m = DraftTree.linear(10, [20, 30, 40]).attention_mask_bool()
    assert all(m[i][j] == (j <= i) for i in range(4) for j in range(4))


def test_branching_mask_blocks_siblings():  # tree.rs:339-355
    m = DraftTree.from_parent_table(BRANCH).attention_mask_bool()
    assert m[3][0] and m[3][1] and m[3][3] and not m[3][2] and not m[3][4] and not m[3][5]
    assert m[5][0] and m[5][2] and m[5][5] and not m[5][1] and not m[5][3] and not m[5][4]


def test_position_ids_offset_by_prefix():  # tree.rs:357-362
    assert DraftTree.linear(0, [1, 2, 3]).position_ids(7) == [7, 8, 9, 10]


def test_rejects_bad_parent_tables():  # tree.rs:364-374
    with pytest.raises(ValueError):
        DraftTree.from_parent_table([(0, 0), (5, 1)])
    with pytest.raises(ValueError):
        DraftTree.from_parent_table([])


def test_path_to_walks_root_first():  # tree.rs:376-380
    assert DraftTree.from_parent_table([(0, 0), (0, 1), (1, 2), (2, 3)]).path_to(3) == [0, 1, 2, 3]


def test_full_attention_bias_prefix_and_tree():  # tree.rs:436-460
    b = DraftTree.linear(0, [1, 2]).full_attention_bias(5)
    assert b.shape == (3, 8)
    assert np.all(b[:, :5] == 0)
    for i in range(3):
        for j in range(3):
            assert (b[i, 5 + j] == 0) if j <= i else (b[i, 5 + j] == -np.inf)


def test_ancestor_mask_words_match_bool_mask():
    rng = np.random.default_rng(2)
    for n in (1, 6, 63, 64, 65, 128):
        par = [0] + [int(rng.integers(0, i)) for i in range(1, n)]
        t = DraftTree(list(range(n)), par)
        w = O.ancestor_masks(t)
        mb = t.attention_mask_bool()
        for i in range(n):
            for j in range(n):
                assert bool((int(w[i, j // 64]) >> (j % 64)) & 1) == mb[i][j]


# ---- medusa.rs ------------------------------------------------------------------
def test_top_k_indices_stable_tie_break():  # medusa.rs:846-858
    assert O.top_k_indices([0.1, 0.5, 0.5, 0.3, 0.5], 3) == [1, 2, 4]
    assert O.top_k_indices([1.0, 2.0], 5) == [1, 0]


def test_cartesian_topology():  # medusa.rs:860-926 (size 1 + sum prod k)
    t = O.build_cartesian_tree(42, [[10, 20], [30, 40]])
    assert len(t) == 7
    assert t.tokens() == [42, 10, 20, 30, 40, 30, 40]
    assert [t.parent_of(i) for i in range(7)] == [0, 0, 0, 1, 1, 2, 2]
    big = O.build_cartesian_tree(1, [list(range(k)) for k in (4, 3, 2, 2, 1, 1)])
    assert len(big) == 1 + 4 + 12 + 24 + 48 + 48 + 48


# ---- eagle.rs prune (eagle.rs:894-950) ---------------------------------------------
def test_prune_keeps_root_and_best_path():
    cart = O.build_cartesian_tree(42, [[10, 20], [30, 40]])
    pr = O.prune_cartesian_tree(cart, [[-0.1, -2.0], [-0.2, -3.0]], 4)
    assert 1 <= len(pr) <= 4 and pr.token_at(0) == 42
    toks = pr.tokens()
    assert 10 in toks and 30 in toks
    # BFS order is preserved: every parent precedes its child
    assert all(pr.parent_of(i) < i for i in range(1, len(pr)))


def test_prune_returns_full_tree_when_under_limit():
    cart = O.build_cartesian_tree(1, [[2], [3]])
    assert len(O.prune_cartesian_tree(cart, [[-0.1], [-0.2]], 100)) == 3


def test_prune_60_of_185_keeps_ancestor_closure():
    rng = np.random.default_rng(4)
    steps = (4, 3, 2, 2, 1, 1)
    cands = [[int(v) for v in rng.integers(0, 1000, k)] for k in steps]
    lps = [sorted((-rng.exponential(size=k)).astype(np.float32).tolist(), reverse=True) for k in steps]
    full = O.build_cartesian_tree(7, cands)
    pr = O.prune_cartesian_tree(full, lps, 60)
    assert len(pr) == 60 and max(pr.depth_of(i) for i in range(60)) <= 6


# ---- eagle3.rs t2d (eagle3.rs:807-825) -----------------------------------------------
def test_t2d_mask_derives_from_d2t():
    inv, mask = O.d2t_maps([0, 3, 5, 9, -1], 10)
    assert mask.tolist() == [True, False, False, True, False, True, False, False, False, True]
    assert inv == {0: 0, 3: 1, 5: 2, 9: 3}


# ---- greedy tree walk (eagle.rs:618-661) -------------------------------------------
def _onehot_rows(n, V, am):
    rows = np.zeros((n, V), np.float32)
    for i, a in enumerate(am):
        rows[i, a] = 1.0
    return rows


def test_greedy_walk_longest_path_and_earliest_leaf_tie():
    # root -> {1: tok 5, 2: tok 6}; 1 -> {3: tok 7}; 2 -> {4: tok 8}
    t = DraftTree.from_parent_table([(0, 9), (0, 5), (0, 6), (1, 7), (2, 8)])
    V = 16
    # target says: after root 5, after node1 7, after node2 8 -> both depth-2 paths fully accepted?
    # root argmax can only be one token: 5 -> path [0,1,3] accepted (2 edges)
    best, bonus = O.greedy_tree_accept(t, _onehot_rows(5, V, [5, 7, 8, 11, 12]))
    assert best == [0, 1, 3] and bonus == 11
    # two leaves accept equally far (1 edge each is impossible from one root argmax), so test the
    # tie on a tree where two leaves share the accepted prefix: root -> 1 -> {3, 4}
    t2 = DraftTree.from_parent_table([(0, 9), (0, 5), (1, 7), (1, 7)])
    best, bonus = O.greedy_tree_accept(t2, _onehot_rows(4, V, [5, 7, 3, 4]))
    assert best == [0, 1, 2] and bonus == 3  # earliest leaf (node 2) wins the tie


def test_greedy_walk_nothing_accepted():
    t = DraftTree.from_parent_table([(0, 9), (0, 5), (1, 7)])
    best, bonus = O.greedy_tree_accept(t, _onehot_rows(3, 16, [4, 7, 1]))
    assert best == [0] and bonus == 4


def test_argmax_fold_semantics():
    assert O.argmax_fold(np.array([0.1, 5.0, 0.1, 4.99], np.float32)) == 1
    assert O.argmax_fold(np.array([1.0, 3.0, 3.0], np.float32)) == 1  # first max
    assert O.argmax_fold(np.array([np.nan, 2.0, np.nan, 2.0], np.float32)) == 1  # NaN skipped
    assert O.argmax_fold(np.array([-np.inf, -np.inf], np.float32)) == 0
    assert O.argmax_fold(np.array([np.nan, np.nan], np.float32)) == 0


# ---- vanilla.rs / tokens.rs unit tests ---------------------------------------------
def test_rejection_step_kats():  # vanilla.rs:379-403
    for u in range(101):
        assert O.rejection_step(0.4, 0.8, u / 100.0)
    assert not O.rejection_step(0.8, 0.4, 0.6)
    assert O.rejection_step(0.8, 0.4, 0.4)
    assert O.rejection_step(0.0, 0.0, 0.99)  # q <= 0 accepts


def test_adjusted_distribution_kats():  # vanilla.rs:405-430
    adj = O.adjusted_distribution(np.array([0.5, 0.3, 0.2]), np.array([0.1, 0.4, 0.5]))
    assert np.allclose(adj, [1.0, 0.0, 0.0], rtol=1e-6)
    with pytest.raises(ValueError):
        O.adjusted_distribution(np.array([0.5, 0.5]), np.array([0.5, 0.5]))
    with pytest.raises(ValueError):
        O.adjusted_distribution(np.array([0.5, 0.5]), np.array([1.0]))


def test_softmax_kats():  # tokens.rs:128-145
    p = O.softmax_t(np.array([1.0, 2.0, 3.0], np.float32), 1.0)
    assert abs(float(p.sum()) - 1.0) < 1e-5
    assert O.softmax_t(np.array([0.1, 5.0, 0.1, 4.99], np.float32), 0.0).tolist() == [0, 1, 0, 0]
    with pytest.raises(ValueError):
        O.softmax_t(np.array([1.0], np.float32), -1.0)


def test_sample_respects_mass_and_frequencies():  # tokens.rs:159-177
    rng = np.random.default_rng(7)
    probs = np.array([0.0, 0.0, 1.0, 0.0], np.float32)
    assert all(O.sample_u(probs, float(u)) == 2 for u in rng.random(1000, dtype=np.float32))
    probs = np.array([0.1, 0.2, 0.3, 0.4], np.float32)
    n = 40000
    counts = np.bincount([O.sample_u(probs, float(u)) for u in rng.random(n, dtype=np.float32)], minlength=4)
    assert np.allclose(counts / n, probs, rtol=0.05)


def _tv(a, b):
    return 0.5 * float(np.abs(np.asarray(a) - np.asarray(b)).sum())


@pytest.mark.parametrize("target,draft,trials,bound", [
    ([0.5, 0.3, 0.15, 0.05], [0.25] * 4, 20000, 0.025),          # vanilla.rs:478-500
    ([0.7, 0.15, 0.1, 0.05], [0.05, 0.1, 0.15, 0.7], 20000, 0.03),  # vanilla.rs:502-520
    ([0.4, 0.3, 0.2, 0.1], [0.4, 0.3, 0.2, 0.1], 10000, 0.025),    # vanilla.rs:522-538
])
def test_leviathan_output_matches_target(target, draft, trials, bound):
    """First committed token of the explicit-uniform Leviathan walk is
    distributed as the target (fixed-distribution mocks, T=1)."""
    rng = np.random.default_rng(11)
    V = len(target)
    tl = np.log(np.asarray(target, np.float32) + 1e-30).astype(np.float32)
    q = np.asarray(draft, np.float32)
    counts = np.zeros(V)
    for _ in range(trials):
        u = rng.random(8, dtype=np.float32)
        d0 = O.sample_u(q, float(u[7]))
        commits, _, _ = O.rejection_linear_accept([tl, tl], [q], [d0], [float(x) for x in u[:2]], 1.0)
        counts[commits[0]] += 1
    assert _tv(counts / trials, target) < bound


def test_leviathan_never_emits_zero_mass_token():  # vanilla.rs:540-570
    rng = np.random.default_rng(99)
    tl = np.array([np.log(0.6), np.log(0.4), -np.inf, -np.inf], np.float32)
    q = np.full(4, 0.25, np.float32)
    for _ in range(2000):
        u = rng.random(3, dtype=np.float32)
        d0 = O.sample_u(q, float(u[2]))
        commits, _, _ = O.rejection_linear_accept([tl, tl], [q], [d0], [float(x) for x in u[:2]], 1.0)
        assert commits[0] < 2


# ---- commit composition with EOS (eagle.rs:664-732, eagle3.rs:758-782) ---------------
def _eos_tree():
    # root 5 -> {1: 10, 2: 11}; 1 -> {3: 12, 4: 13}; 3 -> {5: 14}; 2 -> {6: 15}
    return O.DraftTree([5, 10, 11, 12, 13, 14, 15], [0, 0, 0, 1, 1, 3, 2])


def test_commit_without_eos_keeps_path_and_bonus_in_tree():
    t = _eos_tree()
    best = [0, 1, 3]
    com, stop, keep, bn = O.greedy_tree_commit(t, best, 14, eos=[99])
    assert com == [10, 12, 14] and not stop and bn == 5 and keep == [0, 1, 3, 5]
    com, stop, keep, bn = O.greedy_tree_commit(t, best, 14, eos=[99], strict=True)
    assert com == [10, 12, 14] and not stop and bn is None and keep == [0, 1, 3]
    com, stop, keep, bn = O.greedy_tree_commit(t, best, 77, eos=[])
    assert com == [10, 12, 77] and keep == [0, 1, 3] and bn is None


def test_commit_eos_in_path_truncates_and_skips_bonus():
    t = _eos_tree()
    com, stop, keep, bn = O.greedy_tree_commit(t, [0, 1, 3, 5], 40, eos=[12, 1000])
    assert com == [10, 12] and stop and keep == [0, 1, 3] and bn is None
    # EOS at the first accepted draft
    com, stop, keep, bn = O.greedy_tree_commit(t, [0, 1, 3, 5], 40, eos=[10, 14])
    assert com == [10] and stop and keep == [0, 1] and bn is None


def test_commit_eos_bonus_stops_but_keeps_path():
    t = _eos_tree()
    # the bonus is EOS and also a child of the deepest node: the path is kept,
    # the bonus node joins it (no EOS among the path's own tokens)
    com, stop, keep, bn = O.greedy_tree_commit(t, [0, 1, 3], 14, eos=[14])
    assert com == [10, 12, 14] and stop and keep == [0, 1, 3, 5] and bn == 5
    com, stop, keep, bn = O.greedy_tree_commit(t, [0], 11, eos=[11])
    assert com == [11] and stop and keep == [0, 2] and bn == 2
