"""Host-side draft-tree builders of the C ABI (no GPU needed): the Cartesian
builder (methods/medusa.rs:172-193) and the pruning rule (methods/eagle.rs:763-845).

Pinned by the reference's own unit tests (medusa.rs:861-926, eagle.rs:894-950),
by a hand-derived known answer, and against the oracle's restatement on the
verify-tree shapes the benchmarks use."""
import numpy as np
import pytest

import oracle as O


@pytest.fixture(scope="module")
def S():
    import speculate_hip
    speculate_hip.load_library()
    return speculate_hip


def test_greedy_chain_is_linear(S):
    # medusa.rs:861-873: one candidate per head gives the chain [7, 10, 20, 30]
    t, p = S.tree_cartesian(7, [[10], [20], [30]])
    assert list(t) == [7, 10, 20, 30] and list(p) == [0, 0, 1, 2]


def test_cartesian_layout_and_masks(S):
    # medusa.rs:876-898: 2 x 2 candidates -> 1 + 2 + 4 nodes, four depth-2 paths
    t, p = S.tree_cartesian(0, [[10, 11], [20, 21]])
    assert len(t) == 7
    tree = O.DraftTree(list(t), list(p))
    paths = tree.paths()
    assert len(paths) == 4 and all(len(x) == 3 for x in paths)
    # medusa.rs:901-925: layout 0 root, 1/2 = 10/11, 3/4 = 20 under 1/2
    t, p = S.tree_cartesian(0, [[10, 11], [20]])
    assert list(t) == [0, 10, 11, 20, 20] and list(p) == [0, 0, 0, 1, 2]
    m = O.DraftTree(list(t), list(p)).attention_mask_bool()
    assert m[3][0] and m[3][1] and m[3][3] and not m[3][2] and not m[3][4]
    assert m[4][0] and m[4][2] and m[4][4] and not m[4][1] and not m[4][3]


def test_prune_known_answer(S):
    # eagle.rs:894-929, plus the exact result: scores 10:-0.1, 10>30:-0.3,
    # 20:-2.0, 20>30:-2.2, 10>40:-3.1, 20>40:-5.0; the best 3 are nodes 1, 3, 2.
    full = S.tree_cartesian(42, [[10, 20], [30, 40]])
    t, p = S.tree_prune(full, [[-0.1, -2.0], [-0.2, -3.0]], 4)
    assert list(t) == [42, 10, 20, 30] and list(p) == [0, 0, 0, 1]


def test_prune_under_limit_is_identity(S):
    # eagle.rs:931-949
    full = S.tree_cartesian(1, [[2], [3]])
    t, p = S.tree_prune(full, [[-0.1], [-0.2]], 100)
    assert list(t) == [1, 2, 3] and list(p) == [0, 0, 1]


def test_prune_ties_keep_bfs_order(S):
    # equal scores: the stable sort keeps the earlier BFS node
    full = S.tree_cartesian(5, [[1, 2, 3]])
    t, p = S.tree_prune(full, [[-1.0, -1.0, -1.0]], 3)
    assert list(t) == [5, 1, 2]


def test_prune_ancestor_closure(S):
    # a deep node that outscores its own ancestor pulls the ancestor back in
    full = S.tree_cartesian(9, [[1, 2], [3]])   # 0; 1,2; 3 under 1, 4 under 2
    t, p = S.tree_prune(full, [[-0.1, -5.0], [4.0]], 2)
    # scores: 1: -0.1, 2: -5.0, 1>3: 3.9, 2>3: -1.0; only node 3 is selected
    # (max_total - 1 = 1) and node 1 returns by the closure
    assert list(t) == [9, 1, 3] and list(p) == [0, 0, 1]


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_prune_matches_oracle_on_verify_trees(S, seed):
    """The 60-node (4,3,2,2,1,1) tree and a 64-node depth-7 tree, seeded."""
    rng = np.random.default_rng(seed)
    for branching, keep in (((4, 3, 2, 2, 1, 1), 60), ((4, 3, 2, 2, 2, 1, 1), 64)):
        cands = [[int(v) for v in rng.integers(0, 128256, b)] for b in branching]
        lps = [[float(v) for v in np.sort(np.log(rng.dirichlet(np.ones(b))))[::-1].astype(np.float32)]
               for b in branching]
        t, p = S.tree_cartesian(123, cands)
        ref = O.build_cartesian_tree(123, cands)
        assert list(t) == ref.tokens() and list(p) == ref.parents()
        pt, pp = S.tree_prune((t, p), lps, keep)
        pref = O.prune_cartesian_tree(ref, lps, keep)
        assert list(pt) == pref.tokens() and list(pp) == pref.parents()
        assert len(pt) == keep
        assert max(O.DraftTree(list(pt), list(pp)).depth_of(i) for i in range(len(pt))) <= len(branching)


def test_prune_rejects_bad_tables(S):
    full = S.tree_cartesian(1, [[2, 3], [4]])
    with pytest.raises(S.ArgError):
        S.tree_prune(full, [[-0.1], [-0.2]], 2)   # rank 1 has no log-prob
    with pytest.raises(S.SamplingError):
        S.tree_prune((np.array([1, 2], np.uint32), np.array([0, 1], np.uint32)), [[-0.1]], 1)
