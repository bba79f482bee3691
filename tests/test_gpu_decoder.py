"""Decoder-level GPU parity (through the C ABI) against the oracle decoder.

Contract (per the path's spec): logits and hidden states within 1e-2
relative (max |a-b| / max |b| per row block); first-max argmaxes and greedy
acceptance identical to the oracle's wherever the oracle's top-2 margin
exceeds twice the row's actual device/oracle difference -- such near ties are
counted and bounded, not skipped -- and the device walk always equal to the
walk over the device's own argmaxes; KV compaction bit-exact (a pure row
copy).
"""
import numpy as np
import pytest

import oracle as O
from _fullwidth import argmax_agreement
from _models import MIX_IDS, hip_cfg, oracle_cfg, rel_err

pytestmark = pytest.mark.gpu

TOL = 1e-2
_WEIGHTS = {}


def make_pair(hip, prefix_len=128, seed=1, **over):
    ocfg = oracle_cfg(**over)
    key = tuple(sorted(over.items()))
    if key not in _WEIGHTS:
        _WEIGHTS[key] = O.OracleModel(ocfg).raw
    om = O.OracleModel(ocfg, _WEIGHTS[key])
    od = O.OracleDecoder(om)
    hd = hip.HipQuantDecoder(hip_cfg(hip, ocfg))
    hd.synthesize(MIX_IDS[ocfg.mix], ocfg.seed, ocfg.weight_std)
    prefix = [int(v) for v in np.random.default_rng(seed).integers(0, ocfg.vocab, prefix_len)]
    od.observe(prefix)
    hd.observe(prefix)
    return od, hd, prefix


def greedy_chain(od, n):
    """The oracle's own greedy continuation (then restored)."""
    L = len(od.history)
    chain = []
    for _ in range(n):
        g = O.argmax_fold(od.next_logits())
        chain.append(g)
        od.observe([g])
    od.rollback_to(L)
    return chain


def test_observe_and_next_logits(hip):
    od, hd, _ = make_pair(hip)
    a, b = hd.next_logits(), od.next_logits()
    assert rel_err(a, b) < TOL
    argmax_agreement(a[None], b[None], max_near_frac=1.0)
    assert hd.history() == od.history and hd.cache_len() == len(od.history)


def test_batched_logits_and_greedy_linear(hip):
    od, hd, prefix = make_pair(hip)
    chain = greedy_chain(od, 4)
    drafts = [chain[0], chain[1], (chain[2] + 1) % 32000, chain[3]]
    L = len(prefix)
    b = od.batched_logits(drafts)
    a = hd.batched_logits(drafts)
    assert a.shape == b.shape == (5, 32000)
    for i in range(5):
        assert rel_err(a[i], b[i]) < TOL, i
    assert hd.history() == od.history
    # device greedy acceptance == oracle walk on oracle logits; every row's
    # argmax must agree unless the oracle's top-2 margin is within twice the
    # row's device/oracle difference (counted, not skipped)
    near = argmax_agreement(a, b)
    hd.rollback_to(L)
    commits, n_acc = hd.verify_greedy_linear(drafts)
    d_acc, d_bonus = O.greedy_linear_accept(drafts, [O.argmax_fold(r) for r in a])
    assert n_acc == d_acc and commits == drafts[:d_acc] + [d_bonus]
    am = [O.argmax_fold(r) for r in b]
    exp_acc, exp_bonus = O.greedy_linear_accept(drafts, am)
    assert exp_acc == 2
    if not set(near) & set(range(exp_acc + 1)):
        assert n_acc == exp_acc and commits == drafts[:exp_acc] + [exp_bonus]
    # device argmax == host first-max fold of the device logits (bit-exact logic)
    got_am = hd.last_argmax(5)
    assert [int(v) for v in got_am] == [O.argmax_fold(r) for r in a]


def _tree_with_chain(chain, vocab, seed=5):
    rng = np.random.default_rng(seed)
    r = [int(v) for v in rng.integers(0, vocab, 8)]
    cands = [[r[0], chain[0], r[1]], [chain[1], r[2]], [r[3], chain[2]]]
    return cands


def test_tree_keep_kv_verify_and_commit(hip):
    od, hd, prefix = make_pair(hip)
    chain = greedy_chain(od, 3)
    tree = O.build_cartesian_tree(prefix[-1], _tree_with_chain(chain, 32000))
    n = len(tree)
    P = len(prefix) - 1
    lo, ho = od.tree_logits_keep_kv(tree)
    lg, hg = hd.tree_logits_keep_kv(tree)
    for i in range(n):
        assert rel_err(lg[i], lo[i]) < TOL, i
        assert rel_err(hg[i], ho[i]) < TOL, i
    assert hd.cache_len() == P + n
    # device walk on a fresh copy of the state
    hd.rollback_to(len(prefix))
    path, bonus, bnode = hd.verify_greedy_tree(tree)
    am_o = [O.argmax_fold(r) for r in lo]
    best, exp_bonus = O.greedy_tree_accept(tree, lo, am_o)
    near = argmax_agreement(lg, lo)
    # the device walk is the walk over its own argmaxes ...
    dbest, dbonus = O.greedy_tree_accept(tree, None, [int(v) for v in hd.last_argmax(n)])
    assert path == dbest and bonus == dbonus
    # ... and the oracle's, unless a row on it sits on a near tie
    if not set(near) & set(best):
        assert path == best and bonus == exp_bonus
        assert bnode == (O.bonus_in_tree(tree, best[-1], exp_bonus) or -1)
        assert len(best) == 4  # root + the embedded 3-token greedy chain
    # KV compaction: rows [P, P+len(keep)) become the selected tree rows, bit for bit
    keep = path + ([bnode] if bnode >= 0 else [])
    before = {(l, w, h): hd.read_kv_rows(l, w, h, P, n) for l in (0, 3) for w in (0, 1) for h in (0, 7)}
    prefix_rows = hd.read_kv_rows(2, 0, 5, 0, P)
    hd.commit_tree_path(tree, keep)
    for (l, w, h), rows in before.items():
        after = hd.read_kv_rows(l, w, h, P, len(keep))
        assert np.array_equal(after, rows[keep]), (l, w, h)
    assert np.array_equal(hd.read_kv_rows(2, 0, 5, 0, P), prefix_rows)
    assert hd.cache_len() == P + len(keep)
    assert hd.history() == prefix + [tree.token_at(i) for i in keep[1:]]
    # continue: both sides commit the same path and observe the bonus if it was not in the tree
    od.commit_tree_path(tree, keep)
    if bnode < 0:
        od.observe([bonus])
        hd.observe([bonus])
    a, b = hd.next_logits(), od.next_logits()
    assert rel_err(a, b) < TOL


def test_strict_root_row(hip):
    """tree_logits (strict, quantized_llama.rs:262-325) takes row 0 from a
    single-token pass, bit for bit the next_logits row; the fast path's row 0
    comes from the tree-shaped pass and agrees to rounding; every other row is
    the same tree pass in both."""
    od, hd, prefix = make_pair(hip)
    chain = greedy_chain(od, 3)
    tree = O.build_cartesian_tree(prefix[-1], _tree_with_chain(chain, 32000))
    nl = hd.next_logits()  # cached by the 128-row observe pass
    strict = hd.tree_logits(tree)
    assert hd.cache_len() == len(prefix)
    fast, _ = hd.tree_logits_keep_kv(tree)
    for row in (strict[0], fast[0]):
        # different row counts take different K splits; fp16 activations carry
        # the rounding differences through the layers
        assert rel_err(row, nl.astype(np.float64)) < 2e-3
        argmax_agreement(row[None], nl[None], max_near_frac=1.0)  # tree_logits_consistency.rs:74-122
    assert np.array_equal(strict[1:].view(np.uint32), fast[1:].view(np.uint32))
    # the strict row is exactly the single-token (M = 1) pass of the root
    hd.rollback_to(len(prefix) - 1)
    hd.observe([prefix[-1]])
    assert np.array_equal(strict[0].view(np.uint32), hd.next_logits().view(np.uint32))
    # and the strict tree_logits of the oracle (quantized_llama.rs:262-325)
    ostrict = od.tree_logits(tree)
    assert od.cache_len == len(prefix)
    for i in range(len(tree)):
        assert rel_err(strict[i], ostrict[i]) < TOL, i
    argmax_agreement(strict, ostrict)


def test_strict_tree_logits_qwen2_keeps_tree_row(hip):
    """Qwen2QuantDecoder::tree_logits (quantized_qwen2.rs:184-237): the restoring
    one-token pass runs (and refreshes next_logits) but its row is discarded, so
    every row, row 0 included, is the tree pass's row -- bit for bit the
    fast path's rows -- and within the contract of the oracle's Qwen2 rule."""
    over = dict(arch="qwen2", n_kv_heads=2, mix="q5k_q80", n_layers=2, rms_eps=1e-6, rope_theta=1e6)
    od, hd, prefix = make_pair(hip, prefix_len=70, **over)
    chain = greedy_chain(od, 3)
    tree = O.build_cartesian_tree(prefix[-1], _tree_with_chain(chain, 32000))
    strict = hd.tree_logits(tree)
    assert hd.cache_len() == len(prefix) and hd.history() == prefix
    one = hd.next_logits()  # the restoring pass's row
    fast, _ = hd.tree_logits_keep_kv(tree)
    assert np.array_equal(strict.view(np.uint32), fast.view(np.uint32))
    hd.rollback_to(len(prefix) - 1)
    hd.observe([prefix[-1]])
    assert np.array_equal(one.view(np.uint32), hd.next_logits().view(np.uint32))
    ostrict = od.tree_logits(tree)
    assert od.cache_len == len(prefix)
    for i in range(len(tree)):
        assert rel_err(strict[i], ostrict[i]) < TOL, i
    argmax_agreement(strict, ostrict)


def test_error_semantics_keep_state(hip):
    od, hd, prefix = make_pair(hip, prefix_len=16)
    fresh = hip.HipQuantDecoder(hd.cfg)
    fresh.synthesize(0, 1)
    for call in (fresh.next_logits, lambda: fresh.batched_logits([1]), lambda: fresh.last_hidden_state(),
                 lambda: fresh.tree_logits_keep_kv(O.DraftTree.linear(1, [2])),
                 lambda: fresh.commit_tree_path(O.DraftTree.linear(1, [2]), [0])):
        with pytest.raises(hip.SamplingError):
            call()
    with pytest.raises(hip.CacheRollbackError):
        fresh.rollback_to(1)
    with pytest.raises(hip.SamplingError):
        fresh.observe_returning_last_hidden([])
    fresh.observe([])  # empty observe is a no-op
    assert fresh.history() == []
    # root mismatch / bad parent table leave history and cache untouched
    h0, c0 = hd.history(), hd.cache_len()
    with pytest.raises(hip.SamplingError):
        hd.tree_logits_keep_kv(O.DraftTree.linear(prefix[-1] + 1, [3]))
    with pytest.raises(hip.SamplingError):
        hd.tree_logits_keep_kv(([prefix[-1], 5, 6], [0, 2, 0]))
    with pytest.raises(hip.CacheRollbackError):
        hd.rollback_to(len(prefix) + 1)
    assert hd.history() == h0 and hd.cache_len() == c0
    # rollback then next_logits replays the last token (truncate-and-replay path)
    hd.rollback_to(len(prefix) - 3)
    od.rollback_to(len(prefix) - 3)
    assert rel_err(hd.next_logits(), od.next_logits()) < TOL
    with pytest.raises(hip.ArgError):
        hd.observe([40000])


def test_capacity_error_keeps_state(hip):
    """A verify that does not fit the cache fails before anything moves; the
    decoder then continues exactly where it was (model/mod.rs:35-38)."""
    od, hd, prefix = make_pair(hip, prefix_len=126, ctx_len=128)
    with pytest.raises(hip.ArgError):
        hd.batched_logits([1, 2, 3])  # 125 + 4 rows > 128
    assert hd.history() == prefix and hd.cache_len() == len(prefix)
    with pytest.raises(hip.ArgError):
        hd.verify_greedy_linear([1, 2, 3])
    assert hd.history() == prefix and hd.cache_len() == len(prefix)
    assert rel_err(hd.next_logits(), od.next_logits()) < TOL
    hd.observe([9])
    od.observe([9])
    assert rel_err(hd.next_logits(), od.next_logits()) < TOL
    a = hd.batched_logits([4])  # 127 + 1 rows fit
    b = od.batched_logits([4])
    assert rel_err(a, b) < TOL and hd.cache_len() == 128


def test_apply_lm_head_leaves_verify_state(hip):
    """apply_lm_head / embed_tokens take &self (model/mod.rs:148, 182): a
    pending argmax and device acceptance of the last verify survive them."""
    od, hd, prefix = make_pair(hip, prefix_len=40)
    drafts = greedy_chain(od, 3)
    rows = hd.batched_logits(drafts)
    am = [int(v) for v in hd.last_argmax(4)]
    h = np.random.default_rng(3).standard_normal((37, 512)).astype(np.float32)
    out = hd.apply_lm_head(h)
    assert rel_err(out, od.m.lm_head(h)) < TOL
    hd.embed_tokens([1, 2, 3])
    assert [int(v) for v in hd.last_argmax(4)] == am == [O.argmax_fold(r) for r in rows]
    # the 37 rows ran in chunks of 16: each row equals its own 1-row product
    for i in (0, 16, 36):
        assert np.array_equal(hd.apply_lm_head(h[i:i + 1])[0].view(np.uint32), out[i].view(np.uint32))
    assert hd.history() == prefix + drafts


def test_tree_decoder_tensor_contract(hip):
    """Ranks and dtypes of every Decoder / TreeDecoder output are the
    reference's, replayed through the shape handling of its callers:
    hidden rows are rank-1 [hidden] f32 (quantized_llama.rs:190,211,245-247,391);
    run_eagle unsqueezes one to [1, 1, hidden], hands the draft's F16 output to
    apply_lm_head and reads logits.i((0, seq - 1, ..)) (eagle.rs:515-547);
    run_eagle3 lifts the three layer rows to [1, 1, hidden] and concatenates
    them, and embed_tokens of a (1, 1) id tensor is the [1, 1, hidden] input of
    the midlayer's dims3() (eagle3.rs:598-650); apply_lm_head keeps leading
    dims (QMatMul over the last dim, quantized_llama_local.rs:316-318)."""
    od, hd, prefix = make_pair(hip, prefix_len=40)
    H, V = od.m.cfg.hidden, od.m.cfg.vocab
    f32 = np.dtype(np.float32)
    nl = hd.next_logits()
    assert nl.shape == (V,) and nl.dtype == f32
    rows = hd.batched_logits([5, 6])
    assert rows.shape == (3, V) and rows.dtype == f32
    hd.rollback_to(len(prefix))
    # run_eagle: observe_returning_last_hidden -> [hidden] -> [1, 1, hidden]
    th = hd.observe_returning_last_hidden([7])
    assert th.shape == (H,) and th.dtype == f32
    draft_hidden = th[None, None].astype(np.float16)  # a draft's F16 [1, seq, hidden] output
    logits = hd.apply_lm_head(draft_hidden)
    assert logits.shape == (1, 1, V) and logits.dtype == f32
    last = logits[0, draft_hidden.shape[1] - 1]
    assert last.shape == (V,)
    assert np.array_equal(last.view(np.uint32), hd.apply_lm_head(draft_hidden[0, 0].astype(np.float32)).view(np.uint32))
    # the tree's per-node hidden rows; the bonus node's row becomes the next target_hidden (eagle.rs:727)
    tree = O.build_cartesian_tree(7, [[1, 2], [3]])
    lg, hs = hd.tree_logits_keep_kv(tree)
    assert lg.shape == (len(tree), V) and hs.shape == (len(tree), H) and hs.dtype == f32
    assert hs[len(tree) - 1].shape == (H,) and hs[len(tree) - 1][None, None].shape == (1, 1, H)
    hd.rollback_to(len(prefix) + 1)
    strict = hd.tree_logits(tree)
    assert strict.shape == (len(tree), V)
    ls = hd.last_hidden_state()
    assert ls.shape == (H,) and ls.dtype == f32
    # run_eagle3: last_hidden_states_multi -> three [hidden] rows -> [1, 1, 3 hidden]
    fin, mids = hd.last_hidden_states_multi([0, 1, 2])
    assert fin.shape == (H,) and len(mids) == 3 and all(m.shape == (H,) and m.dtype == f32 for m in mids)
    hidden_in = np.concatenate([m.astype(np.float16)[None, None] for m in mids], axis=-1)
    assert hidden_in.shape == (1, 1, 3 * H)
    emb = hd.embed_tokens(np.array([[prefix[-1]]], np.uint32))
    assert emb.shape == (1, 1, H) and emb.dtype == f32
    assert np.array_equal(emb[0, 0], od.m.embed([prefix[-1]])[0])
    assert hd.embed_tokens([3, 4]).shape == (2, H) and hd.embed_tokens(np.zeros((2, 3), np.int64)).shape == (2, 3, H)
    # leading dims kept, rows unchanged by the reshape
    x = np.random.default_rng(9).standard_normal((2, 3, H)).astype(np.float32)
    out = hd.apply_lm_head(x)
    assert out.shape == (2, 3, V)
    assert np.array_equal(out.reshape(6, V).view(np.uint32), hd.apply_lm_head(x.reshape(6, H)).view(np.uint32))
    with pytest.raises(hip.BackendError):
        hd.apply_lm_head(np.zeros((1, H + 1), np.float32))


def test_greedy_tree_commit_with_eos(hip):
    """EOS-aware commit composition (eagle.rs:664-732) on the device against
    the oracle's, for an EOS inside the accepted path, an EOS bonus and none."""
    od, hd, prefix = make_pair(hip, prefix_len=64)
    chain = greedy_chain(od, 3)
    tree = O.build_cartesian_tree(prefix[-1], _tree_with_chain(chain, 32000))
    n = len(tree)
    lo, _ = od.tree_logits_keep_kv(tree)
    od.rollback_to(len(prefix))
    lg, _ = hd.tree_logits_keep_kv(tree)
    argmax_agreement(lg, lo)
    # the composition is checked over the device's own argmaxes (the walk's
    # numerics are checked above and in test_tree_keep_kv_verify_and_commit)
    am = [int(v) for v in hd.last_argmax(n)]
    hd.rollback_to(len(prefix))
    am_strict = list(am)
    am_strict[0] = O.argmax_fold(hd.next_logits())  # the 1-row pass of the root
    for eos in ([], [chain[1]], [am[0]], [chain[0], am[0]]):
        for strict in (False, True):
            best, bonus = O.greedy_tree_accept(tree, None, am_strict if strict else am)
            hd.rollback_to(len(prefix))
            hd.set_eos_token_ids(eos)
            res = hd.verify_greedy_tree((tree.tokens(), tree.parents()), strict=strict, compose=True)
            com, stop, keep, bn = O.greedy_tree_commit(tree, best, bonus, eos, strict=strict)
            assert res.path == best and res.bonus == bonus
            assert res.committed == com and res.stop == stop, (eos, strict)
            assert res.keep() == keep and res.bonus_node == (bn if bn is not None else -1), (eos, strict)
    # committing the composed path leaves the cache as the oracle's
    hd.rollback_to(len(prefix))
    hd.set_eos_token_ids([chain[1]])
    res = hd.verify_greedy_tree((tree.tokens(), tree.parents()), compose=True)
    hd.commit_tree_path((tree.tokens(), tree.parents()), res.keep())
    od.tree_logits_keep_kv(tree)
    od.commit_tree_path(tree, res.keep())
    assert hd.history() == od.history == prefix + res.committed[:res.keep_len - 1] + (
        [res.bonus] if res.bonus_node >= 0 else [])
    assert hd.cache_len() == od.cache_len == len(prefix) - 1 + len(res.keep())
    hd.observe([11])
    od.observe([11])
    assert rel_err(hd.next_logits(), od.next_logits()) < TOL
    assert n > 4


def test_hidden_state_apis(hip):
    od, hd, prefix = make_pair(hip, prefix_len=32)
    hs = hd.last_hidden_state()
    od.rollback_to(len(prefix) - 1)
    final, mids = od.m.forward([prefix[-1]], [len(prefix) - 1], np.ones((1, len(prefix)), bool), (1, 2))
    od.cache_len = len(prefix)
    od.history = list(prefix)
    assert rel_err(hs, final[0]) < TOL
    fin, hm = hd.last_hidden_states_multi([1, 2])
    assert rel_err(fin, final[0]) < TOL
    assert rel_err(hm[0], mids[0][0]) < TOL and rel_err(hm[1], mids[1][0]) < TOL
    # embeddings are the exact dequantised rows
    ids = [0, 5, 31999, prefix[3]]
    assert np.array_equal(hd.embed_tokens(ids), od.m.embed(ids))
    # apply_lm_head on arbitrary hidden rows
    h = np.random.default_rng(2).standard_normal((3, 512)).astype(np.float32)
    assert rel_err(hd.apply_lm_head(h), od.m.lm_head(h)) < TOL
    # observe_returning_last_hidden == oracle forward of the same token
    hn = hd.observe_returning_last_hidden([7, 8])
    P = len(od.history)
    fo, _ = od.m.forward([7, 8], [P, P + 1], O.causal_mask(P, 2))
    assert rel_err(hn, fo[-1]) < TOL
    assert hd.history() == prefix + [7, 8]


@pytest.mark.parametrize("over", [
    dict(n_kv_heads=2, mix="q4_k_m", n_layers=3),
    dict(arch="qwen2", n_kv_heads=2, mix="q5k_q80", n_layers=2, rms_eps=1e-6, rope_theta=1e6),
    dict(n_heads=4, n_kv_heads=1, head_dim=128, mix="q6_k", n_layers=2),
])
def test_variants_batched_and_tree(hip, over):
    od, hd, prefix = make_pair(hip, prefix_len=70, **over)
    drafts = greedy_chain(od, 5)
    b = od.batched_logits(drafts)
    a = hd.batched_logits(drafts)
    for i in range(len(drafts) + 1):
        assert rel_err(a[i], b[i]) < TOL, (over, i)
    hd.rollback_to(len(prefix))
    od.rollback_to(len(prefix))
    tree = O.build_cartesian_tree(prefix[-1], [[drafts[0], 3, 4], [drafts[1], 9], [drafts[2]]])
    lo, _ = od.tree_logits_keep_kv(tree)
    lg, _ = hd.tree_logits_keep_kv(tree)
    for i in range(len(tree)):
        assert rel_err(lg[i], lo[i]) < TOL, (over, i)


@pytest.mark.parametrize("over,prefix_len,shape", [
    (dict(ctx_len=2048, n_layers=2), 1500, (4, 3, 2, 2)),
    (dict(n_kv_heads=2, head_dim=128, hidden=1024, ctx_len=1024, n_layers=2), 900, (2, 2, 2, 2, 2)),
])
def test_long_context_verify(hip, over, prefix_len, shape):
    """Long prefixes put the attention's key range over many splits (combine
    kernel) and ragged last blocks, for both the M <= 16 kernel (linear
    verify, 5 rows) and the query-parallel M > 16 kernel (89- and 63-node
    trees, whose last query tile is partial)."""
    od, hd, prefix = make_pair(hip, prefix_len=prefix_len, seed=4, **over)
    assert rel_err(hd.next_logits(), od.next_logits()) < TOL
    drafts = greedy_chain(od, 4)
    b = od.batched_logits(drafts)
    a = hd.batched_logits(drafts)
    for i in range(5):
        assert rel_err(a[i], b[i]) < TOL, (over, i)
    hd.rollback_to(len(prefix))
    od.rollback_to(len(prefix))
    rng = np.random.default_rng(prefix_len)
    cands = [[int(t) for t in rng.integers(0, 32000, w)] for w in shape]
    tree = O.build_cartesian_tree(prefix[-1], cands)
    assert len(tree) > 48
    lo, ho = od.tree_logits_keep_kv(tree)
    lg, hg = hd.tree_logits_keep_kv(tree)
    for i in range(len(tree)):
        assert rel_err(lg[i], lo[i]) < TOL, (over, i)
        assert rel_err(hg[i], ho[i]) < TOL, (over, i)
    assert hd.cache_len() == len(prefix) - 1 + len(tree)
