"""Parity at the full workload sizes: the Llama-3-8B-shaped Q4_K_M target (M=5
at 512 cached positions, a 60-node tree at 4096, a 64-node EAGLE-3 tree at
8192 with a 32000 -> 128256 d2t map) and the Qwen2.5-7B-shaped Q5_K/Q8_0
target with QKV bias (M=9 at 2048, rejection sampling at T=1).

The oracle's forward would take minutes at these sizes, so the checks are the
properties that hold at any size (as the reference's own model tests check
them, tests/with_qwen2_05b.rs:95-184, tests/tree_logits_consistency.rs:74-122):
a linear tree is the batched pass bit for bit; the strict tree row 0 is the
one-token pass bit for bit; device acceptance equals the oracle's walk over
the device's own rows (greedy exactly, rejection away from rounding
boundaries); KV compaction moves exactly the accepted rows.
"""
import numpy as np
import pytest

import oracle as O
from test_gpu_rejection import _check_walk, _draft_rows

pytestmark = pytest.mark.gpu

LLAMA8B = dict(n_layers=32, hidden=4096, n_heads=32, n_kv_heads=8, head_dim=128, ffn=14336, vocab=128256,
               rope_theta=500000.0, rms_eps=1e-5)
QWEN7B = dict(n_layers=28, hidden=3584, n_heads=28, n_kv_heads=4, head_dim=128, ffn=18944, vocab=152064,
              rope_theta=1e6, rms_eps=1e-6)


def _decoder(hip, arch, shape, mix, ctx):
    dec = hip.HipQuantDecoder(hip.Config(arch=arch, ctx_len=ctx, max_batch=64, **shape))
    dec.synthesize(mix, 0x5EED0002, 0.02)
    return dec


@pytest.fixture(scope="module")
def llama(hip):
    dec = _decoder(hip, hip.ARCH_LLAMA, LLAMA8B, hip.MIX_Q4_K_M, 4096 + 256)
    yield dec
    dec.close()


def _ids(rng, n, vocab):
    return [int(v) for v in rng.integers(0, vocab, n)]


def _safe(row, tol=1e-2):
    s = np.sort(row.astype(np.float64))[::-1]
    return (s[0] - s[1]) > tol * np.max(np.abs(row))


def test_llama8b_linear_verify_m5(hip, llama):
    """M=5 verify at 512 cached positions (the bench workload)."""
    V = LLAMA8B["vocab"]
    rng = np.random.default_rng(2)
    hist = _ids(rng, 513, V)
    llama.prime_synthetic(hist, 7)
    n0 = len(hist)
    drafts = _ids(rng, 4, V)
    rows = llama.batched_logits(drafts)
    assert rows.shape == (5, V) and np.isfinite(rows).all()
    assert llama.history() == hist + drafts and llama.cache_len() == n0 + 4
    llama.rollback_to(n0)
    # a linear tree through the drafts is the same 5-row pass, bit for bit
    chain = O.DraftTree.linear(hist[-1], drafts)
    trows, _ = llama.tree_logits_keep_kv((chain.tokens(), chain.parents()))
    assert np.array_equal(trows.view(np.uint32), rows.view(np.uint32))
    llama.rollback_to(n0)
    # device greedy acceptance == the host walk over the device's own rows
    am = [O.argmax_fold(r) for r in rows]
    commits, n_acc = llama.verify_greedy_linear(drafts)
    exp_acc, bonus = O.greedy_linear_accept(drafts, am)
    assert n_acc == exp_acc and commits == drafts[:n_acc] + [bonus]
    assert [int(v) for v in llama.last_argmax(5)] == am
    llama.rollback_to(n0)
    # the target's own greedy continuation is accepted in full unless a row
    # sits on a near tie between the one-token and the 5-row passes
    greedy = []
    for _ in range(4):
        greedy.append(O.argmax_fold(llama.next_logits()))
        llama.observe([greedy[-1]])
    llama.rollback_to(n0)
    rows_g = llama.batched_logits(greedy)
    llama.rollback_to(n0)
    commits, n_acc = llama.verify_greedy_linear(greedy)
    if all(_safe(r) for r in rows_g[:4]):
        assert n_acc == 4 and commits[:4] == greedy
    llama.rollback_to(n0)


def _tree(hip, rng, root, vocab, branching, n):
    cands = [_ids(rng, b, vocab) for b in branching]
    lps = [list(np.sort(np.log(rng.dirichlet(np.ones(b))))[::-1].astype(np.float32)) for b in branching]
    toks, pars = hip.tree_prune(hip.tree_cartesian(root, cands), lps, n)
    return toks, pars


def test_llama8b_tree60_verify_and_commit(hip, llama):
    """60-node tree (branching (4,3,2,2,1,1) pruned) at 4096 cached positions."""
    V = LLAMA8B["vocab"]
    rng = np.random.default_rng(4)
    hist = _ids(rng, 4097, V)
    llama.prime_synthetic(hist, 9)
    n1 = len(hist)
    P = n1 - 1
    toks, pars = _tree(hip, rng, hist[-1], V, (4, 3, 2, 2, 1, 1), 60)
    otree = O.DraftTree(list(toks), list(pars))
    n = len(otree)
    assert n == 60
    rows, hidden = llama.tree_logits_keep_kv((toks, pars))
    assert rows.shape == (n, V) and np.isfinite(rows).all() and np.isfinite(hidden).all()
    assert llama.cache_len() == P + n
    before = {(l, w, h): llama.read_kv_rows(l, w, h, P, n) for l in (0, 31) for w in (0, 1) for h in (0, 7)}
    prefix_rows = llama.read_kv_rows(17, 1, 3, P - 64, 64)
    llama.rollback_to(n1)
    # device greedy walk == the host walk over the device's rows
    path, bonus, bnode = llama.verify_greedy_tree((toks, pars))
    am = [O.argmax_fold(r) for r in rows]
    best, exp_bonus = O.greedy_tree_accept(otree, list(rows), am)
    assert path == best and bonus == exp_bonus
    assert bnode == (O.bonus_in_tree(otree, best[-1], exp_bonus) or -1)
    # compaction: rows [P, P + len(keep)) become the kept tree rows, bit for bit
    keep = path + ([bnode] if bnode >= 0 else [])
    llama.commit_tree_path((toks, pars), keep)
    assert llama.cache_len() == P + len(keep)
    assert llama.history() == hist + [int(toks[i]) for i in keep[1:]]
    for (l, w, h), r in before.items():
        assert np.array_equal(llama.read_kv_rows(l, w, h, P, len(keep)), r[keep]), (l, w, h)
    assert np.array_equal(llama.read_kv_rows(17, 1, 3, P - 64, 64), prefix_rows)
    # strict mode: row 0 is the one-token pass of the root, bit for bit
    llama.rollback_to(n1)
    strict = llama.tree_logits((toks, pars))
    assert llama.cache_len() == n1
    llama.rollback_to(n1 - 1)
    llama.observe([hist[-1]])
    assert np.array_equal(strict[0].view(np.uint32), llama.next_logits().view(np.uint32))


def test_eagle3_tree64_rejection_d2t(hip):
    """EAGLE-3 verify: 64-node depth-7 tree over 8192 cached positions, draft
    rows in a 32000-token vocabulary mapped through a seeded injective d2t,
    rejection sampling with seeded uniforms."""
    V, Vd = LLAMA8B["vocab"], 32000
    dec = _decoder(hip, hip.ARCH_LLAMA, LLAMA8B, hip.MIX_Q4_K_M, 8192 + 256)
    try:
        rng = np.random.default_rng(5)
        d2t = rng.choice(V, size=Vd, replace=False).astype(np.int64)
        dec.set_d2t(d2t)
        inv, _ = O.d2t_maps(d2t, V)
        hist = _ids(rng, 8193, V)
        dec.prime_synthetic(hist, 11)
        n1 = len(hist)
        kinds = {"exact": 0, "boundary": 0}
        for T in (1.0, 0.1):
            cand_d = [[int(v) for v in rng.choice(Vd, b, replace=False)] for b in (4, 3, 2, 2, 1, 1, 1)]
            cands = [[int(d2t[v]) for v in c] for c in cand_d]
            lps = [list(np.sort(np.log(rng.dirichlet(np.ones(len(c)))))[::-1].astype(np.float32)) for c in cands]
            toks, pars = hip.tree_prune(hip.tree_cartesian(hist[-1], cands), lps, 64)
            otree = O.DraftTree(list(toks), list(pars))
            n = len(otree)
            assert n == 64 and max(otree.depth_of(i) for i in range(n)) >= 4
            q_d = _draft_rows(rng, n, Vd)
            q_row_of = list(range(n))
            u = [float(x) for x in rng.random(n, dtype=np.float32)]
            rows, _ = dec.tree_logits_keep_kv((toks, pars))
            assert np.isfinite(rows).all()
            dec.rollback_to(n1)
            path, tok, used = dec.verify_rejection_tree((toks, pars), q_d, q_row_of, u, T)
            dec.rollback_to(n1)
            q_t = np.zeros((n, V), np.float32)
            for tid, did in inv.items():
                q_t[:, tid] = q_d[:, did]
            opath, otok, oused = O.rejection_tree_accept(otree, list(rows), list(q_t), q_row_of, u, T)
            kind = _check_walk(path, tok if tok >= 0 else None, opath, otok, otree, list(rows), list(q_t),
                               q_row_of, u, T)
            kinds[kind] += 1
            if kind == "exact":
                assert used == oused
        assert kinds["exact"] >= 1, kinds
    finally:
        dec.close()


def test_qwen7b_rejection_linear_m9(hip):
    """Qwen2.5-7B-shaped target (QKV bias, Q5_K attention, Q8_0 FFN), k=8
    drafts (M=9) at 2048 cached positions, rejection sampling with draft
    rows softmax(N(0, 2)) and seeded uniforms."""
    V, k = QWEN7B["vocab"], 8
    dec = _decoder(hip, hip.ARCH_QWEN2, QWEN7B, hip.MIX_Q5K_Q80, 2048 + 128)
    try:
        rng = np.random.default_rng(3)
        hist = _ids(rng, 2049, V)
        dec.prime_synthetic(hist, 13)
        n0 = len(hist)
        kinds = {"exact": 0, "boundary": 0}
        for T in (1.0, 0.1):
            q = _draft_rows(rng, k, V)
            drafts = [int(O.sample_u(q[i], float(rng.random()))) for i in range(k)]
            u = [float(x) for x in rng.random(k + 1, dtype=np.float32)]
            rows = dec.batched_logits(drafts)
            assert rows.shape == (k + 1, V) and np.isfinite(rows).all()
            dec.rollback_to(n0)
            commits, n_acc, used = dec.verify_rejection_linear(drafts, q, u, T)
            assert dec.history() == hist + drafts and dec.cache_len() == n0 + k
            dec.rollback_to(n0)
            oc, on, ou = O.rejection_linear_accept(list(rows), list(q), drafts, u, T)
            chain = O.DraftTree.linear(hist[-1], drafts)
            dev_fin = commits[n_acc] if len(commits) > n_acc else None
            ora_fin = oc[on] if len(oc) > on else None
            kind = _check_walk(list(range(n_acc + 1)), dev_fin, list(range(on + 1)), ora_fin, chain, list(rows),
                               list(q), list(range(k)) + [-1], u, T)
            kinds[kind] += 1
            if kind == "exact":
                assert commits == oc and n_acc == on and used == ou
        assert kinds["exact"] >= 1, kinds
    finally:
        dec.close()
