"""EAGLE-3 draft on the device (Eagle3DraftCandle, eagle3.rs:307-516, and the
draft half of run_eagle3, :598-673) against the oracle's f16 restatement
(oracle/eagle3.py), through the C ABI.

Contract: the midlayer output and the draft logits within 2e-2 relative
(max |a-b| / max |b|) of the oracle's over several chained steps -- the
draft runs in f16 and rounds after every op, so one-ulp differences of a
product's accumulation order travel through the steps; a round's top-k
draft ids equal top_k_indices (value descending, index ascending) of the
device's own logits bit for bit, their log-probs l - logsumexp(l) within
2e-5 of the f64 value, their target ids d2t[draft id], and against the
oracle's logits on the same inputs at every step the top-k ids agree
wherever the oracle's gap between neighbouring ranks exceeds twice the
step's device/oracle logit difference;
the target decoder's history, cache and logits are as before the round.
"""
import numpy as np
import pytest

import eagle3 as E
import oracle as O
from _models import MIX_IDS, hip_cfg, oracle_cfg, rel_err


def _check_log_probs(got, logits, idx, step):
    """l - logsumexp(l): within 2e-5 of the f64 value; within the rounding bound
    of the reference's sequential f32 sum (n 2^-24 relative) of its own form"""
    l64 = np.asarray(logits, np.float64)
    mx = l64.max()
    ref64 = [float(l64[i] - (np.log(np.exp(l64 - mx).sum()) + mx)) for i in idx]
    assert np.allclose(got, ref64, atol=2e-5), (step, got, ref64)
    seq = E.log_probs(logits, idx)
    assert np.allclose(got, seq, atol=2e-5 + len(l64) * 2.0 ** -24), (step, got, seq)


pytestmark = pytest.mark.gpu

TOL = 2e-2
DRAFT = dict(hidden=512, n_heads=8, n_kv_heads=2, ffn=1024, draft_vocab=4000, target_vocab=32000,
             rope_theta=500000.0, max_pos=1024)


def _draft(hip, std=0.05, seed=11, **over):
    c = dict(DRAFT)
    c.update(over)
    d = hip.HipEagle3Draft(**c)
    d.synthesize(seed, std)
    return d, c


def _oracle_of(hip, d, c):
    ec = E.Eagle3Config(hidden=c["hidden"], n_heads=c["n_heads"], n_kv_heads=c["n_kv_heads"], ffn=c["ffn"],
                        draft_vocab=c["draft_vocab"], target_vocab=c["target_vocab"], rope_theta=c["rope_theta"],
                        max_pos=c["max_pos"])
    shp = E.shapes(ec)
    t = {k: d.get_tensor(k).astype(np.float32).reshape(shp[k]) for k in shp}
    return E.Eagle3Oracle(ec, t), d.get_tensor(hip.D3_D2T)


def test_tensor_round_trip_and_sizes(hip):
    d, c = _draft(hip)
    H = c["hidden"]
    assert d.tensor_bytes(hip.D3_FC) == H * 3 * H * 2
    assert d.tensor_bytes(hip.D3_Q) == H * 2 * H * 2
    assert d.tensor_bytes(hip.D3_K) == 2 * 64 * 2 * H * 2
    assert d.tensor_bytes(hip.D3_D2T) == c["draft_vocab"] * 8
    # the synthetic weights: N(0, 0.05)-like matrices, norms 1 + N(0, 0.1)
    q = d.get_tensor(hip.D3_Q).astype(np.float64)
    assert abs(q.mean()) < 1e-3 and abs(q.std() - 0.05) < 2.5e-3, (q.mean(), q.std())
    nw = d.get_tensor(hip.D3_NORM).astype(np.float64)
    assert abs(nw.mean() - 1) < 0.03 and abs(nw.std() - 0.1) < 0.02, (nw.mean(), nw.std())
    w = np.random.default_rng(0).standard_normal((c["ffn"], H)).astype(np.float16)
    d.set_tensor(hip.D3_UP, w)
    assert np.array_equal(d.get_tensor(hip.D3_UP).reshape(w.shape), w)
    d2t = d.get_tensor(hip.D3_D2T)
    assert len(set(d2t.tolist())) == c["draft_vocab"] and d2t.min() >= 0 and d2t.max() < c["target_vocab"]
    with pytest.raises(hip.ArgError):
        d.set_tensor(hip.D3_UP, w[:-1])
    with pytest.raises(hip.ArgError):
        hip.HipEagle3Draft(hidden=500, n_heads=8, n_kv_heads=2, ffn=1024, draft_vocab=4000, target_vocab=32000)
    d.close()


def test_forward_chain_matches_oracle(hip):
    d, c = _draft(hip)
    o, _ = _oracle_of(hip, d, c)
    H = c["hidden"]
    rng = np.random.default_rng(5)
    h_in = rng.standard_normal(3 * H).astype(np.float32)
    for pos0 in (0, 37):
        d.reset()
        o.reset()
        hd_, ho = h_in, h_in
        for s in range(5):
            emb = (rng.standard_normal(H) * 0.5).astype(np.float32)
            out_d, lg_d = d.forward_hidden(hd_, emb, pos0 + s)
            out_o = o.forward_hidden(ho, emb, pos0 + s)
            lg_o = o.norm_lm_head(out_o)
            print(f"pos0 {pos0} step {s}: hidden {rel_err(out_d, out_o):.2e} logits {rel_err(lg_d, lg_o):.2e}",
                  flush=True)
            assert rel_err(out_d, out_o) < TOL, (pos0, s)
            assert rel_err(lg_d, lg_o) < TOL, (pos0, s)
            # f16 values through and through
            assert np.array_equal(out_d, out_d.astype(np.float16).astype(np.float32))
            # each side feeds its own output on (the chain of run_eagle3)
            hd_, ho = out_d, out_o
    with pytest.raises(hip.ArgError):
        d.forward_hidden(h_in[:100], emb, 0)
    with pytest.raises(hip.ArgError):
        d.forward_hidden(h_in, emb, c["max_pos"])
    d.close()


def test_draft_cache_limit(hip):
    d, c = _draft(hip)
    H = c["hidden"]
    x = np.zeros(H, np.float32)
    for s in range(hip.DRAFT3_MAX_STEPS):
        d.forward_hidden(x, x, s, want_logits=False)
    with pytest.raises(hip.ArgError):
        d.forward_hidden(x, x, 16, want_logits=False)
    d.reset()
    d.forward_hidden(x, x, 0, want_logits=False)
    d.close()


def _target(hip, prefix_len=40, seed=3):
    ocfg = oracle_cfg()
    om = O.OracleModel(ocfg)
    od = O.OracleDecoder(om)
    hd = hip.HipQuantDecoder(hip_cfg(hip, ocfg))
    hd.synthesize(MIX_IDS[ocfg.mix], ocfg.seed, ocfg.weight_std)
    prefix = [int(v) for v in np.random.default_rng(seed).integers(0, ocfg.vocab, prefix_len)]
    od.observe(prefix)
    hd.observe(prefix)
    return od, hd, prefix


def _gap_ok(lg_o, ids_dev, k, diff):
    """the device's top-k equals the oracle's wherever the oracle's neighbouring
    ranks are more than 2 * diff apart; returns the near ties met"""
    order = E.top_k_indices(lg_o, k + 1)
    ties = 0
    for r in range(k):
        if ids_dev[r] == order[r]:
            continue
        a, b = float(lg_o[ids_dev[r]]), float(lg_o[order[r]])
        assert abs(a - b) <= 2 * diff + 1e-6, (r, ids_dev[r], order[r], a, b, diff)
        ties += 1
    return ties


@pytest.mark.parametrize("layers,depth,top_k", [([1, 2, 3], 5, 4), ([0, 0, 3], 3, [8, 2, 1])])
def test_round_matches_device_steps_and_oracle(hip, layers, depth, top_k):
    od, hd, prefix = _target(hip)
    d, c = _draft(hip)
    o, d2t = _oracle_of(hip, d, c)
    ks = [top_k] * depth if np.isscalar(top_k) else top_k
    before = hd.next_logits()
    ids, lps, dids = d.round(hd, layers, depth, top_k)
    # the target is as before
    assert hd.history() == prefix
    assert np.array_equal(hd.next_logits(), before)
    # 1. the device's own steps, replayed one at a time from the same inputs
    fin, mids = hd.last_hidden_states_multi(layers)
    h = np.concatenate(mids)
    tok = prefix[-1]
    d.reset()
    dev_logits, dev_in = [], []
    for s in range(depth):
        dev_in.append(h)
        out, lg = d.forward_hidden(h, hd.embed_tokens([tok])[0], len(prefix) + s)
        dev_logits.append(lg)
        want = E.top_k_indices(lg, ks[s])
        assert dids[s] == want, (s, dids[s], want)
        assert ids[s] == [int(d2t[i]) for i in want]
        _check_log_probs(lps[s], lg, want, s)
        h, tok = out, ids[s][0]
    # 2. the oracle on the same inputs at every step (the device's hidden
    #    input and top-1 token; free-running chains are the forward test's),
    #    the embeddings from the oracle decoder, the draft in the oracle's f16
    P = len(prefix)
    od.rollback_to(P - 1)
    _, omids = od.m.forward([prefix[-1]], [P - 1], np.ones((1, P), bool), tuple(layers))
    od.cache_len, od.history = P, list(prefix)
    assert rel_err(np.concatenate([m[0] for m in omids]), np.concatenate(mids)) < 1e-2
    tok = prefix[-1]
    o.reset()
    ties = 0
    for s in range(depth):
        out = o.forward_hidden(dev_in[s], od.m.embed([tok])[0], P + s)
        lg_o = o.norm_lm_head(out)
        diff = float(np.max(np.abs(dev_logits[s] - lg_o)))
        assert rel_err(dev_logits[s], lg_o) < TOL, s
        ties += _gap_ok(lg_o, dids[s], ks[s], diff)
        tok = ids[s][0]
    print(f"round {layers} depth {depth}: near ties {ties}", flush=True)
    assert ties <= depth
    d.close()
    hd.close()


def test_round_errors_keep_state(hip):
    od, hd, prefix = _target(hip, prefix_len=20)
    d, c = _draft(hip)
    before = hd.next_logits()
    with pytest.raises(hip.ArgError):
        d.round(hd, [1, 2, 3], 0, 2)
    with pytest.raises(hip.ArgError):
        d.round(hd, [1, 2, 3], 17, 2)
    with pytest.raises(hip.ArgError):
        d.round(hd, [1, 2, 3], 2, 9)
    with pytest.raises(hip.BackendError):
        d.round(hd, [1, 2, 4], 2, 2)
    with pytest.raises(hip.SamplingError):
        d.round(hd, [1, 2], 2, 2)
    # positions past the RoPE tables
    short, _ = _draft(hip, max_pos=21)
    with pytest.raises(hip.ArgError):
        short.round(hd, [1, 2, 3], 2, 2)
    short.round(hd, [1, 2, 3], 1, 2)
    # a target of another vocabulary
    other, _ = _draft(hip, target_vocab=31999)
    with pytest.raises(hip.ArgError):
        other.round(hd, [1, 2, 3], 2, 2)
    # a d2t entry outside the target vocabulary
    d2t = d.get_tensor(hip.D3_D2T)
    d2t[7] = -1
    d.set_tensor(hip.D3_D2T, d2t)
    with pytest.raises(hip.ArgError):
        d.round(hd, [1, 2, 3], 2, 2)
    assert hd.history() == prefix
    assert np.array_equal(hd.next_logits(), before)
    hd.reset()
    with pytest.raises(hip.SamplingError):
        short.round(hd, [1, 2, 3], 1, 2)
    for x in (d, short, other, hd):
        x.close()


def test_round_reuses_the_observed_rows(hip):
    """After a collection the decoder collects the same layers on every
    one-token observe; the next round reads those rows instead of running the
    same M=1 forward again.  Same values as an explicit recomputation, and a
    rollback never leaves stale rows behind."""
    od, hd, prefix = _target(hip)
    _, hd2, _ = _target(hip)
    d, c = _draft(hip)
    layers = [1, 2, 3]
    # the first round recomputes the prompt's last token at M=1 (rewriting its
    # KV row through the one-row path), on both decoders alike
    d.round(hd, layers, 2, 2)
    d.round(hd2, layers, 2, 2)
    for t in (5, 77):
        hd.observe([t])
        hd2.observe([t])
        a = d.round(hd, layers, 4, 3)
        hd2.last_hidden_states_multi(layers)  # recomputes
        b = d.round(hd2, layers, 4, 3)
        assert a == b, t
        assert d.round(hd, layers, 4, 3) == a
    # rollback, then another token: rows of the new token
    hd.rollback_to(len(prefix) + 1)
    hd2.rollback_to(len(prefix) + 1)
    hd.observe([9])
    hd2.observe([9])
    a = d.round(hd, layers, 3, 2)
    hd2.last_hidden_states_multi(layers)
    assert a == d.round(hd2, layers, 3, 2)
    # rollback alone: the round recomputes for the shorter history
    hd.rollback_to(len(prefix))
    hd2.rollback_to(len(prefix))
    a = d.round(hd, layers, 3, 2)
    hd2.last_hidden_states_multi(layers)
    assert a == d.round(hd2, layers, 3, 2)
    assert hd.history() == prefix
    for x in (d, hd, hd2):
        x.close()


def test_round_top_k_ties_across_slices(hip):
    """Equal logits in different 1024-entry slices of the draft vocabulary come
    out by index (medusa.rs:846-852), and the log-probs are the log-softmax."""
    od, hd, prefix = _target(hip, prefix_len=12)
    d, c = _draft(hip)
    V, H = c["draft_vocab"], c["hidden"]
    lm = np.zeros((V, H), np.float16)
    d.set_tensor(hip.D3_LM_HEAD, lm)
    ids, lps, dids = d.round(hd, [0, 1, 2], 2, 8)
    assert dids == [list(range(8))] * 2
    assert np.allclose(lps, -np.log(V), atol=1e-5)
    u = (np.random.default_rng(4).standard_normal(H) * 0.05).astype(np.float16)
    for r in (5, 1500, 3000):
        lm[r] = u
    for r in (7, 2500, 3500):
        lm[r] = -u
    d.set_tensor(hip.D3_LM_HEAD, lm)
    ids, lps, dids = d.round(hd, [0, 1, 2], 2, 8)
    d2t = d.get_tensor(hip.D3_D2T)
    for s in range(2):
        a = lps[s][0] - lps[s][3]  # the winners' logit over the zeros
        assert a > 0
        win = [5, 1500, 3000] if dids[s][0] == 5 else [7, 2500, 3500]
        assert dids[s] == win + [0, 1, 2, 3, 4], dids[s]
        lse = np.log(3 * np.exp(a) + 3 * np.exp(-a) + (V - 6))
        assert np.allclose(lps[s], [a - lse] * 3 + [-lse] * 5, atol=1e-5)
        assert ids[s] == [int(d2t[i]) for i in dids[s]]
    d.close()
    hd.close()


@pytest.mark.parametrize("draft_vocab", [1025, 4097])
def test_round_top_k_short_last_slice(hip, draft_vocab):
    """A draft vocabulary of 1024 n + 1 leaves a last 1024-entry top-k slice
    with one logit, fewer than k = 8 eligible entries: its unfilled candidate
    places drop out of the merge, so the round's top-8 equals top_k_indices
    (medusa.rs:477-487) of the device's own step logits and the log-probs are
    l - logsumexp(l); that slice's single entry still takes part (planted as
    the largest logit, it ranks first)."""
    od, hd, prefix = _target(hip, prefix_len=20)
    d, c = _draft(hip, draft_vocab=draft_vocab)
    d2t = d.get_tensor(hip.D3_D2T)
    layers, depth = [1, 2, 3], 3
    fin, mids = hd.last_hidden_states_multi(layers)
    h0 = np.concatenate(mids)
    for planted in (False, True):
        ids, lps, dids = d.round(hd, layers, depth, 8)
        h, tok = h0, prefix[-1]
        d.reset()
        for s in range(depth):
            out, lg = d.forward_hidden(h, hd.embed_tokens([tok])[0], len(prefix) + s)
            want = E.top_k_indices(lg, 8)
            assert dids[s] == want, (draft_vocab, planted, s, dids[s], want)
            assert ids[s] == [int(d2t[i]) for i in want]
            _check_log_probs(lps[s], lg, want, s)
            if planted and s == 0:
                assert want[0] == draft_vocab - 1, want
            h, tok = out, ids[s][0]
        if not planted:
            # the last row := twice the first step's winning row: its logit doubles
            lm = d.get_tensor(hip.D3_LM_HEAD).reshape(draft_vocab, c["hidden"]).copy()
            w0 = dids[0][0]
            lm[draft_vocab - 1] = (lm[w0].astype(np.float32) * 2).astype(np.float16)
            d.set_tensor(hip.D3_LM_HEAD, lm)
    d.close()
    hd.close()
