"""EAGLE-2 draft on the device (EagleDraftCandle, eagle.rs:306-428, and the
draft half of run_eagle, :519-575) against the oracle's f16 restatement
(oracle/eagle2.py), through the C ABI.

Contract: the draft's outputs within 2e-2 relative (max |a-b| / max |b|) of
the oracle's over chained steps; a round's ids equal top_k_indices of the
target's own lm_head (sd_apply_lm_head) on the device draft's outputs, step
by step, bit for bit, their log-probs within 2e-5 of l - logsumexp(l) in f64
(the reference's sequential f32 sum is n 2^-24 off at worst); on the same
inputs at every step the oracle (oracle draft, oracle target lm_head) gives
outputs and logits within 2e-2 and the same top-k wherever its neighbouring
ranks are more than twice the step's logit difference apart; the target is
untouched.  The
target vocabulary of the round test is over 65536 entries, so the top-k merge
takes more than one slice group per lane.
"""
import numpy as np
import pytest

import eagle2 as E2
import eagle3 as E3
import oracle as O
from _models import MIX_IDS, hip_cfg, oracle_cfg, rel_err


def _check_log_probs(got, logits, idx, step):
    """l - logsumexp(l): within 2e-5 of the f64 value; within the rounding bound
    of the reference's sequential f32 sum (n 2^-24 relative) of its own form"""
    l64 = np.asarray(logits, np.float64)
    mx = l64.max()
    ref64 = [float(l64[i] - (np.log(np.exp(l64 - mx).sum()) + mx)) for i in idx]
    assert np.allclose(got, ref64, atol=2e-5), (step, got, ref64)
    seq = E3.log_probs(logits, idx)
    assert np.allclose(got, seq, atol=2e-5 + len(l64) * 2.0 ** -24), (step, got, seq)


pytestmark = pytest.mark.gpu

TOL = 2e-2
VOCAB = 70016  # a multiple of 32, over 65536
DRAFT = dict(hidden=512, n_heads=8, n_kv_heads=2, ffn=1024, vocab=VOCAB, rope_theta=500000.0, max_pos=1024)


def _draft(hip, std=0.05, seed=21, **over):
    c = dict(DRAFT)
    c.update(over)
    d = hip.HipEagleDraft(**c)
    d.synthesize(seed, std)
    return d, c


def _oracle_of(d, c):
    ec = E2.Eagle2Config(hidden=c["hidden"], n_heads=c["n_heads"], n_kv_heads=c["n_kv_heads"], ffn=c["ffn"],
                         vocab=c["vocab"], rope_theta=c["rope_theta"], max_pos=c["max_pos"])
    shp = E2.shapes(ec)
    return E2.Eagle2Oracle(ec, {k: d.get_tensor(k).astype(np.float32).reshape(shp[k]) for k in shp})


_TARGETS = {}


def _target(hip, prefix_len=40, seed=3):
    ocfg = oracle_cfg(vocab=VOCAB)
    if "w" not in _TARGETS:
        _TARGETS["w"] = O.OracleModel(ocfg).raw
    od = O.OracleDecoder(O.OracleModel(ocfg, _TARGETS["w"]))
    hd = hip.HipQuantDecoder(hip_cfg(hip, ocfg))
    hd.synthesize(MIX_IDS[ocfg.mix], ocfg.seed, ocfg.weight_std)
    prefix = [int(v) for v in np.random.default_rng(seed).integers(0, VOCAB, prefix_len)]
    od.observe(prefix)
    hd.observe(prefix)
    return od, hd, prefix


def test_tensors_and_forward_chain_match_oracle(hip):
    d, c = _draft(hip, vocab=4000)
    H = c["hidden"]
    assert d.tensor_bytes(hip.D2_EMBED) == 4000 * H * 2
    assert d.tensor_bytes(hip.D2_FC) == H * 2 * H * 2
    q = d.get_tensor(hip.D2_Q).astype(np.float64)
    assert abs(q.std() - 0.05) < 2.5e-3
    o = _oracle_of(d, c)
    rng = np.random.default_rng(6)
    for pos0 in (0, 77):
        d.reset()
        o.reset()
        h = (rng.standard_normal(H) * 2).astype(np.float32)
        hd_, ho = h, h
        for s in range(5):
            tok = int(rng.integers(0, 4000))
            out_d = d.forward(hd_, tok, pos0 + s)
            out_o = o.forward(ho, tok, pos0 + s)
            print(f"pos0 {pos0} step {s}: {rel_err(out_d, out_o):.2e}", flush=True)
            assert rel_err(out_d, out_o) < TOL, (pos0, s)
            assert np.array_equal(out_d, out_d.astype(np.float16).astype(np.float32))
            hd_, ho = out_d, out_o
    with pytest.raises(hip.ArgError):
        d.forward(h, 4000, 0)
    with pytest.raises(hip.ArgError):
        d.forward(h[:100], 1, 0)
    with pytest.raises(hip.ArgError):
        d.forward(h, 1, c["max_pos"])
    d.close()


@pytest.mark.parametrize("depth,top_k", [(4, 2), (6, [8, 4, 2, 1, 1, 3])])
def test_round_matches_device_steps_and_oracle(hip, depth, top_k):
    od, hd, prefix = _target(hip)
    d, c = _draft(hip)
    o = _oracle_of(d, c)
    ks = [top_k] * depth if np.isscalar(top_k) else top_k
    P = len(prefix)
    h = hd.last_hidden_state()
    before = hd.next_logits()
    ids, lps = d.round(hd, h, depth, top_k)
    assert hd.history() == prefix
    assert np.array_equal(hd.next_logits(), before)
    # 1. the device's own steps with the target's apply_lm_head
    d.reset()
    x, tok, dev_logits, dev_out = h, prefix[-1], [], []
    for s in range(depth):
        out = d.forward(x, tok, P + s)
        lg = hd.apply_lm_head(out)
        dev_logits.append(lg)
        dev_out.append(out)
        want = E3.top_k_indices(lg, ks[s])
        assert ids[s] == want, (s, ids[s], want)
        _check_log_probs(lps[s], lg, want, s)
        x, tok = out, ids[s][0]
    # 2. the oracle on the same inputs, step by step (the device's previous
    #    output and top-1 id; free-running chains are the forward test's)
    od.rollback_to(P - 1)
    fin, _ = od.m.forward([prefix[-1]], [P - 1], np.ones((1, P), bool))
    od.cache_len, od.history = P, list(prefix)
    assert rel_err(h, fin[0]) < 1e-2
    o.reset()
    x, tok, ties = h, prefix[-1], 0
    for s in range(depth):
        out_o = o.forward(x, tok, P + s)
        assert rel_err(dev_out[s], out_o) < TOL, s
        lg_o = od.m.lm_head(dev_out[s][None])[0]  # the target's lm_head, oracle side
        diff = float(np.max(np.abs(dev_logits[s] - lg_o)))
        assert rel_err(dev_logits[s], lg_o) < TOL, s
        order = E3.top_k_indices(lg_o, ks[s])
        for r in range(ks[s]):
            if ids[s][r] != order[r]:
                assert abs(float(lg_o[ids[s][r]]) - float(lg_o[order[r]])) <= 2 * diff + 1e-6, (s, r)
                ties += 1
        x, tok = dev_out[s], ids[s][0]
    print(f"depth {depth}: near ties {ties}", flush=True)
    d.close()
    hd.close()


def test_round_errors_keep_state(hip):
    od, hd, prefix = _target(hip, prefix_len=20)
    d, c = _draft(hip)
    h = hd.last_hidden_state()
    before = hd.next_logits()
    with pytest.raises(hip.ArgError):
        d.round(hd, h, 0, 2)
    with pytest.raises(hip.ArgError):
        d.round(hd, h, 17, 2)
    with pytest.raises(hip.ArgError):
        d.round(hd, h, 2, 9)
    with pytest.raises(hip.ArgError):
        d.round(hd, h[:10], 2, 2)
    short, _ = _draft(hip, max_pos=21)
    with pytest.raises(hip.ArgError):
        short.round(hd, h, 2, 2)
    short.round(hd, h, 1, 2)
    other, _ = _draft(hip, vocab=VOCAB - 16)
    with pytest.raises(hip.ArgError):
        other.round(hd, h, 2, 2)
    assert hd.history() == prefix
    assert np.array_equal(hd.next_logits(), before)
    hd.reset()
    with pytest.raises(hip.SamplingError):
        short.round(hd, h, 1, 2)
    for x in (d, short, other, hd):
        x.close()
