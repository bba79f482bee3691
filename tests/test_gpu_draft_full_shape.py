"""The EAGLE-3 and EAGLE-2 drafts at the reference's own draft configs, against
the oracle's f16 restatements (oracle/eagle3.py, oracle/eagle2.py), through
the C ABI:

* Eagle3DraftConfig::eagle3_llama3_1_8b (eagle3.rs:81-93): hidden 4096,
  32 / 8 heads of 128, FFN 14336, draft vocabulary 32000 -> 128256,
  RoPE theta 500000, 2048 positions;
* EagleDraftConfig::eagle_llama3_8b (eagle.rs:67-80): the same widths with
  the draft's own 128256-entry token table.

These are the shapes the benchmark's draft rounds run, so the kernel
instances met here are the production ones: the draft RMSNorm at hidden 4096
(four elements per thread), the f16 matrix-vector product at K = 4096, 8192
(EAGLE-3 Q/K/V over [input norm, hidden norm]; EAGLE-2 fc over [hidden,
embedding]), 12288 (EAGLE-3 fc over the three target layers) and 14336
(ffn_down), where each wave takes several 512-input chunks, and the draft
attention at head_dim 128.

Contract (as at the small widths): over a chained run each step's output and
logits within 2e-2 relative (max |a-b| / max |b|) of the oracle's, the
device's top-k equal to the oracle's wherever the oracle's neighbouring ranks
are more than twice the step's logit difference apart; a round's ids equal
top_k_indices of the device's own step logits bit for bit.
"""
import numpy as np
import pytest

import eagle2 as E2
import eagle3 as E3
from _models import rel_err

pytestmark = pytest.mark.gpu

TOL = 2e-2
STD = 0.02
E3_REF = dict(hidden=4096, n_heads=32, n_kv_heads=8, ffn=14336, draft_vocab=32000, target_vocab=128256,
              rope_theta=500000.0, max_pos=2048)
E2_REF = dict(hidden=4096, n_heads=32, n_kv_heads=8, ffn=14336, vocab=128256, rope_theta=500000.0, max_pos=2048)
LLAMA8B_1L = dict(arch=0, n_layers=1, hidden=4096, n_heads=32, n_kv_heads=8, head_dim=128, ffn=14336,
                  vocab=128256, rope_theta=500000.0, rms_eps=1e-5)


def _gap_ties(lg_o, ids_dev, k, diff):
    """the device's top-k equals the oracle's wherever the oracle's neighbouring
    ranks are more than 2 * diff apart; returns the near ties met"""
    order = E3.top_k_indices(lg_o, k + 1)
    ties = 0
    for r in range(k):
        if ids_dev[r] == order[r]:
            continue
        a, b = float(lg_o[ids_dev[r]]), float(lg_o[order[r]])
        assert abs(a - b) <= 2 * diff + 1e-6, (r, ids_dev[r], order[r], a, b, diff)
        ties += 1
    return ties


def test_eagle3_reference_config_chain(hip):
    d = hip.HipEagle3Draft(**E3_REF)
    try:
        d.synthesize(31, STD)
        ec = E3.Eagle3Config(**E3_REF)
        shp = E3.shapes(ec)
        o = E3.Eagle3Oracle(ec, {k: d.get_tensor(k).astype(np.float32).reshape(shp[k]) for k in shp})
        H = ec.hidden
        rng = np.random.default_rng(41)
        ties = 0
        # position 2000: the f16 RoPE table's coarse end (t rounded to f16)
        for pos0, steps in ((2000, 3), (0, 2)):
            d.reset()
            o.reset()
            h_dev = h_or = rng.standard_normal(3 * H).astype(np.float32)  # the fc input (K = 12288)
            for s in range(steps):
                emb = (rng.standard_normal(H) * 0.5).astype(np.float32)
                out_d, lg_d = d.forward_hidden(h_dev, emb, pos0 + s)
                out_o = o.forward_hidden(h_or, emb, pos0 + s)
                lg_o = o.norm_lm_head(out_o)
                eh, el = rel_err(out_d, out_o), rel_err(lg_d, lg_o)
                print(f"eagle3 pos {pos0 + s}: hidden {eh:.2e} logits {el:.2e}", flush=True)
                assert eh < TOL and el < TOL, (pos0, s, eh, el)
                assert np.array_equal(out_d, out_d.astype(np.float16).astype(np.float32))
                ties += _gap_ties(lg_o, E3.top_k_indices(lg_d, 8), 8, float(np.max(np.abs(lg_d - lg_o))))
                h_dev, h_or = out_d, out_o
        print(f"eagle3 near ties {ties}", flush=True)
        assert ties <= 2
    finally:
        d.close()


def test_eagle2_reference_config_chain(hip):
    d = hip.HipEagleDraft(**E2_REF)
    try:
        d.synthesize(32, STD)
        ec = E2.Eagle2Config(**E2_REF)
        shp = E2.shapes(ec)
        o = E2.Eagle2Oracle(ec, {k: d.get_tensor(k).astype(np.float32).reshape(shp[k]) for k in shp})
        H = ec.hidden
        rng = np.random.default_rng(42)
        for pos0, steps in ((1990, 3), (3, 2)):
            d.reset()
            o.reset()
            h_dev = h_or = (rng.standard_normal(H) * 2).astype(np.float32)
            for s in range(steps):
                tok = int(rng.integers(0, ec.vocab))
                out_d = d.forward(h_dev, tok, pos0 + s)
                out_o = o.forward(h_or, tok, pos0 + s)
                e = rel_err(out_d, out_o)
                print(f"eagle2 pos {pos0 + s}: {e:.2e}", flush=True)
                assert e < TOL, (pos0, s, e)
                assert np.array_equal(out_d, out_d.astype(np.float16).astype(np.float32))
                # the next step's input is the oracle's output on both sides (each
                # keeps its own KV rows): with random weights the draft amplifies a
                # difference fed back through its hidden input from step to step, so
                # a chain of each side's own outputs would test that amplification
                # rather than one forward at these shapes
                h_dev = h_or = out_o
    finally:
        d.close()


def test_eagle2_reference_config_round_on_llama8b_width_target(hip):
    """A draft round against a target of the Llama-3-8B widths (one layer;
    the round reads only its token-independent lm_head and the caller's
    hidden row): every step's top-k over the 128256 target logits equals
    top_k_indices of the target's apply_lm_head on the device's own step
    output, which the round reproduces bit for bit."""
    hd = hip.HipQuantDecoder(hip.Config(ctx_len=256, max_batch=16, **LLAMA8B_1L))
    d = hip.HipEagleDraft(**E2_REF)
    try:
        hd.synthesize(hip.MIX_Q4_K_M, 0x5EED0004, 0.02)
        d.synthesize(33, STD)
        prefix = [int(v) for v in np.random.default_rng(5).integers(0, 128256, 24)]
        hd.observe(prefix)
        h = hd.last_hidden_state()
        before = hd.next_logits()
        depth, ks = 4, [8, 4, 2, 1]
        ids, lps = d.round(hd, h, depth, ks)
        assert hd.history() == prefix
        assert np.array_equal(hd.next_logits().view(np.uint32), before.view(np.uint32))
        d.reset()
        x, tok = h, prefix[-1]
        for s in range(depth):
            out = d.forward(x, tok, len(prefix) + s)
            lg = hd.apply_lm_head(out)
            want = E3.top_k_indices(lg, ks[s])
            assert ids[s] == want, (s, ids[s], want)
            l64 = lg.astype(np.float64)
            mx = l64.max()
            ref = [float(l64[i] - (np.log(np.exp(l64 - mx).sum()) + mx)) for i in want]
            assert np.allclose(lps[s], ref, atol=2e-5), (s, lps[s], ref)
            x, tok = out, ids[s][0]
    finally:
        d.close()
        hd.close()
