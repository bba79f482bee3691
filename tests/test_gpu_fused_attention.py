"""The fused Q/K/V + attention launch against the separate launches it
replaces.

Up to 16 rows, at widths where the Q/K/V matmul runs eight waves per
workgroup (the Llama-3-8B and Qwen2.5-7B shapes), the attention's workgroups
join the Q/K/V launch and wait there for the matmul's rows.  Both routes run
the same arithmetic, so a decoder created with SD_ATTN_UNFUSED=1 (separate
launches) must give bit-identical logits and KV rows: rows 1..16 over one
key split (a key range that starts inside the new rows' 32-key block, and one
that does not), one row over 5 and 8 splits, the decode step, repeated steps
(the launch must leave its completion word clear, or the next launch's
attention would not wait), a wait that gives up, and the Qwen2 shape (4 KV
heads, QKV bias, half rotation, seven query tiles).  The launch is taken only
where all its workgroups fit on the CUs at once (192 matmul workgroups at the
Llama shape leave 64 CUs for the attention's KV heads x splits x query
tiles): each case asserts which route the fused decoder took, from its
per-launch profile, so the cases past that limit check the fallback.  Parity
with the oracle at these shapes is test_gpu_full_width_llama.py /
test_gpu_full_width_qwen.py's.
"""
import os

import numpy as np
import pytest

from _fullwidth import LLAMA8B, QWEN7B

pytestmark = pytest.mark.gpu

SEED = 0x5EED0009


def make(hip, shape, mix, ctx, unfused):
    if unfused:
        os.environ["SD_ATTN_UNFUSED"] = "1"
    try:
        dec = hip.HipQuantDecoder(hip.Config(arch=0 if shape["arch"] == "llama" else 1, n_layers=2,
                                             hidden=shape["hidden"], n_heads=shape["n_heads"],
                                             n_kv_heads=shape["n_kv_heads"], head_dim=shape["head_dim"],
                                             ffn=shape["ffn"], vocab=shape["vocab"], rope_theta=shape["rope_theta"],
                                             rms_eps=shape["rms_eps"], ctx_len=ctx, max_batch=64))
    finally:
        os.environ.pop("SD_ATTN_UNFUSED", None)
    dec.synthesize(mix, SEED, 0.02)
    return dec


@pytest.fixture(scope="module")
def llama_pair(hip):
    fused = make(hip, LLAMA8B, hip.MIX_Q4_K_M, 4608, False)
    sep = make(hip, LLAMA8B, hip.MIX_Q4_K_M, 4608, True)
    yield fused, sep
    fused.close()
    sep.close()


def same_step(fused, sep, hist, drafts, kv_seed, n_kv, route=None):
    """One verify pass of hist[-1] + drafts after the synthetic prefix hist[:-1]
    on both decoders: logits and the appended K / V rows equal bit for bit.
    route: whether the fused decoder must take the fused launch (None: not
    checked)."""
    for d in (fused, sep):
        d.prime_synthetic(hist, kv_seed)
    P = len(hist) - 1
    if route is not None:
        fused.profile_enable(True)
    try:
        a = fused.batched_logits(drafts)
    finally:
        if route is not None:
            classes = {c for c, _, _ in fused.profile_read()}
            fused.profile_enable(False)
    if route is not None:
        assert ("qkv_attn" in classes) == route, (P, len(drafts), sorted(classes))
    b = sep.batched_logits(drafts)
    assert np.isfinite(a).all()
    assert np.array_equal(a, b), (P, len(drafts), float(np.max(np.abs(a - b))))
    M = len(drafts) + 1
    for layer in (0, 1):
        for which in (0, 1):
            for h in range(n_kv):
                ra = fused.read_kv_rows(layer, which, h, P, M)
                rb = sep.read_kv_rows(layer, which, h, P, M)
                assert np.array_equal(ra, rb), (P, M, layer, which, h)
    return a


# prefixes: 1 split up to 512 positions (500 and 512 put the new rows inside /
# at the start of a 32-key block), 5, 5 and 8 splits at 1100, 2500 and 4000;
# 8 KV heads x splits x query tiles (1, 2, 3, 4 for 1, 5, 9, 16 rows) fit in
# the 64 CUs the matmul leaves up to 512 positions and for one row
@pytest.mark.parametrize("P", [3, 40, 500, 512, 1100, 2500, 4000])
@pytest.mark.parametrize("M", [1, 5, 9, 16])
def test_llama_fused_equals_separate(hip, llama_pair, P, M):
    fused, sep = llama_pair
    V = LLAMA8B["vocab"]
    rng = np.random.default_rng(P * 131 + M)
    hist = [int(v) for v in rng.integers(0, V, P + 1)]
    drafts = [int(v) for v in rng.integers(0, V, M - 1)]
    same_step(fused, sep, hist, drafts, 1000 + P, LLAMA8B["n_kv_heads"], route=P <= 512 or M == 1)


def test_llama_fused_repeated_steps(hip, llama_pair):
    """Several fused launches in a row (32 layers' worth over 16 steps) give
    the first step's result each time: every launch left its completion word
    and split counters clear."""
    fused, sep = llama_pair
    V = LLAMA8B["vocab"]
    rng = np.random.default_rng(77)
    hist = [int(v) for v in rng.integers(0, V, 513)]
    drafts = [int(v) for v in rng.integers(0, V, 4)]
    ref = same_step(fused, sep, hist, drafts, 4242, LLAMA8B["n_kv_heads"], route=True)
    n0 = len(hist)
    for _ in range(16):
        fused.rollback_to(n0)
        again = fused.batched_logits(drafts)
        assert np.array_equal(again, ref)
    # the decode step (one row) through observe / next_logits
    fused.rollback_to(n0)
    sep.rollback_to(n0)
    for t in drafts:
        fused.observe([t])
        sep.observe([t])
        assert np.array_equal(fused.next_logits(), sep.next_logits())


# (P, M) that take the fused launch: one key split, and five (one row)
@pytest.mark.parametrize("P,M", [(512, 5), (2500, 1)])
def test_llama_fused_wait_gives_up_then_recovers(hip, llama_pair, P, M):
    """Fault injection from the host (SD_ATTN_WAIT_TEST=64): the fused
    launch's attention waits for a launch number no producer writes and gives
    up after 64 reads, so every workgroup still ends normally.  The step
    raises BackendError at its synchronisation, and the same handle's next
    step (split counters cleared) equals the separate launches bit for bit."""
    fused, sep = llama_pair
    V = LLAMA8B["vocab"]
    rng = np.random.default_rng(P + 7)
    hist = [int(v) for v in rng.integers(0, V, P + 1)]
    drafts = [int(v) for v in rng.integers(0, V, M - 1)]
    fused.prime_synthetic(hist, 31 + P)
    os.environ["SD_ATTN_WAIT_TEST"] = "64"
    try:
        with pytest.raises(hip.BackendError, match="gave up waiting"):
            fused.batched_logits(drafts)
    finally:
        os.environ.pop("SD_ATTN_WAIT_TEST", None)
    same_step(fused, sep, hist, drafts, 31 + P, LLAMA8B["n_kv_heads"], route=True)


def test_qwen_fused_equals_separate(hip):
    fused = make(hip, QWEN7B, hip.MIX_Q5K_Q80, 2304, False)
    sep = make(hip, QWEN7B, hip.MIX_Q5K_Q80, 2304, True)
    try:
        V = QWEN7B["vocab"]
        rng = np.random.default_rng(9)
        # 144 matmul workgroups leave 112 CUs: 4 KV heads x 9 splits x 4
        # query tiles at 2048 positions do not fit, 4 x 1 x 7 at 300 do
        for P, M, route in ((2048, 9, False), (300, 16, True), (31, 1, True)):
            hist = [int(v) for v in rng.integers(0, V, P + 1)]
            drafts = [int(v) for v in rng.integers(0, V, M - 1)]
            same_step(fused, sep, hist, drafts, 77 + P, QWEN7B["n_kv_heads"], route=route)
    finally:
        fused.close()
        sep.close()
