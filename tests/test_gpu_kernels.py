"""GPU parity of the block generator, the exact dequantiser and the fused
dequant-matmul (K1) against the CPU oracle, through the C ABI."""
import numpy as np
import pytest

import oracle as O
from _models import MIX_IDS, all_tensor_keys, hip_cfg, oracle_cfg, rel_err

pytestmark = pytest.mark.gpu

MIXES = ["q4_k", "q4_k_m", "q5k_q80", "q6_k", "q5_k", "q8_0"]


def _model(hip, mix, **over):
    ocfg = oracle_cfg(mix=mix, **over)
    dec = hip.HipQuantDecoder(hip_cfg(hip, ocfg))
    dec.synthesize(MIX_IDS[mix], ocfg.seed, ocfg.weight_std)
    return ocfg, dec


@pytest.mark.parametrize("mix", MIXES)
def test_synth_blocks_bit_exact(hip, mix):
    """GPU generator == CPU generator, byte for byte, for every tensor."""
    ocfg, dec = _model(hip, mix, n_layers=2, vocab=2048)
    for (li, k) in all_tensor_keys(ocfg):
        fmt, expect = O.synth_tensor(ocfg, li, k)
        f, rows, K, nbytes = dec.tensor_info(li, k)
        assert f == fmt and nbytes == expect.size, (li, k)
        got = dec.get_tensor(li, k)
        assert np.array_equal(got, expect), (mix, li, k)


@pytest.mark.parametrize("mix", MIXES)
def test_dequant_bit_exact(hip, mix):
    """Device dequantisation (device block layout) == oracle dequantisation, bitwise."""
    ocfg, dec = _model(hip, mix, n_layers=1, vocab=2048)
    for (li, k) in all_tensor_keys(ocfg):
        fmt, raw = O.synth_tensor(ocfg, li, k)
        if fmt == O.F32:
            continue
        rows, K = ocfg.shape(k)
        got = dec.dequant_tensor(li, k)
        exp = O.dequant_matrix(fmt, raw, rows, K)
        assert np.array_equal(got.view(np.uint32), exp.view(np.uint32)), (mix, li, k)


@pytest.mark.parametrize("mix", ["q4_k", "q6_k", "q8_0"])
def test_set_tensor_roundtrip(hip, mix):
    """Host GGUF bytes -> device layout -> GGUF bytes is the identity."""
    ocfg = oracle_cfg(mix=mix, n_layers=1, vocab=2048)
    dec = hip.HipQuantDecoder(hip_cfg(hip, ocfg))
    rng = np.random.default_rng(3)
    fmt = ocfg.fmt(0, O.K_FFN_DOWN)
    rows, K = ocfg.shape(O.K_FFN_DOWN)
    raw = O.quantize(fmt, rng.standard_normal(rows * K).astype(np.float32) * 0.02)
    dec.set_tensor(0, O.K_FFN_DOWN, fmt, raw)
    assert np.array_equal(dec.get_tensor(0, O.K_FFN_DOWN), raw)
    got = dec.dequant_tensor(0, O.K_FFN_DOWN)
    assert np.array_equal(got.view(np.uint32), O.dequant_matrix(fmt, raw, rows, K).view(np.uint32))


def int_path(fmt, M):
    """Up to 16 rows, Q4_K and Q5_K weights enter the MFMA as the exact
    integers sc * q, with d, dmin and the mins applied in f32; the other
    formats and larger M use fp16 weights."""
    return M <= 16 and fmt in (O.Q4_K, O.Q5_K)


def kquant_fields(fmt, raw, rows, K):
    """Per weight (q, sc, m, d, dmin) of a Q4_K / Q5_K matrix, decoded from the
    GGUF blocks (ggml's dequantize_row_q4_K / _q5_K element order), each
    [rows, K] float64; checked against the oracle's dequantisation below."""
    bb = O.BLOCK_BYTES[fmt]
    blk = raw.reshape(-1, bb)
    nb = blk.shape[0]
    d = blk[:, 0:2].copy().view(np.float16)[:, 0].astype(np.float64)
    dmin = blk[:, 2:4].copy().view(np.float16)[:, 0].astype(np.float64)
    sc = np.zeros((nb, 8))
    mn = np.zeros((nb, 8))
    for b in range(nb):
        sb = bytes(blk[b, 4:16])
        for j in range(8):
            sc[b, j], mn[b, j] = O.get_scale_min_k4(j, sb)
    q = np.zeros((nb, 256))
    qs = blk[:, 16:144] if fmt == O.Q4_K else blk[:, 48:176]
    for c in range(4):
        lo = (qs[:, 32 * c:32 * c + 32] & 15).astype(np.float64)
        hi = (qs[:, 32 * c:32 * c + 32] >> 4).astype(np.float64)
        if fmt == O.Q5_K:
            qh = blk[:, 16:48]
            lo += 16 * ((qh >> (2 * c)) & 1)
            hi += 16 * ((qh >> (2 * c + 1)) & 1)
        q[:, 64 * c:64 * c + 32] = lo
        q[:, 64 * c + 32:64 * c + 64] = hi
    sub = np.arange(256) // 32
    f = lambda a: a.reshape(rows, K)  # noqa: E731
    return (f(q), f(sc[:, sub]), f(mn[:, sub]), f(np.repeat(d, 256)), f(np.repeat(dmin, 256)))


def wide_kquant_weights(fmt, raw, rows, K):
    """The fp16 weights the M > 16 kernel multiplies with for Q4_K / Q5_K:
    round_f16(q * s16 - m16), s16 = fp16(d * sc), m16 = fp16(dmin * m)
    (exact products and difference in f64, one rounding each)."""
    q, sc, mn, d, dmin = kquant_fields(fmt, raw, rows, K)
    s16 = (d * sc).astype(np.float16).astype(np.float64)
    m16 = (dmin * mn).astype(np.float16).astype(np.float64)
    return (q * s16 - m16).astype(np.float16).astype(np.float32)


def q6k_fields(raw, rows, K):
    """Per weight (q6 - 32, sc, d) of a Q6_K matrix from its GGUF blocks (ggml's
    dequantize_row_q6_K element order), each [rows, K] float64."""
    blk = raw.reshape(-1, 210)
    nb = blk.shape[0]
    ql, qh = blk[:, 0:128].astype(np.int64), blk[:, 128:192].astype(np.int64)
    scs = blk[:, 192:208].copy().view(np.int8).astype(np.float64)
    d = blk[:, 208:210].copy().view(np.float16)[:, 0].astype(np.float64)
    q = np.zeros((nb, 256))
    sc = np.zeros((nb, 256))
    for h in range(2):
        L, H, S = ql[:, 64 * h:64 * h + 64], qh[:, 32 * h:32 * h + 32], scs[:, 8 * h:8 * h + 8]
        for l in range(32):
            base = 128 * h + l
            vals = [(L[:, l] & 15) | (((H[:, l] >> 0) & 3) << 4), (L[:, l + 32] & 15) | (((H[:, l] >> 2) & 3) << 4),
                    (L[:, l] >> 4) | (((H[:, l] >> 4) & 3) << 4), (L[:, l + 32] >> 4) | (((H[:, l] >> 6) & 3) << 4)]
            for j, v in enumerate(vals):
                q[:, base + 32 * j] = v - 32
                sc[:, base + 32 * j] = S[:, l // 16 + 2 * j]
    f = lambda a: a.reshape(rows, K)  # noqa: E731
    return f(q), f(sc), f(np.repeat(d, 256))


def operand_weights(fmt, raw, rows, K, M):
    """The weights K1 multiplies an M-row input with: exact on the integer
    path; round_f16(q * s16 - m16) for Q4_K / Q5_K and round_f16((q6 - 32) *
    fp16(d * sc)) for Q6_K otherwise (exact products, one rounding each);
    round_f16(W) for Q8_0 (one rounding of d * q)."""
    W = O.dequant_matrix(fmt, raw, rows, K)
    if int_path(fmt, M):
        return W
    if fmt in (O.Q4_K, O.Q5_K):
        return wide_kquant_weights(fmt, raw, rows, K)
    if fmt == O.Q6_K:
        q, sc, d = q6k_fields(raw, rows, K)
        s16 = (d * sc).astype(np.float16).astype(np.float64)
        return (q * s16).astype(np.float16).astype(np.float32)
    return O.round_f16(W)


def test_q6k_field_decoder_matches_oracle():
    """The test's Q6_K decoder reproduces the oracle's dequantisation (d * sc
    times q - 32 in f32, as ggml), bit for bit."""
    ocfg = oracle_cfg(mix="q6_k", n_layers=1, vocab=2048)
    fmt, raw = O.synth_tensor(ocfg, 0, O.K_FFN_DOWN)
    rows, K = ocfg.shape(O.K_FFN_DOWN)
    q, sc, d = q6k_fields(raw, rows, K)
    f32 = np.float32
    W = (d.astype(f32) * sc.astype(f32)) * q.astype(f32)
    assert np.array_equal(W.view(np.uint32), O.dequant_matrix(fmt, raw, rows, K).view(np.uint32))


@pytest.mark.parametrize("mix,kind", [("q4_k", O.K_ATTN_Q), ("q5_k", O.K_ATTN_O)])
def test_kquant_field_decoder_matches_oracle(mix, kind):
    """The test's block decoder reproduces the oracle's dequantisation
    (d * sc in f32 times q, minus dmin * m in f32, as ggml), bit for bit."""
    ocfg = oracle_cfg(mix=mix, n_layers=1, vocab=2048)
    fmt, raw = O.synth_tensor(ocfg, 0, kind)
    rows, K = ocfg.shape(kind)
    q, sc, mn, d, dmin = kquant_fields(fmt, raw, rows, K)
    f32 = np.float32
    W = (d.astype(f32) * sc.astype(f32)) * q.astype(f32) - dmin.astype(f32) * mn.astype(f32)
    assert np.array_equal(W.view(np.uint32), O.dequant_matrix(fmt, raw, rows, K).view(np.uint32))


CASES = [("q4_k", 0, O.K_ATTN_Q), ("q4_k", 0, O.K_FFN_DOWN), ("q6_k", 0, O.K_FFN_GATE),
         ("q5_k", 0, O.K_ATTN_O), ("q8_0", 0, O.K_FFN_UP), ("q8_0", 0, O.K_ATTN_K)]


@pytest.mark.parametrize("mix,layer,kind", CASES)
@pytest.mark.parametrize("M", [1, 5, 16, 17, 33, 60, 64, 100, 128])
def test_qmatmul_vs_oracle(hip, mix, layer, kind, M):
    """K1 against (a) its operands in f64 (tight): fp16 activations times the
    weights it uses (operand_weights: exact on the integer path, the emulated
    fp16 roundings otherwise), and (b) the f32 oracle QMatMul (the 1e-2
    relative contract)."""
    ocfg, dec = _model(hip, mix, n_layers=1, vocab=2048)
    fmt, raw = O.synth_tensor(ocfg, layer, kind)
    rows, K = ocfg.shape(kind)
    W = O.dequant_matrix(fmt, raw, rows, K)
    x = np.random.default_rng(M * 7 + kind).standard_normal((M, K)).astype(np.float32)
    y = dec.qmatmul(layer, kind, x)
    Wk = operand_weights(fmt, raw, rows, K, M)
    ref16 = O.round_f16(x).astype(np.float64) @ Wk.astype(np.float64).T
    ref32 = x.astype(np.float64) @ W.astype(np.float64).T
    assert rel_err(y, ref16) < 1e-4, rel_err(y, ref16)
    assert rel_err(y, ref32) < 1e-2, rel_err(y, ref32)


@pytest.mark.parametrize("mix,kind", [("q4_k", O.K_ATTN_Q), ("q5_k", O.K_ATTN_O)])
def test_qmatmul_int_path_one_hot(hip, mix, kind):
    """One-hot activations read single weights back out of the integer path:
    column k of the exact dequantised matrix, bit for bit (the products are
    exact, and no other column contributes)."""
    ocfg, dec = _model(hip, mix, n_layers=1, vocab=2048)
    fmt, raw = O.synth_tensor(ocfg, 0, kind)
    rows, K = ocfg.shape(kind)
    W = O.dequant_matrix(fmt, raw, rows, K)
    ks = [0, 1, 2, 3, 5, 31, 32, 63, 64, 100, 200, 255, 256, K - 1]
    x = np.zeros((len(ks), K), np.float32)
    for i, k in enumerate(ks):
        x[i, k] = 1.0
    y = dec.qmatmul(0, kind, x[:16])
    for i, k in enumerate(ks):
        np.testing.assert_allclose(y[i], W[:, k], rtol=2e-7, atol=1e-9, err_msg=f"k={k}")


@pytest.mark.parametrize("mix,kind", [("q4_k", O.K_ATTN_Q), ("q5_k", O.K_ATTN_O), ("q6_k", O.K_FFN_DOWN),
                                      ("q8_0", O.K_FFN_UP)])
def test_qmatmul_wide_one_hot(hip, mix, kind):
    """Above 16 rows, one-hot activations read the kernel's fp16 weights back
    out bit for bit (operand_weights: the emulated roundings)."""
    ocfg, dec = _model(hip, mix, n_layers=1, vocab=2048)
    fmt, raw = O.synth_tensor(ocfg, 0, kind)
    rows, K = ocfg.shape(kind)
    Wk = operand_weights(fmt, raw, rows, K, 64)
    ks = [0, 1, 2, 3, 5, 15, 16, 31, 32, 33, 63, 64, 100, 127, 128, 160, 200, 224, 255, 256, 300, K - 2, K - 1]
    ks += [K // 4 + 3 * i for i in range(41)]  # 64 rows: the kernel with 4 token tiles
    x = np.zeros((len(ks), K), np.float32)
    for i, k in enumerate(ks):
        x[i, k] = 1.0
    assert len(ks) > 16
    y = dec.qmatmul(0, kind, x)
    for i, k in enumerate(ks):
        assert np.array_equal(y[i].view(np.uint32), Wk[:, k].view(np.uint32)), f"k={k}"


@pytest.mark.parametrize("mix,kind", [("q4_k", O.K_ATTN_Q), ("q6_k", O.K_FFN_DOWN), ("q8_0", O.K_FFN_UP),
                                      ("q5_k", O.K_ATTN_V)])
def test_qmatmul_m_invariant(hip, mix, kind):
    """Up to 16 rows (the linear-verify shapes) row i of an M-row product equals
    the single-row product bit for bit: the K split is a function of the
    matrix only.  Past 16 rows the activation-staged kernel sums K in other
    slices (and uses Q4_K / Q5_K weights rounded to fp16), so rows agree to
    rounding (the reference's own GEMV and GEMM paths differ the same way,
    which is why its strict root mode exists)."""
    ocfg, dec = _model(hip, mix, n_layers=1, vocab=2048)
    fmt = O.synth_tensor(ocfg, 0, kind)[0]
    K = ocfg.shape(kind)[1]
    x = np.random.default_rng(11).standard_normal((128, K)).astype(np.float32)
    picks = (0, 3, 15, 16, 63, 64, 127)
    singles = [dec.qmatmul(0, kind, x[i:i + 1])[0] for i in picks]
    # exact against fp16-rounded weights: ~2e-4 apart (max over the row)
    tol = 1e-3 if int_path(fmt, 1) else 1e-5
    for M in (5, 9, 16, 17, 60, 64, 65, 128):
        y = dec.qmatmul(0, kind, x[:M])
        for j, i in enumerate(picks):
            if i >= M:
                continue
            if M <= 16:
                assert np.array_equal(y[i].view(np.uint32), singles[j].view(np.uint32)), (M, i)
            else:
                assert rel_err(y[i], singles[j].astype(np.float64)) < tol, (M, i)
