"""The CPU baseline (oracle/cpu_q8k.c, oracle/cpu_baseline.py): candle's CPU
path for QMatMul -- per-row Q8_K activation quantisation (ggml's
quantize_row_q8_K) and integer block dot products (vec_dot_q4_K_q8_K /
vec_dot_q6_K_q8_K) -- pinned by known answers of the quantiser, by exact
restatements of the dot products on the dequantised blocks, and by the f64
matmul within the Q8_K quantisation error."""
import numpy as np
import pytest

import cpu_baseline as C
import oracle as O


def test_q8k_quantiser_known_answers():
    x = np.zeros(256, np.float32)
    q = C.quantize_q8k(x)
    assert q["d"][0] == 0 and not q["qs"].any() and not q["bsums"].any()
    # the element of largest magnitude maps to -128 (iscale = -128 / max)
    x[3], x[10] = 2.0, -1.0
    q = C.quantize_q8k(x)
    assert q["d"][0] == np.float32(1.0 / (-128.0 / 2.0))
    assert q["qs"][0][3] == -128 and q["qs"][0][10] == 64
    # a negative maximum: iscale > 0, so it still maps to -128
    x[:] = 0
    x[0], x[1] = -4.0, 1.0
    q = C.quantize_q8k(x)
    assert q["qs"][0][0] == -128 and q["qs"][0][1] == 32
    # +max beside -max of the same magnitude: the later one lands on +128, capped at 127
    x[:] = 0
    x[5], x[6] = 3.0, -3.0
    q = C.quantize_q8k(x)
    assert q["qs"][0][5] == -128 and q["qs"][0][6] == 127


def test_q8k_round_trip_and_bsums():
    rng = np.random.default_rng(3)
    x = rng.standard_normal(1024).astype(np.float32)
    q = C.quantize_q8k(x)
    for b in range(4):
        d = float(q["d"][b])
        xb = x[256 * b:256 * (b + 1)].astype(np.float64)
        assert np.max(np.abs(q["qs"][b] * d - xb)) <= abs(d) * 0.5 * (1 + 1e-6) + 1e-12
        assert np.array_equal(q["bsums"][b], q["qs"][b].reshape(16, 16).astype(np.int32).sum(1))


def _blocks(fmt, rows, K, seed):
    x = (np.random.default_rng(seed).standard_normal((rows, K)) * 0.05).astype(np.float32)
    raw = np.empty(rows * (K // 256) * (144 if fmt == O.Q4_K else 210), np.uint8)
    O.lib().or_quantize(fmt, O._p(x), rows * K // 256, O._p(raw))
    return raw.reshape(rows, -1)


@pytest.mark.parametrize("fmt", [O.Q4_K, O.Q6_K])
def test_dot_products_equal_the_dequantised_sum(fmt):
    """sum over superblocks of d_x * (integer form) = sum_e deq(W)[e] * d_x q8[e]
    (exact algebra; only f32 rounding separates the two), SIMD = plain C bit for bit."""
    K, rows = 1024, 24
    W = _blocks(fmt, rows, K, 11 + fmt)
    rng = np.random.default_rng(fmt)
    for r in range(rows):
        x = rng.standard_normal(K).astype(np.float32)
        xq = C.quantize_q8k(x)
        xd = np.concatenate([xq["qs"][b].astype(np.float64) * float(xq["d"][b]) for b in range(K // 256)])
        w = np.empty(K, np.float32)
        O.lib().or_dequant(fmt, O._p(W[r]), K // 256, O._p(w))
        ref = float(np.dot(w.astype(np.float64), xd))
        scale = float(np.sum(np.abs(w.astype(np.float64) * xd))) + 1e-30
        got_c = C.dot_q8k(fmt, W[r], xq, simd=False)
        got_v = C.dot_q8k(fmt, W[r], xq, simd=True)
        assert abs(got_c - ref) <= 1e-5 * scale, (r, got_c, ref)
        assert got_v == got_c, (r, got_v, got_c)


@pytest.mark.parametrize("fmt", [O.Q4_K, O.Q6_K])
def test_cpu_matmul_tracks_the_f64_matmul(fmt):
    K, N, M = 512, 96, 5
    W = _blocks(fmt, N, K, 40 + fmt)
    x = np.random.default_rng(9).standard_normal((M, K)).astype(np.float32)
    y = C.qmatmul_q8k(fmt, W.reshape(-1), N, K, x)
    ref = np.empty((M, N), np.float32)
    O.lib().or_qmatmul(fmt, O._p(W.reshape(-1)), N, K, O._p(x), M, O._p(ref))
    # the activation rounding of Q8_K: |x - q d| <= d/2 = max|x| / 256 per element
    assert np.max(np.abs(y - ref)) <= 0.02 * np.max(np.abs(ref)), float(np.max(np.abs(y - ref)))


def test_cpu_attention_matches_f64():
    rng = np.random.default_rng(2)
    M, P, nh, nkv, hd = 3, 17, 4, 2, 8
    q = rng.standard_normal((M, nh, hd)).astype(np.float32)
    kc = rng.standard_normal((nkv, P + M, hd)).astype(np.float32)
    vc = rng.standard_normal((nkv, P + M, hd)).astype(np.float32)
    got = C.attention(q, kc, vc, P)
    for i in range(M):
        for h in range(nh):
            kv = h // (nh // nkv)
            s = kc[kv, :P + i + 1].astype(np.float64) @ q[i, h].astype(np.float64) / np.sqrt(hd)
            p = np.exp(s - s.max())
            p /= p.sum()
            ref = p @ vc[kv, :P + i + 1].astype(np.float64)
            assert np.allclose(got[i, h], ref, rtol=1e-5, atol=1e-5)
