"""Pins the oracle's fp16 conversion and GGUF block codecs.

The reference ships no golden vectors for this path (its block arithmetic
lives in candle 0.8.4, not vendored), so the oracle is pinned by:
  * binary16 conversion against numpy's IEEE float16 over every bit pattern;
  * hand-built known-answer blocks whose values follow from the published
    GGUF block layout with small-integer arithmetic (exact in f32), built so
    that swapping low/high nibbles, sub-blocks, scale/min fields or qh bits
    changes the answer;
  * the 12-byte 6-bit scale field being a bijection (96 bits <-> 16 values);
  * encoder/decoder consistency: dequant(quantize(x)) within half a step.
"""
import numpy as np
import pytest

import oracle as O


def test_f16_to_f32_all_patterns():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = O.f16_bits_to_f32(h)
    exp = h.view(np.float16).astype(np.float32)
    nan = np.isnan(exp)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), exp[~nan].view(np.uint32))


def test_f32_to_f16_rounding():
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2**32, 400000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    # add halfway cases, subnormal boundaries and overflow edges
    special = np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e-8, 2.0**-24, 2.0**-25, 3 * 2.0**-26,
                        2.0**-14, 2.0**-14 - 2.0**-25, 1.0 + 2.0**-11, 1.0 + 3 * 2.0**-11, np.inf, -np.inf],
                       np.float32)
    x = np.concatenate([x, special])
    got = O.f32_to_f16_bits(x)
    with np.errstate(over="ignore", invalid="ignore"):
        exp = x.astype(np.float16).view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], exp[~nan])
    assert np.all((got[nan] & 0x7C00) == 0x7C00) and np.all(got[nan] & 0x3FF)


def _scales_field(sc, mn):
    """Pack 8 6-bit scales and mins: bytes 0-3 hold sc0-3 (+ top bits of sc4-7),
    bytes 4-7 hold m0-3 (+ top bits of m4-7), bytes 8-11 hold the low nibbles
    of sc4-7 (low half) and m4-7 (high half)."""
    q = [0] * 12
    for j in range(4):
        q[j] = sc[j] | ((sc[j + 4] >> 4) << 6)
        q[j + 4] = mn[j] | ((mn[j + 4] >> 4) << 6)
        q[j + 8] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    return bytes(q)


def test_scale_min_field_kat():
    # only byte 0 set to 63 -> scale 0 is 63, everything else 0
    q = bytes([63] + [0] * 11)
    assert O.get_scale_min_k4(0, q) == (63, 0)
    for j in range(1, 8):
        assert O.get_scale_min_k4(j, q) == (0, 0)
    # byte 8 = 0x5A -> scale 4 low nibble 0xA, min 4 low nibble 0x5
    q = bytes([0] * 8 + [0x5A, 0, 0, 0])
    assert O.get_scale_min_k4(4, q) == (0xA, 0x5)
    # top two bits of byte 0 are the high bits of scale 4; of byte 4 of min 4
    q = bytes([0xC0, 0, 0, 0, 0x40, 0, 0, 0, 0, 0, 0, 0])
    assert O.get_scale_min_k4(4, q) == (0x30, 0x10)
    assert O.get_scale_min_k4(0, q) == (0, 0)


def test_scale_min_field_bijection():
    rng = np.random.default_rng(1)
    for _ in range(300):
        sc = [int(v) for v in rng.integers(0, 64, 8)]
        mn = [int(v) for v in rng.integers(0, 64, 8)]
        q = _scales_field(sc, mn)
        assert [O.get_scale_min_k4(j, q) for j in range(8)] == list(zip(sc, mn))
    # every one of the 96 bits moves exactly one unpacked value by a power of two
    for bit in range(96):
        q = bytearray(12)
        q[bit // 8] |= 1 << (bit % 8)
        vals = [v for j in range(8) for v in O.get_scale_min_k4(j, bytes(q))]
        nz = [v for v in vals if v]
        assert len(nz) == 1 and (nz[0] & (nz[0] - 1)) == 0, (bit, vals)


def _f16(x):
    return np.array([x], np.float16).view(np.uint16)[0]


def _q4k_block(d, dmin, sc, mn, qfun):
    b = bytearray(144)
    b[0:2] = int(_f16(d)).to_bytes(2, "little")
    b[2:4] = int(_f16(dmin)).to_bytes(2, "little")
    b[4:16] = _scales_field(sc, mn)
    for j in range(4):
        for l in range(32):
            b[16 + 32 * j + l] = qfun(64 * j + l) | (qfun(64 * j + 32 + l) << 4)
    return np.frombuffer(bytes(b), np.uint8)


def test_q4k_known_answer():
    sc = [1, 2, 3, 4, 5, 6, 7, 63]
    mn = [0, 1, 2, 3, 4, 5, 6, 7]
    qf = lambda e: (e * 7 + e // 32) % 16
    blk = _q4k_block(1.0, 0.5, sc, mn, qf)
    y = O.dequant(O.Q4_K, blk, 256)
    exp = np.array([1.0 * sc[e // 32] * qf(e) - 0.5 * mn[e // 32] for e in range(256)], np.float32)
    assert np.array_equal(y, exp)


def test_q4k_zero_scales_and_special_d():
    blk = _q4k_block(0.0, 2.0, [0] * 8, [3] * 8, lambda e: e % 16)
    assert np.array_equal(O.dequant(O.Q4_K, blk, 256), np.full(256, -6.0, np.float32))
    # subnormal super-scale: d = 2^-24
    blk = _q4k_block(2.0 ** -24, 0.0, [1] * 8, [0] * 8, lambda e: 15)
    assert np.all(O.dequant(O.Q4_K, blk, 256) == np.float32(15 * 2.0 ** -24))


def test_q5k_known_answer():
    sc = [2, 3, 5, 7, 11, 13, 17, 19]
    mn = [1, 0, 1, 0, 1, 0, 1, 0]
    q5 = lambda e: (e * 5 + 3) % 32
    b = bytearray(176)
    b[0:2] = int(_f16(0.25)).to_bytes(2, "little")
    b[2:4] = int(_f16(1.0)).to_bytes(2, "little")
    b[4:16] = _scales_field(sc, mn)
    for j in range(4):
        for l in range(32):
            lo, hi = q5(64 * j + l), q5(64 * j + 32 + l)
            b[48 + 32 * j + l] = (lo & 15) | ((hi & 15) << 4)
            b[16 + l] |= ((lo >> 4) << (2 * j)) | ((hi >> 4) << (2 * j + 1))
    y = O.dequant(O.Q5_K, np.frombuffer(bytes(b), np.uint8), 256)
    exp = np.array([0.25 * sc[e // 32] * q5(e) - 1.0 * mn[e // 32] for e in range(256)], np.float32)
    assert np.array_equal(y, exp)


def test_q6k_known_answer():
    sc = [((-1) ** k) * (k + 1) for k in range(16)]
    q6 = lambda e: (e * 11 + 5) % 64
    b = bytearray(210)
    for h in range(2):
        for l in range(32):
            q1, q2, q3, q4 = (q6(128 * h + l), q6(128 * h + 32 + l), q6(128 * h + 64 + l), q6(128 * h + 96 + l))
            b[64 * h + l] = (q1 & 15) | ((q3 & 15) << 4)
            b[64 * h + 32 + l] = (q2 & 15) | ((q4 & 15) << 4)
            b[128 + 32 * h + l] = (q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6)
    for k in range(16):
        b[192 + k] = sc[k] & 0xFF
    b[208:210] = int(_f16(0.5)).to_bytes(2, "little")
    y = O.dequant(O.Q6_K, np.frombuffer(bytes(b), np.uint8), 256)
    exp = np.array([0.5 * sc[e // 16] * (q6(e) - 32) for e in range(256)], np.float32)
    assert np.array_equal(y, exp)


def test_q80_known_answer():
    q = [((-1) ** l) * (l * 4) for l in range(32)]
    b = bytearray(34)
    b[0:2] = int(_f16(-0.125)).to_bytes(2, "little")
    for l in range(32):
        b[2 + l] = q[l] & 0xFF
    y = O.dequant(O.Q8_0, np.frombuffer(bytes(b), np.uint8), 32)
    assert np.array_equal(y, np.array([-0.125 * v for v in q], np.float32))


@pytest.mark.parametrize("fmt,levels", [(O.Q4_K, 15), (O.Q5_K, 31), (O.Q6_K, 63), (O.Q8_0, 254)])
def test_quantize_dequant_consistency(fmt, levels):
    """dequant(quantize(x)) is within one quantisation step of x (encoder and
    decoder agree on the layout; a packing mismatch gives O(range) errors)."""
    rng = np.random.default_rng(fmt)
    n = 256 * 64
    x = (rng.standard_normal(n) * 0.02).astype(np.float32)
    y = O.dequant(fmt, O.quantize(fmt, x), n)
    sub = 32 if fmt in (O.Q4_K, O.Q5_K, O.Q8_0) else 16
    xs = x.reshape(-1, sub)
    span = np.maximum(xs.max(1) - np.minimum(xs.min(1), 0), np.abs(xs).max(1) * 2)
    step = span / levels
    err = np.abs(y.reshape(-1, sub) - xs).max(1)
    # 6-bit scale rounding can stretch a step by up to 1/63 per unit of scale
    assert np.all(err <= 1.6 * step + 1e-6), float((err / step).max())
