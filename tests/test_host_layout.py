"""The tile-interleaved device weight layout, checked on the host (no GPU).

* GGUF -> tiles -> GGUF is the identity for every format.
* For every lane and K-chunk, the fp16 codes the matmul builds from a tile
  block (sd_lane_codes: the kernel's own extraction code, compiled for the
  host) hold exactly the element's GGUF quant value, placed in the fragment
  slot the activation layout pairs it with.  The element codes come from the
  GGUF block specification (ggml's dequantize_row_q4_K / q5_K / q6_K / q8_0
  bit layouts, the format candle's QMatMul reads)."""
import numpy as np
import pytest

F32, Q8_0, Q4_K, Q5_K, Q6_K = 0, 8, 12, 13, 14
SB_BYTES = {Q4_K: 144, Q5_K: 176, Q6_K: 210, Q8_0: 272}
PERM = (0, 2, 1, 3)


@pytest.fixture(scope="module")
def S():
    import speculate_hip
    speculate_hip.load_library()
    return speculate_hip


def q_of(fmt, b, e):
    """Unsigned quant value of element e of one GGUF superblock b (bytes)."""
    if fmt == Q8_0:
        blk = b[34 * (e >> 5):34 * (e >> 5) + 34]
        return int(np.int8(blk[2 + (e & 31)])) + 128
    if fmt in (Q4_K, Q5_K):
        j, hi, l = e >> 6, (e >> 5) & 1, e & 31
        qs = b[16:] if fmt == Q4_K else b[48:]
        q = (qs[32 * j + l] >> 4) if hi else (qs[32 * j + l] & 15)
        if fmt == Q5_K:
            q += 16 * ((b[16 + l] >> (2 * j + hi)) & 1)
        return int(q)
    h, qd, l = e >> 7, (e >> 5) & 3, e & 31
    qlb, qhb = b[64 * h + 32 * (qd & 1) + l], b[128 + 32 * h + l]
    nib = (qlb >> 4) if qd >= 2 else (qlb & 15)
    return int(nib | (((qhb >> (2 * qd)) & 3) << 4))


def code_bits(fmt, slot, q):
    if fmt == Q8_0 or slot < 4:
        return 0x6400 | q           # 1024 + q
    return 0x5400 | (q << 4)        # 64 + q


def rand_blocks(fmt, rows, nsb, seed):
    rng = np.random.default_rng(seed)
    return rng.integers(0, 256, rows * nsb * SB_BYTES[fmt], dtype=np.uint8)


@pytest.mark.parametrize("fmt", [Q4_K, Q5_K, Q6_K, Q8_0])
def test_repack_roundtrip(S, fmt):
    rows, K = 48, 768
    g = rand_blocks(fmt, rows, K // 256, fmt)
    t = S.repack_gguf(fmt, g, rows, K)
    assert t.size == g.size and not np.array_equal(t, g)
    assert np.array_equal(S.unpack_tiles(fmt, t, rows, K), g)


@pytest.mark.parametrize("fmt", [Q4_K, Q5_K, Q6_K, Q8_0])
def test_lane_codes_match_gguf(S, fmt):
    rows, K = 32, 512
    nsb = K // 256
    g = rand_blocks(fmt, rows, nsb, 100 + fmt)
    t = S.repack_gguf(fmt, g, rows, K)
    tbb = 16 * SB_BYTES[fmt]
    for tile in range(rows // 16):
        for sb in range(nsb):
            tb = t[(tile * nsb + sb) * tbb:(tile * nsb + sb + 1) * tbb]
            for lane in range(64):
                r, grp = lane & 15, lane >> 4
                row = 16 * tile + r
                blk = g[(row * nsb + sb) * SB_BYTES[fmt]:(row * nsb + sb + 1) * SB_BYTES[fmt]]
                for c in range(8):
                    words = S.lane_codes(fmt, tb, lane, c)
                    for s in range(8):
                        half = (int(words[s >> 1]) >> (16 * (s & 1))) & 0xFFFF
                        e = 64 * grp + 32 * (s >> 2) + 4 * c + PERM[s & 3]
                        want = code_bits(fmt, s, q_of(fmt, blk, e))
                        assert half == want, (fmt, tile, sb, lane, c, s, hex(half), hex(want))


def test_repack_rejects_bad_shapes(S):
    g = np.zeros(16 * 144, np.uint8)
    with pytest.raises(S.ArgError):
        S.repack_gguf(Q4_K, g, 8, 512)
    with pytest.raises(S.UnsupportedMethod):
        S.repack_gguf(F32, g, 16, 256)


@pytest.mark.parametrize("fmt", [Q4_K, Q5_K])
def test_kquant_header_regrouped(S, fmt):
    """A K-quant tile header keeps d, dmin (bytes 0..3) and holds, for lane
    group g, the word w_g = sc_2g | sc_2g+1 << 6 | m_2g << 12 | m_2g+1 << 18
    with byte k at header byte 4 + 4k + g; (sc_j, m_j) are the GGUF block's
    get_scale_min_k4 values (the oracle's, pinned by its known answers)."""
    import oracle as O
    rows, K = 32, 512
    nsb = K // 256
    g = rand_blocks(fmt, rows, nsb, 100 + fmt)
    t = S.repack_gguf(fmt, g, rows, K)
    tbb = {Q4_K: 2304, Q5_K: 2816}[fmt]
    for row in (0, 5, 16, 31):
        for sb in range(nsb):
            blk = g[(row * nsb + sb) * SB_BYTES[fmt]:][:SB_BYTES[fmt]]
            hdr = t[((row >> 4) * nsb + sb) * tbb + (row & 15) * 16:][:16]
            assert bytes(hdr[:4]) == bytes(blk[:4])
            sm = [O.get_scale_min_k4(j, bytes(blk[4:16])) for j in range(8)]
            for grp in range(4):
                w = sum(int(hdr[4 + 4 * k + grp]) << (8 * k) for k in range(3))
                want = (sm[2 * grp][0] | sm[2 * grp + 1][0] << 6 | sm[2 * grp][1] << 12 | sm[2 * grp + 1][1] << 18)
                assert w == want, (row, sb, grp)
