"""sd_model_qmatmul_noalloc (the allocation-free variant of sd_model_qmatmul)
through the C ABI, on device buffers the test allocates itself with the HIP
runtime the library is linked against: bit-identical to sd_model_qmatmul on
two calls in a row (the second with fewer rows, so the shared scratch holds a
longer previous input), on both the M <= 16 and the M > 16 kernels, on the
handle's stream and on a stream the caller creates, and a clear error for
inputs beyond the scratch."""
import ctypes

import numpy as np
import pytest

from _models import MIX_IDS, hip_cfg, oracle_cfg

pytestmark = pytest.mark.gpu

H2D, D2H = 1, 2


def _hip_runtime():
    # the library's own HIP runtime (already loaded with it: same soname)
    rt = ctypes.CDLL("libamdhip64.so.7")
    rt.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
    rt.hipFree.argtypes = [ctypes.c_void_p]
    rt.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    rt.hipStreamCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
    rt.hipStreamSynchronize.argtypes = [ctypes.c_void_p]
    rt.hipStreamDestroy.argtypes = [ctypes.c_void_p]
    for f in (rt.hipMalloc, rt.hipFree, rt.hipMemcpy, rt.hipDeviceSynchronize, rt.hipStreamCreate,
              rt.hipStreamSynchronize, rt.hipStreamDestroy):
        f.restype = ctypes.c_int
    return rt


class DevBuf:
    def __init__(self, rt, nbytes):
        self.rt, self.p = rt, ctypes.c_void_p()
        assert rt.hipMalloc(ctypes.byref(self.p), nbytes) == 0
        self.n = nbytes

    def put(self, a):
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.n
        assert self.rt.hipMemcpy(self.p, a.ctypes.data_as(ctypes.c_void_p), a.nbytes, H2D) == 0

    def get(self, shape, dtype=np.float32):
        out = np.empty(shape, dtype)
        assert self.rt.hipMemcpy(out.ctypes.data_as(ctypes.c_void_p), self.p, out.nbytes, D2H) == 0
        return out

    def free(self):
        self.rt.hipFree(self.p)


def _noalloc(hip, dec, layer, kind, xbuf, rows, ybuf, stream=None):
    lib = hip.load_library()
    lib.sd_model_qmatmul_noalloc.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p,
                                             ctypes.c_size_t, ctypes.c_void_p, ctypes.c_void_p]
    lib.sd_model_qmatmul_noalloc.restype = ctypes.c_int32
    return lib.sd_model_qmatmul_noalloc(dec._h, layer, kind, xbuf.p, rows, ybuf.p, stream)


@pytest.mark.parametrize("mix,kind,rows", [("q4_k", 9, (12, 5)), ("q4_k_m", 9, (64, 17)), ("q5k_q80", 3, (40, 3)),
                                           ("q6_k", 4, (16, 1))])
def test_noalloc_matches_qmatmul(hip, mix, kind, rows):
    ocfg = oracle_cfg(mix=mix, n_layers=2, vocab=2048)
    dec = hip.HipQuantDecoder(hip_cfg(hip, ocfg))
    try:
        dec.synthesize(MIX_IDS[mix], ocfg.seed, ocfg.weight_std)
        rt = _hip_runtime()
        layer = 1
        N, K = ocfg.shape(kind)
        xb, yb = DevBuf(rt, 128 * K * 4), DevBuf(rt, 128 * N * 4)
        rng = np.random.default_rng(kind * 100 + rows[0])
        try:
            for M in rows:  # the second call has fewer rows than the first
                x = rng.standard_normal((M, K)).astype(np.float32)
                xb.put(x)
                assert _noalloc(hip, dec, layer, kind, xb, M, yb) == 0, hip.load_library().sd_last_error()
                dec.synchronize()
                got = yb.get((M, N))
                ref = dec.qmatmul(layer, kind, x)
                assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (mix, kind, M)
        finally:
            xb.free()
            yb.free()
    finally:
        dec.close()


def test_noalloc_on_a_caller_stream(hip):
    """The stream argument: the call is enqueued on the caller's own stream
    (created here with hipStreamCreate), which the caller synchronises."""
    ocfg = oracle_cfg(mix="q4_k_m", n_layers=2, vocab=2048)
    dec = hip.HipQuantDecoder(hip_cfg(hip, ocfg))
    try:
        dec.synthesize(MIX_IDS["q4_k_m"], ocfg.seed, ocfg.weight_std)
        dec.synchronize()
        rt = _hip_runtime()
        layer, kind = 1, 7
        N, K = ocfg.shape(kind)
        xb, yb = DevBuf(rt, 128 * K * 4), DevBuf(rt, 128 * N * 4)
        stream = ctypes.c_void_p()
        assert rt.hipStreamCreate(ctypes.byref(stream)) == 0
        rng = np.random.default_rng(77)
        try:
            for M in (40, 9, 2):
                x = rng.standard_normal((M, K)).astype(np.float32)
                xb.put(x)
                assert _noalloc(hip, dec, layer, kind, xb, M, yb, stream) == 0, hip.load_library().sd_last_error()
                assert rt.hipStreamSynchronize(stream) == 0
                got = yb.get((M, N))
                ref = dec.qmatmul(layer, kind, x)
                assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), M
        finally:
            rt.hipStreamSynchronize(stream)
            rt.hipStreamDestroy(stream)
            xb.free()
            yb.free()
    finally:
        dec.close()


def test_noalloc_rejects_inputs_beyond_the_scratch(hip):
    ocfg = oracle_cfg(n_layers=1, vocab=2048, ffn=18944)  # ffn_down: K = 18944
    dec = hip.HipQuantDecoder(hip_cfg(hip, ocfg))
    try:
        dec.synthesize(MIX_IDS["q4_k"], ocfg.seed, ocfg.weight_std)
        rt = _hip_runtime()
        K, N = 18944, 512
        xb, yb = DevBuf(rt, 128 * K * 4), DevBuf(rt, 128 * N * 4)
        try:
            x = np.random.default_rng(1).standard_normal((128, K)).astype(np.float32)
            xb.put(x)
            # 128 * 18944 * 2 bytes > 4 MiB
            assert _noalloc(hip, dec, 0, 9, xb, 128, yb) == hip.SD_ERR_ARG
            assert b"scratch" in hip.load_library().sd_last_error()
            assert _noalloc(hip, dec, 0, 9, xb, 0, yb) == hip.SD_ERR_ARG
            # the largest that fits: 110 rows
            assert _noalloc(hip, dec, 0, 9, xb, 110, yb) == 0
            dec.synchronize()
            ref = dec.qmatmul(0, 9, x[:110])
            assert np.array_equal(yb.get((110, N)).view(np.uint32), ref.view(np.uint32))
        finally:
            xb.free()
            yb.free()
    finally:
        dec.close()
