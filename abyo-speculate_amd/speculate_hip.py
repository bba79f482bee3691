"""Python binding of libspeculate_hip.so (the C ABI in include/speculate_hip.h).

``HipQuantDecoder`` mirrors the reference's ``LlamaQuantDecoder`` /
``Qwen2QuantDecoder`` surface -- the ``Decoder`` and ``TreeDecoder`` traits of
crates/speculate/src/model/mod.rs:39-236 -- method for method, with the same
error classes (``SamplingError``, ``CacheRollbackError``, ``BackendError``
standing for Error::Sampling / Error::CacheRollback / Error::Candle).

There is no CPU fallback: importing works anywhere, but constructing a
decoder needs the built HIP library and a GPU, and fails loudly otherwise.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass
from typing import List, Optional, Sequence, Tuple

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# SPECULATE_HIP_LIB selects another build of the same library (the CPU tests
# load the AddressSanitizer build of the host code through it)
LIB_PATH = os.environ.get("SPECULATE_HIP_LIB") or os.path.join(HERE, "libspeculate_hip.so")

# sd_status
SD_OK, SD_ERR_SAMPLING, SD_ERR_ROLLBACK, SD_ERR_BACKEND, SD_ERR_ARG, SD_ERR_UNSUPPORTED = range(6)
# formats (GGML type ids)
F32, Q8_0, Q4_K, Q5_K, Q6_K = 0, 8, 12, 13, 14
# tensor kinds
(TOK_EMBD, OUTPUT, OUTPUT_NORM, ATTN_Q, ATTN_K, ATTN_V, ATTN_OUTPUT, FFN_GATE, FFN_UP, FFN_DOWN,
 ATTN_NORM, FFN_NORM, ATTN_Q_BIAS, ATTN_K_BIAS, ATTN_V_BIAS) = range(15)
ARCH_LLAMA, ARCH_QWEN2 = 0, 1
MIX_Q4_K, MIX_Q4_K_M, MIX_Q5K_Q80, MIX_Q6_K, MIX_Q5_K, MIX_Q8_0 = range(6)
PROFILE_CLASSES = ("qkv", "wo", "gate_up", "down", "lm_head", "attn", "qkv_attn")
BENCH_QKV, BENCH_GATE_UP, BENCH_ALL_LAYERS = 100, 101, -2


class SpeculateError(Exception):
    """Base of the errors raised by the binding."""


class SamplingError(SpeculateError):
    """Error::Sampling (error.rs)."""


class CacheRollbackError(SpeculateError):
    """Error::CacheRollback (error.rs)."""


class BackendError(SpeculateError):
    """Error::Candle: device or runtime failure."""


class ArgError(SpeculateError, ValueError):
    """Invalid argument."""


class UnsupportedMethod(SpeculateError):
    """Error::UnsupportedMethod / unsupported shape or format."""


_ERRS = {SD_ERR_SAMPLING: SamplingError, SD_ERR_ROLLBACK: CacheRollbackError, SD_ERR_BACKEND: BackendError,
         SD_ERR_ARG: ArgError, SD_ERR_UNSUPPORTED: UnsupportedMethod}


class SdConfig(ctypes.Structure):
    _fields_ = [("arch", ctypes.c_int32), ("n_layers", ctypes.c_int32), ("hidden", ctypes.c_int32),
                ("n_heads", ctypes.c_int32), ("n_kv_heads", ctypes.c_int32), ("head_dim", ctypes.c_int32),
                ("ffn", ctypes.c_int32), ("vocab", ctypes.c_int32), ("rope_theta", ctypes.c_float),
                ("rms_eps", ctypes.c_float), ("ctx_len", ctypes.c_int32), ("max_batch", ctypes.c_int32),
                ("tied_output", ctypes.c_int32), ("device", ctypes.c_int32)]


@dataclass
class Config:
    arch: int = ARCH_LLAMA
    n_layers: int = 4
    hidden: int = 512
    n_heads: int = 8
    n_kv_heads: int = 8
    head_dim: int = 64
    ffn: int = 1536
    vocab: int = 32000
    rope_theta: float = 10000.0
    rms_eps: float = 1e-5
    ctx_len: int = 4096
    max_batch: int = 128
    tied_output: int = 0
    device: int = 0

    def to_c(self) -> SdConfig:
        return SdConfig(**{k: getattr(self, k) for k, _ in SdConfig._fields_})


class Draft3Config(ctypes.Structure):
    """sd_draft3_config: Eagle3DraftConfig (crates/speculate/src/methods/eagle3.rs:88-120)"""
    _fields_ = [("hidden", ctypes.c_int32), ("n_heads", ctypes.c_int32), ("n_kv_heads", ctypes.c_int32),
                ("ffn", ctypes.c_int32), ("draft_vocab", ctypes.c_int32), ("target_vocab", ctypes.c_int32),
                ("rms_eps", ctypes.c_float), ("rope_theta", ctypes.c_float), ("max_pos", ctypes.c_int32),
                ("device", ctypes.c_int32)]


class Draft2Config(ctypes.Structure):
    """sd_draft2_config: EagleDraftConfig (crates/speculate/src/methods/eagle.rs:56-65)"""
    _fields_ = [("hidden", ctypes.c_int32), ("n_heads", ctypes.c_int32), ("n_kv_heads", ctypes.c_int32),
                ("ffn", ctypes.c_int32), ("vocab", ctypes.c_int32), ("rms_eps", ctypes.c_float),
                ("rope_theta", ctypes.c_float), ("max_pos", ctypes.c_int32), ("device", ctypes.c_int32)]


# tensor kinds of sd_draft2_set_tensor (eagle.rs:126-131, 279-286, 349-361)
D2_EMBED, D2_FC, D2_Q, D2_K, D2_V, D2_O, D2_GATE, D2_UP, D2_DOWN, D2_POST_NORM = range(10)
# tensor kinds of sd_draft3_set_tensor (the checkpoint's names, eagle3.rs:133-152, 411-425)
D3_FC, D3_Q, D3_K, D3_V, D3_O, D3_GATE, D3_UP, D3_DOWN, D3_LM_HEAD = range(9)
D3_INPUT_NORM, D3_HIDDEN_NORM, D3_POST_NORM, D3_NORM, D3_D2T = range(9, 14)
DRAFT3_MAX_STEPS, DRAFT3_MAX_TOPK = 16, 8

_lib = None


def load_library(path: str = LIB_PATH):
    """Load the HIP library; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(f"HIP library not built: {path} (run __graft_entry__.build())")
    L = ctypes.CDLL(path)
    P, I32, U64, SZ = ctypes.c_void_p, ctypes.c_int32, ctypes.c_uint64, ctypes.c_size_t
    pSZ = ctypes.POINTER(ctypes.c_size_t)
    sigs = {
        "sd_model_create": ([ctypes.POINTER(SdConfig), ctypes.POINTER(P)], I32),
        "sd_model_destroy": ([P], None),
        "sd_model_set_tensor": ([P, I32, I32, I32, P, SZ], I32),
        "sd_model_get_tensor": ([P, I32, I32, P, SZ], I32),
        "sd_model_tensor_info": ([P, I32, I32, P, P, P, P], I32),
        "sd_model_synthesize": ([P, I32, U64, ctypes.c_float], I32),
        "sd_model_dequant_tensor": ([P, I32, I32, P], I32),
        "sd_model_qmatmul": ([P, I32, I32, P, SZ, P], I32),
        "sd_last_error": ([], ctypes.c_char_p),
        "sd_vocab_size": ([P], SZ),
        "sd_history_len": ([P], SZ),
        "sd_history": ([P, P, SZ], SZ),
        "sd_reset": ([P], None),
        "sd_observe": ([P, P, SZ], I32),
        "sd_next_logits": ([P, P], I32),
        "sd_batched_logits": ([P, P, SZ, P], I32),
        "sd_rollback_to": ([P, SZ], I32),
        "sd_set_eos_token_ids": ([P, P, SZ], I32),
        "sd_eos_token_ids": ([P, P, SZ], SZ),
        "sd_tree_logits_keep_kv": ([P, P, P, SZ, P, P], I32),
        "sd_tree_logits": ([P, P, P, SZ, P], I32),
        "sd_commit_tree_path": ([P, P, P, SZ, P, SZ], I32),
        "sd_last_hidden_state": ([P, P], I32),
        "sd_observe_returning_last_hidden": ([P, P, SZ, P], I32),
        "sd_last_hidden_states_multi": ([P, P, SZ, P, P], I32),
        "sd_apply_lm_head": ([P, P, SZ, P], I32),
        "sd_embed_tokens": ([P, P, SZ, P], I32),
        "sd_num_hidden_layers": ([P], SZ),
        "sd_hidden_size": ([P], SZ),
        "sd_verify_greedy_linear": ([P, P, SZ, P, pSZ, pSZ], I32),
        "sd_verify_greedy_tree": ([P, P, P, SZ, I32, P, pSZ, P, P, P, pSZ, pSZ, P], I32),
        "sd_last_argmax": ([P, P, SZ], I32),
        "sd_verify_rejection_linear": ([P, P, SZ, P, P, SZ, ctypes.c_float, SZ, P, pSZ, pSZ, pSZ], I32),
        "sd_verify_rejection_tree": ([P, P, P, SZ, P, SZ, SZ, P, P, SZ, ctypes.c_float, I32, I32, SZ, P, pSZ, P,
                                      pSZ], I32),
        "sd_verify_rejection_linear_device_q": ([P, P, SZ, P, P, SZ, ctypes.c_float, SZ, P, pSZ, pSZ, pSZ], I32),
        "sd_verify_rejection_tree_device_q": ([P, P, P, SZ, P, SZ, SZ, P, P, SZ, ctypes.c_float, I32, I32, SZ, P, pSZ,
                                               P, pSZ], I32),
        "sd_set_d2t": ([P, P, SZ], I32),
        "sd_draft_to_target": ([P, P, SZ, P], I32),
        "sd_t2d_mask": ([P, P, SZ], SZ),
        "sd_prime_synthetic": ([P, P, SZ, U64], I32),
        "sd_profile_enable": ([P, I32], I32),
        "sd_profile_read": ([P, P, P, P, SZ], SZ),
        "sd_synchronize": ([P], I32),
        "sd_bench_qmatmul": ([P, I32, I32, SZ, I32, P, P], I32),
        "sd_read_kv_rows": ([P, I32, I32, I32, SZ, SZ, P], I32),
        "sd_cache_len": ([P], SZ),
        "sd_tree_cartesian": ([ctypes.c_uint32, P, P, SZ, P, P, SZ, pSZ], I32),
        "sd_repack_gguf": ([I32, P, SZ, SZ, P], I32),
        "sd_unpack_tiles": ([I32, P, SZ, SZ, P], I32),
        "sd_lane_codes": ([I32, P, I32, I32, P], I32),
        "sd_tree_prune": ([P, P, SZ, P, P, SZ, SZ, P, P, pSZ], I32),
        "sd_gguf_open": ([ctypes.c_char_p, ctypes.POINTER(P)], I32),
        "sd_gguf_close": ([P], None),
        "sd_gguf_config": ([P, I32, ctypes.POINTER(SdConfig)], I32),
        "sd_gguf_layout": ([P, P, P, P], I32),
        "sd_gguf_tensor_count": ([P], SZ),
        "sd_gguf_tensor_info": ([P, ctypes.c_char_p, P, P, P, P], I32),
        "sd_model_load_gguf": ([P, P], I32),
        "sd_draft2_create": ([ctypes.POINTER(Draft2Config), ctypes.POINTER(P)], I32),
        "sd_draft2_destroy": ([P], None),
        "sd_draft2_tensor_bytes": ([P, I32], SZ),
        "sd_draft2_set_tensor": ([P, I32, P, SZ], I32),
        "sd_draft2_get_tensor": ([P, I32, P, SZ], I32),
        "sd_draft2_synthesize": ([P, U64, ctypes.c_float], I32),
        "sd_draft2_reset": ([P], I32),
        "sd_draft2_forward": ([P, P, SZ, ctypes.c_uint32, SZ, P], I32),
        "sd_draft2_round": ([P, P, P, SZ, P, P, P], I32),
        "sd_draft3_create": ([ctypes.POINTER(Draft3Config), ctypes.POINTER(P)], I32),
        "sd_draft3_destroy": ([P], None),
        "sd_draft3_tensor_bytes": ([P, I32], SZ),
        "sd_draft3_set_tensor": ([P, I32, P, SZ], I32),
        "sd_draft3_get_tensor": ([P, I32, P, SZ], I32),
        "sd_draft3_synthesize": ([P, U64, ctypes.c_float], I32),
        "sd_draft3_reset": ([P], I32),
        "sd_draft3_forward": ([P, P, SZ, P, SZ, P, P], I32),
        "sd_draft3_round": ([P, P, P, SZ, P, P, P, P], I32),
    }
    for name, (args, res) in sigs.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = res
    _lib = L
    return L


def _check(rc: int):
    if rc != SD_OK:
        msg = _lib.sd_last_error().decode(errors="replace")
        raise _ERRS.get(rc, BackendError)(msg)


def _u32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.int64).astype(np.uint32))


def _ptr(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def tree_arrays(tree) -> Tuple[np.ndarray, np.ndarray]:
    """(tokens, parents) of a DraftTree-like object or a (tokens, parents) pair."""
    if isinstance(tree, tuple):
        toks, pars = tree
    else:
        toks, pars = tree.tokens(), tree.parents()
    pars = list(pars)
    if len(pars):
        pars[0] = 0
    return _u32(toks), _u32(pars)


class GgufFile:
    """An opened .gguf file (gguf_file::Content::read, candle-core 0.8.4): the
    header, metadata and tensor directory.  Parsing is host code; no GPU needed."""

    def __init__(self, path: str):
        L = load_library()
        h = ctypes.c_void_p()
        _check(L.sd_gguf_open(os.fsencode(path), ctypes.byref(h)))
        self._h = h
        self.path = path

    def close(self):
        if getattr(self, "_h", None):
            _lib.sd_gguf_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def config(self, arch: int = -1, ctx_len: Optional[int] = None, max_batch: int = 128,
               device: int = 0) -> Config:
        """ModelWeights::from_gguf's hyper-parameters (quantized_llama_local.rs:222-240,
        quantized_qwen2_local.rs:215-230); arch -1 reads general.architecture.
        ctx_len defaults to the file's context_length."""
        c = SdConfig()
        _check(_lib.sd_gguf_config(self._h, arch, ctypes.byref(c)))
        cfg = Config(**{k: getattr(c, k) for k, _ in SdConfig._fields_})
        if ctx_len is not None:
            cfg.ctx_len = ctx_len
        cfg.max_batch = max_batch
        cfg.device = device
        return cfg

    def layout(self) -> Tuple[int, int, int]:
        """(GGUF version, alignment, absolute offset of the data section)."""
        v, a, d = ctypes.c_uint32(), ctypes.c_uint64(), ctypes.c_uint64()
        _check(_lib.sd_gguf_layout(self._h, ctypes.byref(v), ctypes.byref(a), ctypes.byref(d)))
        return v.value, a.value, d.value

    def tensor_count(self) -> int:
        return int(_lib.sd_gguf_tensor_count(self._h))

    def tensor_info(self, name: str) -> Tuple[int, Tuple[int, ...], int]:
        """(GGML type, dims with ne[0] first, offset from the data section)."""
        t, nd = ctypes.c_int32(), ctypes.c_int32()
        ne = np.zeros(4, np.uint64)
        off = ctypes.c_uint64()
        _check(_lib.sd_gguf_tensor_info(self._h, name.encode(), ctypes.byref(t), ctypes.byref(nd), _ptr(ne),
                                        ctypes.byref(off)))
        return t.value, tuple(int(v) for v in ne[:nd.value]), off.value


@dataclass
class TreeCommit:
    """Greedy tree verify + commit composition (eagle.rs:605-732): commit
    path[:keep_len] (+ bonus_node when >= 0) with commit_tree_path; committed
    tokens are EOS-truncated and stop is set when an EOS was committed."""
    path: List[int]
    bonus: int
    bonus_node: int
    committed: List[int]
    keep_len: int
    stop: bool

    def keep(self) -> List[int]:
        return self.path[:self.keep_len] + ([self.bonus_node] if self.bonus_node >= 0 else [])


_hiprt = None


def _hip_runtime():
    """The HIP runtime the library is linked against (already loaded with it)."""
    global _hiprt
    if _hiprt is None:
        load_library()
        path = "libamdhip64.so"
        with open("/proc/self/maps") as f:
            for line in f:
                if "libamdhip64.so" in line:
                    path = line.split()[-1]
                    break
        rt = ctypes.CDLL(path)
        rt.hipSetDevice.argtypes = [ctypes.c_int]
        rt.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
        rt.hipFree.argtypes = [ctypes.c_void_p]
        rt.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        for fn in (rt.hipSetDevice, rt.hipMalloc, rt.hipFree, rt.hipMemcpy):
            fn.restype = ctypes.c_int
        _hiprt = rt
    return _hiprt


class DeviceArray:
    """A host array copied into one GPU's memory with the library's HIP
    runtime: the input of the *_device entry points (draft rows a GPU draft
    model would leave on the device).  `ptr` is the device address; close()
    frees it."""

    def __init__(self, host: np.ndarray, device: int = 0):
        self.host_shape, self.dtype = host.shape, host.dtype
        a = np.ascontiguousarray(host)
        rt = _hip_runtime()
        self._p = ctypes.c_void_p()
        if rt.hipSetDevice(device) != 0 or rt.hipMalloc(ctypes.byref(self._p), max(a.nbytes, 1)) != 0:
            raise BackendError("hipMalloc failed")
        if rt.hipMemcpy(self._p, a.ctypes.data_as(ctypes.c_void_p), a.nbytes, 1) != 0:
            rt.hipFree(self._p)
            raise BackendError("hipMemcpy failed")

    @property
    def ptr(self) -> int:
        return int(self._p.value or 0)

    def close(self):
        if self._p.value:
            _hip_runtime().hipFree(self._p)
            self._p = ctypes.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


class HipQuantDecoder:
    """One quantised target decoder resident on one GPU (LlamaQuantDecoder contract)."""

    @classmethod
    def from_gguf(cls, gguf_path: str, arch: int = -1, ctx_len: Optional[int] = None, max_batch: int = 128,
                  device: int = 0, eos_token_ids: Sequence[int] = ()) -> "HipQuantDecoder":
        """LlamaQuantDecoder::from_gguf / Qwen2QuantDecoder::from_gguf
        (quantized_llama.rs:57-98, quantized_qwen2.rs:55-100) without the
        tokenizer: the config from the file's metadata, then every tensor.
        arch picks the decoder type (ARCH_LLAMA reads llama.* keys); -1 follows
        general.architecture."""
        with GgufFile(gguf_path) as g:
            dec = cls(g.config(arch, ctx_len=ctx_len, max_batch=max_batch, device=device))
            try:
                _check(_lib.sd_model_load_gguf(dec._h, g._h))
            except Exception:
                dec.close()
                raise
        if eos_token_ids:
            dec.set_eos_token_ids(eos_token_ids)
        return dec

    def __init__(self, cfg: Config):
        L = load_library()
        self.cfg = cfg
        c = cfg.to_c()
        h = ctypes.c_void_p()
        _check(L.sd_model_create(ctypes.byref(c), ctypes.byref(h)))
        self._h = h
        self.vocab = cfg.vocab
        self.hidden = cfg.hidden

    def close(self):
        if getattr(self, "_h", None):
            _lib.sd_model_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ---- weights ----
    def set_tensor(self, layer: int, kind: int, fmt: int, data: np.ndarray):
        d = np.ascontiguousarray(data).view(np.uint8)
        _check(_lib.sd_model_set_tensor(self._h, layer, kind, fmt, _ptr(d), d.nbytes))

    def tensor_info(self, layer: int, kind: int):
        f, r, k = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32()
        b = ctypes.c_size_t()
        _check(_lib.sd_model_tensor_info(self._h, layer, kind, ctypes.byref(f), ctypes.byref(r), ctypes.byref(k),
                                         ctypes.byref(b)))
        return f.value, r.value, k.value, b.value

    def get_tensor(self, layer: int, kind: int) -> np.ndarray:
        _, _, _, nbytes = self.tensor_info(layer, kind)
        out = np.empty(nbytes, np.uint8)
        _check(_lib.sd_model_get_tensor(self._h, layer, kind, _ptr(out), nbytes))
        return out

    def synthesize(self, mix: int, seed: int, std: float = 0.02):
        _check(_lib.sd_model_synthesize(self._h, mix, seed, std))

    def dequant_tensor(self, layer: int, kind: int) -> np.ndarray:
        _, r, k, _ = self.tensor_info(layer, kind)
        out = np.empty((r, k), np.float32)
        _check(_lib.sd_model_dequant_tensor(self._h, layer, kind, _ptr(out)))
        return out

    def qmatmul(self, layer: int, kind: int, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        _, r, k, _ = self.tensor_info(layer, kind)
        assert x.shape[1] == k
        y = np.empty((x.shape[0], r), np.float32)
        _check(_lib.sd_model_qmatmul(self._h, layer, kind, _ptr(x), x.shape[0], _ptr(y)))
        return y

    # ---- Decoder ----
    def vocab_size(self) -> int:
        return int(_lib.sd_vocab_size(self._h))

    def history(self) -> List[int]:
        n = int(_lib.sd_history_len(self._h))
        out = np.empty(n, np.uint32)
        _lib.sd_history(self._h, _ptr(out), n)
        return [int(v) for v in out]

    def history_len(self) -> int:
        return int(_lib.sd_history_len(self._h))

    def reset(self):
        _lib.sd_reset(self._h)

    def observe(self, ids: Sequence[int]):
        a = _u32(ids)
        _check(_lib.sd_observe(self._h, _ptr(a), a.size))

    def next_logits(self) -> np.ndarray:
        out = np.empty(self.vocab, np.float32)
        _check(_lib.sd_next_logits(self._h, _ptr(out)))
        return out

    def batched_logits(self, drafts: Sequence[int]) -> np.ndarray:
        a = _u32(drafts)
        out = np.empty((a.size + 1, self.vocab), np.float32)
        _check(_lib.sd_batched_logits(self._h, _ptr(a), a.size, _ptr(out)))
        return out

    def rollback_to(self, n: int):
        if n < 0:
            raise ArgError("negative length")
        _check(_lib.sd_rollback_to(self._h, n))

    def set_eos_token_ids(self, ids: Sequence[int]):
        a = _u32(ids)
        _check(_lib.sd_set_eos_token_ids(self._h, _ptr(a), a.size))

    def eos_token_ids(self) -> List[int]:
        n = int(_lib.sd_eos_token_ids(self._h, None, 0))
        out = np.empty(n, np.uint32)
        _lib.sd_eos_token_ids(self._h, _ptr(out), n)
        return [int(v) for v in out]

    # ---- TreeDecoder ----
    def tree_logits_keep_kv(self, tree, want_logits: bool = True, want_hidden: bool = True):
        t, p = tree_arrays(tree)
        lg = np.empty((t.size, self.vocab), np.float32) if want_logits else None
        hd = np.empty((t.size, self.hidden), np.float32) if want_hidden else None
        _check(_lib.sd_tree_logits_keep_kv(self._h, _ptr(t), _ptr(p), t.size, _ptr(lg), _ptr(hd)))
        return lg, hd

    def tree_logits(self, tree) -> np.ndarray:
        t, p = tree_arrays(tree)
        lg = np.empty((t.size, self.vocab), np.float32)
        _check(_lib.sd_tree_logits(self._h, _ptr(t), _ptr(p), t.size, _ptr(lg)))
        return lg

    def commit_tree_path(self, tree, accepted: Sequence[int]):
        t, p = tree_arrays(tree)
        a = _u32(accepted)
        _check(_lib.sd_commit_tree_path(self._h, _ptr(t), _ptr(p), t.size, _ptr(a), a.size))

    def last_hidden_state(self) -> np.ndarray:
        out = np.empty(self.hidden, np.float32)
        _check(_lib.sd_last_hidden_state(self._h, _ptr(out)))
        return out

    def observe_returning_last_hidden(self, ids: Sequence[int]) -> np.ndarray:
        a = _u32(ids)
        out = np.empty(self.hidden, np.float32)
        _check(_lib.sd_observe_returning_last_hidden(self._h, _ptr(a), a.size, _ptr(out)))
        return out

    def last_hidden_states_multi(self, layers: Sequence[int]):
        a = _u32(layers)
        fin = np.empty(self.hidden, np.float32)
        mids = np.empty((a.size, self.hidden), np.float32)
        _check(_lib.sd_last_hidden_states_multi(self._h, _ptr(a), a.size, _ptr(fin), _ptr(mids)))
        return fin, [mids[i] for i in range(a.size)]

    def apply_lm_head(self, hidden) -> np.ndarray:
        """TreeDecoder::apply_lm_head (quantized_llama_local.rs:316-318): the
        lm_head QMatMul over the last dim, [..., hidden] -> [..., vocab] f32,
        leading dims kept. F16 / F64 input is promoted to f32 first, as the
        quantised path does with a draft's F16 rows (eagle.rs:536-547)."""
        h = np.asarray(hidden)
        if h.ndim == 0 or h.shape[-1] != self.hidden:
            raise BackendError(f"apply_lm_head: last dim of shape {h.shape} must be hidden ({self.hidden})")
        lead = h.shape[:-1]
        flat = np.ascontiguousarray(h.reshape(-1, self.hidden), np.float32)
        out = np.empty((flat.shape[0], self.vocab), np.float32)
        if flat.shape[0]:
            _check(_lib.sd_apply_lm_head(self._h, _ptr(flat), flat.shape[0], _ptr(out)))
        return out.reshape(lead + (self.vocab,))

    def embed_tokens(self, ids) -> np.ndarray:
        """TreeDecoder::embed_tokens (quantized_llama_local.rs:328-330): the
        token table's rows, ids.shape ++ [hidden] f32 (a (1, 1) id tensor gives
        the [1, 1, hidden] input of the EAGLE-3 midlayer, eagle3.rs:641-650)."""
        a = np.asarray(ids)
        shape = a.shape
        flat = _u32(a.reshape(-1))
        out = np.empty((flat.size, self.hidden), np.float32)
        if flat.size:
            _check(_lib.sd_embed_tokens(self._h, _ptr(flat), flat.size, _ptr(out)))
        return out.reshape(shape + (self.hidden,))

    def num_hidden_layers(self) -> int:
        return int(_lib.sd_num_hidden_layers(self._h))

    # ---- device acceptance ----
    def verify_greedy_linear(self, drafts: Sequence[int]) -> Tuple[List[int], int]:
        a = _u32(drafts)
        commits = np.empty(a.size + 1, np.uint32)
        nc, na = ctypes.c_size_t(), ctypes.c_size_t()
        _check(_lib.sd_verify_greedy_linear(self._h, _ptr(a), a.size, _ptr(commits), ctypes.byref(nc),
                                            ctypes.byref(na)))
        return [int(v) for v in commits[:nc.value]], int(na.value)

    def verify_greedy_tree(self, tree, strict: bool = False, compose: bool = False):
        """-> (path, bonus, bonus_node); with compose=True a TreeCommit that
        also holds the EOS-aware commit composition (eagle.rs:664-732)."""
        t, p = tree_arrays(tree)
        path = np.empty(t.size, np.uint32)
        committed = np.empty(t.size, np.uint32)
        plen, ncom, keep = ctypes.c_size_t(), ctypes.c_size_t(), ctypes.c_size_t()
        bonus = ctypes.c_uint32()
        bnode, stop = ctypes.c_int32(), ctypes.c_int32()
        _check(_lib.sd_verify_greedy_tree(self._h, _ptr(t), _ptr(p), t.size, 1 if strict else 0, _ptr(path),
                                          ctypes.byref(plen), ctypes.byref(bonus), ctypes.byref(bnode),
                                          _ptr(committed), ctypes.byref(ncom), ctypes.byref(keep),
                                          ctypes.byref(stop)))
        pth = [int(v) for v in path[:plen.value]]
        if not compose:
            return pth, int(bonus.value), int(bnode.value)
        return TreeCommit(path=pth, bonus=int(bonus.value), bonus_node=int(bnode.value),
                          committed=[int(v) for v in committed[:ncom.value]], keep_len=int(keep.value),
                          stop=bool(stop.value))

    def verify_rejection_linear(self, drafts: Sequence[int], q_rows: np.ndarray, uniforms: Sequence[float],
                                temperature: float, max_commit: int = 0):
        """-> (commits, n_accepted, uniforms_used)."""
        d = _u32(drafts)
        q = np.ascontiguousarray(q_rows, np.float32)
        if d.size and q.shape != (d.size, self.cfg.vocab):
            raise ValueError("q_rows must be [k][vocab]")
        return self._rejection_linear(_lib.sd_verify_rejection_linear, d, _ptr(q), uniforms, temperature, max_commit)

    def verify_rejection_linear_device(self, drafts: Sequence[int], q_rows_dev: int, uniforms: Sequence[float],
                                       temperature: float, max_commit: int = 0):
        """verify_rejection_linear with the [k][vocab] f32 draft rows already in
        this GPU's memory at address q_rows_dev (written and synchronised by
        the caller)."""
        return self._rejection_linear(_lib.sd_verify_rejection_linear_device_q, _u32(drafts),
                                      ctypes.c_void_p(int(q_rows_dev)), uniforms, temperature, max_commit)

    def _rejection_linear(self, fn, d, q_ptr, uniforms, temperature, max_commit):
        u = np.ascontiguousarray(uniforms, np.float32)
        commits = np.empty(d.size + 1, np.uint32)
        nc, na, nu = ctypes.c_size_t(), ctypes.c_size_t(), ctypes.c_size_t()
        _check(fn(self._h, _ptr(d), d.size, q_ptr, _ptr(u), u.size, float(temperature), max_commit, _ptr(commits),
                  ctypes.byref(nc), ctypes.byref(na), ctypes.byref(nu)))
        return [int(v) for v in commits[:nc.value]], int(na.value), int(nu.value)

    def verify_rejection_tree(self, tree, q_rows: np.ndarray, q_row_of: Sequence[int], uniforms: Sequence[float],
                              temperature: float, use_t2d: bool = False, max_commit: int = 0,
                              without_replacement: bool = False):
        """-> (path node indices, final token or -1, uniforms_used).  The
        sibling rule: i.i.d. siblings (q fixed) or, with without_replacement,
        siblings drawn without replacement (rejected tokens zeroed in q)."""
        q = np.ascontiguousarray(q_rows, np.float32)
        if q.ndim != 2:
            raise ValueError("q_rows must be 2-D")
        return self._rejection_tree(_lib.sd_verify_rejection_tree, tree, _ptr(q), q.shape[0], q.shape[1], q_row_of,
                                    uniforms, temperature, use_t2d, max_commit, without_replacement)

    def verify_rejection_tree_device(self, tree, q_rows_dev: int, q_rows_n: int, q_vocab: int,
                                     q_row_of: Sequence[int], uniforms: Sequence[float], temperature: float,
                                     use_t2d: bool = False, max_commit: int = 0, without_replacement: bool = False):
        """verify_rejection_tree with the [q_rows_n][q_vocab] f32 draft rows
        already in this GPU's memory at address q_rows_dev."""
        return self._rejection_tree(_lib.sd_verify_rejection_tree_device_q, tree, ctypes.c_void_p(int(q_rows_dev)),
                                    q_rows_n, q_vocab, q_row_of, uniforms, temperature, use_t2d, max_commit,
                                    without_replacement)

    def _rejection_tree(self, fn, tree, q_ptr, q_n, q_vocab, q_row_of, uniforms, temperature, use_t2d, max_commit,
                        without_replacement):
        t, p = tree_arrays(tree)
        qr = np.ascontiguousarray(q_row_of, np.int32)
        if qr.size != t.size:
            raise ValueError("q_row_of needs one entry per node")
        u = np.ascontiguousarray(uniforms, np.float32)
        path = np.empty(t.size, np.uint32)
        plen, nu = ctypes.c_size_t(), ctypes.c_size_t()
        tok = ctypes.c_int32()
        _check(fn(self._h, _ptr(t), _ptr(p), t.size, q_ptr, q_n, q_vocab, _ptr(qr), _ptr(u), u.size,
                  float(temperature), 1 if use_t2d else 0, 1 if without_replacement else 0, max_commit, _ptr(path),
                  ctypes.byref(plen), ctypes.byref(tok), ctypes.byref(nu)))
        return [int(v) for v in path[:plen.value]], int(tok.value), int(nu.value)

    def set_d2t(self, d2t: Sequence[int]):
        a = np.ascontiguousarray(d2t, np.int64)
        _check(_lib.sd_set_d2t(self._h, _ptr(a), a.size))

    def draft_to_target(self, ids: Sequence[int]):
        a = _u32(ids)
        out = np.empty(a.size, np.uint32)
        _check(_lib.sd_draft_to_target(self._h, _ptr(a), a.size, _ptr(out)))
        return [int(v) for v in out]

    def t2d_mask(self) -> np.ndarray:
        n = _lib.sd_t2d_mask(self._h, None, 0)
        out = np.zeros(n, np.uint8)
        if n:
            _lib.sd_t2d_mask(self._h, _ptr(out), n)
        return out.astype(bool)

    def last_argmax(self, n: int) -> np.ndarray:
        out = np.empty(n, np.int32)
        _check(_lib.sd_last_argmax(self._h, _ptr(out), n))
        return out

    # ---- synthetic state / measurement ----
    def prime_synthetic(self, ids: Sequence[int], kv_seed: int):
        a = _u32(ids)
        _check(_lib.sd_prime_synthetic(self._h, _ptr(a), a.size, kv_seed))

    def profile_enable(self, on: bool):
        _check(_lib.sd_profile_enable(self._h, 1 if on else 0))

    def profile_read(self, cap: int = 65536):
        cls = np.empty(cap, np.int32)
        by = np.empty(cap, np.float64)
        ms = np.empty(cap, np.float32)
        n = int(_lib.sd_profile_read(self._h, _ptr(cls), _ptr(by), _ptr(ms), cap))
        return [(PROFILE_CLASSES[cls[i]], float(by[i]), float(ms[i])) for i in range(n)]

    def bench_qmatmul(self, layer: int, kind: int, rows: int, iters: int = 50) -> Tuple[float, float]:
        """(microseconds per launch, algorithmic bytes per launch) of one dequant-matmul."""
        us, by = ctypes.c_double(), ctypes.c_double()
        _check(_lib.sd_bench_qmatmul(self._h, layer, kind, rows, iters, ctypes.byref(us), ctypes.byref(by)))
        return us.value, by.value

    def synchronize(self):
        _check(_lib.sd_synchronize(self._h))

    def read_kv_rows(self, layer: int, which: int, head: int, pos0: int, n: int) -> np.ndarray:
        out = np.empty((n, self.cfg.head_dim), np.uint16)
        _check(_lib.sd_read_kv_rows(self._h, layer, which, head, pos0, n, _ptr(out)))
        return out

    def cache_len(self) -> int:
        return int(_lib.sd_cache_len(self._h))


# ---- draft-tree builders (host only) ----
def default_layers_for(n_layers: int) -> List[int]:
    """Eagle3RunConfig::default_layers_for (eagle3.rs:540-546): [1, n/2 - 1, n - 4]"""
    return [0, 0, 0] if n_layers < 4 else [1, n_layers // 2 - 1, n_layers - 4]


class HipEagleDraft:
    """EagleDraftCandle (crates/speculate/src/methods/eagle.rs:306-428), the
    EAGLE-2 draft, resident on one GPU: f16 tensors including its own token
    table, the draft's KV cache (at most 16 steps between resets), and a whole
    draft round of run_eagle (:519-575) on the device, with the target's
    lm_head for the draft logits."""

    def __init__(self, hidden: int = 4096, n_heads: int = 32, n_kv_heads: int = 8, ffn: int = 14336,
                 vocab: int = 128256, rms_eps: float = 1e-5, rope_theta: float = 500000.0, max_pos: int = 2048,
                 device: int = 0):
        load_library()
        self.hidden, self.vocab = hidden, vocab
        c = Draft2Config(hidden, n_heads, n_kv_heads, ffn, vocab, rms_eps, rope_theta, max_pos, device)
        self._h = ctypes.c_void_p()
        _check(_lib.sd_draft2_create(ctypes.byref(c), ctypes.byref(self._h)))

    def close(self):
        if getattr(self, "_h", None) and self._h.value:
            _lib.sd_draft2_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def tensor_bytes(self, kind: int) -> int:
        return int(_lib.sd_draft2_tensor_bytes(self._h, kind))

    def set_tensor(self, kind: int, data: np.ndarray):
        a = np.ascontiguousarray(data, np.float16)
        _check(_lib.sd_draft2_set_tensor(self._h, kind, _ptr(a), a.nbytes))

    def get_tensor(self, kind: int) -> np.ndarray:
        a = np.empty(self.tensor_bytes(kind) // 2, np.float16)
        _check(_lib.sd_draft2_get_tensor(self._h, kind, _ptr(a), a.nbytes))
        return a

    def synthesize(self, seed: int, std: float = 0.02):
        _check(_lib.sd_draft2_synthesize(self._h, seed, std))

    def reset(self):
        _check(_lib.sd_draft2_reset(self._h))

    def forward(self, target_hidden: np.ndarray, token: int, position: int) -> np.ndarray:
        """EagleDraftCandle::forward (:390-427) of one position -> [hidden] (f16 values as f32)"""
        h = np.ascontiguousarray(target_hidden, np.float32).reshape(-1)
        out = np.empty(self.hidden, np.float32)
        _check(_lib.sd_draft2_forward(self._h, _ptr(h), h.size, int(token), position, _ptr(out)))
        return out

    def round(self, target: "HipQuantDecoder", target_hidden: np.ndarray, depth: int, top_k) \
            -> Tuple[List[List[int]], List[List[float]]]:
        """The draft half of one run_eagle iteration (:519-575) against target:
        -> (per-step top-k ids, their log-probs)"""
        ks = [int(top_k)] * depth if np.isscalar(top_k) else [int(k) for k in top_k]
        if len(ks) != depth:
            raise ArgError("one top_k per draft step")
        h = np.ascontiguousarray(target_hidden, np.float32).reshape(-1)
        if h.size != self.hidden:
            raise ArgError("target_hidden must be hidden wide")
        k = np.asarray(ks, np.int32)
        ids = np.zeros((max(depth, 1), DRAFT3_MAX_TOPK), np.int32)
        lps = np.zeros(ids.shape, np.float32)
        _check(_lib.sd_draft2_round(self._h, target._h, _ptr(h), depth, _ptr(k), _ptr(ids), _ptr(lps)))
        return ([[int(v) for v in ids[s, :ks[s]]] for s in range(depth)],
                [[float(v) for v in lps[s, :ks[s]]] for s in range(depth)])


class HipEagle3Draft:
    """Eagle3DraftCandle (crates/speculate/src/methods/eagle3.rs:307-516) resident
    on one GPU: f16 tensors, the draft's own KV cache (at most 16 steps between
    resets), and a whole draft round of run_eagle3 (:598-673) on the device."""

    def __init__(self, hidden: int = 4096, n_heads: int = 32, n_kv_heads: int = 8, ffn: int = 14336,
                 draft_vocab: int = 32000, target_vocab: int = 128256, rms_eps: float = 1e-5,
                 rope_theta: float = 500000.0, max_pos: int = 2048, device: int = 0):
        load_library()
        self.hidden, self.draft_vocab, self.target_vocab = hidden, draft_vocab, target_vocab
        c = Draft3Config(hidden, n_heads, n_kv_heads, ffn, draft_vocab, target_vocab, rms_eps, rope_theta, max_pos,
                         device)
        self._h = ctypes.c_void_p()
        _check(_lib.sd_draft3_create(ctypes.byref(c), ctypes.byref(self._h)))

    def close(self):
        if getattr(self, "_h", None) and self._h.value:
            _lib.sd_draft3_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def tensor_bytes(self, kind: int) -> int:
        return int(_lib.sd_draft3_tensor_bytes(self._h, kind))

    def set_tensor(self, kind: int, data: np.ndarray):
        """weights [out][in] and norms [hidden] as f16; D3_D2T as int64 [draft_vocab]"""
        a = np.ascontiguousarray(data, np.int64 if kind == D3_D2T else np.float16)
        _check(_lib.sd_draft3_set_tensor(self._h, kind, _ptr(a), a.nbytes))

    def get_tensor(self, kind: int) -> np.ndarray:
        n = self.tensor_bytes(kind)
        a = np.empty(n // (8 if kind == D3_D2T else 2), np.int64 if kind == D3_D2T else np.float16)
        _check(_lib.sd_draft3_get_tensor(self._h, kind, _ptr(a), a.nbytes))
        return a

    def synthesize(self, seed: int, std: float = 0.02):
        _check(_lib.sd_draft3_synthesize(self._h, seed, std))

    def reset(self):
        _check(_lib.sd_draft3_reset(self._h))

    def forward_hidden(self, hidden_states: np.ndarray, input_emb: np.ndarray, position: int,
                       want_logits: bool = True):
        """forward_hidden (:433-450) + apply_norm_lm_head (:451-454): hidden_states
        of 3 * hidden (fc applied) or hidden; -> (pre-norm midlayer output
        [hidden], draft logits [draft_vocab] or None), both f16 values as f32"""
        h = np.ascontiguousarray(hidden_states, np.float32).reshape(-1)
        e = np.ascontiguousarray(input_emb, np.float32).reshape(-1)
        if e.size != self.hidden:
            raise ArgError("input_emb must be hidden wide")
        out = np.empty(self.hidden, np.float32)
        lg = np.empty(self.draft_vocab, np.float32) if want_logits else None
        _check(_lib.sd_draft3_forward(self._h, _ptr(h), h.size, _ptr(e), position, _ptr(out), _ptr(lg)))
        return out, lg

    def round(self, target: "HipQuantDecoder", layers: Sequence[int], depth: int, top_k) \
            -> Tuple[List[List[int]], List[List[float]], List[List[int]]]:
        """The draft half of one run_eagle3 iteration (:598-673) against target:
        -> (per-step top-k target ids, their log-probs, their draft ids)"""
        ks = [int(top_k)] * depth if np.isscalar(top_k) else [int(k) for k in top_k]
        if len(ks) != depth:
            raise ArgError("one top_k per draft step")
        lay = _u32(layers)
        if lay.size != 3:
            raise SamplingError(f"EAGLE-3 expects 3 layers, got {lay.size}")
        k = np.asarray(ks, np.int32)
        ids = np.zeros((max(depth, 1), DRAFT3_MAX_TOPK), np.int32)
        dids = np.zeros_like(ids)
        lps = np.zeros(ids.shape, np.float32)
        _check(_lib.sd_draft3_round(self._h, target._h, _ptr(lay), depth, _ptr(k), _ptr(ids), _ptr(dids),
                                    _ptr(lps)))
        return ([[int(v) for v in ids[s, :ks[s]]] for s in range(depth)],
                [[float(v) for v in lps[s, :ks[s]]] for s in range(depth)],
                [[int(v) for v in dids[s, :ks[s]]] for s in range(depth)])


def tree_cartesian(root: int, head_top_k: Sequence[Sequence[int]]) -> Tuple[np.ndarray, np.ndarray]:
    """build_cartesian_tree (methods/medusa.rs:172-193) -> (tokens, parents)."""
    L = load_library()
    br = _u32([len(c) for c in head_top_k])
    cand = _u32([t for c in head_top_k for t in c]) if len(br) else _u32([0])
    n = ctypes.c_size_t()
    _check(L.sd_tree_cartesian(root, _ptr(cand), _ptr(br), br.size, None, None, 0, ctypes.byref(n)))
    toks, pars = np.empty(n.value, np.uint32), np.empty(n.value, np.uint32)
    _check(L.sd_tree_cartesian(root, _ptr(cand), _ptr(br), br.size, _ptr(toks), _ptr(pars), n.value,
                               ctypes.byref(n)))
    return toks, pars


def tree_prune(tree, per_step_log_probs: Sequence[Sequence[float]], max_total: int) -> Tuple[np.ndarray, np.ndarray]:
    """prune_cartesian_tree (methods/eagle.rs:763-845) -> (tokens, parents)."""
    L = load_library()
    t, p = tree_arrays(tree)
    br = _u32([len(r) for r in per_step_log_probs])
    lp = np.ascontiguousarray([v for r in per_step_log_probs for v in r] or [0.0], np.float32)
    ot, op = np.empty(t.size, np.uint32), np.empty(t.size, np.uint32)
    n = ctypes.c_size_t()
    _check(L.sd_tree_prune(_ptr(t), _ptr(p), t.size, _ptr(lp), _ptr(br), br.size, max_total, _ptr(ot), _ptr(op),
                           ctypes.byref(n)))
    return ot[:n.value].copy(), op[:n.value].copy()


# ---- device weight layout (host only) ----
def repack_gguf(fmt: int, gguf: np.ndarray, rows: int, K: int) -> np.ndarray:
    """GGUF row-major blocks -> the library's tile-interleaved device order (same size)."""
    L = load_library()
    src = np.ascontiguousarray(gguf).view(np.uint8)
    out = np.empty_like(src)
    _check(L.sd_repack_gguf(fmt, _ptr(src), rows, K, _ptr(out)))
    return out


def unpack_tiles(fmt: int, tiles: np.ndarray, rows: int, K: int) -> np.ndarray:
    L = load_library()
    src = np.ascontiguousarray(tiles).view(np.uint8)
    out = np.empty_like(src)
    _check(L.sd_unpack_tiles(fmt, _ptr(src), rows, K, _ptr(out)))
    return out


def lane_codes(fmt: int, tile_block: np.ndarray, lane: int, chunk: int) -> np.ndarray:
    """The 4 code words lane `lane` builds for K-chunk `chunk` of one tile block."""
    L = load_library()
    tb = np.ascontiguousarray(tile_block).view(np.uint8)
    out = np.empty(4, np.uint32)
    _check(L.sd_lane_codes(fmt, _ptr(tb), lane, chunk, _ptr(out)))
    return out
