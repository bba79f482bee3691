"""GGUF writer for the tests: builds .gguf bytes from metadata and tensors
following the published GGUF v1-v3 layout (the same layout the oracle's
reader and the library read; pinned separately by the hand-assembled
known-answer file in test_gguf_host.py)."""
from __future__ import annotations

import struct
from typing import Dict, List, Sequence, Tuple

import numpy as np

import oracle as O
from _models import all_tensor_keys

U8, I8, U16, I16, U32, I32, F32V, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32V: "<f", BOOL: "<B", U64: "<Q",
        I64: "<q", F64: "<d"}
GGML_F32, GGML_F16 = 0, 1

KIND_NAMES = {O.K_TOK_EMBD: "token_embd.weight", O.K_OUTPUT: "output.weight", O.K_OUTPUT_NORM: "output_norm.weight",
              O.K_ATTN_Q: "attn_q.weight", O.K_ATTN_K: "attn_k.weight", O.K_ATTN_V: "attn_v.weight",
              O.K_ATTN_O: "attn_output.weight", O.K_FFN_GATE: "ffn_gate.weight", O.K_FFN_UP: "ffn_up.weight",
              O.K_FFN_DOWN: "ffn_down.weight", O.K_ATTN_NORM: "attn_norm.weight", O.K_FFN_NORM: "ffn_norm.weight",
              O.K_BQ: "attn_q.bias", O.K_BK: "attn_k.bias", O.K_BV: "attn_v.bias"}


def _len(n: int, version: int) -> bytes:
    return struct.pack("<I" if version == 1 else "<Q", n)


def _str(s: str, version: int) -> bytes:
    b = s.encode()
    return _len(len(b), version) + b


def _val(t: int, v, version: int) -> bytes:
    if t == STRING:
        return _str(v, version)
    if t == ARRAY:
        et, items = v
        return struct.pack("<I", et) + _len(len(items), version) + b"".join(_val(et, x, version) for x in items)
    return struct.pack(_FMT[t], v)


def gguf_bytes(metadata: Sequence[Tuple[str, int, object]], tensors: Sequence[Tuple[str, int, Tuple[int, ...], bytes]],
               version: int = 3, alignment: int = 32) -> bytes:
    """metadata: (key, value type, value); tensors: (name, GGML type, dims
    with ne[0] first, raw bytes).  Tensor data start at multiples of
    `alignment` (write general.alignment yourself when it is not 32)."""
    out = [b"GGUF", struct.pack("<I", version), _len(len(tensors), version), _len(len(metadata), version)]
    for k, t, v in metadata:
        out += [_str(k, version), struct.pack("<I", t), _val(t, v, version)]
    off = 0
    offsets = []
    for name, gt, dims, raw in tensors:
        offsets.append(off)
        out += [_str(name, version), struct.pack("<I", len(dims))]
        out += [struct.pack("<I" if version == 1 else "<Q", d) for d in dims]
        out += [struct.pack("<I", gt), struct.pack("<Q", off)]
        off += (len(raw) + alignment - 1) // alignment * alignment
    head = b"".join(out)
    head += b"\0" * ((-len(head)) % alignment)
    data = bytearray()
    for (_, _, _, raw), o in zip(tensors, offsets):
        data += b"\0" * (o - len(data))
        data += raw
    return head + bytes(data)


def model_metadata(cfg: O.ModelConfig, rope_base: bool = True, vocab_tokens: bool = False) -> List:
    p = cfg.arch + "."
    md = [("general.architecture", STRING, cfg.arch),
          (p + "attention.head_count", U32, cfg.n_heads),
          (p + "attention.head_count_kv", U32, cfg.n_kv_heads),
          (p + "embedding_length", U32, cfg.hidden),
          (p + "context_length", U32, cfg.ctx_len),
          (p + "block_count", U32, cfg.n_layers),
          (p + "feed_forward_length", U32, cfg.ffn),
          (p + "attention.layer_norm_rms_epsilon", F32V, cfg.rms_eps)]
    if cfg.arch == "llama":
        md.append(("llama.rope.dimension_count", U32, cfg.head_dim))
    if rope_base:
        md.append((p + "rope.freq_base", F32V, cfg.rope_theta))
    if vocab_tokens:
        md.append(("tokenizer.ggml.tokens", ARRAY, (STRING, [f"t{i}" for i in range(cfg.vocab)])))
    return md


def model_tensors(cfg: O.ModelConfig, tensors: Dict[Tuple[int, int], Tuple[int, np.ndarray]],
                  f16_vectors: bool = False) -> List:
    """GGUF tensor entries for a model's tensors (F32 vectors optionally stored as F16)."""
    out = []
    for (li, k) in all_tensor_keys(cfg):
        fmt, raw = tensors[(li, k)]
        rows, K = cfg.shape(k)
        name = KIND_NAMES[k] if li < 0 else f"blk.{li}.{KIND_NAMES[k]}"
        if fmt == O.F32 and rows == 1:
            v = np.frombuffer(raw.tobytes(), np.float32)
            if f16_vectors:
                out.append((name, GGML_F16, (K,), v.astype(np.float16).tobytes()))
            else:
                out.append((name, GGML_F32, (K,), v.tobytes()))
        else:
            out.append((name, fmt, (K, rows), raw.tobytes()))
    return out
