"""GGUF reader and the from_gguf hyper-parameter reads -- TEST INFRASTRUCTURE ONLY.

Only ``tests/`` may import this module, to check the library's GGUF
loader; the product never imports it.

* ``read_gguf`` restates ``gguf_file::Content::read`` of candle-core 0.8.4
  (the reference's pinned dependency, ``Cargo.lock``; its source is not part
  of the reference checkout), i.e. the published GGUF v1-v3 layout: magic
  "GGUF", u32 version, tensor and metadata counts (u32 in v1, u64 from v2),
  typed metadata values (strings and array lengths u32 in v1, u64 from v2),
  the tensor directory (name, u32 n_dims, dims (u32 in v1), u32 GGML type,
  u64 offset), then the data section at the next multiple of
  ``general.alignment`` (default 32; an unsigned or non-negative 8/16/32-bit
  integer value, anything else keeps the default).
* ``gguf_config`` restates the metadata reads of ``ModelWeights::from_gguf``
  (``crates/speculate/src/model/quantized_llama_local.rs:222-252``,
  ``quantized_qwen2_local.rs:215-241``): the keys in the same order, strict
  u32 / f32 typing (``Value::to_u32`` / ``to_f32``), ``rope.freq_base``
  defaulting to 10000 when absent or not an f32, head_dim =
  embedding_length // head_count, the tied-output fallback when
  ``output.weight`` is absent.  The FFN width and the vocabulary are the rows
  of ``blk.0.ffn_gate.weight`` and ``token_embd.weight``, the shapes the
  forward multiplies with.

Pinned by a hand-assembled known-answer file (``tests/test_gguf_host.py``,
every offset counted from the layout above) in v3 and v1, by truncation at
every byte, and by the round trip through the test writer.  Errors are
``GgufError`` (the reference's Error::Candle) and ``GgufUnsupported``.
"""
from __future__ import annotations

import struct
from typing import Dict, Tuple

MAGIC = 0x46554747
SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<B", 10: "<Q", 11: "<q", 12: "<d"}
STRING, ARRAY = 8, 9
# GGML type -> (elements per block, bytes per block), the types candle-core 0.8.4 knows
BLOCK = {0: (1, 4), 1: (1, 2), 30: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34),
         9: (32, 36), 10: (256, 84), 11: (256, 110), 12: (256, 144), 13: (256, 176), 14: (256, 210),
         15: (256, 292)}


class GgufError(Exception):
    pass


class GgufUnsupported(Exception):
    pass


class _Reader:
    def __init__(self, data: bytes):
        self.d = data
        self.at = 0

    def take(self, n: int) -> bytes:
        if n > len(self.d) - self.at:
            raise GgufError("gguf: unexpected end of file")
        b = self.d[self.at:self.at + n]
        self.at += n
        return b

    def scalar(self, fmt: str):
        return struct.unpack(fmt, self.take(struct.calcsize(fmt)))[0]

    def length(self, version: int) -> int:
        return self.scalar("<I" if version == 1 else "<Q")

    def string(self, version: int) -> str:
        return self.take(self.length(version)).decode("latin-1")

    def value(self, t: int, version: int, depth: int = 0):
        if t in SCALAR:
            v = self.scalar(SCALAR[t])
            if t == 7 and v > 1:
                raise GgufError(f"gguf: bool value {v}")
            return v
        if t == STRING:
            return self.string(version)
        if t == ARRAY:
            if depth >= 8:
                raise GgufError("gguf: arrays nested too deeply")
            et = self.scalar("<I")
            n = self.length(version)
            if et in SCALAR:
                size = struct.calcsize(SCALAR[et])
                if n > (len(self.d) - self.at) // size:
                    raise GgufError("gguf: unexpected end of file")
                if et == 7:
                    return (et, [self.value(et, version) for _ in range(n)])
                raw = self.take(n * size)
                return (et, list(struct.unpack("<" + SCALAR[et][1] * n, raw)) if n else [])
            if et not in (STRING, ARRAY):
                raise GgufError(f"gguf: unknown metadata value type {et}")
            out = []
            for _ in range(n):
                out.append(self.value(et, version, depth + 1))
            return (et, out)
        raise GgufError(f"gguf: unknown metadata value type {t}")


def read_gguf(data: bytes) -> Dict:
    """{"version", "alignment", "data_offset", "metadata": {key: (type, value)},
    "tensors": {name: (ggml type, dims with ne[0] first, offset, bytes)}}."""
    r = _Reader(data)
    magic = r.scalar("<I")
    if magic != MAGIC:
        raise GgufError(f"gguf: unknown magic 0x{magic:08x}")
    version = r.scalar("<I")
    if version not in (1, 2, 3):
        raise GgufError(f"gguf: unsupported version {version}")
    n_tensors = r.length(version)
    n_kv = r.length(version)
    md = {}
    for _ in range(n_kv):
        key = r.string(version)
        t = r.scalar("<I")
        md[key] = (t, r.value(t, version))
    tensors = {}
    for _ in range(n_tensors):
        name = r.string(version)
        nd = r.scalar("<I")
        if nd > 4:
            raise GgufError(f"gguf: tensor {name} has {nd} dims")
        dims = []
        elems = 1
        for _ in range(nd):
            ne = r.scalar("<I" if version == 1 else "<Q")
            if elems * ne > 1 << 62:
                raise GgufError(f"gguf: tensor {name} is too large")
            elems *= ne
            dims.append(ne)
        t = r.scalar("<I")
        off = r.scalar("<Q")
        if t not in BLOCK:
            raise GgufError(f"gguf: unknown dtype {t} for tensor {name}")
        be, bb = BLOCK[t]
        if (dims[0] if dims else 1) % be:
            raise GgufError(f"gguf: tensor {name}: rows are not whole blocks")
        tensors[name] = (t, tuple(dims), off, elems // be * bb)
    align = 32
    if "general.alignment" in md:
        t, v = md["general.alignment"]
        if t in (0, 2, 4) or (t in (1, 3, 5) and v >= 0):
            align = v
    if align == 0:
        raise GgufError("gguf: general.alignment is 0")
    data_off = (r.at + align - 1) // align * align
    return {"version": version, "alignment": align, "data_offset": data_off, "metadata": md, "tensors": tensors}


def _u32(g: Dict, key: str) -> int:
    if key not in g["metadata"]:
        raise GgufError(f"cannot find {key} in GGUF metadata")
    t, v = g["metadata"][key]
    if t != 4:
        raise GgufError(f"not a u32: {key}")
    if v > 0x7FFFFFFF:
        raise GgufUnsupported(f"{key} = {v} is out of range")
    return v


def _tensor(g: Dict, name: str):
    if name not in g["tensors"]:
        raise GgufError(f"cannot find tensor info for {name}")
    return g["tensors"][name]


def gguf_config(g: Dict, arch: int = -1) -> Dict:
    """The decoder hyper-parameters of a parsed file; arch 0 llama, 1 qwen2,
    -1 from general.architecture.  ctx_len is the file's context_length."""
    md = g["metadata"]
    if arch < 0:
        if "general.architecture" not in md:
            raise GgufError("cannot find general.architecture in GGUF metadata")
        t, v = md["general.architecture"]
        if t != STRING:
            raise GgufError("not a string: general.architecture")
        if v not in ("llama", "qwen2"):
            raise GgufUnsupported(f"gguf: architecture '{v}'")
        arch = 0 if v == "llama" else 1
    p = "llama." if arch == 0 else "qwen2."
    n_heads = _u32(g, p + "attention.head_count")
    n_kv = _u32(g, p + "attention.head_count_kv")
    hidden = _u32(g, p + "embedding_length")
    ctx = _u32(g, p + "context_length")
    n_layers = _u32(g, p + "block_count")
    rope_dim = _u32(g, "llama.rope.dimension_count") if arch == 0 else None
    key = p + "attention.layer_norm_rms_epsilon"
    if key not in md:
        raise GgufError(f"cannot find {key} in GGUF metadata")
    if md[key][0] != 6:
        raise GgufError(f"not a f32: {key}")
    eps = md[key][1]
    theta = 10000.0
    if p + "rope.freq_base" in md and md[p + "rope.freq_base"][0] == 6:
        theta = md[p + "rope.freq_base"][1]
    if n_heads == 0:
        raise GgufError(p + "attention.head_count is 0")
    head_dim = hidden // n_heads
    if arch == 0 and rope_dim != head_dim:
        raise GgufUnsupported(f"llama.rope.dimension_count {rope_dim} != head_dim {head_dim}")
    gate = _tensor(g, "blk.0.ffn_gate.weight")
    embd = _tensor(g, "token_embd.weight")
    dim1 = lambda t: t[1][1] if len(t[1]) > 1 else 1  # noqa: E731
    if dim1(gate) > 0x7FFFFFFF or dim1(embd) > 0x7FFFFFFF:
        raise GgufUnsupported("gguf: tensor too large")
    return dict(arch=arch, n_layers=n_layers, hidden=hidden, n_heads=n_heads, n_kv_heads=n_kv, head_dim=head_dim,
                ffn=dim1(gate), vocab=dim1(embd), rope_theta=float(theta), rms_eps=float(eps), ctx_len=ctx,
                tied_output=0 if "output.weight" in g["tensors"] else 1)


def tensor_names(cfg: Dict) -> Tuple[Tuple[str, int, int], ...]:
    """(name, layer, kind) of every tensor from_gguf loads, in its order
    (quantized_llama_local.rs:242-281, quantized_qwen2_local.rs:232-283);
    kinds are the library's tensor kind ids."""
    out = [("token_embd.weight", -1, 0), ("output_norm.weight", -1, 2)]
    if not cfg["tied_output"]:
        out.append(("output.weight", -1, 1))
    for i in range(cfg["n_layers"]):
        b = f"blk.{i}."
        out += [(b + "attn_q.weight", i, 3), (b + "attn_k.weight", i, 4), (b + "attn_v.weight", i, 5)]
        if cfg["arch"] == 1:
            out += [(b + "attn_q.bias", i, 12), (b + "attn_k.bias", i, 13), (b + "attn_v.bias", i, 14)]
        out += [(b + "attn_output.weight", i, 6), (b + "ffn_gate.weight", i, 7), (b + "ffn_down.weight", i, 9),
                (b + "ffn_up.weight", i, 8), (b + "attn_norm.weight", i, 10), (b + "ffn_norm.weight", i, 11)]
    return tuple(out)
