"""GGUF reader (host code, no GPU): the library's parser against the oracle's
restatement of gguf_file::Content::read (candle-core 0.8.4) and of
ModelWeights::from_gguf's metadata reads, on a hand-assembled known-answer
file, every truncation of it, whole model files from the test writer, the
reference's error cases and seeded byte mutations."""
import os
import struct

import numpy as np
import pytest

import gguf_reader as G
import oracle as O
from _gguf import (ARRAY, F32V, STRING, U32, U64, F64, gguf_bytes, model_metadata, model_tensors)
from _models import oracle_cfg


def _kat_v3() -> bytes:
    """Hand-assembled GGUF v3: 3 metadata entries, 1 tensor.  Offsets counted
    from the layout: header 24 B; general.alignment = 64 (u32) 33 B -> 57;
    llama.block_count = 1 (u32) 33 B -> 90; tokenizer.ggml.tokens = ["a",
    "bc", ""] 29 + 4 + 4 + 8 + 9 + 10 + 8 B -> 162; tensor output_norm.weight,
    1 dim of 8, F32, offset 0: 26 + 4 + 8 + 4 + 8 B -> 212; data at 256."""
    b = b"GGUF" + struct.pack("<IQQ", 3, 1, 3)
    b += struct.pack("<Q", 17) + b"general.alignment" + struct.pack("<II", 4, 64)
    b += struct.pack("<Q", 17) + b"llama.block_count" + struct.pack("<II", 4, 1)
    b += struct.pack("<Q", 21) + b"tokenizer.ggml.tokens" + struct.pack("<IIQ", 9, 8, 3)
    b += struct.pack("<Q", 1) + b"a" + struct.pack("<Q", 2) + b"bc" + struct.pack("<Q", 0)
    b += struct.pack("<Q", 18) + b"output_norm.weight" + struct.pack("<IQIQ", 1, 8, 0, 0)
    assert len(b) == 212
    b += b"\0" * 44
    return b + np.arange(8, dtype=np.float32).tobytes()


def _kat_v1() -> bytes:
    """The same content in GGUF v1 (u32 counts, lengths and dims): header 16 B;
    entries 21 + 4 + 4 B -> 45, -> 74; tokens 25 + 4 + 4 + 4 + 5 + 6 + 4 B
    -> 126; tensor 22 + 4 + 4 + 4 + 8 B -> 168; data at 192."""
    b = b"GGUF" + struct.pack("<III", 1, 1, 3)
    b += struct.pack("<I", 17) + b"general.alignment" + struct.pack("<II", 4, 64)
    b += struct.pack("<I", 17) + b"llama.block_count" + struct.pack("<II", 4, 1)
    b += struct.pack("<I", 21) + b"tokenizer.ggml.tokens" + struct.pack("<III", 9, 8, 3)
    b += struct.pack("<I", 1) + b"a" + struct.pack("<I", 2) + b"bc" + struct.pack("<I", 0)
    b += struct.pack("<I", 18) + b"output_norm.weight" + struct.pack("<IIIQ", 1, 8, 0, 0)
    assert len(b) == 168
    b += b"\0" * 24
    return b + np.arange(8, dtype=np.float32).tobytes()


def _write(tmp_path, data: bytes, name="m.gguf") -> str:
    p = os.path.join(str(tmp_path), name)
    with open(p, "wb") as f:
        f.write(data)
    return p


def _lib_view(hip, path, archs=(-1, 0, 1)):
    """("ok", layout, tensors, configs) or ("err", class name) from the library."""
    try:
        g = hip.GgufFile(path)
    except hip.BackendError:
        return ("err", "backend")
    with g:
        cfgs = {}
        for a in archs:
            try:
                c = g.config(a)
                cfgs[a] = dict(arch=c.arch, n_layers=c.n_layers, hidden=c.hidden, n_heads=c.n_heads,
                               n_kv_heads=c.n_kv_heads, head_dim=c.head_dim, ffn=c.ffn, vocab=c.vocab,
                               rope_theta=c.rope_theta, rms_eps=c.rms_eps, ctx_len=c.ctx_len,
                               tied_output=c.tied_output)
            except hip.BackendError:
                cfgs[a] = "backend"
            except hip.UnsupportedMethod:
                cfgs[a] = "unsupported"
        return ("ok", g.layout(), g.tensor_count(), cfgs)


def _oracle_view(data: bytes, archs=(-1, 0, 1)):
    try:
        g = G.read_gguf(data)
    except G.GgufError:
        return ("err", "backend")
    cfgs = {}
    for a in archs:
        try:
            c = G.gguf_config(g, a)
            c["rope_theta"] = float(np.float32(c["rope_theta"]))
            c["rms_eps"] = float(np.float32(c["rms_eps"]))
            cfgs[a] = c
        except G.GgufError:
            cfgs[a] = "backend"
        except G.GgufUnsupported:
            cfgs[a] = "unsupported"
    return ("ok", (g["version"], g["alignment"], g["data_offset"]), len(g["tensors"]), cfgs)


@pytest.mark.parametrize("version", [3, 1])
def test_known_answer_file(hip, tmp_path, version):
    data = _kat_v3() if version == 3 else _kat_v1()
    start = 256 if version == 3 else 192
    g = G.read_gguf(data)
    assert (g["version"], g["alignment"], g["data_offset"]) == (version, 64, start)
    assert g["metadata"]["llama.block_count"] == (4, 1)
    assert g["metadata"]["tokenizer.ggml.tokens"] == (9, (8, ["a", "bc", ""]))
    assert g["tensors"] == {"output_norm.weight": (0, (8,), 0, 32)}
    with hip.GgufFile(_write(tmp_path, data)) as f:
        assert f.layout() == (version, 64, start)
        assert f.tensor_count() == 1
        assert f.tensor_info("output_norm.weight") == (0, (8,), 0)
        vals = np.frombuffer(data[start:start + 32], np.float32)
        assert np.array_equal(vals, np.arange(8, dtype=np.float32))
        with pytest.raises(hip.BackendError, match="cannot find tensor info for output.weight"):
            f.tensor_info("output.weight")
        # from_gguf's first metadata read fails first
        with pytest.raises(hip.BackendError, match="cannot find llama.attention.head_count in GGUF metadata"):
            f.config(0)


def test_every_truncation_fails_cleanly(hip, tmp_path):
    """Cut before the end of the directory: an error from both readers, never
    a crash; cut inside the data: the directory still parses (the data are
    read, and bounds-checked, when a tensor loads)."""
    data = _kat_v3()
    for n in range(len(data)):
        p = _write(tmp_path, data[:n], "t.gguf")
        lib, ora = _lib_view(hip, p, archs=()), _oracle_view(data[:n], archs=())
        assert lib == ora, n
        assert (lib[0] == "err") == (n < 212), n


def _small_cfg(**over):
    d = dict(n_layers=2, hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=512, vocab=256, ctx_len=2048,
             rope_theta=500000.0, rms_eps=1e-6)
    d.update(over)
    return oracle_cfg(**d)


def _model_file(cfg, **kw):
    tensors = {k: O.synth_tensor(cfg, *k) for k in __import__("_models").all_tensor_keys(cfg)}
    md = model_metadata(cfg, **{k: v for k, v in kw.items() if k in ("rope_base", "vocab_tokens")})
    return gguf_bytes(md, model_tensors(cfg, tensors), version=kw.get("version", 3))


@pytest.mark.parametrize("arch,tied,version", [("llama", False, 3), ("qwen2", False, 3), ("llama", True, 2),
                                               ("qwen2", True, 1)])
def test_model_config(hip, tmp_path, arch, tied, version):
    cfg = _small_cfg(arch=arch, tied_output=tied, mix="q4_k_m" if arch == "llama" else "q5k_q80")
    data = _model_file(cfg, version=version, vocab_tokens=True)
    p = _write(tmp_path, data)
    lib, ora = _lib_view(hip, p), _oracle_view(data)
    assert lib == ora
    want = dict(arch=0 if arch == "llama" else 1, n_layers=2, hidden=256, n_heads=4, n_kv_heads=2, head_dim=64,
                ffn=512, vocab=256, rope_theta=500000.0, rms_eps=float(np.float32(1e-6)), ctx_len=2048,
                tied_output=int(tied))
    assert lib[3][-1] == want
    # the decoder type picks the key prefix: the other one's keys are missing
    other = 1 if arch == "llama" else 0
    assert lib[3][other] == "backend"
    with hip.GgufFile(p) as g:
        for name, layer, kind in G.tensor_names(G.gguf_config(G.read_gguf(data))):
            t, dims, off = g.tensor_info(name)
            fmt = cfg.fmt(layer, kind)
            rows, K = cfg.shape(kind)
            assert t == fmt and dims == ((K,) if rows == 1 else (K, rows)), name


def test_rope_base_default(hip, tmp_path):
    """rope.freq_base: absent or not an f32 -> 10000 (.and_then(to_f32).unwrap_or)."""
    cfg = _small_cfg()
    md = model_metadata(cfg, rope_base=False)
    tens = model_tensors(cfg, {k: O.synth_tensor(cfg, *k) for k in __import__("_models").all_tensor_keys(cfg)})
    for extra in ([], [("llama.rope.freq_base", F64, 500000.0)], [("llama.rope.freq_base", U32, 7)]):
        data = gguf_bytes(md + extra, tens)
        lib = _lib_view(hip, _write(tmp_path, data))
        assert lib == _oracle_view(data)
        assert lib[3][-1]["rope_theta"] == 10000.0


def _drop(md, key):
    return [e for e in md if e[0] != key]


def test_reference_error_cases(hip, tmp_path):
    cfg = _small_cfg()
    keys = {k: O.synth_tensor(cfg, *k) for k in __import__("_models").all_tensor_keys(cfg)}
    md = model_metadata(cfg)
    tens = model_tensors(cfg, keys)
    order = ["llama.attention.head_count", "llama.attention.head_count_kv", "llama.embedding_length",
             "llama.context_length", "llama.block_count", "llama.rope.dimension_count",
             "llama.attention.layer_norm_rms_epsilon"]
    # each missing key is named, and all earlier ones are read first
    for i, key in enumerate(order):
        m = md
        for k in order[i:]:
            m = _drop(m, k)
        data = gguf_bytes(m, tens)
        with hip.GgufFile(_write(tmp_path, data)) as g:
            with pytest.raises(hip.BackendError, match=f"cannot find {key} in GGUF metadata"):
                g.config(0)
        with pytest.raises(G.GgufError, match=f"cannot find {key} in GGUF metadata"):
            G.gguf_config(G.read_gguf(data), 0)
    # strict typing: a u64 where from_gguf calls to_u32
    bad = [(k, U64, v) if k == "llama.block_count" else (k, t, v) for k, t, v in md]
    data = gguf_bytes(bad, tens)
    with hip.GgufFile(_write(tmp_path, data)) as g, pytest.raises(hip.BackendError, match="not a u32"):
        g.config(0)
    # partial rotary embedding is not a shape the library runs
    bad = [(k, t, 32) if k == "llama.rope.dimension_count" else (k, t, v) for k, t, v in md]
    data = gguf_bytes(bad, tens)
    assert _lib_view(hip, _write(tmp_path, data))[3][0] == "unsupported" == _oracle_view(data)[3][0]
    # other architectures
    bad = [("general.architecture", STRING, "falcon") if k == "general.architecture" else (k, t, v)
           for k, t, v in md]
    data = gguf_bytes(bad, tens)
    assert _lib_view(hip, _write(tmp_path, data))[3][-1] == "unsupported"
    # the FFN width needs blk.0.ffn_gate.weight
    data = gguf_bytes(md, [e for e in tens if e[0] != "blk.0.ffn_gate.weight"])
    with hip.GgufFile(_write(tmp_path, data)) as g:
        with pytest.raises(hip.BackendError, match="cannot find tensor info for blk.0.ffn_gate.weight"):
            g.config(0)
    # header errors
    good = gguf_bytes(md, tens)
    for data, msg in ((b"GGUX" + good[4:], "unknown magic"), (good[:4] + struct.pack("<I", 4) + good[8:],
                                                              "unsupported version")):
        with pytest.raises(hip.BackendError, match=msg):
            hip.GgufFile(_write(tmp_path, data))
        with pytest.raises(G.GgufError, match=msg):
            G.read_gguf(data)
    with pytest.raises(hip.BackendError, match="open gguf"):
        hip.GgufFile(os.path.join(str(tmp_path), "absent.gguf"))


def test_alignment_and_metadata_types(hip, tmp_path):
    """general.alignment of each integer type; arrays of every element type,
    nested arrays, bools."""
    cfg = _small_cfg(n_layers=1)
    tens = model_tensors(cfg, {k: O.synth_tensor(cfg, *k) for k in __import__("_models").all_tensor_keys(cfg)})
    extra = [("x.u8", 0, 7), ("x.i8", 1, -7), ("x.u16", 2, 700), ("x.i16", 3, -700), ("x.i32", 5, -70000),
             ("x.f32", F32V, 1.5), ("x.bool", 7, 1), ("x.u64", U64, 1 << 40), ("x.i64", 11, -(1 << 40)),
             ("x.f64", F64, 2.5), ("x.arr_u8", ARRAY, (0, [1, 2, 3])), ("x.arr_bool", ARRAY, (7, [0, 1])),
             ("x.arr_f64", ARRAY, (F64, [1.0, 2.0])), ("x.nested", ARRAY, (ARRAY, [(U32, [1, 2]), (STRING, ["q"])])),
             ("x.empty", ARRAY, (STRING, []))]
    for at, av in ((U32, 64), (0, 16), (2, 128), (5, 256), (3, -8), (U64, 64), (F32V, 64.0)):
        md = model_metadata(cfg) + extra + [("general.alignment", at, av)]
        eff = av if at in (0, 2, U32, 5) and av >= 0 else 32
        data = gguf_bytes(md, tens, alignment=eff)
        lib = _lib_view(hip, _write(tmp_path, data))
        assert lib == _oracle_view(data)
        assert lib[1][1] == eff and lib[1][2] % eff == 0
    bad = model_metadata(cfg) + [("x.bool", 7, 2)]
    data = gguf_bytes(bad, tens)
    assert _lib_view(hip, _write(tmp_path, data)) == ("err", "backend") == _oracle_view(data)
    bad = model_metadata(cfg) + [("x.arr_bool", ARRAY, (7, [0, 3]))]
    data = gguf_bytes(bad, tens)
    assert _lib_view(hip, _write(tmp_path, data)) == ("err", "backend") == _oracle_view(data)
    zero = model_metadata(cfg) + [("general.alignment", U32, 0)]
    data = gguf_bytes(zero, tens, alignment=32)
    assert _lib_view(hip, _write(tmp_path, data)) == ("err", "backend") == _oracle_view(data)


def test_seeded_header_mutations(hip, tmp_path):
    """Random byte changes in the header and directory: both readers fail, or
    both read the same layout, directory size and configs."""
    cfg = _small_cfg(n_layers=1)
    data = _model_file(cfg, vocab_tokens=False)
    head = G.read_gguf(data)["data_offset"]
    rng = np.random.default_rng(1234)
    seen = {"ok": 0, "err": 0}
    for i in range(400):
        b = bytearray(data)
        for _ in range(int(rng.integers(1, 4))):
            b[int(rng.integers(0, head))] = int(rng.integers(0, 256))
        b = bytes(b)
        lib, ora = _lib_view(hip, _write(tmp_path, b, "f.gguf")), _oracle_view(b)
        assert lib == ora, i
        seen[lib[0]] += 1
    assert seen["ok"] > 20 and seen["err"] > 20, seen
