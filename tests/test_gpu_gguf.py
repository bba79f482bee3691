"""GGUF loading on the GPU: a .gguf file written from a model's tensors loads
into the same device weights, byte for byte, and the same logits, bit for
bit, as uploading the tensors one by one; against the oracle forward of the
same tensors to the 1e-2 contract.  Covers Llama (Q4_K_M) and Qwen2 (Q5_K /
Q8_0 with QKV bias), the tied-output fallback, F16 norms, and the errors that
leave the decoder as it was."""
import os

import numpy as np
import pytest

import oracle as O
from _gguf import U32, gguf_bytes, model_metadata, model_tensors
from _models import all_tensor_keys, hip_cfg, oracle_cfg, rel_err

pytestmark = pytest.mark.gpu


def _cfg(**over):
    d = dict(n_layers=2, hidden=512, n_heads=8, n_kv_heads=2, head_dim=64, ffn=1024, vocab=2048, ctx_len=512,
             rope_theta=500000.0, rms_eps=1e-6)
    d.update(over)
    return oracle_cfg(**d)


def _tensors(cfg, seed=5):
    """Synthetic blocks, with norms drawn around 1 (not all ones) so that a
    swapped norm would show."""
    rng = np.random.default_rng(seed)
    t = {}
    for (li, k) in all_tensor_keys(cfg):
        fmt, raw = O.synth_tensor(cfg, li, k)
        if k in (O.K_OUTPUT_NORM, O.K_ATTN_NORM, O.K_FFN_NORM):
            raw = (1.0 + 0.1 * rng.standard_normal(cfg.hidden)).astype(np.float32).view(np.uint8)
        t[(li, k)] = (fmt, raw)
    return t


def _write(tmp_path, data, name="m.gguf"):
    p = os.path.join(str(tmp_path), name)
    with open(p, "wb") as f:
        f.write(data)
    return p


def _twin(hip, cfg, tensors):
    dec = hip.HipQuantDecoder(hip_cfg(hip, cfg))
    for (li, k), (fmt, raw) in tensors.items():
        dec.set_tensor(li, k, fmt, raw)
    return dec


def _logits(dec, prefix, drafts):
    dec.reset()
    dec.observe(prefix)
    return dec.batched_logits(drafts)


@pytest.mark.parametrize("arch,mix", [("llama", "q4_k_m"), ("qwen2", "q5k_q80")])
def test_gguf_load_equals_tensor_upload(hip, tmp_path, arch, mix):
    cfg = _cfg(arch=arch, mix=mix)
    tensors = _tensors(cfg)
    path = _write(tmp_path, gguf_bytes(model_metadata(cfg), model_tensors(cfg, tensors)))
    dec = hip.HipQuantDecoder.from_gguf(path, ctx_len=cfg.ctx_len)
    want = hip_cfg(hip, cfg)
    assert np.float32(dec.cfg.rms_eps) == np.float32(want.rms_eps)  # stored as f32 in the file
    dec.cfg.rms_eps = want.rms_eps
    assert dec.cfg == want
    for (li, k), (fmt, raw) in tensors.items():
        f, rows, K, nbytes = dec.tensor_info(li, k)
        assert f == fmt and (rows, K) == cfg.shape(k) and nbytes == raw.size, (li, k)
        assert np.array_equal(dec.get_tensor(li, k), raw), (li, k)
    twin = _twin(hip, cfg, tensors)
    rng = np.random.default_rng(9)
    prefix = [int(v) for v in rng.integers(0, cfg.vocab, 40)]
    drafts = [int(v) for v in rng.integers(0, cfg.vocab, 4)]
    got = _logits(dec, prefix, drafts)
    assert np.array_equal(got.view(np.uint32), _logits(twin, prefix, drafts).view(np.uint32))
    od = O.OracleDecoder(O.OracleModel(cfg, tensors))
    od.observe(prefix)
    assert rel_err(got, od.batched_logits(drafts)) < 1e-2
    dec.close()
    twin.close()


def test_gguf_tied_output_and_f16_norms(hip, tmp_path):
    """No output.weight: lm_head is token_embd (quantized_llama_local.rs:248-252);
    norms stored as F16 load as their exact f32 values."""
    cfg = _cfg(tied_output=True, mix="q4_k")
    tensors = _tensors(cfg, seed=6)
    path = _write(tmp_path, gguf_bytes(model_metadata(cfg), model_tensors(cfg, tensors, f16_vectors=True)))
    with hip.GgufFile(path) as g:
        assert g.config().tied_output == 1
    dec = hip.HipQuantDecoder.from_gguf(path, arch=hip.ARCH_LLAMA, ctx_len=cfg.ctx_len)
    widened = {}
    for key, (fmt, raw) in tensors.items():
        if fmt == O.F32:
            raw = np.frombuffer(raw.tobytes(), np.float32).astype(np.float16).astype(np.float32).view(np.uint8)
        widened[key] = (fmt, raw)
    for (li, k), (fmt, raw) in widened.items():
        assert np.array_equal(dec.get_tensor(li, k), raw), (li, k)
    twin = _twin(hip, cfg, widened)
    rng = np.random.default_rng(10)
    prefix = [int(v) for v in rng.integers(0, cfg.vocab, 33)]
    drafts = [int(v) for v in rng.integers(0, cfg.vocab, 3)]
    got = _logits(dec, prefix, drafts)
    assert np.array_equal(got.view(np.uint32), _logits(twin, prefix, drafts).view(np.uint32))
    od = O.OracleDecoder(O.OracleModel(cfg, widened))
    od.observe(prefix)
    assert rel_err(got, od.batched_logits(drafts)) < 1e-2
    dec.close()
    twin.close()


def test_gguf_load_errors_leave_the_decoder_unchanged(hip, tmp_path):
    cfg = _cfg(mix="q4_k")
    tensors = _tensors(cfg, seed=7)
    md, ents = model_metadata(cfg), model_tensors(cfg, tensors)
    dec = _twin(hip, cfg, tensors)
    rng = np.random.default_rng(11)
    prefix = [int(v) for v in rng.integers(0, cfg.vocab, 20)]
    drafts = [int(v) for v in rng.integers(0, cfg.vocab, 2)]
    before = _logits(dec, prefix, drafts)

    def load(data, exc, match):
        with hip.GgufFile(_write(tmp_path, data, "e.gguf")) as g:
            with pytest.raises(exc, match=match):
                hip._check(hip._lib.sd_model_load_gguf(dec._h, g._h))
        assert np.array_equal(_logits(dec, prefix, drafts).view(np.uint32), before.view(np.uint32))

    # a file of another shape
    other = _cfg(mix="q4_k", n_layers=1)
    load(gguf_bytes(model_metadata(other), model_tensors(other, _tensors(other))), hip.ArgError, "config")
    # a matrix in a format the library does not run (Q4_0: 18-byte blocks of 32)
    rows, K = cfg.shape(O.K_ATTN_K)
    q40 = rng.integers(0, 256, rows * K // 32 * 18, dtype=np.uint8).tobytes()
    bad = [(n, 2, d, q40) if n == "blk.1.attn_k.weight" else (n, t, d, r) for n, t, d, r in ents]
    load(gguf_bytes(md, bad), hip.UnsupportedMethod, "blk.1.attn_k.weight")
    # a tensor shaped unlike the metadata says
    bad = [(n, t, (d[0] // 2,), r[:len(r) // 2]) if n == "blk.0.ffn_norm.weight" else (n, t, d, r)
           for n, t, d, r in ents]
    load(gguf_bytes(md, bad), hip.BackendError, "blk.0.ffn_norm.weight: shape")
    # a missing tensor, named as from_gguf names it
    load(gguf_bytes(md, [e for e in ents if e[0] != "blk.1.ffn_up.weight"]), hip.BackendError,
         "cannot find tensor info for blk.1.ffn_up.weight")
    # a file cut short inside the last tensor's data
    full = gguf_bytes(md, ents)
    load(full[:-100], hip.BackendError, "past the end of the file")
    # an alignment that puts the data section past the end of the file
    load(gguf_bytes(md + [("general.alignment", U32, 1 << 24)], ents), hip.BackendError, "past the end of the file")
    dec.close()
