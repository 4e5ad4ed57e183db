"""CPU checks of the C ABI library: it loads, exports every declared symbol, and
its host-only tooling (quantizers, seeded synthesis) behaves.  No device calls."""
import os
import re

import numpy as np
import pytest

from dotllm_amd import F32, Q4_0, Q4_K, Q5_K, Q6_K, Q8_0, _lib, byte_count, gguf, synth
from oracle import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    text = open(os.path.join(ROOT, "include", "llmdot_hip.h")).read()
    return sorted(set(re.findall(r"^\s*(?:const char\*|int32_t)\s+(llmdot_hip_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    names = declared_functions()
    assert len(names) == 50
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) - {"llmdot_hip_last_error"} == set(_lib.SIGNATURES)


def test_byte_count_matches_tensor_size():
    # TensorSizeTests.ByteCount_ReturnsExpectedSize
    assert byte_count(F32, 1024) == 4096 and byte_count(1, 1024) == 2048
    assert byte_count(Q8_0, 256) == 272 and byte_count(Q4_0, 256) == 144
    with pytest.raises(NotImplementedError):
        byte_count(999, 1024)
    for t in (Q4_K, Q5_K, Q6_K, Q8_0, Q4_0, F32):
        assert byte_count(t, 4096) == O.byte_count(t, 4096)


@pytest.mark.parametrize("t,step", [(Q8_0, 1 / 127), (Q4_0, 1 / 7), (Q4_K, 1 / 7), (Q5_K, 1 / 15), (Q6_K, 1 / 31)])
def test_quantize_roundtrip_through_reference_dequant(t, step):
    """The quantizers write layouts the reference decodes: the oracle's
    dequantisation recovers the input to within the format's step."""
    rng = np.random.default_rng(0)
    x = rng.normal(0, 0.02, size=(8, 1024)).astype(np.float32)
    q = synth.quantize(t, x)
    assert q.size == 8 * byte_count(t, 1024)
    y = O.dequantize(q, t, 8, 1024).reshape(8, 1024)
    blk = 32
    for r in range(8):
        for b in range(0, 1024, blk):
            xs, ys = x[r, b:b + blk], y[r, b:b + blk]
            span = float(xs.max() - xs.min())
            assert np.max(np.abs(xs - ys)) <= 1.2 * step * max(span, float(np.abs(xs).max()) * 2) + 1e-6


def test_synth_is_independent_of_thread_count():
    a = np.zeros(64 * byte_count(Q4_K, 512), dtype=np.uint8)
    b = np.zeros_like(a)
    synth.synth_tensor(Q4_K, 64, 512, 42, a, threads=1)
    synth.synth_tensor(Q4_K, 64, 512, 42, b, threads=7)
    assert np.array_equal(a, b)
    c = np.zeros(64 * 512 * 4, dtype=np.uint8)
    synth.synth_tensor(F32, 64, 512, 42, c, threads=3)
    w = c.view(np.float32)
    assert abs(float(w.mean())) < 1e-3 and abs(float(w.std()) - 0.02) < 1e-3


def test_synth_image_parses(tiny_image):
    g = gguf.read(tiny_image)
    cfg = gguf.resolve(g)
    assert (cfg.hidden_size, cfg.layer_count, cfg.head_count, cfg.head_count_kv, cfg.head_dim) == (512, 4, 8, 8, 64)
    assert (cfg.ffn_dim, cfg.vocab_size, cfg.eos_token_id, cfg.bos_token_id) == (1408, 32000, -1, 1)
    assert abs(cfg.norm_epsilon - 1e-5) < 1e-12 and cfg.rope_freq_base == 10000.0
    assert not cfg.tied_embeddings
    t = g.tensor("blk.0.attn_q.weight")
    assert (t.rows, t.cols, t.ggml_type) == (512, 512, Q8_0)
    assert t.data.nbytes == byte_count(Q8_0, 512 * 512)
    m = O.Model(tiny_image)
    assert (m.config.hidden, m.config.vocab, m.config.eos) == (512, 32000, -1)


def test_model_mix_types():
    tl = {n: t for n, _, _, t in synth.tensor_list(synth.SPECS["mistral7b"])}
    assert tl["output.weight"] == Q6_K and tl["blk.3.attn_v.weight"] == Q6_K
    assert tl["blk.3.attn_q.weight"] == Q4_K and tl["token_embd.weight"] == Q4_K
    assert tl["blk.0.attn_norm.weight"] == F32
    total = sum(byte_count(t, r * c) for n, r, c, t in synth.tensor_list(synth.SPECS["mistral7b"])
                if n != "token_embd.weight")
    assert total == 4069056512   # weight bytes read per 7B decode token (norms included)


def test_device_count_without_gpu_is_not_an_exception():
    from dotllm_amd.backend import device_count
    assert device_count() >= 0


def test_gguf_tool_roundtrip(tmp_path):
    """The shipped GGUF writer: a quantized file reads back with the reader the
    engine uses, and the oracle decodes its blocks to the quantizer's output."""
    rng = np.random.default_rng(2)
    w = rng.normal(0, 0.02, size=(64, 512)).astype(np.float32)
    norm = np.ones(512, np.float32)
    np.savez(tmp_path / "t.npz", **{"blk.0.attn_q.weight": w, "blk.0.attn_norm.weight": norm})
    for name, t in (("q4_k", Q4_K), ("q6_k", Q6_K), ("q8_0", Q8_0)):
        out = tmp_path / f"t_{name}.gguf"
        assert synth.main(["quantize", str(tmp_path / "t.npz"), str(out), "--type", name]) == 0
        m = gguf.read(str(out))
        ti = m.tensor("blk.0.attn_q.weight")
        assert (ti.ggml_type, ti.rows, ti.cols) == (t, 64, 512)
        assert m.tensor("blk.0.attn_norm.weight").ggml_type == F32
        blocks = np.asarray(ti.data)
        assert blocks.size == byte_count(t, 64 * 512)
        assert np.array_equal(blocks, synth.quantize(t, w))
        y = O.dequantize(blocks, t, 64, 512).reshape(64, 512)
        assert np.max(np.abs(y - w)) < 0.02


def test_gguf_tool_writes_loadable_model(tmp_path):
    out = tmp_path / "tiny.gguf"
    assert synth.main(["model", "tiny", str(out), "--context", "64"]) == 0
    raw = np.fromfile(out, dtype=np.uint8)
    assert np.array_equal(raw, synth.build_image("tiny", context=64))
    cfg = gguf.resolve(gguf.read(str(out)))
    assert (cfg.hidden_size, cfg.layer_count, cfg.vocab_size) == (512, 4, 32000)
