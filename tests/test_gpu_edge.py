"""Edge cases of the decode loop and the op-level contract against the oracle.

  * ArgMax NaN rules (VectorMath.ArgMax, VM:412-425): the scan starts from
    input[0] and compares with '>', so a NaN at index 0 is never replaced
    (result 0) and a NaN anywhere else never wins -- both in the op-level
    ArgMax and in the LM head's fused argmax, including a NaN logit that is
    the first row of a head workgroup.
  * EOS (InferenceEngine.cs:112-115): generation stops right after yielding
    the end-of-sequence token.
  * Tied embeddings (InferenceEngine.cs:585-589): without output.weight the
    LM head reads token_embd.weight.
  * Re-uploading a norm weight that a live model holds as an fp32 copy (F16
    norms, LoadedModel.GetDequantizedWeights, LM:63-75): the model reads the
    new values.
"""
import numpy as np
import pytest

from dotllm_amd import _lib, gguf, synth
from dotllm_amd.engine import InferenceEngine, LoadedModel, greedy
from oracle import oracle as O

pytestmark = pytest.mark.gpu

LOGIT_TOL = 2e-2


def test_argmax_nan_rules(hip):
    rng = np.random.default_rng(5)
    for n in (9, 4096, 4097, 32000, 128256):
        x = rng.normal(size=n).astype(np.float32)
        x[0] = np.nan
        assert hip.arg_max(x) == 0 == O.argmax(x), n
        y = x.copy()
        y[0] = 0.0
        y[rng.integers(1, n, size=max(1, n // 100))] = np.nan
        assert hip.arg_max(y) == O.argmax(y) == int(np.nanargmax(y)), n
        z = np.full(n, np.nan, dtype=np.float32)
        assert hip.arg_max(z) == 0 == O.argmax(z), n


def _nan_rows(img, rows):
    """Sets every block scale of the given output.weight rows (Q8_0) to NaN."""
    t = gguf.read(img).tensor("output.weight")
    assert t.ggml_type == _lib.Q8_0
    rb = _lib.byte_count(_lib.Q8_0, t.cols)
    for r in rows:
        row = t.data[r * rb:(r + 1) * rb]
        for b in range(0, rb, 34):
            row[b:b + 2] = np.frombuffer(np.float16(np.nan).tobytes(), dtype=np.uint8)


@pytest.mark.parametrize("nan_first", [False, True])
def test_head_argmax_nan_logits(hip, nan_first):
    """Every fourth logit (each LM-head workgroup's first row among them) NaN:
    the greedy token is the oracle's ArgMax of its own logits at every step;
    with logit 0 NaN as well it is always token 0."""
    img = synth.build_image("tiny", seed=77).copy()
    rows = [r for r in range(4, 32000, 4)] + ([0] if nan_first else [])
    _nan_rows(img, rows)
    prompt = synth.prompt(32000, 6, seed=3)
    ref = O.Model(img, kv_fp16=True)
    rt, rl = ref.generate(prompt, 6, return_logits=True)
    ref.close()
    assert all(np.isnan(rl[:, 4]))
    eng = InferenceEngine(LoadedModel.load(img), hip, kv_fp16=True)
    gt, gl = eng.generate_all(prompt, greedy(6), return_logits=True)
    eng.dispose()
    assert gt == rt
    if nan_first:
        assert gt == [0] * 6
    assert np.array_equal(np.isnan(gl), np.isnan(rl))
    ok = ~np.isnan(rl)
    assert float(np.max(np.abs(gl[ok] - rl[ok]))) <= LOGIT_TOL


def test_generate_stops_at_eos(hip):
    """EOS set to the token the oracle yields at step 5: six tokens, the last
    being EOS, identical to the oracle's; without EOS the run continues."""
    # sigma 0.05: the default 0.02 tiny model settles on one repeated token
    base = synth.build_image("tiny", seed=1234, sigma=0.05)
    prompt = synth.prompt(32000, 16, seed=7)
    ref = O.Model(base, kv_fp16=True)
    free, _ = ref.generate(prompt, 12, eos=-1)
    ref.close()
    eos = free[5]
    assert eos not in free[:5], "pick a seed whose step-5 token is new"
    img = synth.build_image("tiny", seed=1234, sigma=0.05, eos=eos)
    lm = LoadedModel.load(img)
    assert lm.config.eos_token_id == eos
    ref = O.Model(img, kv_fp16=True)
    rt, _ = ref.generate(prompt, 12)
    ref.close()
    assert rt == free[:6]
    eng = InferenceEngine(lm, hip, kv_fp16=True)
    gt, _ = eng.generate_all(prompt, greedy(12))
    assert gt == rt
    eng.dispose()


def test_tied_embeddings(hip):
    """No output.weight: logits from token_embd.weight (Q8_0, tied)."""
    img = synth.build_image("tiny", seed=4321, tied=True)
    lm = LoadedModel.load(img)
    assert lm.config.tied_embeddings and not lm.gguf.has("output.weight")
    prompt = synth.prompt(32000, 16, seed=9)
    ref = O.Model(img, kv_fp16=True)
    assert ref.config.tied_embeddings == 1
    rt, rl = ref.generate(prompt, 32, return_logits=True)
    ref.close()
    eng = InferenceEngine(lm, hip, kv_fp16=True)
    gt, gl = eng.generate_all(prompt, greedy(32), return_logits=True)
    eng.dispose()
    assert gt == rt
    assert float(np.max(np.abs(gl - rl))) <= LOGIT_TOL


def test_f16_norm_reupload_reaches_model(hip):
    """F16 norm weights are held by the model as fp32 copies; re-uploading
    different bytes in place must change what the live model computes, to
    exactly what a model created on the new bytes computes."""
    from dotllm_amd.backend import HipBackend
    img = synth.build_image("tiny", seed=99, norm_type=_lib.F16)
    lm = LoadedModel.load(img)
    be = HipBackend(0)
    eng = InferenceEngine(lm, be, kv_fp16=True)
    before = eng.process_token(11, 0)
    t = lm.tensor("blk.1.ffn_norm.weight")
    assert t.ggml_type == _lib.F16
    new = np.random.default_rng(0).uniform(0.5, 1.5, size=t.cols).astype(np.float16).view(np.uint8)
    be.upload_weight(lm.key_prefix + "blk.1.ffn_norm.weight", _lib.F16, new, t.rows, t.cols)
    after = eng.process_token(11, 0)
    eng.dispose()
    be.dispose()
    assert not np.array_equal(before, after)
    img2 = img.copy()
    gguf.read(img2).tensor("blk.1.ffn_norm.weight").data[:] = new
    be2 = HipBackend(0)
    fresh = InferenceEngine(LoadedModel.load(img2), be2, kv_fp16=True)
    want = fresh.process_token(11, 0)
    fresh.dispose()
    be2.dispose()
    assert np.array_equal(after, want)
    ref = O.Model(img2, kv_fp16=True)
    rl = ref.process_token(11, 0)
    ref.close()
    assert float(np.max(np.abs(after - rl))) <= LOGIT_TOL
