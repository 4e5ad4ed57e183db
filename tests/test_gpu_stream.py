"""Streaming Generate (llmdot_hip_generate_begin / _next): the
IAsyncEnumerable of InferenceEngine.Generate (IE:74-132) a batch of tokens per
device round trip.  The stream must yield exactly the one-shot Generate's
tokens and logits for every batch size, stop after EOS inside a batch
(IE:112-115), stop when the caller stops (cancellation, IE:103), end at the KV
cache's end, and be ended by any other call that changes the model's state."""
import ctypes as C

import numpy as np
import pytest

from dotllm_amd import _lib, synth
from dotllm_amd._lib import lib
from dotllm_amd.engine import GenerationOptions, InferenceEngine, LoadedModel, SamplingOptions, greedy

pytestmark = pytest.mark.gpu


def _next(eng, k, vocab=None):
    toks = np.zeros(k, np.int32)
    lg = np.zeros((k, vocab), np.float32) if vocab else None
    n, done = C.c_int32(0), C.c_int32(0)
    rc = lib().llmdot_hip_generate_next(eng.handle, k, toks.ctypes.data_as(C.POINTER(C.c_int32)), C.byref(n),
                                        C.byref(done), _lib.ptr(lg) if lg is not None else None)
    return rc, toks[:n.value].tolist(), (lg[:n.value] if lg is not None else None), bool(done.value)


def _begin(eng, prompt, n, eos=-1):
    p = np.ascontiguousarray(prompt, np.int32)
    return lib().llmdot_hip_generate_begin(eng.handle, p.ctypes.data_as(C.POINTER(C.c_int32)), p.size, n, eos,
                                           None, None)


def test_stream_equals_one_shot(hip, tiny_image):
    """Batches of 1, 3 and 7 tokens: the same 40 tokens and the same logits
    (bit for bit: the same kernels on the same inputs) as the one-shot call."""
    prompt = synth.prompt(32000, 12, seed=21)
    eng = InferenceEngine(LoadedModel.load(tiny_image), hip, kv_fp16=True, context=128)
    try:
        ref, ref_l = eng.generate_all(prompt, greedy(40), return_logits=True)
        for k in (1, 3, 7):
            assert _begin(eng, prompt, 40) == 0
            toks, logits, done = [], [], False
            while not done:
                rc, t, lg, done = _next(eng, k, eng.vocab)
                assert rc == 0 and 0 < len(t) <= k
                toks += t
                logits.append(lg)
            assert toks == ref, k
            assert np.array_equal(np.concatenate(logits), ref_l), k
            rc, t, _, done = _next(eng, k)
            assert rc == 0 and t == [] and done   # further calls report the end
        assert list(eng.generate(prompt, greedy(40), chunk=5)) == ref
    finally:
        eng.dispose()


def test_stream_stops_at_eos_inside_a_batch(hip):
    base = synth.build_image("tiny", seed=1234, sigma=0.05)
    prompt = synth.prompt(32000, 16, seed=7)
    eng = InferenceEngine(LoadedModel.load(base), hip, kv_fp16=True, context=64)
    free, _ = eng.generate_all(prompt, greedy(12))
    eng.dispose()
    eos = free[5]
    assert eos not in free[:5]
    img = synth.build_image("tiny", seed=1234, sigma=0.05, eos=eos)
    eng = InferenceEngine(LoadedModel.load(img), hip, kv_fp16=True, context=64)
    try:
        assert _begin(eng, prompt, 12, eos) == 0
        rc, t, _, done = _next(eng, 4)
        assert rc == 0 and t == free[:4] and not done
        rc, t, _, done = _next(eng, 4)      # tokens 4, 5 (= EOS); 6 and 7 are not returned
        assert rc == 0 and t == free[4:6] and done
        assert list(eng.generate(prompt, greedy(12), chunk=3)) == free[:6]
    finally:
        eng.dispose()


def test_stream_cancellation_and_session_end(hip, tiny_image):
    """Stopping after 5 tokens leaves the model usable: a new Generate gives the
    full one-shot result; a decode step ends a session (next fails)."""
    prompt = synth.prompt(32000, 10, seed=3)
    eng = InferenceEngine(LoadedModel.load(tiny_image), hip, kv_fp16=True, context=96)
    try:
        ref, _ = eng.generate_all(prompt, greedy(20))
        got = []
        for tok in eng.generate(prompt, greedy(20)):
            got.append(tok)
            if len(got) == 5:
                break
        assert got == ref[:5]
        assert list(eng.generate(prompt, greedy(20), chunk=4)) == ref
        assert _begin(eng, prompt, 20) == 0
        assert _next(eng, 2)[1] == ref[:2]
        eng.process_token(ref[1], len(prompt) + 1)
        rc, t, _, _ = _next(eng, 2)
        assert rc == _lib.E_INVALID and t == []
    finally:
        eng.dispose()


def test_stream_reaches_end_of_cache(hip, tiny_image):
    """Context 24, prompt 10: positions 10..23 leave room for 15 tokens; the
    batch holding the 15th returns it with LLMDOT_E_RANGE."""
    prompt = synth.prompt(32000, 10, seed=5)
    eng = InferenceEngine(LoadedModel.load(tiny_image), hip, kv_fp16=True, context=24)
    try:
        ref, _ = eng.generate_all(prompt, greedy(30))
        assert len(ref) == 15
        assert _begin(eng, prompt, 30) == 0
        toks, rc, done = [], 0, False
        while not done:
            rc, t, _, done = _next(eng, 4)
            toks += t
            if rc != 0:
                break
        assert rc == _lib.E_RANGE and done and toks == ref
        assert list(eng.generate(prompt, greedy(30), chunk=4)) == ref
    finally:
        eng.dispose()


def test_stream_sampled_equals_one_shot(hip, tiny_image):
    """Sampled: the same draws give the same tokens streamed (batches of 2) as
    in one call; the recent-token history carries across batches."""
    prompt = synth.prompt(32000, 16, seed=8)
    s = SamplingOptions(top_k=40, top_p=0.95, temperature=0.8, repeat_penalty=1.1, repeat_penalty_window_size=8)
    opts = GenerationOptions(max_tokens=24, sampling=s)
    draws = np.random.default_rng(2).random(24, dtype=np.float32)
    eng = InferenceEngine(LoadedModel.load(tiny_image), hip, kv_fp16=True, context=64)
    try:
        ref, _ = eng.generate_all(prompt, opts, draws=draws)
        assert len(ref) == 24
        assert list(eng.generate(prompt, opts, chunk=2, draws=draws)) == ref
        assert list(eng.generate(prompt, opts, chunk=24, draws=draws)) == ref
    finally:
        eng.dispose()
