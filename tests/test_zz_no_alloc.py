"""llmdot_hip_sample_noalloc (the allocation-free sampler over device pointers)
against llmdot_hip_sample on the same inputs, through the C ABI.

Each case runs two calls in a row on one context, the second with a smaller
vocabulary, so the second call reads scratch the first one left behind; the
token must equal llmdot_hip_sample's every time.  Sizes beyond the scratch are
rejected before anything is enqueued.
"""
import ctypes as C

import numpy as np
import pytest

from dotllm_amd import _lib
from dotllm_amd.backend import HipBackend, sampling_struct
from dotllm_amd.engine import SamplingOptions

pytestmark = pytest.mark.gpu

MAX_N = 262144


class _Dev:
    """Device buffers owned by one context (freed at close)."""

    def __init__(self, be):
        self.be, self.ptrs = be, []

    def put(self, arr):
        arr = np.ascontiguousarray(arr)
        p = C.c_void_p()
        _lib.check(_lib.lib().llmdot_hip_device_alloc(self.be.handle, max(arr.nbytes, 4), C.byref(p)))
        self.ptrs.append(p)
        if arr.nbytes:
            _lib.check(_lib.lib().llmdot_hip_memcpy_h2d(self.be.handle, p, _lib.ptr(arr), arr.nbytes))
        return p

    def get_i32(self, p):
        out = np.zeros(1, dtype=np.int32)
        _lib.check(_lib.lib().llmdot_hip_memcpy_d2h(self.be.handle, _lib.ptr(out), p, 4))
        return int(out[0])

    def close(self):
        for p in self.ptrs:
            _lib.lib().llmdot_hip_device_free(self.be.handle, p)
        self.ptrs = []


def _noalloc(be, dev, logits, opt, recent, r):
    lp = dev.put(logits.astype(np.float32))
    rp = dev.put(np.asarray(recent, dtype=np.int32)) if len(recent) else None
    tp = dev.put(np.full(1, -7, dtype=np.int32))
    s = sampling_struct(opt)
    rc = _lib.lib().llmdot_hip_sample_noalloc(be.handle, lp, logits.size, C.byref(s), rp, len(recent), float(r), tp)
    _lib.check(rc)
    _lib.check(_lib.lib().llmdot_hip_synchronize(be.handle))
    return dev.get_i32(tp)


CASES = [
    ("greedy", SamplingOptions(temperature=0.0)),
    ("topk40", SamplingOptions(temperature=0.8, top_k=40, repeat_penalty=1.1)),
    ("topp", SamplingOptions(temperature=1.3, top_k=0, top_p=0.9, repeat_penalty=1.0)),
    ("full", SamplingOptions(temperature=0.7, top_k=0, top_p=1.0, repeat_penalty=1.2)),
]


@pytest.mark.parametrize("name,opt", CASES, ids=[c[0] for c in CASES])
def test_noalloc_matches_sample(name, opt):
    be = HipBackend(0)
    dev = _Dev(be)
    try:
        rng = np.random.default_rng(hash(name) & 0xFFFF)
        for n in (128256, 32000):   # the second call is smaller: stale scratch must not leak in
            logits = (rng.normal(size=n) * 3).astype(np.float32)
            recent = rng.integers(0, n, size=80).tolist()
            for r in (0.05, 0.5, 0.97):
                want = be.sample(logits, opt, recent, r)
                got = _noalloc(be, dev, logits, opt, recent, r)
                assert got == want, (name, n, r, got, want)
    finally:
        dev.close()
        be.dispose()


def test_noalloc_nan_first_and_no_history():
    be = HipBackend(0)
    dev = _Dev(be)
    try:
        x = np.random.default_rng(3).normal(size=5000).astype(np.float32)
        x[0] = np.nan
        assert _noalloc(be, dev, x, SamplingOptions(temperature=0.0), [], 0.5) == 0 == be.arg_max(x)
        y = x[1:].copy()
        assert _noalloc(be, dev, y, SamplingOptions(temperature=0.0), [], 0.5) == int(np.argmax(y))
        opt = SamplingOptions(temperature=0.9, top_k=5, repeat_penalty=1.3)
        assert _noalloc(be, dev, y, opt, [], 0.3) == be.sample(y, opt, [], 0.3)
    finally:
        dev.close()
        be.dispose()


def test_noalloc_rejects_oversize():
    be = HipBackend(0)
    dev = _Dev(be)
    try:
        x = np.zeros(MAX_N + 1, dtype=np.float32)
        lp = dev.put(x)
        tp = dev.put(np.zeros(1, dtype=np.int32))
        s = sampling_struct(SamplingOptions(temperature=0.0))
        rc = _lib.lib().llmdot_hip_sample_noalloc(be.handle, lp, MAX_N + 1, C.byref(s), None, 0, 0.5, tp)
        assert rc == _lib.E_UNSUPPORTED
        assert b"262144" in _lib.lib().llmdot_hip_last_error()
    finally:
        dev.close()
        be.dispose()
