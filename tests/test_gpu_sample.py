"""Parity of the device sampler (Sampler.Sample, Sampler.cs:24-170) with the
oracle, the uniform draw r given to both.

top-k path (0 < TopK < n): the device does the reference's arithmetic (the same
selection, VectorMath.Softmax summation order and sequential draw), so the token
must equal the oracle's for every draw; the logits are continuous random values,
so no two are equal.
top-p path (TopP < 1): the device computes the reference as written -- the
softmax in its summation order, FindNucleus's selection-sort order (ties
included), the values it writes into the probability buffer it still reads
from (Sampler.cs:30, 48-50, 150), the sequential float running sum, the
renormalised draw, and the fall-through draw over the rewritten buffer, which
returns a rank (Sampler.cs:61) -- so the token must equal the oracle's
(aliased=True, the reference as written) for every draw, with no exemption.
no top-p (TopP >= 1, TopK off): the draw over all n probabilities in index
order is placed with fp64 running sums, the reference's with a sequential float
sum, so the token must equal the oracle's unless r lies within float rounding
of a cumulative boundary: a mismatch is accepted only if the oracle itself
returns the device's token for r moved by at most 1e-4.
"""
from dataclasses import replace

import numpy as np
import pytest

from dotllm_amd.engine import GenerationOptions, InferenceEngine, LoadedModel, SamplingOptions
from oracle import oracle as O

pytestmark = pytest.mark.gpu

R_ALL = [0.0, 1e-6, 0.013, 0.11, 0.29, 0.5, 0.61, 0.77, 0.93, 0.999, 0.9999999, 1.0]
R_FEW = [0.0, 0.29, 0.77, 0.9999999]
LOGIT_TOL = 2e-2


def opts(temperature, top_k, top_p=1.0, penalty=1.0, window=0):
    return SamplingOptions(top_k=top_k, top_p=top_p, temperature=temperature, repeat_penalty=penalty,
                           repeat_penalty_window_size=window)


def ref(x, o, recent, r, aliased=True):
    return O.sample(x, o.temperature, o.top_k, o.top_p, o.repeat_penalty, o.repeat_penalty_window_size, recent, r,
                    aliased=aliased)


def near_boundary(x, o, recent, r, tok, eps=1e-4, aliased=True):
    for d in (eps / 16, -eps / 16, eps / 4, -eps / 4, eps, -eps):
        if ref(x, o, recent, min(max(r + d, 0.0), 1.0), aliased) == tok:
            return True
        if o.top_p < 1.0 and ref(x, replace(o, top_p=o.top_p + d), recent, r, aliased) == tok:
            return True
    return False


def logits_for(n, seed, scale=3.0):
    return np.random.default_rng(seed).normal(0, scale, n).astype(np.float32)


def test_greedy_is_argmax(hip):
    x = logits_for(32000, 1)
    for r in (0.0, 0.5):
        assert hip.sample(x, opts(0.0, 40, 0.9, 1.1, 64), [int(np.argmax(x))], r) == int(np.argmax(x))


TOPK_CASES = [(100, 1, 0.8), (100, 3, 1.0), (100, 40, 0.7), (1000, 999, 1.3), (32000, 40, 0.8),
              (32000, 4096, 1.1), (128256, 40, 0.8), (128256, 4096, 0.6), (13, 12, 0.9), (37, 11, 2.0)]


@pytest.mark.parametrize("n,k,temp", TOPK_CASES)
def test_top_k_matches_oracle(hip, n, k, temp):
    x = logits_for(n, n + k)
    o = opts(temp, k)
    for r in (R_ALL if n * k <= 4_000_000 else R_FEW):
        assert hip.sample(x, o, [], r) == ref(x, o, [], r), r


def test_top_k_with_repeat_penalty(hip):
    """Duplicates apply once per occurrence, only the last `window` entries count,
    ids outside the vocabulary are skipped; penalised values of both signs."""
    n = 32000
    x = logits_for(n, 5)
    top = np.argsort(-x)[:12]
    x[top[3]] = -abs(x[top[3]])
    recent = [int(top[0]), int(top[1]), int(top[0]), -3, n + 7, int(top[3]), int(top[2]), int(top[2]), int(top[0])]
    for pen, window in ((1.1, 64), (2.5, 64), (3.0, 4), (0.5, 6)):
        o = opts(0.9, 40, 1.0, pen, window)
        for r in R_ALL:
            assert hip.sample(x, o, recent, r) == ref(x, o, recent, r), (pen, window, r)


TOPP_CASES = [(100, 0, 0.5), (100, 100, 0.9), (4096, 0, 0.95), (4096, 0, 0.5), (32000, 0, 0.9),
              (32000, 32000, 0.95), (37, 0, 0.9), (1000, 0, 0.01), (1000, 0, 0.99999994), (13, 0, 0.99999994),
              (5000, 0, 0.999), (8, 0, 0.7)]


def aliasing_touches(x, o, top_p):
    """Whether any rank inside the reference's nucleus (or the whole buffer,
    when the nucleus spans all n) reads a slot already rewritten."""
    p = np.exp((x / o.temperature - np.max(x / o.temperature)).astype(np.float64))
    p /= p.sum()
    order = np.argsort(-p, kind="stable")
    m = min(int(np.searchsorted(np.cumsum(p[order]), top_p)) + 1, x.size)
    return any(int(order[i]) < i for i in range(m))


@pytest.mark.parametrize("n,k,top_p", TOPP_CASES)
def test_top_p_matches_reference(hip, n, k, top_p):
    """Continuous random logits: every draw's token is the reference's as
    written (the aliased buffers), exactly."""
    x = logits_for(n, n + 3, 2.0)
    o = opts(0.8, k, top_p)
    for r in (R_ALL if n <= 5000 else R_FEW):
        assert hip.sample(x, o, [], r) == ref(x, o, [], r), r


@pytest.mark.parametrize("n,step,top_p", [(200, 0.5, 0.9), (4096, 0.25, 0.95), (4096, 1.0, 0.8), (1000, 0.5, 0.99999994),
                                          (30, 2.0, 0.9)])
def test_top_p_ties_match_reference(hip, n, step, top_p):
    """Logits rounded to a grid, so many probabilities are exactly equal: the
    reference's selection sort orders equal values by the positions its swaps
    left them at, which decides which rewritten slots later ranks read; every
    draw's token is the reference's, exactly."""
    x = (np.round(logits_for(n, 31 + n, 2.0) / step) * step).astype(np.float32)
    assert np.unique(x).size < n // 2 + 1
    o = opts(0.8, 0, top_p)
    for r in R_ALL:
        assert hip.sample(x, o, [], r) == ref(x, o, [], r), r


def test_top_p_aliasing_is_exercised():
    """The cases above include nuclei in which ranks read rewritten slots, so
    they would fail for the separate-buffer form (the oracle shows the two forms
    differ on at least one of their draws)."""
    def first_difference():
        for n, k, top_p in TOPP_CASES:
            x = logits_for(n, n + 3, 2.0)
            o = opts(0.8, k, top_p)
            if not aliasing_touches(x, o, top_p):
                continue
            for r in (R_ALL if n <= 5000 else R_FEW):
                if ref(x, o, [], r, aliased=True) != ref(x, o, [], r, aliased=False):
                    return (n, k, top_p, r)
        return None
    assert first_difference() is not None


def test_top_p_nucleus_spanning_all(hip):
    """Ten tokens carry all but ~1.1e-4 of the mass and 9990 carry ~1.1e-8
    each, below half an ulp of the running sum near 1, so FindNucleus's float
    sum stalls at 0.9998741, under TopP = 0.99999994, and never closes: the
    draw walks the rewritten buffer (Sampler.cs:61) and returns a rank.  The
    device takes the same branch (all n candidates, its global-memory path) and
    returns the same; a draw beyond the stalled sum returns the last rank."""
    n = 10000
    x = np.empty(n, np.float32)
    x[:10] = -0.01 * np.arange(10)
    x[10:] = -12.9 - 1e-5 * np.arange(n - 10)
    o = opts(0.8, 0, 0.99999994)
    want = [ref(x, o, [], r) for r in R_ALL]
    assert want[-2:] == [n - 1, n - 1]            # r = 0.9999999 and 1.0 lie past the stalled sum
    assert [hip.sample(x, o, [], r) for r in R_ALL] == want


@pytest.mark.parametrize("n", [4096, 37])
def test_temperature_only_matches_oracle(hip, n):
    """TopP = 1, TopK off: the fp64-placed draw over the probabilities in index
    order equals the reference's except within float rounding of a boundary."""
    x = logits_for(n, n + 3, 2.0)
    o = opts(0.8, 0, 1.0)
    mismatches = 0
    for r in R_ALL:
        want, got = ref(x, o, [], r), hip.sample(x, o, [], r)
        if got != want:
            mismatches += 1
            assert near_boundary(x, o, [], r, got), (r, want, got)
    assert mismatches <= 1


def test_top_k_limit(hip):
    x = logits_for(32000, 9)
    with pytest.raises(NotImplementedError, match="TopK"):   # LLMDOT_E_UNSUPPORTED
        hip.sample(x, opts(0.8, 5000), [], 0.5)
    assert hip.sample(x, opts(0.8, 32000, 1.0), [], 0.5) == ref(x, opts(0.8, 32000, 1.0), [], 0.5)


@pytest.mark.parametrize("top_k,top_p", [(40, 0.95), (0, 0.9)])
def test_generate_sampled(hip, tiny_image, top_k, top_p):
    """The device loop: every token is the oracle sampler's draw from the logits
    it was sampled from, with the recent-token list (prompt, then the tokens so
    far); and those logits are the oracle model's for the sampled tokens fed
    back, so the loop fed the draw, not the argmax, into the next step."""
    prompt = [int(t) for t in np.random.default_rng(3).integers(0, 32000, 16)]
    n = 24 if top_k else 10   # the oracle's aliased top-p over all 32000 candidates is the slow part
    s = opts(0.8, top_k, top_p, 1.1, 8)
    draws = np.random.default_rng(11).random(n, dtype=np.float32)
    eng = InferenceEngine(LoadedModel.load(tiny_image), hip, kv_fp16=False, context=64)
    toks, logits = eng.generate_all(prompt, GenerationOptions(max_tokens=n, sampling=s), return_logits=True,
                                    draws=draws)
    assert len(toks) == n
    for i in range(n):
        recent = prompt + toks[:i]
        assert toks[i] == ref(logits[i], s, recent, float(draws[i])), i
    m = O.Model(tiny_image, kv_fp16=False, context=64)
    pos = 0
    for t in prompt:
        rl = m.process_token(t, pos)
        pos += 1
    for i in range(n):
        assert float(np.max(np.abs(rl - logits[i]))) <= LOGIT_TOL, i
        rl = m.process_token(toks[i], pos)
        pos += 1
    m.close()
    # greedy options still take the argmax path
    g, _ = eng.generate_all(prompt, GenerationOptions(max_tokens=4, sampling=opts(0.0, top_k, top_p)))
    assert len(g) == 4
    eng.dispose()
