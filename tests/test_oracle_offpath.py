"""Pins of the oracle's off-path IComputeBackend members: LayerNorm (ICB:12),
Gelu / GeluScalar (ICB:18-19), Softcap (ICB:25) and Conv1D (ICB:26).

Each is checked against the reference's own tests (VectorMathTests.cs:20-33,
VectorMathExtendedTests.cs:20-93, ConvLayerTests.cs:66-115) and against what
the mathematics fixes independently of the oracle's code: fp64 closed forms,
the known error of TanhApproxVector's Pade form against tanh, its clamp to
exactly +-1, exact sums of small integers, and mean/scale invariances.
"""
import math

import numpy as np
import pytest

from oracle import oracle as O

VEC = 8


def _tail(n):
    return range(n - n % VEC, n)


def _gelu64(x):
    x = np.asarray(x, dtype=np.float64)
    return 0.5 * x * (1.0 + np.tanh(math.sqrt(2.0 / math.pi) * (x + 0.044715 * x ** 3)))


# ---- reference tests -----------------------------------------------------------

def test_layer_norm_zero_bias_output_is_normalized():
    """VectorMathTests.cs:20-33."""
    out = O.layer_norm(np.array([1, 2, 3], np.float32), np.ones(3, np.float32), np.zeros(3, np.float32), 1e-5)
    assert -0.01 <= float(np.mean(out)) <= 0.01


def test_gelu_vector_matches_scalar_gelu():
    """VectorMathExtendedTests.cs:21-32 (4 elements: all on the scalar tail)."""
    x = np.array([-1, 0, 0.5, 1], np.float32)
    got = O.gelu(x)
    for i in range(4):
        assert abs(got[i] - O.gelu_scalar(x[i])) <= 0.05


def test_gelu_scalar_signs():
    """VectorMathExtendedTests.cs:34-56."""
    assert abs(O.gelu_scalar(0.0)) <= 1e-4
    assert 0.0 < O.gelu_scalar(1.0) < 1.0
    assert -1.0 < O.gelu_scalar(-1.0) < 0.0


def test_softcap_matches_cap_times_tanh():
    """VectorMathExtendedTests.cs:81-93."""
    vals = [-2.0, 0.0, 1.0, 2.0]
    got = O.softcap(vals, 3.0)
    for v, g in zip(vals, got):
        assert abs(g - 3.0 * math.tanh(v / 3.0)) <= 0.05


def test_conv1d_reference_cases():
    """ConvLayerTests.cs:67-115: identity (kernel 1), averaging, two channels."""
    assert np.allclose(O.conv1d([3, 5], [1, 1], 1, 2), [3, 5], atol=1e-4)
    assert abs(O.conv1d([1, 2, 3], [1 / 3] * 3, 3, 1)[0] - 2.0) <= 1e-2
    assert np.allclose(O.conv1d([1, 2, 3, 4], [1, 0.5, 0.5, 1], 2, 2), [2.0, 5.5], atol=1e-4)


# ---- closed forms and invariants -----------------------------------------------------

@pytest.mark.parametrize("n", [1, 7, 8, 13, 1000, 4099])
@pytest.mark.parametrize("bias", [False, True])
def test_layer_norm_closed_form(n, bias):
    """(x - mean) / sqrt(var + eps) * w + b in fp64 with the population
    variance (a divisor n - 1, a dropped mean or a missing bias fail)."""
    rng = np.random.default_rng(n)
    x = (rng.normal(0, 3, n) + 5).astype(np.float32)
    w = rng.normal(1, 0.3, n).astype(np.float32)
    b = rng.normal(0, 1, n).astype(np.float32) if bias else None
    eps = 1e-5
    got = O.layer_norm(x, w, b, eps).astype(np.float64)
    x64 = x.astype(np.float64)
    mean = x64.mean()
    var = ((x64 - mean) ** 2).mean()
    want = w * (x64 - mean) / math.sqrt(var + eps) + (b if bias else 0.0)
    assert np.max(np.abs(got - want)) <= 2e-5 * max(1.0, float(np.max(np.abs(want))))


def test_layer_norm_shift_and_scale_invariance():
    """LayerNorm(a x + c) = LayerNorm(x) for a > 0 (eps negligible)."""
    rng = np.random.default_rng(3)
    x = rng.normal(0, 1, 777).astype(np.float32)
    w = np.ones(777, np.float32)
    base = O.layer_norm(x, w, None, 1e-12)
    moved = O.layer_norm((4 * x + 10).astype(np.float32), w, None, 1e-12)
    assert np.max(np.abs(base - moved)) <= 1e-4


def test_layer_norm_constant_row():
    """A constant row has zero variance: the output is the bias (x - mean = 0 exactly)."""
    x = np.full(24, 2.5, np.float32)
    b = np.arange(24, dtype=np.float32)
    assert np.array_equal(O.layer_norm(x, np.ones(24, np.float32), b, 1e-5), b)


def test_gelu_tail_is_the_tanh_formula():
    """Tail elements (past the last full 8-lane block) follow 0.5 x (1 +
    tanh(sqrt(2/pi)(x + 0.044715 x^3))) to fp32 rounding."""
    rng = np.random.default_rng(5)
    x = rng.normal(0, 3, 1007).astype(np.float32)
    got = O.gelu(x)
    for i in _tail(x.size):
        want = float(_gelu64(x[i]))
        assert abs(got[i] - want) <= 4e-7 * max(1.0, abs(want))
    for v in (-3.5, -0.25, 0.0, 0.7, 2.0, 6.0):
        assert abs(O.gelu_scalar(v) - float(_gelu64(v))) <= 4e-7 * max(1.0, abs(v))


def test_gelu_vector_lanes():
    """The vector lanes (VM:183-187) take TanhApproxVector (the Pade form and
    its clamp to exactly +-1 past |4|, pinned by the softcap test) of the
    argument as written there, x c (1 + c3 x x x) -- not GELU's c (x + c3 x^3).
    Pinned independently of the oracle's expression:
      * x = 0 gives exactly 0, and x >= 8 exactly x (argument past the clamp);
      * x <= -4 gives exactly x: 1 + c3 x^3 < 0 there, so the argument is
        positive and past the clamp.  GELU's x^2 form, a dropped cubic term or
        a flipped sign all give exactly 0 instead (negative argument);
      * at x = 1 (where x^3 = x^2) the lane is within 0.5 * 0.0236 of GELU(1),
        fixing c and c3 to the Pade bound; the tail test fixes them exactly,
        and the oracle shares the constants between the two forms."""
    x = np.array([0, 1, 8, 10, 20, 50, 1, 0], np.float32)
    g = O.gelu(x)
    assert g[0] == 0.0 and g[7] == 0.0
    assert abs(float(g[1]) - float(_gelu64(1.0))) <= 0.5 * 0.0236
    assert g[1] == g[6]
    assert np.array_equal(g[2:6], x[2:6])
    neg = np.array([-4, -5, -6, -8, -10, -20, -50, -100], np.float32)
    assert np.array_equal(O.gelu(neg), neg)
    # the same values on the scalar tail are GELU's (about 0 for x <= -4)
    tail = O.gelu(neg[:4])
    assert np.all(np.abs(tail) < 1e-3)


def test_softcap_tail_and_lanes():
    """Tail: cap tanh(x / cap) to fp32 rounding; lanes: within cap 0.025 of it
    and exactly +-cap where |x / cap| > 4."""
    rng = np.random.default_rng(7)
    cap = 30.0
    x = rng.normal(0, 60, 1003).astype(np.float32)
    got = O.softcap(x, cap).astype(np.float64)
    want = cap * np.tanh(x.astype(np.float64) / cap)
    for i in _tail(x.size):
        assert abs(got[i] - want[i]) <= 4e-7 * cap
    assert np.all(np.abs(got - want) <= cap * 0.025 + 1e-5)
    lanes = np.arange(x.size) < x.size - x.size % VEC
    clamp = lanes & (np.abs(x / np.float32(cap)) > 4)
    assert np.any(clamp) and np.all(got[clamp] == np.sign(x[clamp]) * cap)


@pytest.mark.parametrize("ks", [1, 2, 3, 8, 13, 32])
def test_conv1d_exact_on_integers(ks):
    """Small integers sum exactly in any order: every channel equals the
    integer dot product (a transposed [ks][dim] layout fails)."""
    dim = 37
    rng = np.random.default_rng(ks)
    x = rng.integers(-8, 9, dim * ks).astype(np.float32)
    w = rng.integers(-8, 9, dim * ks).astype(np.float32)
    want = (x.reshape(dim, ks).astype(np.int64) * w.reshape(dim, ks).astype(np.int64)).sum(axis=1)
    assert np.array_equal(O.conv1d(x, w, ks, dim), want.astype(np.float32))


@pytest.mark.parametrize("ks", [4, 8, 21])
def test_conv1d_random_against_fp64(ks):
    dim = 64
    rng = np.random.default_rng(10 + ks)
    x = rng.normal(0, 1, dim * ks).astype(np.float32)
    w = rng.normal(0, 1, dim * ks).astype(np.float32)
    want = (x.reshape(dim, ks).astype(np.float64) * w.reshape(dim, ks)).sum(axis=1)
    assert np.max(np.abs(O.conv1d(x, w, ks, dim) - want)) <= 1e-5
