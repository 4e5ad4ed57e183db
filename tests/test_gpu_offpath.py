"""The IComputeBackend members of other model templates on the device:
LayerNorm (ICB:12), Gelu / GeluScalar (ICB:18-19), Softcap (ICB:25) and
Conv1D (ICB:26), against the oracle (tests/test_oracle_offpath.py pins it).

Bars: the vector lanes (TanhApproxVector, plain arithmetic) and Conv1D are
bit-exact; tail elements go through the device tanhf instead of the host libm
(within 4 ulp); LayerNorm's mean and variance are block sums in another order
than the reference's 8-lane sums (within 2e-6 relative)."""
import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _ulps(a, b):
    a = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    return np.abs(a - b)


@pytest.mark.parametrize("n", [1, 3, 8, 13, 4096, 4099])
@pytest.mark.parametrize("bias", [False, True])
def test_layer_norm(hip, n, bias):
    rng = np.random.default_rng(n + 7 * bias)
    x = (rng.normal(0, 2, n) + 3).astype(np.float32)
    w = rng.normal(1, 0.2, n).astype(np.float32)
    b = rng.normal(0, 1, n).astype(np.float32) if bias else None
    out = np.zeros(n, np.float32)
    hip.layer_norm(x, w, b, out, 1e-5)
    ref = O.layer_norm(x, w, b, 1e-5)
    assert np.max(np.abs(out - ref)) <= 2e-6 * max(1.0, float(np.max(np.abs(ref))))


def test_layer_norm_empty_bias_and_constant_row(hip):
    """An empty bias span is no bias; a constant row gives exactly the bias."""
    x = np.full(40, 1.5, np.float32)
    b = np.arange(40, dtype=np.float32)
    out = np.zeros(40, np.float32)
    hip.layer_norm(x, np.ones(40, np.float32), b, out, 1e-5)
    assert np.array_equal(out, b)
    y = np.random.default_rng(1).normal(size=40).astype(np.float32)
    o1, o2 = np.zeros(40, np.float32), np.zeros(40, np.float32)
    hip.layer_norm(y, np.ones(40, np.float32), np.zeros(0, np.float32), o1, 1e-5)
    hip.layer_norm(y, np.ones(40, np.float32), None, o2, 1e-5)
    assert np.array_equal(o1, o2)


@pytest.mark.parametrize("n", [1, 4, 8, 13, 1000, 14339])
def test_gelu(hip, n):
    x = np.random.default_rng(n).normal(0, 3, n).astype(np.float32)
    out = np.zeros(n, np.float32)
    hip.gelu(x, out)
    ref = O.gelu(x)
    n8 = n & ~7
    assert np.array_equal(out[:n8], ref[:n8])
    assert np.all(_ulps(out[n8:], ref[n8:]) <= 4)


def test_gelu_scalar(hip):
    for v in (-3.5, -1.0, -0.25, 0.0, 0.5, 1.0, 2.0, 6.0):
        got, want = hip.gelu_scalar(v), O.gelu_scalar(v)
        assert _ulps(got, want) <= 4, v
    assert hip.gelu_scalar(0.0) == 0.0


@pytest.mark.parametrize("n,cap", [(4, 3.0), (13, 30.0), (4099, 50.0)])
def test_softcap(hip, n, cap):
    x = np.random.default_rng(n).normal(0, 2 * cap, n).astype(np.float32)
    y = x.copy()
    hip.softcap(y, cap)
    ref = O.softcap(x, cap)
    n8 = n & ~7
    assert np.array_equal(y[:n8], ref[:n8])
    assert np.all(_ulps(y[n8:], ref[n8:]) <= 4)


@pytest.mark.parametrize("ks,dim", [(1, 5), (1, 4099), (2, 2), (3, 1), (4, 1024), (8, 77), (13, 300), (32, 2048)])
def test_conv1d_bit_exact(hip, ks, dim):
    rng = np.random.default_rng(ks * 1000 + dim)
    x = rng.normal(0, 1, ks * dim).astype(np.float32)
    w = rng.normal(0, 1, ks * dim).astype(np.float32)
    out = np.zeros(dim, np.float32)
    hip.conv1d(x, w, out, ks, dim)
    assert np.array_equal(out, O.conv1d(x, w, ks, dim))


def test_conv1d_reference_cases(hip):
    """ConvLayerTests.cs:67-115 through the device."""
    out = np.zeros(2, np.float32)
    hip.conv1d(np.array([1, 2, 3, 4], np.float32), np.array([1, 0.5, 0.5, 1], np.float32), out, 2, 2)
    assert np.allclose(out, [2.0, 5.5], atol=1e-4)
    out1 = np.zeros(1, np.float32)
    hip.conv1d(np.array([1, 2, 3], np.float32), np.full(3, 1 / 3, np.float32), out1, 3, 1)
    assert abs(out1[0] - 2.0) <= 1e-2
    with pytest.raises(IndexError):
        hip.conv1d(np.zeros(3, np.float32), np.zeros(4, np.float32), out, 2, 2)
