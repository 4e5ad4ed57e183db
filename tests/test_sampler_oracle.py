"""The oracle's Sampler.Sample (Sampler.cs:24-170) against the reference's
sampler tests (tests/Llmdot.Core.Tests/Sampling/SamplerTests.cs) and against
closed forms.  The reference's tests fix the draw through Random(seed); here the
draw r is an input, so each property is checked for every r of a grid."""
import numpy as np
import pytest

from oracle import oracle as O

R_GRID = [0.0, 1e-7, 0.001, 0.1, 0.25, 0.3333, 0.5, 0.6667, 0.75, 0.9, 0.999, 0.9999999, 1.0]


def sample(logits, temperature=1.0, top_k=0, top_p=1.0, penalty=1.0, window=0, recent=(), r=0.5):
    return O.sample(np.asarray(logits, np.float32), temperature, top_k, top_p, penalty, window, list(recent), r)


def make_logits(size, peak, value=10.0):   # SamplerTests.MakeLogits
    x = np.full(size, 0.01, np.float32)
    x[peak] = value
    return x


def test_temperature_zero_returns_argmax():
    assert sample(make_logits(100, 42), temperature=0.0) == 42
    assert sample(make_logits(100, 7, 20.0), temperature=0.0, top_k=5, top_p=0.5, penalty=2.0, window=64, recent=[7]) == 7
    x = np.zeros(100, np.float32)
    x[10], x[20], x[30] = 5, 10, 7
    assert sample(x, temperature=0.0) == 20


@pytest.mark.parametrize("r", R_GRID)
def test_top_k_limits_to_k_tokens(r):
    x = np.full(100, 0.001, np.float32)
    x[0], x[1], x[2] = 100, 90, 80
    assert 0 <= sample(x, top_k=3, r=r) <= 2
    x = np.zeros(100, np.float32)
    x[42] = 10
    assert sample(x, top_k=1, r=r) == 42   # TopK_One_ReturnsArgMaxWithTemperature


@pytest.mark.parametrize("r", R_GRID)
def test_top_p(r):
    x = np.full(100, 0.001, np.float32)
    x[0], x[1], x[2] = 10, 5, 3
    assert sample(x, top_k=0, top_p=0.5, r=r) <= 2
    x = np.full(100, 0.01, np.float32)
    x[0] = 100
    assert sample(x, top_k=0, top_p=0.01, r=r) == 0


@pytest.mark.parametrize("r", R_GRID)
def test_repeat_penalty_cases(r):
    x = np.zeros(100, np.float32)
    x[50], x[51] = 100, 50
    assert sample(x, temperature=0.5, top_k=100, penalty=100.0, window=64, recent=[50], r=r) != 50
    x = np.full(100, -1.0, np.float32)
    x[50], x[30] = -0.5, 10
    cdf0 = np.cumsum(_softmax_ref64(x))
    if cdf0[29] < r <= cdf0[30]:   # token 30 holds 99.8% of the mass
        assert sample(x, r=r) == 30
    # with the penalty 30's logit is 0.1: the draw follows the index-order CDF
    y = x.copy()
    y[30] = 0.1
    cdf = np.cumsum(_softmax_ref64(y))
    if np.min(np.abs(cdf - r)) > 1e-4:
        assert sample(x, penalty=100.0, window=64, recent=[30], r=r) == min(int(np.searchsorted(cdf, r)), 99)
    x = np.zeros(100, np.float32)
    x[42] = 10
    if 1e-6 <= r <= 0.999999:   # token 42 holds all but ~1e-7 of the mass
        for kw in (dict(penalty=100.0, window=0, recent=[42]), dict(penalty=1.0, window=64, recent=[42]),
                   dict(penalty=100.0, window=64, recent=[])):
            assert sample(x, temperature=0.5, **kw, r=r) == 42


def test_repeat_penalty_semantics_by_argmax():
    """top_k = 1 returns the argmax of the penalised, scaled logits: division
    for positive values, multiplication otherwise, once per occurrence, only
    the last `window` entries."""
    x = np.zeros(16, np.float32)
    x[5], x[6], x[7] = 3.0, 2.0, -0.1
    assert sample(x, top_k=1, penalty=2.0, window=8, recent=[]) == 5
    assert sample(x, top_k=1, penalty=2.0, window=8, recent=[5]) == 6        # 1.5 < 2
    y = x.copy()
    y[6] = 1.0
    assert sample(y, top_k=1, penalty=2.0, window=8, recent=[5]) == 5        # 1.5 > 1
    assert sample(y, top_k=1, penalty=2.0, window=8, recent=[5, 5]) == 6     # 0.75 < 1
    assert sample(y, top_k=1, penalty=2.0, window=1, recent=[5, 9]) == 5     # 5 outside the window
    z = np.full(16, -1.0, np.float32)
    z[3] = -0.5
    assert sample(z, top_k=1, penalty=3.0, window=4, recent=[3]) != 3        # -1.5 < -1
    assert sample(z, top_k=1, penalty=3.0, window=4, recent=[3, 99, -4]) != 3   # ids out of range are skipped


def _softmax_ref64(v):
    """VectorMath.Softmax's terms (ExpApprox on the first 8 floor(n/8) values,
    exp on the tail, arguments rounded to float), normalised in fp64."""
    v = np.asarray(v, np.float32)
    d = (v - np.float32(np.max(v))).astype(np.float32)
    n8 = v.size & ~7
    e = np.array([O.exp_approx(float(t)) if i < n8 else np.exp(np.float64(t)) for i, t in enumerate(d)])
    return e / e.sum()


@pytest.mark.parametrize("seed", range(4))
def test_top_k_draw_is_the_inverse_cdf(seed):
    """The chosen token is where the cumulative distribution of the k largest
    (descending, ExpApprox terms as the reference's Softmax has them) first
    reaches r; away from boundaries the fp64 closed form decides."""
    rng = np.random.default_rng(seed)
    x = rng.normal(0, 2, 500).astype(np.float32)
    k, T = 25, 0.9
    scaled = x * np.float32(np.float32(1.0) / np.float32(T))
    order = np.argsort(-scaled, kind="stable")[:k]
    cdf = np.cumsum(_softmax_ref64(scaled[order]))
    for r in np.linspace(0.0005, 0.9995, 37):
        j = int(np.searchsorted(cdf, r))
        if np.min(np.abs(cdf - r)) < 5e-3:
            continue
        assert sample(x, temperature=T, top_k=k, r=r) == order[j]


@pytest.mark.parametrize("seed", range(3))
def test_nucleus_size_and_draw_closed_form(seed):
    """The nucleus of the true probabilities (FindNucleus with a buffer of its
    own): its size and the renormalised draw inside it follow the fp64
    cumulative distribution in descending order.  (With the reference's
    aliasing, random logits over 300 ids reach back into rewritten slots;
    the tests below pin that form.)"""
    rng = np.random.default_rng(100 + seed)
    n = 300
    x = rng.normal(0, 1.5, n).astype(np.float32)
    p = _softmax_ref64(x)
    order = np.argsort(-p, kind="stable")
    cdf = np.cumsum(p[order])
    for top_p in (0.3, 0.6, 0.9):
        m = int(np.searchsorted(cdf, top_p)) + 1
        if np.min(np.abs(cdf - top_p)) < 5e-3:
            continue
        S = cdf[m - 1]
        for r in np.linspace(0.01, 0.99, 25):
            j = int(np.searchsorted(cdf[:m] / S, r))
            if np.min(np.abs(cdf[:m] / S - r)) < 5e-3:
                continue
            tok = O.sample(x, 1.0, 0, top_p, 1.0, 0, [], r, aliased=False)
            assert tok == order[j], (top_p, r)


def test_full_distribution_draw_walks_index_order():
    """TopP >= 1 (and no top-k): r is placed on the cumulative sum in index order."""
    x = np.log(np.array([0.1, 0.2, 0.3, 0.4], np.float32))   # 4 < 8: expf terms only
    for r, want in ((0.05, 0), (0.15, 1), (0.35, 2), (0.65, 3), (0.95, 3)):
        assert sample(x, top_k=0, top_p=1.0, r=r) == want


def _nucleus_sorted(p):
    """FindNucleus's selection sort (Sampler.cs:133-144) of the indices."""
    idx = list(range(len(p)))
    for i in range(len(p) - 1):
        m = i
        for j in range(i + 1, len(p)):
            if p[idx[j]] > p[idx[m]]:
                m = j
        idx[i], idx[m] = idx[m], idx[i]
    return idx


def test_top_p_buffer_aliasing_constructed():
    """The reference hands FindNucleus the buffer that holds the probabilities
    as its output (Sampler.cs:30, 48-50).  Probabilities 0.1, 0.2, 0.4, 0.3 at
    TopP 0.95: sorted ranks are ids 2, 3, 1, 0; writing rank 1 (0.3) into slot 1
    overwrites id 1's 0.2, so rank 2 reads 0.3, the sum reaches 1.0 >= 0.95 and
    the nucleus closes at 3 tokens with weights 0.4, 0.3, 0.3.  With a buffer of
    its own the sum is 0.9 after 3, the nucleus is all 4 tokens, and the draw
    walks the probabilities in token order."""
    x = np.log(np.array([0.1, 0.2, 0.4, 0.3], np.float32))   # n < 8: exp terms only
    assert _nucleus_sorted(_softmax_ref64(x)) == [2, 3, 1, 0]
    # aliased: draw over (id 2: 0.4, id 3: 0.3, id 1: 0.3)
    for r, want in ((0.05, 2), (0.39, 2), (0.45, 3), (0.69, 3), (0.75, 1), (0.99, 1)):
        assert sample(x, top_p=0.95, r=r) == want, r
    # own buffer: the full distribution in index order (0.1, 0.2, 0.4, 0.3)
    for r, want in ((0.05, 0), (0.15, 1), (0.45, 2), (0.75, 3), (0.99, 3)):
        assert O.sample(x, 1.0, 0, 0.95, 1.0, 0, [], r, aliased=False) == want, r
    # the two differ at r = 0.05, 0.15, 0.45, 0.75
    assert sum(sample(x, top_p=0.95, r=r) != O.sample(x, 1.0, 0, 0.95, 1.0, 0, [], r, aliased=False)
               for r in (0.05, 0.15, 0.45, 0.75)) == 4


def test_top_p_aliasing_fall_through_returns_a_rank():
    """When the (rewritten) running sum reaches TopP only at the last rank, the
    nucleus is all n tokens and the reference draws from `scaled` (Sampler.cs:61),
    which now holds the sorted probabilities: the result is a rank, not a token
    id.  Probabilities 0.1, 0.3, 0.6 at TopP 0.999: ranks are ids 2, 1, 0, no
    slot is read after it is written except rank 2 (id 0) reading slot 0 (now
    0.6), so the buffer becomes 0.6, 0.3, 0.6 (sum 1.5) and r = 0.5 returns 0
    (rank 0, which is id 2)."""
    x = np.log(np.array([0.1, 0.3, 0.6], np.float32))
    assert _nucleus_sorted(_softmax_ref64(x)) == [2, 1, 0]
    assert sample(x, top_p=0.999, r=0.5) == 0
    assert sample(x, top_p=0.999, r=0.7) == 1
    assert sample(x, top_p=0.999, r=1.0) == 2
    # own buffer: r walks 0.1, 0.3, 0.6 in token order
    assert O.sample(x, 1.0, 0, 0.999, 1.0, 0, [], 0.3, aliased=False) == 1
    assert O.sample(x, 1.0, 0, 0.999, 1.0, 0, [], 0.5, aliased=False) == 2


@pytest.mark.parametrize("seed", range(6))
def test_top_p_aliasing_is_harmless_without_a_back_reference(seed):
    """The two forms agree whenever no rank inside the nucleus has a token id
    below its rank (indices[i] >= i for every i < nucleus size) and the nucleus
    is proper: then every value is read before its slot is written.  Random
    logits with the peak mass on high ids, checked over an r grid."""
    rng = np.random.default_rng(seed)
    n = 200
    x = rng.normal(0, 1.0, n).astype(np.float32)
    x[100:110] += 6.0     # the nucleus sits on ids 100..109
    p = _softmax_ref64(x)
    idx = _nucleus_sorted(p)
    for top_p in (0.5, 0.8, 0.9):
        m = int(np.searchsorted(np.cumsum(p[idx]), top_p)) + 1
        assert m < n and all(idx[i] >= i for i in range(m))
        for r in R_GRID:
            assert sample(x, top_p=top_p, r=r) == O.sample(x, 1.0, 0, top_p, 1.0, 0, [], r, aliased=False)
