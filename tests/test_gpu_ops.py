"""Op-level parity of the HIP backend against the oracle (IComputeBackend members).

Bars: dequantisation bit-exact; GEMV max|y - y_ref| / max|y_ref| <= 1e-3;
elementwise ops bit-exact where the reference's per-element formula is
reproduced (Add, Mul, Scale, RoPE with the host cos/sin, SiLU's ExpApprox lanes,
RmsNorm's per-element product given the same 1/rms), otherwise the stated
tolerance.  All calls go through the C ABI (libllmdot_hip.so).
"""
import numpy as np
import pytest

from dotllm_amd import F16, F32, Q4_0, Q4_K, Q5_K, Q6_K, Q8_0, BF16, byte_count, synth
from dotllm_amd._lib import Q2_K, Q3_K, Q4_1, Q5_0, Q5_1
from oracle import oracle as O

pytestmark = pytest.mark.gpu

GEMV_TOL = 1e-3


def rel_err(y, ref):
    return float(np.max(np.abs(y.astype(np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


def weights(t, rows, cols, seed):
    w = np.random.default_rng(seed).normal(0, 0.02, size=(rows, cols)).astype(np.float32)
    return synth.quantize(t, w)


def random_blocks(t, rows, cols, seed):
    """Random block bytes with finite fp16 scale fields (exercises every bit pattern of q/scales)."""
    rng = np.random.default_rng(seed)
    b = rng.integers(0, 256, size=rows * byte_count(t, cols), dtype=np.uint8)
    be, bb = {Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210), Q8_0: (32, 34), Q4_0: (32, 18),
              Q2_K: (256, 84), Q3_K: (256, 110), Q4_1: (32, 20), Q5_0: (32, 22), Q5_1: (32, 24)}[t]
    blocks = b.reshape(-1, bb)
    halves = rng.uniform(-2, 2, size=(blocks.shape[0], 2)).astype(np.float16).view(np.uint8)
    if t in (Q4_K, Q5_K, Q2_K, Q3_K, Q4_1, Q5_1):
        blocks[:, 0:4] = halves.reshape(-1, 4)
    elif t == Q6_K:
        blocks[:, 208:210] = halves[:, :2]
    else:
        blocks[:, 0:2] = halves[:, :2]
    return b


@pytest.mark.parametrize("t", [Q4_K, Q5_K, Q6_K, Q8_0, Q4_0])
@pytest.mark.parametrize("kind", ["quantized", "random"])
def test_dequantize_bit_exact(hip, t, kind):
    rows, cols = 7, 1024
    src = weights(t, rows, cols, 11) if kind == "quantized" else random_blocks(t, rows, cols, 12)
    ref = O.dequantize(src, t, rows, cols)
    out = np.zeros(rows * cols, dtype=np.float32)
    hip.dequantize_to_float(src, out, t, rows, cols)
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("t", [Q2_K, Q3_K])
@pytest.mark.parametrize("rows,cols", [(1, 256), (7, 1024), (33, 4096)])
def test_dequantize_lowbit_kquants_bit_exact(hip, t, rows, cols):
    """Reference-layout Q2_K / Q3_K (DequantizeK.cs:8-74) over random blocks:
    every element bit for bit, including Q3_K's last 8 values of each block,
    which the reference reads from the next block's first two bytes (zeros
    after the tensor's last block)."""
    src = random_blocks(t, rows, cols, 40 + rows)
    ref = O.dequantize(src, t, rows, cols)
    out = np.zeros(rows * cols, dtype=np.float32)
    hip.dequantize_to_float(src, out, t, rows, cols)
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("t", [Q4_1, Q5_0, Q5_1])
@pytest.mark.parametrize("rows,cols", [(1, 32), (7, 1024), (33, 4128)])
def test_dequantize_generic_types_bit_exact(hip, t, rows, cols):
    """Q4_1, Q5_0, Q5_1 (TensorOps.DequantizeGeneric, TO:580-652) over random
    blocks with finite scales, every element bit for bit; 4128 columns give
    rows of an odd number of 22-byte blocks (2-byte aligned rows)."""
    src = random_blocks(t, rows, cols, 60 + rows)
    ref = O.dequantize(src, t, rows, cols)
    out = np.zeros(rows * cols, dtype=np.float32)
    hip.dequantize_to_float(src, out, t, rows, cols)
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("t", [Q4_1, Q5_0, Q5_1])
@pytest.mark.parametrize("rows,cols", [(300, 2048), (257, 4128), (1024, 4096)])
def test_generic_type_gemv(hip, t, rows, cols):
    """MatMul of Q4_1 / Q5_0 / Q5_1 weights (the reference dequantises the row
    and takes the 8-lane dot product, TO:92-111, 510-531) within 1e-3 of the
    oracle's MatMul and of the fp64 product of the dequantised rows."""
    w = random_blocks(t, rows, cols, rows + 11)
    x = np.random.default_rng(cols + 1).normal(0, 1, size=cols).astype(np.float32)
    ref = O.matmul(x, w, t, cols, rows)
    exact = O.dequantize(w, t, rows, cols).reshape(rows, cols).astype(np.float64) @ x.astype(np.float64)
    y = np.zeros(rows, dtype=np.float32)
    hip.mat_mul(x, w, y, t, cols, rows)
    assert rel_err(y, ref) <= GEMV_TOL and rel_err(y, exact) <= GEMV_TOL


@pytest.mark.parametrize("t", [F16, BF16, F32])
def test_dequantize_float_types_bit_exact(hip, t):
    rng = np.random.default_rng(5)
    x = rng.normal(0, 3, size=4096).astype(np.float32)
    src = x.view(np.uint8) if t == F32 else synth.quantize(t, x)
    ref = O.dequantize(src, t, 1, 4096)
    out = np.zeros(4096, dtype=np.float32)
    hip.dequantize_to_float(src, out, t, 1, 4096)
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))


def test_dequantize_half_all_patterns(hip):
    """Every binary16 bit pattern except NaNs, through DequantizeToFloat(F16)."""
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    keep = ((h & 0x7C00) != 0x7C00) | ((h & 0x3FF) == 0)
    h = h[keep]
    src = h.view(np.uint8)
    ref = O.dequantize(src, F16, 1, h.size)
    out = np.zeros(h.size, dtype=np.float32)
    hip.dequantize_to_float(src, out, F16, 1, h.size)
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))
    assert np.array_equal(ref, h.view(np.float16).astype(np.float32))


@pytest.mark.parametrize("t,rows,cols", [(Q4_K, 512, 4096), (Q5_K, 256, 2048), (Q6_K, 300, 3072),
                                         (Q8_0, 257, 1408), (Q4_0, 96, 512), (F32, 64, 256), (F16, 48, 512)])
def test_gemv_matches_reference(hip, t, rows, cols):
    rng = np.random.default_rng(rows + cols)
    if t in (F32, F16):
        w32 = rng.normal(0, 0.02, size=(rows, cols)).astype(np.float32)
        w = w32.view(np.uint8).reshape(-1) if t == F32 else synth.quantize(F16, w32)
    else:
        w = weights(t, rows, cols, 3)
    x = rng.normal(0, 1, size=cols).astype(np.float32)
    ref = (O.matmul_f32(x, w.view(np.float32), cols, rows) if t == F32 else O.matmul(x, w, t, cols, rows))
    y = np.zeros(rows, dtype=np.float32)
    hip.mat_mul(x, w, y, t, cols, rows)
    assert rel_err(y, ref) <= GEMV_TOL


@pytest.mark.parametrize("t,rows,cols", [(Q2_K, 300, 2048), (Q2_K, 4096, 4096), (Q3_K, 257, 4096),
                                         (Q3_K, 1024, 14336), (Q3_K, 3, 256)])
def test_lowbit_kquant_gemv(hip, t, rows, cols):
    """Q2_K / Q3_K GEMV (TensorOps.cs:293-362) on random blocks within 1e-3 of
    the oracle's MatMul, and of the fp64 product of the oracle's dequantised
    rows; with a resident weight key as well as host bytes."""
    w = random_blocks(t, rows, cols, rows + 7)
    blocks = w.reshape(-1, 84 if t == Q2_K else 110)
    blocks[:, 0:4] = np.random.default_rng(rows).uniform(-0.05, 0.05, size=(blocks.shape[0], 2)).astype(
        np.float16).view(np.uint8)
    x = np.random.default_rng(cols).normal(0, 1, size=cols).astype(np.float32)
    ref = O.matmul(x, w, t, cols, rows)
    wd = O.dequantize(w, t, rows, cols).reshape(rows, cols).astype(np.float64)
    exact = wd @ x.astype(np.float64)
    y = np.zeros(rows, dtype=np.float32)
    hip.mat_mul(x, w, y, t, cols, rows)
    assert rel_err(y, ref) <= GEMV_TOL and rel_err(y, exact) <= GEMV_TOL
    key = f"lowbit.{t}.{rows}.{cols}"
    y2 = np.zeros(rows, dtype=np.float32)
    hip.mat_mul(x, w, y2, t, cols, rows, weight_key=key)
    hip.release_weight(key)
    assert np.array_equal(y, y2)


@pytest.mark.parametrize("rows,cols", [(4096, 4096), (14336, 4096), (4096, 14336)])
def test_q4k_gemv_full_shapes(hip, rows, cols):
    """The isolated Q4_K GEMV workload at its three shapes: weights N(0, 0.02)
    quantized to the reference's Q4_K layout, x ~ N(0, 1).  The GEMV within
    1e-3 of the reference MatMul (TO:364-395), and the whole matrix's
    dequantisation bit-exact (DK:76-106)."""
    w = np.zeros(rows * byte_count(Q4_K, cols), dtype=np.uint8)
    synth.synth_tensor(Q4_K, rows, cols, 0xC2 + rows + cols, w)
    x = np.random.default_rng(rows ^ cols).normal(0, 1, size=cols).astype(np.float32)
    O.set_threads(16)
    try:
        ref = O.matmul(x, w, Q4_K, cols, rows)
        deq = O.dequantize(w, Q4_K, rows, cols)
    finally:
        O.set_threads(1)
    y = np.zeros(rows, dtype=np.float32)
    hip.mat_mul(x, w, y, Q4_K, cols, rows)
    err = rel_err(y, ref)
    out = np.zeros(rows * cols, dtype=np.float32)
    hip.dequantize_to_float(w, out, Q4_K, rows, cols)
    print(f"Q4_K {rows} x {cols}: GEMV relative error {err:.2e}")
    assert err <= GEMV_TOL
    assert np.array_equal(out.view(np.uint32), deq.view(np.uint32))


def test_gemv_resident_weight_key(hip):
    rows, cols = 128, 512
    w = weights(Q4_K, rows, cols, 9)
    x = np.random.default_rng(1).normal(0, 1, size=cols).astype(np.float32)
    y1 = np.zeros(rows, dtype=np.float32)
    hip.mat_mul(x, w, y1, Q4_K, cols, rows, weight_key="blk.0.test.weight")
    assert hip.has_weight("blk.0.test.weight")
    y2 = np.zeros(rows, dtype=np.float32)
    hip.mat_mul(x, None, y2, Q4_K, cols, rows, weight_key="blk.0.test.weight")
    assert np.array_equal(y1, y2)
    hip.release_weight("blk.0.test.weight")
    with pytest.raises(KeyError):
        hip.mat_mul(x, None, y2, Q4_K, cols, rows, weight_key="blk.0.test.weight")


def test_gemv_batched_rows(hip):
    """aRows > 1 (TO:92-111): every row of a against the same weights."""
    rows, cols, a_rows = 64, 512, 3
    w = weights(Q8_0, rows, cols, 4)
    a = np.random.default_rng(2).normal(0, 1, size=a_rows * cols).astype(np.float32)
    ref = O.matmul(a, w, Q8_0, cols, rows, result_len=a_rows * rows)
    y = np.zeros(a_rows * rows, dtype=np.float32)
    hip.mat_mul(a, w, y, Q8_0, cols, rows)
    assert rel_err(y, ref) <= GEMV_TOL


def test_matmul_f32_known_answer(hip):
    """TensorOpsTests.MatMulF32_2x3Times3x2: [50, 68, 122, 167]."""
    a = np.array([1, 2, 3, 4, 5, 6], dtype=np.float32)
    b = np.array([7, 8, 9, 10, 11, 12], dtype=np.float32)
    r = np.zeros(4, dtype=np.float32)
    hip.mat_mul_f32(a, b, r, 3, 2)
    assert np.allclose(r, [50, 68, 122, 167], atol=1e-3)


def test_rms_norm(hip):
    x = np.random.default_rng(3).normal(0, 2, size=4096).astype(np.float32)
    w = np.random.default_rng(4).normal(1, 0.1, size=4096).astype(np.float32)
    ref = O.rms_norm(x, w, 1e-5)
    out = np.zeros_like(x)
    hip.rms_norm(x, w, out, 1e-5)
    assert np.max(np.abs(out - ref) / np.maximum(np.abs(ref), 1e-6)) <= 4e-7 * 8


def test_rms_norm_known_answer(hip):
    out = np.zeros(2, dtype=np.float32)
    hip.rms_norm(np.array([3, 4], dtype=np.float32), np.ones(2, dtype=np.float32), out, 1e-5)
    mag = np.sqrt((9 + 16) / 2 + 1e-5)
    assert np.allclose(out, [3 / mag, 4 / mag], atol=1e-3)


@pytest.mark.parametrize("pos", [0, 1, 17, 4095])
def test_rope_bit_exact(hip, pos):
    hd = 128
    freq = (1.0 / np.power(np.float32(10000.0), np.arange(64, dtype=np.float32) * 2 / hd)).astype(np.float32)
    rng = np.random.default_rng(pos)
    q = rng.normal(size=hd).astype(np.float32)
    k = rng.normal(size=hd).astype(np.float32)
    rq, rk = O.rope_table(q, k, hd, pos, freq)
    q2, k2 = q.copy(), k.copy()
    hip.apply_rope(q2, k2, hd, pos, freq)
    assert np.array_equal(q2, rq) and np.array_equal(k2, rk)
    q3 = q.copy()
    hip.apply_rope(q3, q3, hd, pos, freq)           # same span: rotated once
    assert np.array_equal(q3, rq)


def test_rope_base_overload(hip):
    q = np.ones(128, dtype=np.float32)
    k = np.ones(128, dtype=np.float32)
    hip.apply_rope(q, k, 128, 1, freq_base=10000.0, rotary_dim=128)
    rq, rk = O.rope_base(np.ones(128, np.float32), np.ones(128, np.float32), 128, 1, 10000.0, 128)
    assert np.array_equal(q, rq) and np.array_equal(k, rk)
    assert q[64] != 1.0


@pytest.mark.parametrize("n", [1, 5, 8, 13, 64, 1000, 4097])
def test_softmax(hip, n):
    x = np.random.default_rng(n).normal(0, 3, size=n).astype(np.float32)
    ref = O.softmax(x)
    y = x.copy()
    hip.softmax(y)
    assert np.max(np.abs(y - ref)) <= 1e-6
    assert abs(float(y.sum()) - 1.0) < 1e-3


def test_softmax_softcap(hip):
    x = np.array([10, 20, 30, 40, 1, 2, 3, 4, 5], dtype=np.float32)
    ref = O.softmax(x, softcap=5.0)
    y = x.copy()
    hip.softmax(y, softcap=5.0)
    assert np.max(np.abs(y - ref)) <= 1e-6


@pytest.mark.parametrize("n", [8, 13, 14336])
def test_silu(hip, n):
    x = np.random.default_rng(n).normal(0, 4, size=n).astype(np.float32)
    ref = O.silu(x)
    y = np.zeros_like(x)
    hip.silu(x, y)
    n8 = n & ~7
    assert np.array_equal(y[:n8], ref[:n8])                 # ExpApprox lanes: bit-exact
    assert np.allclose(y[n8:], ref[n8:], rtol=2e-6, atol=1e-7)
    z = x.copy()
    hip.silu_in_place(z)
    assert np.array_equal(z, y)


def test_elementwise_bit_exact(hip):
    rng = np.random.default_rng(0)
    a = rng.normal(size=1001).astype(np.float32)
    b = rng.normal(size=1001).astype(np.float32)
    out = np.zeros_like(a)
    hip.add(a, b, out)
    assert np.array_equal(out, O.add(a, b))
    hip.mul(a, b, out)
    assert np.array_equal(out, O.mul(a, b))
    hip.scale(a, 0.37, out)
    assert np.array_equal(out, O.scale(a, 0.37))
    c = a.copy()
    hip.add(c, b)
    assert np.array_equal(c, O.add(a, b))


@pytest.mark.parametrize("n", [4, 100, 32000, 128256])
def test_argmax(hip, n):
    x = np.random.default_rng(n).normal(size=n).astype(np.float32)
    assert hip.arg_max(x) == O.argmax(x) == int(np.argmax(x))


def test_argmax_ties_first_index(hip):
    x = np.zeros(50000, dtype=np.float32)
    x[[7, 20000, 45000]] = 5.0
    assert hip.arg_max(x) == 7 == O.argmax(x)
    assert hip.arg_max(np.array([1, 5, 3, 2], dtype=np.float32)) == 1   # VectorMathTests.ArgMax_ReturnsIndex


def test_unsupported_type_raises(hip):
    with pytest.raises(NotImplementedError):
        hip.mat_mul(np.zeros(256, np.float32), np.zeros(40 * 8, np.uint8), np.zeros(1, np.float32), 9, 256, 1)   # Q8_1
