"""Pins the oracle (oracle/oracle.c, the CPU restatement of the reference's
managed decode path) before it is trusted as the GPU path's reference.

Sources of truth, in order: the reference's own known-answer tests (cited by
file:line under tests/Llmdot.Core.Tests), blocks built field by field with an
independent bit writer (the expected values come from the fields chosen, with
powers of two so that no evaluation order can change them), fp64 brute force,
and closed-form invariants.  CPU only.
"""
import math

import numpy as np
import pytest

from dotllm_amd import BF16, F16, F32, Q4_0, Q4_K, Q5_K, Q6_K, Q8_0, synth
from oracle import oracle as O


def f32(x):
    return np.float32(x)


def bits(x):
    return int(np.float32(x).view(np.uint32))


# ---------------------------------------------------------------- half / bf16 --

def test_half_known_values():
    """DequantizeTests.cs:64-70."""
    assert O.half_to_float(0x3C00) == 1.0
    assert O.half_to_float(0xBC00) == -1.0
    assert O.half_to_float(0x3800) == 0.5
    assert O.half_to_float(0x0000) == 0.0


def test_half_exhaustive_matches_ieee():
    """HalfHelper.HalfToFloat (HH:7-33) is the IEEE binary16 -> binary32 widening,
    with every NaN mapped to float.NaN (0xFFC00000)."""
    for h in range(1 << 16):
        got = bits(O.half_to_float(h))
        want = np.array([h], dtype=np.uint16).view(np.float16).astype(np.float32)[0]
        if np.isnan(want):
            assert got == 0xFFC00000, hex(h)
        else:
            assert got == bits(want), hex(h)


def test_bf16_known_values():
    """DequantizeTests.cs:72-89 (little-endian bf16 bytes)."""
    for raw, want in ((b"\x80\x3F", 1.0), (b"\x00\x40", 2.0), (b"\x80\xBF", -1.0)):
        assert O.dequantize(np.frombuffer(raw, np.uint8), BF16, 1, 1)[0] == want


def test_f32_identity():
    """DequantizeTests.cs:12-23."""
    v = np.array([1.0, -2.5, 3.14, 0.0], dtype=np.float32)
    assert np.array_equal(O.dequantize(v.view(np.uint8), F32, 1, 4), v)


def test_f16_rows():
    h = np.array([0x3C00, 0xC000, 0x3555, 0x0001], dtype=np.uint16)
    want = h.view(np.float16).astype(np.float32)
    assert np.array_equal(O.dequantize(h.view(np.uint8), F16, 1, 4), want)


# ---------------------------------------------------------------- Q4_0 / Q8_0 --

def test_q4_0_known_answer():
    """DequantizeTests.cs:25-43: d = 1.0, all nibbles 0 -> every value -8."""
    src = np.zeros(36, dtype=np.uint8)
    src[1] = 0x3C
    src[19] = 0x3C
    assert np.all(O.dequantize(src, Q4_0, 1, 64) == -8.0)


def test_q8_0_known_answer():
    """DequantizeTests.cs:45-61: d = 1.0, all quants 0 -> every value 0."""
    src = np.zeros(68, dtype=np.uint8)
    src[1] = 0x3C
    src[35] = 0x3C
    assert np.all(O.dequantize(src, Q8_0, 1, 64) == 0.0)


def test_q4_0_layout():
    """Q4_0: fp16 d, 16 bytes; element j < 16 is the low nibble of byte j,
    element j + 16 the high nibble; value d * (q - 8)."""
    src = np.zeros(18, dtype=np.uint8)
    src[0:2] = np.array([0x3800], np.uint16).view(np.uint8)   # d = 0.5
    q = np.arange(32) % 16
    for j in range(16):
        src[2 + j] = q[j] | (q[j + 16] << 4)
    assert np.array_equal(O.dequantize(src, Q4_0, 1, 32), (0.5 * (q - 8)).astype(np.float32))


def test_q8_0_layout():
    src = np.zeros(34, dtype=np.uint8)
    src[0:2] = np.array([0x4000], np.uint16).view(np.uint8)   # d = 2.0
    q = np.array([(-128 + 9 * i) % 256 - 128 for i in range(32)], dtype=np.int8)
    src[2:] = q.view(np.uint8)
    assert np.array_equal(O.dequantize(src, Q8_0, 1, 32), (2.0 * q.astype(np.float32)))


# ------------------------------------------------ reference-layout Q4_K / Q5_K --

def _put_bits(buf, base, bit, value, width):
    """LSB-first bit writer: bit b of the stream is bit b % 8 of byte b // 8."""
    for k in range(width):
        b = bit + k
        if (value >> k) & 1:
            buf[base + b // 8] |= 1 << (b % 8)


def _kblock(t, d, dmin, sc, m, q):
    """One reference-layout Q4_K (144 B) / Q5_K (176 B) block from its fields:
    sc[g], m[g] at bits 12g and 12g + 6 of the stream at byte 4 (DK:76-136)."""
    size = 144 if t == Q4_K else 176
    b = np.zeros(size, dtype=np.uint8)
    b[0:2] = np.array([d], np.float16).view(np.uint8)
    b[2:4] = np.array([dmin], np.float16).view(np.uint8)
    for g in range(8):
        _put_bits(b, 4, 12 * g, sc[g], 6)
        _put_bits(b, 4, 12 * g + 6, m[g], 6)
    for i in range(256):
        if t == Q4_K:
            b[16 + i // 2] |= (q[i] & 0xF) << (4 * (i % 2))
        else:
            b[48 + i // 2] |= (q[i] & 0xF) << (4 * (i % 2))
            b[16 + i // 8] |= ((q[i] >> 4) & 1) << (i % 8)
    return b


@pytest.mark.parametrize("t", [Q4_K, Q5_K])
def test_kquant_special_block(t):
    """d = 1, dmin = 0, all 6-bit fields = 1, q = i % 16 -> x = i % 16 - offset."""
    q = np.arange(256) % 16
    blk = _kblock(t, 1.0, 0.0, [1] * 8, [1] * 8, q)
    off = 8 if t == Q4_K else 16
    assert np.array_equal(O.dequantize(blk, t, 1, 256), (q - off).astype(np.float32))


@pytest.mark.parametrize("t", [Q4_K, Q5_K])
def test_kquant_field_bit_walk(t):
    """Each of the 16 six-bit fields alone, at every bit: only its sub-block moves."""
    qmax = 15 if t == Q4_K else 31
    off = 8 if t == Q4_K else 16
    q = (np.arange(256) * 7) % (qmax + 1)
    for field in range(16):
        g, is_min = field // 2, field % 2
        for v in (1, 2, 4, 8, 16, 32, 63):
            sc = [0] * 8
            m = [0] * 8
            (m if is_min else sc)[g] = v
            blk = _kblock(t, 0.5, 0.25, sc, m, q)
            x = O.dequantize(blk, t, 1, 256)
            want = np.zeros(256, dtype=np.float64)
            s = slice(32 * g, 32 * g + 32)
            want[s] = 0.5 * sc[g] * (q[s] - off) - 0.25 * m[g]
            assert np.array_equal(x, want.astype(np.float32)), (field, v)


@pytest.mark.parametrize("t", [Q4_K, Q5_K])
def test_kquant_every_q_value(t):
    """Every quant value in every position of sub-block 3, with sc = 5, m = 3."""
    qmax = 15 if t == Q4_K else 31
    off = 8 if t == Q4_K else 16
    for shift in range(qmax + 1):
        q = (np.arange(256) + shift) % (qmax + 1)
        sc, m = [0] * 8, [0] * 8
        sc[3], m[3] = 5, 3
        blk = _kblock(t, 0.125, 2.0, sc, m, q)
        x = O.dequantize(blk, t, 1, 256)
        s = slice(96, 128)
        assert np.array_equal(x[s], (0.125 * 5 * (q[s] - off) - 2.0 * 3).astype(np.float32))


# ------------------------------------------------------------------------ Q6_K --

def _q6block(d, scales, q):
    """ggml Q6_K (210 B): element e = n + 32 t + l (n in {0, 128}, t 0..3, l 0..31)
    has its low 4 bits in ql[n/2 + l + 32 (t & 1)] (high nibble when t >= 2), its
    high 2 bits at bits 2t of qh[n/4 + l], its scale sc[n/16 + l/16 + 2t] and the
    value d * sc * (q - 32) (DK:142-187)."""
    b = np.zeros(210, dtype=np.uint8)
    for e in range(256):
        n, r = (e // 128) * 128, e % 128
        t, l = r // 32, r % 32
        v = q[e]
        ql = n // 2 + l + 32 * (t & 1)
        b[ql] |= (v & 0xF) << (4 * (t >> 1))
        b[128 + n // 4 + l] |= ((v >> 4) & 3) << (2 * t)
    b[192:208] = np.array(scales, dtype=np.int8).view(np.uint8)
    b[208:210] = np.array([d], np.float16).view(np.uint8)
    return b


def test_q6k_layout_and_scales():
    rng = np.random.default_rng(4)
    for trial in range(20):
        q = rng.integers(0, 64, size=256)
        scales = rng.integers(-128, 128, size=16)
        blk = _q6block(0.25, scales, q)
        x = O.dequantize(blk, Q6_K, 1, 256)
        want = np.zeros(256)
        for e in range(256):
            n, r = (e // 128) * 128, e % 128
            t, l = r // 32, r % 32
            want[e] = 0.25 * scales[n // 16 + l // 16 + 2 * t] * (q[e] - 32)
        assert np.array_equal(x, want.astype(np.float32)), trial


# ------------------------------------------------- reference-layout Q2_K / Q3_K --
# No reference test covers these formats; the blocks below are written field by
# field from DequantizeK.cs:8-74 and the expected values are closed forms.

Q2_K, Q3_K = 10, 11


def _q2block(d, dmin, sc, mi, q):
    """Reference Q2_K (84 B): d, dmin; scale/min of sub-block s (16 elements,
    s = 4 (i / 64) + (i % 64) / 16) in the low nibbles of bytes 4 + 2s and
    5 + 2s; 2-bit q of element i at bits 2 (i % 4) of byte 20 + i / 4.  The two
    fields overlap in bytes 20..35: q is written last, so the scale/min nibbles
    of sub-blocks 8..15 are whatever q leaves there (sc/mi for s >= 8 are
    ignored)."""
    b = np.zeros(84, dtype=np.uint8)
    b[0:2] = np.array([d], np.float16).view(np.uint8)
    b[2:4] = np.array([dmin], np.float16).view(np.uint8)
    for s in range(8):
        b[4 + 2 * s] = sc[s] & 0xF
        b[5 + 2 * s] = mi[s] & 0xF
    for i in range(256):
        b[20 + i // 4] &= ~(3 << (2 * (i % 4))) & 0xFF
        b[20 + i // 4] |= (q[i] & 3) << (2 * (i % 4))
    return b


def test_q2k_scales_and_values():
    """q = 0 everywhere: sub-blocks 0..7 give -sc/2 - (dmin/4) mi (d = 1,
    dmin = 0.25); sub-blocks 8..15 read their scale/min nibbles from the zero q
    bytes, so they give d*0*(0 - 1/2) - dmin*0 = -0.0."""
    sc, mi = [1, 2, 3, 5, 7, 11, 13, 15], [0, 1, 2, 3, 4, 8, 12, 15]
    x = O.dequantize(_q2block(1.0, 0.25, sc, mi, [0] * 256), Q2_K, 1, 256)
    for s in range(8):
        assert np.array_equal(x[16 * s:16 * s + 16], np.full(16, -sc[s] / 2 - 0.25 * mi[s], np.float32)), s
    assert np.array_equal(x[128:].view(np.uint32), np.full(128, 0x80000000, np.uint32))


def test_q2k_every_q_value_and_the_overlap():
    """Elements 64..127 (q bytes 36..51, clear of the scale bytes) walk every q
    value; elements 0..15 set bytes 20..23, whose low nibbles are the scale and
    min of sub-blocks 8 and 9 (elements 128..159): q0 | q1 << 2."""
    q = [0] * 256
    for i in range(64, 128):
        q[i] = (i * 3) % 4
    q[0], q[1] = 3, 2      # byte 20 low nibble = 3 | 2 << 2 = 11: sub-block 8's scale
    q[4], q[5] = 1, 1      # byte 21: 1 | 1 << 2 = 5: sub-block 8's min
    q[8], q[9] = 2, 0      # byte 22: 2: sub-block 9's scale
    q[12], q[13] = 0, 3    # byte 23: 12: sub-block 9's min
    sc = [0, 0, 0, 0, 4, 6, 9, 15]
    mi = [0, 0, 0, 0, 1, 0, 3, 2]
    x = O.dequantize(_q2block(0.5, 0.125, sc, mi, q), Q2_K, 1, 256).astype(np.float64)
    for i in range(64, 128):
        s = i // 16
        assert x[i] == np.float32(0.5 * sc[s] * (q[i] - 0.5) - 0.125 * mi[s]), i
    assert np.all(x[128:144] == np.float32(0.5 * 11 * (0 - 0.5) - 0.125 * 5))
    assert np.all(x[144:160] == np.float32(0.5 * 2 * (0 - 0.5) - 0.125 * 12))


def _q3block(d, sc, m, q, size=110):
    """Reference Q3_K (110 B): d; 6-bit scale of group g (16 elements) at bits 6g
    of the stream at byte 4; high-bit mask of element i at bit i % 8 of byte
    16 + i / 8; 2-bit q at bits 2 (i % 4) of byte 48 + i / 4.  The q field needs
    112 bytes: elements 248..255 live in bytes 110 and 111, which belong to the
    next block, so the buffer returned is 112 bytes (the caller overlaps it)."""
    b = np.zeros(112, dtype=np.uint8)
    b[0:2] = np.array([d], np.float16).view(np.uint8)
    for g in range(16):
        _put_bits(b, 4, 6 * g, sc[g], 6)
    for i in range(256):
        b[16 + i // 8] |= (m[i] & 1) << (i % 8)
        b[48 + i // 4] |= (q[i] & 3) << (2 * (i % 4))
    return b


def test_q3k_values_scales_and_mask():
    """value = d * sc[g] * (q - 4 m) for every q and mask bit; the scale field of
    each group at every bit position of its 6."""
    rng = np.random.default_rng(8)
    for trial in range(6):
        q = rng.integers(0, 4, 256)
        m = rng.integers(0, 2, 256)
        sc = [1 << (trial % 6)] * 16 if trial < 6 else rng.integers(0, 64, 16)
        sc = list(sc)
        sc[trial] = 63
        b = _q3block(0.25, sc, m, q)
        q[248:] = 0  # bytes 110..111 are not part of the block: zero after the tensor
        x = O.dequantize(b[:110], Q3_K, 1, 256).astype(np.float64)
        want = np.array([0.25 * sc[i // 16] * (q[i] - 4 * m[i]) for i in range(256)])
        assert np.array_equal(x, want.astype(np.float32)), trial


def test_q3k_reads_two_bytes_of_the_next_block():
    """Two blocks: the first's last 8 values take their q bits from the second
    block's d bytes (DK:64 reads byte 48 + 63 = 111 of a 110-byte block)."""
    q = np.zeros(256, np.int64)
    q[248:] = [1, 2, 3, 0, 3, 3, 1, 0]
    b0 = _q3block(1.0, [2] * 16, [0] * 256, q)
    tail = b0[110:112].copy()
    b1 = _q3block(0.0, [0] * 16, [0] * 256, np.zeros(256, np.int64))
    b1[0:2] = tail   # the second block's d: its bytes are the first block's q tail
    src = np.concatenate([b0[:110], b1[:110]])
    x = O.dequantize(src, Q3_K, 2, 256)
    assert np.array_equal(x[248:256], (2.0 * q[248:]).astype(np.float32))
    d1 = float(np.frombuffer(tail.tobytes(), np.float16)[0])
    assert np.array_equal(x[256:], np.zeros(256, np.float32) * d1)   # scales 0: zeros of the block's sign


# ---------------------------------------------------------- Q4_1 / Q5_0 / Q5_1 --
# TensorOps.DequantizeGeneric (TO:580-652): blocks of 32 written field by field.

Q4_1, Q5_0, Q5_1 = 3, 6, 7


def _q45block(t, d, m, q):
    """Q4_1 (20 B: d, m, nibbles), Q5_0 (22 B: d, qh, nibbles), Q5_1 (24 B: d,
    m, qh, nibbles); element j < 16 in the low nibble of quant byte j, j + 16
    in its high nibble; the fifth bit of element e is bit e of qh."""
    size, oq, oh = {Q4_1: (20, 4, None), Q5_0: (22, 6, 2), Q5_1: (24, 8, 4)}[t]
    b = np.zeros(size, dtype=np.uint8)
    b[0:2] = np.array([d], np.float16).view(np.uint8)
    if t != Q5_0:
        b[2:4] = np.array([m], np.float16).view(np.uint8)
    qh = 0
    for e in range(32):
        b[oq + (e & 15)] |= (q[e] & 15) << (4 * (e >> 4))
        qh |= ((q[e] >> 4) & 1) << e
    if oh is not None:
        b[oh:oh + 4] = np.array([qh], np.uint32).view(np.uint8)
    return b


@pytest.mark.parametrize("t", [Q4_1, Q5_0, Q5_1])
def test_generic_types_every_value(t):
    """Every quant value at every position (a rotating pattern), with the
    closed forms d q + m (Q4_1), d (q - 16) (Q5_0), d q + m (Q5_1)."""
    top = 16 if t == Q4_1 else 32
    for shift in range(top):
        q = [(e + shift) % top for e in range(32)]
        d, m = 0.5, -1.25
        x = O.dequantize(_q45block(t, d, m, q), t, 1, 32).astype(np.float64)
        if t == Q5_0:
            want = [d * (v - 16) for v in q]
        else:
            want = [d * v + m for v in q]
        assert np.array_equal(x, np.asarray(want, np.float32)), shift


def test_q5_high_bit_walk():
    """One set bit of qh at a time moves exactly that element by 16 d."""
    for t in (Q5_0, Q5_1):
        base = O.dequantize(_q45block(t, 0.25, 0.0, [3] * 32), t, 1, 32)
        for e in range(32):
            q = [3] * 32
            q[e] = 19
            x = O.dequantize(_q45block(t, 0.25, 0.0, q), t, 1, 32)
            diff = np.nonzero(x != base)[0]
            assert list(diff) == [e] and x[e] - base[e] == np.float32(4.0), (t, e)


# ------------------------------------------------------------------------ GEMV --

@pytest.mark.parametrize("t", [Q2_K, Q3_K])
def test_kquant_lowbit_gemv_equals_fp64_brute_force(t):
    """Q2_K / Q3_K MatMul (TO:293-362) over random blocks (finite d) against the
    fp64 dot product of the oracle's dequantised rows."""
    rng = np.random.default_rng(t)
    rows, cols = 40, 1024
    bb = 84 if t == Q2_K else 110
    w = rng.integers(0, 256, size=rows * cols // 256 * bb, dtype=np.uint8)
    blocks = w.reshape(-1, bb)
    blocks[:, 0:4] = rng.uniform(-0.05, 0.05, size=(blocks.shape[0], 2)).astype(np.float16).view(np.uint8)
    x = rng.normal(0, 1, size=cols).astype(np.float32)
    wd = O.dequantize(w, t, rows, cols).reshape(rows, cols).astype(np.float64)
    ref = wd @ x.astype(np.float64)
    y = O.matmul(x, w, t, cols, rows)
    assert np.max(np.abs(y - ref)) / np.max(np.abs(ref)) < 2e-6


@pytest.mark.parametrize("t", [Q4_K, Q5_K, Q6_K, Q8_0, Q4_0, F16])
def test_gemv_equals_fp64_brute_force(t):
    """MatMul (TO:60-112 and the fused kernels) against the fp64 dot product of
    the oracle's own dequantised rows."""
    from dotllm_amd import synth
    rng = np.random.default_rng(t)
    rows, cols = 48, 512
    w = synth.quantize(t, rng.normal(0, 0.05, size=(rows, cols)).astype(np.float32))
    x = rng.normal(0, 1, size=cols).astype(np.float32)
    wd = O.dequantize(w, t, rows, cols).reshape(rows, cols).astype(np.float64)
    ref = wd @ x.astype(np.float64)
    y = O.matmul(x, w, t, cols, rows)
    assert np.max(np.abs(y - ref)) / np.max(np.abs(ref)) < 2e-6


def test_matmul_f32_known_answers():
    """TensorOpsTests.cs:8-33 (b holds bCols rows of aCols)."""
    a = np.array([1, 2, 3], np.float32)
    eye = np.eye(3, dtype=np.float32).reshape(-1)
    assert np.array_equal(O.matmul_f32(a, eye, 3, 3), a)
    a2 = np.array([1, 2, 3, 4, 5, 6], np.float32)
    b = np.array([7, 8, 9, 10, 11, 12], np.float32)
    np.testing.assert_allclose(O.matmul_f32(a2, b, 3, 2, result_len=4), [50, 68, 122, 167], atol=1e-3)


# ----------------------------------------------------------------- vector math --

def test_rms_norm_known_answer():
    """VectorMathTests.cs:8-20."""
    out = O.rms_norm(np.array([3, 4], np.float32), np.array([1, 1], np.float32), 1e-5)
    mag = math.sqrt((9 + 16) / 2 + 1e-5)
    np.testing.assert_allclose(out, [3 / mag, 4 / mag], atol=1e-3)


def test_rms_norm_closed_form():
    rng = np.random.default_rng(1)
    x = rng.normal(0, 3, size=1000).astype(np.float32)
    w = rng.normal(1, 0.2, size=1000).astype(np.float32)
    want = w.astype(np.float64) * x / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-6)
    np.testing.assert_allclose(O.rms_norm(x, w, 1e-6), want, rtol=2e-6, atol=1e-6)


def test_softmax_sums_to_one():
    """VectorMathTests.cs:34-54."""
    assert abs(float(np.sum(O.softmax([1, 2, 3, 4]))) - 1) < 1e-3
    assert abs(float(np.sum(O.softmax([10, 20, 30, 40], softcap=5.0))) - 1) < 1e-3


def test_silu_known_answers():
    """VectorMathTests.cs:56-78."""
    assert abs(O.silu(np.array([0.0], np.float32))[0]) < 1e-3
    assert abs(O.silu(np.array([100.0], np.float32))[0] - 100) < 0.1


def test_exp_approx_hand_values():
    """ExpApprox (VM:137-166), evaluated by hand from its steps in float32:
    x = -1: k = (int)(-1.4427 + 0.5) = 0, y = -1, c = 0.5,
    p = 1 - 1 + 0.5 + 0.5*(-1)*0.3333333 + 0.5*1*0.2 = 0.43333335."""
    assert O.exp_approx(0.0) == 1.0
    assert O.exp_approx(-1.0) == f32(0.43333335)
    # x = 1: k = 1, y = 1 - ln2, ExpApprox = 2 (1 + y + y^2/2 + y^3/6 + y^4/10)
    y = 1 - math.log(2)
    assert abs(O.exp_approx(1.0) - 2 * (1 + y + y * y / 2 + y ** 3 / 6 + y ** 4 / 10)) < 1e-6
    assert O.exp_approx(100.0) == math.inf
    assert O.exp_approx(-100.0) == 0.0


def test_exp_approx_discontinuity():
    """The truncating range reduction (int)(x log2e + 0.5) keeps k = 0 down to
    x log2e = -1.5, where the polynomial is 22% above exp; there ExpApprox
    jumps by about 18% (what any non-bit-exact SiLU or softmax input can fall
    across)."""
    edge = -1.5 * math.log(2)
    lo = O.exp_approx(float(np.nextafter(f32(edge), f32(-10))))
    hi = O.exp_approx(float(np.nextafter(f32(edge), f32(10))))
    assert hi / lo > 1.15
    xs = np.linspace(-20, 20, 4001)
    rel = np.array([O.exp_approx(float(x)) for x in xs]) / np.exp(xs)
    assert np.all(np.abs(rel - 1) < 0.25)


def test_silu_tail_uses_expf():
    """Silu (VM:99-116): the last n % 8 elements use MathF.Exp, the rest ExpApprox."""
    x = np.array([-1.0] * 11, np.float32)
    y = O.silu(x)
    lanes = f32(-1.0) / (f32(1.0) + O.exp_approx(1.0))
    tail = f32(-1.0) / (f32(1.0) + np.exp(f32(1.0)))
    assert np.all(y[:8] == lanes)
    np.testing.assert_allclose(y[8:], tail, rtol=1e-6)


def test_argmax_known_answers():
    """VectorMathTests.cs:80-86 and SamplerTests.cs:19-70 (temperature 0)."""
    assert O.argmax([1, 5, 3, 2]) == 1
    logits = np.full(100, 0.01, np.float32)
    logits[42] = 10
    assert O.argmax(logits) == 42
    logits = np.zeros(100, np.float32)
    logits[10], logits[20], logits[30] = 5, 10, 7
    assert O.argmax(logits) == 20
    assert O.argmax([2, 7, 7, 1]) == 1          # first of equal maxima


def test_add_scale_known_answers():
    """VectorMathTests.cs:88-108."""
    assert np.array_equal(O.add([1, 2, 3], [4, 5, 6]), [5, 7, 9])
    assert np.array_equal(O.scale([1, 2, 3], 2), [2, 4, 6])


# ------------------------------------------------------------------------ RoPE --

def test_rope_known_answers():
    """TensorOpsTests.cs:35-81."""
    q = np.ones(128, np.float32)
    qa, ka = O.rope_base(q, q, 128, 1, 10000.0, 128)
    assert qa[64] != 1.0 and ka[64] != 1.0
    q0 = np.array([1, 0, 1, 0], np.float32)
    qb, kb = O.rope_base(q0, q0, 4, 0, 10000.0, 4)
    np.testing.assert_allclose(qb[:2], [1, 0], atol=1e-3)
    assert abs(kb[0] - 1) < 1e-3
    same, _ = O.rope_base(q, None, 128, 1, 10000.0, 128, same=True)
    np.testing.assert_allclose(same, qa, atol=1e-4)


def test_rope_is_a_rotation():
    """NeoX pairs (i, i + half): each pair keeps its norm and turns by pos * freq_i."""
    rng = np.random.default_rng(2)
    hd, pos, base = 64, 37, 10000.0
    q = rng.normal(size=hd).astype(np.float32)
    qr, _ = O.rope_base(q, q.copy(), hd, pos, base, hd)
    half = hd // 2
    for i in range(half):
        a = complex(q[i], q[i + half])
        b = complex(qr[i], qr[i + half])
        assert abs(abs(a) - abs(b)) < 1e-5
        ang = pos / base ** (2 * i / hd)
        assert abs(b - a * complex(math.cos(ang), math.sin(ang))) < 2e-4 * max(1, abs(a))


def _kv_fill_closed_form(seed, layer, kind, pos, e):
    """The documented seeded KV value (llmdot_hip.h, llmdot_hip_model_kv_fill_random)."""
    mask = (1 << 64) - 1
    key = ((2 * layer + kind) << 44) | (pos << 20) | e
    z = (seed + 0x9E3779B97F4A7C15 * (key + 1)) & mask
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & mask
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & mask
    z ^= z >> 31
    return (np.float32(z >> 40) * np.float32(1.0 / 16777216.0) - np.float32(0.5)) * np.float32(3.0)


@pytest.mark.parametrize("kv_fp16", [False, True])
def test_kv_fill_closed_form(kv_fp16):
    """The oracle's seeded KV fill is the documented function of (seed, layer,
    kind, position, element), so a cache of any layout or capacity filled by
    the HIP library holds the same values (the long-context parity tests rely
    on it).  Positions past n stay untouched (zero)."""
    img = synth.build_image("tiny", seed=1234, context=64)
    m = O.Model(img, kv_fp16=kv_fp16, context=64)
    m.kv_fill_random(40, seed=3)
    for layer, pos in ((0, 0), (2, 37), (3, 39)):
        k, v = m.kv_read(layer, pos)
        for kind, got in ((0, k), (1, v)):
            want = np.array([_kv_fill_closed_form(3, layer, kind, pos, e) for e in range(got.size)], np.float32)
            if kv_fp16:
                want = want.astype(np.float16).astype(np.float32)
            assert np.array_equal(got, want), (layer, pos, kind)
    k, v = m.kv_read(1, 40)
    assert not k.any() and not v.any()
    assert float(np.max(np.abs(m.kv_read(2, 5)[0]))) <= 1.5
    m.close()
