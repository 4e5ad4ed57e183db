"""HipBackend: the IComputeBackend contract on MI355X.

Mirrors ``public interface IComputeBackend : IDisposable``
(src/Llmdot.Core/Inference/Backends/IComputeBackend.cs:7-29) member by member
over host numpy spans, calling the C ABI of libllmdot_hip.so.  Weights passed
to :meth:`mat_mul` with a ``weight_key`` are uploaded once and stay resident in
HBM in their native GGUF block layout (the Metal backend's persistent-buffer
cache, src/Llmdot.Metal/MetalBackend.cs:92-100, does the same per key).

Errors surface as exceptions with the reference's types: ValueError for
ArgumentException, NotImplementedError for NotSupportedException, KeyError for
KeyNotFoundException, IndexError for ArgumentOutOfRangeException (and for
spans shorter than the reference would index).  Every member runs on the
device, including those the LLaMA-like decode path never calls (LayerNorm,
Gelu, GeluScalar, Softcap, Conv1D).
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib
from ._lib import check, lib, ptr

_EXC = {_lib.E_INVALID: ValueError, _lib.E_UNSUPPORTED: NotImplementedError,
        _lib.E_NOT_FOUND: KeyError, _lib.E_RANGE: IndexError}


def _call(rc: int) -> None:
    try:
        check(rc)
    except _lib.HipError as e:
        exc = _EXC.get(e.code)
        if exc is not None:
            raise exc(str(e)) from None
        raise


def _f32(a, name: str) -> np.ndarray:
    if not (isinstance(a, np.ndarray) and a.dtype == np.float32 and a.flags["C_CONTIGUOUS"]):
        raise ValueError(f"{name} must be a C-contiguous float32 array")
    return a


def device_count() -> int:
    n = C.c_int32(0)
    rc = lib().llmdot_hip_device_count(C.byref(n))
    return n.value if rc == 0 else 0


def sampling_struct(options) -> "_lib.Sampling":
    """SamplingOptions fields as the C struct."""
    from ._lib import Sampling
    return Sampling(float(options.temperature), int(options.top_k), float(options.top_p),
                    float(options.repeat_penalty), int(options.repeat_penalty_window_size))


class HipBackend:
    """IComputeBackend over one MI355X device (context + stream + weight cache)."""

    def __init__(self, device: int = 0):
        self._ctx = C.c_void_p()
        _call(lib().llmdot_hip_create(device, C.byref(self._ctx)))
        self.device = device

    # -- IDisposable -------------------------------------------------------
    def dispose(self) -> None:
        if self._ctx:
            lib().llmdot_hip_destroy(self._ctx)
            self._ctx = C.c_void_p()

    close = dispose

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.dispose()

    def __del__(self):
        try:
            self.dispose()
        except Exception:
            pass

    @property
    def handle(self) -> C.c_void_p:
        return self._ctx

    def device_info(self) -> dict:
        info = _lib.DeviceInfo()
        _call(lib().llmdot_hip_get_device_info(self._ctx, C.byref(info)))
        return {"name": info.name.decode(), "arch": info.arch.decode(), "compute_units": info.compute_units,
                "clock_mhz": info.clock_mhz, "hbm_bytes": info.hbm_bytes}

    # -- persistent weights ----------------------------------------------------
    def upload_weight(self, key: str, ggml_type: int, data: np.ndarray, rows: int, cols: int) -> None:
        data = np.ascontiguousarray(data).reshape(-1).view(np.uint8)
        _call(lib().llmdot_hip_upload_weight(self._ctx, key.encode(), ggml_type, ptr(data), data.nbytes, rows, cols))

    def release_weight(self, key: str) -> None:
        if not self._ctx:   # disposed: the context released (or will release) every weight
            return
        _call(lib().llmdot_hip_release_weight(self._ctx, key.encode()))

    def has_weight(self, key: str) -> bool:
        v = C.c_int32(0)
        _call(lib().llmdot_hip_has_weight(self._ctx, key.encode(), C.byref(v)))
        return bool(v.value)

    # -- IComputeBackend members --------------------------------------------
    def mat_mul(self, a, b, result, b_type: int, a_cols: int, b_cols: int, weight_key: str | None = None) -> None:
        """ICB:9 MatMul(a, b, result, bType, aCols, bCols, weightKey)."""
        a, result = _f32(a, "a"), _f32(result, "result")
        bp = None
        if b is not None:
            b = np.ascontiguousarray(b).reshape(-1).view(np.uint8)
            bp = ptr(b)
        _call(lib().llmdot_hip_matmul(self._ctx, ptr(a), bp, ptr(result), result.size, b_type, a_cols, b_cols,
                                      weight_key.encode() if weight_key else None))

    def mat_mul_f32(self, a, b, result, a_cols: int, b_cols: int, weight_key: str | None = None) -> None:
        """ICB:10 MatMulF32(a, b, result, aCols, bCols, weightKey)."""
        a, result = _f32(a, "a"), _f32(result, "result")
        bp = ptr(_f32(b, "b")) if b is not None else None
        _call(lib().llmdot_hip_matmul_f32(self._ctx, ptr(a), bp, ptr(result), result.size, a_cols, b_cols,
                                          weight_key.encode() if weight_key else None))

    def rms_norm(self, inp, weights, output, epsilon: float) -> None:
        """ICB:11 RmsNorm(input, weights, output, epsilon)."""
        inp, weights, output = _f32(inp, "input"), _f32(weights, "weights"), _f32(output, "output")
        _call(lib().llmdot_hip_rms_norm(self._ctx, ptr(inp), ptr(weights), ptr(output), inp.size, epsilon))

    def apply_rope(self, query, key, head_dim: int, position: int, freq_table=None, *, freq_base: float | None = None,
                   rotary_dim: int = 0) -> None:
        """ICB:14 ApplyRoPE(query, key, headDim, position, freqTable); with freq_base, ICB:13."""
        query = _f32(query, "query")
        same = key is None or key is query or (isinstance(key, np.ndarray) and np.shares_memory(key, query))
        kp = None if same else ptr(_f32(key, "key"))
        if freq_base is not None:
            _call(lib().llmdot_hip_apply_rope_base(self._ctx, ptr(query), kp, head_dim, position, freq_base,
                                                   rotary_dim, int(same)))
        else:
            ft = _f32(freq_table, "freq_table")
            _call(lib().llmdot_hip_apply_rope(self._ctx, ptr(query), kp, head_dim, position, ptr(ft), ft.size,
                                              int(same)))

    def softmax(self, inp, softcap: float | None = None) -> None:
        """ICB:15 Softmax(input, softcap) in place."""
        inp = _f32(inp, "input")
        _call(lib().llmdot_hip_softmax(self._ctx, ptr(inp), inp.size, int(softcap is not None),
                                       float(softcap) if softcap is not None else 0.0))

    def silu(self, inp, result) -> None:
        """ICB:16 Silu(input, result)."""
        inp, result = _f32(inp, "input"), _f32(result, "result")
        _call(lib().llmdot_hip_silu(self._ctx, ptr(inp), ptr(result), inp.size))

    def silu_in_place(self, inp) -> None:
        """ICB:17 SiluInPlace(input)."""
        inp = _f32(inp, "input")
        _call(lib().llmdot_hip_silu(self._ctx, ptr(inp), ptr(inp), inp.size))

    def add(self, a, b, result=None) -> None:
        """ICB:20 Add(a, b) in place, or ICB:21 Add(a, b, result)."""
        a, b = _f32(a, "a"), _f32(b, "b")
        out = a if result is None else _f32(result, "result")
        _call(lib().llmdot_hip_add(self._ctx, ptr(a), ptr(b), ptr(out), out.size))

    def scale(self, inp, scale: float, result=None) -> None:
        """ICB:22 Scale(input, scale, result) or ICB:23 Scale(input, scale) in place."""
        inp = _f32(inp, "input")
        out = inp if result is None else _f32(result, "result")
        _call(lib().llmdot_hip_scale(self._ctx, ptr(inp), scale, ptr(out), inp.size))

    def mul(self, a, b, result) -> None:
        """ICB:24 Mul(a, b, result)."""
        a, b, result = _f32(a, "a"), _f32(b, "b"), _f32(result, "result")
        _call(lib().llmdot_hip_mul(self._ctx, ptr(a), ptr(b), ptr(result), result.size))

    def dequantize_to_float(self, src, dst, ggml_type: int, num_rows: int, row_elements: int) -> None:
        """ICB:27 DequantizeToFloat(src, dst, type, numRows, rowElements) -- bit-exact."""
        src = np.ascontiguousarray(src).reshape(-1).view(np.uint8)
        dst = _f32(dst, "dst")
        _call(lib().llmdot_hip_dequantize(self._ctx, ptr(src), ptr(dst), ggml_type, num_rows, row_elements))

    def arg_max(self, inp) -> int:
        """ICB:28 ArgMax(input)."""
        inp = _f32(inp, "input")
        idx = C.c_int32(0)
        _call(lib().llmdot_hip_argmax(self._ctx, ptr(inp), inp.size, C.byref(idx)))
        return idx.value

    def sample(self, logits, options, recent_tokens, r: float) -> int:
        """Sampler.Sample (Sampler.cs:24-62) on the device.  options: an object
        with temperature, top_k, top_p, repeat_penalty and
        repeat_penalty_window_size (SamplingOptions); recent_tokens: the
        recent-token list; r: the uniform draw (Random.NextSingle())."""
        x = _f32(logits, "logits")
        rec = np.ascontiguousarray(np.asarray(list(recent_tokens) or [0], dtype=np.int32))
        opt = sampling_struct(options)
        tok = C.c_int32(0)
        _call(lib().llmdot_hip_sample(self._ctx, ptr(x), x.size, C.byref(opt),
                                      rec.ctypes.data_as(C.POINTER(C.c_int32)), len(recent_tokens), float(r),
                                      C.byref(tok)))
        return tok.value

    # Members the LLaMA-like decode path does not call (other templates), on
    # the device like the rest (ICB:12, 18, 19, 25, 26).
    def layer_norm(self, inp, weights, bias, output, epsilon: float) -> None:
        """ICB:12 LayerNorm(input, weights, bias, output, epsilon); bias None or
        empty is the reference's empty bias span."""
        inp, weights, output = _f32(inp, "input"), _f32(weights, "weights"), _f32(output, "output")
        n = inp.size
        if weights.size < n or output.size < n:
            raise IndexError("weights and output must hold input.Length elements")
        bp = None
        if bias is not None and np.asarray(bias).size > 0:
            bias = _f32(bias, "bias")
            if bias.size < n:
                raise IndexError("bias must be empty or hold input.Length elements")
            bp = ptr(bias)
        _call(lib().llmdot_hip_layer_norm(self._ctx, ptr(inp), ptr(weights), bp, ptr(output), n, epsilon))

    def gelu(self, inp, result) -> None:
        """ICB:18 Gelu(input, result)."""
        inp, result = _f32(inp, "input"), _f32(result, "result")
        if result.size < inp.size:
            raise IndexError("result must hold input.Length elements")
        _call(lib().llmdot_hip_gelu(self._ctx, ptr(inp), ptr(result), inp.size))

    def gelu_scalar(self, x: float) -> float:
        """ICB:19 GeluScalar(x): the one-element Gelu (its scalar form)."""
        a = np.array([x], dtype=np.float32)
        out = np.zeros(1, dtype=np.float32)
        _call(lib().llmdot_hip_gelu(self._ctx, ptr(a), ptr(out), 1))
        return float(out[0])

    def softcap(self, inp, cap: float) -> None:
        """ICB:25 Softcap(input, cap) in place."""
        inp = _f32(inp, "input")
        _call(lib().llmdot_hip_softcap(self._ctx, ptr(inp), inp.size, cap))

    def conv1d(self, inp, weights, output, kernel_size: int, input_dim: int) -> None:
        """ICB:26 Conv1D(input, weights, output, kernelSize, inputDim): input and
        weights [inputDim][kernelSize], output [inputDim]."""
        inp, weights, output = _f32(inp, "input"), _f32(weights, "weights"), _f32(output, "output")
        if kernel_size < 1 or input_dim < 0:
            raise ValueError("kernel_size must be positive and input_dim non-negative")
        need = kernel_size * input_dim
        if inp.size < need or weights.size < need or output.size < input_dim:
            raise IndexError("input and weights must hold kernelSize * inputDim elements, output inputDim")
        _call(lib().llmdot_hip_conv1d(self._ctx, ptr(inp), ptr(weights), ptr(output), kernel_size, input_dim))
