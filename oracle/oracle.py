"""ctypes wrapper of oracle/liboracle.so -- TEST INFRASTRUCTURE ONLY.

The oracle is the CPU restatement of the reference's managed decode path
(see oracle.h).  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import this module, and only to compute expected values
or as the timed CPU baseline.  Build it with ``make -C oracle`` (gcc, -ffp-contract=off).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")


def build() -> str:
    subprocess.run(["make", "-C", HERE, "-B"], check=True, stdout=subprocess.DEVNULL)
    return LIB_PATH


class Config(C.Structure):
    _fields_ = [("hidden", C.c_int), ("layers", C.c_int), ("context", C.c_int), ("vocab", C.c_int),
                ("ffn", C.c_int), ("heads", C.c_int), ("kv_heads", C.c_int), ("head_dim", C.c_int),
                ("rope_dim", C.c_int), ("rope_scaling_linear", C.c_int), ("rope_scaling_factor", C.c_float),
                ("eps", C.c_float), ("rope_base", C.c_float), ("bos", C.c_int), ("eos", C.c_int),
                ("tied_embeddings", C.c_int), ("sliding_window", C.c_int)]


_P, _I, _F = C.c_void_p, C.c_int, C.c_float
_SIG = {
    "orc_half_to_float": ([C.c_uint16], C.c_float),
    "orc_float_to_half": ([C.c_float], C.c_uint16),
    "orc_byte_count": ([C.c_uint32, C.c_uint64], C.c_int64),
    "orc_extract6": ([_P, _I, _I], _I),
    "orc_exp_approx": ([_F], _F),
    "orc_dequantize": ([_P, _P, C.c_uint32, _I, _I], _I),
    "orc_matmul": ([_P, _P, _P, _I, C.c_uint32, _I, _I], _I),
    "orc_matmul_f32": ([_P, _P, _P, _I, _I, _I], None),
    "orc_rms_norm": ([_P, _P, _P, _I, _F], None),
    "orc_softmax": ([_P, _I, _I, _F], None),
    "orc_silu": ([_P, _P, _I], None),
    "orc_gelu_scalar": ([_F], _F),
    "orc_gelu": ([_P, _P, _I], None),
    "orc_softcap": ([_P, _I, _F], None),
    "orc_layer_norm": ([_P, _P, _P, _P, _I, _F], None),
    "orc_conv1d": ([_P, _P, _P, _I, _I], None),
    "orc_silu_inplace": ([_P, _I], None),
    "orc_add_inplace": ([_P, _P, _I], None),
    "orc_add": ([_P, _P, _P, _I], None),
    "orc_scale": ([_P, _F, _P, _I], None),
    "orc_mul": ([_P, _P, _P, _I], None),
    "orc_rope_table": ([_P, _P, _I, _I, _P, _I, _I], None),
    "orc_rope_base": ([_P, _P, _I, _I, _F, _I, _I], None),
    "orc_argmax": ([_P, _I], _I),
    "orc_sample": ([_P, _I, _F, _I, _F, _F, _I, _P, _I, _F], _I),
    "orc_sample_ex": ([_P, _I, _F, _I, _F, _F, _I, _P, _I, _F, _I], _I),
    "orc_set_threads": ([_I], None),
    "orc_set_order": ([_I], None),
    "orc_get_order": ([], _I),
    "orc_get_threads": ([], _I),
    "orc_model_open_buffer": ([_P, C.c_size_t, _I, C.c_char_p, _I], _P),
    "orc_model_open_file": ([C.c_char_p, _I, C.c_char_p, _I], _P),
    "orc_model_close": ([_P], None),
    "orc_model_config": ([_P, C.POINTER(Config)], None),
    "orc_model_set_context": ([_P, _I], _I),
    "orc_process_token": ([_P, _I, _I, _P], _I),
    "orc_prefill": ([_P, _P, _I, _I, _P], _I),
    "orc_matmul_rows": ([_P, _I, _P, C.c_uint32, _I, _I, _P], _I),
    "orc_generate": ([_P, _P, _I, _I, _I, _P, C.POINTER(C.c_int), _P], _I),
    "orc_kv_fill_random": ([_P, _I, C.c_uint64], _I),
    "orc_kv_read": ([_P, _I, _I, _P, _P], _I),
}

_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        h = C.CDLL(LIB_PATH)
        for name, (args, res) in _SIG.items():
            fn = getattr(h, name)
            fn.argtypes = args
            fn.restype = res
        _lib = h
    return _lib


def _p(a):
    return None if a is None else C.c_void_p(a.ctypes.data)


def set_threads(n: int) -> None:
    lib().orc_set_threads(int(n))


def set_order(order: int) -> None:
    """0: the reference's reduction order; 1, 2, 3: other valid fp32 orders (see oracle.h)."""
    lib().orc_set_order(int(order))


def half_to_float(h: int) -> float:
    return lib().orc_half_to_float(h)


def exp_approx(x: float) -> float:
    return lib().orc_exp_approx(float(x))


def byte_count(t: int, n: int) -> int:
    return lib().orc_byte_count(t, n)


Q3_K = 11


def _blocks(b: np.ndarray, ggml_type: int) -> np.ndarray:
    """The block bytes as one uint8 vector; for Q3_K with two zero bytes after
    them.  The reference's Q3_K reads its 2-bit values up to byte 111 of a
    110-byte block (DequantizeK.cs:64, TensorOps.cs:353): inside a tensor that
    is the next block's first two bytes, after the last block the reference's
    span check throws; here, as on the device, those two bytes read zero."""
    b = np.ascontiguousarray(b).reshape(-1).view(np.uint8)
    if ggml_type == Q3_K:
        b = np.concatenate([b, np.zeros(2, np.uint8)])
    return b


def dequantize(src: np.ndarray, ggml_type: int, num_rows: int, row_elements: int) -> np.ndarray:
    src = _blocks(src, ggml_type)
    dst = np.zeros(num_rows * row_elements, dtype=np.float32)
    if lib().orc_dequantize(_p(src), _p(dst), ggml_type, num_rows, row_elements) != 0:
        raise NotImplementedError(f"Dequantization for type {ggml_type} not yet implemented.")
    return dst


def matmul(a: np.ndarray, b: np.ndarray, ggml_type: int, a_cols: int, b_cols: int, result_len: int | None = None):
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = _blocks(b, ggml_type)
    n = result_len or b_cols
    out = np.zeros(n, dtype=np.float32)
    if lib().orc_matmul(_p(a), _p(b), _p(out), n, ggml_type, a_cols, b_cols) != 0:
        raise NotImplementedError(f"MatMul for type {ggml_type}")
    return out


def matmul_rows(a: np.ndarray, b: np.ndarray, ggml_type: int, a_cols: int, b_cols: int) -> np.ndarray:
    """[rows][b_cols]: each activation row as its own single-row MatMul, through
    the batched path of the prompt processing (bitwise the same)."""
    a = np.ascontiguousarray(a, dtype=np.float32).reshape(-1, a_cols)
    b = _blocks(b, ggml_type)
    out = np.zeros((a.shape[0], b_cols), dtype=np.float32)
    if lib().orc_matmul_rows(_p(a), a.shape[0], _p(b), ggml_type, a_cols, b_cols, _p(out)) != 0:
        raise NotImplementedError(f"MatMul for type {ggml_type}")
    return out


def matmul_f32(a, b, a_cols, b_cols, result_len=None):
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    n = result_len or b_cols
    out = np.zeros(n, dtype=np.float32)
    lib().orc_matmul_f32(_p(a), _p(b), _p(out), n, a_cols, b_cols)
    return out


def rms_norm(x, w, eps):
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    out = np.zeros_like(x)
    lib().orc_rms_norm(_p(x), _p(w), _p(out), x.size, eps)
    return out


def softmax(x, softcap=None):
    x = np.array(x, dtype=np.float32)
    lib().orc_softmax(_p(x), x.size, int(softcap is not None), float(softcap or 0.0))
    return x


def silu(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros_like(x)
    lib().orc_silu(_p(x), _p(out), x.size)
    return out


def gelu_scalar(x):
    """VectorMath.Gelu(float), VM:169-170."""
    return float(lib().orc_gelu_scalar(float(x)))


def gelu(x):
    """VectorMath.Gelu(input, result), VM:172-193."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros_like(x)
    lib().orc_gelu(_p(x), _p(out), x.size)
    return out


def softcap(x, cap):
    """VectorMath.Softcap, VM:286-302 (returns the capped copy)."""
    x = np.array(x, dtype=np.float32)
    lib().orc_softcap(_p(x), x.size, float(cap))
    return x


def layer_norm(x, w, b, eps):
    """VectorMath.LayerNorm, VM:342-405; b None is the empty bias span."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    out = np.zeros_like(x)
    bp = None if b is None else _p(np.ascontiguousarray(b, dtype=np.float32))
    lib().orc_layer_norm(_p(x), _p(w), bp, _p(out), x.size, float(eps))
    return out


def conv1d(x, w, kernel_size, input_dim):
    """TensorOps.Conv1D, TO:745-775: x and w are [input_dim][kernel_size]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    out = np.zeros(input_dim, dtype=np.float32)
    lib().orc_conv1d(_p(x), _p(w), _p(out), int(kernel_size), int(input_dim))
    return out


def silu_inplace(x):
    x = np.array(x, dtype=np.float32)
    lib().orc_silu_inplace(_p(x), x.size)
    return x


def add(a, b):
    a = np.ascontiguousarray(a, dtype=np.float32); b = np.ascontiguousarray(b, dtype=np.float32)
    out = np.zeros_like(a); lib().orc_add(_p(a), _p(b), _p(out), a.size); return out


def mul(a, b):
    a = np.ascontiguousarray(a, dtype=np.float32); b = np.ascontiguousarray(b, dtype=np.float32)
    out = np.zeros_like(a); lib().orc_mul(_p(a), _p(b), _p(out), a.size); return out


def scale(a, s):
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.zeros_like(a); lib().orc_scale(_p(a), float(s), _p(out), a.size); return out


def rope_table(q, k, head_dim, position, freq, same=False):
    q = np.array(q, dtype=np.float32)
    k = q if same else np.array(k, dtype=np.float32)
    freq = np.ascontiguousarray(freq, dtype=np.float32)
    lib().orc_rope_table(_p(q), _p(k), head_dim, position, _p(freq), freq.size, int(same))
    return q, k


def rope_base(q, k, head_dim, position, freq_base, rotary_dim, same=False):
    q = np.array(q, dtype=np.float32)
    k = q if same else np.array(k, dtype=np.float32)
    lib().orc_rope_base(_p(q), _p(k), head_dim, position, freq_base, rotary_dim, int(same))
    return q, k


def argmax(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    return lib().orc_argmax(_p(x), x.size)


def sample(logits, temperature, top_k, top_p, repeat_penalty, window, recent, r, aliased=True):
    """Sampler.Sample (Sampler.cs:24-62) with the uniform draw r given.

    aliased=True is the reference as written, FindNucleus writing its sorted
    values into the buffer that holds the probabilities it reads
    (Sampler.cs:30, 48-50, 150); aliased=False gives it a buffer of its own."""
    x = np.ascontiguousarray(logits, dtype=np.float32)
    rec = np.ascontiguousarray(list(recent) if len(recent) else [0], dtype=np.int32)
    return lib().orc_sample_ex(_p(x), x.size, float(temperature), int(top_k), float(top_p), float(repeat_penalty),
                               int(window), _p(rec), len(recent), float(r), int(bool(aliased)))


class Model:
    """The reference decode path over a GGUF image (numpy uint8) or file."""

    def __init__(self, source, kv_fp16: bool = False, context: int | None = None):
        err = C.create_string_buffer(512)
        if isinstance(source, (str, os.PathLike)):
            self._buf = None
            self._m = lib().orc_model_open_file(os.fsencode(source), int(kv_fp16), err, 512)
        else:
            self._buf = np.ascontiguousarray(source).reshape(-1).view(np.uint8)
            self._m = lib().orc_model_open_buffer(_p(self._buf), self._buf.nbytes, int(kv_fp16), err, 512)
        if not self._m:
            raise ValueError(err.value.decode())
        if context:
            if lib().orc_model_set_context(self._m, int(context)) != 0:
                raise MemoryError("KV cache allocation failed")
        c = Config()
        lib().orc_model_config(self._m, C.byref(c))
        self.config = c

    def close(self):
        if self._m:
            lib().orc_model_close(self._m)
            self._m = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def process_token(self, token: int, position: int) -> np.ndarray:
        out = np.zeros(self.config.vocab, dtype=np.float32)
        rc = lib().orc_process_token(self._m, int(token), int(position), _p(out))
        if rc != 0:
            raise IndexError(f"ProcessToken failed ({rc})")
        return out

    def prefill(self, tokens, pos0: int = 0) -> np.ndarray:
        """Logits of the last of len(tokens) ProcessToken calls from pos0, with the
        chunk's tokens going through each layer together (bitwise the same)."""
        t = np.ascontiguousarray(np.asarray(tokens, dtype=np.int32))
        out = np.zeros(self.config.vocab, dtype=np.float32)
        rc = lib().orc_prefill(self._m, _p(t), t.size, int(pos0), _p(out))
        if rc != 0:
            raise IndexError(f"prefill failed ({rc})")
        return out

    def generate(self, prompt, max_tokens: int, eos: int | None = None, return_logits: bool = False):
        p = np.ascontiguousarray(np.asarray(prompt, dtype=np.int32))
        toks = np.zeros(max(max_tokens, 1), dtype=np.int32)
        logits = np.zeros((max(max_tokens, 1), self.config.vocab), dtype=np.float32) if return_logits else None
        n = C.c_int(0)
        rc = lib().orc_generate(self._m, _p(p), p.size, max_tokens, self.config.eos if eos is None else eos,
                                _p(toks), C.byref(n), _p(logits))
        if rc != 0:
            raise IndexError(f"Generate failed ({rc})")
        k = n.value
        return toks[:k].tolist(), (logits[:k] if return_logits else None)

    def kv_fill_random(self, n: int, seed: int = 1):
        if lib().orc_kv_fill_random(self._m, n, seed) != 0:
            raise IndexError("fill past the KV cache")

    def kv_read(self, layer: int, position: int):
        kvd = self.config.kv_heads * self.config.head_dim
        k = np.zeros(kvd, dtype=np.float32)
        v = np.zeros(kvd, dtype=np.float32)
        if lib().orc_kv_read(self._m, layer, position, _p(k), _p(v)) != 0:
            raise IndexError("kv_read out of range")
        return k, v
