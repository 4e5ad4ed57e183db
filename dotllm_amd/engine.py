"""LoadedModel + InferenceEngine over the device-resident decode step.

Mirrors the reference's public entry points for the hot path:
  LoadedModel.Load(stream)                (src/Llmdot.Core/Inference/LoadedModel.cs:45-55)
  new InferenceEngine(model, backend)     (src/Llmdot.Core/Inference/InferenceEngine.cs:42)
  engine.Generate(prompt, options, ct)    (InferenceEngine.cs:74-132), greedy sampling
                                          (src/Llmdot.Core/Sampling/Sampler.cs:26-27)
GenerationOptions / SamplingOptions carry the reference's defaults
(GenerationOptions.cs:6-12, SamplingOptions.cs:7-15).

Unlike the reference, which pushes every op through IComputeBackend with host
spans, the engine keeps weights, KV cache and activations in HBM and runs the
whole token loop on the device (llmdot_hip_generate): one captured HIP graph per
decode step, token feedback through device memory.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field

import numpy as np

from . import _lib, gguf
from ._lib import lib
from .backend import HipBackend, _call


@dataclass
class SamplingOptions:
    top_k: int = 40
    top_p: float = 0.95
    temperature: float = 0.8
    repeat_penalty: float = 1.1
    repeat_penalty_window_size: int = 64
    seed: int = -1


@dataclass
class GenerationOptions:
    max_tokens: int = 256
    sampling: SamplingOptions = field(default_factory=SamplingOptions)
    stop_sequences: tuple = ()


def greedy(max_tokens: int) -> GenerationOptions:
    return GenerationOptions(max_tokens=max_tokens, sampling=SamplingOptions(temperature=0.0))


# Tensor names of the LLaMA-like template (src/Llmdot.Core/Loading/TensorNameResolver.cs:22-107).
LAYER_TENSORS = ("attn_norm", "attn_q", "attn_k", "attn_v", "attn_qkv", "attn_q_norm", "attn_k_norm", "attn_output",
                 "ffn_norm", "ffn_gate", "ffn_up", "ffn_down")


class LoadedModel:
    """A parsed GGUF model (tensors are zero-copy views of the file or image).

    Device copies of its tensors live in a backend under `key_prefix + name`;
    the prefix is unique per LoadedModel, so engines of different models that
    share one backend never see each other's weights, while engines of the
    same model share one copy.
    """

    _next_id = 0

    def __init__(self, g: gguf.GgufModel, config: gguf.TransformerConfig):
        self.gguf = g
        self.config = config
        LoadedModel._next_id += 1
        self.key_prefix = f"model{LoadedModel._next_id}/"
        self._users = {}   # id(backend) -> number of live engines using the uploaded copy

    @classmethod
    def load(cls, source) -> "LoadedModel":
        g = gguf.read(source)
        return cls(g, gguf.resolve(g))

    def tensor(self, name: str) -> gguf.TensorInfo:
        return self.gguf.tensor(name)

    def decode_tensor_names(self) -> list:
        cfg = self.config
        names = ["token_embd.weight"]
        for l in range(cfg.layer_count):
            for t in LAYER_TENSORS:
                n = f"blk.{l}.{t}.weight"
                if self.gguf.has(n):
                    names.append(n)
        names.append("output_norm.weight" if self.gguf.has("output_norm.weight") else "token_embd_norm.weight")
        if self.gguf.has("output.weight"):
            names.append("output.weight")
        return names


class InferenceEngine:
    """Greedy decode of a LLaMA-like GGUF model on one MI355X."""

    def __init__(self, model: LoadedModel, backend: HipBackend | None = None, *, kv_fp16: bool = True,
                 context: int | None = None):
        cfg = model.config
        if cfg.ffn_type != "swiglu":
            raise NotImplementedError("only SwiGLU FFN tensors are supported")
        if any(h != cfg.head_count_kv for h in cfg.kv_heads_per_layer):
            raise NotImplementedError("per-layer KV head counts are not supported")
        self.model = model
        self.backend = backend or HipBackend()
        self._own_backend = backend is None
        self.context = int(context or cfg.context_length)
        prefix = model.key_prefix
        for name in model.decode_tensor_names():
            t = model.tensor(name)
            if not self.backend.has_weight(prefix + name):
                self.backend.upload_weight(prefix + name, t.ggml_type, t.data, t.rows, t.cols)
        model._users[id(self.backend)] = model._users.get(id(self.backend), 0) + 1
        self._weights_held = True
        d = _lib.ModelDesc()
        d.hidden, d.layers = cfg.hidden_size, cfg.layer_count
        d.heads, d.kv_heads, d.head_dim = cfg.head_count, cfg.head_count_kv, cfg.head_dim
        d.ffn, d.vocab, d.context = cfg.ffn_dim, cfg.vocab_size, self.context
        d.rope_dim = cfg.rope_dimension_count
        d.eps, d.rope_base = cfg.norm_epsilon, cfg.rope_freq_base
        d.rope_linear_factor = (cfg.rope_scaling_factor
                                if cfg.rope_scaling_type == "linear" and cfg.rope_scaling_factor > 1 else 1.0)
        d.kv_fp16 = 1 if kv_fp16 else 0
        d.bos = cfg.bos_token_id
        d.sliding_window = int(cfg.sliding_window)
        d.key_prefix = prefix.encode()
        self._m = C.c_void_p()
        _call(lib().llmdot_hip_model_create(self.backend.handle, C.byref(d), C.byref(self._m)))
        self.vocab = cfg.vocab_size

    def dispose(self) -> None:
        if getattr(self, "_m", None):
            lib().llmdot_hip_model_destroy(self._m)
            self._m = C.c_void_p()
        if getattr(self, "_weights_held", False) and self.backend is not None:
            # the last engine of this model on this backend frees the device copy
            self._weights_held = False
            users = self.model._users
            users[id(self.backend)] -= 1
            if users[id(self.backend)] == 0:
                del users[id(self.backend)]
                for name in self.model.decode_tensor_names():
                    self.backend.release_weight(self.model.key_prefix + name)
        if getattr(self, "_own_backend", False) and self.backend is not None:
            self.backend.dispose()
            self.backend = None

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
        return self._m

    # -- Generate ------------------------------------------------------------
    def generate(self, prompt_tokens, options: GenerationOptions | None = None, chunk: int = 1, draws=None):
        """InferenceEngine.Generate (IE:74-132) as a stream: yields each token id
        as soon as the device has it (llmdot_hip_generate_begin / _next, `chunk`
        tokens per device round trip; the step for the next token is already
        running while the caller handles this one).  Stopping the iteration is
        the cancellation: nothing further is computed."""
        options = options or GenerationOptions()
        if options.stop_sequences:
            raise NotImplementedError("stop sequences need the tokenizer")
        if chunk < 1:
            raise ValueError("chunk must be at least 1")
        prompt = np.ascontiguousarray(np.asarray(prompt_tokens, dtype=np.int32))
        n = int(options.max_tokens)
        pp = prompt.ctypes.data_as(C.POINTER(C.c_int32))
        eos = int(self.model.config.eos_token_id)
        if options.sampling.temperature > 0:
            from .backend import sampling_struct
            d = np.ascontiguousarray(draws if draws is not None else self.draws_for(options.sampling, n),
                                     dtype=np.float32)
            if d.size < n:
                raise ValueError("one uniform draw per generated token is needed")
            opt = sampling_struct(options.sampling)
            _call(lib().llmdot_hip_generate_begin(self._m, pp, prompt.size, n, eos, C.byref(opt),
                                                  d.ctypes.data_as(C.POINTER(C.c_float))))
        else:
            _call(lib().llmdot_hip_generate_begin(self._m, pp, prompt.size, n, eos, None, None))
        out = np.zeros(chunk, dtype=np.int32)
        n_out, done = C.c_int32(0), C.c_int32(0)
        while not done.value:
            rc = lib().llmdot_hip_generate_next(self._m, chunk, out.ctypes.data_as(C.POINTER(C.c_int32)),
                                                C.byref(n_out), C.byref(done), None)
            if rc == _lib.E_RANGE:   # the KV cache ended: these tokens, then stop
                yield from out[:n_out.value].tolist()
                return
            _call(rc)
            yield from out[:n_out.value].tolist()

    @staticmethod
    def draws_for(sampling: SamplingOptions, n: int) -> np.ndarray:
        """Uniform draws for n tokens.  The reference builds new Random(Seed) for
        every draw when Seed >= 0 (Sampler.cs:160), so every token uses the same
        value; this host uses numpy's generator for that value (System.Random's
        sequence is not reproduced: a C# caller passes its own NextSingle())."""
        if sampling.seed >= 0:
            r = np.random.default_rng(sampling.seed).random(dtype=np.float32)
            return np.full(max(n, 1), r, dtype=np.float32)
        return np.random.default_rng().random(max(n, 1), dtype=np.float32)

    def generate_all(self, prompt_tokens, options: GenerationOptions, return_logits: bool = False, draws=None):
        """Greedy when Temperature <= 0 (Sampler.cs:26-27), else the device sampler
        with the given uniform draws (draws_for(options.sampling) by default)."""
        if options.stop_sequences:
            raise NotImplementedError("stop sequences need the tokenizer")
        prompt = np.ascontiguousarray(np.asarray(prompt_tokens, dtype=np.int32))
        n = int(options.max_tokens)
        out = np.zeros(max(n, 1), dtype=np.int32)
        logits = np.zeros((max(n, 1), self.vocab), dtype=np.float32) if return_logits else None
        n_out = C.c_int32(0)
        pp = prompt.ctypes.data_as(C.POINTER(C.c_int32))
        eos = int(self.model.config.eos_token_id)
        lp = _lib.ptr(logits) if logits is not None else None
        if options.sampling.temperature > 0:
            from .backend import sampling_struct
            d = np.ascontiguousarray(draws if draws is not None else self.draws_for(options.sampling, n),
                                     dtype=np.float32)
            if d.size < n:
                raise ValueError("one uniform draw per generated token is needed")
            opt = sampling_struct(options.sampling)
            rc = lib().llmdot_hip_generate_sampled(self._m, pp, prompt.size, n, eos, C.byref(opt),
                                                   d.ctypes.data_as(C.POINTER(C.c_float)),
                                                   out.ctypes.data_as(C.POINTER(C.c_int32)), C.byref(n_out), lp)
        else:
            rc = lib().llmdot_hip_generate(self._m, pp, prompt.size, n, eos,
                                           out.ctypes.data_as(C.POINTER(C.c_int32)), C.byref(n_out), lp)
        k = n_out.value
        if rc == _lib.E_RANGE and k > 0:
            return out[:k].tolist(), (logits[:k] if logits is not None else None)
        _call(rc)
        return out[:k].tolist(), (logits[:k] if logits is not None else None)

    # -- single steps -----------------------------------------------------------
    def process_token(self, token: int, position: int) -> np.ndarray:
        """ProcessToken (IE:134-146): returns the vocab logits."""
        logits = np.zeros(self.vocab, dtype=np.float32)
        am = C.c_int32(0)
        _call(lib().llmdot_hip_decode_step(self._m, int(token), int(position), _lib.ptr(logits), C.byref(am)))
        return logits

    def prefill(self, tokens, pos0: int = 0):
        t = np.ascontiguousarray(np.asarray(tokens, dtype=np.int32))
        logits = np.zeros(self.vocab, dtype=np.float32)
        am = C.c_int32(0)
        _call(lib().llmdot_hip_prefill(self._m, t.ctypes.data_as(C.POINTER(C.c_int32)), t.size, int(pos0),
                                       _lib.ptr(logits), C.byref(am)))
        return logits, am.value

    def reset(self) -> None:
        _call(lib().llmdot_hip_model_reset(self._m))

    def kv_read(self, layer: int, position: int):
        kvd = self.model.config.kv_dim
        k = np.zeros(kvd, dtype=np.float32)
        v = np.zeros(kvd, dtype=np.float32)
        _call(lib().llmdot_hip_kv_read(self._m, layer, position, _lib.ptr(k), _lib.ptr(v)))
        return k, v

    # -- measurement ---------------------------------------------------------------
    def step_bytes(self, position: int) -> float:
        b = C.c_double(0)
        _call(lib().llmdot_hip_model_step_bytes(self._m, int(position), C.byref(b)))
        return b.value

    def kv_fill_random(self, n: int, seed: int = 1) -> None:
        _call(lib().llmdot_hip_model_kv_fill_random(self._m, int(n), int(seed)))

    def time_prefill(self, tokens, pos0: int = 0) -> float:
        """Milliseconds (HIP events) of the batched prompt path over tokens from pos0."""
        t = np.ascontiguousarray(np.asarray(tokens, dtype=np.int32))
        ms = C.c_float(0)
        _call(lib().llmdot_hip_model_time_prefill(self._m, t.ctypes.data_as(C.POINTER(C.c_int32)), t.size, int(pos0),
                                                  C.byref(ms)))
        return ms.value

    def time_decode(self, first_token: int, position: int, steps: int, per_kernel: bool = False) -> dict:
        t = _lib.StepTiming()
        _call(lib().llmdot_hip_model_time_decode(self._m, int(first_token), int(position), int(steps),
                                                 int(per_kernel), C.byref(t)))
        return {"total_ms": t.total_ms, "gemv_ms": t.gemv_ms, "gemv_launches": t.gemv_launches,
                "gemv_bytes": t.gemv_bytes}
