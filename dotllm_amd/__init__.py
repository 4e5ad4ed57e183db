"""dotllm_amd -- MI355X (gfx950) backend for the llmdot decode token loop.

Layers:
  libllmdot_hip.so  HIP kernels + C ABI (include/llmdot_hip.h)
  backend.HipBackend        IComputeBackend mirror over host spans
  engine.InferenceEngine    device-resident greedy decode (Generate)
  gguf / synth              GGUF reader/writer and seeded synthetic models
"""
from ._lib import (BF16, F16, F32, Q4_0, Q4_K, Q5_K, Q6_K, Q8_0, HipError, byte_count)  # noqa: F401

__all__ = ["HipBackend", "InferenceEngine", "LoadedModel", "GenerationOptions", "SamplingOptions"]


def __getattr__(name):
    if name == "HipBackend":
        from .backend import HipBackend
        return HipBackend
    if name in ("InferenceEngine", "LoadedModel", "GenerationOptions", "SamplingOptions"):
        from . import engine
        return getattr(engine, name)
    raise AttributeError(name)
