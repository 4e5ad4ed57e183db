"""Seeded synthetic GGUF models for the workloads this backend is measured on.

The reference ships no model files and no quantizer.  These builders write
GGUF images (in memory, optionally to disk) whose weights are N(0, sigma)
generated from (seed, tensor name, element index) and quantized by
``llmdot_hip_synth_weights`` into the block layouts the reference decodes.
RMSNorm weights are F32 ones.  ``tokenizer.ggml.tokens`` defines the
vocabulary size (ArchitectureResolver.cs:185-190) and
``tokenizer.ggml.eos_token_id`` is -1 so greedy runs are never cut short.

Shapes:
  tiny      llama  d512  L4  H8/8   hd64  F1408  V32000   all Q8_0
  llama1b   llama  d2048 L16 H32/8  hd64  F8192  V128256  Q4_K_M mix, theta 500000
  mistral7b llama  d4096 L32 H32/8  hd128 F14336 V32000   Q4_K_M mix, theta 10000
  phi3mini  phi3   d3072 L32 H32/32 hd96  F8192  V32064   Q6_K/Q8_0 mix, theta 10000
  small5    llama  d1024 L4  H8/4   hd128 F2816  V32000   Q5_K_M mix, theta 10000
Q4_K_M mix: Q6_K for output.weight and every attn_v, Q4_K for every other
matrix including token_embd.  The phi3mini mix: Q6_K for token_embd, output,
attn_v and ffn_down; Q8_0 for attn_q, attn_k, attn_output, ffn_gate, ffn_up.
Q5_K_M mix: as Q4_K_M with Q5_K in place of Q4_K (small5 exercises Q5_K and a
query-group size of 2 end to end).
"""
from __future__ import annotations

import ctypes as C
import os
import zlib

import numpy as np

from . import _lib, gguf
from ._lib import F32, Q4_K, Q6_K, Q8_0, byte_count, check, lib

SPECS = {
    "tiny": dict(arch="llama", hidden=512, layers=4, heads=8, kv_heads=8, head_dim=64, ffn=1408, vocab=32000,
                 rope_base=10000.0, context=512, mix="q8_0"),
    "llama1b": dict(arch="llama", hidden=2048, layers=16, heads=32, kv_heads=8, head_dim=64, ffn=8192,
                    vocab=128256, rope_base=500000.0, context=1024, mix="q4_k_m"),
    "mistral7b": dict(arch="llama", hidden=4096, layers=32, heads=32, kv_heads=8, head_dim=128, ffn=14336,
                      vocab=32000, rope_base=10000.0, context=4608, mix="q4_k_m"),
    "phi3mini": dict(arch="phi3", hidden=3072, layers=32, heads=32, kv_heads=32, head_dim=96, ffn=8192,
                     vocab=32064, rope_base=10000.0, context=2560, mix="phi3"),
    "small5": dict(arch="llama", hidden=1024, layers=4, heads=8, kv_heads=4, head_dim=128, ffn=2816, vocab=32000,
                   rope_base=10000.0, context=512, mix="q5_k_m"),
}


def tensor_type(mix: str, name: str) -> int:
    if name.endswith("_norm.weight"):
        return F32
    if mix == "q8_0":
        return Q8_0
    if mix == "q4_k_m":
        return Q6_K if (name == "output.weight" or ".attn_v." in name) else Q4_K
    if mix == "q5_k_m":
        return Q6_K if (name == "output.weight" or ".attn_v." in name) else _lib.Q5_K
    if mix == "phi3":
        if name in ("token_embd.weight", "output.weight") or ".attn_v." in name or ".ffn_down." in name:
            return Q6_K
        return Q8_0
    raise ValueError(f"unknown mix {mix}")


def tensor_list(spec: dict, fused_qkv: bool = False, qk_norm: bool = False) -> list:
    """(name, rows, cols, ggml_type) in file order.  fused_qkv: one
    blk.N.attn_qkv.weight of q + 2 kv rows (Q, then K, then V, in attn_q's
    type) in place of the three attention projections, the layout of Phi-3
    GGUFs (QkvLayout.Fused).  qk_norm: per-head RmsNorm weights
    blk.N.attn_q_norm.weight and blk.N.attn_k_norm.weight (head_dim each)."""
    d, f, v = spec["hidden"], spec["ffn"], spec["vocab"]
    q, kv = spec["heads"] * spec["head_dim"], spec["kv_heads"] * spec["head_dim"]
    out = [("token_embd.weight", v, d)]
    for l in range(spec["layers"]):
        p = f"blk.{l}."
        qkv = ([(p + "attn_qkv.weight", q + 2 * kv, d)] if fused_qkv else
               [(p + "attn_q.weight", q, d), (p + "attn_k.weight", kv, d), (p + "attn_v.weight", kv, d)])
        qkn = [(p + "attn_q_norm.weight", 1, spec["head_dim"]), (p + "attn_k_norm.weight", 1, spec["head_dim"])] \
            if qk_norm else []
        out += [(p + "attn_norm.weight", 1, d)] + qkv + qkn + [
            (p + "attn_output.weight", d, q), (p + "ffn_norm.weight", 1, d),
            (p + "ffn_gate.weight", f, d), (p + "ffn_up.weight", f, d), (p + "ffn_down.weight", d, f)]
    out += [("output_norm.weight", 1, d), ("output.weight", v, d)]
    return [(n, r, c, tensor_type(spec["mix"], n.replace("attn_qkv", "attn_q"))) for n, r, c in out]


def tensor_seed(seed: int, name: str) -> int:
    return (int(seed) * 0x9E3779B1 + zlib.crc32(name.encode())) & 0xFFFFFFFFFFFFFFFF


def metadata(spec: dict, context: int | None = None, eos: int = -1, sliding_window: int = 0) -> list:
    a = spec["arch"]
    ctx = int(context or spec["context"])
    toks = [f"<t{i}>" for i in range(spec["vocab"])]
    swa = [(f"{a}.attention.sliding_window", gguf.U32, int(sliding_window))] if sliding_window else []
    return swa + [
        ("general.architecture", gguf.STR, a),
        ("general.name", gguf.STR, f"synthetic-{a}"),
        ("general.alignment", gguf.U32, 32),
        (f"{a}.embedding_length", gguf.U32, spec["hidden"]),
        (f"{a}.block_count", gguf.U32, spec["layers"]),
        (f"{a}.context_length", gguf.U32, ctx),
        (f"{a}.feed_forward_length", gguf.U32, spec["ffn"]),
        (f"{a}.attention.head_count", gguf.U32, spec["heads"]),
        (f"{a}.attention.head_count_kv", gguf.U32, spec["kv_heads"]),
        (f"{a}.attention.key_length", gguf.U32, spec["head_dim"]),
        (f"{a}.attention.layer_norm_rms_epsilon", gguf.F32V, 1e-5),
        (f"{a}.rope.freq_base", gguf.F32V, spec["rope_base"]),
        (f"{a}.rope.dimension_count", gguf.U32, spec["head_dim"]),
        ("tokenizer.ggml.model", gguf.STR, "gpt2"),
        ("tokenizer.ggml.tokens", gguf.ARR, (gguf.STR, toks)),
        ("tokenizer.ggml.bos_token_id", gguf.I32, 1),
        ("tokenizer.ggml.eos_token_id", gguf.I32, int(eos)),
    ]


def synth_tensor(ggml_type: int, rows: int, cols: int, seed: int, out: np.ndarray, sigma: float = 0.02,
                 threads: int | None = None) -> None:
    """Fills ``out`` (uint8, exactly ByteCount bytes) with a seeded quantized tensor."""
    nt = int(threads or min(16, os.cpu_count() or 1))
    check(lib().llmdot_hip_synth_weights(ggml_type, rows, cols, seed, sigma, C.c_void_p(out.ctypes.data), nt))


def tensor_sigma(name: str, spec: dict, sigma: float, scaled_init: bool) -> float:
    """Init std of a tensor: sigma for every matrix (the workloads' stated
    init, N(0, 0.02) everywhere).  With scaled_init, the two projections that
    write into the residual stream (attn_output, ffn_down) take
    sigma / sqrt(2 L) instead, the usual scaled initialisation of an L-layer
    transformer, which keeps the residual stream from growing layer by layer;
    it is an option, not the default."""
    if scaled_init and (".attn_output." in name or ".ffn_down." in name):
        return sigma / float(np.sqrt(2.0 * spec["layers"]))
    return sigma


def build_image(name: str, seed: int = 1234, sigma: float = 0.02, context: int | None = None,
                threads: int | None = None, spec: dict | None = None, scaled_init: bool = False,
                eos: int = -1, tied: bool = False, norm_type: int = F32, fused_qkv: bool = False,
                qk_norm: bool = False, sliding_window: int = 0) -> np.ndarray:
    """Builds the whole GGUF file image in memory (uint8 numpy array).

    eos: tokenizer.ggml.eos_token_id (-1: never stops); tied: no output.weight,
    so the LM head reads token_embd.weight (InferenceEngine.cs:585-589);
    norm_type: F32 or F16 RMSNorm weights (ones either way); fused_qkv: Q, K
    and V rows in one attn_qkv tensor, each range filled exactly as the
    separate tensor of the same type would be (same seed), so a fused image
    holds the same weights as the separate one wherever the types agree;
    qk_norm: per-head Q/K RmsNorm weights (1 + 0.3 N(0, 1), seeded), so that a
    path that skipped or misplaced them would show; sliding_window:
    {arch}.attention.sliding_window (attend to the last N positions)."""
    spec = spec or SPECS[name]
    tl = [(n, r, c, (norm_type if n.endswith("_norm.weight") else t)) for n, r, c, t in tensor_list(spec, fused_qkv, qk_norm)
          if not (tied and n == "output.weight")]
    qd, kvd = spec["heads"] * spec["head_dim"], spec["kv_heads"] * spec["head_dim"]
    infos = [(n, (c,) if r == 1 else (c, r), t, byte_count(t, r * c)) for n, r, c, t in tl]
    hdr, offsets, total = gguf.header_bytes(metadata(spec, context, eos, sliding_window), infos)
    img = np.empty(total, dtype=np.uint8)
    img[:len(hdr)] = np.frombuffer(hdr, dtype=np.uint8)
    base = len(hdr)
    for (n, r, c, t), off, info in zip(tl, offsets, infos):
        nb = info[3]
        view = img[base + off: base + off + nb]
        if n.endswith(("attn_q_norm.weight", "attn_k_norm.weight")):
            w = 1.0 + 0.3 * np.random.default_rng(tensor_seed(seed, n)).standard_normal(c)
            if t == F32:
                view.view(np.float32)[:] = w.astype(np.float32)
            elif t == _lib.F16:
                view.view(np.float16)[:] = w.astype(np.float16)
            else:
                raise ValueError("norm weights are F32 or F16")
        elif n.endswith("_norm.weight"):
            if t == F32:
                view.view(np.float32)[:] = 1.0
            elif t == _lib.F16:
                view.view(np.float16)[:] = 1.0
            else:
                raise ValueError("norm weights are F32 or F16")
        elif n.endswith("attn_qkv.weight"):
            rb = byte_count(t, c)
            o = 0
            for part, pr in (("attn_q", qd), ("attn_k", kvd), ("attn_v", kvd)):
                pn = n.replace("attn_qkv", part)
                synth_tensor(t, pr, c, tensor_seed(seed, pn), view[o:o + pr * rb],
                             tensor_sigma(pn, spec, sigma, scaled_init), threads)
                o += pr * rb
        else:
            synth_tensor(t, r, c, tensor_seed(seed, n), view, tensor_sigma(n, spec, sigma, scaled_init), threads)
        nxt = base + off + nb
        pad = (32 - nxt % 32) % 32
        img[nxt:nxt + pad] = 0
    return img


def prompt(vocab: int, n: int, seed: int = 7) -> list:
    """Uniform random token ids in [0, vocab)."""
    return np.random.Generator(np.random.PCG64(seed)).integers(0, vocab, size=n).astype(np.int32).tolist()


def quantize(ggml_type: int, x: np.ndarray) -> np.ndarray:
    """Quantizes a [rows, cols] float32 matrix into GGUF blocks (reference layouts)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, cols = (1, x.size) if x.ndim == 1 else x.shape
    out = np.zeros(rows * byte_count(ggml_type, cols), dtype=np.uint8)
    check(lib().llmdot_hip_quantize(ggml_type, _lib.ptr(x), rows, cols, _lib.ptr(out)))
    return out


# ------------------------------------------------------------ command line --

QUANT_NAMES = {"f32": F32, "q8_0": Q8_0, "q4_0": _lib.Q4_0, "q4_k": Q4_K, "q5_k": _lib.Q5_K, "q6_k": Q6_K}


def write_model(name: str, path: str, seed: int = 1234, context: int | None = None, sigma: float = 0.02,
                fused_qkv: bool = False) -> int:
    """Writes the seeded synthetic model `name` (SPECS) as a GGUF file; returns its size."""
    img = build_image(name, seed=seed, sigma=sigma, context=context, fused_qkv=fused_qkv)
    with open(path, "wb") as f:
        f.write(img.tobytes())
    return int(img.size)


def quantize_tensors(tensors: dict, ggml_type: int, path: str, metadata_items: list | None = None) -> int:
    """Writes fp32 tensors (name -> 1-D or [rows, cols] array) as a GGUF file:
    2-D tensors quantized to ggml_type, 1-D tensors kept F32 (norm weights).
    GGUF dims are [cols, rows] (Tensor.cs:12-13).  Returns the file size."""
    infos, blobs = [], []
    for n, a in tensors.items():
        a = np.ascontiguousarray(a, dtype=np.float32)
        if a.ndim == 1 or ggml_type == F32:
            q = a.reshape(-1).view(np.uint8)
            dims = (a.shape[-1],) if a.ndim == 1 else (a.shape[1], a.shape[0])
            t = F32
        elif a.ndim == 2:
            if a.shape[1] % _lib.BLOCK[ggml_type][0]:
                raise ValueError(f"{n}: width {a.shape[1]} is not a multiple of the block size")
            q, dims, t = quantize(ggml_type, a), (a.shape[1], a.shape[0]), ggml_type
        else:
            raise ValueError(f"{n}: only 1-D and 2-D tensors")
        infos.append((n, dims, t, int(q.size)))
        blobs.append(q)
    md = [("general.alignment", gguf.U32, 32)] + list(metadata_items or [])
    hdr, offsets, total = gguf.header_bytes(md, infos)
    img = np.zeros(total, dtype=np.uint8)
    img[:len(hdr)] = np.frombuffer(hdr, dtype=np.uint8)
    for off, q in zip(offsets, blobs):
        img[len(hdr) + off: len(hdr) + off + q.size] = q
    with open(path, "wb") as f:
        f.write(img.tobytes())
    return int(total)


def main(argv=None) -> int:
    """python -m dotllm_amd.synth model NAME OUT.gguf [--seed S] [--context N] [--sigma X] [--fused-qkv]
    python -m dotllm_amd.synth quantize IN.npz OUT.gguf --type q4_k|q5_k|q6_k|q8_0|q4_0|f32"""
    import argparse
    ap = argparse.ArgumentParser(prog="python -m dotllm_amd.synth",
                                 description="GGUF writer: seeded synthetic models and reference-layout quantization")
    sub = ap.add_subparsers(dest="cmd", required=True)
    m = sub.add_parser("model", help="write a seeded synthetic model")
    m.add_argument("name", choices=sorted(SPECS))
    m.add_argument("out")
    m.add_argument("--seed", type=int, default=1234)
    m.add_argument("--context", type=int, default=None)
    m.add_argument("--sigma", type=float, default=0.02)
    m.add_argument("--fused-qkv", action="store_true", help="one attn_qkv tensor per layer (the Phi-3 GGUF layout)")
    q = sub.add_parser("quantize", help="quantize the fp32 arrays of an .npz file into a GGUF file")
    q.add_argument("inp")
    q.add_argument("out")
    q.add_argument("--type", required=True, choices=sorted(QUANT_NAMES))
    args = ap.parse_args(argv)
    if args.cmd == "model":
        n = write_model(args.name, args.out, args.seed, args.context, args.sigma, args.fused_qkv)
    else:
        with np.load(args.inp, allow_pickle=False) as z:
            tensors = {k: z[k] for k in z.files}
        n = quantize_tensors(tensors, QUANT_NAMES[args.type], args.out)
    print(f"wrote {args.out}: {n} bytes")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
