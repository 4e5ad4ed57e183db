"""GGUF container: reader, writer and the TransformerConfig resolution.

Reader: GgufReader.Read (src/Llmdot.Core/Loading/GgufReader.cs:8-128): magic,
version >= 2, tensor/kv counts, typed metadata, tensor infos (dims read as
u64, stored as u32), data section aligned to ``general.alignment`` (u32,
default 32).  Tensors are exposed as zero-copy numpy views of the file (or of
an in-memory image), in their native GGUF block layout.

Config: ArchitectureResolver.Resolve (src/Llmdot.Core/Loading/ArchitectureResolver.cs:14-112)
for the LLaMA-like template (llama, phi3, qwen2, stablelm).

Writer: the inverse layout (GGUF v3), used to synthesise seeded models.
"""
from __future__ import annotations

import mmap
import os
import struct
from dataclasses import dataclass, field

import numpy as np

from ._lib import byte_count

# GgufValueType (src/Llmdot.Core/Loading/GgufValueType.cs:3-18)
U8, I8, U16, I16, U32, I32, F32V, BOOL, STR, ARR, U64, I64, F64 = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32V: "<f",
           BOOL: "<B", U64: "<Q", I64: "<q", F64: "<d"}

LLAMA_LIKE = {"llama", "phi3", "qwen2", "stablelm"}
SUPPORTED = {"llama", "phi3", "qwen2", "phi2", "gptneox", "gemma", "gemma2", "stablelm", "lfm2", "lfm2_moe"}


@dataclass
class TensorInfo:
    name: str
    dims: tuple            # GGUF order: dims[0] = columns (input dim), dims[1] = rows
    ggml_type: int
    offset: int
    element_count: int
    data: np.ndarray | None = None   # uint8 view, ByteCount(type, element_count) bytes

    @property
    def cols(self) -> int:   # Tensor.ColumnCount (src/Llmdot.Core/Tensors/Tensor.cs:13)
        return int(self.dims[0]) if self.dims else 0

    @property
    def rows(self) -> int:   # Tensor.RowCount (Tensor.cs:12)
        return int(self.dims[1]) if len(self.dims) > 1 else 1


@dataclass
class GgufModel:
    version: int
    metadata: dict
    metadata_types: dict
    tensors: list
    data_offset: int
    buffer: object = None

    def tensor(self, name: str) -> TensorInfo:
        for t in self.tensors:
            if t.name.lower() == name.lower() and t.data is not None:
                return t
        raise KeyError(f"Tensor '{name}' not found.")

    def has(self, name: str) -> bool:
        return any(t.name.lower() == name.lower() and t.data is not None for t in self.tensors)


class _Cursor:
    def __init__(self, buf):
        self.buf = buf
        self.p = 0

    def take(self, n):
        if self.p + n > len(self.buf):
            raise ValueError("truncated GGUF")
        b = self.buf[self.p:self.p + n]
        self.p += n
        return b

    def scalar(self, fmt):
        return struct.unpack(fmt, self.take(struct.calcsize(fmt)))[0]

    def string(self):
        n = self.scalar("<Q")
        return bytes(self.take(n)).decode("utf-8", "replace")

    def value(self, vt):
        if vt == STR:
            return self.string()
        if vt == ARR:
            et = self.scalar("<I")
            n = self.scalar("<Q")
            return [self.value(et) for _ in range(n)]
        if vt == BOOL:
            return self.scalar("<B") != 0   # one byte, GgufReader.cs:68
        if vt not in _SCALAR:
            raise ValueError(f"Unsupported GGUF value type: {vt}")
        return self.scalar(_SCALAR[vt])


def read(source) -> GgufModel:
    """Parses a GGUF file path, bytes-like object or uint8 numpy array."""
    if isinstance(source, (str, os.PathLike)):
        f = open(source, "rb")
        buf = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
        f.close()
        arr = np.frombuffer(buf, dtype=np.uint8)
    elif isinstance(source, np.ndarray):
        arr = source.reshape(-1).view(np.uint8)
        buf = arr
    else:
        arr = np.frombuffer(source, dtype=np.uint8)
        buf = source
    mv = memoryview(arr)
    c = _Cursor(mv)
    if bytes(c.take(4)) != b"GGUF":
        raise ValueError("Invalid GGUF magic. Expected 'GGUF'.")
    version = c.scalar("<I")
    if version < 2:
        raise ValueError(f"Unsupported GGUF version: {version}. Minimum supported: 2.")
    n_tensors = c.scalar("<Q")
    n_kv = c.scalar("<Q")
    meta, mtypes = {}, {}
    for _ in range(n_kv):
        k = c.string()
        vt = c.scalar("<I")
        meta[k] = c.value(vt)
        mtypes[k] = vt
    infos = []
    for _ in range(n_tensors):
        name = c.string()
        nd = c.scalar("<I")
        dims = tuple(int(c.scalar("<Q")) & 0xFFFFFFFF for _ in range(nd))
        gt = c.scalar("<I")
        off = c.scalar("<Q")
        ec = 1 if dims else 0
        for d in dims:
            ec = (ec * d) & 0xFFFFFFFF    # uint product, GgufReader.cs:113-115
        infos.append(TensorInfo(name, dims, gt, off, ec))
    align = meta.get("general.alignment", 32) if mtypes.get("general.alignment") == U32 else 32
    data_off = c.p + (align - c.p % align) % align
    for t in infos:
        try:
            nb = byte_count(t.ggml_type, t.element_count)
        except NotImplementedError:
            continue
        start = data_off + t.offset
        if nb == 0 or start + nb > len(arr):
            continue        # LoadedModel.LoadTensors skips these (LM:84-88)
        t.data = arr[start:start + nb]
    return GgufModel(version, meta, mtypes, infos, data_off, buf)


@dataclass
class TransformerConfig:
    """The members of the reference's TransformerConfig used by the LLaMA-like decode path."""
    architecture: str
    hidden_size: int
    layer_count: int
    context_length: int
    vocab_size: int
    ffn_dim: int
    head_count: int
    head_count_kv: int
    head_dim: int
    norm_epsilon: float
    rope_freq_base: float
    rope_dimension_count: int
    rope_scaling_type: str = "none"
    rope_scaling_factor: float = 1.0
    tied_embeddings: bool = False
    sliding_window: int = 0
    bos_token_id: int = 1
    eos_token_id: int = 2
    qkv_fused: bool = False
    ffn_type: str = "swiglu"
    qk_norm: bool = False            # attn_q_norm / attn_k_norm tensors (IE:354-365)
    kv_heads_per_layer: tuple = ()   # HeadCountKvPerLayer when the metadata gives a list
    extra: dict = field(default_factory=dict)

    @property
    def q_dim(self) -> int:      # TransformerConfig.QDim
        return self.head_count * self.head_dim

    @property
    def kv_dim(self) -> int:     # TransformerConfig.KvDim
        return self.head_count_kv * self.head_dim


def resolve(model: GgufModel) -> TransformerConfig:
    """ArchitectureResolver.Resolve (AR:14-112), LLaMA-like template only."""
    meta = model.metadata
    arch = str(meta.get("general.architecture", "") or "")
    if not arch.strip():
        raise ValueError("GGUF model missing 'general.architecture' metadata key.")
    if arch.lower() not in SUPPORTED:
        raise ValueError(f"Unsupported GGUF architecture: '{arch}'.")
    if arch.lower() not in LLAMA_LIKE:
        raise NotImplementedError(f"architecture '{arch}' does not use the LLaMA-like template")

    def get(key, default=None):
        return meta.get(f"{arch}.{key}", default)

    hidden = int(get("embedding_length", 0))
    heads = int(get("attention.head_count", 0))
    hkv_raw = get("attention.head_count_kv")
    if isinstance(hkv_raw, list) and hkv_raw:
        hkv = max(int(v) for v in hkv_raw)
    else:
        hkv = int(hkv_raw) if hkv_raw is not None else heads
    head_dim = int(get("attention.key_length", hidden // max(heads, 1)))
    toks = meta.get("tokenizer.ggml.tokens")
    vocab = len(toks) if isinstance(toks, list) else 0
    if f"{arch}.attention.layer_norm_rms_epsilon" in meta:
        eps = float(np.float32(meta[f"{arch}.attention.layer_norm_rms_epsilon"]))
    else:
        raise ValueError(f"No RMS norm epsilon found for architecture '{arch}'.")
    names = {t.name for t in model.tensors}
    return TransformerConfig(
        architecture=arch,
        hidden_size=hidden,
        layer_count=int(get("block_count", 0)),
        context_length=int(get("context_length", 0)),
        vocab_size=vocab,
        ffn_dim=int(get("feed_forward_length", 0)),
        head_count=heads,
        head_count_kv=hkv,
        head_dim=head_dim,
        norm_epsilon=eps,
        rope_freq_base=float(np.float32(get("rope.freq_base", 10000.0))),
        rope_dimension_count=int(get("rope.dimension_count", head_dim)),
        rope_scaling_type=str(get("rope.scaling.type", "") or "none").lower(),
        rope_scaling_factor=float(np.float32(get("rope.scaling.factor", 1.0))),
        tied_embeddings="output.weight" not in names,
        sliding_window=int(get("attention.sliding_window", 0)),
        bos_token_id=int(meta.get("tokenizer.ggml.bos_token_id", 1)),
        eos_token_id=int(meta.get("tokenizer.ggml.eos_token_id", 2)),
        qkv_fused=any("attn_qkv" in n for n in names),
        ffn_type="swiglu" if any("ffn_gate" in n for n in names) else "standard",
        qk_norm=any("attn_q_norm" in n or "attn_k_norm" in n for n in names),
        kv_heads_per_layer=tuple(int(v) for v in hkv_raw) if isinstance(hkv_raw, list) else (),
    )


# ------------------------------------------------------------------ writer --

def _w_str(out: list, s: str) -> None:
    b = s.encode("utf-8")
    out.append(struct.pack("<Q", len(b)))
    out.append(b)


def _w_value(out: list, vt: int, v) -> None:
    if vt == STR:
        _w_str(out, v)
    elif vt == ARR:
        et, items = v
        out.append(struct.pack("<IQ", et, len(items)))
        for it in items:
            _w_value(out, et, it)
    else:
        out.append(struct.pack(_SCALAR[vt], int(v) if vt == BOOL else v))


def header_bytes(metadata: list, tensors: list, alignment: int = 32) -> tuple:
    """Serialises the GGUF v3 header.

    metadata: list of (key, value_type, value); arrays as (ARR, (elem_type, items)).
    tensors:  list of (name, dims (GGUF order), ggml_type, nbytes).
    Returns (header bytes padded to the alignment, [data offsets], total size).
    """
    out = [b"GGUF", struct.pack("<IQQ", 3, len(tensors), len(metadata))]
    for key, vt, v in metadata:
        _w_str(out, key)
        out.append(struct.pack("<I", vt))
        _w_value(out, vt, v)
    offsets, off = [], 0
    for name, dims, gt, nbytes in tensors:
        _w_str(out, name)
        out.append(struct.pack("<I", len(dims)))
        for d in dims:
            out.append(struct.pack("<Q", d))
        out.append(struct.pack("<IQ", gt, off))
        offsets.append(off)
        off += nbytes
        off += (alignment - off % alignment) % alignment
    hdr = b"".join(out)
    hdr += b"\0" * ((alignment - len(hdr) % alignment) % alignment)
    return hdr, offsets, len(hdr) + off
