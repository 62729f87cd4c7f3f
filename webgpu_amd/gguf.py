"""GGUF tensor/quant-type descriptors, header parser and model configuration.

Host-side mirror of the reference's ``src/core/gguf.ts``: the same type table
(``QUANTS``, gguf.ts:6-11), the same header validation and error messages
(``parseGGUFHeader``, gguf.ts:48-77; ``readGGUF``, :78-83) and the same metadata-driven
``modelConfig`` (gguf.ts:108-213) for the dense decoder families (llama / qwen2 /
qwen3) and Gemma 3. The qwen35 hybrid-recurrent family is rejected: its recurrent
layers are not part of this runtime.
"""
from __future__ import annotations

import math
import struct
from dataclasses import dataclass, field
from typing import Any, Dict, List, Optional

#: GGUF quantization type id -> block layout (gguf.ts:6-11).
QUANTS: Dict[int, Dict[str, Any]] = {
    0: {"name": "F32", "block": 1, "bytes": 4},
    1: {"name": "F16", "block": 1, "bytes": 2},
    2: {"name": "Q4_0", "block": 32, "bytes": 18},
    8: {"name": "Q8_0", "block": 32, "bytes": 34},
    12: {"name": "Q4_K", "block": 256, "bytes": 144},
    13: {"name": "Q5_K", "block": 256, "bytes": 176},
    14: {"name": "Q6_K", "block": 256, "bytes": 210},
}
F32, F16, Q4_0, Q8_0, Q4_K, Q5_K, Q6_K = 0, 1, 2, 8, 12, 13, 14

MAGIC = 0x46554747
MAX_HEADER = 64 * 1024 ** 2


@dataclass
class Tensor:
    """A tensor directory entry (gguf.ts:4). ``offset`` is absolute in the file."""
    name: str
    dims: List[int]
    type: int
    offset: int
    bytes: int
    rowBytes: int


@dataclass
class GGUF:
    metadata: Dict[str, Any]
    tensors: Dict[str, Tensor]
    dataOffset: int
    parameters: int


class NeedMore(Exception):
    """The header continues beyond the bytes read so far (gguf.ts:41)."""


class _Reader:
    def __init__(self, data) -> None:
        self.b = memoryview(data)
        self.offset = 0

    def need(self, n: int) -> None:
        if self.offset + n > len(self.b):
            raise NeedMore()

    def u32(self) -> int:
        self.need(4)
        v = struct.unpack_from("<I", self.b, self.offset)[0]
        self.offset += 4
        return v

    def u64(self) -> int:
        self.need(8)
        v = struct.unpack_from("<Q", self.b, self.offset)[0]
        self.offset += 8
        if v > 2 ** 53 - 1:
            raise ValueError("GGUF integer exceeds safe file addressing.")
        return v

    def string(self) -> str:
        n = self.u64()
        if n > 16 * 1024 ** 2:
            raise ValueError("Oversized GGUF string.")
        self.need(n)
        v = bytes(self.b[self.offset:self.offset + n]).decode("utf-8", errors="replace")
        self.offset += n
        return v

    _FMT = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<B", 11: "<q", 12: "<d"}

    def value(self, type_: int, depth: int = 0) -> Any:
        if depth > 2:
            raise ValueError("Invalid nested metadata.")
        if type_ == 8:
            return self.string()
        if type_ == 9:
            t = self.u32()
            n = self.u64()
            if n > 2_000_000:
                raise ValueError("Oversized GGUF array.")
            return [self.value(t, depth + 1) for _ in range(n)]
        if type_ == 10:
            return self.u64()
        fmt = self._FMT.get(type_)
        if fmt is None:
            raise ValueError(f"Unknown GGUF metadata type {type_}.")
        w = struct.calcsize(fmt)
        self.need(w)
        v = struct.unpack_from(fmt, self.b, self.offset)[0]
        self.offset += w
        return bool(v) if type_ == 7 else v


def parse_gguf_header(data, file_size: int) -> GGUF:
    """parseGGUFHeader (gguf.ts:48-77). Raises NeedMore when ``data`` is too short."""
    r = _Reader(data)
    if r.u32() != MAGIC:
        raise ValueError("Select a GGUF model file.")
    version = r.u32()
    if version not in (2, 3):
        raise ValueError(f"GGUF version {version} is unsupported.")
    count, kv_count = r.u64(), r.u64()
    if count > 100_000 or kv_count > 100_000:
        raise ValueError("Invalid GGUF counts.")
    metadata: Dict[str, Any] = {}
    for _ in range(kv_count):
        key = r.string()
        metadata[key] = r.value(r.u32())
    tensors: Dict[str, Tensor] = {}
    parameters = 0
    for _ in range(count):
        name = r.string()
        nd = r.u32()
        if nd < 1 or nd > 4 or name in tensors:
            raise ValueError("Invalid tensor directory.")
        dims = [r.u64() for _ in range(nd)]
        type_ = r.u32()
        offset = r.u64()
        q = QUANTS.get(type_)
        if q is None:
            raise ValueError(f"Unsupported tensor quantization {type_} in {name}. Use Q4_K_M, Q5_K_M, Q6_K or Q8_0.")
        n = math.prod(dims)
        if n > 2 ** 53 - 1 or any(d < 1 for d in dims) or dims[0] % q["block"] != 0:
            raise ValueError(f"Invalid shape for {name}.")
        row_bytes = dims[0] // q["block"] * q["bytes"]
        tensors[name] = Tensor(name, dims, type_, offset, n // q["block"] * q["bytes"], row_bytes)
        parameters += n
    alignment = metadata.get("general.alignment", 32)
    if not isinstance(alignment, int) or isinstance(alignment, bool) or alignment < 1 or alignment > 4096 or (alignment & (alignment - 1)):
        raise ValueError("Invalid GGUF alignment.")
    data_offset = -(-r.offset // alignment) * alignment
    for t in tensors.values():
        t.offset += data_offset
        if t.offset + t.bytes > file_size:
            raise ValueError(f"Truncated model: {t.name}.")
    return GGUF(metadata, tensors, data_offset, parameters)


def read_gguf(source) -> GGUF:
    """readGGUF (gguf.ts:78-83): doubling header reads from 4 MiB up to 64 MiB."""
    n = min(source.size, 4 * 1024 ** 2)
    while True:
        try:
            return parse_gguf_header(source.read(0, n), source.size)
        except NeedMore:
            if n >= source.size or n >= MAX_HEADER:
                raise ValueError("GGUF header exceeds 64 MiB or is truncated.")
            n = min(source.size, n * 2)


DENSE = {"llama", "qwen2", "qwen3"}


@dataclass
class ModelConfig:
    """ModelConfig (gguf.ts:87-107) for the dense families and Gemma 3."""
    architecture: str
    family: str
    hidden: int
    intermediate: int
    layers: int
    heads: int
    kvHeads: int
    headDim: int
    vocab: int
    epsilon: float
    theta: float
    localTheta: float
    window: int
    period: int
    attentionScale: float
    ropeScale: float
    name: str
    parameters: int
    rotaryDim: int
    maxContext: int
    rope: str
    slidingWindow: int
    qkNorm: bool = True
    ffnGate: bool = True
    activation: str = "silu"
    bias: Dict[str, bool] = field(default_factory=lambda: {"q": False, "k": False, "v": False, "output": False})


def _is_num(v) -> bool:
    return isinstance(v, (int, float)) and not isinstance(v, bool)


def model_config(g: GGUF) -> ModelConfig:
    """modelConfig (gguf.ts:108-213) for llama/qwen2/qwen3 (family 'llama') and gemma3."""
    raw = g.metadata.get("general.architecture")
    if not isinstance(raw, str) or not raw:
        raise ValueError("The GGUF file has no architecture metadata.")
    arch = raw
    family = "gemma3" if arch == "gemma3" else ("llama" if arch in DENSE else None)
    if family is None:
        raise ValueError(f"Supported text architectures: Gemma 3, Llama 3.x and Mistral (llama), Qwen2 and Qwen3. The {arch} architecture is not supported.")

    def num(key: str, fallback: Optional[float] = None) -> float:
        v = g.metadata.get(f"{arch}.{key}", fallback)
        if isinstance(v, bool):
            v = float(v)
        if not _is_num(v) or not math.isfinite(v) or v <= 0:
            raise ValueError(f"Missing or invalid {arch} metadata: {key}.")
        return v

    def opt(key: str, fallback: float) -> float:
        return fallback if g.metadata.get(f"{arch}.{key}") is None else num(key)

    layers, hidden, heads = num("block_count"), num("embedding_length"), num("attention.head_count")
    head_dim = opt("attention.key_length", hidden / heads) if family == "llama" else num("attention.key_length")
    embd = g.tensors.get("token_embd.weight")
    vocab = embd.dims[1] if embd is not None and len(embd.dims) > 1 else 0
    cfg = ModelConfig(
        architecture=arch, family=family, hidden=hidden, layers=layers, heads=heads, headDim=head_dim,
        kvHeads=opt("attention.head_count_kv", heads) if family == "llama" else num("attention.head_count_kv"),
        intermediate=num("feed_forward_length"), vocab=vocab,
        epsilon=num("attention.layer_norm_rms_epsilon", 1e-6),
        theta=opt("rope.freq_base", 10_000) if family == "llama" else num("rope.freq_base", 1_000_000),
        localTheta=opt("rope.freq_base", 10_000) if family == "llama" else num("rope.local.freq_base", 10_000),
        window=0 if family == "llama" else num("attention.sliding_window", 1024),
        period=6 if family == "gemma3" else 0,
        attentionScale=1 / math.sqrt(hidden / heads if family == "gemma3" and layers == 62 else head_dim),
        ropeScale=1.0,
        name=str(g.metadata.get("general.name", arch)), parameters=g.parameters,
        rotaryDim=opt("rope.dimension_count", head_dim) if family == "llama" else head_dim,
        maxContext=num("context_length", 32768),
        rope="norm" if arch == "llama" else "neox",
        slidingWindow=math.floor(opt("attention.sliding_window", 0)) if family == "llama" else num("attention.sliding_window", 1024),
    )
    if family == "gemma3":
        cfg.activation = "gelu"
    # A linear RoPE factor is a plain position divisor; llama3/yarn keep unscaled positions (gguf.ts:173-176).
    if str(g.metadata.get(f"{arch}.rope.scaling.type", "linear")) == "linear":
        cfg.ropeScale = 1 / num("rope.scaling.factor", 1)
    if not (isinstance(cfg.maxContext, int) or float(cfg.maxContext).is_integer()):
        raise ValueError("Invalid model context length.")
    ints = [layers, hidden, heads, head_dim, cfg.kvHeads, cfg.intermediate, cfg.rotaryDim]
    if (any(not float(n).is_integer() or n < 1 for n in ints) or cfg.period < 0 or heads % cfg.kvHeads
            or head_dim % 2 or cfg.rotaryDim % 2 or cfg.rotaryDim > head_dim or not cfg.vocab or layers > 128
            or heads > 256 or head_dim > 512 or hidden > 16384 or cfg.intermediate > 131072 or cfg.vocab > 1_000_000):
        raise ValueError("Unsupported model dimensions.")
    for key in ("layers", "hidden", "heads", "headDim", "kvHeads", "intermediate", "rotaryDim", "maxContext", "window", "slidingWindow"):
        setattr(cfg, key, int(getattr(cfg, key)))

    def shape(name: str, dims: List[int]) -> None:
        t = g.tensors.get(name)
        if t is None or list(t.dims) != list(dims):
            raise ValueError(f"Missing or invalid tensor {name}.")

    H, L = cfg.hidden, cfg.layers
    if family == "llama":
        if "blk.0.ffn_gate_inp.weight" in g.tensors or "blk.0.ffn_gate_exps.weight" in g.tensors:
            raise ValueError("Mixture-of-experts models are not supported.")
        cfg.ffnGate = "blk.0.ffn_gate.weight" in g.tensors
        cfg.qkNorm = "blk.0.attn_q_norm.weight" in g.tensors
        for key in ("q", "k", "v", "output"):
            cfg.bias[key] = f"blk.0.attn_{key}.bias" in g.tensors
        attn, kv = cfg.heads * cfg.headDim, cfg.kvHeads * cfg.headDim
        shape("token_embd.weight", [H, cfg.vocab])
        shape("output_norm.weight", [H])
        if "output.weight" in g.tensors:
            shape("output.weight", [H, cfg.vocab])
        for l in range(L):
            p = f"blk.{l}."
            shape(p + "attn_norm.weight", [H])
            shape(p + "ffn_norm.weight", [H])
            shape(p + "attn_q.weight", [H, attn])
            shape(p + "attn_k.weight", [H, kv])
            shape(p + "attn_v.weight", [H, kv])
            shape(p + "attn_output.weight", [attn, H])
            if cfg.bias["q"]:
                shape(p + "attn_q.bias", [attn])
            if cfg.bias["k"]:
                shape(p + "attn_k.bias", [kv])
            if cfg.bias["v"]:
                shape(p + "attn_v.bias", [kv])
            if cfg.bias["output"]:
                shape(p + "attn_output.bias", [H])
            if cfg.qkNorm:
                for key in ("attn_q_norm", "attn_k_norm"):
                    shape(p + key + ".weight", [cfg.headDim])
            if cfg.ffnGate:
                shape(p + "ffn_gate.weight", [H, cfg.intermediate])
            shape(p + "ffn_up.weight", [H, cfg.intermediate])
            shape(p + "ffn_down.weight", [cfg.intermediate, H])
        return cfg
    shape("token_embd.weight", [H, cfg.vocab])
    shape("output_norm.weight", [H])
    if "output.weight" in g.tensors:
        shape("output.weight", [H, cfg.vocab])
    for l in range(L):
        p = f"blk.{l}."
        for key in ("attn_norm", "post_attention_norm", "ffn_norm", "post_ffw_norm"):
            shape(p + key + ".weight", [H])
        for key in ("attn_q_norm", "attn_k_norm"):
            shape(p + key + ".weight", [cfg.headDim])
        shape(p + "attn_q.weight", [H, cfg.heads * cfg.headDim])
        for key in ("attn_k", "attn_v"):
            shape(p + key + ".weight", [H, cfg.kvHeads * cfg.headDim])
        shape(p + "attn_output.weight", [cfg.heads * cfg.headDim, H])
        for key in ("ffn_gate", "ffn_up"):
            shape(p + key + ".weight", [H, cfg.intermediate])
        shape(p + "ffn_down.weight", [cfg.intermediate, H])
    return cfg
