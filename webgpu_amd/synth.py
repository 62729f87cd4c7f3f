"""Seeded synthetic GGUF files for the decoder shapes this runtime is measured on.

No checkpoints are available offline, so models are random-init GGUFs with the exact
tensor directory, metadata and block layouts of real files:

* ``tiny``      — the check:dense model of scripts/verify-dense.mjs:60-135 reshaped as
                  specified: F32, arch ``qwen3`` without Q/K-norm or bias tensors (so the
                  half-split RoPE path of gguf.ts:168-170), 2 layers, hidden 64, 4/2 heads,
                  head_dim 16, FFN 128 SwiGLU, vocab 256, eps 1e-5, theta 1e4; matrices
                  N(0, 0.02) from the reference's LCG (verify-dense.mjs:25) with Box-Muller;
                  norm vectors 1.
* ``qwen3-0.6b``, ``llama3-8b``, ``gemma3-27b`` — Q4_K_M-style mixes (Q4_K attention/FFN,
                  Q6_K attn_v and output / tied embedding) at the real shapes.

Quantized blocks are drawn from numpy's PCG64 (seeded per tensor): Q4_K blocks get
uniform 6-bit scales/mins and 4-bit quants with dmin = 7.5 d, which centres every
sub-block (E[sc*q] = 7.5 E[m] * sc-mean), and d sized so the weights have std ~0.02;
Q6_K blocks get uniform quants and int8 scales with d sized the same way (often an f16
subnormal, which the decode must and does handle). Norm vectors are 1 + U(-0.1, 0.1) as
the reference's ``eins`` (verify-dense.mjs:74).

Tied heads: where ``token_embd`` is also the output matrix, logit j is the normed state
dotted with w * e_j, and with all-positive output-norm weights the current token's own
embedding (a large share of the state at Gemma's sqrt(hidden) input scale) scores itself
highest, so greedy decoding repeats one token forever. ``signed_out_norm`` draws the
output-norm entries with random signs, which takes that self-affinity to zero mean; the
Qwen3-0.6B shape also draws its embeddings at std 1 (``embd_std``), so the current token,
not the context average, sets the next one. Both are choices of random initialisation
only: the tensor directory, types and shapes are unchanged.
"""
from __future__ import annotations

import math
import struct
from dataclasses import dataclass, field
from typing import Callable, Dict, List, Optional, Tuple

import numpy as np

from .gguf import F32, Q4_K, Q6_K, Q8_0, QUANTS, MAGIC

ALIGN = 32


def lcg(seed: int) -> Callable[[], float]:
    """The reference's LCG (verify-dense.mjs:25): uniform in [0, 1)."""
    state = seed & 0xFFFFFFFF

    def nxt() -> float:
        nonlocal state
        state = (state * 1664525 + 1013904223) & 0xFFFFFFFF
        return state / 4294967296.0
    return nxt


def lcg_normal(seed: int, n: int, std: float) -> np.ndarray:
    """N(0, std) via Box-Muller over LCG draws, as float32."""
    r = lcg(seed)
    out = np.empty(n, np.float64)
    for i in range(0, n, 2):
        u1, u2 = 1.0 - r(), r()
        rad = math.sqrt(-2.0 * math.log(u1))
        out[i] = rad * math.cos(2 * math.pi * u2)
        if i + 1 < n:
            out[i + 1] = rad * math.sin(2 * math.pi * u2)
    return (out * std).astype(np.float32)


# ------------------------------------------------------------------ block generators

def q4k_blocks(rng: np.random.Generator, nb: int, std: float = 0.02) -> np.ndarray:
    """nb random Q4_K super-blocks (144 bytes each), centred, weight std ~ ``std``."""
    b = np.frombuffer(rng.bytes(nb * 144), np.uint8).copy().reshape(nb, 144)
    d = (std / 245.0) * rng.uniform(0.75, 1.25, nb)
    b[:, 0:2] = d.astype(np.float16).view(np.uint8).reshape(nb, 2)
    b[:, 2:4] = (7.5 * d).astype(np.float16).view(np.uint8).reshape(nb, 2)
    return b.reshape(-1)


def q6k_blocks(rng: np.random.Generator, nb: int, std: float = 0.02) -> np.ndarray:
    """nb random Q6_K super-blocks (210 bytes each), weight std ~ ``std``."""
    b = np.frombuffer(rng.bytes(nb * 210), np.uint8).copy().reshape(nb, 210)
    d = (std / 1365.0) * rng.uniform(0.75, 1.25, nb)
    b[:, 208:210] = d.astype(np.float16).view(np.uint8).reshape(nb, 2)
    return b.reshape(-1)


def q5k_blocks(rng: np.random.Generator, nb: int, std: float = 0.02) -> np.ndarray:
    """nb random Q5_K super-blocks (176 bytes each), centred, weight std ~ ``std``."""
    b = np.frombuffer(rng.bytes(nb * 176), np.uint8).copy().reshape(nb, 176)
    d = (std / 480.0) * rng.uniform(0.75, 1.25, nb)
    b[:, 0:2] = d.astype(np.float16).view(np.uint8).reshape(nb, 2)
    b[:, 2:4] = (15.5 * d).astype(np.float16).view(np.uint8).reshape(nb, 2)
    return b.reshape(-1)


def q4_0_blocks(rng: np.random.Generator, nb: int, std: float = 0.02) -> np.ndarray:
    """nb random Q4_0 blocks (18 bytes each), weight std ~ ``std``."""
    b = np.frombuffer(rng.bytes(nb * 18), np.uint8).copy().reshape(nb, 18)
    d = (std / 4.6) * rng.uniform(0.75, 1.25, nb)
    b[:, 0:2] = d.astype(np.float16).view(np.uint8).reshape(nb, 2)
    return b.reshape(-1)


def f16_values(rng: np.random.Generator, n: int, std: float = 0.02) -> np.ndarray:
    """n normal F16 weights of standard deviation ``std``, as bytes."""
    return (rng.standard_normal(n) * std).astype(np.float16).view(np.uint8).copy()


def q8_0_blocks(rng: np.random.Generator, nb: int, std: float = 0.02) -> np.ndarray:
    b = np.frombuffer(rng.bytes(nb * 34), np.uint8).copy().reshape(nb, 34)
    d = (std / 73.9) * rng.uniform(0.75, 1.25, nb)
    b[:, 0:2] = d.astype(np.float16).view(np.uint8).reshape(nb, 2)
    return b.reshape(-1)


def microbench_q4k(rng: np.random.Generator, rows: int, cols: int) -> np.ndarray:
    """Q4_K matvec microbench blocks: uniform scale/min/quant bytes, fp16 d and dmin
    drawn log-uniform in [2^-12, 2^-8]."""
    nb = rows * cols // 256
    b = np.frombuffer(rng.bytes(nb * 144), np.uint8).copy().reshape(nb, 144)
    for o in (0, 2):
        v = np.exp2(rng.uniform(-12, -8, nb)).astype(np.float16)
        b[:, o:o + 2] = v.view(np.uint8).reshape(nb, 2)
    return b.reshape(-1)


def microbench_q6k(rng: np.random.Generator, rows: int, cols: int) -> np.ndarray:
    nb = rows * cols // 256
    b = np.frombuffer(rng.bytes(nb * 210), np.uint8).copy().reshape(nb, 210)
    v = np.exp2(rng.uniform(-16, -12, nb)).astype(np.float16)
    b[:, 208:210] = v.view(np.uint8).reshape(nb, 2)
    return b.reshape(-1)


# ------------------------------------------------------------------ model specs

@dataclass
class Spec:
    name: str
    arch: str
    layers: int
    hidden: int
    heads: int
    kv_heads: int
    head_dim: int
    ffn: int
    vocab: int
    eps: float
    theta: float
    qk_norm: bool
    tied: bool
    types: Dict[str, int]          # role -> GGUF type
    local_theta: float = 10000.0
    window: int = 1024
    context_length: int = 32768
    std: float = 0.02
    norm_ones: bool = False         # norm vectors exactly 1 (tiny) instead of 1 + U(-0.1, 0.1)
    seed: int = 1234
    embd_std: Optional[float] = None  # token_embd std (default: std)
    signed_out_norm: bool = False     # output_norm entries carry random signs


SPECS: Dict[str, Spec] = {
    "tiny": Spec("tiny", "qwen3", 2, 64, 4, 2, 16, 128, 256, 1e-5, 10000.0, False, False,
                 {"embd": F32, "output": F32, "attn": F32, "v": F32, "ffn": F32}, norm_ones=True, seed=13,
                 context_length=2048),
    "qwen3-0.6b": Spec("qwen3-0.6b", "qwen3", 28, 1024, 16, 8, 128, 3072, 151936, 1e-6, 1_000_000.0, True, True,
                       {"embd": Q6_K, "output": Q6_K, "attn": Q4_K, "v": Q6_K, "ffn": Q4_K}, context_length=40960,
                       embd_std=1.0, signed_out_norm=True),
    "llama3-8b": Spec("llama3-8b", "llama", 32, 4096, 32, 8, 128, 14336, 128256, 1e-5, 500_000.0, False, False,
                      {"embd": Q4_K, "output": Q6_K, "attn": Q4_K, "v": Q6_K, "ffn": Q4_K}, context_length=8192),
    "gemma3-27b": Spec("gemma3-27b", "gemma3", 62, 5376, 32, 16, 128, 21504, 262144, 1e-6, 1_000_000.0, True, True,
                       {"embd": Q6_K, "output": Q6_K, "attn": Q4_K, "v": Q6_K, "ffn": Q4_K}, context_length=131072),
    # The Gemma-3-27B widths at six layers: five local (window 1024) and one global layer
    # (period 6), so a prompt past 1151 tokens wraps the local rings inside the model. At
    # this depth modelConfig takes the attention scale 1/sqrt(head_dim) (gguf.ts:134).
    "gemma3-27b-6l": Spec("gemma3-27b-6l", "gemma3", 6, 5376, 32, 16, 128, 21504, 262144, 1e-6, 1_000_000.0, True,
                          True, {"embd": Q6_K, "output": Q6_K, "attn": Q4_K, "v": Q6_K, "ffn": Q4_K},
                          context_length=131072, signed_out_norm=True),
    # Small quantized models for the sanitizer runs: every weight type, both rope modes, a
    # Gemma-3 layer period of six with 16-token local windows (a 40-token prompt in 8-token
    # batches wraps their rings) and head dims off the 64/128/256 fast paths.
    "mini-gemma3": Spec("mini-gemma3", "gemma3", 6, 256, 4, 2, 64, 512, 1024, 1e-6, 1_000_000.0, True, True,
                        {"embd": Q6_K, "output": Q6_K, "attn": Q4_K, "v": Q6_K, "ffn": Q4_K}, window=16,
                        context_length=4096, seed=21),
    "mini-llama": Spec("mini-llama", "llama", 3, 256, 8, 2, 32, 768, 512, 1e-5, 500_000.0, False, False,
                       {"embd": Q8_0, "output": Q6_K, "attn": Q8_0, "v": Q8_0, "ffn": Q4_K},
                       context_length=4096, seed=22),
}


def tensor_list(s: Spec) -> List[Tuple[str, List[int], int, str]]:
    """(name, dims, type, role) in file order."""
    t: List[Tuple[str, List[int], int, str]] = []
    H, qd, kd = s.hidden, s.heads * s.head_dim, s.kv_heads * s.head_dim
    t.append(("token_embd.weight", [H, s.vocab], s.types["embd"], "embd"))
    t.append(("output_norm.weight", [H], F32, "norm"))
    if not s.tied:
        t.append(("output.weight", [H, s.vocab], s.types["output"], "output"))
    for l in range(s.layers):
        p = f"blk.{l}."
        t.append((p + "attn_norm.weight", [H], F32, "norm"))
        t.append((p + "attn_q.weight", [H, qd], s.types["attn"], "attn"))
        t.append((p + "attn_k.weight", [H, kd], s.types["attn"], "attn"))
        t.append((p + "attn_v.weight", [H, kd], s.types["v"], "v"))
        t.append((p + "attn_output.weight", [qd, H], s.types["attn"], "attn"))
        if s.qk_norm:
            t.append((p + "attn_q_norm.weight", [s.head_dim], F32, "norm"))
            t.append((p + "attn_k_norm.weight", [s.head_dim], F32, "norm"))
        if s.arch == "gemma3":
            t.append((p + "post_attention_norm.weight", [H], F32, "norm"))
            t.append((p + "post_ffw_norm.weight", [H], F32, "norm"))
        t.append((p + "ffn_norm.weight", [H], F32, "norm"))
        t.append((p + "ffn_gate.weight", [H, s.ffn], s.types["ffn"], "ffn"))
        t.append((p + "ffn_up.weight", [H, s.ffn], s.types["ffn"], "ffn"))
        t.append((p + "ffn_down.weight", [s.ffn, H], s.types["ffn"], "ffn"))
    return t


def metadata(s: Spec) -> List[Tuple[str, int, object]]:
    a = s.arch
    m: List[Tuple[str, int, object]] = [
        ("general.architecture", 8, a), ("general.name", 8, f"synthetic-{s.name}"),
        (f"{a}.block_count", 4, s.layers), (f"{a}.context_length", 4, s.context_length),
        (f"{a}.embedding_length", 4, s.hidden), (f"{a}.feed_forward_length", 4, s.ffn),
        (f"{a}.attention.head_count", 4, s.heads), (f"{a}.attention.head_count_kv", 4, s.kv_heads),
        (f"{a}.attention.key_length", 4, s.head_dim), (f"{a}.attention.value_length", 4, s.head_dim),
        (f"{a}.attention.layer_norm_rms_epsilon", 6, s.eps), (f"{a}.rope.freq_base", 6, s.theta),
    ]
    if a == "gemma3":
        m += [(f"{a}.rope.local.freq_base", 6, s.local_theta), (f"{a}.attention.sliding_window", 4, s.window)]
    else:
        m += [(f"{a}.rope.dimension_count", 4, s.head_dim)]
    return m


def _header(meta, tensors, offsets) -> bytes:
    out = bytearray()
    out += struct.pack("<IIQQ", MAGIC, 3, len(tensors), len(meta))

    def s(v: str) -> None:
        b = v.encode()
        out.extend(struct.pack("<Q", len(b)) + b)

    def scalar(typ: int, val) -> None:
        if typ == 8:
            s(val)
        elif typ == 4:
            out.extend(struct.pack("<I", val))
        elif typ == 5:
            out.extend(struct.pack("<i", val))
        elif typ == 6:
            out.extend(struct.pack("<f", val))
        elif typ == 7:
            out.extend(struct.pack("<B", 1 if val else 0))
        else:
            raise ValueError(typ)
    for key, typ, val in meta:
        s(key)
        out.extend(struct.pack("<I", typ))
        if typ == 9:  # array: (element type, values)
            et, vals = val
            out.extend(struct.pack("<IQ", et, len(vals)))
            for v in vals:
                scalar(et, v)
        else:
            scalar(typ, val)
    for (name, dims, typ, _), off in zip(tensors, offsets):
        s(name)
        out.extend(struct.pack("<I", len(dims)))
        for d in dims:
            out.extend(struct.pack("<Q", d))
        out.extend(struct.pack("<IQ", typ, off))
    return bytes(out)


def tensor_bytes(dims: List[int], typ: int) -> int:
    q = QUANTS[typ]
    return int(np.prod(dims)) // q["block"] * q["bytes"]


def build(spec: Spec | str, seed: Optional[int] = None) -> np.ndarray:
    """The whole GGUF file as a uint8 array (header, alignment padding, tensor data)."""
    s = SPECS[spec] if isinstance(spec, str) else spec
    seed = s.seed if seed is None else seed
    tensors = tensor_list(s)
    offsets, off = [], 0
    for _, dims, typ, _ in tensors:
        off = -(-off // ALIGN) * ALIGN
        offsets.append(off)
        off += tensor_bytes(dims, typ)
    header = _header(metadata(s), tensors, offsets)
    data_start = -(-len(header) // ALIGN) * ALIGN
    total = data_start + (-(-off // ALIGN) * ALIGN)
    f = np.zeros(total, np.uint8)
    f[:len(header)] = np.frombuffer(header, np.uint8)
    for i, ((name, dims, typ, role), o) in enumerate(zip(tensors, offsets)):
        n = int(np.prod(dims))
        dst = f[data_start + o: data_start + o + tensor_bytes(dims, typ)]
        tseed = (seed * 1_000_003 + i * 7919) & 0x7FFFFFFF
        std = s.embd_std if role == "embd" and s.embd_std is not None else s.std
        if role == "norm":
            if s.norm_ones:
                v = np.ones(n, np.float32)
            else:
                v = (1.0 + np.random.default_rng(tseed).uniform(-0.1, 0.1, n)).astype(np.float32)
            if s.signed_out_norm and name == "output_norm.weight":
                v *= np.where(np.random.default_rng(tseed + 1).integers(0, 2, n) == 1, 1.0, -1.0).astype(np.float32)
            dst[:] = v.view(np.uint8)
        elif typ == F32:
            dst[:] = lcg_normal(tseed, n, std).view(np.uint8)
        else:
            rng = np.random.default_rng(tseed)
            nb = n // QUANTS[typ]["block"]
            gen = {Q4_K: q4k_blocks, Q6_K: q6k_blocks, Q8_0: q8_0_blocks}[typ]
            dst[:] = gen(rng, nb, std)
    return f


def prompt_ids(vocab: int, n: int, seed: int = 7) -> List[int]:
    """Random prompt token ids, uniform in [0, vocab)."""
    return [int(v) for v in np.random.default_rng(seed).integers(0, vocab, n)]
