"""ctypes wrapper of liborc.so, the float64 CPU oracle (oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, as the checker or the timed CPU baseline. The product never imports it.
"""
from __future__ import annotations

import ctypes as C
import math
import os
import subprocess
from typing import List, Optional, Sequence

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "liborc.so")

_P, _I32, _I64, _D = C.c_void_p, C.c_int32, C.c_int64, C.c_double


def build() -> str:
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        l = C.CDLL(LIB)
        l.orc_half.restype = _D; l.orc_half.argtypes = [C.c_uint16]
        l.orc_decode.restype = _D; l.orc_decode.argtypes = [_P, _I32, _I64]
        l.orc_dequant_row.restype = C.c_int; l.orc_dequant_row.argtypes = [_P, _I32, _I64, _P]
        l.orc_dequant_f32.restype = C.c_int; l.orc_dequant_f32.argtypes = [_P, _I32, _I64, _P]
        l.orc_matmul.restype = C.c_int
        l.orc_matmul.argtypes = [_I32, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64]
        l.orc_norm.restype = None; l.orc_norm.argtypes = [_P, _P, _P, _I64, _D]
        l.orc_rope.restype = None
        l.orc_rope.argtypes = [_P, _P, _I64, _I64, _I64, _D, _D, _D, _I64, _I64, _I32]
        l.orc_attention.restype = None
        l.orc_attention.argtypes = [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _D, _I64, _I64, _I64]
        l.orc_argmax.restype = _I64; l.orc_argmax.argtypes = [_P, _I64]
        l.orc_model_create.restype = _P; l.orc_model_create.argtypes = [_P, C.POINTER(_I32)]
        l.orc_model_tensor.restype = C.c_int; l.orc_model_tensor.argtypes = [_P, C.c_char_p, _I32, _I64, _I64, _P]
        l.orc_model_forward.restype = C.c_int; l.orc_model_forward.argtypes = [_P, C.POINTER(_I32), _I32, _I32, _P]
        l.orc_model_destroy.restype = None; l.orc_model_destroy.argtypes = [_P]
        l.orc_threads.restype = C.c_int; l.orc_threads.argtypes = []
        l.orc_round_f16.restype = _D; l.orc_round_f16.argtypes = [_D]
        _lib = l
    return _lib


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def round_f16(x: float) -> float:
    """x rounded to the nearest binary16 value (ties to even), as a float."""
    return lib().orc_round_f16(x)


def half(h: int) -> float:
    return lib().orc_half(h)


def decode(data: np.ndarray, type_: int, i: int) -> float:
    return lib().orc_decode(_ptr(data), type_, i)


def dequant(data: np.ndarray, type_: int, count: int, f32: bool = True) -> np.ndarray:
    data = np.ascontiguousarray(data, np.uint8)
    out = np.empty(count, np.float32 if f32 else np.float64)
    rc = (lib().orc_dequant_f32 if f32 else lib().orc_dequant_row)(_ptr(data), type_, count, _ptr(out))
    if rc:
        raise ValueError("oracle dequant failed")
    return out


def matmul(type_: int, w: np.ndarray, x: np.ndarray, cols: int, rows: int, stride: int, row_base: int,
           input_offset: int, batch: int) -> np.ndarray:
    w = np.ascontiguousarray(w, np.uint8)
    x = np.ascontiguousarray(x, np.float32)
    y = np.zeros((batch - 1) * stride + row_base + rows, np.float64)
    if lib().orc_matmul(type_, _ptr(w), _ptr(x), _ptr(y), cols, rows, stride, row_base, input_offset, batch):
        raise ValueError("oracle matmul failed")
    return y


def norm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float64)
    w = np.ascontiguousarray(w, np.float64)
    y = np.empty_like(x)
    lib().orc_norm(_ptr(x), _ptr(w), _ptr(y), x.size, eps)
    return y


def rope(x: np.ndarray, w: Optional[np.ndarray], heads: int, hd: int, start: int, theta: float, scale: float,
         eps: float, rotary_dim: int, batch: int, mode: int) -> np.ndarray:
    y = np.array(x, np.float64, copy=True)
    wv = np.ascontiguousarray(w, np.float64) if w is not None else None
    lib().orc_rope(_ptr(y), _ptr(wv) if wv is not None else None, heads, hd, start, theta, scale, eps,
                   rotary_dim, batch, mode)
    return y


def attention(q, k, v, heads, kv_heads, hd, start, scale, window, capacity, batch) -> np.ndarray:
    q = np.ascontiguousarray(q, np.float64)
    k = np.ascontiguousarray(k, np.float64)
    v = np.ascontiguousarray(v, np.float64)
    y = np.zeros(batch * heads * hd, np.float64)
    lib().orc_attention(_ptr(q), _ptr(k), _ptr(v), _ptr(y), heads, kv_heads, hd, start, scale, window, capacity, batch)
    return y


def argmax(logits: np.ndarray) -> int:
    a = np.ascontiguousarray(logits, np.float32)
    return int(lib().orc_argmax(_ptr(a), a.size))


MASK64 = (1 << 64) - 1


def splitmix64_at(seed: int, index: int) -> int:
    """The index-th output (from 0) of splitmix64 seeded with ``seed`` (Steele, Lea and
    Flood, OOPSLA 2014): the generator whose uniforms stand in for Math.random()."""
    z = (seed + (index + 1) * 0x9E3779B97F4A7C15) & MASK64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & MASK64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & MASK64
    return z ^ (z >> 31)


def uniform(seed: int, index: int) -> float:
    """The 53-bit uniform in [0, 1) drawn for the token at position ``index``."""
    return (splitmix64_at(seed, index) >> 11) * 2.0 ** -53


def sample(logits, temperature: float, top_k: int, top_p: float, u: float) -> int:
    """sample() of src/core/engine.ts:305-324 with Math.random() = u.

    Best finite logit (first index of the maximum); temperature 0 returns it. Otherwise the
    top_k finite logits in descending order with ties to the lower index (the order the
    reference's insertion into a stably sorted list leaves, :312-315), f64 probabilities
    exp((l - best) / T) (:314), their sum (:317), the prefix whose share reaches top_p
    (:318-319) and the draw u * retained walked down it (:320-322)."""
    l = np.asarray(logits, np.float32)
    idx = np.flatnonzero(np.isfinite(l))
    if idx.size == 0:
        raise ValueError("Inference produced non-finite logits.")
    vals = l[idx]
    best_id = int(idx[int(np.argmax(vals))])
    best = float(l[best_id])
    if temperature == 0:
        return best_id
    cand = idx[np.argsort(-vals.astype(np.float64), kind="stable")[:top_k]]
    probs = [math.exp((float(l[i]) - best) / temperature) for i in cand]
    total = 0.0
    for p in probs:
        total += p
    retained, cutoff = 0.0, 0
    while cutoff < len(probs):
        retained += probs[cutoff]
        cutoff += 1
        if retained / total >= top_p:
            break
    draw = u * retained
    for i in range(cutoff):
        draw -= probs[i]
        if draw <= 0:
            return int(cand[i])
    return best_id


def threads() -> int:
    return int(lib().orc_threads())


class OrcConfig(C.Structure):
    _fields_ = [(n, C.c_int32) for n in (
        "family", "rope_adjacent", "hidden", "intermediate", "layers", "heads", "kv_heads", "head_dim", "vocab",
        "rotary_dim", "window", "period", "qk_norm", "ffn_gate", "gelu", "bias_q", "bias_k", "bias_v",
        "bias_output", "tied_output", "context", "batch")] + [(n, C.c_double) for n in (
        "epsilon", "theta", "local_theta", "attention_scale", "rope_scale", "embed_scale")] + [("kv_f16", C.c_int32)]


def config_struct(gguf, cfg, context: int, kv_f16: bool = False) -> OrcConfig:
    """The oracle's orc_config for a parsed GGUF and its model config."""
    c = OrcConfig()
    gemma = cfg.family == "gemma3"
    c.family = 1 if gemma else 0
    c.rope_adjacent = 1 if cfg.rope == "norm" else 0
    c.hidden, c.intermediate, c.layers = cfg.hidden, cfg.intermediate, cfg.layers
    c.heads, c.kv_heads, c.head_dim, c.vocab = cfg.heads, cfg.kvHeads, cfg.headDim, cfg.vocab
    c.rotary_dim = cfg.rotaryDim
    c.window = cfg.window if gemma else cfg.slidingWindow
    c.period = cfg.period
    c.qk_norm = int(cfg.qkNorm)
    c.ffn_gate = int(cfg.ffnGate)
    c.gelu = int(cfg.activation == "gelu")
    c.bias_q, c.bias_k, c.bias_v, c.bias_output = (int(cfg.bias[k]) for k in ("q", "k", "v", "output"))
    c.tied_output = 0 if "output.weight" in gguf.tensors else 1
    c.context, c.batch = context, 128
    c.epsilon, c.theta, c.local_theta = cfg.epsilon, cfg.theta, cfg.localTheta
    c.attention_scale, c.rope_scale = cfg.attentionScale, cfg.ropeScale
    c.embed_scale = math.sqrt(cfg.hidden) if cfg.architecture == "gemma3" else 1.0
    c.kv_f16 = 1 if kv_f16 else 0
    return c


class OracleModel:
    """The f64 reference forward over the raw bytes of a GGUF file."""

    def __init__(self, file: np.ndarray, gguf, cfg, context: int, capacities: Sequence[int],
                 kv_f16: bool = False) -> None:
        self.file = np.ascontiguousarray(file, np.uint8)
        self.cfg = cfg
        c = config_struct(gguf, cfg, context, kv_f16)
        caps = (C.c_int32 * cfg.layers)(*capacities)
        self.m = lib().orc_model_create(C.byref(c), caps)
        base = self.file.ctypes.data
        for t in gguf.tensors.values():
            ne1 = t.dims[1] if len(t.dims) > 1 else 1
            lib().orc_model_tensor(self.m, t.name.encode(), t.type, t.dims[0], ne1, base + t.offset)

    def forward(self, ids: Sequence[int], start: int, logits: bool = True) -> Optional[np.ndarray]:
        n = len(ids)
        arr = (C.c_int32 * n)(*ids)
        out = np.empty(self.cfg.vocab, np.float64) if logits else None
        if lib().orc_model_forward(self.m, arr, n, start, _ptr(out) if logits else None):
            raise ValueError("oracle forward failed")
        return out

    def greedy(self, prompt: Sequence[int], steps: int, chunk: int = 128) -> tuple:
        """Greedy tokens after `prompt` and the top-2 margin of every step."""
        logits = None
        for i in range(0, len(prompt), chunk):
            logits = self.forward(prompt[i:i + chunk], i)
        toks, margins = [], []
        pos = len(prompt)
        for s in range(steps):
            top = int(np.argmax(logits))
            second = float(np.max(np.delete(logits, top)))
            toks.append(top)
            margins.append(float(logits[top] - second))
            if s + 1 < steps:
                logits = self.forward([toks[-1]], pos)
                pos += 1
        return toks, margins

    def close(self) -> None:
        if self.m:
            lib().orc_model_destroy(self.m)
            self.m = None

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass
