"""An independent numpy float64 forward used to pin the C oracle's model path.

It follows the structure of the reference's own CPU check (scripts/verify-dense.mjs:
138-211): tokens are processed one at a time with per-layer Python lists of past keys and
values (no ring buffer, no batching), weights are F32 tensors read straight from the file
bytes, and the Gemma-3 body follows src/core/engine.ts:158-174. Small F32 GGUF variants
cover the branches the tiny model does not: biases, an ungated MLP, adjacent-pair and
partial RoPE, linear RoPE scaling, sliding windows, Q/K norm and Gemma's local/global
layers with post-norms and GeGLU.
"""
from __future__ import annotations

import math
from typing import Dict, List, Tuple

import numpy as np

from webgpu_amd import synth
from webgpu_amd.gguf import F32, model_config, parse_gguf_header


def _w(f: np.ndarray, g, name: str) -> np.ndarray:
    t = g.tensors[name]
    a = f[t.offset:t.offset + t.bytes].view(np.float32).astype(np.float64)
    return a.reshape(t.dims[::-1]) if len(t.dims) == 2 else a


def _rms(x, w, eps):
    return x / math.sqrt(float(np.mean(x * x)) + eps) * w


def _rotate(v: np.ndarray, pos: int, theta: float, scale: float, rot: int, adjacent: bool) -> np.ndarray:
    v = v.copy()
    for j in range(rot // 2):
        ang = pos * scale / theta ** (2 * j / rot)
        c, s = math.cos(ang), math.sin(ang)
        a, b = (2 * j, 2 * j + 1) if adjacent else (j, j + rot // 2)
        l, r = v[a], v[b]
        v[a], v[b] = l * c - r * s, l * s + r * c
    return v


def forward(f: np.ndarray, g, c, ids: List[int]) -> np.ndarray:
    gemma = c.family == "gemma3"
    H, hd, nh, nkv = c.hidden, c.headDim, c.heads, c.kvHeads
    grp = nh // nkv
    keys: List[List[np.ndarray]] = [[] for _ in range(c.layers)]
    vals: List[List[np.ndarray]] = [[] for _ in range(c.layers)]
    emb = _w(f, g, "token_embd.weight")
    logits = None
    for pos, tok in enumerate(ids):
        x = emb[tok].copy() * (math.sqrt(H) if gemma else 1.0)
        for l in range(c.layers):
            p = f"blk.{l}."
            local = c.period > 1 and l % c.period != c.period - 1
            h = _rms(x, _w(f, g, p + "attn_norm.weight"), c.epsilon)
            q = _w(f, g, p + "attn_q.weight") @ h
            k = _w(f, g, p + "attn_k.weight") @ h
            v = _w(f, g, p + "attn_v.weight") @ h
            if c.bias["q"]:
                q = q + _w(f, g, p + "attn_q.bias")
            if c.bias["k"]:
                k = k + _w(f, g, p + "attn_k.bias")
            if c.bias["v"]:
                v = v + _w(f, g, p + "attn_v.bias")
            qh, kh = q.reshape(nh, hd), k.reshape(nkv, hd)
            if gemma or c.qkNorm:
                qn, kn = _w(f, g, p + "attn_q_norm.weight"), _w(f, g, p + "attn_k_norm.weight")
                qh = np.stack([_rms(r, qn, c.epsilon) for r in qh])
                kh = np.stack([_rms(r, kn, c.epsilon) for r in kh])
            theta = c.localTheta if (gemma and local) else c.theta
            scale = 1.0 if (gemma and local) else c.ropeScale
            rot = hd if gemma else c.rotaryDim
            adjacent = c.rope == "norm"
            qh = np.stack([_rotate(r, pos, theta, scale, rot, adjacent) for r in qh])
            kh = np.stack([_rotate(r, pos, theta, scale, rot, adjacent) for r in kh])
            keys[l].append(kh)
            vals[l].append(v.reshape(nkv, hd))
            if gemma:
                window = c.window if local else 10 ** 9
            else:
                window = c.slidingWindow if c.slidingWindow > 0 else 10 ** 9
            first = max(0, pos + 1 - window)
            att = np.zeros((nh, hd))
            for hh in range(nh):
                K = np.stack([keys[l][t][hh // grp] for t in range(first, pos + 1)])
                V = np.stack([vals[l][t][hh // grp] for t in range(first, pos + 1)])
                s = K @ qh[hh] * c.attentionScale
                w = np.exp(s - s.max())
                att[hh] = (w / w.sum()) @ V
            proj = _w(f, g, p + "attn_output.weight") @ att.reshape(-1)
            if c.bias["output"]:
                proj = proj + _w(f, g, p + "attn_output.bias")
            x = x + (_rms(proj, _w(f, g, p + "post_attention_norm.weight"), c.epsilon) if gemma else proj)
            h = _rms(x, _w(f, g, p + "ffn_norm.weight"), c.epsilon)
            up = _w(f, g, p + "ffn_up.weight") @ h
            if c.ffnGate:
                gt = _w(f, g, p + "ffn_gate.weight") @ h
                if c.activation == "gelu":
                    act = 0.5 * gt * (1 + np.tanh(0.7978845608 * (gt + 0.044715 * gt ** 3)))
                else:
                    act = gt / (1 + np.exp(-gt))
                prod = act * up
            else:
                prod = up / (1 + np.exp(-up))
            down = _w(f, g, p + "ffn_down.weight") @ prod
            x = x + (_rms(down, _w(f, g, p + "post_ffw_norm.weight"), c.epsilon) if gemma else down)
        hN = _rms(x, _w(f, g, "output_norm.weight"), c.epsilon)
        head = _w(f, g, "output.weight") if "output.weight" in g.tensors else emb
        logits = head @ hN
    return logits


# ------------------------------------------------------------------ small F32 variants

def _file(meta, tensors: List[Tuple[str, List[int], np.ndarray]]) -> np.ndarray:
    entries = [(n, d, F32, "") for n, d, _ in tensors]
    offsets, off = [], 0
    for _, dims, _ in tensors:
        off = -(-off // 32) * 32
        offsets.append(off)
        off += int(np.prod(dims)) * 4
    header = synth._header(meta, entries, offsets)
    start = -(-len(header) // 32) * 32
    f = np.zeros(start + off, np.uint8)
    f[:len(header)] = np.frombuffer(header, np.uint8)
    for (_, dims, v), o in zip(tensors, offsets):
        b = v.astype(np.float32).view(np.uint8)
        f[start + o:start + o + b.size] = b
    return f


def variant_file(kind: str):
    rng = np.random.default_rng(sum(kind.encode()))
    H, nh, nkv, hd, F, V = 64, 4, 2, 16, 96, 80
    L = 7 if kind == "gemma3" else 2
    arch = {"llama-bias-gate": "llama", "qwen3-qknorm-partial": "qwen3", "gemma3": "gemma3"}[kind]
    qd, kd = nh * hd, nkv * hd
    T: List[Tuple[str, List[int], np.ndarray]] = []

    def mat(name, cols, rows, std=0.15):
        T.append((name, [cols, rows], rng.standard_normal(rows * cols) * std))

    def vec(name, n, center=1.0, spread=0.1):
        T.append((name, [n], center + rng.uniform(-spread, spread, n)))

    mat("token_embd.weight", H, V, 0.5)
    vec("output_norm.weight", H)
    if kind != "gemma3":
        mat("output.weight", H, V, 0.3)
    for l in range(L):
        p = f"blk.{l}."
        vec(p + "attn_norm.weight", H)
        mat(p + "attn_q.weight", H, qd)
        mat(p + "attn_k.weight", H, kd)
        mat(p + "attn_v.weight", H, kd)
        mat(p + "attn_output.weight", qd, H)
        if kind == "llama-bias-gate":
            vec(p + "attn_q.bias", qd, 0.0, 0.1)
            vec(p + "attn_k.bias", kd, 0.0, 0.1)
            vec(p + "attn_v.bias", kd, 0.0, 0.1)
            vec(p + "attn_output.bias", H, 0.0, 0.1)
        if kind != "llama-bias-gate":
            vec(p + "attn_q_norm.weight", hd)
            vec(p + "attn_k_norm.weight", hd)
        if kind == "gemma3":
            vec(p + "post_attention_norm.weight", H)
            vec(p + "post_ffw_norm.weight", H)
        vec(p + "ffn_norm.weight", H)
        if kind != "llama-bias-gate":
            mat(p + "ffn_gate.weight", H, F)
        mat(p + "ffn_up.weight", H, F)
        mat(p + "ffn_down.weight", F, H)
    meta = [("general.architecture", 8, arch), ("general.name", 8, kind),
            (f"{arch}.block_count", 4, L), (f"{arch}.context_length", 4, 4096),
            (f"{arch}.embedding_length", 4, H), (f"{arch}.feed_forward_length", 4, F),
            (f"{arch}.attention.head_count", 4, nh), (f"{arch}.attention.head_count_kv", 4, nkv),
            (f"{arch}.attention.key_length", 4, hd), (f"{arch}.attention.layer_norm_rms_epsilon", 6, 1e-5)]
    if kind == "llama-bias-gate":
        meta += [(f"{arch}.rope.freq_base", 6, 10000.0), (f"{arch}.rope.dimension_count", 4, 12),
                 (f"{arch}.attention.sliding_window", 4, 6)]
    elif kind == "qwen3-qknorm-partial":
        meta += [(f"{arch}.rope.freq_base", 6, 1e6), (f"{arch}.rope.dimension_count", 4, 8),
                 (f"{arch}.rope.scaling.type", 8, "linear"), (f"{arch}.rope.scaling.factor", 6, 2.0)]
    else:
        meta += [(f"{arch}.rope.freq_base", 6, 1e6), (f"{arch}.rope.local.freq_base", 6, 1e4),
                 (f"{arch}.attention.sliding_window", 4, 4)]
    f = _file(meta, T)
    g = parse_gguf_header(f, f.size)
    return f, g, model_config(g)
