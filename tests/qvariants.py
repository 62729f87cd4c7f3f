"""Small quantized GGUF variants for the GPU parity tests: the planar-weight prompt path
(grouped GEMMs and their fused finishes) and the quantized decode path under model features
the three shaped decoders do not use.

* ``qwen2-bias``: Q/K/V biases, half-split RoPE, SwiGLU (gguf.ts:168-170 detects the bias).
* ``llama-partial``: adjacent-pair RoPE over 32 of 64 dims, Q/K/V and output biases, an
  ungated FFN (SiLU of up), a sliding window.
* ``qwen3-mixed``: Q/K norm, partial rotary with linear RoPE scaling, and a Q8_0 K
  projection beside Q4_K Q and Q6_K V (three weight types: the Q/K/V group falls back to
  one launch per matrix).
* ``llama-q5q4``: the Q5_K_M / Q4_0 mixes of real files: Q5_K Q, K, gate, up and head,
  Q6_K V (one Q/K/V launch of two types), Q4_0 O, down and embedding table.
* ``qwen3-f16``: every matrix F16 (the GGUF row-major layout: the F16 decode matvec and
  the generic prompt GEMM), with Q/K norm.
* ``llama-q80-w96``: every matrix Q8_0 at hidden width 96, which is not a whole 64-column
  tile: the matrices reading the hidden state keep the GGUF layout, so decode runs the
  generic step (batched kernels at one token, the position read from device state).
* ``llama-xcd``: Q4_K with a Q6_K V at hidden 1024, 16 query x 128 and 8 KV heads, FFN 2048:
  the widths at which the prompt finishes (Q/K/V, GLU, residual) and the decode attention
  merge take their work by the XCD that wrote the partials (head dim 128, a multiple of 8
  head slots and of 8 KV heads, hidden and FFN multiples of 1024).

Dimensions (but for ``llama-q80-w96``) are the smallest the planar K-quant kernels take: hidden 256 (Q4_K/Q6_K rows of
whole 256-element blocks), 4 query heads x 64, 2 KV heads, FFN 512, vocab 300. Matrix blocks
come from the synthetic generators (webgpu_amd/synth.py); norm and bias vectors are f32.
"""
from typing import List, Tuple

import numpy as np

from webgpu_amd import synth
from webgpu_amd.gguf import F16, F32, Q4_0, Q4_K, Q5_K, Q6_K, Q8_0, QUANTS, model_config, parse_gguf_header
from webgpu_amd.tokenizer import byte_alphabet

KINDS = ("qwen2-bias", "llama-partial", "qwen3-mixed", "llama-q5q4", "qwen3-f16", "llama-q80-w96", "llama-xcd")


CHAT_SPECIALS = ["<|im_start|>", "<|im_end|>", "<|endoftext|>"]
CHAT_MERGES = ["h e", "he l", "hel l", "hell o", "Ġ w", "Ġw o", "Ġwo r", "Ġwor l", "Ġworl d", "u s", "us e", "use r"]


def _tokenizer_meta(vocab: int):
    """A byte-level BPE vocabulary of ``vocab`` entries with ChatML control tokens: the 256
    single-byte symbols, a few merges, the specials, then unused fillers."""
    tokens = [*byte_alphabet(), *["".join(m.split(" ")) for m in CHAT_MERGES], *CHAT_SPECIALS]
    tokens += [f"<unused{i}>" for i in range(vocab - len(tokens))]
    types = [1] * (256 + len(CHAT_MERGES)) + [3] * (vocab - 256 - len(CHAT_MERGES))
    return [("tokenizer.ggml.model", 8, "gpt2"), ("tokenizer.ggml.pre", 8, "qwen2"),
            ("tokenizer.ggml.tokens", 9, (8, tokens)), ("tokenizer.ggml.merges", 9, (8, CHAT_MERGES)),
            ("tokenizer.ggml.token_type", 9, (5, types)),
            ("tokenizer.ggml.eos_token_id", 4, tokens.index("<|im_end|>")),
            ("tokenizer.chat_template", 8, "{% for m in messages %}<|im_start|>{{ m.role }}\n{{ m.content }}<|im_end|>\n{% endfor %}")]


def build(kind: str, tokenizer: bool = False):
    """(file bytes, parsed header, model config) of variant ``kind``; with ``tokenizer`` the
    file also carries a byte-level BPE vocabulary with a ChatML template."""
    rng = np.random.default_rng(sum(kind.encode()) * 31 + 5)
    H, nh, nkv, hd, F, V, L = 256, 4, 2, 64, 512, 300, 2
    if kind == "llama-xcd":
        H, nh, nkv, hd, F = 1024, 16, 8, 128, 2048
    w96 = kind == "llama-q80-w96"
    if w96:
        H = 96
    arch = {"qwen2-bias": "qwen2", "llama-partial": "llama", "qwen3-mixed": "qwen3", "llama-q5q4": "llama",
            "qwen3-f16": "qwen3", "llama-q80-w96": "llama", "llama-xcd": "llama"}[kind]
    qd, kd = nh * hd, nkv * hd
    T: List[Tuple[str, List[int], int, np.ndarray]] = []

    def mat(name, cols, rows, typ, std=0.05):
        nb = rows * cols // QUANTS[typ]["block"]
        gen = {Q4_K: synth.q4k_blocks, Q6_K: synth.q6k_blocks, Q8_0: synth.q8_0_blocks,
               Q5_K: synth.q5k_blocks, Q4_0: synth.q4_0_blocks, F16: synth.f16_values}[typ]
        T.append((name, [cols, rows], typ, gen(rng, nb, std)))

    def vec(name, n, center=1.0, spread=0.1):
        v = (center + rng.uniform(-spread, spread, n)).astype(np.float32)
        T.append((name, [n], F32, v.view(np.uint8)))

    q5, f16 = kind == "llama-q5q4", kind == "qwen3-f16"
    mat("token_embd.weight", H, V, Q4_0 if q5 else F16 if f16 else Q8_0 if w96 else Q6_K, 0.5)
    vec("output_norm.weight", H)
    mat("output.weight", H, V, Q5_K if q5 else F16 if f16 else Q8_0 if w96 else Q6_K, 0.3)
    k_type = Q8_0 if kind in ("qwen3-mixed", "llama-q80-w96") else Q5_K if q5 else F16 if f16 else Q4_K
    big, small = (Q5_K, Q4_0) if q5 else (F16, F16) if f16 else (Q8_0, Q8_0) if w96 else (Q4_K, Q4_K)
    v_type = F16 if f16 else Q8_0 if w96 else Q6_K
    for l in range(L):
        p = f"blk.{l}."
        vec(p + "attn_norm.weight", H)
        mat(p + "attn_q.weight", H, qd, big)
        mat(p + "attn_k.weight", H, kd, k_type)
        mat(p + "attn_v.weight", H, kd, v_type)
        mat(p + "attn_output.weight", qd, H, small)
        if kind in ("qwen2-bias", "llama-partial"):
            vec(p + "attn_q.bias", qd, 0.0, 0.2)
            vec(p + "attn_k.bias", kd, 0.0, 0.2)
            vec(p + "attn_v.bias", kd, 0.0, 0.2)
        if kind == "llama-partial":
            vec(p + "attn_output.bias", H, 0.0, 0.1)
        if kind in ("qwen3-mixed", "qwen3-f16"):
            vec(p + "attn_q_norm.weight", hd)
            vec(p + "attn_k_norm.weight", hd)
        vec(p + "ffn_norm.weight", H)
        if kind != "llama-partial":
            mat(p + "ffn_gate.weight", H, F, big)
        mat(p + "ffn_up.weight", H, F, big)
        mat(p + "ffn_down.weight", F, H, small)
    meta = [("general.architecture", 8, arch), ("general.name", 8, kind),
            (f"{arch}.block_count", 4, L), (f"{arch}.context_length", 4, 4096),
            (f"{arch}.embedding_length", 4, H), (f"{arch}.feed_forward_length", 4, F),
            (f"{arch}.attention.head_count", 4, nh), (f"{arch}.attention.head_count_kv", 4, nkv),
            (f"{arch}.attention.key_length", 4, hd), (f"{arch}.attention.value_length", 4, hd),
            (f"{arch}.attention.layer_norm_rms_epsilon", 6, 1e-5)]
    if kind == "qwen2-bias":
        meta += [(f"{arch}.rope.freq_base", 6, 1e6), (f"{arch}.rope.dimension_count", 4, hd)]
    elif kind == "llama-partial":
        meta += [(f"{arch}.rope.freq_base", 6, 1e4), (f"{arch}.rope.dimension_count", 4, 32),
                 (f"{arch}.attention.sliding_window", 4, 24)]
    elif kind in ("llama-q5q4", "llama-q80-w96", "llama-xcd"):
        meta += [(f"{arch}.rope.freq_base", 6, 5e5), (f"{arch}.rope.dimension_count", 4, hd)]
    else:
        meta += [(f"{arch}.rope.freq_base", 6, 1e6), (f"{arch}.rope.dimension_count", 4, 48),
                 (f"{arch}.rope.scaling.type", 8, "linear"), (f"{arch}.rope.scaling.factor", 6, 2.0)]
    if tokenizer:
        meta += _tokenizer_meta(V)
    entries = [(n, d, t, "") for n, d, t, _ in T]
    offsets, off = [], 0
    for _, dims, typ, _ in T:
        off = -(-off // 32) * 32
        offsets.append(off)
        off += synth.tensor_bytes(dims, typ)
    header = synth._header(meta, entries, offsets)
    start = -(-len(header) // 32) * 32
    f = np.zeros(start + -(-off // 32) * 32, np.uint8)
    f[:len(header)] = np.frombuffer(header, np.uint8)
    for (_, _, _, data), o in zip(T, offsets):
        f[start + o:start + o + data.size] = data
    g = parse_gguf_header(f, f.size)
    return f, g, model_config(g)
