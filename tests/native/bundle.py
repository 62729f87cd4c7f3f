"""Writes a model bundle for the sanitizer drivers (oracle_san, wgd_san): a synthetic
GGUF's tensors with both model configs, the KV capacities and a prompt, in a flat
little-endian file the C/C++ drivers parse without a GGUF reader of their own.

Layout: "WGDB", u32 version 1; u32 size + bytes of the oracle config; u32 size + bytes of
wgd_model_config; u32 layers, i32 capacities[layers]; u32 n, i32 prompt[n]; u32 chunk;
u32 steps; u32 tensors, then per tensor: u32 name length, name, i32 type, u32 n_dims,
u64 dims[n_dims], u64 bytes, the raw GGUF bytes.
"""
from __future__ import annotations

import struct

from oracle import orc
from webgpu_amd import synth
from webgpu_amd.context import attention_memory
from webgpu_amd.engine import _config_struct
from webgpu_amd.gguf import model_config, parse_gguf_header


def write_bundle(path: str, name: str, context: int, chunk: int, prompt_len: int, steps: int, seed: int = 7):
    f = synth.build(name)
    g = parse_gguf_header(f, f.size)
    c = model_config(g)
    caps = list(attention_memory(c, context, chunk)["capacities"])
    ocfg = orc.config_struct(g, c, context)
    wcfg = _config_struct(c, context, chunk)
    wcfg.tied_output = 0 if "output.weight" in g.tensors else 1
    ids = synth.prompt_ids(c.vocab, prompt_len, seed)
    out = bytearray(b"WGDB" + struct.pack("<I", 1))
    for s in (ocfg, wcfg):
        b = bytes(s)
        out += struct.pack("<I", len(b)) + b
    out += struct.pack("<I", c.layers) + struct.pack(f"<{c.layers}i", *caps)
    out += struct.pack("<I", prompt_len) + struct.pack(f"<{prompt_len}i", *ids)
    out += struct.pack("<II", chunk, steps)
    tensors = list(g.tensors.values())
    out += struct.pack("<I", len(tensors))
    for t in tensors:
        nm = t.name.encode()
        out += struct.pack("<I", len(nm)) + nm + struct.pack("<iI", t.type, len(t.dims))
        out += struct.pack(f"<{len(t.dims)}Q", *t.dims) + struct.pack("<Q", t.bytes)
        out += f[t.offset:t.offset + t.bytes].tobytes()
    with open(path, "wb") as fh:
        fh.write(out)
    return f, g, c, caps, ids
