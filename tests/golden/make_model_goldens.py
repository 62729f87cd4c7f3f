"""Writes the whole-workload greedy fixtures ``tests/golden/model_<name>.npz``.

Runs in the build container only (the f64 oracle on the host cores; the 8B case takes
tens of minutes). For each seeded synthetic GGUF it records what the reference's greedy
loop produces (src/core/engine.ts:284-298, scripts/verify-dense.mjs:281-286): the prompt
prefilled in 128-token batches, then free-running greedy tokens, each step's top-2 margin
and max|logit|, and the full logits after the prompt and at the last step. A fixture also
holds an xxh64 of the GGUF bytes, so a change to the generator fails loudly instead of
comparing against another model.

Identical greedy tokens are only a fair demand where the oracle's choice is not within
the logits tolerance: a step whose top-2 margin is below 1e-3 * max|logit| could flip
under any implementation that meets that tolerance. So prompt seeds are tried in order
from 7, a seed is dropped at its first such step, and the fixture keeps the first seed
whose every step clears the tolerance, with the dropped seeds listed.

At the 8B shape one oracle attempt costs 10-20 minutes and most seeds meet a step inside
the tolerance within 256 tokens (seeds 7-10 did, at steps 52, 30, 85 and 250). Its prompt
seeds were therefore screened first on the device (the engine's own logits, every step's
top-2 margin at least 1.15e-3 of max|logit| over the 512 + 256 tokens; 5 of seeds 11-1499
passed: 236, 613, 739, 864, 1321), and the oracle then confirms the screened seeds given
with --seeds, in order: the fixture is still the oracle's tokens and margins. The seed is
a screened one, so the 8B token identity holds on a seed chosen for its margins.

A free-running run that settles on one repeated token tests little beyond a fixed point,
and a margin screen favours exactly those runs (a repeated token wins by a wide margin).
So the tied-head shapes use signed output norms (see webgpu_amd/synth.py), and their seeds
were screened on the device for both the margins (1.3e-3) and diversity: Qwen3-0.6B, at
least 64 distinct tokens in 256 (4 of seeds 7-399 passed: 62, 314, 334, 397); Gemma at 1280
tokens, 24 of 32 (10 of seeds 7-39, the first 7, 8, 9); Gemma at 8192 tokens, 36 of 48 (6 of
seeds 7-39, the first 12, 17, 25). The oracle then confirms them in the order given with
--seeds (397, 314, 334 / 7, 8, 9 / 12, 17, 25). The fixture records the distinct count.

    python tests/golden/make_model_goldens.py [name ...] [--seeds 613,739]
"""
import os
import sys
import time

import numpy as np
import xxhash

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import orc  # noqa: E402
from webgpu_amd import synth  # noqa: E402
from webgpu_amd.context import attention_memory  # noqa: E402
from webgpu_amd.gguf import model_config, parse_gguf_header  # noqa: E402

# name -> (synthetic model, prompt tokens, greedy tokens, context)
WORKLOADS = {
    "qwen3-0.6b": ("qwen3-0.6b", 64, 256, 1024),
    "gemma3-27b-6l": ("gemma3-27b-6l", 1280, 32, 1536),
    # the Gemma-3-27B workload's own prompt (8192 tokens in 64 batches) at full width over
    # six layers, the sixth global: its attention reads every prompt key
    "gemma3-27b-6l-8k": ("gemma3-27b-6l", 8192, 48, 8448),
    "llama3-8b": ("llama3-8b", 512, 256, 1024),
}
CHUNK = 128
MARGIN = 1e-3   # the logits tolerance, relative to max|logit|
FIRST_SEED, MAX_SEEDS = 7, 24
HERE = os.path.dirname(os.path.abspath(__file__))


def file_hash(f: np.ndarray) -> str:
    return xxhash.xxh64(memoryview(f)).hexdigest()


def run(ora, c, name: str, pseed: int, prompt_len: int, steps: int, t0: float):
    """The greedy run for one prompt seed, or None at its first step inside the tolerance."""
    ids = synth.prompt_ids(c.vocab, prompt_len, pseed)
    logits = None
    for i in range(0, prompt_len, CHUNK):
        part = ids[i:i + CHUNK]
        logits = ora.forward(part, i, logits=i + len(part) == prompt_len)
    print(f"{name} seed {pseed}: prompt of {prompt_len} done ({time.time() - t0:.0f} s)", flush=True)
    first_logits = logits.astype(np.float32)
    toks, margins, maxabs = [], [], []
    pos = prompt_len
    for s in range(steps):
        order = np.argsort(-logits, kind="stable")
        top = int(order[0])
        assert top == int(np.argmax(logits))
        toks.append(top)
        margins.append(float(logits[order[0]] - logits[order[1]]))
        maxabs.append(float(np.abs(logits).max()))
        if margins[-1] < MARGIN * maxabs[-1]:
            print(f"{name} seed {pseed}: step {s} margin {margins[-1] / maxabs[-1]:.2e} of max|logit|; "
                  f"next seed ({time.time() - t0:.0f} s)", flush=True)
            return None
        if s + 1 < steps:
            logits = ora.forward([top], pos)
            pos += 1
        if s % 32 == 31:
            print(f"{name} seed {pseed}: token {s + 1}/{steps} ({time.time() - t0:.0f} s)", flush=True)
    return ids, toks, margins, maxabs, first_logits, logits.astype(np.float32)


def make(name: str, seeds=None) -> str:
    model, prompt_len, steps, context = WORKLOADS[name]
    t0 = time.time()
    f = synth.build(model)
    g = parse_gguf_header(f, f.size)
    c = model_config(g)
    caps = attention_memory(c, context, CHUNK)["capacities"]
    rejected = []
    got = None
    for pseed in seeds or range(FIRST_SEED, FIRST_SEED + MAX_SEEDS):
        # a fresh oracle per seed: its rings start empty, as a freshly loaded engine's do
        ora = orc.OracleModel(f, g, c, context, caps)
        try:
            got = run(ora, c, name, pseed, prompt_len, steps, t0)
        finally:
            ora.close()
        if got is not None:
            break
        rejected.append(pseed)
    if got is None:
        raise RuntimeError(f"{name}: no prompt seed in {MAX_SEEDS} clears the margin")
    ids, toks, margins, maxabs, first_logits, last_logits = got
    rel = np.array(margins) / np.array(maxabs)
    out = os.path.join(HERE, f"model_{name}.npz")
    np.savez_compressed(out, name=name, model=model, gguf_xxh64=file_hash(f), prompt_seed=pseed,
                        rejected_seeds=np.array(rejected), distinct=len(set(toks)),
                        prompt_len=prompt_len, steps=steps, context=context, chunk=CHUNK,
                        prompt=np.array(ids, np.int32), tokens=np.array(toks, np.int32), margins=np.array(margins),
                        maxabs=np.array(maxabs), first_logits=first_logits, last_logits=last_logits)
    print(f"{name}: wrote {out}; prompt seed {pseed} (dropped {rejected}); {len(set(toks))} distinct tokens "
          f"{toks[:12]}...; "
          f"min relative top-2 margin {rel.min():.3e} at step {int(rel.argmin())}; {time.time() - t0:.0f} s", flush=True)
    return out


if __name__ == "__main__":
    args = sys.argv[1:]
    seeds = None
    if "--seeds" in args:
        i = args.index("--seeds")
        seeds = [int(v) for v in args[i + 1].split(",")]
        del args[i:i + 2]
    for n in args or list(WORKLOADS):
        make(n, seeds)
