"""Parity of the quantized model variants (tests/qvariants.py) on the MI355X against the
float64 oracle: two prompt batches (the planar-weight GEMM path with its fused Q/K/V,
GLU and residual finishes, or its per-matrix fallback) then greedy decode steps on the
quantized matvec path. Same contract as the shaped decoders: logits within 1e-3
max-relative error and greedy tokens identical, with no exception for small margins. The
prompt seed is the first from 3 whose oracle steps all have a top-2 margin of at least the
logits tolerance (1e-3 max|logit|), the rule the whole-workload fixtures follow, so an
identical token is a fair demand at every step.
"""
import numpy as np
import pytest

from oracle import orc
from tests import qvariants
from webgpu_amd import synth
from webgpu_amd.context import attention_memory
from webgpu_amd.engine import LoadOptions, PagedEngine

pytestmark = pytest.mark.gpu
LOGIT_TOL = 1e-3


def max_rel(got, want):
    return float(np.abs(np.asarray(got, np.float64) - want).max() / np.abs(want).max())


def oracle_run(f, g, c, context, caps, batch, seed, steps):
    """The oracle's prompt (batches of `batch`) and greedy steps for one prompt seed: the ids,
    the logits after the prompt and after each step, the tokens and the smallest top-2 margin
    relative to max|logit|."""
    ora = orc.OracleModel(f, g, c, context, caps)
    try:
        ids = synth.prompt_ids(c.vocab, 100, seed=seed)
        for i in range(0, len(ids), batch):  # batches of 64 and 36 tokens
            part = ids[i:i + batch]
            want = ora.forward(part, i, logits=i + len(part) == len(ids))
        logits, toks, worst, pos = [want], [], np.inf, len(ids)
        for s in range(steps):
            order = np.argsort(-want, kind="stable")
            toks.append(int(order[0]))
            worst = min(worst, float(want[order[0]] - want[order[1]]) / float(np.abs(want).max()))
            if s + 1 < steps:
                want = ora.forward([toks[-1]], pos)
                logits.append(want)
                pos += 1
        return ids, logits, toks, worst
    finally:
        ora.close()


@pytest.mark.parametrize("kind", qvariants.KINDS)
def test_quantized_variant_prefill_and_decode(kind):
    f, g, c = qvariants.build(kind)
    context, batch, steps = 256, 64, 5
    caps = attention_memory(c, context, batch)["capacities"]
    for seed in range(3, 40):
        ids, wants, toks, worst = oracle_run(f, g, c, context, caps, batch, seed, steps)
        if worst >= LOGIT_TOL:
            break
    assert worst >= LOGIT_TOL, f"{kind}: no prompt seed in 3-39 whose oracle margins clear the tolerance"
    eng = PagedEngine()
    eng.load(f, LoadOptions(contextLength=context, batchSize=batch))
    try:
        for i in range(0, len(ids), batch):
            part = ids[i:i + batch]
            got = eng.forward(part, i, i + len(part) == len(ids))
        errs, pos = [], len(ids)
        for s in range(steps):
            errs.append(max_rel(got, wants[s]))
            assert int(np.argmax(got)) == toks[s], \
                f"{kind} seed {seed} step {s}: GPU token {int(np.argmax(got))} vs oracle {toks[s]}"
            if s + 1 < steps:
                got = eng.forward([toks[s]], pos, True)
                pos += 1
        print(f"\n{kind}: prompt seed {seed}, min oracle margin {worst:.2e} of max|logit|, "
              f"max-rel logits error {max(errs):.3e}, tokens {toks}")
        assert max(errs) <= LOGIT_TOL, f"{kind}: logits max-rel error {max(errs):.3e}"
    finally:
        eng.dispose()


@pytest.mark.parametrize("kind", ["llama-partial", "qwen3-mixed", "llama-q5q4", "qwen3-f16", "llama-q80-w96", "llama-xcd"])
def test_quantized_variant_graph_decode_matches_eager(kind):
    # the captured per-token graph (quantized matvecs, fused decode attention) against one
    # eager forward per token from the same prefix
    f, g, c = qvariants.build(kind)
    eng = PagedEngine()
    eng.load(f, LoadOptions(contextLength=256, batchSize=64))
    try:
        ids = synth.prompt_ids(c.vocab, 30, seed=9)
        first = eng.forward_argmax(ids, 0)
        dev = eng.decode(first, 30, 40)  # positions 30..69 pass the sliding window of 24
        eager, tok = [], first
        for i in range(40):
            tok = eng.forward_argmax([tok], 30 + i)
            eager.append(tok)
        assert dev == eager
    finally:
        eng.dispose()


def test_generate_from_chat_messages():
    # the text front-end end to end: the GGUF's own byte-level BPE vocabulary and ChatML
    # framing turn messages into the prompt; the greedy continuation equals the oracle's
    # on the same ids, and each event's text is the decode of the tokens so far
    from webgpu_amd.engine import GenerationOptions
    f, g, c = qvariants.build("qwen2-bias", tokenizer=True)
    eng = PagedEngine()
    eng.load(f, LoadOptions(contextLength=256, batchSize=64))
    ora = orc.OracleModel(f, g, c, 256, attention_memory(c, 256, 64)["capacities"])
    try:
        tok = eng.tokenizer
        assert tok is not None and tok.style == "chatml"
        messages = [{"role": "user", "content": "hello world, user"}]
        ids = tok.chat(messages)
        events = list(eng.generate(messages, GenerationOptions(temperature=0, maxTokens=8)))
        want, logits, pos = [], ora.forward(ids, 0), len(ids)
        for _ in range(8):
            t = int(np.argmax(logits))
            if t in tok.eos:
                break
            want.append(t)
            logits = ora.forward([t], pos)
            pos += 1
        assert [e.token for e in events] == want
        for i, e in enumerate(events):
            assert e.text == tok.decode(want[:i + 1]) and e.promptTokens == len(ids)
    finally:
        ora.close()
        eng.dispose()


def test_sliding_ring_survives_a_turn_that_ends_inside_a_device_chunk():
    # window 24, batch 8: rings of 31 slots. The first turn ends at an end-of-turn token
    # early in a device chunk, whose later positions were already written; the second
    # turn continues the cached prefix and must equal a recompute from scratch.
    from types import SimpleNamespace
    from webgpu_amd.engine import GenerationOptions
    f, g, c = qvariants.build("llama-partial")
    eng = PagedEngine()
    eng.load(f, LoadOptions(contextLength=256, batchSize=8))
    try:
        assert max(eng.kvCapacities) == 31
        ids = synth.prompt_ids(c.vocab, 30, seed=21)
        free = SimpleNamespace(eos=set(), decode=lambda t: "")
        gen = [e.token for e in eng.generate(ids, GenerationOptions(temperature=0, maxTokens=12), tokenizer=free)]
        stop = gen[2]
        turn = SimpleNamespace(eos={stop}, decode=lambda t: "")
        eng.reset()
        first = [e.token for e in eng.generate(ids, GenerationOptions(temperature=0, maxTokens=40), tokenizer=turn)]
        assert first == gen[:gen.index(stop)]
        follow = ids + first + [stop, 5, 6, 7, 8]
        cached = [e.token for e in eng.generate(follow, GenerationOptions(temperature=0, maxTokens=20), tokenizer=free)]
        eng.reset()
        fresh = [e.token for e in eng.generate(follow, GenerationOptions(temperature=0, maxTokens=20), tokenizer=free)]
        assert cached == fresh
    finally:
        eng.dispose()


def test_runtime_api_drives_the_engine_on_its_worker_thread():
    # the sdk.ts surface end to end: load, a two-turn chat that reuses the prefix, a
    # stopped reply, reset, dispose
    from webgpu_amd.engine import AbortError, GenerationOptions
    from webgpu_amd.runtime import WebGPU
    f, g, c = qvariants.build("qwen2-bias", tokenizer=True)
    rt = WebGPU()
    ref = PagedEngine()
    try:
        info = rt.load(f, LoadOptions(contextLength=256, performance="fast"))
        assert info.batchSize == 128 and info.performance == "fast" and info.fileBytes == f.size
        turn1 = [{"role": "user", "content": "hello world"}]
        a = list(rt.generate(turn1, GenerationOptions(temperature=0, maxTokens=6)))
        turn2 = turn1 + [{"role": "assistant", "content": a[-1].text if a else ""},
                         {"role": "user", "content": "hello user"}]
        b = [e.token for e in rt.generate(turn2, GenerationOptions(temperature=0, maxTokens=6))]
        ref.load(f, LoadOptions(contextLength=256, batchSize=128))
        assert [e.token for e in a] == [e.token for e in ref.generate(turn1, GenerationOptions(temperature=0, maxTokens=6))]
        assert b == [e.token for e in ref.generate(turn2, GenerationOptions(temperature=0, maxTokens=6))]
        it = rt.generate(turn1, GenerationOptions(temperature=0, maxTokens=200))
        next(it, None)
        rt.stop()
        try:
            rest, stopped = list(it), False
        except AbortError:
            stopped = True
        assert stopped or len(rest) + 1 < 200   # else the reply had ended at its end-of-turn token
        rt.reset()
    finally:
        rt.dispose()
        ref.dispose()
