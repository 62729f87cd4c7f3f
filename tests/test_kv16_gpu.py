"""The f16 K/V ring option on the MI355X, against the float64 oracle.

The reference keeps its K/V rings in f32 (src/core/engine.ts:98-101). With an f16 ring
every cached key and value is rounded to the nearest binary16 value (ties to even) when it
is stored and widened exactly when it is read; scores, softmax and the weighted sum stay
f32. The oracle restates the same rounding (orc_round_f16, pinned against numpy's IEEE
conversion in tests/test_oracle.py), so the f16 path is held to the f32 path's tolerances:
absolute 1e-3 for long-context attention (verify-context.ts:39), 1e-4 for prompt batches,
logits within 1e-3 max-relative and identical greedy tokens for whole models.
"""
import numpy as np
import pytest

from oracle import orc
from webgpu_amd import synth
from webgpu_amd.context import attention_memory
from webgpu_amd.engine import GenerationOptions, LoadOptions, PagedEngine
from webgpu_amd.gguf import model_config, parse_gguf_header
from webgpu_amd.gpu import WgdError

pytestmark = pytest.mark.gpu


def to_ring16(gpu, values: np.ndarray, name: str):
    """An f16 ring holding `values` through wgd_kv_store_f16 (the cacheKV copy)."""
    src = gpu.upload(values.astype(np.float32), name + " f32")
    ring = gpu.buffer(values.size * 2, name)
    gpu.kv_store_f16(src, ring, values.size)
    gpu.destroy(src)
    return ring


def test_kv_store_f16_rounds_to_nearest_even(gpu):
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(20000) * 10.0 ** rng.integers(-8, 5, 20000)).astype(np.float32)
    # ties between neighbouring halves, the subnormal range, the largest half and overflow
    h = np.arange(1, 2048, dtype=np.uint16).view(np.float16).astype(np.float32)
    ties = ((h[:-1].astype(np.float64) + h[1:]) / 2).astype(np.float32)
    special = np.array([65504, 65519, 65520, 1e5, -1e5, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26, 0.0, -0.0], np.float32)
    x = np.concatenate([x, ties, special])
    src = gpu.upload(x, "src")
    # a copy split at a wrap: the tail of the values into the ring's head, at element offsets
    ring = gpu.buffer((x.size + 100) * 2, "ring")
    gpu.kv_store_f16(src, ring, x.size - 37, 37, 100)
    gpu.kv_store_f16(src, ring, 37, 0, 0)
    got = np.frombuffer(gpu.read(ring, (x.size + 100) * 2), np.uint16)
    with np.errstate(over="ignore"):  # values past the f16 range round to infinity, as intended
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got[100:100 + x.size - 37], want[37:]) and np.array_equal(got[:37], want[:37])
    with pytest.raises(WgdError):
        gpu.kv_store_f16(src, ring, x.size, 0, 101)  # one half past the ring
    for b in (src, ring):
        gpu.destroy(b)


@pytest.mark.parametrize("context,start,batch,window,capacity,hd", [
    (4096, 2047, 3, 4096, 4096, 128), (32768, 32765, 3, 32768, 32768, 256), (32768, 32765, 1, 32768, 32768, 128),
    (32768, 32760, 8, 129, 136, 128), (4096, 4000, 2, 300, 301, 512)])
def test_attention_f16kv_long_context_and_ring(gpu, context, start, batch, window, capacity, hd):
    heads, kvh = 4, 2
    rng = np.random.default_rng(start + hd)
    q = (rng.standard_normal(batch * heads * hd) * 3).astype(np.float32)
    k = rng.standard_normal(capacity * kvh * hd).astype(np.float32)
    v = rng.standard_normal(capacity * kvh * hd).astype(np.float32)
    qb, yb = gpu.upload(q, "q"), gpu.buffer(q.nbytes, "y")
    kb, vb = to_ring16(gpu, k, "k16"), to_ring16(gpu, v, "v16")
    gpu.attention_f16kv(qb, kb, vb, yb, heads, kvh, hd, start, 1 / np.sqrt(hd), window, capacity, context, batch)
    got = gpu.read_f32(yb, q.size)
    k16, v16 = k.astype(np.float16).astype(np.float64), v.astype(np.float16).astype(np.float64)
    want = orc.attention(q, k16, v16, heads, kvh, hd, start, 1 / np.sqrt(hd), window, capacity, batch)
    err = np.abs(got - want).max()
    assert np.all(np.isfinite(got)) and err <= 1e-3, f"max abs error {err:.3e}"
    for b in (qb, yb, kb, vb):
        gpu.destroy(b)


# prompt batches: the matrix-core kernel (head_dim 64/128/256) and the generic one (96)
@pytest.mark.parametrize("heads,kvh,hd,start,batch,window,capacity", [
    (32, 8, 128, 384, 128, 4096, 1024), (16, 2, 256, 50, 20, 24, 128), (8, 2, 64, 1000, 48, 200, 256),
    (8, 4, 96, 30, 40, 4096, 128)])
def test_prompt_attention_f16kv_batches(gpu, heads, kvh, hd, start, batch, window, capacity):
    rng = np.random.default_rng(start + batch)
    q = rng.standard_normal(batch * heads * hd).astype(np.float32) * 2
    k = rng.standard_normal(capacity * kvh * hd).astype(np.float32)
    v = rng.standard_normal(capacity * kvh * hd).astype(np.float32)
    qb, yb = gpu.upload(q, "q"), gpu.buffer(q.nbytes, "y")
    kb, vb = to_ring16(gpu, k, "k16"), to_ring16(gpu, v, "v16")
    scale = 1 / np.sqrt(hd)
    gpu.attention_f16kv(qb, kb, vb, yb, heads, kvh, hd, start, scale, window, capacity, capacity, batch)
    got = gpu.read_f32(yb, q.size)
    want = orc.attention(q, k.astype(np.float16).astype(np.float64), v.astype(np.float16).astype(np.float64),
                         heads, kvh, hd, start, scale, window, capacity, batch)
    err = np.abs(got - want).max()
    assert np.all(np.isfinite(got)) and err <= 1e-4, f"max abs error {err:.3e}"
    for b in (qb, yb, kb, vb):
        gpu.destroy(b)


def max_rel(got, want):
    return float(np.abs(np.asarray(got, np.float64) - want).max() / np.abs(want).max())


def check_kv16_model(name, prompt_len, steps, context, chunk, seed=7):
    """Prompt in chunks, then teacher-forced decode steps, both on f16 rings, against the
    oracle with the same rings: logits within 1e-3 and equal greedy tokens at every step;
    then the device decode loop (captured graph) repeats the eager tokens."""
    f = synth.build(name)
    g = parse_gguf_header(f, f.size)
    c = model_config(g)
    caps = attention_memory(c, context, chunk)["capacities"]
    eng = PagedEngine()
    eng.load(f, LoadOptions(contextLength=context, batchSize=chunk, kvCacheType="f16"))
    ora = orc.OracleModel(f, g, c, context, caps, kv_f16=True)
    try:
        ids = synth.prompt_ids(c.vocab, prompt_len, seed)
        for i in range(0, prompt_len, chunk):
            part = ids[i:i + chunk]
            last = i + len(part) == prompt_len
            want = ora.forward(part, i, logits=last)
            got = eng.forward(part, i, last)
        errs, toks = [max_rel(got, want)], []
        for s in range(steps):
            tok = int(np.argmax(want))
            assert int(np.argmax(got)) == tok, f"{name} f16 KV step {s}: GPU token {int(np.argmax(got))} vs oracle {tok}"
            toks.append(tok)
            if s + 1 < steps:
                want = ora.forward([tok], prompt_len + s)
                got = eng.forward([tok], prompt_len + s, True)
                errs.append(max_rel(got, want))
        print(f"\n{name} f16 KV: max-rel logits error {max(errs):.3e}, tokens {toks[:8]}", flush=True)
        assert max(errs) <= 1e-3, f"{name} f16 KV: logits max-rel error {max(errs):.3e}"
        # the same continuation from the device decode loop after a fresh prefill
        eng.reset()
        events = list(eng.generate(ids, GenerationOptions(temperature=0, maxTokens=steps)))
        assert [e.token for e in events] == toks
        return eng
    finally:
        ora.close()
        eng.dispose()


@pytest.mark.parametrize("name,prompt,steps,context,chunk", [
    ("qwen3-0.6b", 64, 16, 512, 128),    # head_dim 128: MFMA prompt attention, 16-byte-lane decode kernel
    ("mini-gemma3", 40, 8, 256, 8),      # local rings of 23 slots wrapped inside the prompt, head_dim 64
    ("mini-llama", 20, 8, 256, 8)])      # head_dim 32: the generic prompt and decode kernels
def test_model_f16_kv_cache_matches_the_oracle(name, prompt, steps, context, chunk):
    check_kv16_model(name, prompt, steps, context, chunk, seed=8 if name.startswith("mini") else 7)


def test_f16_kv_cache_halves_the_rings():
    f = synth.build("tiny")
    sizes = {}
    for kv in ("f32", "f16"):
        eng = PagedEngine()
        eng.load(f, LoadOptions(contextLength=2048, batchSize=8, kvCacheType=kv))
        sizes[kv] = eng.stats()["gpuBytes"]
        eng.dispose()
    c = model_config(parse_gguf_header(f, f.size))
    ring_f32 = attention_memory(c, 2048, 8)["kvBytes"]
    assert ring_f32 == 2 * attention_memory(c, 2048, 8, 2)["kvBytes"]
    assert sizes["f32"] - sizes["f16"] == ring_f32 // 2
    with pytest.raises(ValueError):
        PagedEngine().load(f, LoadOptions(kvCacheType="bf16"))
