"""Device sampling (sample.hip) against the oracle's restatement of sample()
(src/core/engine.ts:305-324): the same token for the same logits, settings and uniform
(the index-th output of splitmix64(seed)), bit-exact, over vocabulary sizes of real models,
ties, non-finite logits and rows where thousands of logits share one value. Then the
model's token pick: graph decode, eager steps and the oracle on the device's own logits
agree, and a seeded generation repeats itself."""
import numpy as np
import pytest

from oracle import orc
from tests import qvariants
from webgpu_amd import synth
from webgpu_amd.engine import GenerationOptions, LoadOptions, PagedEngine
from webgpu_amd.gpu import WgdError, WGD_E_INVALID, WGD_E_NONFINITE

pytestmark = pytest.mark.gpu


def _cases():
    rng = np.random.default_rng(17)
    yield "normal-1000", (rng.standard_normal(1000) * 2).astype(np.float32), 0.7, 40, 0.9
    yield "vocab-151936", (rng.standard_normal(151936) * 3).astype(np.float32), 0.8, 40, 0.95
    yield "vocab-262144-k200", (rng.standard_normal(262144) * 2).astype(np.float32), 1.0, 200, 1.0
    yield "rounded-ties", np.round(rng.standard_normal(5000) * 2).astype(np.float32), 1.0, 200, 1.0
    yield "all-equal", np.full(5000, 0.25, np.float32), 1.0, 200, 0.5
    yield "one-binade", (0.5 + 0.5 * rng.random(50000)).astype(np.float32), 0.3, 200, 0.99
    l = (rng.standard_normal(3000)).astype(np.float32)
    l[rng.integers(0, 3000, 40)] = np.nan
    l[rng.integers(0, 3000, 20)] = np.inf
    l[rng.integers(0, 3000, 20)] = -np.inf
    yield "non-finite", l, 0.5, 10, 0.8
    yield "signed-zeros", np.array([0.0, -0.0, -1.0, 0.0, -0.0, -3.0], np.float32), 2.0, 4, 1.0
    yield "one", np.array([-5.0], np.float32), 0.7, 40, 0.9
    yield "fewer-than-k", np.array([1.0, np.nan, 2.0, 2.0, -1.0, np.inf, 0.5], np.float32), 1.2, 40, 0.9


@pytest.mark.parametrize("name,logits,t,k,p", list(_cases()), ids=[c[0] for c in _cases()])
def test_device_sample_matches_the_oracle(gpu, name, logits, t, k, p):
    buf = gpu.upload(logits, "logits")
    try:
        seed = 0x5EED + len(logits)
        got = [gpu.sample(buf, logits.size, t, k, p, seed, i) for i in range(40)]
        want = [orc.sample(logits, t, k, p, orc.uniform(seed, i)) for i in range(40)]
        assert got == want, name
        assert gpu.sample(buf, logits.size, 0.0, k, p, seed, 0) == orc.sample(logits, 0.0, k, p, 0.0)
    finally:
        gpu.destroy(buf)


def test_device_sample_rejects_what_the_reference_rejects(gpu):
    buf = gpu.upload(np.array([1.0, 2.0], np.float32), "logits")
    bad = gpu.upload(np.array([np.nan, np.inf, -np.inf], np.float32), "bad")
    try:
        for t, k, p in ((-0.1, 40, 0.9), (2.5, 40, 0.9), (0.7, 0, 0.9), (0.7, 201, 0.9), (0.7, 40, 0.0), (0.7, 40, 1.5)):
            with pytest.raises(WgdError) as e:
                gpu.sample(buf, 2, t, k, p, 1, 0)
            assert e.value.status == WGD_E_INVALID
        with pytest.raises(WgdError) as e:
            gpu.sample(bad, 3, 0.7, 40, 0.9, 1, 0)
        assert e.value.status == WGD_E_NONFINITE
    finally:
        gpu.destroy(buf)
        gpu.destroy(bad)


@pytest.mark.parametrize("kind", ["qwen2-bias", "llama-q5q4"])
def test_model_sampling_graph_eager_and_oracle_agree(kind):
    f, g, c = qvariants.build(kind)
    eng = PagedEngine()
    eng.load(f, LoadOptions(contextLength=256, batchSize=64))
    try:
        ids = synth.prompt_ids(c.vocab, 30, seed=4)
        t, k, p, seed = 1.3, 60, 0.97, 123456789
        eng.set_sampling(t, k, p, seed)
        first = eng.forward_argmax(ids, 0)
        dev = eng.decode(first, 30, 24)                  # one graph replay per token
        # eager steps from the same prefix: the token at position q uses uniform(seed, q)
        eng.forward_argmax(ids, 0)
        tok, eager = first, []
        for i in range(24):
            logits = eng.forward([tok], 30 + i, True)
            nxt = eng.forward_argmax([tok], 30 + i)
            assert nxt == orc.sample(logits, t, k, p, orc.uniform(seed, 31 + i)), (kind, i)
            eager.append(nxt)
            tok = nxt
        assert dev == eager
        assert first == orc.sample(eng.forward(ids, 0, True), t, k, p, orc.uniform(seed, 30))
        eng.set_sampling(0.0)
        assert eng.forward_argmax(ids, 0) == int(np.argmax(eng.forward(ids, 0, True)))
    finally:
        eng.dispose()


def test_seeded_generation_repeats():
    f, g, c = qvariants.build("qwen2-bias", tokenizer=True)
    eng = PagedEngine()
    eng.load(f, LoadOptions(contextLength=256, batchSize=64))
    try:
        msgs = [{"role": "user", "content": "hello world"}]
        a = [e.token for e in eng.generate(msgs, GenerationOptions(maxTokens=40, seed=99))]
        b = [e.token for e in eng.generate(msgs, GenerationOptions(maxTokens=40, seed=99))]
        assert a == b and len(a) >= 1
    finally:
        eng.dispose()
