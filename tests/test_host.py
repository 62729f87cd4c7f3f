"""Host logic on the CPU: GGUF parsing, model configuration, context/KV-ring sizing and
the token loop, ported from the reference's node tests (tests/model-config.test.ts,
tests/context.test.ts, tests/gguf.test.ts), plus the C-ABI library's exports."""
import ctypes
import os
import re
import struct

import numpy as np
import pytest

from webgpu_amd import synth
from webgpu_amd.context import attention_memory, cache_copies, output_limit, validate_context
from webgpu_amd.engine import GenerationOptions, PagedEngine
from webgpu_amd.gguf import GGUF, NeedMore, Tensor, model_config, parse_gguf_header

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


# ---------------------------------------------------------------- model-config.test.ts:10-36
def dense_gguf(arch, bias=False, qk_norm=False, gate=True, full_kv=False) -> GGUF:
    hidden, heads, kvh, hd, layers, inter, vocab = 64, 4, 4 if full_kv else 2, 16, 2, 128, 96
    t = [("token_embd.weight", [hidden, vocab]), ("output_norm.weight", [hidden]), ("output.weight", [hidden, vocab])]
    for l in range(layers):
        p = f"blk.{l}."
        t += [(p + "attn_norm.weight", [hidden]), (p + "ffn_norm.weight", [hidden]),
              (p + "attn_q.weight", [hidden, heads * hd]), (p + "attn_k.weight", [hidden, kvh * hd]),
              (p + "attn_v.weight", [hidden, kvh * hd]), (p + "attn_output.weight", [heads * hd, hidden])]
        if bias:
            t += [(p + "attn_q.bias", [heads * hd]), (p + "attn_k.bias", [kvh * hd]), (p + "attn_v.bias", [kvh * hd])]
        if qk_norm:
            t += [(p + "attn_q_norm.weight", [hd]), (p + "attn_k_norm.weight", [hd])]
        if gate:
            t += [(p + "ffn_gate.weight", [hidden, inter])]
        t += [(p + "ffn_up.weight", [hidden, inter]), (p + "ffn_down.weight", [inter, hidden])]
    meta = {"general.architecture": arch, "general.name": f"{arch} test", f"{arch}.block_count": layers,
            f"{arch}.embedding_length": hidden, f"{arch}.attention.head_count": heads,
            f"{arch}.attention.head_count_kv": kvh, f"{arch}.attention.key_length": hd,
            f"{arch}.feed_forward_length": inter, f"{arch}.context_length": 8192}
    return GGUF(meta, {n: Tensor(n, d, 0, 0, 0, 0) for n, d in t}, 0, 0)


def test_llama3_selects_dense_decoder_full_context_no_qk_norm():
    c = model_config(dense_gguf("llama"))
    assert (c.family, c.layers, c.heads, c.kvHeads, c.headDim, c.rotaryDim, c.theta) == ("llama", 2, 4, 2, 16, 16, 10000)
    assert c.attentionScale == 0.25 and c.activation == "silu" and c.qkNorm is False
    assert c.bias == {"q": False, "k": False, "v": False, "output": False} and c.ffnGate is True
    assert c.period == 0 and c.rope == "norm" and c.slidingWindow == 0


def test_rope_scaling_and_sliding_windows_from_metadata():
    m = dense_gguf("llama")
    m.metadata.update({"llama.attention.sliding_window": 4096, "llama.rope.scaling.type": "linear",
                       "llama.rope.scaling.factor": 4})
    c = model_config(m)
    assert c.slidingWindow == 4096 and c.ropeScale == 0.25
    l31 = dense_gguf("llama")
    l31.metadata.update({"llama.rope.scaling.type": "llama3", "llama.rope.scaling.factor": 8})
    assert model_config(l31).ropeScale == 1
    q = dense_gguf("qwen2")
    q.metadata.update({"qwen2.rope.scaling.type": "linear", "qwen2.rope.scaling.factor": 2})
    assert model_config(q).ropeScale == 0.5


def test_bias_and_qk_norm_detected_from_tensors():
    q2 = model_config(dense_gguf("qwen2", bias=True))
    assert q2.bias == {"q": True, "k": True, "v": True, "output": False} and not q2.qkNorm and q2.rope == "neox"
    q3 = model_config(dense_gguf("qwen3", qk_norm=True))
    assert q3.qkNorm and q3.rope == "neox" and not any(q3.bias.values())


def test_ungated_mlp_detected():
    assert model_config(dense_gguf("llama", gate=False)).ffnGate is False


def test_validation_rejects_moe_bad_shapes_missing_tensors():
    moe = dense_gguf("llama")
    moe.tensors["blk.0.ffn_gate_inp.weight"] = Tensor("blk.0.ffn_gate_inp.weight", [64, 4], 0, 0, 0, 0)
    with pytest.raises(ValueError, match="Mixture-of-experts"):
        model_config(moe)
    bad = dense_gguf("llama")
    bad.tensors["blk.1.attn_v.weight"].dims = [64, 64]
    with pytest.raises(ValueError, match="attn_v"):
        model_config(bad)
    miss = dense_gguf("qwen2", bias=True)
    del miss.tensors["blk.1.attn_k.bias"]
    with pytest.raises(ValueError, match=r"attn_k\.bias"):
        model_config(miss)
    nonorm = dense_gguf("llama")
    del nonorm.tensors["blk.1.ffn_norm.weight"]
    with pytest.raises(ValueError, match="ffn_norm"):
        model_config(nonorm)
    with pytest.raises(ValueError, match="Supported text architectures"):
        model_config(dense_gguf("falcon"))


def test_key_length_fallback():
    g = dense_gguf("llama", full_kv=True)
    del g.metadata["llama.attention.key_length"], g.metadata["llama.attention.head_count_kv"]
    c = model_config(g)
    assert (c.headDim, c.kvHeads, c.rotaryDim) == (16, 4, 16)


@pytest.mark.parametrize("name", ["tiny", "qwen3-0.6b", "llama3-8b", "gemma3-27b"])
def test_synthetic_configs_match_the_measured_shapes(name):
    s = synth.SPECS[name]
    entries = synth.tensor_list(s)
    offsets = [0] * len(entries)
    hdr = synth._header(synth.metadata(s), entries, offsets)
    # Header-only parse: give the parser a file size that covers the data.
    g = parse_gguf_header(hdr, 1 << 62)
    c = model_config(g)
    assert (c.layers, c.hidden, c.heads, c.kvHeads, c.headDim, c.intermediate, c.vocab) == (
        s.layers, s.hidden, s.heads, s.kv_heads, s.head_dim, s.ffn, s.vocab)
    if name == "tiny":
        assert c.rope == "neox" and not c.qkNorm and c.epsilon == pytest.approx(1e-5) and c.theta == 10000
    if name == "llama3-8b":
        assert c.rope == "norm" and c.theta == 500000 and "output.weight" in g.tensors
    if name == "gemma3-27b":
        assert c.family == "gemma3" and c.period == 6 and c.window == 1024 and c.activation == "gelu"
        assert c.attentionScale == pytest.approx(1 / np.sqrt(5376 / 32))


# ---------------------------------------------------------------- gguf.test.ts / parseGGUFHeader
def test_header_rejects_bad_magic_version_and_truncation():
    with pytest.raises(ValueError, match="GGUF model"):
        parse_gguf_header(bytes(64), 64)
    v9 = struct.pack("<IIQQ", 0x46554747, 9, 0, 0)
    with pytest.raises(ValueError, match="version"):
        parse_gguf_header(v9, len(v9))
    f = synth.build("tiny")
    with pytest.raises(NeedMore):
        parse_gguf_header(f[:100], f.size)
    with pytest.raises(ValueError, match="Truncated"):
        parse_gguf_header(f, f.size - 64)
    g = parse_gguf_header(f, f.size)
    t = g.tensors["blk.1.ffn_down.weight"]
    assert t.dims == [128, 64] and t.rowBytes == 512 and t.offset % 32 == 0 and g.dataOffset % 32 == 0


# ---------------------------------------------------------------- context.test.ts:8-67
def test_context_limits():
    for n in (256, 4096, 12000, 32768):
        validate_context(n)
    for n in (255, 32769, 4096.5, float("nan")):
        with pytest.raises(ValueError, match="Context must"):
            validate_context(n)
    with pytest.raises(ValueError, match="model declares"):
        validate_context(32768, 8192)
    assert output_limit(32768, 100, 32768) == 32668
    assert output_limit(8192, 24000, 32768) == 8192
    assert output_limit(8192, 32767, 32768) == 1
    with pytest.raises(ValueError, match="prompt has"):
        output_limit(8192, 32768, 32768)
    with pytest.raises(ValueError, match="maxTokens"):
        output_limit(32769, 100, 32768)


class _Cfg:
    def __init__(self, **kw):
        self.__dict__.update(kw)


def test_gemma_local_rings_keep_window_for_whole_batch_including_wrap():
    c = _Cfg(family="gemma3", layers=6, period=6, window=1024, kvHeads=4, headDim=128, slidingWindow=1024)
    m = attention_memory(c, 32768, 128)
    assert m["capacities"] == [1151] * 5 + [32768]
    assert m["totalBytes"] == (5 * 1151 + 32768) * 4 * 128 * 8
    capacity, window, batch = 136, 129, 8
    for start in (128, 135, 136, 2047, 32760):
        ring = [-1] * capacity
        for t in range(max(0, start - capacity), start):
            ring[t % capacity] = t
        for cp in cache_copies(start, batch, capacity):
            for j in range(cp["count"]):
                ring[cp["target"] + j] = start + cp["source"] + j
        for b in range(batch):
            for t in range(max(0, start + b + 1 - window), start + b + 1):
                assert ring[t % capacity] == t


def test_llama_allocates_full_context():
    c = _Cfg(family="llama", layers=3, period=0, window=0, kvHeads=2, headDim=16, slidingWindow=0)
    m = attention_memory(c, 4096, 8)
    assert m["capacities"] == [4096] * 3 and m["kvBytes"] == 3 * 4096 * 2 * 16 * 8


def test_token_loop_runs_to_the_exact_context_boundary():
    """context.test.ts:55-67 with forward mocked: 1000-token prompt, 4096 context."""
    eng = PagedEngine()
    positions = []
    eng.context, eng.batch, eng.model, eng.kvCapacities = 4096, 128, object(), [4096]

    def fwd(ids, start, logits=False):
        positions.append(start + len(ids) - 1)

    def fwd_argmax(ids, start):
        positions.append(start + len(ids) - 1)
        return 0

    def decode(token, start, count):
        positions.extend(range(start, start + count))
        return [0] * count
    eng.forward, eng.forward_argmax, eng.decode = fwd, fwd_argmax, decode
    eng.stats = lambda: {}
    eng.set_sampling = lambda *a: None
    count = 0
    for ev in eng.generate([0] * 1000, GenerationOptions(temperature=0, maxTokens=32768)):
        count += 1
        assert ev.promptTokens == 1000 and ev.contextLength == 4096
    assert count == 3096 and max(positions) == 4094
    assert not eng.busy


def _scripted_engine(context, batch, caps):
    eng = PagedEngine()
    eng.context, eng.batch, eng.model, eng.kvCapacities = context, batch, object(), caps
    counts = []
    eng.forward = lambda ids, start, logits=False: None
    eng.forward_argmax = lambda ids, start: 7

    def decode(token, start, count):
        counts.append(count)
        return [7] * count
    eng.decode = decode
    eng.stats = lambda: {}
    eng.set_sampling = lambda *a: None
    return eng, counts


def test_device_chunks_stay_within_the_sliding_ring_slack():
    # a ring of window + batch - 1 slots survives at most `batch` positions written past
    # the cached prefix, so a model with one decodes at most `batch` tokens per chunk
    eng, counts = _scripted_engine(256, 8, [31, 256])
    assert len(list(eng.generate([1, 2, 3], GenerationOptions(temperature=0, maxTokens=100)))) == 100
    assert max(counts) == 8
    eng, counts = _scripted_engine(256, 8, [256, 256])
    list(eng.generate([1, 2, 3], GenerationOptions(temperature=0, maxTokens=100)))
    assert max(counts) == 32


def test_abort_signal_stops_generation_and_drops_the_prefix():
    from webgpu_amd.engine import AbortError, AbortSignal
    eng, _ = _scripted_engine(512, 16, [512])
    sig = AbortSignal()
    got = []
    with pytest.raises(AbortError, match="Stopped by user"):
        for ev in eng.generate([1, 2, 3], GenerationOptions(temperature=0, maxTokens=50), signal=sig):
            got.append(ev.token)
            if len(got) == 3:
                sig.abort()
    assert len(got) == 3 and eng.tokensInCache == [] and not eng.busy


def test_generation_options_are_validated_like_the_reference():
    eng, _ = _scripted_engine(512, 16, [512])
    for bad in (dict(temperature=-1), dict(temperature=2.5), dict(topK=0), dict(topK=201),
                dict(topP=0), dict(topP=1.5), dict(temperature=float("nan"))):
        with pytest.raises(ValueError, match="Invalid sampling settings"):
            eng.generate([1], GenerationOptions(**bad))
    with pytest.raises(ValueError, match="maxTokens"):
        eng.generate([1], GenerationOptions(temperature=0, maxTokens=0))


def test_an_unstarted_generation_leaves_the_engine_free():
    eng, _ = _scripted_engine(512, 16, [512])
    eng.generate([1, 2], GenerationOptions(temperature=0, maxTokens=4))   # never iterated
    assert not eng.busy
    assert len(list(eng.generate([1, 2], GenerationOptions(temperature=0, maxTokens=4)))) == 4


def test_load_options_follow_the_performance_presets():
    from webgpu_amd.engine import LoadOptions
    eng = PagedEngine()
    with pytest.raises(ValueError, match="Performance must be"):
        eng.load(b"\0" * 64, LoadOptions(performance="turbo"))
    for mode, batch in (("lite", 8), ("low-memory", 16), ("fast", 128)):
        eng = PagedEngine()
        with pytest.raises(ValueError):   # not a GGUF: fails after the options are taken
            eng.load(b"\0" * 64, LoadOptions(performance=mode))
        assert eng.batch == batch and eng.performance == mode
    eng = PagedEngine()
    with pytest.raises(ValueError):
        eng.load(b"\0" * 64, LoadOptions(performance="lite", batchSize=64))
    assert eng.batch == 64


def test_generate_rejects_concurrent_and_unloaded_use():
    eng = PagedEngine()
    with pytest.raises(RuntimeError, match="Load a model"):
        eng.generate([1, 2])
    eng.model, eng.busy = object(), True
    with pytest.raises(RuntimeError, match="already running"):
        eng.generate([1, 2])


# ---------------------------------------------------------------- the C ABI library
def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(os.path.join(ROOT, "webgpu_amd", "libwgd.so"))
    header = open(os.path.join(ROOT, "include", "wgd.h")).read()
    names = sorted(set(re.findall(r"^\s*(?:[\w ]+\*?\s*)\b(wgd_\w+)\(", header, re.M)))
    assert len(names) >= 36
    for n in names:
        assert hasattr(lib, n), f"libwgd.so does not export {n}"


def test_python_bindings_cover_the_header():
    from webgpu_amd.gpu import SIGNATURES
    header = open(os.path.join(ROOT, "include", "wgd.h")).read()
    names = set(re.findall(r"^\s*(?:[\w ]+\*?\s*)\b(wgd_\w+)\(", header, re.M))
    assert names == set(SIGNATURES)


def test_create_without_a_device_reports_an_error():
    """No GPU here: wgd_create must fail with a message, not crash."""
    if os.path.exists("/dev/kfd"):
        pytest.skip("a device is present")
    from webgpu_amd.gpu import Compute, WgdError
    with pytest.raises(WgdError, match="HIP device|No HIP"):
        Compute().init()
