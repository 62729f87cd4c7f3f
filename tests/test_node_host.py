"""The Node host over the N-API addon (webgpu_amd/node): the reference's own runtime
(src/core is TypeScript on Node) driving libwgd.

CPU: the addon loads in Node and exports the engine surface; the Node GGUF parser,
modelConfig and attentionMemory agree with the Python mirror on the same file. GPU: the
tiny check:dense model through PagedEngine.load/forward/generate under Node matches the
float64 oracle (logits within 1e-3 max-relative, identical greedy tokens), as the smoke
check does through the Python host.
"""
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

from webgpu_amd import synth
from webgpu_amd.gguf import model_config, parse_gguf_header

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ADDON = os.path.join(ROOT, "webgpu_amd", "node", "wgd_napi.node")
RUNNER = os.path.join(ROOT, "tests", "node", "engine_run.mjs")
NODE = shutil.which("node")

needs_node = pytest.mark.skipif(NODE is None or not os.path.exists(ADDON), reason="node or the built addon is missing")


def run_node(*args, timeout=120):
    r = subprocess.run([NODE, RUNNER, *map(str, args)], capture_output=True, text=True, timeout=timeout)
    assert r.returncode == 0, r.stderr[-3000:]
    return json.loads(r.stdout.strip().splitlines()[-1])


@needs_node
def test_node_generate_rules_without_a_device():
    r = subprocess.run([NODE, os.path.join(ROOT, "tests", "node", "engine_rules.mjs")],
                       capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr[-3000:]
    out = json.loads(r.stdout.strip().splitlines()[-1])
    assert out["slidingTokens"] == 100 and out["slidingMaxChunk"] == 8 and out["fullMaxChunk"] == 32
    assert out["abortError"] == "AbortError" and out["abortSeen"] == 3
    assert out["abortCache"] == 0 and out["abortBusy"] is False
    assert out["invalid"] == ["Invalid sampling settings."] * 5


@pytest.fixture(scope="module")
def tiny_file(tmp_path_factory):
    f = synth.build("tiny")
    path = tmp_path_factory.mktemp("gguf") / "tiny.gguf"
    f.tofile(str(path))
    return str(path), f


@needs_node
def test_addon_exports_engine_surface():
    code = f"const a = require({json.dumps(ADDON)}); console.log(JSON.stringify(Object.keys(a).sort()))"
    r = subprocess.run([NODE, "-e", code], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    assert json.loads(r.stdout) == sorted(NODE_EXPORTS)


# One binding per C-ABI entry point of include/wgd.h (the measurement helpers
# wgd_probe_read, wgd_model_attention_timing and wgd_matvec_shapes, and the
# wgd_last_error/size getters folded into thrown errors aside).
NODE_EXPORTS = ["create", "destroy", "adapterName", "memory", "done", "modelCreate", "modelTensor", "modelReady",
                "modelForward", "modelDecode", "modelSampling", "modelDestroy", "bufferCreate", "bufferDestroy",
                "bufferSize", "uploadWeights", "write", "read", "copy", "clear", "matmul", "quantizedBytes",
                "quantize", "matvec", "dequant", "norm", "ropeNorm", "ropeNeox", "ropeAdjacent", "attention",
                "attentionNoalloc", "attentionF16kv", "kvStoreF16", "add", "silu", "gelu", "biasAdd", "activate",
                "argmax", "sample", "embed"]


@needs_node
def test_addon_launchers_check_their_handles_without_a_device():
    from webgpu_amd.gpu import lib
    code = (f"const a = require({json.dumps(ADDON)});"
            "const grab = (f) => { try { f(); return null; } catch (e) { return [e.code, e.message]; } };"
            "console.log(JSON.stringify({qx: a.quantizedBytes(4096), noCtx: grab(() => a.clear({}, {})),"
            " args: grab(() => a.matmul(null)), neg: grab(() => a.quantizedBytes(-1))}))")
    r = subprocess.run([NODE, "-e", code], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    out = json.loads(r.stdout)
    assert out["qx"] == lib().wgd_quantized_bytes(4096)
    assert out["noCtx"] == ["WGD_E_STATE", "The GPU context was disposed."]
    assert out["args"] == ["WGD_E_INVALID", "missing arguments"]
    assert out["neg"][0] == "WGD_E_INVALID"


@needs_node
def test_node_gguf_config_matches_python(tiny_file):
    path, f = tiny_file
    got = run_node(path, "config")
    g = parse_gguf_header(f, f.size)
    c = model_config(g)
    for key in ("architecture", "family", "hidden", "intermediate", "layers", "heads", "kvHeads", "headDim", "vocab",
                "rotaryDim", "window", "period", "slidingWindow", "rope", "qkNorm", "ffnGate", "activation", "maxContext"):
        assert got["config"][key] == getattr(c, key), key
    for key in ("epsilon", "theta", "localTheta", "attentionScale", "ropeScale"):
        assert got["config"][key] == pytest.approx(getattr(c, key), rel=1e-12), key
    assert got["config"]["bias"] == c.bias
    assert got["dataOffset"] == g.dataOffset
    assert {t[0]: t[1:] for t in got["tensors"]} == {n: [t.type, t.offset, t.bytes] for n, t in g.tensors.items()}


@needs_node
def test_node_rejects_a_non_gguf_file(tmp_path):
    p = tmp_path / "x.bin"
    p.write_bytes(b"\0" * 64)
    r = subprocess.run([NODE, RUNNER, str(p), "config"], capture_output=True, text=True, timeout=60)
    assert r.returncode != 0 and "Select a GGUF model file." in r.stderr


@pytest.mark.gpu
@needs_node
def test_node_engine_tiny_greedy_matches_oracle(tiny_file):
    from oracle import orc
    from webgpu_amd.context import attention_memory
    path, f = tiny_file
    g = parse_gguf_header(f, f.size)
    c = model_config(g)
    ids = synth.prompt_ids(c.vocab, 8)
    got = run_node(path, "greedy", ",".join(map(str, ids)), 4, timeout=300)
    ora = orc.OracleModel(f, g, c, 512, attention_memory(c, 512, 128)["capacities"])
    try:
        want = ora.forward(ids, 0)
        expected, _ = ora.greedy(ids, 4)
    finally:
        ora.close()
    logits = np.asarray(got["logits"], np.float64)
    err = float(np.abs(logits - want).max() / np.abs(want).max())
    assert err <= 1e-3, err
    assert got["tokens"] == list(expected)


@needs_node
@pytest.mark.gpu
def test_node_and_python_hosts_sample_the_same_tokens(tiny_file):
    # both hosts set the same device token pick: one seed, one sequence
    from webgpu_amd.engine import GenerationOptions, LoadOptions, PagedEngine
    path, f = tiny_file
    c = model_config(parse_gguf_header(f, f.size))
    ids = synth.prompt_ids(c.vocab, 8)
    got = run_node(path, "greedy", ",".join(map(str, ids)), 24, "1.1:987654321", timeout=300)
    eng = PagedEngine()
    eng.load(path, LoadOptions(contextLength=512, batchSize=128))
    try:
        want = [e.token for e in eng.generate(ids, GenerationOptions(maxTokens=24, temperature=1.1, seed=987654321))]
    finally:
        eng.dispose()
    assert got["tokens"] == want and len(want) == 24


@needs_node
def test_node_runtime_api_rules_without_a_device():
    # sdk.mjs + worker.mjs with a scripted engine in the worker thread
    r = subprocess.run([NODE, os.path.join(ROOT, "tests", "node", "sdk_rules.mjs")], capture_output=True, text=True,
                       timeout=60)
    assert r.returncode == 0, r.stderr[-3000:]
    out = json.loads(r.stdout.strip().splitlines()[-1])
    assert out["noModel"] == ["Error", "Load a model first."]
    assert out["badLoad"] == ["Error", "Unsupported GGUF version."]
    assert out["info"]["fileBytes"] == 123 and out["progress"] == [0.5]
    assert out["tokens"] == [0, 1, 2, 3, 4] and out["first"] == 0
    assert out["busy"] == ["Error", "The runtime is busy."]
    assert out["stopped"] == ["AbortError", "Stopped by user"]
    assert out["afterStop"] == 3 and out["afterBreak"] == 4
    assert out["pending"] == ["Error", "Runtime disposed."]
    assert out["disposed"] == ["Error", "This runtime was disposed. Create a new WebGPU instance."]


@needs_node
@pytest.mark.gpu
def test_node_runtime_api_drives_the_engine(tiny_file):
    from webgpu_amd.engine import GenerationOptions, LoadOptions, PagedEngine
    path, f = tiny_file
    c = model_config(parse_gguf_header(f, f.size))
    ids = synth.prompt_ids(c.vocab, 8)
    r = subprocess.run([NODE, os.path.join(ROOT, "tests", "node", "sdk_run.mjs"), path, ",".join(map(str, ids)), "6"],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-3000:]
    got = json.loads(r.stdout.strip().splitlines()[-1])
    eng = PagedEngine()
    eng.load(path, LoadOptions(contextLength=512, batchSize=128))
    try:
        want = [e.token for e in eng.generate(ids, GenerationOptions(maxTokens=6, temperature=0))]
    finally:
        eng.dispose()
    assert got == {"batchSize": 128, "tokens": want}


@needs_node
@pytest.mark.gpu
def test_node_launchers_match_oracle(tmp_path):
    """Every buffer and kernel binding of the addon, driven from Node, against the float64
    oracle (matmul/norm/rope/attention bars of verify.ts:11 and verify-context.ts:39; exact
    for dequant, embedding and the token picks)."""
    from oracle import orc
    from webgpu_amd.gguf import Q4_K
    rng = np.random.default_rng(5)
    cols, rows, batch, eps = 512, 72, 9, 1e-6
    w = synth.q4k_blocks(rng, rows * cols // 256, 0.05)
    x = rng.standard_normal((batch + 1) * cols).astype(np.float32)
    nw = (1 + 0.1 * rng.standard_normal(cols)).astype(np.float32)
    n, nb = 256, 3
    xn, wn = rng.standard_normal(n * nb).astype(np.float32), rng.standard_normal(n).astype(np.float32)
    rope = dict(heads=4, hd=64, start=37, theta=10000.0, rot=32, batch=2)
    rope_x = rng.standard_normal(rope["heads"] * rope["hd"] * rope["batch"]).astype(np.float32)
    rope_w = (1 + 0.1 * rng.standard_normal(rope["hd"])).astype(np.float32)
    e = 1000
    g, u = rng.standard_normal(e).astype(np.float32), rng.standard_normal(e).astype(np.float32)
    bias = rng.standard_normal(24).astype(np.float32)
    att = dict(heads=8, kvHeads=2, hd=128, start=300, scale=0.088, window=100, capacity=120, context=4096, batch=5)
    q = rng.standard_normal(att["batch"] * att["heads"] * att["hd"]).astype(np.float32)
    k = rng.standard_normal(att["capacity"] * att["kvHeads"] * att["hd"]).astype(np.float32)
    v = rng.standard_normal(att["capacity"] * att["kvHeads"] * att["hd"]).astype(np.float32)
    vocab = 5000
    logits = rng.standard_normal(vocab).astype(np.float32)
    logits[[10, 20]] = [np.nan, np.inf]
    sample = dict(temperature=0.9, topK=40, topP=0.9, seedHi=3, seedLo=123456789, index=77)
    table = rng.standard_normal(10 * 64).astype(np.float32)
    ids = np.array([3, 9, 0], np.int32)
    files = dict(w=w, x=x, nw=nw, xn=xn, wn=wn, rope_x=rope_x, rope_w=rope_w, g=g, u=u, bias=bias, q=q, k=k, v=v,
                 logits=logits, table=table, ids=ids)
    for name, arr in files.items():
        np.ascontiguousarray(arr).tofile(str(tmp_path / f"{name}.bin"))
    spec = dict(matmul=dict(type=Q4_K, cols=cols, rows=rows, batch=batch), eps=eps, norm=dict(n=n, batch=nb),
                rope=rope, elementwise=dict(n=e, width=24), attention=att, vocab=vocab, sample=sample,
                embed=dict(hidden=64, n=3, scale=1.0))
    (tmp_path / "spec.json").write_text(json.dumps(spec))
    r = subprocess.run([NODE, os.path.join(ROOT, "tests", "node", "kernels_run.mjs"), str(tmp_path)],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-3000:]
    res = json.loads(r.stdout.strip().splitlines()[-1])
    got = lambda name, dt=np.float32: np.fromfile(str(tmp_path / f"{name}.out.bin"), dt)

    def near(a, want, tol=1e-3, label=""):
        want = np.asarray(want, np.float64)
        err = np.abs(a.astype(np.float64) - want)
        assert np.all(np.isfinite(a)) and np.all(err <= tol * np.maximum(1.0, np.abs(want))), (label, err.max())

    stride, base = rows + 3, 2
    want = orc.matmul(Q4_K, w, x, cols, rows, stride, base, 1, batch)
    gemm = got("gemm")
    for b in range(batch):
        near(gemm[b * stride + base: b * stride + base + rows], want[b * stride + base: b * stride + base + rows],
             label="gemm")
    near(got("matvec_raw"), orc.matmul(Q4_K, w, x, cols, rows, rows, 0, 0, 1), label="matvec")
    normed = orc.norm(x[:cols], nw, eps).astype(np.float32)
    near(got("matvec_normed"), orc.matmul(Q4_K, w, normed, cols, rows, rows, 0, 0, 1), label="normed matvec")
    assert np.array_equal(got("dequant").view(np.uint32), orc.dequant(w, Q4_K, rows * cols).view(np.uint32))
    near(got("norm"), np.concatenate([orc.norm(xn[i * n:(i + 1) * n], wn, eps) for i in range(nb)]), label="norm")
    args = (rope["heads"], rope["hd"], rope["start"], rope["theta"], 1.0)
    near(got("rope_norm"), orc.rope(rope_x, rope_w, *args, eps, 0, rope["batch"], 0), label="rope norm")
    near(got("rope_neox"), orc.rope(rope_x, None, *args, 0, rope["rot"], rope["batch"], 1), label="rope neox")
    near(got("rope_adjacent"), orc.rope(rope_x, None, *args, 0, 0, rope["batch"], 2), label="rope adjacent")
    g64, u64 = g.astype(np.float64), u.astype(np.float64)
    silu = g64 / (1 + np.exp(-g64)) * u64
    gelu = 0.5 * g64 * (1 + np.tanh(0.7978845608 * (g64 + 0.044715 * g64 ** 3))) * u64
    near(got("silu"), silu, 1e-5, "silu")
    near(got("gelu"), gelu, 1e-5, "gelu")
    near(got("add"), u64 + g64, 1e-6, "add")
    biased = (u + g).astype(np.float64) + np.tile(bias, e // 24 + 1)[:e]
    near(got("bias_add"), biased, 1e-6, "bias")
    ba = got("bias_add").astype(np.float64)
    near(got("activate"), ba / (1 + np.exp(-ba)), 1e-5, "activate")
    want_att = orc.attention(q, k, v, att["heads"], att["kvHeads"], att["hd"], att["start"], att["scale"],
                             att["window"], att["capacity"], att["batch"])
    assert np.abs(got("attention") - want_att).max() <= 1e-3
    assert np.array_equal(got("attention"), got("attention_noalloc"))
    picks = got("picks", np.int32).tolist()
    best = orc.argmax(logits)
    drawn = orc.sample(logits, 0.9, 40, 0.9, orc.uniform((3 << 32) | 123456789, 77))
    assert picks == [best, best, drawn]
    assert np.array_equal(got("embed"), table.reshape(10, 64)[ids].ravel())
    errs = res["errors"]
    assert errs["overrun"][0] == "WGD_E_INVALID" and "range outside buffer" in errs["overrun"][1]
    assert errs["badType"][0] == "WGD_E_INVALID"
    assert errs["negative"] == ["WGD_E_INVALID", "n must be an integer in [0, 2^32)"]
    assert errs["wrongHandle"] == ["WGD_E_INVALID", "expected a live buffer of this context"]
    assert errs["destroyed"] == ["WGD_E_INVALID", "expected a live buffer of this context"]
    assert errs["bufferSize"] == rows * 4 and errs["memory"] is True


@needs_node
@pytest.mark.gpu
def test_node_engine_qwen3_0_6b_prompt_and_greedy_tokens(tmp_path):
    """Qwen3-0.6B through the Node engine: the 64-token prompt of the whole-workload fixture,
    then 12 greedy tokens; logits after the prompt within 1e-3 max-relative of the oracle's
    and tokens identical to the fixture's first 12."""
    z = np.load(os.path.join(ROOT, "tests", "golden", "model_qwen3-0.6b.npz"), allow_pickle=False)
    path = tmp_path / "qwen3-0.6b.gguf"
    synth.build("qwen3-0.6b").tofile(str(path))
    prompt = [int(t) for t in z["prompt"]]
    got = run_node(str(path), "greedy", ",".join(map(str, prompt)), 12, timeout=600)
    logits = np.asarray(got["logits"], np.float64)
    err = float(np.abs(logits - z["first_logits"]).max() / np.abs(z["first_logits"]).max())
    print(f"\nnode qwen3-0.6b: logits max-rel {err:.2e}, tokens {got['tokens']}", flush=True)
    assert err <= 1e-3
    assert got["tokens"] == [int(t) for t in z["tokens"][:12]]
