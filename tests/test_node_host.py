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
    assert json.loads(r.stdout) == sorted(["create", "destroy", "adapterName", "memory", "done", "modelCreate",
                                           "modelTensor", "modelReady", "modelForward", "modelDecode", "modelSampling",
                                           "modelDestroy"])


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
