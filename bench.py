"""Decode throughput of the dense-decoder token loop on one MI355X, with the Q4_K
dequant-matvec roofline and the float64 CPU path timed beside it.

Workload: the Llama-3-8B-shaped random-init Q4_K_M GGUF (32 layers, hidden 4096, 32/8
heads, FFN 14336, vocab 128256; Q4_K attention/FFN, Q6_K attn_v and output). A 512-token
prompt is prefilled in 128-token batches (dequant-GEMM on MFMA), then W warmup and K
timed greedy decode steps run on the device (one HIP-graph replay per token). A step is
one token: forward of one token through every layer plus the head and argmax.

roofline: the Q4_K dequant-matvec at the 14336x4096 FFN shape (ne0 = 14336 inputs,
4096 outputs), timed with a HIP event pair around every launch on the library's stream,
rotating 24 distinct weight copies (~800 MB, far beyond the 256 MB Infinity Cache) so the
bytes come from HBM. achieved = algorithmic bytes (weights + 4*in + 4*out) / mean launch
time. traffic = HBM bytes per launch from the committed rocprofv3 counter summary of the
same microbench (profiles/k_mv_matvec_microbench.md). The other microbench shapes (4096x4096,
4096x14336 Q4_K; 4096x128256 Q6_K) are reported under "matvec".

prefill_tok_s: the 512-token prompt after one untimed pass, median of three passes.
prefill_gemm: the prompt-batch dequant-GEMM at the 8B layer shapes with 128 tokens as
single-matrix wgd_matmul calls (input split, GEMM and split-K reduction), timed with HIP
events; its MFMA utilisation counts the three bf16 MFMAs per product of the hi/lo operand
split against the 2.5 PFLOP/s dense bf16 peak.

cpu_baseline: the float64 C oracle (OpenMP over the host cores) decoding the same 8B
model on a bounded sample (8-token prompt, then as many greedy tokens as fit ~15 s).

--model qwen3-0.6b / gemma3-27b run the other shaped decoders (64-token prompt and 256
tokens; 8192-token prompt in 64 batches and 128 tokens at context 8448) with the same
JSON line; the default is the headline workload above.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import platform
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from webgpu_amd import synth  # noqa: E402
from webgpu_amd.engine import LoadOptions, PagedEngine  # noqa: E402
from webgpu_amd.gguf import F16, F32, Q4_0, Q4_K, Q5_K, Q6_K, Q8_0, QUANTS  # noqa: E402
from webgpu_amd.gpu import Compute  # noqa: E402

PEAK_HBM = 8.0e12  # MI355X published HBM3E bandwidth, bytes/s
# HBM bytes per launch of the roofline kernel, from rocprofv3 FETCH_SIZE + WRITE_SIZE scaled by a
# 256 MiB copy in the same program (the summary holds the commands and the raw counts).
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "k_mv_matvec_microbench.md")


# The sources of the roofline kernel and its file's own build flags; the counter summary records
# their digest, so a line whose traffic comes from a profile of another version of the kernel
# says so.
KERNEL_SOURCES = [os.path.join(ROOT, "webgpu_amd", "csrc", f) for f in ("matvec.hip", "matvec.h", "decode.h")]


def kernel_source_digest() -> str:
    import hashlib
    from webgpu_amd.build import FILE_FLAGS
    h = hashlib.sha256()
    for path in KERNEL_SOURCES:
        with open(path, "rb") as fh:
            h.update(fh.read())
    h.update(" ".join(FILE_FLAGS.get("matvec.hip", [])).encode())
    return h.hexdigest()[:16]


def profiled_traffic(type_name: str, shape: str):
    """(traffic_bytes of the committed counter summary for this shape or None, whether the
    summary was taken of the current kernel sources)."""
    traffic, digest = None, None
    try:
        with open(TRAFFIC_PROFILE) as fh:
            for line in fh:
                f = line.split()
                if len(f) == 4 and f[0] == "traffic_bytes" and f[1] == type_name and f[2] == shape:
                    traffic = int(f[3])
                if len(f) == 2 and f[0] == "kernel_source_sha256":
                    digest = f[1]
    except OSError:
        pass
    return traffic, digest == kernel_source_digest()
METRIC = "decode tok/s (1 GPU) + Q4_K matvec HBM GB/s as % of peak"

# Workloads: the default (the headline) and the other shaped decoders, each with its prompt,
# decode length and context (a prompt of `prompt` tokens in 128-token batches, then `steps`
# greedy tokens).
WORKLOADS = {
    "llama3-8b": dict(prompt=512, steps=256, context=1024, title="Llama-3-8B-shaped Q4_K_M"),
    "qwen3-0.6b": dict(prompt=64, steps=256, context=1024, title="Qwen3-0.6B-shaped Q4_K_M"),
    "gemma3-27b": dict(prompt=8192, steps=128, context=8448, title="Gemma-3-27B-shaped Q4_K_M"),
}


class Events:
    """hipEvent pairs on a given stream (the library's own)."""

    def __init__(self) -> None:
        self.hip = C.CDLL("libamdhip64.so")
        self.hip.hipEventCreate.argtypes = [C.POINTER(C.c_void_p)]
        self.hip.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]
        self.hip.hipEventSynchronize.argtypes = [C.c_void_p]
        self.hip.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
        self.hip.hipEventDestroy.argtypes = [C.c_void_p]

    def create(self, n: int):
        evs = []
        for _ in range(n):
            e = C.c_void_p()
            assert self.hip.hipEventCreate(C.byref(e)) == 0
            evs.append(e)
        return evs

    def record(self, e, stream) -> None:
        assert self.hip.hipEventRecord(e, stream) == 0

    def elapsed_ms(self, a, b) -> float:
        assert self.hip.hipEventSynchronize(b) == 0
        ms = C.c_float()
        assert self.hip.hipEventElapsedTime(C.byref(ms), a, b) == 0
        return ms.value

    def destroy(self, evs) -> None:
        for e in evs:
            self.hip.hipEventDestroy(e)


def matvec_bench(gpu: Compute, ev: Events, type_: int, cols: int, rows: int, launches: int = 96) -> dict:
    q = QUANTS[type_]
    wbytes = rows * cols // q["block"] * q["bytes"]
    copies = max(2, min(24, int(800e6 // wbytes) + 1))
    rng = np.random.default_rng(cols * 7 + rows)
    if type_ in (Q4_K, Q6_K):
        base = (synth.microbench_q4k if type_ == Q4_K else synth.microbench_q6k)(rng, rows, cols)
    else:
        gen = {Q5_K: synth.q5k_blocks, Q8_0: synth.q8_0_blocks, Q4_0: synth.q4_0_blocks, F16: synth.f16_values,
               F32: lambda r, n: (r.standard_normal(n) * 0.02).astype(np.float32).view(np.uint8)}[type_]
        base = gen(rng, rows * cols // q["block"])
    ws = []
    for i in range(copies):
        data = base if i == 0 else np.roll(base, q["bytes"] * i * 7)  # distinct bytes per copy
        ws.append(gpu.upload_weights(type_, cols, rows, data, f"w{i}"))
    x = gpu.upload(rng.standard_normal(cols).astype(np.float32), "x")
    qx = gpu.quantized_buffer(cols)
    y = gpu.buffer(rows * 4, "y")
    stream = gpu.stream
    gpu.quantize(x, cols, qx)  # the activation row is quantized once; the kernel timed is the matvec
    for i in range(copies):
        gpu.matvec(type_, ws[i], qx, y, cols, rows)
    gpu.done()
    # One event pair over `launches` back-to-back launches (rotating copies): the mean time
    # per launch, comparable with the profiler's per-kernel durations. Repeated 5 times.
    evs = ev.create(2)
    times = []
    for rep in range(5):
        ev.record(evs[0], stream)
        for i in range(launches):
            gpu.matvec(type_, ws[i % copies], qx, y, cols, rows)
        ev.record(evs[1], stream)
        times.append(ev.elapsed_ms(evs[0], evs[1]) * 1e-3 / launches)
    ev.destroy(evs)
    for w in ws:
        gpu.destroy(w)
    gpu.destroy(x)
    gpu.destroy(qx)
    gpu.destroy(y)
    alg = wbytes + 4 * cols + 4 * rows
    mean = float(np.mean(times))
    return {"shape": f"{cols}x{rows}", "type": q["name"], "bytes": alg, "us": mean * 1e6,
            "best_us": float(np.min(times)) * 1e6, "GBps": alg / mean / 1e9, "frac": alg / mean / PEAK_HBM,
            "copies": copies}


PROBE_CONFIGS = [(256, 512, 8), (512, 256, 8), (512, 512, 4), (1024, 256, 4), (256, 1024, 4), (1024, 512, 4)]


def probe_bench(gpu: Compute, ev: Events, nbytes: int, out_floats: int = 0, launches: int = 96) -> dict:
    """The per-launch floor of reading `nbytes` once (wgd_probe_read): a plain streaming read
    of 16-byte loads rotating over copies totalling ~900 MB (beyond the Infinity Cache), best
    of a few grid shapes, timed like the matvec (a HIP event pair around back-to-back
    launches, which the library issues itself). With out_floats it also stores a result
    vector of that length, as a matvec stores its rows."""
    stride = (nbytes + 4095) // 4096 * 4096
    copies = max(2, min(96, int(900e6 // nbytes) + 1))
    src = gpu.buffer(copies * stride, "probe src")
    out = gpu.buffer(max(4, out_floats * 4), "probe out")
    best = None
    evs = ev.create(2)
    for wgs, threads, depth in PROBE_CONFIGS:
        gpu.probe_read(src, nbytes, copies, copies, wgs, threads, depth, out, out_floats)
        gpu.done()
        times = []
        for rep in range(3):
            ev.record(evs[0], gpu.stream)
            gpu.probe_read(src, nbytes, copies, launches, wgs, threads, depth, out, out_floats)
            ev.record(evs[1], gpu.stream)
            times.append(ev.elapsed_ms(evs[0], evs[1]) * 1e-3 / launches)
        t = float(np.mean(times))
        if best is None or t < best["us"] * 1e-6:
            best = {"bytes": nbytes, "out_floats": out_floats, "us": t * 1e6, "GBps": nbytes / t / 1e9,
                    "frac": nbytes / t / PEAK_HBM, "grid": f"{wgs}x{threads} depth {depth}"}
    ev.destroy(evs)
    gpu.destroy(src)
    gpu.destroy(out)
    return best


PEAK_BF16 = 2.5e15  # MI355X dense bf16 MFMA peak, flop/s
GEMM_SHAPES = [(Q4_K, 4096, 14336, 128), (Q4_K, 14336, 4096, 128), (Q4_K, 4096, 4096, 128), (Q6_K, 4096, 1024, 128)]


def gemm_bench(gpu: Compute, ev: Events, type_: int, cols: int, rows: int, batch: int, launches: int = 20) -> dict:
    """One prompt-batch dequant-GEMM (batch tokens x rows x cols, planar weights) timed with a
    HIP event pair around `launches` back-to-back calls on the library's stream. Algorithmic
    flops are 2 * batch * rows * cols; the kernel issues three bf16 MFMAs per product (hi/lo
    operand split), so its MFMA work is three times that."""
    rng = np.random.default_rng(cols * 5 + rows)
    gen = synth.microbench_q4k if type_ == Q4_K else synth.microbench_q6k
    w = gpu.upload_weights(type_, cols, rows, gen(rng, rows, cols), "gemm w")
    x = gpu.upload(rng.standard_normal(batch * cols).astype(np.float32), "gemm x")
    y = gpu.buffer(batch * rows * 4, "gemm y")
    for _ in range(3):
        gpu.matmul(type_, w, x, y, cols, rows, rows, 0, 0, batch)
    gpu.done()
    evs = ev.create(2)
    times = []
    for rep in range(3):
        ev.record(evs[0], gpu.stream)
        for _ in range(launches):
            gpu.matmul(type_, w, x, y, cols, rows, rows, 0, 0, batch)
        ev.record(evs[1], gpu.stream)
        times.append(ev.elapsed_ms(evs[0], evs[1]) * 1e-3 / launches)
    ev.destroy(evs)
    for b in (w, x, y):
        gpu.destroy(b)
    t = float(np.mean(times))
    flops = 2.0 * batch * rows * cols
    return {"shape": f"{cols}x{rows}", "type": QUANTS[type_]["name"], "batch": batch, "us": t * 1e6,
            "tflops": flops / t / 1e12, "mfma_tflops": 3 * flops / t / 1e12, "mfma_frac": 3 * flops / t / PEAK_BF16}


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), as the baseline's hardware."""
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.lower().startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def cpu_baseline(f: np.ndarray, title: str, seconds: float = 15.0) -> dict:
    from oracle import orc
    from webgpu_amd.context import attention_memory
    from webgpu_amd.gguf import model_config, parse_gguf_header
    g = parse_gguf_header(f, f.size)
    c = model_config(g)
    m = orc.OracleModel(f, g, c, 1024, attention_memory(c, 1024, 128)["capacities"])
    ids = synth.prompt_ids(c.vocab, 8)
    logits = m.forward(ids, 0)
    tok, pos, n, t0 = int(np.argmax(logits)), 8, 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds or n < 2:
        logits = m.forward([tok], pos)
        tok, pos, n = int(np.argmax(logits)), pos + 1, n + 1
    dt = time.perf_counter() - t0
    m.close()
    cpu = cpu_model()
    return {"value": n / dt, "unit": "tok/s", "cores": orc.threads(), "kind": "port", "cpu": cpu,
            "host_cpus": os.cpu_count(),
            "sample": f"float64 C oracle, {title} decode: 8-token prompt then {n} greedy tokens "
                      f"in {dt:.1f} s on {orc.threads()} threads of {cpu}"}


def trace_summary(directory: str) -> None:
    """Per-token kernel table of an `--eager` decode run traced by `rocprofv3 --kernel-trace
    --output-format csv -d DIR`: every kernel from the first decode token's `k_token_start`
    on, grouped by name and grid, with launches and microseconds per token."""
    import collections
    import csv
    import glob
    path = glob.glob(os.path.join(directory, "**", "*kernel_trace.csv"), recursive=True)[0]
    rows = sorted(csv.DictReader(open(path)), key=lambda r: int(r["Start_Timestamp"]))
    first = next(i for i, r in enumerate(rows) if "k_token_start" in r["Kernel_Name"])
    dec = rows[first:]
    ntok = sum(1 for r in dec if "k_token_start" in r["Kernel_Name"])
    agg = collections.defaultdict(list)
    for r in dec:
        name = r["Kernel_Name"].split("(")[0][:90] or "(unnamed)"
        grid = f'{int(r["Grid_Size_X"]) // int(r["Workgroup_Size_X"])}x{r["Workgroup_Size_X"]}'
        agg[(name, grid)].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    tot = sum(sum(v) for v in agg.values())
    span = (int(dec[-1]["End_Timestamp"]) - int(dec[0]["Start_Timestamp"])) / 1e3
    print(f"decode tokens {ntok}; kernel time {tot / ntok:.1f} us/token; span {span / ntok:.1f} us/token "
          "(eager, host round trip per token)")
    print("| kernel | grid (wg x threads) | launches / token | mean us | us / token | share |")
    print("|---|---|---|---|---|---|")
    for (k, g), v in sorted(agg.items(), key=lambda kv: -sum(kv[1])):
        print(f"| `{k}` | {g} | {len(v) / ntok:.2f} | {sum(v) / len(v):.2f} | {sum(v) / ntok:.1f} | {100 * sum(v) / tot:.1f}% |")


def attention_timings(eng, a, spec, context: int, pos: int):
    """Decode attention alone (one layer's launch pair, HIP events over 50 launches), at the
    middle and the end of the timed window; Gemma-3 at a local (sliding) and a global layer.
    Bytes: the K and V rows of every attended key (min(pos + 1, window) keys x kv_heads x
    head_dim x 2)."""
    attn = []
    esz = 2 if a.kv == "f16" else 4
    cfg = eng.config
    gemma = cfg.family == "gemma3"
    layers = [0, cfg.period - 1] if gemma else [0]
    for layer in layers:
        window = cfg.window if gemma and layer % cfg.period != cfg.period - 1 else context
        for p in sorted({pos + a.steps // 2, pos + a.steps}):
            if p >= context:
                continue
            us = eng.attention_timing(layer, p, 50)
            nbytes = min(p + 1, window) * spec.kv_heads * spec.head_dim * 2 * esz
            attn.append({"layer": layer, "pos": p, "keys": min(p + 1, window), "us": us, "bytes": nbytes,
                         "GBps": nbytes / us / 1e3, "frac": nbytes / us / 1e3 / (PEAK_HBM / 1e9)})
            print(f"[bench] decode attention layer {layer} at position {p}: {us:.2f} us, {nbytes / us / 1e3:.0f} GB/s "
                  f"({100 * nbytes / us / 1e3 / (PEAK_HBM / 1e9):.1f}% of 8 TB/s)", file=sys.stderr, flush=True)
    return attn


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--model", default="llama3-8b", choices=sorted(WORKLOADS),
                    help="shaped decoder to run (the default is the headline workload)")
    ap.add_argument("--steps", type=int, default=None, help="timed decode tokens (default: per model)")
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--prompt", type=int, default=None, help="prompt tokens (default: per model)")
    ap.add_argument("--eager", action="store_true",
                    help="decode with one forward per token (eager launches, host round trip per token) instead of "
                         "graph replays: for kernel traces, whose profiler does not follow graph launches; the "
                         "tok/s of such a run is not the metric")
    ap.add_argument("--no-attention-timing", action="store_true", help="skip the decode attention timing")
    ap.add_argument("--trace-summary", metavar="DIR",
                    help="print the per-token kernel table of an --eager decode traced into DIR by rocprofv3, then exit")
    ap.add_argument("--kv", default="f32", choices=["f32", "f16"],
                    help="K/V ring element type (f32 as the reference; f16 halves the ring bytes)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-matvec", action="store_true", help="skip the matvec microbench")
    ap.add_argument("--matvec-only", action="store_true",
                    help="only the matvec microbench and a 256 MiB device copy (counter calibration), no JSON line")
    ap.add_argument("--gemm-only", action="store_true", help="only the prompt-GEMM microbench, no JSON line")
    ap.add_argument("--attention-only", action="store_true",
                    help="load and prefill the model, then only the decode attention timings (and a 256 MiB device "
                         "copy for counter calibration), no JSON line")
    ap.add_argument("--probe", action="store_true",
                    help="only the plain-read probe (the per-launch read floor) at the matvec byte counts, with and "
                         "without a result store; one JSON line per case")
    ap.add_argument("--sample-only", action="store_true",
                    help="only the device sampler (T 0.7, top-k 40, top-p 0.9) on normal logits rows of three vocabulary "
                         "sizes, 30 draws each, no JSON line")
    a = ap.parse_args()
    if a.trace_summary:
        trace_summary(a.trace_summary)
        return
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the token loop runs on a single MI355X (multi-GPU sharding is a design "
              "only); run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    if a.matvec_only:
        gpu = Compute().init()
        ev = Events()
        # a plain copy of known size: its FETCH_SIZE / WRITE_SIZE per dispatch scale the counters
        n = 256 << 20
        src, dst = gpu.buffer(n, "copy src"), gpu.buffer(n, "copy dst")
        for _ in range(4):
            gpu.copy(src, dst, n)
        gpu.done()
        gpu.destroy(src)
        gpu.destroy(dst)
        # the roofline shapes, then the FFN-up shape in every type with a planar layout
        for s in [(Q4_K, 14336, 4096), (Q4_K, 4096, 4096), (Q4_K, 4096, 14336), (Q6_K, 4096, 128256),
                  (Q5_K, 14336, 4096), (Q6_K, 14336, 4096), (Q8_0, 14336, 4096), (Q4_0, 14336, 4096),
                  (F16, 14336, 4096), (F32, 14336, 4096)]:
            m = matvec_bench(gpu, ev, *s)
            print(f"[bench] matvec {m['type']} {m['shape']}: {m['us']:.2f} us, {m['GBps']:.0f} GB/s "
                  f"({100 * m['frac']:.1f}% of 8 TB/s)", file=sys.stderr, flush=True)
        gpu.dispose()
        return
    if a.probe:
        gpu = Compute().init()
        ev = Events()
        # the Q4_K weight bytes of 4096x4096 and of 14336x4096 / 4096x14336, and a 66 MB pair
        for nbytes, rows in ((9437184, 4096), (33030144, 4096), (33030144, 14336), (66060288, 14336)):
            for out_floats in (0, rows):
                r = probe_bench(gpu, ev, nbytes, out_floats)
                print(json.dumps({"probe": r}), flush=True)
                print(f"[bench] probe {nbytes} B, {out_floats} result floats: {r['us']:.2f} us, {r['GBps']:.0f} GB/s "
                      f"({100 * r['frac']:.1f}% of 8 TB/s) at {r['grid']}", file=sys.stderr, flush=True)
        gpu.dispose()
        return
    if a.sample_only:
        gpu = Compute().init()
        rng = np.random.default_rng(0)
        for n in (128256, 151936, 262144):
            buf = gpu.upload((rng.standard_normal(n) * 3).astype(np.float32), "logits")
            t0 = time.perf_counter()
            for i in range(30):
                gpu.sample(buf, n, 0.7, 40, 0.9, 1, i)
            print(f"[bench] sample {n} entries: {(time.perf_counter() - t0) / 30 * 1e6:.1f} us per call "
                  f"(host round trip included)", file=sys.stderr, flush=True)
            gpu.destroy(buf)
        gpu.dispose()
        return
    if a.gemm_only:
        gpu = Compute().init()
        ev = Events()
        for sh in GEMM_SHAPES:
            g = gemm_bench(gpu, ev, *sh)
            print(f"[bench] gemm {g['type']} {g['shape']} x {g['batch']} tokens: {g['us']:.1f} us, {g['tflops']:.0f} TFLOP/s "
                  f"({g['mfma_tflops']:.0f} TFLOP/s of bf16 MFMA, {100 * g['mfma_frac']:.1f}% of peak)", file=sys.stderr, flush=True)
        gpu.dispose()
        return
    wl = WORKLOADS[a.model]
    if a.prompt is None:
        a.prompt = wl["prompt"]
    if a.steps is None:
        a.steps = wl["steps"]
    context = wl["context"]
    if a.prompt + a.warmup + a.steps > context:
        context = min(32768, 1 << (a.prompt + a.warmup + a.steps - 1).bit_length())
    spec = synth.SPECS[a.model]

    t = time.perf_counter()
    f = synth.build(a.model)
    print(f"[bench] synthetic {a.model} GGUF {f.size / 1e9:.2f} GB in {time.perf_counter() - t:.1f} s",
          file=sys.stderr, flush=True)
    eng = PagedEngine()
    t = time.perf_counter()
    eng.load(f, LoadOptions(contextLength=context, batchSize=128, kvCacheType=a.kv))
    print(f"[bench] loaded in {time.perf_counter() - t:.1f} s on {eng.gpu.adapterName}", file=sys.stderr, flush=True)
    ids = synth.prompt_ids(eng.config.vocab, a.prompt, seed=7)

    # prefill (reported, not the metric): one untimed pass loads every kernel, then the median
    # of three timed passes over the same positions (each rewrites the same KV slots)
    def prefill():
        eng.gpu.done()
        t = time.perf_counter()
        for i in range(0, a.prompt, 128):
            chunk = ids[i:i + 128]
            if i + len(chunk) == a.prompt:
                tok = eng.forward_argmax(chunk, i)
            else:
                eng.forward(chunk, i, False)
        eng.gpu.done()
        return time.perf_counter() - t, tok
    prefill()
    if a.attention_only:
        n = 256 << 20  # a plain copy of known size: its counters per dispatch scale the attention's
        src, dst = eng.gpu.buffer(n, "copy src"), eng.gpu.buffer(n, "copy dst")
        for _ in range(4):
            eng.gpu.copy(src, dst, n)
        eng.gpu.done()
        eng.gpu.destroy(src)
        eng.gpu.destroy(dst)
        attention_timings(eng, a, spec, context, a.prompt)
        eng.dispose()
        return
    runs = [prefill() for _ in range(3)]
    prefill_s, token = sorted(runs)[1]
    print(f"[bench] prefill {a.prompt} tokens in {prefill_s * 1e3:.1f} ms (median of 3 after a warm-up pass)",
          file=sys.stderr, flush=True)

    # warm-up steps run over the first positions after the prompt, then the timed steps decode
    # the same positions again (rewriting the same ring slots), so the timed window is the
    # workload's span [prompt, prompt + steps) whatever the warm-up count
    pos = a.prompt

    def decode(n):
        if not a.eager:
            return eng.decode(token, pos, n)
        out, t = [], token
        for i in range(n):
            t = eng.forward_argmax([t], pos + i)
            out.append(t)
        return out
    if a.warmup:
        decode(a.warmup)
    eng.gpu.done()
    t0 = time.perf_counter()
    toks = decode(a.steps)
    eng.gpu.done()
    dt = time.perf_counter() - t0
    value = a.steps / dt
    print(f"[bench] decode {a.steps} tokens in {dt * 1e3:.1f} ms -> {value:.1f} tok/s", file=sys.stderr, flush=True)

    # the same decode with the reference's default sampling (reported, not the metric): the
    # same positions again, each step drawing on the device (its own decode graph)
    sampled = None
    if not a.eager:
        eng.set_sampling(0.7, 40, 0.9, seed=1)
        eng.decode(token, pos, 2)
        eng.gpu.done()
        t0 = time.perf_counter()
        eng.decode(token, pos, a.steps)
        eng.gpu.done()
        sampled = a.steps / (time.perf_counter() - t0)
        eng.set_sampling(0.0)
        print(f"[bench] decode with sampling (T 0.7, top-k 40, top-p 0.9): {sampled:.1f} tok/s", file=sys.stderr,
              flush=True)

    attn = [] if a.no_attention_timing else attention_timings(eng, a, spec, context, pos)

    result = {
        "metric": METRIC, "value": value, "unit": "tok/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": dt * 1e3 / a.steps, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "decode_sampled_tok_s": sampled,
        "dtype": "f32", "data": "synthetic (seeded random-init Q4_K_M GGUF)",
        "config": {"workload": f"{a.model}-shape Q4_K_M greedy decode", "prompt": a.prompt, "prefill_batch": 128,
                   "decode_tokens": a.steps, "context": context, "kv_cache": a.kv,
                   "layers": spec.layers, "hidden": spec.hidden, "heads": spec.heads, "kv_heads": spec.kv_heads,
                   "ffn": spec.ffn, "vocab": spec.vocab},
        "prefill_tok_s": a.prompt / prefill_s,
        "decode_window": [pos, pos + a.steps],
        "attention": attn,
    }
    eng.dispose()

    if not a.no_matvec:
        gpu = Compute().init()
        ev = Events()
        shapes = [(Q4_K, 14336, 4096), (Q4_K, 4096, 4096), (Q4_K, 4096, 14336), (Q6_K, 4096, 128256)]
        mv = [matvec_bench(gpu, ev, *s) for s in shapes]
        gm = [gemm_bench(gpu, ev, *sh) for sh in GEMM_SHAPES]
        # the plain-read floor for the same weight bytes, with the matvec's result store
        pr = {m["shape"]: probe_bench(gpu, ev, m["bytes"] - 4 * int(m["shape"].split("x")[0]) - 4 * int(m["shape"].split("x")[1]),
                                      int(m["shape"].split("x")[1])) for m in mv[:3]}
        gpu.dispose()
        head = mv[0]
        traffic, current = profiled_traffic(head["type"], head["shape"])
        result["roofline"] = {"bound": "hbm", "achieved": head["GBps"], "peak": PEAK_HBM / 1e9, "unit": "GB/s",
                              "frac": head["frac"], "traffic": traffic,
                              "traffic_source": "counters of the current kernel sources" if current else
                              "counters of an older version of matvec.hip (profile not regenerated)",
                              "kernel": f"k_matvec<Q4K> {head['shape']} (in x out), {head['bytes']} B per launch",
                              "mean_us": head["us"]}
        result["matvec"] = mv
        result["probe"] = [{"shape": k, "read_us": v["us"], "read_frac": v["frac"], "grid": v["grid"],
                            "matvec_us": next(m["us"] for m in mv if m["shape"] == k),
                            "matvec_over_probe": next(m["us"] for m in mv if m["shape"] == k) / v["us"]}
                           for k, v in pr.items()]
        result["prefill_gemm"] = gm
        for m in mv:
            print(f"[bench] matvec {m['type']} {m['shape']}: {m['us']:.2f} us, {m['GBps']:.0f} GB/s "
                  f"({100 * m['frac']:.1f}% of 8 TB/s)", file=sys.stderr, flush=True)
        for g in gm:
            print(f"[bench] gemm {g['type']} {g['shape']} x {g['batch']} tokens: {g['us']:.1f} us, {g['tflops']:.0f} TFLOP/s "
                  f"({100 * g['mfma_frac']:.1f}% of bf16 MFMA peak)", file=sys.stderr, flush=True)
    if not a.no_cpu:
        result["cpu_baseline"] = cpu_baseline(f, wl["title"])
        print(f"[bench] cpu baseline {result['cpu_baseline']['value']:.3f} tok/s", file=sys.stderr, flush=True)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
