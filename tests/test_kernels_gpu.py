"""Kernel parity on the MI355X through the C ABI, against the float64 oracle.

Ports the reference's in-browser GPU checks (src/verify.ts:16-74, src/verify-context.ts:
8-40, src/verify-qwen.ts:87-97) and adds bit-exact dequantization for every GGUF type.
Tolerances: dequantized weights bit-exact; kernels within the reference's own bounds
(|got - want| <= 1e-3 * max(1, |want|) for matmul/norm/rope, verify.ts:11; absolute
1e-3 for long-context attention, verify-context.ts:39; 2e-3 relative for partial RoPE,
verify-qwen.ts:12).
"""
import math

import numpy as np
import pytest

from oracle import orc
from webgpu_amd import synth
from webgpu_amd.gguf import F16, F32, Q4_0, Q4_K, Q5_K, Q6_K, Q8_0, QUANTS
from webgpu_amd.gpu import WgdError, WGD_E_NONFINITE

pytestmark = pytest.mark.gpu
ALL = [F32, F16, Q4_0, Q8_0, Q4_K, Q5_K, Q6_K]
# synthetic block generators of the types with a decode matvec
GEN = {Q4_K: synth.q4k_blocks, Q5_K: synth.q5k_blocks, Q6_K: synth.q6k_blocks, Q8_0: synth.q8_0_blocks,
       Q4_0: synth.q4_0_blocks, F16: synth.f16_values,
       F32: lambda rng, n, std=0.05: (rng.standard_normal(n) * std).astype(np.float32).view(np.uint8)}


def near(got, want, tol=1e-3, label=""):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    assert np.all(np.isfinite(got)), f"{label}: non-finite output"
    err = np.abs(got - want) / np.maximum(1.0, np.abs(want))
    assert err.max() <= tol, f"{label}: max scaled error {err.max():.3e} at {int(err.argmax())}"
    return float(err.max())


def verify_pattern(type_, rows=5, cols=256):
    """The byte pattern of verify.ts:17-25: (i*17+93)%256 with d/dmin forced."""
    q = QUANTS[type_]
    nbytes = rows * cols // q["block"] * q["bytes"]
    packed = np.array([(i * 17 + 93) % 256 for i in range(-(-nbytes // 4) * 4)], np.uint8)
    if type_ == F32:
        packed = (np.sin(np.arange(packed.size // 4)) * 0.5).astype(np.float32).view(np.uint8).copy()
    elif type_ == F16:
        for i in range(0, packed.size, 2):
            packed[i], packed[i + 1] = i % 256, 0x30
    else:
        for off in range(0, nbytes, q["bytes"]):
            s = off + 208 if type_ == Q6_K else off
            packed[s], packed[s + 1] = 0, 0x20
            if type_ in (Q4_K, Q5_K):
                packed[off + 2], packed[off + 3] = 0, 0x1C
    return packed[:nbytes].copy()


# ---------------------------------------------------------------- exact dequantization
@pytest.mark.parametrize("type_", ALL)
def test_dequant_bit_exact(gpu, type_):
    rng = np.random.default_rng(100 + type_)
    q = QUANTS[type_]
    n = 64 * 256
    nb = n // q["block"]
    raw = np.frombuffer(rng.bytes(nb * q["bytes"]), np.uint8).copy()
    for data in (raw, verify_pattern(type_, rows=64, cols=256)):
        want = orc.dequant(data, type_, n)
        w = gpu.upload(data, "weights")
        out = gpu.buffer(n * 4, "deq")
        gpu.dequant(type_, w, out, n)
        got = gpu.read_f32(out, n)
        gpu.destroy(w)
        gpu.destroy(out)
        nan = np.isnan(want)
        assert np.array_equal(np.isnan(got), nan)
        assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


# ---------------------------------------------------------------- verify.ts:16-38
@pytest.mark.parametrize("type_", ALL)
@pytest.mark.parametrize("batch", [128, 3, 1])
def test_matmul_offsets_all_types(gpu, type_, batch):
    rows, cols = 5, 256
    packed = verify_pattern(type_, rows, cols)
    x = (np.cos(np.arange((batch + 1) * cols) * 0.17) * 0.1).astype(np.float32)
    want = orc.matmul(type_, packed, x, cols, rows, rows + 2, 2, 1, batch)
    wb, xb = gpu.upload(packed, "w"), gpu.upload(x, "x")
    yb = gpu.buffer(batch * (rows + 2) * 4, "y")
    gpu.matmul(type_, wb, xb, yb, cols, rows, rows + 2, 2, 1, batch)
    y = gpu.read_f32(yb, batch * (rows + 2))
    for b in range(batch):
        near(y[b * (rows + 2) + 2: b * (rows + 2) + 2 + rows], want[b * (rows + 2) + 2: b * (rows + 2) + 2 + rows],
             label=f"type {type_} batch {b}")
    for buf in (wb, xb, yb):
        gpu.destroy(buf)


# the three Q4_K microbench shapes (4096x4096, 14336 -> 4096, 4096 -> 14336) and the Q6_K head
# (4096 -> 128256) as the bench launches them, then shapes off the whole-tile grid
@pytest.mark.parametrize("type_,rows,cols", [(Q4_K, 4096, 4096), (Q4_K, 4096, 14336), (Q4_K, 14336, 4096),
                                             (Q6_K, 128256, 4096), (Q4_K, 1024, 14336), (Q4_K, 3072, 1024),
                                             (Q6_K, 1024, 4096), (Q6_K, 520, 5376), (Q8_0, 512, 4096),
                                             (Q4_K, 300, 3072), (Q5_K, 1024, 4096), (Q5_K, 520, 14336),
                                             (Q4_0, 512, 4096), (Q4_0, 300, 3136), (F16, 4096, 4096),
                                             (F16, 1030, 14336), (F16, 300, 3072), (F32, 4096, 4096),
                                             (F32, 1030, 14336), (F32, 300, 3072), (F32, 256, 64)])
def test_fast_matvec_real_shapes(gpu, type_, rows, cols):
    rng = np.random.default_rng(rows + cols)
    gen = GEN[type_]
    w = gen(rng, rows * cols // QUANTS[type_]["block"])
    x = rng.standard_normal(cols).astype(np.float32)
    want = orc.matmul(type_, w, x, cols, rows, rows, 0, 0, 1)
    wb = gpu.upload_weights(type_, cols, rows, w)
    xb, yb = gpu.upload(x, "x"), gpu.buffer(rows * 4, "y")
    gpu.matmul(type_, wb, xb, yb, cols, rows, rows, 0, 0, 1)
    got = gpu.read_f32(yb, rows)
    near(got, want, 1e-4, f"{type_} {rows}x{cols}")
    for buf in (wb, xb, yb):
        gpu.destroy(buf)


@pytest.mark.parametrize("type_", [Q4_K, Q5_K, Q6_K, Q8_0, Q4_0, F16])
def test_prompt_gemm_on_mfma(gpu, type_):
    rng = np.random.default_rng(7 + type_)
    rows, cols, batch = 200, 1024, 77
    gen = GEN[type_]
    w = gen(rng, rows * cols // QUANTS[type_]["block"])
    x = rng.standard_normal((batch + 2) * cols).astype(np.float32)
    want = orc.matmul(type_, w, x, cols, rows, rows, 0, 2, batch)
    for planar in (False, True):
        wb = gpu.upload_weights(type_, cols, rows, w) if planar else gpu.upload(w, "w")
        xb, yb = gpu.upload(x, "x"), gpu.buffer(batch * rows * 4, "y")
        gpu.matmul(type_, wb, xb, yb, cols, rows, rows, 0, 2, batch)
        near(gpu.read_f32(yb, batch * rows), want, 1e-4, f"gemm {type_} planar={planar}")
        for buf in (wb, xb, yb):
            gpu.destroy(buf)


@pytest.mark.parametrize("type_", [Q8_0, Q4_0])
def test_widths_outside_the_planar_tiles_stay_in_the_gguf_layout(gpu, type_):
    # 96 columns is not a whole 64-column GEMM tile: the matrix keeps its GGUF layout and
    # every batch runs the generic kernels on it
    rng = np.random.default_rng(96 + type_)
    rows, cols = 40, 96
    w = GEN[type_](rng, rows * cols // 32)
    for batch in (1, 70):
        x = rng.standard_normal(batch * cols).astype(np.float32)
        want = orc.matmul(type_, w, x, cols, rows, rows, 0, 0, batch)
        wb = gpu.upload_weights(type_, cols, rows, w)
        xb, yb = gpu.upload(x, "x"), gpu.buffer(batch * rows * 4, "y")
        gpu.matmul(type_, wb, xb, yb, cols, rows, rows, 0, 0, batch)
        near(gpu.read_f32(yb, batch * rows), want, 1e-4, f"{type_} width 96 batch {batch}")
        for buf in (wb, xb, yb):
            gpu.destroy(buf)


@pytest.mark.parametrize("type_,rows,cols,batch", [(Q4_K, 4096, 4096, 128), (Q6_K, 1024, 4096, 130),
                                                   (Q8_0, 384, 2048, 128), (Q4_K, 640, 14336, 64),
                                                   (Q5_K, 1024, 4096, 128), (Q4_0, 512, 4096, 130),
                                                   (Q4_K, 33280, 1024, 64)])
def test_prompt_gemm_real_shapes(gpu, type_, rows, cols, batch):
    """Planar prompt GEMM at layer shapes: whole 128-token tiles, a second token tile,
    split-K partial sums, a row offset inside a wider output (stride/rowBase, verify.ts:16-38).
    33280 rows are 260 row tiles, which one K split would run at half of the chip's two
    workgroups per CU; they take 3 splits, 780 workgroups, and a three-way partial sum."""
    rng = np.random.default_rng(rows * 3 + cols + batch)
    gen = GEN[type_]
    w = gen(rng, rows * cols // QUANTS[type_]["block"])
    x = rng.standard_normal((batch + 1) * cols).astype(np.float32)
    stride, base = rows + 8, 5
    want = orc.matmul(type_, w, x, cols, rows, stride, base, 1, batch)
    wb = gpu.upload_weights(type_, cols, rows, w)
    xb, yb = gpu.upload(x, "x"), gpu.buffer(batch * stride * 4, "y")
    gpu.matmul(type_, wb, xb, yb, cols, rows, stride, base, 1, batch)
    y = gpu.read_f32(yb, batch * stride).reshape(batch, stride)
    want = np.concatenate([want, np.zeros(batch * stride - want.size)]).reshape(batch, stride)
    near(y[:, base:base + rows].ravel(), want[:, base:base + rows].ravel(), 1e-4, f"gemm {type_} {rows}x{cols}x{batch}")
    for buf in (wb, xb, yb):
        gpu.destroy(buf)


# ---------------------------------------------------------------- verify.ts:39-54
@pytest.mark.parametrize("window", [2, 16])
def test_attention_small(gpu, window):
    heads, kvh, hd, start, n, context = 4, 2, 8, 3, 2, 16
    q = np.sin(np.arange(n * heads * hd)).astype(np.float32)
    k = np.cos(np.arange(context * kvh * hd)).astype(np.float32)
    v = np.sin(np.arange(context * kvh * hd) / 3).astype(np.float32)
    bufs = [gpu.upload(a, nm) for a, nm in ((q, "q"), (k, "k"), (v, "v"))] + [gpu.buffer(q.nbytes, "y")]
    gpu.attention(*bufs, heads, kvh, hd, start, 0.3, window, 0, context, n)
    got = gpu.read_f32(bufs[3], q.size)
    want = orc.attention(q, k, v, heads, kvh, hd, start, 0.3, window, context, n)
    near(got, want, label="attention")
    for b in bufs:
        gpu.destroy(b)


# ---------------------------------------------------------------- verify-context.ts:8-40
@pytest.mark.parametrize("context,start,batch,window,capacity,hd", [
    (4096, 2047, 3, 4096, 4096, 128), (32768, 32765, 3, 32768, 32768, 256),
    (32768, 32765, 3, 32768, 32768, 512), (32768, 32760, 8, 129, 136, 128)])
def test_attention_long_context_and_ring(gpu, context, start, batch, window, capacity, hd):
    heads, kvh = 2, 1
    key = lambda t, d: np.sin(t * 0.013 + d * 0.37)
    value = lambda t, d: np.cos(t * 0.019 + d * 0.23)
    q = (np.sin(np.arange(batch * heads * hd) * 0.7) * 12).astype(np.float32)
    k = np.zeros(capacity * hd, np.float32)
    v = np.zeros_like(k)
    d = np.arange(hd)
    for t in range(max(0, start + batch - capacity), start + batch):
        k[(t % capacity) * hd:(t % capacity + 1) * hd] = key(t, d)
        v[(t % capacity) * hd:(t % capacity + 1) * hd] = value(t, d)
    bufs = [gpu.upload(a, nm) for a, nm in ((q, "q"), (k, "k"), (v, "v"))] + [gpu.buffer(q.nbytes, "y")]
    gpu.attention(*bufs, heads, kvh, hd, start, 0.125, window, capacity, context, batch)
    got = gpu.read_f32(bufs[3], q.size)
    want = orc.attention(q, k, v, heads, kvh, hd, start, 0.125, window, capacity, batch)
    err = np.abs(got - want).max()
    assert np.all(np.isfinite(got)) and err <= 1e-3, f"max abs error {err:.3e}"
    for b in bufs:
        gpu.destroy(b)


# Prompt batches (the matrix-core path for head_dim 64/128/256): causal from position 0,
# a batch deep in the context, a ragged batch with one query head per KV head, a sliding
# window shorter than the batch's key range, and a wrapped ring. The last two split the
# keys 7 and 15 ways (the merge's 8- and 16-split forms; the others merge at most 4).
@pytest.mark.parametrize("heads,kvh,hd,start,batch,window,capacity", [
    (32, 8, 128, 0, 128, 4096, 1024), (32, 8, 128, 384, 128, 4096, 1024), (8, 8, 64, 100, 37, 4096, 256),
    (16, 2, 256, 50, 20, 24, 128), (8, 2, 128, 1000, 48, 200, 256), (6, 2, 64, 7, 131, 4096, 512),
    (4, 4, 64, 400, 16, 4096, 512), (4, 4, 64, 900, 16, 4096, 1024)])
def test_prompt_attention_batches(gpu, heads, kvh, hd, start, batch, window, capacity):
    rng = np.random.default_rng(start + batch)
    q = rng.standard_normal(batch * heads * hd).astype(np.float32) * 2
    k = rng.standard_normal(capacity * kvh * hd).astype(np.float32)
    v = rng.standard_normal(capacity * kvh * hd).astype(np.float32)
    bufs = [gpu.upload(a, nm) for a, nm in ((q, "q"), (k, "k"), (v, "v"))] + [gpu.buffer(q.nbytes, "y")]
    scale = 1 / np.sqrt(hd)
    gpu.attention(*bufs, heads, kvh, hd, start, scale, window, capacity, capacity, batch)
    got = gpu.read_f32(bufs[3], q.size)
    want = orc.attention(q, k, v, heads, kvh, hd, start, scale, window, capacity, batch)
    err = np.abs(got - want).max()
    assert np.all(np.isfinite(got)) and err <= 1e-4, f"max abs error {err:.3e}"
    for b in bufs:
        gpu.destroy(b)


# ---------------------------------------------------------------- verify.ts:55-66, verify-qwen.ts:87-97
def test_norm_and_qk_norm_rope(gpu):
    heads, hd, start, n = 4, 8, 3, 2
    q = np.sin(np.arange(n * heads * hd)).astype(np.float32)
    w = (1 + np.arange(hd) * 0.1).astype(np.float32)
    qb, wb, yb = gpu.upload(q, "q"), gpu.upload(w, "w"), gpu.buffer(q.nbytes, "y")
    gpu.norm(qb, wb, yb, hd, 1e-6, n * heads)
    normal = gpu.read_f32(yb, q.size)
    want = np.concatenate([orc.norm(q[g * hd:(g + 1) * hd], w, 1e-6) for g in range(n * heads)])
    near(normal, want, label="RMS norm")
    gpu.rope(qb, wb, heads, hd, start, 10000.0, 0.125, 1e-6, 0, n)
    near(gpu.read_f32(qb, q.size), orc.rope(q, w, heads, hd, start, 10000.0, 0.125, 1e-6, 0, n, 0), label="QK norm + RoPE")
    for b in (qb, wb, yb):
        gpu.destroy(b)


def test_partial_rope_and_plain_rotations(gpu):
    full, rot, heads, start, batch = 256, 64, 2, 17, 128
    series = lambda n, s=1.0: (np.sin(np.arange(n) * 0.31 + 0.7) * s).astype(np.float32)
    x = series(batch * heads * full)
    rw = (series(full) + 1).astype(np.float32)
    xb, wb = gpu.upload(x, "x"), gpu.upload(rw, "w")
    gpu.rope(xb, wb, heads, full, start, 1e7, 1.0, 1e-6, rot, batch)
    want = orc.rope(x, rw, heads, full, start, 1e7, 1.0, 1e-6, rot, batch, 0)
    near(gpu.read_f32(xb, x.size), want, 2e-3, "partial RoPE")
    for mode, fn in ((1, gpu.rope_neox), (2, gpu.rope_adjacent)):
        gpu.write(xb, x)
        fn(xb, heads, full, 32000, 500000.0, 1.0, 0, batch)
        want = orc.rope(x, None, heads, full, 32000, 500000.0, 1.0, 0.0, 0, batch, mode)
        near(gpu.read_f32(xb, x.size), want, 1e-4, f"rope mode {mode} at long positions")
    gpu.destroy(xb)
    gpu.destroy(wb)


# ---------------------------------------------------------------- elementwise
def test_elementwise(gpu):
    rng = np.random.default_rng(2)
    n = 10000
    g, u = rng.standard_normal(n).astype(np.float32) * 3, rng.standard_normal(n).astype(np.float32)
    gb, ub, yb = gpu.upload(g, "g"), gpu.upload(u, "u"), gpu.buffer(n * 4, "y")
    g64, u64 = g.astype(np.float64), u.astype(np.float64)
    gpu.silu(gb, ub, yb, n)
    near(gpu.read_f32(yb, n), g64 / (1 + np.exp(-g64)) * u64, 1e-5, "SwiGLU")
    gpu.gelu(gb, ub, yb, n)
    near(gpu.read_f32(yb, n), 0.5 * g64 * (1 + np.tanh(0.7978845608 * (g64 + 0.044715 * g64 ** 3))) * u64, 1e-5, "GeGLU")
    gpu.write(yb, u)
    gpu.add(gb, yb, n)
    near(gpu.read_f32(yb, n), g64 + u64, 1e-6, "add")
    b = rng.standard_normal(100).astype(np.float32)
    bb = gpu.upload(b, "b")
    gpu.write(yb, u)
    gpu.bias_add(yb, bb, n, 100)
    near(gpu.read_f32(yb, n), u64 + np.tile(b.astype(np.float64), n // 100), 1e-6, "bias")
    gpu.write(yb, g)
    gpu.activate(yb, n)
    near(gpu.read_f32(yb, n), g64 / (1 + np.exp(-g64)), 1e-5, "SiLU")
    for buf in (gb, ub, yb, bb):
        gpu.destroy(buf)


# ---------------------------------------------------------------- sample(T=0), quant.test.ts:46-49
def test_argmax_rules(gpu):
    cases = [np.array([np.nan, -2, 7, 3], np.float32), np.array([1, 5, 5, -np.inf, np.inf], np.float32),
             np.array([-0.0, 0.0, -1.0], np.float32)]
    for c in cases:
        b = gpu.upload(c, "logits")
        assert gpu.argmax(b, c.size) == orc.argmax(c)
        gpu.destroy(b)
    big = np.random.default_rng(4).standard_normal(262144).astype(np.float32)
    big[[5, 200000]] = big.max() + 1  # tie: the first index wins
    b = gpu.upload(big, "logits")
    assert gpu.argmax(b, big.size) == 5 == orc.argmax(big)
    gpu.destroy(b)
    bad = gpu.upload(np.array([np.nan, -np.inf, np.inf], np.float32), "logits")
    with pytest.raises(WgdError) as e:
        gpu.argmax(bad, 3)
    assert e.value.status == WGD_E_NONFINITE and "non-finite" in str(e.value)
    gpu.destroy(bad)


# ---------------------------------------------------------------- embedding gather
@pytest.mark.parametrize("type_", [F32, Q4_K, Q5_K, Q6_K, Q8_0, Q4_0])
def test_embed_gather_bit_exact(gpu, type_):
    rng = np.random.default_rng(type_)
    hidden, rows = 512, 40
    if type_ == F32:
        table = rng.standard_normal(hidden * rows).astype(np.float32).view(np.uint8).copy()
    else:
        gen = GEN[type_]
        table = gen(rng, hidden * rows // QUANTS[type_]["block"])
    ids = np.array([3, 0, 39, 3, 17], np.int32)
    full = orc.dequant(table, type_, hidden * rows, f32=False).reshape(rows, hidden)
    for scale in (1.0, math.sqrt(hidden)):
        want = (full[ids] * scale).astype(np.float32).reshape(-1)
        for planar in (False, True):
            tb = gpu.upload_weights(type_, hidden, rows, table) if planar else gpu.upload(table, "table")
            ib, ob = gpu.upload(ids, "ids"), gpu.buffer(ids.size * hidden * 4, "out")
            gpu.embed(type_, tb, ib, ob, hidden, ids.size, scale)
            assert np.array_equal(gpu.read_f32(ob, ids.size * hidden).view(np.uint32), want.view(np.uint32))
            for b in (tb, ib, ob):
                gpu.destroy(b)


def test_embed_rejects_out_of_range_ids(gpu):
    table = gpu.upload(np.zeros(64 * 4, np.float32), "table")
    ib, ob = gpu.upload(np.array([4], np.int32), "ids"), gpu.buffer(64 * 4, "out")
    with pytest.raises(WgdError):
        gpu.embed(F32, table, ib, ob, 64, 1, 1.0)
    for b in (table, ib, ob):
        gpu.destroy(b)


# ---------------------------------------------------------------- verify.ts:67-74 queue ordering
def test_queue_ordering_of_a_reused_weight_buffer(gpu):
    reused, vec, out = gpu.buffer(16, "reused"), gpu.upload(np.ones(4, np.float32), "ones"), gpu.buffer(8, "out")
    gpu.write(reused, np.array([1, 2, 3, 4], np.float32))
    gpu.matmul(F32, reused, vec, out, 4, 1, 2, 0, 0, 1)
    gpu.write(reused, np.array([5, 6, 7, 8], np.float32))
    gpu.matmul(F32, reused, vec, out, 4, 1, 2, 1, 0, 1)
    assert list(gpu.read_f32(out, 2)) == [10.0, 26.0]
    for b in (reused, vec, out):
        gpu.destroy(b)


def test_bounds_checks_reject_overruns(gpu):
    w, x, y = gpu.buffer(144, "w"), gpu.buffer(256 * 4, "x"), gpu.buffer(4, "y")
    with pytest.raises(WgdError):
        gpu.matmul(Q4_K, w, x, y, 256, 2, 2, 0, 0, 1)  # 2 rows need 288 weight bytes
    with pytest.raises(WgdError):
        gpu.matmul(Q4_K, w, x, y, 256, 1, 1, 1, 0, 1)  # rowBase 1 writes past y
    # offsets whose sum with the size wraps 64 bits are outside the buffers too
    with pytest.raises(WgdError):
        gpu.copy(x, y, 4, 2 ** 64 - 2, 0)
    with pytest.raises(WgdError):
        gpu.copy(x, y, 4, 0, 2 ** 64 - 2)
    with pytest.raises(WgdError):
        gpu.copy(x, y, 8, 0, 0)  # 8 bytes into the 4-byte y
    gpu.copy(x, y, 4, 4, 0)
    for b in (w, x, y):
        gpu.destroy(b)


# ---------------------------------------------------------------- quantized activation + matvec entries
@pytest.mark.parametrize("type_,rows,cols", [(Q4_K, 512, 4096), (Q6_K, 256, 5376), (Q8_0, 128, 1024),
                                             (Q5_K, 256, 4096), (Q4_0, 128, 2048), (F16, 200, 2048),
                                             (F32, 200, 2048)])
def test_quantize_with_rms_norm_then_matvec(gpu, type_, rows, cols):
    """wgd_quantize(x, norm w) + wgd_matvec == W @ (x * rsqrt(mean(x^2) + eps) * w)."""
    rng = np.random.default_rng(rows)
    gen = GEN[type_]
    w = gen(rng, rows * cols // QUANTS[type_]["block"])
    x = (rng.standard_normal(cols) * 3).astype(np.float32)
    nw = (1 + rng.uniform(-0.1, 0.1, cols)).astype(np.float32)
    xn = orc.norm(x, nw, 1e-6).astype(np.float32)
    want = orc.matmul(type_, w, xn, cols, rows, rows, 0, 0, 1)
    wb = gpu.upload_weights(type_, cols, rows, w)
    xb, nb, yb = gpu.upload(x, "x"), gpu.upload(nw, "norm"), gpu.buffer((rows + 3) * 4, "y")
    qb = gpu.quantized_buffer(cols)
    gpu.quantize(xb, cols, qb, nb, 1e-6)
    gpu.matvec(type_, wb, qb, yb, cols, rows, 3)
    near(gpu.read_f32(yb, rows + 3)[3:], want, 1e-4, f"normed matvec {type_}")
    for b in (wb, xb, nb, yb, qb):
        gpu.destroy(b)


@pytest.mark.parametrize("type_,rows,cols,normed", [(Q4_K, 4096, 4096, True), (Q4_K, 1024, 14336, False),
                                                    (Q6_K, 1024, 5376, True), (Q5_K, 2048, 4096, True),
                                                    (Q8_0, 1024, 5376, True), (Q4_0, 512, 4096, True)])
def test_every_launch_shape_gives_the_same_bits(gpu, type_, rows, cols, normed):
    """The decode step keeps whichever launch shape its measurement finds fastest, so every shape
    it may pick (rows per workgroup, pipeline depth; the K split fixed) must give the same bits.
    Inputs with a pending RMSNorm are the case where a reduction could follow the workgroup."""
    rng = np.random.default_rng(cols + rows)
    w = GEN[type_](rng, rows * cols // QUANTS[type_]["block"])
    x = (rng.standard_normal(cols) * 2).astype(np.float32)
    nw = (1 + rng.uniform(-0.2, 0.2, cols)).astype(np.float32)
    wb, xb, nb = gpu.upload_weights(type_, cols, rows, w), gpu.upload(x, "x"), gpu.upload(nw, "norm")
    qb = gpu.quantized_buffer(cols)
    gpu.quantize(xb, cols, qb, nb if normed else None, 1e-6)
    cap = 96
    yb = gpu.buffer(cap * rows * 4, "y per shape")
    n = gpu.matvec_shapes(type_, wb, qb, yb, cols, rows, cap)
    assert n >= 4, f"only {n} launch shapes"
    y = gpu.read_f32(yb, n * rows).reshape(n, rows)
    differ = [k for k in range(1, n) if not np.array_equal(y[k].view(np.uint32), y[0].view(np.uint32))]
    assert not differ, f"launch shapes {differ} of {n} differ from the cost model's"
    xn = orc.norm(x, nw, 1e-6).astype(np.float32) if normed else x
    near(y[0], orc.matmul(type_, w, xn, cols, rows, rows, 0, 0, 1), 1e-4, f"matvec {type_}")
    for b in (wb, xb, nb, yb, qb):
        gpu.destroy(b)
