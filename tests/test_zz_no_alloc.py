"""wgd_attention_noalloc: the allocation-free variant of wgd_attention.

It has no counterpart in the reference (for callers that cannot allocate device memory).
Its split-K partials live in a static array of the library's device memory, so it must
give wgd_attention's results bit for bit (the same split plan, the same sums), allocate
nothing through the context, and reject sizes whose partials exceed the array. Two calls in
a row, the second smaller, check that the array's leftover contents from the first call do
not leak into the second.
"""
import re

import numpy as np
import pytest

from webgpu_amd.gpu import WgdError, lib

pytestmark = pytest.mark.gpu


def _case(gpu, rng, heads, kvh, hd, start, batch, window, capacity):
    q = (rng.standard_normal(batch * heads * hd) * 2).astype(np.float32)
    k = rng.standard_normal(capacity * kvh * hd).astype(np.float32)
    v = rng.standard_normal(capacity * kvh * hd).astype(np.float32)
    bufs = [gpu.upload(a, nm) for a, nm in ((q, "q"), (k, "k"), (v, "v"))]
    return bufs, q.size


def test_noalloc_attention_matches_the_allocating_entry_point():
    from webgpu_amd.gpu import Compute
    gpu = Compute().init()
    try:
        rng = np.random.default_rng(11)
        # a prompt batch deep in the context (MFMA kernel, several splits), then a smaller
        # ragged batch on the generic kernel (head_dim 96) over a wrapped ring
        cases = [(32, 8, 128, 700, 128, 4096, 1024), (6, 2, 96, 300, 9, 64, 128)]
        for heads, kvh, hd, start, batch, window, capacity in cases:
            bufs, n = _case(gpu, rng, heads, kvh, hd, start, batch, window, capacity)
            y0, y1 = gpu.buffer(n * 4, "y0"), gpu.buffer(n * 4, "y1")
            scale = float(1 / np.sqrt(hd))
            before = gpu.allocated
            gpu.attention_noalloc(*bufs, y1, heads, kvh, hd, start, scale, window, capacity, capacity, batch)
            got = gpu.read_f32(y1, n)
            assert gpu.allocated == before, "the allocation-free entry point allocated through the context"
            gpu.attention(*bufs, y0, heads, kvh, hd, start, scale, window, capacity, capacity, batch)
            want = gpu.read_f32(y0, n)
            assert np.isfinite(got).all()
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), \
                f"max abs difference {np.abs(got - want).max():.3e} for {heads}/{kvh} heads, hd {hd}, batch {batch}"
            for b in bufs + [y0, y1]:
                gpu.destroy(b)
        # sizes beyond the static scratch fail with a clear error and launch nothing
        limit = int(lib().wgd_attention_noalloc_limit())
        heads, kvh, hd, batch, cap = 64, 8, 512, 128, 4096
        per_split = batch * heads * (hd + 2)
        # head_dim 512 runs the generic kernel: 2-query blocks for groups of 8 heads, and keys
        # split over about four workgroups per CU (attn_plan in attention.hip); one split
        # needs no scratch at all
        cus = int(re.search(r"(\d+) CUs", gpu.adapterName).group(1))
        nsplit = cus * 4 // (kvh * (batch // 2))
        if nsplit < 2 or nsplit * per_split <= limit:
            pytest.skip(f"{cus} CUs give {nsplit} key splits, whose partials fit the static scratch")
        bufs, n = _case(gpu, rng, heads, kvh, hd, 3000, batch, 4096, cap)
        y = gpu.buffer(n * 4, "y")
        with pytest.raises(WgdError, match="static scratch holds"):
            gpu.attention_noalloc(*bufs, y, heads, kvh, hd, 3000, 0.05, 4096, cap, cap, batch)
        for b in bufs + [y]:
            gpu.destroy(b)
    finally:
        gpu.dispose()
