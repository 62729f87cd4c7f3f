"""The float64 oracle under AddressSanitizer + UndefinedBehaviorSanitizer (CPU).

tests/native/oracle_san is oracle/oracle.c linked with a driver, both built with
-fsanitize=address,undefined and no recovery: any out-of-bounds access, leak, signed
overflow or misaligned access in the checker ends the run with a report and a non-zero
status. The driver checks each kernel against an independent statement of its result
(block decode vs element decode, matmul vs row dot products, rotation keeping pair
lengths, window-1 attention returning the own value row, ...), and runs bundled models
whose logits must equal the uninstrumented library's bit for bit.
"""
import os
import subprocess

import numpy as np
import pytest

from oracle import orc
from tests.native.bundle import write_bundle

HERE = os.path.dirname(os.path.abspath(__file__))
NATIVE = os.path.join(HERE, "native")
EXE = os.path.join(NATIVE, "_build", "oracle_san")
ENV = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0:halt_on_error=1",
           UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1", OMP_NUM_THREADS="4")


@pytest.fixture(scope="module")
def exe():
    subprocess.run(["make", "-s", "-C", NATIVE, "oracle"], check=True)
    return EXE


def run(args):
    r = subprocess.run(args, capture_output=True, text=True, env=ENV, timeout=600)
    report = r.stdout + r.stderr
    assert r.returncode == 0 and "Sanitizer" not in report and "runtime error" not in report, report[-4000:]
    return report


def test_oracle_ops_under_sanitizers(exe):
    assert "ok" in run([exe, "ops"])


@pytest.mark.parametrize("name,prompt,chunk,steps", [("tiny", 12, 8, 4), ("mini-gemma3", 40, 8, 6),
                                                     ("mini-llama", 20, 8, 5)])
def test_oracle_model_under_sanitizers(exe, tmp_path, name, prompt, chunk, steps):
    path, out = str(tmp_path / "m.bundle"), str(tmp_path / "m.out")
    f, g, c, caps, ids = write_bundle(path, name, 256, chunk, prompt, steps)
    run([exe, "model", path, out])
    raw = np.fromfile(out, np.uint8)
    v = c.vocab
    first = raw[:8 * v].view(np.float64)
    toks = raw[8 * v:8 * v + 4 * steps].view(np.int32)
    last = raw[8 * v + 4 * steps:].view(np.float64)
    ora = orc.OracleModel(f, g, c, 256, caps)
    want = None
    for i in range(0, prompt, chunk):
        want = ora.forward(ids[i:i + chunk], i, logits=i + chunk >= prompt)
    np.testing.assert_array_equal(first, want)
    expect, _ = orc.OracleModel(f, g, c, 256, caps).greedy(ids, steps, chunk)
    assert toks.tolist() == expect
    assert last.shape == (v,) and np.isfinite(last).all()
