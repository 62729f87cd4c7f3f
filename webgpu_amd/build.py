"""Builds libwgd.so (HIP, gfx950) in-tree with hipcc: one object per source, then a link.

Usage: python -m webgpu_amd.build [--jobs N]. The library lands next to this file so it
travels with the source tree; nothing is installed.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "libwgd.so")
BUILD = os.path.join(HERE, "_build")
SOURCES = ["runtime.hip", "quant.hip", "matvec.hip", "gemm.hip", "ops.hip", "attention.hip", "model.hip", "sample.hip", "probe.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950", "-O3", "-fPIC", "-std=c++17",
    # Packed FP32 arithmetic stays off: only scalar f32 VALU forms are emitted.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-value", "-Wno-pass-failed", "-Wno-unused-function", "-Wno-unused-variable", "-Wno-unused-but-set-variable",
    "-I" + os.path.join(HERE, "..", "include"),
]
# The decode matvec waits on its weight loads for about half of a wavefront's life. LLVM's
# memory-clause scheduling strategy groups those loads, which makes the 14336x4096 Q4_K
# launch 3.6% faster and the Q6_K head 2.6% faster. Scheduling reorders no floating-point
# arithmetic, so the results are the same bits.
FILE_FLAGS = {"matvec.hip": ["-mllvm", "-amdgpu-sched-strategy=max-memory-clause"]}


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *FLAGS, *FILE_FLAGS.get(src, []), "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    noise = "is not a recognized feature for this target"
    msgs = [l for l in r.stderr.splitlines() if noise not in l and l.strip()]
    if msgs:
        sys.stderr.write("\n".join(msgs) + "\n")
    return obj


def build(jobs: int = 6) -> str:
    os.makedirs(BUILD, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = OUT + ".tmp"
    # -z defs: every symbol the library uses must be defined in it or in a linked library
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-Wl,-z,defs", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, OUT)
    build_napi()
    return OUT


NODE_INCLUDE = os.environ.get("NODE_INCLUDE", "/usr/include/node")
NAPI_SRC = os.path.join(HERE, "node", "wgd_napi.cc")
NAPI_OUT = os.path.join(HERE, "node", "wgd_napi.node")


def build_napi() -> str:
    """The Node addon over libwgd's C ABI (g++, no node-gyp): N-API symbols resolve against
    the node binary at load time, libwgd.so through an $ORIGIN rpath. Skipped when the Node
    headers are absent."""
    if not os.path.exists(os.path.join(NODE_INCLUDE, "node_api.h")):
        return ""
    tmp = NAPI_OUT + ".tmp"
    cmd = ["g++", "-std=c++17", "-O2", "-fPIC", "-shared", "-Wall", "-DNODE_GYP_MODULE_NAME=wgd_napi",
           "-I" + NODE_INCLUDE, "-I" + os.path.join(HERE, "..", "include"), NAPI_SRC,
           "-L" + HERE, "-lwgd", "-Wl,-rpath,$ORIGIN/..", "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"N-API addon build failed:\n{r.stderr}")
    os.replace(tmp, NAPI_OUT)
    return NAPI_OUT


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=6)
    print(build(ap.parse_args().jobs))
