"""Shared test setup: the `gpu` marker, the repo on sys.path, a session HIP context.

GPU tests call libwgd through its C ABI and compare against the float64 oracle in
oracle/ (the checker). Each GPU test announces itself on stdout before it starts, so a
run that loses the device still names the case.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and libwgd.so")


def pytest_runtest_setup(item):
    if item.get_closest_marker("gpu") is not None:
        sys.__stdout__.write(f"\n[gpu-case] {item.nodeid}\n")
        sys.__stdout__.flush()


@pytest.fixture(scope="session")
def gpu():
    from webgpu_amd.gpu import Compute
    c = Compute().init()
    yield c
    c.dispose()
