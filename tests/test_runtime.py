"""The runtime API (webgpu_amd/runtime.py) against the rules of src/sdk.ts and
src/worker.ts, with a scripted engine standing in for the GPU one: one request at a time,
stop and early exit, errors and their AbortError kind, progress, reset and dispose."""
import threading
import time

import pytest

from webgpu_amd.engine import AbortError, ModelInfo, TokenEvent
from webgpu_amd.runtime import WebGPU


class ScriptedEngine:
    """The engine surface the worker drives; tokens come from a counter, and ``gate``
    (when set) holds each token until the test releases it."""
    instances = []

    def __init__(self, progress):
        self.progress = progress
        self.gate = None
        self.cache = []
        self.disposed = False
        self.thread = None
        ScriptedEngine.instances.append(self)

    def load(self, source, options, signal=None):
        self.thread = threading.current_thread()
        if source == "bad":
            raise ValueError("Unsupported GGUF version.")
        self.progress({"phase": "loading", "detail": "Uploading weights", "fraction": 0.5})
        signal.throw_if_aborted()
        return ModelInfo(None, 123, "test", 512, None, 16, "low-memory", {})

    def generate(self, messages, options=None, signal=None):
        if not messages:
            raise ValueError("Provide user/assistant text messages.")
        assert threading.current_thread() is self.thread
        self.cache = [1, 2, 3]
        try:
            for i in range(options if isinstance(options, int) else 5):
                if self.gate is not None:
                    self.gate.acquire()
                signal.throw_if_aborted()
                yield TokenEvent(i, "x" * (i + 1), "x", i + 1, 3, 512, 0.0, {})
        except BaseException:
            self.cache = []
            raise

    def reset(self):
        self.cache = []

    def dispose(self):
        self.disposed = True


@pytest.fixture
def rt():
    ScriptedEngine.instances.clear()
    r = WebGPU(ScriptedEngine)
    yield r
    r.dispose()


def test_load_reports_progress_and_returns_the_model_info(rt):
    seen = []
    rt.onProgress = seen.append
    info = rt.load("model.gguf")
    assert info.fileBytes == 123 and info.performance == "low-memory"
    assert seen == [{"phase": "loading", "detail": "Uploading weights", "fraction": 0.5}]
    # every engine call runs on the worker thread, not the caller's
    assert ScriptedEngine.instances[0].thread is not threading.current_thread()


def test_generate_streams_every_token(rt):
    rt.load("model.gguf")
    events = list(rt.generate([{"role": "user", "content": "hi"}]))
    assert [e.token for e in events] == [0, 1, 2, 3, 4] and events[-1].text == "xxxxx"


def test_errors_reach_the_caller_and_free_the_runtime(rt):
    with pytest.raises(RuntimeError, match="Load a model first"):
        list(rt.generate([{"role": "user", "content": "hi"}]))
    with pytest.raises(RuntimeError, match="Unsupported GGUF version"):
        rt.load("bad")
    rt.load("model.gguf")
    with pytest.raises(RuntimeError, match="Provide user/assistant") as e:
        list(rt.generate([]))
    assert not isinstance(e.value, AbortError)
    assert len(list(rt.generate([{"role": "user", "content": "hi"}]))) == 5


def test_a_second_request_while_one_runs_is_busy(rt):
    rt.load("model.gguf")
    eng = ScriptedEngine.instances[0]
    eng.gate = threading.Semaphore(0)
    it = rt.generate([{"role": "user", "content": "hi"}])
    eng.gate.release()
    assert next(it).token == 0
    with pytest.raises(RuntimeError, match="The runtime is busy"):
        list(rt.generate([{"role": "user", "content": "again"}]))
    with pytest.raises(RuntimeError, match="The runtime is busy"):
        rt.reset()
    for _ in range(4):
        eng.gate.release()
    assert [e.token for e in it] == [1, 2, 3, 4]
    rt.reset()


def test_stop_aborts_with_abort_error_and_drops_the_prefix(rt):
    rt.load("model.gguf")
    eng = ScriptedEngine.instances[0]
    eng.gate = threading.Semaphore(0)
    it = rt.generate([{"role": "user", "content": "hi"}])
    eng.gate.release()
    assert next(it).token == 0
    rt.stop()
    eng.gate.release()
    with pytest.raises(AbortError, match="Stopped by user"):
        list(it)
    assert eng.cache == []
    eng.gate = None
    assert len(list(rt.generate([{"role": "user", "content": "hi"}]))) == 5


def test_leaving_the_loop_early_stops_the_worker_without_an_error(rt):
    rt.load("model.gguf")
    eng = ScriptedEngine.instances[0]
    for ev in rt.generate([{"role": "user", "content": "hi"}], 10 ** 9):
        if ev.token == 2:
            break
    # the loop has returned only after the worker finished: the runtime is free
    assert len(list(rt.generate([{"role": "user", "content": "hi"}]))) == 5


def test_load_replaces_and_disposes_the_previous_engine(rt):
    rt.load("model.gguf")
    rt.load("model.gguf")
    a, b = ScriptedEngine.instances
    assert a.disposed and not b.disposed


def test_dispose_fails_the_pending_request_and_every_later_call():
    ScriptedEngine.instances.clear()
    rt = WebGPU(ScriptedEngine)
    rt.load("model.gguf")
    eng = ScriptedEngine.instances[0]
    eng.gate = threading.Semaphore(0)
    it = rt.generate([{"role": "user", "content": "hi"}])
    eng.gate.release()
    next(it)
    done = threading.Event()

    def release():
        while not done.is_set():
            eng.gate.release()
            time.sleep(0.01)
    t = threading.Thread(target=release)
    t.start()
    try:
        rt.dispose()
        with pytest.raises(RuntimeError, match="Runtime disposed"):
            list(it)
        with pytest.raises(RuntimeError, match="was disposed"):
            rt.load("model.gguf")
        assert eng.disposed
    finally:
        done.set()
        t.join()
