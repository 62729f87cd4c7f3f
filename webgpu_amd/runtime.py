"""``WebGPU``: the runtime API of ``src/sdk.ts`` with the worker of ``src/worker.ts``.

In the reference a browser Worker owns every GPU resource and the page talks to it by
messages. Here one worker thread owns the engine and its libwgd context (a context is
used from one host thread), and the caller's thread talks to it through queues with the
same message kinds (progress, token, done, error) and the same rules:

* one request at a time: a second one while the first runs fails with "The runtime is
  busy." (sdk.ts:16, worker.ts:9);
* ``stop()`` aborts the running request (worker.ts:8); the engine raises ``AbortError``
  at its next check and drops its cached prefix (engine.ts:299);
* leaving a ``generate`` loop early stops the generation and waits for the worker to
  finish before returning (sdk.ts:37-44), without raising;
* ``dispose()`` ends the worker; a pending request fails with "Runtime disposed." and
  every later call with the disposed error (sdk.ts:15,48).
"""
from __future__ import annotations

import queue
import threading
from typing import Any, Callable, Iterator, Optional

from .engine import AbortError, AbortSignal, GenerationOptions, LoadOptions, PagedEngine, TokenEvent

_STOP = object()


class WebGPU:
    """The reference's ``class WebGPU`` (sdk.ts:6-49) over a worker thread."""

    def __init__(self, engine_factory: Callable[..., Any] = PagedEngine) -> None:
        self.onProgress: Optional[Callable[[dict], None]] = None
        self._factory = engine_factory
        self._sequence = 0
        self._busy = False
        self._disposed = False
        self._lock = threading.Lock()
        self._pending: Optional[queue.Queue] = None
        # the running request's abort flag: created with the request, so a stop() that
        # follows it at once still reaches it (the cancel message of sdk.ts:46 queues
        # behind the request it cancels)
        self._signal: Optional[AbortSignal] = None
        self._inbox: queue.Queue = queue.Queue()
        # worker state (worker.ts:3-5): only the worker thread touches the engine
        self._engine = None
        self._thread = threading.Thread(target=self._worker, name="wgd-worker", daemon=True)
        self._thread.start()

    # ------------------------------------------------------------------ caller side
    def _request(self, action: str, payload: dict) -> queue.Queue:
        with self._lock:
            if self._disposed:
                raise RuntimeError("This runtime was disposed. Create a new WebGPU instance.")
            if self._busy:
                raise RuntimeError("The runtime is busy.")
            self._busy = True
            self._sequence += 1
            replies: queue.Queue = queue.Queue()
            self._pending, self._signal = replies, AbortSignal()
            item = (self._sequence, action, payload, replies, self._signal)
        self._inbox.put(item)
        return replies

    def _next(self, replies: queue.Queue):
        """The next message of a request. A done or error message ends the request (the
        runtime is free again); an error message raises."""
        m = replies.get()
        if m["type"] == "progress" and self.onProgress is not None:
            self.onProgress(m["value"])
        elif m["type"] in ("done", "error"):
            with self._lock:
                if self._pending is replies:
                    self._pending, self._signal, self._busy = None, None, False
            if m["type"] == "error":
                raise (AbortError if m.get("aborted") else RuntimeError)(m["error"])
        return m

    def _wait(self, replies: queue.Queue):
        while True:
            m = self._next(replies)
            if m["type"] == "done":
                return m.get("value")

    def load(self, source, options: Optional[LoadOptions] = None):
        """Load a GGUF (a path or bytes) on the worker; returns its ModelInfo."""
        return self._wait(self._request("load", {"source": source, "options": options}))

    def generate(self, messages, options: Optional[GenerationOptions] = None) -> Iterator[TokenEvent]:
        """TokenEvents of one reply as the worker produces them (sdk.ts:34-45). The request
        is sent when iteration starts, as for the reference's async generator."""
        replies = self._request("generate", {"messages": messages, "options": options})
        ended = False
        try:
            while True:
                try:
                    m = self._next(replies)
                except RuntimeError:
                    ended = True
                    raise
                if m["type"] == "token":
                    yield m["value"]
                elif m["type"] == "done":
                    ended = True
                    return
        finally:
            if not ended:
                # left early: stop the worker and wait for its answer, whatever it is
                self.stop()
                try:
                    self._wait(replies)
                except RuntimeError:
                    pass

    def stop(self) -> None:
        """Abort the running request (worker.ts:8)."""
        with self._lock:
            signal = self._signal
        if signal is not None:
            signal.abort("Stopped by user")

    def reset(self) -> None:
        """Forget the cached conversation prefix."""
        self._wait(self._request("reset", {}))

    def dispose(self) -> None:
        with self._lock:
            self._disposed = True
            pending, signal = self._pending, self._signal
            self._pending, self._signal, self._busy = None, None, False
        if signal is not None:
            signal.abort("Runtime disposed.")
        self._inbox.put(_STOP)
        if pending is not None:
            pending.put({"type": "error", "error": "Runtime disposed."})
        if threading.current_thread() is not self._thread:
            self._thread.join()

    # ------------------------------------------------------------------ worker side
    def _worker(self) -> None:
        while True:
            item = self._inbox.get()
            if item is _STOP:
                break
            rid, action, payload, replies, signal = item
            post = replies.put
            try:
                if action == "load":
                    if self._engine is not None:
                        self._engine.dispose()
                    self._engine = self._factory(lambda p: post({"id": rid, "type": "progress", "value": p}))
                    info = self._engine.load(payload["source"], payload["options"], signal=signal)
                    post({"id": rid, "type": "done", "value": info})
                elif action == "generate":
                    if self._engine is None:
                        raise RuntimeError("Load a model first.")
                    for token in self._engine.generate(payload["messages"], payload["options"], signal=signal):
                        post({"id": rid, "type": "token", "value": token})
                    post({"id": rid, "type": "done"})
                elif action == "reset":
                    if self._engine is not None:
                        self._engine.reset()
                    post({"id": rid, "type": "done"})
                else:
                    raise RuntimeError("Unknown runtime action.")
            except Exception as e:  # noqa: BLE001 - every failure is reported to the caller
                post({"id": rid, "type": "error", "error": str(e), "aborted": signal.aborted})
        if self._engine is not None:
            self._engine.dispose()
            self._engine = None
