"""``PagedEngine``: host mirror of ``src/core/engine.ts`` driving the native decoder.

The public surface follows the reference engine (engine.ts:26-324): ``load`` →
``ModelInfo``, ``generate`` → TokenEvents, ``reset``, ``dispose``, ``info`` and the
greedy ``sample``. GGUF parsing, configuration and KV-ring sizing run on the host exactly
as in gguf.ts/context.ts; weights are uploaded once and stay resident (the pager of
pager.ts collapses), and each forward / decode step runs inside libwgd on the GPU.

``generate`` takes chat messages (``[{"role": "user", "content": ...}]``), framed by the
GGUF's own tokenizer (tokenizer.py, picked as engine.ts:67-69 does), or prompt token ids.
A ``tokenizer`` argument (any object with ``chat``, ``decode`` and ``eos``) overrides the
model's. ``load`` and ``generate`` take an ``AbortSignal`` (the AbortController of
engine.ts:51,257): an aborted signal stops them at the next weight upload, prompt batch or
token with ``AbortError``, and a stopped generation drops the cached prefix as the
reference does (engine.ts:299).
"""
from __future__ import annotations

import ctypes as C
import math
import mmap
import os
import threading
import time
from dataclasses import dataclass, field
from typing import Any, Dict, Iterator, List, Optional, Sequence

import numpy as np

from .context import MAX_CONTEXT, MAX_MESSAGE_CHARS, attention_memory, output_limit, validate_context
from .gguf import GGUF, ModelConfig, Tensor, model_config, read_gguf
from .gpu import Compute, ModelConfigC, WgdError, lib
from .tokenizer import tokenizer_for

BATCHES = (1, 8, 16, 32, 64, 128)
# engine.ts:14-18. The prompt batch of each performance mode; the budget and page size of
# the reference presets belong to its weight pager, which has no counterpart here (every
# weight is resident).
PRESETS = {"lite": 8, "low-memory": 16, "fast": 128}


class AbortError(RuntimeError):
    """A load or generation stopped through its ``AbortSignal`` (the DOMException named
    'AbortError' of worker.ts:9)."""


class AbortSignal:
    """A thread-safe abort flag with the AbortSignal surface the engine uses."""

    def __init__(self) -> None:
        self._event = threading.Event()
        self.reason = "Stopped by user"

    @property
    def aborted(self) -> bool:
        return self._event.is_set()

    def abort(self, reason: str = "Stopped by user") -> None:
        self.reason = reason
        self._event.set()

    def throw_if_aborted(self) -> None:
        if self._event.is_set():
            raise AbortError(self.reason)


def _check(signal: Optional[AbortSignal]) -> None:
    if signal is not None:
        signal.throw_if_aborted()


class ByteSource:
    """Random-access bytes (source.ts:2-6) over a file (mmap) or an in-memory buffer."""

    def __init__(self, data, name: str = "model.gguf") -> None:
        self._mm = None
        if isinstance(data, (str, os.PathLike)):
            self.name = os.path.basename(str(data))
            fd = os.open(str(data), os.O_RDONLY)
            try:
                size = os.fstat(fd).st_size
                if size < 24:
                    raise ValueError("Invalid model file size.")
                self._mm = mmap.mmap(fd, size, prot=mmap.PROT_READ)
            finally:
                os.close(fd)
            self._view = np.frombuffer(self._mm, np.uint8)
        else:
            self.name = name
            self._view = np.frombuffer(data, np.uint8) if not isinstance(data, np.ndarray) else data.reshape(-1).view(np.uint8)
        self.size = int(self._view.size)
        if self.size < 24:
            raise ValueError("Invalid model file size.")

    def read(self, offset: int, length: int) -> np.ndarray:
        if offset < 0 or length < 1 or offset + length > self.size:
            raise ValueError("Invalid model byte range.")
        return self._view[offset:offset + length]

    def close(self) -> None:
        self._view = None
        if self._mm is not None:
            self._mm.close()
            self._mm = None


@dataclass
class LoadOptions:
    """engine.ts:19. ``batchSize`` defaults to the performance mode's batch.
    ``gpuBudgetMiB`` caps the context's device allocations (None: no cap); the reference's
    16 GiB ceiling is a browser limit and is not applied. ``kvCacheType`` "f16" keeps the K/V
    rings in half precision (values rounded to nearest even when cached, attention math in
    f32): half the ring memory and the bytes a decode step reads. The reference's rings are
    f32 (engine.ts:98-101), the default."""
    contextLength: int = 512
    batchSize: Optional[int] = None
    gpuBudgetMiB: Optional[int] = None
    performance: str = "low-memory"
    device: int = 0
    kvCacheType: str = "f32"


@dataclass
class GenerationOptions:
    """engine.ts:21, validated as engine.ts:261-264, with the reference's defaults.
    ``seed`` picks the uniforms that stand in for Math.random() (None: a fresh one per
    call); the same seed, settings and prompt give the same tokens."""
    maxTokens: int = 128
    temperature: float = 0.7
    topK: int = 40
    topP: float = 0.9
    seed: Optional[int] = None


@dataclass
class TokenEvent:
    token: int
    text: str
    delta: str
    tokens: int
    promptTokens: int
    contextLength: int
    seconds: float
    stats: Dict[str, Any] = field(default_factory=dict)


@dataclass
class ModelInfo:
    """engine.ts:23."""
    config: ModelConfig
    fileBytes: int
    adapter: str
    contextLength: int
    gpuBudgetMiB: Optional[int]
    batchSize: int
    performance: str
    stats: Dict[str, Any]


def _config_struct(c: ModelConfig, context: int, batch: int, kv_f16: bool = False) -> ModelConfigC:
    s = ModelConfigC()
    gemma = c.family == "gemma3"
    s.family = 1 if gemma else 0
    s.rope_adjacent = 1 if c.rope == "norm" else 0
    s.hidden, s.intermediate, s.layers = c.hidden, c.intermediate, c.layers
    s.heads, s.kv_heads, s.head_dim, s.vocab = c.heads, c.kvHeads, c.headDim, c.vocab
    s.rotary_dim = c.rotaryDim
    s.window = c.window if gemma else c.slidingWindow
    s.period = c.period
    s.qk_norm = 1 if c.qkNorm else 0
    s.ffn_gate = 1 if c.ffnGate else 0
    s.gelu = 1 if c.activation == "gelu" else 0
    s.bias_q, s.bias_k, s.bias_v, s.bias_output = (1 if c.bias[k] else 0 for k in ("q", "k", "v", "output"))
    s.context, s.batch = context, batch
    s.epsilon, s.theta, s.local_theta = c.epsilon, c.theta, c.localTheta
    s.attention_scale, s.rope_scale = c.attentionScale, c.ropeScale
    s.embed_scale = math.sqrt(c.hidden) if c.architecture == "gemma3" else 1.0
    s.kv_f16 = 1 if kv_f16 else 0
    return s


class PagedEngine:
    """The dense-decoder engine with every weight resident on one MI355X."""

    def __init__(self, progress=None) -> None:
        self.progress = progress or (lambda p: None)
        self.gpu: Optional[Compute] = None
        self.model: Optional[int] = None
        self.source: Optional[ByteSource] = None
        self.gguf: Optional[GGUF] = None
        self.config: Optional[ModelConfig] = None
        self.context = 512
        self.batch = 16
        self.budget: Optional[int] = None
        self.performance = "low-memory"
        self.kvCapacities: List[int] = []
        self.kvCacheType = "f32"
        self.busy = False
        self.disposed = False
        self.tokensInCache: List[int] = []
        self.tokenizer = None

    # ------------------------------------------------------------------ load
    def load(self, source, options: Optional[LoadOptions] = None, signal: Optional[AbortSignal] = None) -> ModelInfo:
        """PagedEngine.load (engine.ts:51-114): parse, configure, upload, seal."""
        o = options or LoadOptions()
        if o.performance not in PRESETS:
            raise ValueError("Performance must be lite, low-memory or fast.")
        self.performance = o.performance
        self.context = o.contextLength
        self.batch = o.batchSize if o.batchSize is not None else PRESETS[o.performance]
        validate_context(self.context)
        if self.batch not in BATCHES:
            raise ValueError("Batch size must be 1, 8, 16, 32, 64 or 128.")
        if o.gpuBudgetMiB is not None and (not isinstance(o.gpuBudgetMiB, int) or o.gpuBudgetMiB < 512):
            raise ValueError("GPU budget must be at least 512 MiB.")
        self.budget = o.gpuBudgetMiB
        if o.kvCacheType not in ("f32", "f16"):
            raise ValueError("KV cache type must be f32 or f16.")
        self.kvCacheType = o.kvCacheType
        self.source = source if isinstance(source, ByteSource) else ByteSource(source)
        self.progress({"phase": "loading", "detail": "Reading GGUF metadata", "fraction": 0.05})
        self.gguf = read_gguf(self.source)
        self.config = c = model_config(self.gguf)
        validate_context(self.context, c.maxContext)
        # the GGUF's tokenizer (None for a file that carries none: token-id prompts only)
        self.tokenizer = tokenizer_for(self.gguf.metadata, c.architecture, c.family)
        memory = attention_memory(c, self.context, self.batch, 2 if o.kvCacheType == "f16" else 4)
        self.kvCapacities = list(memory["capacities"])
        self.gpu = Compute(o.gpuBudgetMiB, o.device)
        try:
            self.gpu.init()
            cfg = _config_struct(c, self.context, self.batch, o.kvCacheType == "f16")
            cfg.tied_output = 0 if "output.weight" in self.gguf.tensors else 1
            caps = (C.c_int32 * c.layers)(*self.kvCapacities)
            out = C.c_void_p()
            self.gpu.check(lib().wgd_model_create(self.gpu.ctx, C.byref(cfg), caps, C.byref(out)))
            self.model = out.value
            tensors = [t for t in self.gguf.tensors.values()
                       if len(t.dims) in (1, 2) and (not t.name.startswith("blk.") or int(t.name.split(".")[1]) < c.layers)]
            for i, t in enumerate(tensors):
                _check(signal)
                self._upload(t)
                if i % 64 == 0:
                    self.progress({"phase": "loading", "detail": "Uploading weights", "fraction": 0.1 + 0.85 * i / len(tensors)})
            self.gpu.check(lib().wgd_model_ready(self.model))
            self.progress({"phase": "ready", "detail": "Ready.", "fraction": 1.0})
            return self.info()
        except Exception:
            self.dispose()
            raise

    def _upload(self, t: Tensor) -> None:
        data = self.source.read(t.offset, t.bytes)
        dims = (C.c_uint64 * len(t.dims))(*t.dims)
        self.gpu.check(lib().wgd_model_tensor(self.model, t.name.encode(), t.type, len(t.dims), dims,
                                              data.ctypes.data, t.bytes))

    def info(self) -> ModelInfo:
        return ModelInfo(self.config, self.source.size if self.source else 0, self.gpu.adapterName if self.gpu else "",
                         self.context, self.budget, self.batch, self.performance, self.stats())

    def stats(self) -> Dict[str, Any]:
        return {"gpuBytes": self.gpu.allocated if self.gpu else 0, "peakGpuBytes": self.gpu.peak if self.gpu else 0}

    # ------------------------------------------------------------------ forward
    def forward(self, ids: Sequence[int], start: int, logits: bool) -> Optional[np.ndarray]:
        """forward(ids, start, logits) (engine.ts:138-180): returns the last row's logits."""
        if self.model is None:
            raise RuntimeError("Load a model first.")
        n = len(ids)
        arr = (C.c_int32 * n)(*ids)
        out = np.empty(self.config.vocab, np.float32) if logits else None
        self.gpu.check(lib().wgd_model_forward(self.model, arr, n, start,
                                               out.ctypes.data if logits else None, None))
        return out

    def set_sampling(self, temperature: float, top_k: int = 40, top_p: float = 0.9, seed: int = 0) -> None:
        """The token pick of forward_argmax and decode: greedy at temperature 0, else
        sampled on the device with the uniforms of ``seed``."""
        self.gpu.check(lib().wgd_model_sampling(self.model, float(temperature), int(top_k), float(top_p),
                                                int(seed) & (2 ** 64 - 1)))

    def attention_timing(self, layer: int, pos: int, reps: int = 50) -> float:
        """Measurement: mean device microseconds of the decode step's attention launch of
        `layer` at position `pos` (it overwrites ring slot pos % capacity)."""
        us = C.c_double(0.0)
        self.gpu.check(lib().wgd_model_attention_timing(self.model, int(layer), int(pos), int(reps), C.byref(us)))
        return us.value

    def forward_argmax(self, ids: Sequence[int], start: int) -> int:
        """forward + the token pick (greedy, or sampled: set_sampling) on the device."""
        n = len(ids)
        arr = (C.c_int32 * n)(*ids)
        tok = C.c_int32(-1)
        self.gpu.check(lib().wgd_model_forward(self.model, arr, n, start, None, C.byref(tok)))
        return tok.value

    def decode(self, token: int, start: int, count: int) -> List[int]:
        """``count`` greedy steps on the device from ``token`` at ``start``."""
        out = (C.c_int32 * count)()
        self.gpu.check(lib().wgd_model_decode(self.model, token, start, count, out))
        return list(out)

    # ------------------------------------------------------------------ generate
    def generate(self, prompt, options: Optional[GenerationOptions] = None, tokenizer=None,
                 chunk: int = 32, signal: Optional[AbortSignal] = None) -> Iterator[TokenEvent]:
        """PagedEngine.generate (engine.ts:257-301): greedy at temperature 0, else top-k /
        top-p sampling on the device (wgd_model_sampling).

        Prefix reuse, output limit, chunked prefill and the busy guard follow the
        reference; the decode loop runs on the device ``chunk`` tokens at a time.

        A device chunk may run past an end-of-turn token: its keys land in ring slots
        beyond the cached prefix. A sliding ring holds the window plus one prompt batch
        (context.ts:14-23), so at most ``batch`` such positions leave every key the next
        turn reads in place; the chunk is capped to the batch on models with one."""
        if self.busy:
            raise RuntimeError("A generation is already running.")
        if self.disposed or self.model is None:
            raise RuntimeError("Load a model first.")
        o = options or GenerationOptions()
        if not isinstance(o.maxTokens, int) or o.maxTokens < 1 or o.maxTokens > MAX_CONTEXT:
            raise ValueError(f"maxTokens must be 1–{MAX_CONTEXT}.")
        t, k, p = o.temperature, o.topK, o.topP
        if (not isinstance(t, (int, float)) or not math.isfinite(t) or t < 0 or t > 2 or not isinstance(k, int)
                or k < 1 or k > 200 or not isinstance(p, (int, float)) or not math.isfinite(p) or p <= 0 or p > 1):
            raise ValueError("Invalid sampling settings.")
        tokenizer = tokenizer if tokenizer is not None else self.tokenizer
        messages = isinstance(prompt, (list, tuple)) and len(prompt) > 0 and all(isinstance(m, dict) for m in prompt)
        if messages:
            # engine.ts:260: user/assistant text messages of bounded length
            if any(m.get("role") not in ("user", "assistant") or not isinstance(m.get("content"), str) or
                   len(m["content"]) > MAX_MESSAGE_CHARS for m in prompt):
                raise ValueError(f"Provide user/assistant text messages (at most {MAX_MESSAGE_CHARS:,} characters each).")
            if tokenizer is None:
                raise ValueError("This model carries no tokenizer: pass prompt token ids.")
            ids = list(tokenizer.chat(prompt))
        else:
            ids = [int(t) for t in prompt]
        if not ids:
            raise ValueError("Provide a non-empty prompt.")
        eos = set(getattr(tokenizer, "eos", ()) or ())
        chunk = max(1, chunk)
        if any(cap < self.context for cap in self.kvCapacities):
            chunk = min(chunk, self.batch)
        return self._generate(ids, o, tokenizer, eos, chunk, signal)

    def _generate(self, prompt: List[int], o: GenerationOptions, tokenizer, eos, chunk: int,
                  signal: Optional[AbortSignal]) -> Iterator[TokenEvent]:
        # the guard is taken when iteration starts, as for the reference's async generator
        if self.busy:
            raise RuntimeError("A generation is already running.")
        self.busy = True
        try:
            limit = output_limit(o.maxTokens, len(prompt), self.context)
            seed = o.seed if o.seed is not None else int.from_bytes(os.urandom(8), "little")
            self.set_sampling(o.temperature, o.topK, o.topP, seed)
            shared = 0
            while shared < len(prompt) and shared < len(self.tokensInCache) and prompt[shared] == self.tokensInCache[shared]:
                shared += 1
            shared = min(shared, len(prompt) - 1)
            if shared < len(self.tokensInCache) and any(cap < self.context for cap in self.kvCapacities):
                shared = 0
            started = time.perf_counter()
            self.tokensInCache = self.tokensInCache[:shared]
            token = -1
            for i in range(shared, len(prompt), self.batch):
                _check(signal)
                batch = prompt[i:i + self.batch]
                last = i + len(batch) == len(prompt)
                if last:
                    token = self.forward_argmax(batch, i)
                else:
                    self.forward(batch, i, False)
                self.tokensInCache.extend(batch)
            generated: List[int] = []
            text = ""
            pending: List[int] = []
            for i in range(limit):
                _check(signal)
                if not pending and i > 0:
                    count = min(chunk, limit - i)
                    pending = self.decode(token, len(self.tokensInCache), count)
                    # decode fed `token` and the first count-1 outputs; they enter the
                    # cache as they are yielded below.
                    self.tokensInCache.append(token)
                    token = pending.pop(0)
                elif i > 0:
                    self.tokensInCache.append(token)
                    token = pending.pop(0)
                if token in eos:
                    break
                generated.append(token)
                full = tokenizer.decode(generated) if tokenizer is not None else ""
                delta = full[len(text):]
                text = full
                yield TokenEvent(token, text, delta, len(generated), len(prompt), self.context,
                                 time.perf_counter() - started, self.stats())
        except BaseException:
            self.tokensInCache = []
            raise
        finally:
            self.busy = False

    def reset(self) -> None:
        if self.busy:
            raise RuntimeError("Stop generation first.")
        self.tokensInCache = []

    def dispose(self) -> None:
        self.disposed = True
        if self.model is not None and self.gpu is not None and self.gpu.ctx:
            lib().wgd_model_destroy(self.model)
        self.model = None
        if self.gpu is not None:
            self.gpu.dispose()
        self.tokensInCache = []

    def sample(self, logits: np.ndarray, temperature: float = 0.0, top_k: int = 40, top_p: float = 0.9,
               seed: int = 0, index: int = 0) -> int:
        """sample() (engine.ts:305-324) on the device: the first strict maximum over finite
        logits at temperature 0, else a top-k / top-p draw with the index-th uniform of
        ``seed``; raises when no logit is finite."""
        buf = self.gpu.upload(np.asarray(logits, np.float32), "sample logits")
        try:
            n = int(np.asarray(logits).size)
            if temperature == 0:
                return self.gpu.argmax(buf, n)
            return self.gpu.sample(buf, n, temperature, top_k, top_p, seed, index)
        finally:
            self.gpu.destroy(buf)
