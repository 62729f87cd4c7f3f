"""``Compute``: host mirror of ``src/core/gpu.ts`` over the libwgd C ABI.

Every method calls straight into ``libwgd.so`` (HIP, gfx950); there is no CPU fallback.
A missing library or device raises at construction, and a non-zero status from the
library is raised as ``WgdError`` carrying ``wgd_last_error`` (the reference throws the
same way, gpu.ts:20-27). Kernel methods take the WGSL uniform parameters of the
pipeline they replace (src/core/shaders.ts).
"""
from __future__ import annotations

import ctypes as C
import os
from typing import Optional

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libwgd.so")

WGD_OK, WGD_E_INVALID, WGD_E_BUDGET, WGD_E_DEVICE, WGD_E_NONFINITE, WGD_E_STATE = range(6)

# C ABI exports, as declared in include/wgd.h (name -> (restype, argtypes)).
_P, _U32, _U64, _I32, _F, _D = C.c_void_p, C.c_uint32, C.c_uint64, C.c_int32, C.c_float, C.c_double
SIGNATURES = {
    "wgd_create": (C.c_int, [_I32, _U64, C.POINTER(_P)]),
    "wgd_destroy": (None, [_P]),
    "wgd_last_error": (C.c_char_p, [_P]),
    "wgd_adapter_name": (C.c_char_p, [_P]),
    "wgd_allocated": (_U64, [_P]),
    "wgd_peak": (_U64, [_P]),
    "wgd_buffer_create": (C.c_int, [_P, _U64, C.c_char_p, C.POINTER(_P)]),
    "wgd_buffer_destroy": (C.c_int, [_P, _P]),
    "wgd_buffer_size": (_U64, [_P]),
    "wgd_upload_weights": (C.c_int, [_P, _I32, _U32, _U32, _P, _U64, C.c_char_p, C.POINTER(_P)]),
    "wgd_stream": (_P, [_P]),
    "wgd_write": (C.c_int, [_P, _P, _U64, _P, _U64]),
    "wgd_read": (C.c_int, [_P, _P, _U64, _P, _U64]),
    "wgd_copy": (C.c_int, [_P, _P, _P, _U64, _U64, _U64]),
    "wgd_clear": (C.c_int, [_P, _P]),
    "wgd_done": (C.c_int, [_P]),
    "wgd_matmul": (C.c_int, [_P, _I32, _P, _P, _P, _U32, _U32, _U32, _U32, _U32, _U32]),
    "wgd_dequant": (C.c_int, [_P, _I32, _P, _P, _U64]),
    "wgd_quantized_bytes": (_U64, [_U32]),
    "wgd_quantize": (C.c_int, [_P, _P, _U32, _P, _F, _P]),
    "wgd_matvec": (C.c_int, [_P, _I32, _P, _P, _P, _U32, _U32, _U32]),
    "wgd_matvec_shapes": (C.c_int, [_P, _I32, _P, _P, _P, _U32, _U32, _U32, C.POINTER(_U32)]),
    "wgd_norm": (C.c_int, [_P, _P, _P, _P, _U32, _F, _U32]),
    "wgd_rope_norm": (C.c_int, [_P, _P, _P, _U32, _U32, _U32, _F, _F, _F, _U32, _U32]),
    "wgd_rope_neox": (C.c_int, [_P, _P, _U32, _U32, _U32, _F, _F, _U32, _U32]),
    "wgd_rope_adjacent": (C.c_int, [_P, _P, _U32, _U32, _U32, _F, _F, _U32, _U32]),
    "wgd_attention": (C.c_int, [_P, _P, _P, _P, _P, _U32, _U32, _U32, _U32, _F, _U32, _U32, _U32, _U32]),
    "wgd_attention_noalloc": (C.c_int, [_P, _P, _P, _P, _P, _U32, _U32, _U32, _U32, _F, _U32, _U32, _U32, _U32]),
    "wgd_attention_noalloc_limit": (_U64, []),
    "wgd_attention_f16kv": (C.c_int, [_P, _P, _P, _P, _P, _U32, _U32, _U32, _U32, _F, _U32, _U32, _U32, _U32]),
    "wgd_kv_store_f16": (C.c_int, [_P, _P, _P, _U64, _U64, _U64]),
    "wgd_probe_read": (C.c_int, [_P, _P, _U64, _U32, _U32, _U32, _U32, _U32, _P, _U32]),
    "wgd_add": (C.c_int, [_P, _P, _P, _U32]),
    "wgd_silu": (C.c_int, [_P, _P, _P, _P, _U32]),
    "wgd_gelu": (C.c_int, [_P, _P, _P, _P, _U32]),
    "wgd_bias_add": (C.c_int, [_P, _P, _P, _U32, _U32]),
    "wgd_activate": (C.c_int, [_P, _P, _U32]),
    "wgd_argmax": (C.c_int, [_P, _P, _U32, _P, C.POINTER(_I32)]),
    "wgd_sample": (C.c_int, [_P, _P, _U32, C.c_double, _U32, C.c_double, C.c_uint64, _U32, C.POINTER(_I32)]),
    "wgd_model_attention_timing": (C.c_int, [_P, C.c_int32, C.c_int32, C.c_int32, C.POINTER(C.c_double)]),
    "wgd_model_sampling": (C.c_int, [_P, C.c_double, _U32, C.c_double, C.c_uint64]),
    "wgd_embed": (C.c_int, [_P, _I32, _P, _P, _P, _U32, _U32, _D]),
    "wgd_model_create": (C.c_int, [_P, _P, C.POINTER(_I32), C.POINTER(_P)]),
    "wgd_model_tensor": (C.c_int, [_P, C.c_char_p, _I32, _I32, C.POINTER(_U64), _P, _U64]),
    "wgd_model_ready": (C.c_int, [_P]),
    "wgd_model_forward": (C.c_int, [_P, C.POINTER(_I32), _I32, _I32, _P, C.POINTER(_I32)]),
    "wgd_model_decode": (C.c_int, [_P, _I32, _I32, _I32, C.POINTER(_I32)]),
    "wgd_model_destroy": (None, [_P]),
}


class WgdError(RuntimeError):
    def __init__(self, status: int, message: str) -> None:
        super().__init__(message)
        self.status = status


_lib: Optional[C.CDLL] = None


def lib() -> C.CDLL:
    """Loads libwgd.so (built in-tree by ``python -m webgpu_amd.build``)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m webgpu_amd.build`. "
                               "There is no CPU fallback.")
        l = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(l, name)
            f.restype = res
            f.argtypes = args
        _lib = l
    return _lib


class ModelConfigC(C.Structure):
    """wgd_model_config (include/wgd.h)."""
    _fields_ = [(n, C.c_int32) for n in (
        "family", "rope_adjacent", "hidden", "intermediate", "layers", "heads", "kv_heads", "head_dim", "vocab",
        "rotary_dim", "window", "period", "qk_norm", "ffn_gate", "gelu", "bias_q", "bias_k", "bias_v",
        "bias_output", "tied_output", "context", "batch")] + [(n, C.c_float) for n in (
        "epsilon", "theta", "local_theta", "attention_scale", "rope_scale")] + [("embed_scale", C.c_double),
                                                                                  ("kv_f16", C.c_int32)]


class Buffer:
    """A device buffer handle (GPUBuffer of the reference)."""
    __slots__ = ("ptr", "size", "label")

    def __init__(self, ptr: int, size: int, label: str) -> None:
        self.ptr, self.size, self.label = ptr, size, label


def _host(data) -> np.ndarray:
    a = np.ascontiguousarray(data)
    return a.view(np.uint8).reshape(-1) if a.dtype != np.uint8 else a.reshape(-1)


class Compute:
    """Mirror of ``Compute`` (gpu.ts:2-67) backed by one HIP context and stream."""

    def __init__(self, budget_mib: Optional[int] = None, device: int = 0) -> None:
        self.limit = 0 if budget_mib is None else int(budget_mib) * 1024 ** 2
        self.device = device
        self.ctx: Optional[int] = None
        self.adapterName = ""

    # -- lifecycle -------------------------------------------------------------------
    def init(self) -> "Compute":
        l = lib()
        out = C.c_void_p()
        st = l.wgd_create(self.device, self.limit, C.byref(out))
        if st:
            raise WgdError(st, l.wgd_last_error(None).decode())
        self.ctx = out.value
        self.adapterName = l.wgd_adapter_name(self.ctx).decode()
        return self

    def check(self, status: int) -> None:
        if status:
            raise WgdError(status, lib().wgd_last_error(self.ctx).decode())

    def dispose(self) -> None:
        if self.ctx:
            lib().wgd_destroy(self.ctx)
            self.ctx = None

    @property
    def allocated(self) -> int:
        return lib().wgd_allocated(self.ctx) if self.ctx else 0

    @property
    def peak(self) -> int:
        return lib().wgd_peak(self.ctx) if self.ctx else 0

    # -- buffers ---------------------------------------------------------------------
    def buffer(self, size: int, label: str = "buffer") -> Buffer:
        out = C.c_void_p()
        self.check(lib().wgd_buffer_create(self.ctx, int(size), label.encode(), C.byref(out)))
        return Buffer(out.value, lib().wgd_buffer_size(out.value), label)

    def destroy(self, b: Buffer) -> None:
        self.check(lib().wgd_buffer_destroy(self.ctx, b.ptr))

    def write(self, b: Buffer, data, offset: int = 0) -> None:
        h = _host(data)
        self.check(lib().wgd_write(self.ctx, b.ptr, offset, h.ctypes.data, h.nbytes))

    def upload(self, data, label: str = "upload") -> Buffer:
        h = _host(data)
        b = self.buffer(max(4, h.nbytes), label)
        self.write(b, h)
        return b

    def upload_weights(self, type_: int, cols: int, rows: int, data, label: str = "weights") -> Buffer:
        """WeightPager.page collapsed: one upload of a whole matrix in the device layout."""
        h = _host(data)
        out = C.c_void_p()
        self.check(lib().wgd_upload_weights(self.ctx, type_, cols, rows, h.ctypes.data, h.nbytes, label.encode(),
                                            C.byref(out)))
        return Buffer(out.value, lib().wgd_buffer_size(out.value), label)

    @property
    def stream(self) -> int:
        return lib().wgd_stream(self.ctx)

    def read(self, b: Buffer, size: int, offset: int = 0) -> bytes:
        out = np.empty(int(size), np.uint8)
        self.check(lib().wgd_read(self.ctx, b.ptr, offset, out.ctypes.data, int(size)))
        return out.tobytes()

    def read_f32(self, b: Buffer, count: int, offset: int = 0) -> np.ndarray:
        out = np.empty(int(count), np.float32)
        self.check(lib().wgd_read(self.ctx, b.ptr, offset, out.ctypes.data, out.nbytes))
        return out

    def copy(self, src: Buffer, dst: Buffer, size: int, src_offset: int = 0, dst_offset: int = 0) -> None:
        self.check(lib().wgd_copy(self.ctx, src.ptr, dst.ptr, size, src_offset, dst_offset))

    def clear(self, buffers) -> None:
        for b in buffers:
            self.check(lib().wgd_clear(self.ctx, b.ptr))

    def done(self) -> None:
        self.check(lib().wgd_done(self.ctx))

    # -- kernels (WGSL pipelines of src/core/shaders.ts) -------------------------------
    def matmul(self, type_: int, w: Buffer, x: Buffer, y: Buffer, cols: int, rows: int, stride: int,
               row_base: int, input_offset: int, batch: int = 1) -> None:
        self.check(lib().wgd_matmul(self.ctx, type_, w.ptr, x.ptr, y.ptr, cols, rows, stride, row_base,
                                    input_offset, batch))

    def quantized_buffer(self, cols: int, label: str = "quantized activation") -> Buffer:
        return self.buffer(lib().wgd_quantized_bytes(cols), label)

    def quantize(self, x: Buffer, cols: int, qx: Buffer, norm_weight: Optional[Buffer] = None,
                 epsilon: float = 0.0) -> None:
        self.check(lib().wgd_quantize(self.ctx, x.ptr, cols, norm_weight.ptr if norm_weight else None, epsilon, qx.ptr))

    def matvec(self, type_: int, w: Buffer, qx: Buffer, y: Buffer, cols: int, rows: int, row_base: int = 0) -> None:
        self.check(lib().wgd_matvec(self.ctx, type_, w.ptr, qx.ptr, y.ptr, cols, rows, row_base))

    def matvec_shapes(self, type_: int, w: Buffer, qx: Buffer, y: Buffer, cols: int, rows: int,
                      max_shapes: int) -> int:
        """wgd_matvec once per launch shape the decode step's measurement may pick; returns the
        number of shapes run (shape k wrote y[k * rows:(k + 1) * rows])."""
        n = C.c_uint32(0)
        self.check(lib().wgd_matvec_shapes(self.ctx, type_, w.ptr, qx.ptr, y.ptr, cols, rows, max_shapes, C.byref(n)))
        return n.value

    def dequant(self, type_: int, w: Buffer, out: Buffer, count: int) -> None:
        self.check(lib().wgd_dequant(self.ctx, type_, w.ptr, out.ptr, count))

    def norm(self, x: Buffer, w: Buffer, y: Buffer, n: int, epsilon: float, batch: int = 1) -> None:
        self.check(lib().wgd_norm(self.ctx, x.ptr, w.ptr, y.ptr, n, epsilon, batch))

    def rope(self, x: Buffer, w: Buffer, heads: int, hd: int, start: int, theta: float, scale: float,
             epsilon: float, rotary_dim: int, batch: int = 1) -> None:
        self.check(lib().wgd_rope_norm(self.ctx, x.ptr, w.ptr, heads, hd, start, theta, scale, epsilon,
                                       rotary_dim, batch))

    def rope_neox(self, x: Buffer, heads: int, hd: int, start: int, theta: float, scale: float,
                  rotary_dim: int, batch: int = 1) -> None:
        self.check(lib().wgd_rope_neox(self.ctx, x.ptr, heads, hd, start, theta, scale, rotary_dim, batch))

    def rope_adjacent(self, x: Buffer, heads: int, hd: int, start: int, theta: float, scale: float,
                      rotary_dim: int, batch: int = 1) -> None:
        self.check(lib().wgd_rope_adjacent(self.ctx, x.ptr, heads, hd, start, theta, scale, rotary_dim, batch))

    def attention(self, q: Buffer, k: Buffer, v: Buffer, y: Buffer, heads: int, kv_heads: int, hd: int,
                  start: int, scale: float, window: int, capacity: int, context: int, batch: int = 1) -> None:
        self.check(lib().wgd_attention(self.ctx, q.ptr, k.ptr, v.ptr, y.ptr, heads, kv_heads, hd, start, scale,
                                       window, capacity, context, batch))

    def attention_noalloc(self, q: Buffer, k: Buffer, v: Buffer, y: Buffer, heads: int, kv_heads: int, hd: int,
                          start: int, scale: float, window: int, capacity: int, context: int, batch: int = 1) -> None:
        """attention() with its split-K scratch in the library's static device array: no
        allocation (for graph capture and allocation-free callers)."""
        self.check(lib().wgd_attention_noalloc(self.ctx, q.ptr, k.ptr, v.ptr, y.ptr, heads, kv_heads, hd, start,
                                               scale, window, capacity, context, batch))

    def attention_f16kv(self, q: Buffer, k: Buffer, v: Buffer, y: Buffer, heads: int, kv_heads: int, hd: int,
                        start: int, scale: float, window: int, capacity: int, context: int, batch: int = 1) -> None:
        """attention() over K/V rings of f16 elements (f32 arithmetic)."""
        self.check(lib().wgd_attention_f16kv(self.ctx, q.ptr, k.ptr, v.ptr, y.ptr, heads, kv_heads, hd, start, scale,
                                             window, capacity, context, batch))

    def kv_store_f16(self, src: Buffer, dst: Buffer, count: int, src_offset: int = 0, dst_offset: int = 0) -> None:
        """cacheKV's ring copy into an f16 ring: dst[dst_offset + i] = f16(src[src_offset + i])
        (element offsets, round to nearest even)."""
        self.check(lib().wgd_kv_store_f16(self.ctx, src.ptr, dst.ptr, count, src_offset, dst_offset))

    def probe_read(self, src: Buffer, nbytes: int, copies: int, launches: int, workgroups: int, threads: int,
                   depth: int, out: Optional[Buffer] = None, out_floats: int = 0) -> None:
        """`launches` plain streaming reads of nbytes, rotating over `copies` copies in src (the
        per-launch read floor; measurement only)."""
        self.check(lib().wgd_probe_read(self.ctx, src.ptr, nbytes, copies, launches, workgroups, threads, depth,
                                        out.ptr if out is not None else None, out_floats))

    def add(self, delta: Buffer, state: Buffer, n: int) -> None:
        self.check(lib().wgd_add(self.ctx, delta.ptr, state.ptr, n))

    def silu(self, gate: Buffer, up: Buffer, y: Buffer, n: int) -> None:
        self.check(lib().wgd_silu(self.ctx, gate.ptr, up.ptr, y.ptr, n))

    def gelu(self, gate: Buffer, up: Buffer, y: Buffer, n: int) -> None:
        self.check(lib().wgd_gelu(self.ctx, gate.ptr, up.ptr, y.ptr, n))

    def bias_add(self, y: Buffer, b: Buffer, n: int, width: int) -> None:
        self.check(lib().wgd_bias_add(self.ctx, y.ptr, b.ptr, n, width))

    def activate(self, x: Buffer, n: int) -> None:
        self.check(lib().wgd_activate(self.ctx, x.ptr, n))

    def argmax(self, logits: Buffer, n: int) -> int:
        idx = C.c_int32(-1)
        self.check(lib().wgd_argmax(self.ctx, logits.ptr, n, None, C.byref(idx)))
        return idx.value

    def sample(self, logits: Buffer, n: int, temperature: float, top_k: int, top_p: float, seed: int,
               index: int) -> int:
        """sample() on the device with the index-th uniform of ``seed``."""
        tok = C.c_int32(-1)
        self.check(lib().wgd_sample(self.ctx, logits.ptr, n, float(temperature), int(top_k), float(top_p),
                                    int(seed) & (2 ** 64 - 1), int(index), C.byref(tok)))
        return tok.value

    def embed(self, type_: int, table: Buffer, ids: Buffer, out: Buffer, hidden: int, n: int, scale: float = 1.0) -> None:
        self.check(lib().wgd_embed(self.ctx, type_, table.ptr, ids.ptr, out.ptr, hidden, n, scale))
