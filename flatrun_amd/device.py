"""Device-resident buffers, streams and the device-pointer entry points.

This is the decode-time path: raw GGUF blocks are uploaded once
(:meth:`DeviceBuffer.from_host`) and every matvec reads them straight from
HBM through ``frq_dev_gemv``. Any object exposing ``data_ptr()`` (a torch
CUDA tensor) can be passed where a device buffer is expected, so callers that
keep activations in torch tensors need no copies.
"""

from __future__ import annotations

import ctypes

import numpy as np

from . import _lib
from ._lib import check, lib


def _addr(obj) -> int:
    if obj is None:
        return 0
    if isinstance(obj, DeviceBuffer):
        return obj.ptr
    if hasattr(obj, "data_ptr"):
        return int(obj.data_ptr())
    if isinstance(obj, int):
        return obj
    raise TypeError(f"expected a device buffer, got {type(obj).__name__}")


def _nbytes(obj) -> int:
    if isinstance(obj, DeviceBuffer):
        return obj.nbytes
    if hasattr(obj, "data_ptr") and isinstance(getattr(obj, "nbytes", None), int):   # DeviceWeight
        return obj.nbytes
    if hasattr(obj, "untyped_storage"):
        return int(obj.numel() * obj.element_size())
    raise TypeError(f"cannot size {type(obj).__name__}")


def _stream(s) -> int:
    if s is None:
        return 0
    if isinstance(s, Stream):
        return s.handle
    if hasattr(s, "cuda_stream"):
        return int(s.cuda_stream)
    return int(s)


class DeviceBuffer:
    """An allocation in device memory (hipMalloc), freed with the object."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        check(lib().frq_malloc(ctypes.byref(p), self.nbytes))
        self.ptr = int(p.value or 0)

    @classmethod
    def from_host(cls, arr: np.ndarray, stream=None) -> "DeviceBuffer":
        a = np.ascontiguousarray(arr)
        buf = cls(a.nbytes)
        if a.nbytes:
            if stream is None:
                check(lib().frq_memcpy_h2d(buf.ptr, a.ctypes.data, a.nbytes))
            else:
                check(lib().frq_memcpy_h2d_async(buf.ptr, a.ctypes.data, a.nbytes, _stream(stream)))
        return buf

    def to_host(self, dtype=np.uint8, count: int | None = None) -> np.ndarray:
        dt = np.dtype(dtype)
        n = self.nbytes // dt.itemsize if count is None else int(count)
        out = np.empty(n, dtype=dt)
        if out.nbytes:
            check(lib().frq_memcpy_d2h(out.ctypes.data, self.ptr, out.nbytes))
        return out

    def free(self) -> None:
        if getattr(self, "ptr", 0):
            try:
                lib().frq_free(self.ptr)
            finally:
                self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def data_ptr(self) -> int:
        return self.ptr


class PinnedBuffer:
    """Page-locked host memory (hipHostMalloc) viewed as a numpy array."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        check(lib().frq_host_alloc(ctypes.byref(p), self.nbytes))
        self.ptr = int(p.value or 0)
        self.array = np.ctypeslib.as_array((ctypes.c_uint8 * max(self.nbytes, 1)).from_address(self.ptr))[: self.nbytes]

    def free(self) -> None:
        if getattr(self, "ptr", 0):
            self.array = None
            try:
                lib().frq_host_free(self.ptr)
            finally:
                self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Stream:
    """A HIP stream at the default priority (non-blocking w.r.t. the null stream)."""

    def __init__(self):
        p = ctypes.c_void_p()
        check(lib().frq_stream_create(ctypes.byref(p)))
        self.handle = int(p.value or 0)

    def synchronize(self) -> None:
        check(lib().frq_stream_synchronize(self.handle))

    def wait(self, event: "Event") -> None:
        check(lib().frq_stream_wait_event(self.handle, event.handle))

    def destroy(self) -> None:
        if getattr(self, "handle", 0):
            try:
                lib().frq_stream_destroy(self.handle)
            finally:
                self.handle = 0

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


class Event:
    def __init__(self):
        p = ctypes.c_void_p()
        check(lib().frq_event_create(ctypes.byref(p)))
        self.handle = int(p.value or 0)

    def record(self, stream=None) -> None:
        check(lib().frq_event_record(self.handle, _stream(stream)))

    def synchronize(self) -> None:
        check(lib().frq_event_synchronize(self.handle))

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float()
        check(lib().frq_event_elapsed_ms(ctypes.byref(ms), self.handle, end.handle))
        return float(ms.value)

    def destroy(self) -> None:
        if getattr(self, "handle", 0):
            try:
                lib().frq_event_destroy(self.handle)
            finally:
                self.handle = 0

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


class Graph:
    """A recorded launch sequence, replayed with one call.

    ``with Graph.capture(stream) as g: ...`` records every launch issued on
    ``stream`` inside the block (nothing runs then); ``g.launch(stream)``
    replays it. The stream must be a :class:`Stream`, not the null stream.
    """

    def __init__(self, handle: int):
        self.handle = handle

    @classmethod
    def capture(cls, stream: "Stream"):
        return _Capture(stream)

    def launch(self, stream=None) -> None:
        check(lib().frq_graph_launch(self.handle, _stream(stream)))

    def destroy(self) -> None:
        if getattr(self, "handle", 0):
            try:
                lib().frq_graph_destroy(self.handle)
            finally:
                self.handle = 0

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


class _Capture:
    def __init__(self, stream: "Stream"):
        if not isinstance(stream, Stream):
            raise TypeError("graph capture needs a device.Stream")
        self.stream = stream
        self.graph: Graph | None = None

    def __enter__(self) -> "_Capture":
        check(lib().frq_stream_begin_capture(self.stream.handle))
        return self

    def __exit__(self, et, ev, tb) -> None:
        h = ctypes.c_void_p()
        rc = lib().frq_stream_end_capture(self.stream.handle, ctypes.byref(h))
        if et is None:
            check(rc)
            self.graph = Graph(int(h.value or 0))
        elif rc == 0 and h.value:
            lib().frq_graph_destroy(h.value)

    def launch(self, stream=None) -> None:
        self.graph.launch(stream)

    def destroy(self) -> None:
        if self.graph is not None:
            self.graph.destroy()


def synchronize() -> None:
    check(lib().frq_device_synchronize())


def qtype_id(q) -> int:
    if isinstance(q, str):
        return _lib.QTYPES[q.upper()]
    return int(q)


def gemv(qtype, w, x, y, n: int, k: int, batch: int = 1, stream=None, w_bytes: int | None = None) -> None:
    """y[b, :n] = W[n, k] . x[b, :k] on device buffers (enqueued, not synchronised)."""
    q = qtype_id(qtype)
    wb = _nbytes(w) if w_bytes is None else int(w_bytes)
    check(lib().frq_dev_gemv(q, _addr(w), wb, _addr(x), _addr(y), int(n), int(k), int(batch), _stream(stream)))


GROUP_MAX = 4


def _group_arrays(parts):
    if not 1 <= len(parts) <= GROUP_MAX:
        raise ValueError(f"a group holds 1..{GROUP_MAX} matrices, got {len(parts)}")
    qt = (ctypes.c_int * len(parts))(*[qtype_id(p[0]) for p in parts])
    wp = (ctypes.c_void_p * len(parts))(*[_addr(p[1]) for p in parts])
    return qt, wp


def gemv_group(parts, x, k: int, batch: int = 1, y_stride: int = 0, stream=None) -> None:
    """Matrices sharing x in one launch where possible (frq_dev_gemv_group;
    a single matrix runs frq_dev_gemv's kernel).

    ``parts``: up to 4 tuples ``(qtype, w, n, y[, w_bytes])``; ``y`` is the
    device output of batch row 0 (an int address is accepted, e.g. an offset
    into one concatenated buffer); row b of matrix i goes to
    ``y_i + b * (y_stride or n_i)`` floats."""
    qt, wp = _group_arrays(parts)
    c = len(parts)
    wb = (ctypes.c_size_t * c)(*[int(p[4]) if len(p) > 4 else _nbytes(p[1]) for p in parts])
    nn = (ctypes.c_int64 * c)(*[int(p[2]) for p in parts])
    yy = (ctypes.c_void_p * c)(*[_addr(p[3]) for p in parts])
    check(lib().frq_dev_gemv_group(c, qt, wp, wb, nn, _addr(x), int(k), yy, int(batch), int(y_stride),
                                   _stream(stream)))


def gemv_group_fusable(parts, k: int) -> bool:
    """True if ``parts`` ((qtype, w, ...) tuples) run as one launch."""
    qt, wp = _group_arrays(parts)
    return bool(lib().frq_gemv_group_fusable(len(parts), qt, wp, int(k)))


def gemv_tuned(qtype, w, x, y, n: int, k: int, kernel: int = 0, cpl: int = 0, rows: int = 0, unroll: int = 0,
               stream=None, w_bytes: int | None = None, slices: int = 0) -> dict:
    """One GEMV with an explicit launch geometry; returns the geometry used
    (fields of frq_gemv_config)."""
    q = qtype_id(qtype)
    wb = _nbytes(w) if w_bytes is None else int(w_bytes)
    cfg = _lib.GemvConfig(kernel=kernel, cpl=cpl, rows=rows, unroll=unroll, slices=slices)
    check(lib().frq_dev_gemv_tuned(q, _addr(w), wb, _addr(x), _addr(y), int(n), int(k), ctypes.addressof(cfg),
                                   _stream(stream)))
    return cfg.as_dict()


def gemm_bf16(qtype, w, x_bf16, y, m: int, n: int, k: int, stream=None, w_bytes: int | None = None) -> None:
    """y[m, n] = x[m, k] . W[n, k]^T on the matrix cores (W: Q4_K, Q6_K or Q8_0
    blocks; x: bf16 bits, row-major; y: fp32). Enqueued, not synchronised."""
    wb = _nbytes(w) if w_bytes is None else int(w_bytes)
    check(lib().frq_dev_gemm_bf16(qtype_id(qtype), _addr(w), wb, _addr(x_bf16), _addr(y), int(m), int(n), int(k),
                                  _stream(stream)))


def gemm_bf16_group(parts, x_bf16, m: int, k: int, y_stride: int = 0, stream=None) -> None:
    """Matrices sharing x in one GEMM launch (frq_dev_gemm_bf16_group).
    ``parts``: up to 4 tuples ``(qtype, w, n, y[, w_bytes])``; ``y`` is the
    device output (an int address is accepted, e.g. an offset into one
    concatenated buffer); row r of matrix i goes to ``y_i + r * (y_stride or n_i)``
    floats."""
    qt, wp = _group_arrays(parts)
    c = len(parts)
    wb = (ctypes.c_size_t * c)(*[int(p[4]) if len(p) > 4 else _nbytes(p[1]) for p in parts])
    nn = (ctypes.c_int64 * c)(*[int(p[2]) for p in parts])
    yy = (ctypes.c_void_p * c)(*[_addr(p[3]) for p in parts])
    check(lib().frq_dev_gemm_bf16_group(c, qt, wp, wb, nn, _addr(x_bf16), int(m), int(k), yy, int(y_stride),
                                        _stream(stream)))


def gemm_q4k_bf16(w, x_bf16, y, m: int, n: int, k: int, stream=None, w_bytes: int | None = None) -> None:
    gemm_bf16("Q4_K", w, x_bf16, y, m, n, k, stream=stream, w_bytes=w_bytes)


def memcpy_h2d_async(dst, src_host_ptr: int, nbytes: int, stream=None) -> None:
    """Enqueues a host -> device copy (the host memory should be pinned for it
    to run asynchronously)."""
    check(lib().frq_memcpy_h2d_async(_addr(dst), int(src_host_ptr), int(nbytes), _stream(stream)))


def copy(dst, src, nbytes: int, stream=None) -> None:
    """dst[:nbytes] = src[:nbytes] with the library's streaming copy kernel (enqueued)."""
    check(lib().frq_dev_copy(_addr(dst), _addr(src), int(nbytes), _stream(stream)))


READ_XOR_WORDS = 2048


def read_xor(src, nbytes: int, out, stream=None) -> None:
    """Read src[:nbytes] with the library's streaming read kernel (enqueued):
    out (READ_XOR_WORDS device words) receives per-workgroup XORs of its
    32-bit words, zeros past the grid; the XOR of all of out is that of src."""
    check(lib().frq_dev_read_xor(_addr(src), int(nbytes), _addr(out), _stream(stream)))


def dequant(qtype, w, y, n_elems: int, stream=None, w_bytes: int | None = None) -> None:
    """y[:n_elems] = dequant(w) on device buffers (enqueued)."""
    q = qtype_id(qtype)
    wb = _nbytes(w) if w_bytes is None else int(w_bytes)
    check(lib().frq_dev_dequant(q, _addr(w), wb, int(n_elems), _addr(y), _stream(stream)))


def dequant_f16(qtype, w, y, n_elems: int, stream=None, w_bytes: int | None = None) -> None:
    """y[:n_elems] = fp16 bit patterns of dequant(w), rounded to nearest even
    (enqueued)."""
    q = qtype_id(qtype)
    wb = _nbytes(w) if w_bytes is None else int(w_bytes)
    check(lib().frq_dev_dequant_f16(q, _addr(w), wb, int(n_elems), _addr(y), _stream(stream)))


def gemv_swiglu(gate, up, x, k: int, gateup, act, batch: int = 1, stream=None) -> None:
    """gateup[r] = [W_gate x_r | W_up x_r] and act[r] = silu(gate) * up for
    `batch` rows of x, enqueued (frq_dev_gemv_swiglu: one launch for a Q4_K
    pair at batch 1, else the grouped launch and frq_dev_silu_mul, same
    bits). ``gate`` / ``up``: ``(qtype, w, inter[, w_bytes])``."""
    qg, wg, inter = gate[0], gate[1], int(gate[2])
    qu, wu = up[0], up[1]
    gb = int(gate[3]) if len(gate) > 3 else _nbytes(wg)
    ub = int(up[3]) if len(up) > 3 else _nbytes(wu)
    if int(up[2]) != inter:
        raise ValueError(f"gate and up need the same output size, got {inter} and {up[2]}")
    check(lib().frq_dev_gemv_swiglu(qtype_id(qg), _addr(wg), gb, qtype_id(qu), _addr(wu), ub, inter, _addr(x),
                                    int(k), _addr(gateup), _addr(act), int(batch), _stream(stream)))


def gemv_swiglu_fusable(gate, up, k: int) -> bool:
    """True if gemv_swiglu runs ``gate`` and ``up`` ((qtype, w, ...)) and the
    activation as one launch at batch 1."""
    return bool(lib().frq_gemv_swiglu_fusable(qtype_id(gate[0]), _addr(gate[1]), qtype_id(up[0]), _addr(up[1]),
                                              int(k)))


def silu_mul(gateup, out, rows: int, inter: int, ld_in: int = 0, ld_out: int = 0, stream=None) -> None:
    """out[r, :inter] = silu(gate) * up for the grouped gate|up rows of
    gateup (gate first; rows ld_in floats apart, default 2 inter; out rows
    ld_out apart, default inter), enqueued (frq_dev_silu_mul)."""
    li = int(ld_in) or 2 * int(inter)
    lo = int(ld_out) or int(inter)
    check(lib().frq_dev_silu_mul(_addr(gateup), li, _addr(out), lo, int(rows), int(inter), _stream(stream)))
