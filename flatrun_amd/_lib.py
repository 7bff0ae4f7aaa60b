"""ctypes binding of libfrq_hip.so (the C ABI declared in include/frq.h).

The library is built in-tree by ``python -m flatrun_amd.build``. There is no
CPU fallback: :func:`lib` raises :class:`LibraryMissing` when the shared
object is absent or cannot be loaded, and every compute entry point reports
``FRQ_ERR_NO_DEVICE`` on a machine without a HIP device.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

LIB_PATH = Path(os.environ.get("FRQ_LIB", Path(__file__).resolve().parent / "libfrq_hip.so"))

# frq_status codes (include/frq.h)
OK, ERR_INVALID, ERR_SHAPE, ERR_SIZE, ERR_UNSUPPORTED, ERR_NO_DEVICE, ERR_HIP, ERR_ALIGN = range(8)
STATUS_NAMES = {
    OK: "FRQ_OK", ERR_INVALID: "FRQ_ERR_INVALID", ERR_SHAPE: "FRQ_ERR_SHAPE", ERR_SIZE: "FRQ_ERR_SIZE",
    ERR_UNSUPPORTED: "FRQ_ERR_UNSUPPORTED", ERR_NO_DEVICE: "FRQ_ERR_NO_DEVICE", ERR_HIP: "FRQ_ERR_HIP",
    ERR_ALIGN: "FRQ_ERR_ALIGN",
}

# GGML type ids (src/flatrun/backend/gguf.py:59-86)
Q8_0, Q4_K, Q5_K, Q6_K, Q1_0 = 8, 12, 13, 14, 41
Q4_0, Q5_0, Q5_1 = 2, 6, 7          # dequant only
QTYPES = {"Q8_0": Q8_0, "Q4_K": Q4_K, "Q5_K": Q5_K, "Q6_K": Q6_K, "Q1_0": Q1_0,
          "Q4_0": Q4_0, "Q5_0": Q5_0, "Q5_1": Q5_1}
BLOCKS = {Q8_0: (34, 32), Q4_K: (144, 256), Q5_K: (176, 256), Q6_K: (210, 256), Q1_0: (18, 128)}


GEMV_AUTO, GEMV_SPLITK, GEMV_ROWS, GEMV_MX, GEMV_MB = 0, 1, 2, 4, 8   # frq_gemv_config.kernel (3 and 5 are not used)


class GemvConfig(ctypes.Structure):
    """frq_gemv_config (include/frq.h)."""
    _fields_ = [("kernel", ctypes.c_int32), ("cpl", ctypes.c_int32), ("rows", ctypes.c_int32),
                ("unroll", ctypes.c_int32), ("slices", ctypes.c_int32), ("waves_per_wg", ctypes.c_int32),
                ("items", ctypes.c_int64)]

    def as_dict(self) -> dict:
        return {f: getattr(self, f) for f, _ in self._fields_}


class LibraryMissing(RuntimeError):
    """libfrq_hip.so is not built or cannot be loaded."""


class FrqError(RuntimeError):
    """A libfrq_hip call refused its arguments: a shape, size, alignment or
    quant type it does not take, or no device. Subclasses RuntimeError, the
    exception the reference runtime catches to fall back to NumPy for a
    layout the kernel rejects (runtime/backend.py:259-268)."""

    def __init__(self, code: int, message: str):
        super().__init__(f"{STATUS_NAMES.get(code, code)}: {message}")
        self.code = code


class FrqDeviceError(Exception):
    """A HIP runtime failure inside libfrq_hip (FRQ_ERR_HIP): a launch,
    allocation, copy or synchronization that the runtime reported failed.
    Deliberately not a RuntimeError: the reference runtime treats any
    RuntimeError from a kernel as a rejected layout and recomputes in NumPy
    (runtime/backend.py:259-268), which would turn a device failure into a
    silent 100-1000x slowdown. This one propagates to the caller."""

    def __init__(self, code: int, message: str):
        super().__init__(f"{STATUS_NAMES.get(code, code)}: {message}")
        self.code = code


def error_for(code: int, message: str) -> Exception:
    """The exception a failed call with status `code` raises."""
    return FrqDeviceError(code, message) if code == ERR_HIP else FrqError(code, message)


_c = ctypes
_vp, _sz, _i64, _i32 = _c.c_void_p, _c.c_size_t, _c.c_int64, _c.c_int
_u8p = _c.POINTER(_c.c_uint8)
_f32p = _c.POINTER(_c.c_float)
_i64p = _c.POINTER(_c.c_int64)
_i32p = _c.POINTER(_c.c_int)

# name -> argtypes; every function returns int (frq_status) unless listed in _RESTYPES
SIGNATURES: dict[str, list] = {
    "frq_version": [],
    "frq_is_neon": [],
    "frq_last_error": [],
    "frq_device_count": [_i32p],
    "frq_block_info": [_i32, _i64p, _i64p],
    "frq_dequant_q4_k": [_vp, _sz, _i64, _i64, _vp],
    "frq_dequant_q8_0": [_vp, _sz, _i64, _i64, _vp],
    "frq_dequant_q6_k": [_vp, _sz, _i64, _i64, _vp],
    "frq_dequant": [_i32, _vp, _sz, _i64, _vp],
    "frq_dequant_f16": [_i32, _vp, _sz, _i64, _vp],
    "frq_matmul_q4_k": [_vp, _sz, _vp, _sz, _sz, _sz, _vp],
    "frq_matmul_q4_k_batched": [_vp, _i32, _sz, _sz, _vp, _sz, _sz, _sz, _vp],
    "frq_matmul_q8_0": [_vp, _sz, _vp, _sz, _sz, _sz, _vp],
    "frq_matmul_q8_0_batched": [_vp, _i32, _sz, _sz, _vp, _sz, _sz, _sz, _vp],
    "frq_matmul_q6_k": [_vp, _sz, _vp, _sz, _sz, _sz, _vp],
    "frq_matmul_q6_k_batched": [_vp, _i32, _sz, _sz, _vp, _sz, _sz, _sz, _vp],
    "frq_matmul": [_i32, _vp, _sz, _vp, _sz, _sz, _sz, _vp],
    "frq_dev_dequant": [_i32, _vp, _sz, _i64, _vp, _vp],
    "frq_dev_dequant_f16": [_i32, _vp, _sz, _i64, _vp, _vp],
    "frq_dev_gemv": [_i32, _vp, _sz, _vp, _vp, _i64, _i64, _i64, _vp],
    "frq_dev_gemv_noalloc": [_i32, _vp, _sz, _vp, _vp, _i64, _i64, _i64, _vp],
    "frq_dev_gemv_group": [_i32, _vp, _vp, _vp, _vp, _vp, _i64, _vp, _i64, _i64, _vp],
    "frq_gemv_group_fusable": [_i32, _vp, _vp, _i64],
    "frq_dev_gemv_tuned": [_i32, _vp, _sz, _vp, _vp, _i64, _i64, _c.c_void_p, _vp],
    "frq_dev_copy": [_vp, _vp, _sz, _vp],
    "frq_dev_read_xor": [_vp, _sz, _vp, _vp],
    "frq_dev_silu_mul": [_vp, _i64, _vp, _i64, _i64, _i64, _vp],
    "frq_dev_gemv_swiglu": [_i32, _vp, _sz, _i32, _vp, _sz, _i64, _vp, _i64, _vp, _vp, _i64, _vp],
    "frq_gemv_swiglu_fusable": [_i32, _vp, _i32, _vp, _i64],
    "frq_set_device": [_i32],
    "frq_malloc": [_c.POINTER(_vp), _sz],
    "frq_free": [_vp],
    "frq_host_alloc": [_c.POINTER(_vp), _sz],
    "frq_host_free": [_vp],
    "frq_memcpy_h2d": [_vp, _vp, _sz],
    "frq_memcpy_d2h": [_vp, _vp, _sz],
    "frq_memcpy_h2d_async": [_vp, _vp, _sz, _vp],
    "frq_memcpy_d2h_async": [_vp, _vp, _sz, _vp],
    "frq_memset_async": [_vp, _i32, _sz, _vp],
    "frq_stream_create": [_c.POINTER(_vp)],
    "frq_stream_destroy": [_vp],
    "frq_stream_synchronize": [_vp],
    "frq_stream_wait_event": [_vp, _vp],
    "frq_event_create": [_c.POINTER(_vp)],
    "frq_event_destroy": [_vp],
    "frq_event_record": [_vp, _vp],
    "frq_event_synchronize": [_vp],
    "frq_event_elapsed_ms": [_f32p, _vp, _vp],
    "frq_device_synchronize": [],
    "frq_dev_gemm_q4_k_bf16": [_vp, _sz, _vp, _vp, _i64, _i64, _i64, _vp],
    "frq_gemm_q4_k_bf16": [_vp, _vp, _sz, _i64, _i64, _i64, _vp],
    "frq_dev_gemm_bf16": [_i32, _vp, _sz, _vp, _vp, _i64, _i64, _i64, _vp],
    "frq_dev_gemm_bf16_group": [_i32, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _vp, _i64, _vp],
    "frq_gemm_bf16": [_i32, _vp, _vp, _sz, _i64, _i64, _i64, _vp],
    "frq_stream_begin_capture": [_vp],
    "frq_stream_end_capture": [_vp, _c.POINTER(_vp)],
    "frq_graph_launch": [_vp, _vp],
    "frq_graph_destroy": [_vp],
}
_RESTYPES = {"frq_version": _c.c_char_p, "frq_last_error": _c.c_char_p}

_LIB = None
_LOAD_ERROR: BaseException | None = None
_LOCK = threading.Lock()


def lib():
    """The loaded library; raises LibraryMissing if it cannot be loaded."""
    global _LIB, _LOAD_ERROR
    if _LIB is not None:
        return _LIB
    with _LOCK:
        if _LIB is None:
            if not LIB_PATH.is_file():
                _LOAD_ERROR = LibraryMissing(
                    f"{LIB_PATH} not found; build it with `python -m flatrun_amd.build`")
                raise _LOAD_ERROR
            try:
                h = ctypes.CDLL(str(LIB_PATH))
            except OSError as exc:
                _LOAD_ERROR = LibraryMissing(f"cannot load {LIB_PATH}: {exc}")
                raise _LOAD_ERROR from exc
            for name, argtypes in SIGNATURES.items():
                fn = getattr(h, name)
                fn.argtypes = argtypes
                fn.restype = _RESTYPES.get(name, _c.c_int)
            _LIB = h
    return _LIB


def load_error() -> BaseException | None:
    try:
        lib()
    except LibraryMissing as exc:
        return exc
    return None


def check(rc: int) -> None:
    """Raise for a failed status: FrqDeviceError for a HIP runtime failure,
    FrqError (a RuntimeError) for everything else."""
    if rc != OK:
        msg = lib().frq_last_error().decode(errors="replace")
        raise error_for(rc, msg)


def device_count() -> int:
    n = ctypes.c_int(0)
    check(lib().frq_device_count(ctypes.byref(n)))
    return int(n.value)


def version() -> str:
    return lib().frq_version().decode()


def ptr(a) -> int:
    """Address of a numpy array's data (0 for an empty array)."""
    return a.ctypes.data if a.size else 0
