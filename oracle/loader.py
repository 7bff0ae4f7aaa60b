"""Loaders for the oracle's native builds (test infrastructure only).

* :func:`c_oracle` -- ctypes handle on ``oracle/liboracle.so`` (the C
  restatement in ``oracle/native_ref.c``) with numpy-friendly wrappers.
* :func:`ref_C` -- the reference's own ``_C`` pybind11 module built from
  ``src/flatrun_native/_C.cpp`` into ``oracle/_ref/`` (``make -C oracle ref``),
  or ``None`` when that build is absent.
* :func:`build` -- runs ``make`` in ``oracle/`` (the reference build only when
  the reference checkout is present).
"""

from __future__ import annotations

import ctypes
import importlib.machinery
import importlib.util
import os
import subprocess
import sysconfig
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REF_ROOT = Path(os.environ.get("FRQ_REFERENCE_ROOT", "/root/reference"))
_EXT = sysconfig.get_config_var("EXT_SUFFIX")


def build(force: bool = False) -> None:
    """Compile liboracle.so, and oracle/_ref when the reference is present."""
    subprocess.run(["make", "-s", "-C", str(HERE)] + (["-B"] if force else []), check=True)
    if (REF_ROOT / "src/flatrun_native/_C.cpp").is_file():
        subprocess.run(["make", "-s", "-C", str(HERE), "ref", f"REF={REF_ROOT}"] + (["-B"] if force else []),
                       check=True)


_C_LIB = None


class _COracle:
    def __init__(self, lib):
        self.lib = lib
        u8p, f32p = ctypes.POINTER(ctypes.c_uint8), ctypes.POINTER(ctypes.c_float)
        for q in ("q4_k", "q6_k", "q8_0"):
            fn = getattr(lib, f"oracle_dequant_{q}")
            fn.argtypes = [u8p, ctypes.c_size_t, f32p]
            fn.restype = None
            fn = getattr(lib, f"oracle_matmul_{q}")
            fn.argtypes = [u8p, f32p, f32p, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_int]
            fn.restype = None
        lib.oracle_fp16_to_fp32.argtypes = [ctypes.c_uint16]
        lib.oracle_fp16_to_fp32.restype = ctypes.c_float

    _BLK = {"Q4_K": (144, 256), "Q6_K": (210, 256), "Q8_0": (34, 32)}

    @staticmethod
    def _p(a, ct):
        return a.ctypes.data_as(ctypes.POINTER(ct))

    def fp16_to_fp32(self, h: int) -> float:
        return float(self.lib.oracle_fp16_to_fp32(int(h)))

    def dequant(self, qname: str, raw: np.ndarray, n_elems: int) -> np.ndarray:
        bb, be = self._BLK[qname]
        raw = np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1)
        nblk = raw.size // bb
        out = np.empty(nblk * be, dtype=np.float32)
        getattr(self.lib, f"oracle_dequant_{qname.lower()}")(self._p(raw, ctypes.c_uint8), nblk,
                                                              self._p(out, ctypes.c_float))
        return out[:n_elems]

    def matmul(self, qname: str, x: np.ndarray, raw: np.ndarray, n: int, k: int, threads: int = 1) -> np.ndarray:
        bb, be = self._BLK[qname]
        raw = np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1)
        if k % be or raw.size != n * (k // be) * bb:
            raise ValueError("oracle matmul: size mismatch")
        x = np.ascontiguousarray(x, dtype=np.float32)
        fn = getattr(self.lib, f"oracle_matmul_{qname.lower()}")
        if x.ndim == 1:
            y = np.empty(n, dtype=np.float32)
            fn(self._p(raw, ctypes.c_uint8), self._p(x, ctypes.c_float), self._p(y, ctypes.c_float), n, k, threads)
            return y
        y = np.empty((x.shape[0], n), dtype=np.float32)
        for s in range(x.shape[0]):
            xs = np.ascontiguousarray(x[s])
            ys = y[s]
            fn(self._p(raw, ctypes.c_uint8), self._p(xs, ctypes.c_float), self._p(ys, ctypes.c_float), n, k, threads)
        return y


def c_oracle() -> _COracle:
    """The C restatement (builds it on first use if missing)."""
    global _C_LIB
    if _C_LIB is None:
        so = HERE / "liboracle.so"
        if not so.is_file():
            subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
        _C_LIB = _COracle(ctypes.CDLL(str(so)))
    return _C_LIB


_REF_MOD = False


def ref_C():
    """The reference's compiled ``_C`` module from oracle/_ref, or None."""
    global _REF_MOD
    if _REF_MOD is False:
        path = HERE / "_ref" / f"_C{_EXT}"
        if path.is_file():
            loader = importlib.machinery.ExtensionFileLoader("_C", str(path))
            spec = importlib.util.spec_from_file_location("_C", str(path), loader=loader)
            mod = importlib.util.module_from_spec(spec)
            loader.exec_module(mod)
            _REF_MOD = mod
        else:
            _REF_MOD = None
    return _REF_MOD
