"""Shared pytest configuration.

Markers: ``gpu`` -- needs a HIP device and the built libfrq_hip.so. GPU tests
never skip silently when the library is missing: the ``frq`` fixture raises,
so a GPU run without the native library fails loudly.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN = ROOT / "tests" / "golden"

# Matvec tolerance of the contract: max relative error 1e-5 with
# fp32 accumulation, measured normwise (max|dy| / max|y|) and componentwise
# (|dy_i| / sum_j |w_ij x_j|) against the fp64 oracle and the NumPy matvec.
MATVEC_RTOL = 1e-5


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP (MI355X) device and the built libfrq_hip.so")


@pytest.fixture(scope="session")
def frq():
    """The native library on a GPU machine; raises (never skips) if missing."""
    from flatrun_amd import _lib

    lib = _lib.lib()                       # LibraryMissing -> error, not skip
    n = _lib.device_count()
    if n <= 0:
        raise RuntimeError("gpu test collected but no HIP device is visible")
    return lib


@pytest.fixture(scope="session")
def backend(frq):
    from flatrun_amd import NativeBackend

    b = NativeBackend()
    assert b.available
    return b


@pytest.fixture(scope="session")
def ref_C():
    """The reference's compiled _C module from oracle/_ref, or skip."""
    from oracle.loader import ref_C as load

    mod = load()
    if mod is None:
        pytest.skip("oracle/_ref not built (reference checkout absent)")
    return mod


def matvec_errors(y, y64, absw64):
    """(normwise, componentwise) relative error of y against the fp64 oracle."""
    y = np.asarray(y, dtype=np.float64)
    d = np.abs(y - y64)
    scale = np.max(np.abs(y64)) if y64.size else 0.0
    normwise = float(d.max() / scale) if scale > 0 else float(d.max() if d.size else 0.0)
    with np.errstate(divide="ignore", invalid="ignore"):
        comp = np.where(absw64 > 0, d / absw64, np.where(d > 0, np.inf, 0.0))
    return normwise, float(comp.max() if comp.size else 0.0)


def assert_matvec_close(y, y64, absw64, rtol=MATVEC_RTOL, what=""):
    nw, cw = matvec_errors(y, y64, absw64)
    assert nw <= rtol, f"{what} normwise rel err {nw:.3e} > {rtol}"
    assert cw <= rtol, f"{what} componentwise rel err {cw:.3e} > {rtol}"
    return nw, cw


def assert_rel_close_to(y, y_ref, rtol=MATVEC_RTOL, what=""):
    """max|y - y_ref| / max|y_ref| <= rtol (e.g. against the fp32 NumPy matvec)."""
    y, y_ref = np.asarray(y, np.float64), np.asarray(y_ref, np.float64)
    scale = np.max(np.abs(y_ref)) if y_ref.size else 0.0
    err = float(np.max(np.abs(y - y_ref)) / scale) if scale > 0 else float(np.max(np.abs(y - y_ref), initial=0.0))
    assert err <= rtol, f"{what} rel err {err:.3e} > {rtol}"
    return err


def bits_equal(a, b) -> bool:
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))
