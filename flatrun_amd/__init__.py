"""flatrun_amd -- MI355X (gfx950) GGUF dequant + quantized matvec.

Drop-in for the reference's native accelerator package ``flatrun_native``
(``src/flatrun_native/python/__init__.py``): the same public names
(``NativeBackend``, ``Q4K_GEMM_BLOCK``, ``is_available``, ``is_neon``,
``version``), the same method signatures and dispatch (1-D ``x`` -> matvec,
2-D ``x`` -> batched), the same exception types (``ValueError`` for a bad
``x`` shape, ``RuntimeError`` when unavailable or when the kernel rejects a
layout). The kernels are hand-written HIP for gfx950 reached through ctypes
(``flatrun_amd._lib``); there is no CPU fallback inside this package --
``--backend python`` stays the reference's own NumPy path.

Typical use::

    from flatrun_amd import NativeBackend
    b = NativeBackend()
    y = b.matmul_q4k(x, raw_q4k_bytes, n, k)          # host buffers
    w = b.upload(raw_q4k_bytes)                       # resident in HBM
    y = b.matmul_q4k(x, w, n, k)                      # no weight copy
"""

from __future__ import annotations

import os
import threading

import numpy as np

from . import _C, _lib
from ._lib import FrqDeviceError, FrqError, LibraryMissing
from .loader import dequant_handle
from .residency import WeightCache

__all__ = [
    "NativeBackend",
    "dequant_handle",
    "DeviceWeight",
    "Q4K_GEMM_BLOCK",
    "is_available",
    "is_neon",
    "version",
    "FrqDeviceError",
    "FrqError",
    "LibraryMissing",
]

# Block size of the Q4_K format (python/__init__.py:37-38).
Q4K_GEMM_BLOCK = 256


def is_available() -> bool:
    """True when libfrq_hip.so loads and a HIP device is visible."""
    try:
        return _lib.device_count() > 0
    except (LibraryMissing, FrqError, FrqDeviceError):
        return False


def version() -> str:
    """Build identifier, or the reason the library is unavailable."""
    err = _lib.load_error()
    if err is not None:
        return f"flatrun_amd (unavailable: {err})"
    return _C.version()


def is_neon() -> bool:
    """Always False: the library targets gfx950, not ARM NEON."""
    return False


class DeviceWeight:
    """Raw GGUF block bytes resident in device memory.

    ``DeviceWeight(raw)`` uploads a copy it owns; :meth:`view` names a byte
    range of an existing device buffer (a tensor of a
    :class:`flatrun_amd.gguf.ResidentModel` arena), which it keeps alive but
    does not free. ``qtype``, ``shape`` and ``name`` describe the tensor when
    known (None otherwise)."""

    def __init__(self, raw: np.ndarray):
        from .device import DeviceBuffer
        raw = np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1)
        self.nbytes = int(raw.size)
        self.buffer = DeviceBuffer.from_host(raw)
        self.offset = 0
        self.qtype = self.shape = self.name = None

    @classmethod
    def view(cls, buffer, offset: int, nbytes: int, *, qtype=None, shape=None, name=None) -> "DeviceWeight":
        if offset < 0 or nbytes < 0 or offset + nbytes > buffer.nbytes:
            raise ValueError(f"view [{offset}, {offset + nbytes}) outside a {buffer.nbytes}-byte buffer")
        w = cls.__new__(cls)
        w.buffer, w.offset, w.nbytes = buffer, int(offset), int(nbytes)
        w.qtype, w.shape, w.name = qtype, shape, name
        return w

    def data_ptr(self) -> int:
        return self.buffer.ptr + self.offset


def _raw_bytes(weight) -> np.ndarray:
    if hasattr(weight, "as_numpy"):          # reference tensor handle (core/tensor.py)
        weight = weight.as_numpy()
    return np.ascontiguousarray(weight, dtype=np.uint8)


_GIB = 1 << 30


def _cache_capacity(setting) -> int:
    """Bytes of device weight cache from a constructor argument or the
    FLATRUN_AMD_WEIGHT_CACHE setting: off for None / False / 0 / "" / "0",
    64 GiB for True / "1", else a byte count ("48G", "512M" or digits)."""
    if setting is None or setting is False:
        return 0
    if setting is True:
        return 64 * _GIB
    if isinstance(setting, int):
        return max(0, setting)
    txt = str(setting).strip().upper()
    if txt in ("", "0", "OFF", "NO", "FALSE"):
        return 0
    if txt in ("1", "ON", "YES", "TRUE"):
        return 64 * _GIB
    mult = {"K": 1 << 10, "M": 1 << 20, "G": _GIB, "T": 1 << 40}.get(txt[-1:], 1)
    num = txt[:-1] if txt[-1:] in "KMGT" else txt
    try:
        return max(0, int(float(num) * mult))
    except ValueError as e:
        raise ValueError(f"FLATRUN_AMD_WEIGHT_CACHE={setting!r}: expected 0/1 or a size such as 48G") from e


class NativeBackend:
    """Facade over the gfx950 kernels; mirrors python/__init__.py:85-227.

    Holds a device scratch buffer for resident-weight calls and, when
    enabled, a device weight cache. Safe to share across threads: calls that
    use the scratch or the cache run one at a time (a lock), as the
    reference's calls do under the GIL.

    ``weight_cache`` (default: the FLATRUN_AMD_WEIGHT_CACHE environment
    setting, off when unset) keeps a device copy of every host weight passed
    to a matmul, keyed by its content (byte count and 128-bit digest,
    flatrun_amd.residency), so a forwarder that passes the same weights every
    step -- as fresh copies, which is what the reference's mmap handles
    return -- pays the host to device weight copy once and a hash per call.
    True = up to 64 GiB, an int or "48G"-style string = that many bytes.

    :meth:`attach_stream` binds a :class:`flatrun_amd.streaming.SchedulerStream`:
    weights of the layer it has streamed for the scheduler are then taken
    from its device ring (checked before the cache).

    Attributes
    ----------
    available : bool
        True if the library loaded and a device is visible. Methods on an
        unavailable backend raise RuntimeError.
    """

    def __init__(self, weight_cache=None) -> None:
        self.available = is_available()
        self._neon = False
        self._scratch = None
        self._lock = threading.RLock()
        cap = _cache_capacity(os.environ.get("FLATRUN_AMD_WEIGHT_CACHE") if weight_cache is None else weight_cache)
        self._cache = WeightCache(cap) if cap > 0 else None
        self._stream_src = None

    def attach_stream(self, stream) -> None:
        """Take the weights of the scheduler's current layer from `stream`'s
        device ring (a SchedulerStream; None detaches). Weights it does not
        hold go the usual way."""
        with self._lock:
            self._stream_src = stream

    def cache_stats(self) -> dict:
        """Weight-cache occupancy: bytes, entries, hits, misses (zeros when off)."""
        c = self._cache
        if c is None:
            return {"enabled": False, "bytes": 0, "entries": 0, "hits": 0, "misses": 0}
        return {"enabled": True, "capacity": c.capacity, "bytes": c.bytes, "entries": len(c),
                "hits": c.hits, "misses": c.misses}

    def _cached(self, weight, held=()):
        """The device copy of a host weight from the attached stream or the
        cache, else None. The caller holds the lock until its launch has
        finished: a later lookup may evict (free) a cache entry, except the
        entries in `held` (those the caller's pending launch reads)."""
        if isinstance(weight, DeviceWeight) or (self._cache is None and self._stream_src is None):
            return None
        raw = _raw_bytes(weight).reshape(-1)
        if self._stream_src is not None:
            dw = self._stream_src.lookup(raw)
            if dw is not None:
                return dw
        if self._cache is None:
            return None
        return self._cache.lookup(raw, DeviceWeight, held=held)

    def _scratch_for(self, need: int):
        """The scratch buffer, grown to `need` bytes; the caller holds the lock
        and keeps the returned object (not its address) for the whole call."""
        from . import device
        if self._scratch is None or self._scratch.nbytes < need:
            self._scratch = device.DeviceBuffer(need)
        return self._scratch

    # ------------------------------------------------------------ helpers
    def _require(self) -> None:
        if not self.available:
            raise RuntimeError(
                "flatrun_amd is not available: " + version()
                + " (build with `python -m flatrun_amd.build` on a host with ROCm; a HIP device is required)")

    def _matmul(self, qname: str, x, weight, n: int, k: int):
        self._require()
        x_c = np.ascontiguousarray(x, dtype=np.float32)
        if (self._cache is not None or self._stream_src is not None) and not isinstance(weight, DeviceWeight):
            with self._lock:
                cached = self._cached(weight)
                if cached is not None:
                    return self._matmul_resident(qname, x_c, cached, n, k)
        if isinstance(weight, DeviceWeight):
            return self._matmul_resident(qname, x_c, weight, n, k)
        w_c = _raw_bytes(weight)
        fn1 = getattr(_C, f"matmul_{qname.lower()}")
        fn2 = getattr(_C, f"matmul_{qname.lower()}_batched")
        if x_c.ndim == 1:
            if x_c.shape[0] != k:
                raise ValueError(f"x.shape[0]={x_c.shape[0]} != k={k}")
            return fn1(x_c, w_c, int(n), int(k))
        if x_c.ndim == 2:
            return fn2(x_c, w_c, int(n), int(k))
        raise ValueError(f"x must be 1-D or 2-D, got shape {x_c.shape}")

    def _matmul_resident(self, qname: str, x_c: np.ndarray, weight: DeviceWeight, n: int, k: int):
        from . import device
        if x_c.ndim == 1:
            if x_c.shape[0] != k:
                raise ValueError(f"x.shape[0]={x_c.shape[0]} != k={k}")
            seq = 1
        elif x_c.ndim == 2:
            if x_c.shape[1] != k:
                raise FrqError(_lib.ERR_SHAPE, f"{qname} matmul (batched): x.shape[1] != k")
            seq = x_c.shape[0]
        else:
            raise ValueError(f"x must be 1-D or 2-D, got shape {x_c.shape}")
        n, k = int(n), int(k)
        out = np.empty((seq, n), dtype=np.float32)
        if seq and n:
            xb = (seq * k * 4 + 255) // 256 * 256
            with self._lock:
                scratch = self._scratch_for(xb + seq * n * 4)
                base = scratch.ptr
                if x_c.size:
                    _lib.check(_lib.lib().frq_memcpy_h2d(base, x_c.ctypes.data, x_c.nbytes))
                device.gemv(qname, weight, base, base + xb, n, k, batch=seq, w_bytes=weight.nbytes)
                _lib.check(_lib.lib().frq_memcpy_d2h(out.ctypes.data, base + xb, out.nbytes))
        return out[0] if x_c.ndim == 1 else out

    def upload(self, weight) -> DeviceWeight:
        """Copy raw block bytes to device memory once; pass the result as
        ``weight`` to any matmul to skip the per-call weight copy."""
        self._require()
        return DeviceWeight(_raw_bytes(weight))

    def load_gguf(self, path, names=None, **kw):
        """Every (or the named) tensor of a GGUF file resident in HBM:
        returns a :class:`flatrun_amd.gguf.ResidentModel`; ``model[name]`` is
        a DeviceWeight to pass as ``weight`` to any matmul."""
        self._require()
        from .gguf import ResidentModel
        return ResidentModel(path, names, **kw)

    # ------------------------------------------------------------ matmuls
    def matmul_q4k(self, x, weight, n: int, k: int):
        """Fused Q4_K dequant + matvec. x (k,) -> (n,), x (seq, k) -> (seq, n)."""
        return self._matmul("Q4_K", x, weight, n, k)

    def matmul_q8_0(self, x, weight, n: int, k: int):
        """Fused Q8_0 dequant + matvec (python/__init__.py:155-182)."""
        return self._matmul("Q8_0", x, weight, n, k)

    def matmul_q6_k(self, x, weight, n: int, k: int):
        """Fused Q6_K dequant + matvec (python/__init__.py:184-209)."""
        return self._matmul("Q6_K", x, weight, n, k)

    # the runtime backend's spelling (runtime/backend.py:111, 273)
    matmul_q6k = matmul_q6_k

    def matmul_fused(self, x, parts, k: int):
        """Several projections of the same x, concatenated along the output:
        ``parts`` = [(quant, weight, n), ...] (1..4 entries, quant a GGML type
        name, weight raw bytes or a DeviceWeight) returns
        ``np.concatenate([W_0 x, W_1 x, ...], axis=-1)`` -- what the
        forwarder builds from separate matmul calls for q/k/v
        (model/qwen2.py:1510-1519) and gate/up (:1690-1702) -- from one
        launch per x row when there are two or more weights, every one
        Q4_K or Q6_K (see frq_dev_gemv_group). x (k,) -> (sum n,), x (seq, k) -> (seq, sum n).
        A fused launch computes with the element-wise kernels: where a
        separate call takes the matrix cores (a large Q4_K matrix) the two
        agree to the fp32 accumulation tolerance, otherwise bit for bit."""
        self._require()
        from . import device
        x_c = np.ascontiguousarray(x, dtype=np.float32)
        if x_c.ndim == 1:
            if x_c.shape[0] != k:
                raise ValueError(f"x.shape[0]={x_c.shape[0]} != k={k}")
            seq = 1
        elif x_c.ndim == 2:
            if x_c.shape[1] != k:
                raise FrqError(_lib.ERR_SHAPE, "fused matmul (batched): x.shape[1] != k")
            seq = x_c.shape[0]
        else:
            raise ValueError(f"x must be 1-D or 2-D, got shape {x_c.shape}")
        if not 1 <= len(parts) <= device.GROUP_MAX:
            raise ValueError(f"matmul_fused takes 1..{device.GROUP_MAX} parts, got {len(parts)}")
        with self._lock:   # cache entries and the scratch stay valid until the results are back
            ns = [int(n) for _, _, n in parts]
            total = sum(ns)
            out = np.empty((seq, total), dtype=np.float32)
            temps = []
            try:
                ws = []
                for q, wgt, n in parts:
                    cached = self._cached(wgt, held=ws)
                    if cached is not None:
                        ws.append(cached)
                    elif isinstance(wgt, DeviceWeight):
                        ws.append(wgt)
                    else:
                        raw = _raw_bytes(wgt).reshape(-1)
                        dw = DeviceWeight(raw) if raw.size else None
                        temps.append(dw)
                        ws.append(dw)
                if seq and total:
                    xb = (seq * k * 4 + 255) // 256 * 256
                    with self._lock:
                        scratch = self._scratch_for(xb + seq * total * 4)
                        base = scratch.ptr
                        if x_c.size:
                            _lib.check(_lib.lib().frq_memcpy_h2d(base, x_c.ctypes.data, x_c.nbytes))
                        grp, off = [], 0
                        for (q, _, n), w in zip(parts, ws):
                            grp.append((q, w if w is not None else 0, n, base + xb + 4 * off,
                                        w.nbytes if w is not None else 0))
                            off += int(n)
                        device.gemv_group(grp, base, k, batch=seq, y_stride=total)
                        _lib.check(_lib.lib().frq_memcpy_d2h(out.ctypes.data, base + xb, out.nbytes))
            finally:
                for t in temps:
                    if t is not None:
                        t.buffer.free()
        return out[0] if x_c.ndim == 1 else out

    def matmul_q5_k(self, x, weight, n: int, k: int):
        """Fused Q5_K dequant + matvec (no native counterpart in the reference)."""
        return self._matmul("Q5_K", x, weight, n, k)

    def matmul_q1_0(self, x, weight, n: int, k: int):
        """Fused Q1_0 dequant + matvec (no native counterpart in the reference)."""
        return self._matmul("Q1_0", x, weight, n, k)

    def _gemm_bf16(self, qname: str, x, weight, n: int, k: int):
        self._require()
        if not isinstance(weight, DeviceWeight):
            return _C.matmul_bf16(qname, x, _raw_bytes(weight), n, k)
        from . import device
        xb = _C.to_bf16_bits(x)
        x2 = xb.reshape(1, -1) if xb.ndim == 1 else xb
        if x2.ndim != 2 or x2.shape[1] != k:
            raise ValueError(f"x must be ({k},) or (seq, {k}), got {np.shape(x)}")
        xd = device.DeviceBuffer.from_host(x2)
        yd = device.DeviceBuffer(max(1, x2.shape[0] * n * 4))
        try:
            device.gemm_bf16(qname, weight, xd, yd, x2.shape[0], n, k, w_bytes=weight.nbytes)
            device.synchronize()
            y = yd.to_host(np.float32)[: x2.shape[0] * n].reshape(x2.shape[0], n)
        finally:
            xd.free()
            yd.free()
        return y[0] if xb.ndim == 1 else y

    def matmul_q4k_bf16(self, x, weight, n: int, k: int):
        """Prefill GEMM on the matrix cores: x (seq, k) rounded to bf16, W
        dequantized to bf16, fp32 accumulation -> (seq, n) float32. The fp32
        per-token path (the reference's contract) is ``matmul_q4k``."""
        return self._gemm_bf16("Q4_K", x, weight, n, k)

    def matmul_q6k_bf16(self, x, weight, n: int, k: int):
        """As matmul_q4k_bf16 for Q6_K weights (fp32 path: ``matmul_q6_k``)."""
        return self._gemm_bf16("Q6_K", x, weight, n, k)

    def matmul_q8_0_bf16(self, x, weight, n: int, k: int):
        """As matmul_q4k_bf16 for Q8_0 weights (fp32 path: ``matmul_q8_0``)."""
        return self._gemm_bf16("Q8_0", x, weight, n, k)

    def matmul_fused_bf16(self, x, parts, k: int):
        """matmul_fused for the prefill GEMM: ``parts`` = [(quant, weight, n),
        ...] (1..4 entries; Q4_K, Q6_K or Q8_0; weight raw bytes or a
        DeviceWeight), x (seq, k) or (k,) rounded to bf16 ->
        ``np.concatenate([x W_0^T, x W_1^T, ...], axis=-1)`` in one GEMM launch
        (frq_dev_gemm_bf16_group)."""
        self._require()
        from . import device
        xb = _C.to_bf16_bits(x)
        x2 = xb.reshape(1, -1) if xb.ndim == 1 else xb
        if x2.ndim != 2 or x2.shape[1] != k:
            raise ValueError(f"x must be ({k},) or (seq, {k}), got {np.shape(x)}")
        if not 1 <= len(parts) <= device.GROUP_MAX:
            raise ValueError(f"matmul_fused_bf16 takes 1..{device.GROUP_MAX} parts, got {len(parts)}")
        seq, ns = x2.shape[0], [int(n) for _, _, n in parts]
        total = sum(ns)
        out = np.empty((seq, total), dtype=np.float32)
        with self._lock:
            temps, ws = [], []
            xd = device.DeviceBuffer.from_host(x2)
            yd = device.DeviceBuffer(max(1, seq * total * 4))
            try:
                for _, wgt, _ in parts:
                    if isinstance(wgt, DeviceWeight):
                        ws.append(wgt)
                    else:
                        raw = _raw_bytes(wgt).reshape(-1)
                        dw = DeviceWeight(raw) if raw.size else None
                        temps.append(dw)
                        ws.append(dw)
                if seq and total:
                    grp, off = [], 0
                    for (q, _, n), w in zip(parts, ws):
                        grp.append((q, w if w is not None else 0, n, yd.ptr + 4 * off, w.nbytes if w is not None else 0))
                        off += int(n)
                    device.gemm_bf16_group(grp, xd, seq, k, y_stride=total)
                    device.synchronize()
                    out[:] = yd.to_host(np.float32, seq * total).reshape(seq, total)
            finally:
                for t in temps:
                    if t is not None:
                        t.buffer.free()
                xd.free()
                yd.free()
        return out[0] if xb.ndim == 1 else out

    # ------------------------------------------------------------ dequant
    def dequant_q4k(self, weight, shape: tuple[int, int]):
        """Pure Q4_K dequant to f32 (out, in) (python/__init__.py:211-227)."""
        self._require()
        return _C.dequant_q4_k(_raw_bytes(weight), shape)

    def dequant_q8_0(self, weight, shape: tuple[int, int]):
        self._require()
        return _C.dequant_q8_0(_raw_bytes(weight), shape)

    def dequant_q6_k(self, weight, shape: tuple[int, int]):
        self._require()
        return _C.dequant_q6_k(_raw_bytes(weight), shape)

    def dequant_q5_k(self, weight, shape):
        self._require()
        return _C.dequant_q5_k(_raw_bytes(weight), shape)

    def dequant_q1_0(self, weight, shape):
        self._require()
        return _C.dequant_q1_0(_raw_bytes(weight), shape)

    def dequant_q4_0(self, weight, shape):
        """Q4_0 dequant (the reference decodes it in NumPy, dequant/gguf.py:81-107)."""
        self._require()
        return _C.dequant_q4_0(_raw_bytes(weight), shape)

    def dequant_q5_0(self, weight, shape):
        """Q5_0 dequant (dequant/gguf.py:302-330)."""
        self._require()
        return _C.dequant_q5_0(_raw_bytes(weight), shape)

    def dequant_q5_1(self, weight, shape):
        """Q5_1 dequant (dequant/gguf.py:333-362)."""
        self._require()
        return _C.dequant_q5_1(_raw_bytes(weight), shape)
