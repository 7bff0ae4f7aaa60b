"""Handle-level dequant on the GPU: ``dequant_handle(handle, dtype="float16")``
with the reference's semantics (src/flatrun/dequant/loader.py:51-88).

The handle's ``metadata.quantization`` picks the format; the raw block bytes
come from ``handle.as_numpy()`` (a zero-copy view for mmap handles, a copy
for the reference's ``MmapTensorHandle``) and are decoded by the library:
fp16 output straight from the kernels (``frq_dequant_f16``: the fp32
dequant value rounded once to nearest even, which is what the reference's
decoders produce, an fp32 array cast by ``_finish`` with ``astype``,
gguf.py:61-73), fp32 output from ``frq_dequant``, any other dtype from the
fp32 result with ``astype``. A tensor without a quantization tag is returned
as ``as_numpy()`` cast to ``dtype``, as in the reference.
"""

from __future__ import annotations

import numpy as np

from . import _C, _lib
from .gguf import GGML_TYPES, TYPE_IDS

# the formats of the reference's _GGUF_DECODERS (loader.py:31-40)
GGUF_DECODERS = ("Q1_0", "Q4_0", "Q5_0", "Q5_1", "Q8_0", "Q4_K", "Q5_K", "Q6_K")


def _block(qname: str) -> tuple[int, int]:
    t = GGML_TYPES[TYPE_IDS[qname]]
    return t.type_size, t.block_size


def dequant(qname: str, raw, shape, dtype="float32") -> np.ndarray:
    """Decode raw blocks of format `qname` into an array of `shape` and
    `dtype` (the reference decoders' signature: ceil-div blocks, tail
    trimmed). A byte count that does not match the shape raises ValueError,
    as the reference decoders' reshape does."""
    dt = np.dtype(dtype)
    shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
    size = int(np.prod(shape)) if shape else 1
    if size == 0:
        return np.empty(0, dtype=dt).reshape(shape)
    w = np.ascontiguousarray(np.frombuffer(raw, dtype=np.uint8) if isinstance(raw, (bytes, bytearray, memoryview))
                             else np.asarray(raw, dtype=np.uint8)).reshape(-1)
    bb, be = _block(qname)
    nblk = -(-size // be)
    if w.size != nblk * bb:
        raise ValueError(f"{qname}: {size} elements need {nblk * bb} bytes of blocks, got {w.size}")
    if dt == np.float16:
        out = np.empty(size, dtype=np.uint16)
        _lib.check(_lib.lib().frq_dequant_f16(TYPE_IDS[qname], w.ctypes.data, w.size, size, out.ctypes.data))
        return out.view(np.float16).reshape(shape)
    y = _C.dequant(qname, w, shape)
    return y if dt == np.float32 else y.astype(dt, copy=False)


def dequant_handle(handle, dtype: str = "float16") -> np.ndarray:
    """Dequantize one tensor handle (loader.py:51-88): the handle's
    ``metadata.quantization`` selects the decoder; no tag returns
    ``handle.as_numpy()`` cast to `dtype`; ``MLX_4BIT`` and unknown tags raise
    ValueError."""
    q = handle.metadata.quantization
    if q is None:
        arr = handle.as_numpy()
        if arr.dtype != np.dtype(dtype):
            arr = arr.astype(dtype)
        return arr
    if q == "MLX_4BIT":
        raise ValueError("Use dequant_mlx_weight() for MLX 4-bit tensors")
    if q not in GGUF_DECODERS:
        raise ValueError(f"flatrun has no decoder for ggml quant type {q!r}. "
                         f"Supported types: {sorted(GGUF_DECODERS)}.")
    return dequant(q, handle.as_numpy(), handle.metadata.shape, np.dtype(dtype))


__all__ = ["GGUF_DECODERS", "dequant", "dequant_handle"]
