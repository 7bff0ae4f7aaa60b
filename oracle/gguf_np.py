"""NumPy restatement of the reference GGUF dequantizers (oracle; test-only).

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s ``cpu_baseline`` leg, never by ``flatrun_amd``.

Every function follows the op order and the dtypes of the matching function in
``src/flatrun/dequant/gguf.py`` of the reference, because the GPU dequant
kernels are held to *bit-exact* agreement with those functions:

* Q8_0  ``y = fl32(q * d)``                                   (gguf.py:112-127)
* Q4_K  ``y = fl32(fl32(fl32(d*sc) * q) - fl32(dmin*m))``      (gguf.py:166-220)
* Q5_K  ``y = fl32(fl64(fl32(d*sc) * v) - fl32(dmin*m))``      (gguf.py:223-263)
        -- ``np.where(..., 16.0, 0.0)`` is float64, so ``v`` and the product
        are float64 and the result is rounded twice (f64, then f32 on store).
* Q6_K  ``y = fl32(fl32(d*sc) * (q - 32))``                    (gguf.py:365-420)
* Q1_0  ``y = +d`` if bit set else ``-d``, bits LSB-first      (gguf.py:266-299)
* Q4_0  ``y = fl32((q - 8) * d)``, low nibbles first half      (gguf.py:81-107)
* Q5_0  ``y = fl32((q - 16) * d)``, 5th bit from ``qh``        (gguf.py:302-330)
* Q5_1  ``y = fl32(fl32(d * q) + m)``                          (gguf.py:333-362)

Like the reference, every decoder accepts a size that is not a multiple of the
block and trims the decoded tail (``_finish``, gguf.py:61-73); the tail block
must still be present in ``raw`` (ceil-div block count).

Parity pins (tests/test_oracle_*.py):
* Q4_K, Q6_K, Q8_0: bit-exact against the reference's own compiled C++
  dequant (``oracle/_ref``, built from ``src/flatrun_native/_C.cpp``) on seeded
  blocks, and against committed vectors written from that build
  (``tests/golden/ref_native_vectors.npz``); closed-form hand blocks that pin
  element order, the 6-bit scale high bits and every Q6_K ``qh`` bit pair;
  the reference KATs of ``src/flatrun/tests/test_dequant.py``.
* Q5_K: golden vectors written by importing the reference decoder
  (``tests/golden/make_q5k_vectors.py``) when that import is permitted, plus
  closed-form blocks (qh bit -> +16 per element, double-rounding cases) and
  the zero-block KAT.
* Q1_0: the reference KATs (0xAA/0x01 pattern, zero block, 130-element tail)
  and the closed form ``+-d``.
* Q4_0 / Q5_0 / Q5_1: the reference KATs (test_dequant.py:60-72, 212-238),
  plus hand blocks that set one qs nibble or one qh bit at a time and check
  the one element it lands on (element order and bit position), and the
  exactness of every product (fp16 scale times a <= 5-bit integer).
"""

from __future__ import annotations

import numpy as np

QK_K = 256

# GGML type id -> (name, bytes per block, elements per block);
# the ids and sizes are those of ``_GGML_TYPES`` (backend/gguf.py:59-86).
GGML_TYPES = {
    8: ("Q8_0", 34, 32),
    12: ("Q4_K", 144, 256),
    13: ("Q5_K", 176, 256),
    14: ("Q6_K", 210, 256),
    41: ("Q1_0", 18, 128),
    2: ("Q4_0", 18, 32),
    6: ("Q5_0", 22, 32),
    7: ("Q5_1", 24, 32),
}
BLOCK = {name: (nbytes, nel) for _, (name, nbytes, nel) in GGML_TYPES.items()}


def _u8(raw) -> np.ndarray:
    """bytes / bytearray / ndarray -> flat uint8 view (gguf.py:29-41)."""
    if isinstance(raw, np.ndarray):
        a = raw if raw.dtype == np.uint8 else raw.astype(np.uint8)
        return a.reshape(-1)
    return np.frombuffer(bytes(raw), dtype=np.uint8)


def _blocks(raw, shape, qname):
    size = int(np.prod(shape))
    nbytes, nel = BLOCK[qname]
    nblk = -(-size // nel)
    arr = _u8(raw)
    if arr.size != nblk * nbytes:
        raise ValueError(f"{qname}: expected {nblk * nbytes} bytes for {size} elements, got {arr.size}")
    return size, nblk, arr.reshape(nblk, nbytes)


def _half(col2: np.ndarray) -> np.ndarray:
    """Two little-endian bytes per row -> float32 (gguf.py:50-58)."""
    return np.ascontiguousarray(col2).view("<f2").astype(np.float32).reshape(-1)


def _done(dec: np.ndarray, size: int, shape, dtype) -> np.ndarray:
    """Trim block padding and reshape (gguf.py:61-73)."""
    return dec.reshape(-1)[:size].astype(dtype, copy=False).reshape(shape)


def scale_min_k4(sc12: np.ndarray):
    """12 packed bytes -> (sc, m), each (nblk, 8) float32 (gguf.py:135-163).

    j < 4 : sc = b[j] & 63,                       m = b[j+4] & 63
    j >= 4: sc = (b[j+4] & 15) | (b[j-4] >> 6) << 4, m = (b[j+4] >> 4) | (b[j] >> 6) << 4
    """
    b = sc12.astype(np.uint16)
    lo, mid, hi = b[:, 0:4], b[:, 4:8], b[:, 8:12]
    sc = np.concatenate([lo & 63, (hi & 15) | ((lo >> 6) << 4)], axis=1)
    m = np.concatenate([mid & 63, (hi >> 4) | ((mid >> 6) << 4)], axis=1)
    return sc.astype(np.float32), m.astype(np.float32)


def _nibbles_k(qs128: np.ndarray) -> np.ndarray:
    """128 qs bytes -> (nblk, 8, 32) uint8 where sub-block j = 2g + hi.

    Group g uses bytes 32g..32g+31: the low nibbles are elements 64g+i and the
    high nibbles 64g+32+i (gguf.py:209-219).
    """
    q = qs128.reshape(-1, 4, 1, 32)
    return np.concatenate([q & 0x0F, q >> 4], axis=2).reshape(-1, 8, 32)


def dequant_q8_0(raw, shape, dtype=np.float32) -> np.ndarray:
    size = int(np.prod(shape))
    if size == 0:
        return np.empty(0, dtype=dtype).reshape(shape)
    size, nblk, a = _blocks(raw, shape, "Q8_0")
    d = _half(a[:, 0:2])
    q = a[:, 2:34].view(np.int8).astype(np.float32)
    return _done(q * d[:, None], size, shape, dtype)


def dequant_q4_k(raw, shape, dtype=np.float32) -> np.ndarray:
    size = int(np.prod(shape))
    if size == 0:
        return np.empty(0, dtype=dtype).reshape(shape)
    size, nblk, a = _blocks(raw, shape, "Q4_K")
    d = _half(a[:, 0:2])
    dmin = _half(a[:, 2:4])
    sc, m = scale_min_k4(a[:, 4:16])
    scale = d[:, None] * sc            # fl32(d*sc)      (nblk, 8)
    offs = dmin[:, None] * m           # fl32(dmin*m)    (nblk, 8)
    q = _nibbles_k(a[:, 16:144]).astype(np.float32)
    dec = scale[:, :, None] * q - offs[:, :, None]
    return _done(dec, size, shape, dtype)


def dequant_q5_k(raw, shape, dtype=np.float32) -> np.ndarray:
    size = int(np.prod(shape))
    if size == 0:
        return np.empty(0, dtype=dtype).reshape(shape)
    size, nblk, a = _blocks(raw, shape, "Q5_K")
    d = _half(a[:, 0:2])
    dmin = _half(a[:, 2:4])
    sc, m = scale_min_k4(a[:, 4:16])
    scale = d[:, None] * sc            # float32
    offs = dmin[:, None] * m           # float32
    qh = a[:, 16:48]                   # (nblk, 32), shared by all groups
    q4 = _nibbles_k(a[:, 48:176]).astype(np.float32)          # (nblk, 8, 32)
    j = np.arange(8, dtype=np.uint8)
    bit = (qh[:, None, :] >> j[None, :, None]) & 1             # sub-block j tests bit j
    v = q4.astype(np.float64) + 16.0 * bit                     # float64, exact
    dec64 = scale[:, :, None].astype(np.float64) * v - offs[:, :, None].astype(np.float64)
    return _done(dec64.astype(np.float32), size, shape, dtype)


def dequant_q6_k(raw, shape, dtype=np.float32) -> np.ndarray:
    size = int(np.prod(shape))
    if size == 0:
        return np.empty(0, dtype=dtype).reshape(shape)
    size, nblk, a = _blocks(raw, shape, "Q6_K")
    ql = a[:, 0:128].reshape(nblk, 2, 2, 32)     # [half][lo32/hi32][l]
    qh = a[:, 128:192].reshape(nblk, 2, 32)      # [half][l]
    sc = a[:, 192:208].view(np.int8).astype(np.float32).reshape(nblk, 2, 8)
    d = _half(a[:, 208:210])
    # element 128*h + 32*k + l, k = 0..3:
    #   nibble source ql[h][k & 1][l], low nibble for k < 2, high for k >= 2
    #   high bits (qh[h][l] >> 2k) & 3, scale sc[h][l // 16 + 2k]
    k = np.arange(4)
    nib = ql[:, :, k & 1, :]                                   # (nblk, 2, 4, 32)
    nib = np.where((k >= 2)[None, None, :, None], nib >> 4, nib & 0x0F)
    hb = (qh[:, :, None, :] >> (2 * k)[None, None, :, None].astype(np.uint8)) & 3
    q = (nib | (hb << 4)).astype(np.float32) - 32.0            # exact
    l = np.arange(32)
    sidx = (l // 16)[None, :] + 2 * k[:, None]                 # (4, 32)
    s = d[:, None, None, None] * sc[:, :, sidx]                # fl32(d*sc) (nblk, 2, 4, 32)
    return _done(s * q, size, shape, dtype)


def dequant_q1_0(raw, shape, dtype=np.float32) -> np.ndarray:
    size = int(np.prod(shape))
    if size == 0:
        return np.empty(0, dtype=dtype).reshape(shape)
    size, nblk, a = _blocks(raw, shape, "Q1_0")
    d = _half(a[:, 0:2])
    bits = np.unpackbits(a[:, 2:18], axis=1, bitorder="little")   # LSB-first
    sign = np.where(bits == 1, np.float32(1.0), np.float32(-1.0))
    return _done(sign * d[:, None], size, shape, dtype)


def _q5_high(a: np.ndarray, off: int) -> tuple[np.ndarray, np.ndarray]:
    """16 * (5th bit) for elements j and j + 16 of each block: bit j and bit
    j + 16 of the little-endian uint32 at byte ``off`` (gguf.py:316-319)."""
    qh = a[:, off:off + 4].copy().view(np.uint32).reshape(-1)
    j = np.arange(16, dtype=np.uint32)
    lo = ((qh[:, None] >> j[None, :]) & np.uint32(1)) << np.uint32(4)
    hi = ((qh[:, None] >> (j[None, :] + np.uint32(16))) & np.uint32(1)) << np.uint32(4)
    return lo.astype(np.uint8), hi.astype(np.uint8)


def dequant_q4_0(raw, shape, dtype=np.float32) -> np.ndarray:
    size = int(np.prod(shape))
    if size == 0:
        return np.empty(0, dtype=dtype).reshape(shape)
    size, nblk, a = _blocks(raw, shape, "Q4_0")
    d = _half(a[:, 0:2])
    qs = a[:, 2:18]
    q = np.concatenate([qs & 0x0F, qs >> 4], axis=1).astype(np.float32) - np.float32(8.0)
    return _done(q * d[:, None], size, shape, dtype)


def dequant_q5_0(raw, shape, dtype=np.float32) -> np.ndarray:
    size = int(np.prod(shape))
    if size == 0:
        return np.empty(0, dtype=dtype).reshape(shape)
    size, nblk, a = _blocks(raw, shape, "Q5_0")
    d = _half(a[:, 0:2])
    hlo, hhi = _q5_high(a, 2)
    qs = a[:, 6:22]
    q = np.concatenate([(qs & 0x0F) | hlo, (qs >> 4) | hhi], axis=1).astype(np.float32) - np.float32(16.0)
    return _done(q * d[:, None], size, shape, dtype)


def dequant_q5_1(raw, shape, dtype=np.float32) -> np.ndarray:
    size = int(np.prod(shape))
    if size == 0:
        return np.empty(0, dtype=dtype).reshape(shape)
    size, nblk, a = _blocks(raw, shape, "Q5_1")
    d = _half(a[:, 0:2])
    m = _half(a[:, 2:4])
    hlo, hhi = _q5_high(a, 4)
    qs = a[:, 8:24]
    q = np.concatenate([(qs & 0x0F) | hlo, (qs >> 4) | hhi], axis=1).astype(np.float32)
    return _done(d[:, None] * q + m[:, None], size, shape, dtype)


DEQUANT = {
    "Q4_0": dequant_q4_0,
    "Q5_0": dequant_q5_0,
    "Q5_1": dequant_q5_1,
    "Q8_0": dequant_q8_0,
    "Q4_K": dequant_q4_k,
    "Q5_K": dequant_q5_k,
    "Q6_K": dequant_q6_k,
    "Q1_0": dequant_q1_0,
}


def matmul_numpy(qname: str, x: np.ndarray, raw, n: int, k: int) -> np.ndarray:
    """The reference's NumPy matvec: ``dequant(raw, (n, k), f32) @ x``
    (``PythonBackend.matmul_*``, runtime/backend.py:203-213). x is (k,) or
    (seq, k); for 2-D x the reference forwarder computes ``x @ W.T``."""
    w = DEQUANT[qname](raw, (n, k), np.float32)
    x = np.asarray(x, dtype=np.float32)
    return w @ x if x.ndim == 1 else x @ w.T


def matmul_f64(qname: str, x: np.ndarray, raw, n: int, k: int) -> np.ndarray:
    """fp64 yardstick: exact fp32 weights upcast, fp64 products and sums."""
    w = DEQUANT[qname](raw, (n, k), np.float32).astype(np.float64)
    x64 = np.asarray(x, dtype=np.float32).astype(np.float64)
    return w @ x64 if x64.ndim == 1 else x64 @ w.T


def abs_matmul_f64(qname: str, x: np.ndarray, raw, n: int, k: int) -> np.ndarray:
    """``sum_j |w_ij x_j|`` -- the scale for the componentwise error bound."""
    w = np.abs(DEQUANT[qname](raw, (n, k), np.float32).astype(np.float64))
    x64 = np.abs(np.asarray(x, dtype=np.float32).astype(np.float64))
    return w @ x64 if x64.ndim == 1 else x64 @ w.T
