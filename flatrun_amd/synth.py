"""Seeded synthetic GGUF blocks for tests and benchmarks.

``make_blocks(qname, n, k, seed)`` returns the raw bytes of an (n, k) weight
with the distributions of the benchmark workloads:

* Q8_0: d = fp16(U[1e-4, 1e-2]), q int8 U[-127, 127]
* Q4_K: d, dmin = fp16(U[1e-4, 5e-3]); 8 scales and 8 mins U[0, 63]; q U[0, 15]
* Q5_K: as Q4_K, plus the 5th bit of every element Bernoulli(0.5)
* Q6_K: q6 U[0, 63]; 16 int8 scales U[-64, 63]; d fp16(U[1e-4, 5e-3])
* Q1_0: d = fp16(U[1e-3, 1e-2]); sign bits Bernoulli(0.5)
* Q4_0 / Q5_0: d = fp16(U[1e-3, 1e-2]); nibbles (and 5th bits) uniform
* Q5_1: d = fp16(U[1e-3, 1e-2]), m = fp16(U[-0.1, 0.1]); as Q5_0

Uniform random bytes are exactly uniform on every packed field: the 12-byte
K-quant scale field is a bijection of the sixteen 6-bit values (high bits
included, unlike the reference's test generators, which leave them zero),
each Q4_K / Q5_K nibble and each Q6_K (4-bit + 2-bit) pair is uniform, and
each sign bit is Bernoulli(0.5). So only the fp16 scales and the Q8_0 / Q6_K
int8 fields are drawn separately.

The ``pack_*`` helpers build blocks from logical values (the inverse of the
decoders in src/flatrun/dequant/gguf.py) for hand-made test blocks.
"""

from __future__ import annotations

import numpy as np

BLOCK = {"Q8_0": (34, 32), "Q4_K": (144, 256), "Q5_K": (176, 256), "Q6_K": (210, 256), "Q1_0": (18, 128),
         "Q4_0": (18, 32), "Q5_0": (22, 32), "Q5_1": (24, 32)}


def nbytes(qname: str, n: int, k: int) -> int:
    bb, be = BLOCK[qname]
    if k % be:
        raise ValueError(f"{qname}: k={k} is not a multiple of {be}")
    return n * (k // be) * bb


def _f16(rng, lo, hi, count) -> np.ndarray:
    return rng.uniform(lo, hi, count).astype(np.float16).view(np.uint16)


def _put_u16(blocks: np.ndarray, off: int, v: np.ndarray) -> None:
    blocks[:, off] = (v & 0xFF).astype(np.uint8)
    blocks[:, off + 1] = (v >> 8).astype(np.uint8)


def make_blocks(qname: str, n: int, k: int, seed: int = 0) -> np.ndarray:
    """Raw bytes (uint8, 1-D) of an (n, k) weight in format ``qname``."""
    bb, be = BLOCK[qname]
    total = nbytes(qname, n, k)
    nblk = total // bb
    rng = np.random.default_rng(seed)
    raw = rng.integers(0, 256, size=total, dtype=np.uint8)
    b = raw.reshape(nblk, bb)
    if qname == "Q8_0":
        _put_u16(b, 0, _f16(rng, 1e-4, 1e-2, nblk))
        b[:, 2:34] = rng.integers(-127, 128, size=(nblk, 32), dtype=np.int8).view(np.uint8)
    elif qname in ("Q4_K", "Q5_K"):
        _put_u16(b, 0, _f16(rng, 1e-4, 5e-3, nblk))
        _put_u16(b, 2, _f16(rng, 1e-4, 5e-3, nblk))
    elif qname in ("Q4_0", "Q5_0", "Q5_1"):
        _put_u16(b, 0, _f16(rng, 1e-3, 1e-2, nblk))
        if qname == "Q5_1":
            _put_u16(b, 2, _f16(rng, -0.1, 0.1, nblk))
    elif qname == "Q6_K":
        b[:, 192:208] = rng.integers(-64, 64, size=(nblk, 16), dtype=np.int8).view(np.uint8)
        _put_u16(b, 208, _f16(rng, 1e-4, 5e-3, nblk))
    elif qname == "Q1_0":
        _put_u16(b, 0, _f16(rng, 1e-3, 1e-2, nblk))
    else:
        raise ValueError(qname)
    return raw


def make_x(k: int, seed: int = 1, batch: int | None = None) -> np.ndarray:
    rng = np.random.default_rng(seed)
    shape = (k,) if batch is None else (batch, k)
    return rng.standard_normal(shape).astype(np.float32)


# ------------------------------------------------------------------ packers

def _h(v) -> np.ndarray:
    return np.asarray(v, dtype=np.float16).reshape(-1).view(np.uint16)


def pack_scale_min_k4(sc: np.ndarray, m: np.ndarray) -> np.ndarray:
    """(nblk, 8) 6-bit scales and mins -> (nblk, 12) bytes (inverse of
    get_scale_min_k4, gguf.py:135-163)."""
    sc = np.asarray(sc, dtype=np.uint8).reshape(-1, 8)
    m = np.asarray(m, dtype=np.uint8).reshape(-1, 8)
    if (sc > 63).any() or (m > 63).any():
        raise ValueError("scales and mins are 6-bit")
    out = np.empty((sc.shape[0], 12), dtype=np.uint8)
    out[:, 0:4] = (sc[:, 0:4] & 63) | ((sc[:, 4:8] >> 4) << 6)
    out[:, 4:8] = (m[:, 0:4] & 63) | ((m[:, 4:8] >> 4) << 6)
    out[:, 8:12] = (sc[:, 4:8] & 15) | ((m[:, 4:8] & 15) << 4)
    return out


def _pack_k_nibbles(q: np.ndarray) -> np.ndarray:
    """(nblk, 256) values 0..15 -> (nblk, 128) qs bytes (group g: byte 32g+i
    holds element 64g+i low and 64g+32+i high)."""
    q = np.asarray(q, dtype=np.uint8).reshape(-1, 4, 2, 32)
    return (q[:, :, 0, :] | (q[:, :, 1, :] << 4)).reshape(-1, 128)


def pack_q4_k(d, dmin, sc, m, q) -> np.ndarray:
    q = np.asarray(q).reshape(-1, 256)
    if (q > 15).any() or (q < 0).any():
        raise ValueError("Q4_K values are 4-bit")
    nblk = q.shape[0]
    b = np.zeros((nblk, 144), dtype=np.uint8)
    _put_u16(b, 0, np.broadcast_to(_h(d), (nblk,)))
    _put_u16(b, 2, np.broadcast_to(_h(dmin), (nblk,)))
    b[:, 4:16] = pack_scale_min_k4(sc, m)
    b[:, 16:144] = _pack_k_nibbles(q)
    return b.reshape(-1)


def pack_q5_k(d, dmin, sc, m, q) -> np.ndarray:
    q = np.asarray(q).reshape(-1, 256)
    if (q > 31).any() or (q < 0).any():
        raise ValueError("Q5_K values are 5-bit")
    nblk = q.shape[0]
    b = np.zeros((nblk, 176), dtype=np.uint8)
    _put_u16(b, 0, np.broadcast_to(_h(d), (nblk,)))
    _put_u16(b, 2, np.broadcast_to(_h(dmin), (nblk,)))
    b[:, 4:16] = pack_scale_min_k4(sc, m)
    hi = (q >> 4).astype(np.uint8).reshape(nblk, 8, 32)          # sub-block j -> bit j of qh[i]
    qh = np.zeros((nblk, 32), dtype=np.uint8)
    for j in range(8):
        qh |= hi[:, j, :] << j
    b[:, 16:48] = qh
    b[:, 48:176] = _pack_k_nibbles(q & 15)
    return b.reshape(-1)


def pack_q6_k(d, scales, q) -> np.ndarray:
    """q: (nblk, 256) values 0..63 (stored q; decoded value is q - 32)."""
    q = np.asarray(q).reshape(-1, 256).astype(np.uint8)
    if (q > 63).any():
        raise ValueError("Q6_K values are 6-bit")
    nblk = q.shape[0]
    b = np.zeros((nblk, 210), dtype=np.uint8)
    qq = q.reshape(nblk, 2, 4, 32)                                # [half][k][l]
    ql = np.zeros((nblk, 2, 2, 32), dtype=np.uint8)
    ql[:, :, 0, :] = (qq[:, :, 0, :] & 15) | ((qq[:, :, 2, :] & 15) << 4)
    ql[:, :, 1, :] = (qq[:, :, 1, :] & 15) | ((qq[:, :, 3, :] & 15) << 4)
    qh = np.zeros((nblk, 2, 32), dtype=np.uint8)
    for kk in range(4):
        qh |= (qq[:, :, kk, :] >> 4) << (2 * kk)
    b[:, 0:128] = ql.reshape(nblk, 128)
    b[:, 128:192] = qh.reshape(nblk, 64)
    b[:, 192:208] = np.asarray(scales, dtype=np.int8).reshape(-1, 16).view(np.uint8)
    _put_u16(b, 208, np.broadcast_to(_h(d), (nblk,)))
    return b.reshape(-1)


def pack_q8_0(d, q) -> np.ndarray:
    q = np.asarray(q, dtype=np.int8).reshape(-1, 32)
    nblk = q.shape[0]
    b = np.zeros((nblk, 34), dtype=np.uint8)
    _put_u16(b, 0, np.broadcast_to(_h(d), (nblk,)))
    b[:, 2:34] = q.view(np.uint8)
    return b.reshape(-1)


def pack_q1_0(d, bits) -> np.ndarray:
    bits = np.asarray(bits, dtype=np.uint8).reshape(-1, 128)
    nblk = bits.shape[0]
    b = np.zeros((nblk, 18), dtype=np.uint8)
    _put_u16(b, 0, np.broadcast_to(_h(d), (nblk,)))
    b[:, 2:18] = np.packbits(bits, axis=1, bitorder="little")
    return b.reshape(-1)
