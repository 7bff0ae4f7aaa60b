"""A NumPy model of the matrix-core Q1_0 GEMV's arithmetic (finite x).

The kernel (frq_gemv_mx.hip) works per 32-element group g of each 128-element
block: with max |x_g| < 2^e (frexp; e = 0 for a zero group) each x becomes
m = trunc(x 2^(30-e)), |m| < 2^30, written as four balanced int8 digits; the
int8 matrix cores give, per row and digit i, C_i = sum over set bits of
digit_i and J_i = sum of digit_i; S = sum_i 256^i (2 C_i - J_i) =
sum_e (+-m_e) exactly, and the group adds ldexp(fl(fl(S) * d), e - 30) to its
lane's fp32 sum. Wave v owns blocks [vL, vL + L); a block past the row's end
repeats the wave's last block with d = 0. A row's result is, in fp32 and in
this order, ((g0 + g1) + (g2 + g3)) per wave, then the waves in order.

This is a model of the kernel, not of the reference: the oracle
(oracle/gguf_np.py) is what parity is checked against; the model lets a GPU
test compare the kernel's bits with what its arithmetic must give, and the
CPU tests check the scheme's error bound.
"""

from __future__ import annotations

import numpy as np

GROUP = 32


def balanced_digits(m: np.ndarray) -> np.ndarray:
    """(..., 4) int8 digits of int32 m (|m| < 2^30) with m = sum_i d_i 256^i:
    the bytes of m + 0x808080 minus 128 for the low three, the top byte as a
    signed byte."""
    u = (np.asarray(m, np.int64) + 0x808080) & 0xFFFFFFFF
    b = np.stack([(u >> (8 * i)) & 0xFF for i in range(4)], axis=-1).astype(np.int64)
    b[..., :3] -= 128
    b[..., 3] = np.where(b[..., 3] >= 128, b[..., 3] - 256, b[..., 3])
    return b.astype(np.int8)


def group_split(x: np.ndarray):
    """x (nb * 128,) fp32 -> (m int64 (nb, 4, 32), eo int (nb, 4)) with
    m = trunc(x 2^(30-e)) and eo = e - 30 per 32-element group."""
    xg = np.asarray(x, np.float32).reshape(-1, 4, GROUP).astype(np.float64)
    mx = np.max(np.abs(xg), axis=2)
    e = np.frexp(mx)[1].astype(np.int64)                       # mx < 2^e; 0 for 0
    m = np.trunc(np.ldexp(xg, (30 - e)[:, :, None])).astype(np.int64)
    return m, e - 30


def _blocks(raw, n, nb):
    a = np.asarray(raw, np.uint8).reshape(n, nb, 18)
    d = a[:, :, 0:2].copy().view("<f2").astype(np.float32)[:, :, 0]
    bits = np.unpackbits(a[:, :, 2:18], axis=2, bitorder="little").reshape(n, nb, 4, GROUP)
    return d, bits


def group_values(raw, x, n: int, k: int):
    """fp32 (n, nb, 4) arrays (fl(S), ldexp(fl(fl(S) * d), e - 30)) of every
    (row, block, group)."""
    nb = k // 128
    m, eo = group_split(x)
    d, bits = _blocks(raw, n, nb)
    mf = m.astype(np.float64)
    msum = mf.sum(axis=2)                                       # sum of m per (block, group), exact
    vs = np.empty((n, nb, 4), np.float32)
    out = np.empty((n, nb, 4), np.float32)
    for r0 in range(0, n, 256):
        bb = bits[r0:r0 + 256].astype(np.float64)
        s = 2.0 * np.einsum("rbge,bge->rbg", bb, mf) - msum[None]   # sum of +-m, exact (< 2^36)
        v = s.astype(np.float32)
        vs[r0:r0 + 256] = v
        t = v * d[r0:r0 + 256, :, None]
        out[r0:r0 + 256] = np.ldexp(t, np.broadcast_to(eo[None], t.shape).astype(np.int32)).astype(np.float32)
    return vs, out


def default_blocks_per_wave(nb: int) -> int:
    L = 2
    while L < 8 and (nb + L - 1) // L > 8:
        L *= 2
    return L


def emulate(raw, x, n: int, k: int, L: int) -> np.ndarray:
    """The kernel's fp32 result for finite x with L blocks per wavefront."""
    nb = k // 128
    vs, gv = group_values(raw, x, n, k)                         # (n, nb, 4)
    y = np.zeros(n, np.float32)
    for v in range((nb + L - 1) // L):
        b0 = v * L
        lw = min(L, nb - b0)
        acc = np.zeros((n, 4), np.float32)
        for j in range(L):
            if j < lw:
                acc = (acc + gv[:, b0 + j, :]).astype(np.float32)
            else:                                               # the last block again, times d = 0
                acc = (acc + vs[:, b0 + lw - 1, :] * np.float32(0.0)).astype(np.float32)
        wave = ((acc[:, 0] + acc[:, 1]) + (acc[:, 2] + acc[:, 3])).astype(np.float32)
        y = (y + wave).astype(np.float32)
    return y
