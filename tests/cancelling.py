"""Weight columns whose every weight is exactly zero while the block's
scales are not: the case where a matvec written as scale algebra,
s * sum(q x) - t * sum(x) or d * (sum(q x) - 32 * sum(x)), cancels two large
terms when x has an outlier in that column, so its fp32 error is set by
(|s q| + |t|) |x_j| instead of |w_j x_j| = 0.

Per format (element e of a 256-element super-block, sub-block e // 32):
  Q4_K, Q5_K  dmin := d, m_j := sc_j := 41 for the column's scale pair j,
              code q = 1:  w = fl(fl(d * 41) * 1) - fl(d * 41) = 0
              (gguf.py:166-263 op order; Q5_K's f64 step is exact here);
  Q6_K        code q = 32 (low nibble 0, high bits 2), scale kept nonzero:
              w = d * sc * (32 - 32) = 0 (gguf.py:365-420);
  Q8_0        q = 0 with d nonzero (gguf.py:112-127).
Q1_0 weights are +-d and never zero.
"""

from __future__ import annotations

import numpy as np

from oracle import gguf_np as G

BLOCK = {"Q4_K": (144, 256), "Q5_K": (176, 256), "Q6_K": (210, 256), "Q8_0": (34, 32)}
CANCEL_FORMATS = tuple(BLOCK)
_SC = 41                                       # 6-bit scale = min of the zeroed pair


def _k4_pair(blk: np.ndarray, j: int, v: int) -> None:
    """Set scale pair j (sc and m, get_scale_min_k4 layout) of blocks `blk`
    (rows x bytes view) to (v, v); scales start at byte 4."""
    s = 4
    if j < 4:
        blk[:, s + j] = (blk[:, s + j] & 0xC0) | v
        blk[:, s + j + 4] = (blk[:, s + j + 4] & 0xC0) | v
    else:
        lo, hi = v & 0x0F, v >> 4
        blk[:, s + j + 4] = lo | (lo << 4)
        blk[:, s + j - 4] = (blk[:, s + j - 4] & 0x3F) | (hi << 6)
        blk[:, s + j] = (blk[:, s + j] & 0x3F) | (hi << 6)


def cancel_columns(q: str, raw: np.ndarray, n: int, k: int, cols) -> np.ndarray:
    """A copy of `raw` (n x k weights of format q) in which every column of
    `cols` is exactly zero in every row, with nonzero block scales."""
    bb, be = BLOCK[q]
    nb = k // be
    r = np.asarray(raw, np.uint8).reshape(n, nb * bb).copy()
    for col in cols:
        b, e = divmod(int(col), be)
        blk = r[:, b * bb:(b + 1) * bb]                      # view into r
        if q == "Q8_0":
            if np.any((blk[:, 0] == 0) & ((blk[:, 1] & 0x7F) == 0)):
                blk[:, 0:2] = np.frombuffer(np.float16(0.01).tobytes(), np.uint8)
            blk[:, 2 + e] = 0
        elif q in ("Q4_K", "Q5_K"):
            blk[:, 2:4] = blk[:, 0:2]                         # dmin = d
            sb, p, i = e // 32, e // 64, e % 64
            _k4_pair(blk, sb, _SC)
            qs = 16 if q == "Q4_K" else 48
            byte = qs + 32 * p + (i % 32)
            if i < 32:
                blk[:, byte] = (blk[:, byte] & 0xF0) | 1
            else:
                blk[:, byte] = (blk[:, byte] & 0x0F) | 0x10
            if q == "Q5_K":                                   # high bit of the code: 0
                blk[:, 16 + (i % 32)] &= np.uint8(~(1 << (2 * p + (0 if i < 32 else 1))) & 0xFF)
        elif q == "Q6_K":
            h, rr = divmod(e, 128)
            kq, l = divmod(rr, 32)
            byte = 64 * h + l + (32 if kq & 1 else 0)
            if kq < 2:
                blk[:, byte] &= 0xF0
            else:
                blk[:, byte] &= 0x0F
            qh = 128 + 32 * h + l
            blk[:, qh] = (blk[:, qh] & np.uint8(~(3 << (2 * kq)) & 0xFF)) | (2 << (2 * kq))
            sc = 192 + 8 * h + l // 16 + 2 * kq
            blk[:, sc] = np.where(blk[:, sc] == 0, 23, blk[:, sc])
        else:
            raise ValueError(q)
    out = r.reshape(-1)
    w = G.DEQUANT[q](out, (n, k), np.float32)
    assert np.all(w[:, list(cols)] == 0), "cancelling columns are not zero"
    return out


def outlier_x(k: int, cols, seed: int, big=(2.0**24, -(2.0**20), 2.0**28)) -> np.ndarray:
    """N(0, 1) x with outlier values `big` (cycled) at the columns `cols`."""
    x = np.random.default_rng(seed).standard_normal(k).astype(np.float32)
    for i, c in enumerate(cols):
        x[c] = np.float32(big[i % len(big)])
    return x
