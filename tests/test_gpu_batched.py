"""The fp32-contract batched matvec (frq_gemm_f32.hip) against the oracle.

The reference's batched entry points (matmul_<q>_batched, _C.cpp:154-283)
multiply every row of x by W with an fp32 matvec. The library runs two or
more rows of Q4_K, Q6_K or Q8_0 through one matrix-core GEMM that reads W
once per tile of x rows, with W as exact integer codes and x as three bf16
pieces (a few rows: the small-M matvec of frq_gemv_mr.hip, W read once
per two or three rows), so the contract is the matvec's: 1e-5 of fp64,
normwise and componentwise, for every row. Cases: seq = 4, 32 and 512 (the reference CLI
re-prefills the whole sequence on every step) at the benchmark shapes,
ragged row counts around the 32 / 64-row tiles, K-split and unsplit grids,
x with outliers on zero-weight columns and massive activations, strided
output rows (the grouped call's concatenation), and the no-allocation entry
point.
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import assert_matvec_close, bits_equal
from flatrun_amd import _C, _lib, device, synth
from oracle import gguf_np as G

pytestmark = pytest.mark.gpu


def dev_batched(q, raw, xs, n, k):
    b = xs.shape[0]
    w = device.DeviceBuffer.from_host(raw)
    xd = device.DeviceBuffer.from_host(xs)
    yd = device.DeviceBuffer(4 * n * b)
    try:
        nan = np.full(n * b, np.nan, np.float32)
        _lib.check(_lib.lib().frq_memcpy_h2d(yd.ptr, nan.ctypes.data, nan.nbytes))
        device.gemv(q, w, xd, yd, n, k, batch=b)
        device.synchronize()
        return yd.to_host(np.float32).reshape(b, n)
    finally:
        w.free()
        xd.free()
        yd.free()


def oracle_rows(q, raw, xs, n, k, y, what):
    y64 = G.matmul_f64(q, xs, raw, n, k)
    a64 = G.abs_matmul_f64(q, xs, raw, n, k)
    worst = (0.0, 0.0)
    for r in range(xs.shape[0]):
        nw, cw = assert_matvec_close(y[r], y64[r], a64[r], what=f"{what} row {r}")
        worst = (max(worst[0], nw), max(worst[1], cw))
    return worst


@pytest.mark.parametrize("q,n,k,seq", [
    ("Q4_K", 3584, 18944, 4), ("Q4_K", 3584, 18944, 32), ("Q4_K", 14336, 4096, 512),
    ("Q6_K", 4096, 14336, 4), ("Q6_K", 1024, 4096, 32), ("Q6_K", 4096, 14336, 512),
    ("Q8_0", 4864, 896, 4), ("Q8_0", 4864, 896, 32), ("Q8_0", 4096, 4096, 512),
])
def test_batched_seq_sizes(frq, q, n, k, seq):
    raw = synth.make_blocks(q, n, k, seed=n + k + seq)
    xs = synth.make_x(k, seed=seq, batch=seq)
    y = dev_batched(q, raw, xs, n, k)
    assert np.all(np.isfinite(y))
    oracle_rows(q, raw, xs, n, k, y, f"{q} {n}x{k} seq {seq}")


@pytest.mark.parametrize("q", ["Q4_K", "Q6_K", "Q8_0"])
@pytest.mark.parametrize("seq", [2, 3, 31, 33, 63, 65, 100])
def test_batched_ragged_rows(frq, q, seq):
    """Row counts around the 32- and 64-row tiles and N not a tile multiple."""
    n, k = 300, 1024
    raw = synth.make_blocks(q, n, k, seed=seq + 5)
    xs = synth.make_x(k, seed=seq + 6, batch=seq)
    oracle_rows(q, raw, xs, n, k, dev_batched(q, raw, xs, n, k), f"{q} seq {seq}")


@pytest.mark.parametrize("q", ["Q4_K", "Q6_K", "Q8_0"])
def test_batched_host_entry_and_rows(frq, q):
    """The reference-shaped host entry (_C.matmul_<q>_batched) returns the
    device path's values; a batch of one is the single-row matvec."""
    n, k = 700, 2048
    raw = synth.make_blocks(q, n, k, seed=9)
    xs = synth.make_x(k, seed=10, batch=8)
    y = getattr(_C, f"matmul_{q.lower()}_batched")(xs, raw, n, k)
    assert bits_equal(y, dev_batched(q, raw, xs, n, k))
    oracle_rows(q, raw, xs, n, k, y, f"{q} host batched")
    y1 = getattr(_C, f"matmul_{q.lower()}_batched")(xs[:1], raw, n, k)
    assert bits_equal(y1[0], getattr(_C, f"matmul_{q.lower()}")(xs[0], raw, n, k))


def _zero_col_q4k(raw, n, k, col):
    nb = k // 256
    r = raw.reshape(n, nb * 144).copy()
    b, e = divmod(col, 256)
    sb, (p, i) = e // 32, divmod(e, 64)
    off = b * 144
    r[:, off + 16 + 32 * p + (i % 32)] &= 0xF0 if i < 32 else 0x0F
    if sb < 4:
        r[:, off + 8 + sb] &= 0xC0
    else:
        r[:, off + 8 + sb] &= 0x0F
        r[:, off + 4 + sb] &= 0x3F
    out = r.reshape(-1)
    assert np.all(G.dequant_q4_k(out, (n, k))[:, col] == 0)
    return out


def test_batched_outliers_and_massive_activations(frq):
    """x pieces carry every fp32 bit: an outlier of 2^24 on an exactly-zero
    weight column leaves the other elements their precision, and LLM-style
    massive activations (1e3 .. 1e4) among N(0, 1) stay within 1e-5."""
    n, k, seq = 512, 4096, 6
    raw = _zero_col_q4k(synth.make_blocks("Q4_K", n, k, seed=40), n, k, 0)
    xs = synth.make_x(k, seed=41, batch=seq)
    xs[0, 0] = 2.0**24
    xs[1, 0] = -(2.0**20)
    rng = np.random.default_rng(42)
    for r in (2, 3):
        idx = rng.choice(k, 10, replace=False)
        xs[r, idx] = (rng.uniform(1e3, 1e4, 10) * rng.choice([-1, 1], 10)).astype(np.float32)
    xs[4] *= np.float32(1e-20)
    xs[5, ::7] = 0.0
    oracle_rows("Q4_K", raw, xs, n, k, dev_batched("Q4_K", raw, xs, n, k), "outliers")


@pytest.mark.parametrize("q,n,k,seq", [("Q4_K", 300, 8192, 4), ("Q6_K", 200, 4096, 8), ("Q8_0", 256, 2048, 3)])
def test_batched_strided_group_output(frq, q, n, k, seq):
    """The grouped call with batch > 1 runs each matrix's rows of x through
    the batched kernel into the concatenated layout: the same bits as the
    matrix alone."""
    raws = [synth.make_blocks(q, n, k, seed=60 + i) for i in range(2)]
    xs = synth.make_x(k, seed=62, batch=seq)
    ws = [device.DeviceBuffer.from_host(r) for r in raws]
    xd = device.DeviceBuffer.from_host(xs)
    yd = device.DeviceBuffer(4 * seq * 2 * n)
    try:
        device.gemv_group([(q, ws[0], n, yd.ptr, raws[0].nbytes), (q, ws[1], n, yd.ptr + 4 * n, raws[1].nbytes)],
                          xd, k, batch=seq, y_stride=2 * n)
        device.synchronize()
        y = yd.to_host(np.float32).reshape(seq, 2 * n)
        for i in range(2):
            assert bits_equal(y[:, i * n:(i + 1) * n], dev_batched(q, raws[i], xs, n, k)), i
    finally:
        for b in ws + [xd, yd]:
            b.free()


def test_batched_noalloc_equals_dev_gemv(frq):
    """frq_dev_gemv_noalloc takes the same batched kernel (its partials in the
    fixed scratch): the same bits."""
    q, n, k, seq = "Q4_K", 3584, 18944, 4
    raw = synth.make_blocks(q, n, k, seed=70)
    xs = synth.make_x(k, seed=71, batch=seq)
    want = dev_batched(q, raw, xs, n, k)
    w, xd, yd = device.DeviceBuffer.from_host(raw), device.DeviceBuffer.from_host(xs), device.DeviceBuffer(4 * n * seq)
    try:
        _lib.check(_lib.lib().frq_dev_gemv_noalloc(device.qtype_id(q), w.ptr, raw.nbytes, xd.ptr, yd.ptr, n, k, seq, 0))
        device.synchronize()
        assert bits_equal(yd.to_host(np.float32).reshape(seq, n), want)
    finally:
        w.free()
        xd.free()
        yd.free()


def test_batched_noalloc_fewer_splits(frq):
    """A batched shape whose split-K partials exceed the fixed 3 MiB (16 rows
    x 14336 x 8 splits = 7.3 MB): the no-allocation entry point splits k
    fewer ways instead of refusing, within the same bound."""
    q, n, k, seq = "Q4_K", 14336, 4096, 16
    raw = synth.make_blocks(q, n, k, seed=72)
    xs = synth.make_x(k, seed=73, batch=seq)
    w, xd, yd = device.DeviceBuffer.from_host(raw), device.DeviceBuffer.from_host(xs), device.DeviceBuffer(4 * n * seq)
    try:
        _lib.check(_lib.lib().frq_dev_gemv_noalloc(device.qtype_id(q), w.ptr, raw.nbytes, xd.ptr, yd.ptr, n, k, seq, 0))
        device.synchronize()
        oracle_rows(q, raw, xs, n, k, yd.to_host(np.float32).reshape(seq, n), "noalloc batched")
    finally:
        w.free()
        xd.free()
        yd.free()


@pytest.mark.parametrize("n,k,seq", [(3584, 18944, 2), (3584, 18944, 3), (3584, 18944, 6), (3584, 18944, 7),
                                     (18944, 3584, 3), (4096, 4096, 2), (1536, 8960, 5)])
def test_batched_q4k_few_rows(frq, n, k, seq):
    """Two, three, and (where k > 8192) five or six rows of x on a Q4_K
    matrix run the small-M element-wise kernel in launches of two or three
    rows: each row has the bits it gets in a batch of two (a row's result
    does not depend on its batch); from seven rows on, the GEMM. Either way
    within the matvec bound, with an outlier of 2^24 in the last row. (Four
    rows, and five to eight at k <= 8192, take the fp32 matrix-core kernel:
    test_gpu_gemv_mb.py.)"""
    raw = synth.make_blocks("Q4_K", n, k, seed=n + seq)
    xs = synth.make_x(k, seed=seq + 80, batch=seq)
    xs[seq - 1, 5] = 2.0**24
    y = dev_batched("Q4_K", raw, xs, n, k)
    if seq <= 6:
        for r in range(seq):
            pair = np.stack([xs[r], xs[(r + 1) % seq]])
            assert bits_equal(y[r], dev_batched("Q4_K", raw, pair, n, k)[0]), r
    oracle_rows("Q4_K", raw, xs, n, k, y, f"Q4_K {n}x{k} rows {seq}")


_F32_MAX = float(np.finfo(np.float32).max)


def _extreme_batch(k, seq, seed, W):
    """x rows of every class the three bf16 pieces cannot carry unscaled,
    plus ordinary rows, repeated to `seq` rows. Returns (xs, class names).
    The largest row is scaled from W so that every sum_j |w_ij x_j| stays
    below FLT_MAX / 8: its exact results are finite, and no fp32 summation
    order overflows."""
    rng = np.random.default_rng(seed)

    def large(v):
        top = float(np.max(np.abs(W) @ np.abs(v)))
        return v * 2.0 ** np.floor(np.log2(_F32_MAX / (8.0 * top)))
    sign = lambda: rng.choice(np.array([-1.0, 1.0]), k)  # noqa: E731
    classes = {
        "normal": lambda: rng.standard_normal(k),
        "x 2^-120": lambda: rng.standard_normal(k) * 2.0**-120,          # normal fp32, pieces below bf16's range
        "x 2^-140": lambda: rng.standard_normal(k) * 2.0**-140,          # subnormal fp32
        "subnormal": lambda: sign() * rng.integers(1, 1 << 23, k) * 2.0**-149,
        "x 2^110": lambda: rng.standard_normal(k) * 2.0**110,
        "large (sums near FLT_MAX / 8)": lambda: large(rng.standard_normal(k)),
        "tiny among normal": lambda: np.where(rng.random(k) < 0.05, sign() * 2.0**-125, rng.standard_normal(k)),
        "zeros": lambda: np.zeros(k),
        "inf": lambda: (lambda v: (v.__setitem__(rng.integers(0, k, 3), [np.inf, np.inf, -np.inf]), v)[1])(
            rng.standard_normal(k)),
        "+inf only": lambda: (lambda v: (v.__setitem__(rng.integers(0, k, 2), np.inf), v)[1])(rng.standard_normal(k)),
        "nan": lambda: (lambda v: (v.__setitem__(int(rng.integers(0, k)), np.nan), v)[1])(rng.standard_normal(k)),
    }
    names = list(classes)
    xs = np.empty((seq, k), np.float32)
    tags = []
    for r in range(seq):
        nm = names[r % len(names)]
        xs[r] = classes[nm]().astype(np.float32)
        tags.append(nm)
    return xs, tags


def _check_extreme_row(y, W, x, what):
    """fp32 result of W x against the exact one (fp64, per weight).
    Finite x: |dy_i| <= 1e-5 sum_j |w_ij x_j| + k 2^-150 (the second term is
    what any fp32 result with at most k roundings into the subnormal range can
    add: it matters only for rows whose terms lie near 2^-149, and no fp32
    path, single-row or batched, meets 1e-5 componentwise there). Non-finite
    x: the IEEE result of the per-weight sum, bit for bit in class (NaN, +inf,
    -inf)."""
    x64 = x.astype(np.float64)
    if np.all(np.isfinite(x64)):
        y64 = W @ x64
        a64 = np.abs(W) @ np.abs(x64)
        tol = 1e-5 * a64 + W.shape[1] * 2.0**-150
        over = np.abs(y64) > _F32_MAX
        assert np.all(np.isinf(y[over]) & (np.sign(y[over]) == np.sign(y64[over]))), what
        ok = ~over
        err = np.abs(y[ok].astype(np.float64) - y64[ok])
        assert np.all(err <= tol[ok]), f"{what}: worst {np.max(err / tol[ok]):.3g} x the bound"
        return
    # per weight: NaN from any NaN x, any 0 * inf, or opposite infinities; else the infinity's sign
    bad = ~np.isfinite(x64)
    Wb, xb = W[:, bad], x64[bad]
    with np.errstate(invalid="ignore"):
        prods = Wb * xb[None, :]
    want_nan = np.any(np.isnan(prods), axis=1) | (np.any(prods == np.inf, axis=1) & np.any(prods == -np.inf, axis=1))
    want = np.where(want_nan, np.nan, np.where(np.any(prods == np.inf, axis=1), np.inf, -np.inf))
    assert np.array_equal(np.isnan(y), np.isnan(want)), f"{what}: NaN pattern"
    fin = ~np.isnan(want)
    assert np.array_equal(y[fin], want[fin]), f"{what}: infinities"


@pytest.mark.parametrize("q,n,k", [("Q4_K", 512, 4096), ("Q6_K", 256, 4096), ("Q8_0", 384, 2048)])
@pytest.mark.parametrize("seq", [4, 32, 512])
def test_batched_extreme_x_rows(frq, q, n, k, seq):
    """Rows of x at 2^-120, 2^-140 (subnormal), all-subnormal, 2^110, as large
    as the row's sums allow (~2^120 here), tiny values among normal ones,
    zeros, +-inf and NaN, through the
    small-M matvec (seq 4) and the fp32-contract GEMM (32, 512 rows, K-split
    and not). Every row meets the contract of _check_extreme_row; the same
    rows computed one at a time (batch 1) give the same non-finite classes;
    an ordinary row's bits do not depend on the rows beside it."""
    raw = synth.make_blocks(q, n, k, seed=7 * n + seq)
    W = G.DEQUANT[q](raw, (n, k), np.float32).astype(np.float64)
    xs, tags = _extreme_batch(k, seq, seed=seq + k, W=W)
    y = dev_batched(q, raw, xs, n, k)
    for r in range(seq):
        _check_extreme_row(y[r], W, xs[r], f"{q} {n}x{k} seq {seq} row {r} ({tags[r]})")
    # batch 1, one row per class
    seen = set()
    for r in range(seq):
        if tags[r] in seen:
            continue
        seen.add(tags[r])
        y1 = dev_batched(q, raw, xs[r:r + 1], n, k)[0]
        _check_extreme_row(y1, W, xs[r], f"{q} batch 1 ({tags[r]})")
        assert np.array_equal(np.isnan(y1), np.isnan(y[r])), tags[r]
        assert np.array_equal(np.isinf(y1), np.isinf(y[r])), tags[r]
    # ordinary rows: the same bits with every other row ordinary too
    calm = xs.copy()
    normal = [r for r in range(seq) if tags[r] == "normal"]
    rng = np.random.default_rng(3)
    for r in range(seq):
        if tags[r] != "normal":
            calm[r] = rng.standard_normal(k).astype(np.float32)
    yc = dev_batched(q, raw, calm, n, k)
    assert bits_equal(y[normal], yc[normal])
