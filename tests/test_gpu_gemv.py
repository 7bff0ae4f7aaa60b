"""GPU fused dequant + matvec kernels against the oracle.

Contract: max relative error 1e-5 with fp32 accumulation, both normwise
(max|dy| / max|y|) and componentwise (|dy_i| / sum_j |w_ij x_j|), against the
fp64 oracle (exact fp32 weights, fp64 sums); and 1e-5 normwise against the
reference's NumPy matvec (dequant @ x, fp32 BLAS) and its native scalar
matvec (committed vectors / C restatement).
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import GOLDEN, MATVEC_RTOL, assert_matvec_close, assert_rel_close_to, bits_equal
from flatrun_amd import _C, device, synth
from oracle import gguf_np as G
from oracle.loader import c_oracle

pytestmark = pytest.mark.gpu

QS = ["Q8_0", "Q4_K", "Q5_K", "Q6_K", "Q1_0"]


def gpu_matmul(q, x, raw, n, k):
    t = q.lower()
    return getattr(_C, f"matmul_{t}")(x, raw, n, k) if np.ndim(x) == 1 else getattr(_C, f"matmul_{t}_batched")(x, raw, n, k)


def check(q, raw, x, n, k, y):
    y64 = G.matmul_f64(q, x, raw, n, k)
    absw = G.abs_matmul_f64(q, x, raw, n, k)
    assert_matvec_close(y, y64, absw, what=f"{q} {n}x{k} vs fp64")
    assert_rel_close_to(y, G.matmul_numpy(q, x, raw, n, k), what=f"{q} {n}x{k} vs numpy")


# k values chosen to hit every work-unit size and 1..8 waves per workgroup
SHAPES = {
    "Q4_K": [(1, 256), (5, 512), (37, 1024), (130, 3584), (64, 4096), (19, 18944), (33, 14336)],
    "Q5_K": [(1, 256), (9, 768), (70, 4096), (21, 14336)],
    "Q6_K": [(1, 256), (11, 512), (40, 3584), (64, 4096), (17, 14336), (9, 18944)],
    "Q8_0": [(1, 32), (3, 96), (48, 896), (70, 4096), (25, 14336)],
    "Q1_0": [(1, 128), (6, 384), (33, 4096), (12, 16384)],
}


@pytest.mark.parametrize("q,n,k", [(q, n, k) for q in QS for (n, k) in SHAPES[q]])
def test_gemv_shapes(frq, q, n, k):
    raw = synth.make_blocks(q, n, k, seed=n + k)
    x = synth.make_x(k, seed=k)
    check(q, raw, x, n, k, gpu_matmul(q, x, raw, n, k))


@pytest.mark.parametrize("q", QS)
def test_gemv_batched_equals_rows(frq, q):
    be = synth.BLOCK[q][1]
    n, k = 45, 8 * be
    raw = synth.make_blocks(q, n, k, seed=3)
    xs = synth.make_x(k, seed=4, batch=3)
    yb = gpu_matmul(q, xs, raw, n, k)
    assert yb.shape == (3, n)
    for s in range(3):
        assert bits_equal(yb[s], gpu_matmul(q, xs[s], raw, n, k))
    check(q, raw, xs, n, k, yb)


@pytest.mark.parametrize("q", ["Q4_K", "Q6_K", "Q8_0"])
def test_gemv_vs_reference_native_vectors(frq, q):
    z = np.load(GOLDEN / "ref_native_vectors.npz")
    t = q.lower()
    raw, (n, k) = z[f"{t}_raw"], z[f"{t}_shape"]
    assert_rel_close_to(gpu_matmul(q, z[f"{t}_x"], raw, n, k), z[f"{t}_matmul"], what="1-D vs reference native")
    assert_rel_close_to(gpu_matmul(q, z[f"{t}_x3"], raw, n, k), z[f"{t}_matmul3"], what="batched vs reference native")


@pytest.mark.parametrize("q", ["Q4_K", "Q6_K", "Q8_0"])
def test_gemv_vs_native_restatement(frq, q):
    be = synth.BLOCK[q][1]
    n, k = 200, 16 * be
    raw = synth.make_blocks(q, n, k, seed=17)
    x = synth.make_x(k, seed=18)
    assert_rel_close_to(gpu_matmul(q, x, raw, n, k), c_oracle().matmul(q, x, raw, n, k, threads=4),
                        what="vs native scalar order")


def test_gemv_edge_values(frq):
    """x with zeros, huge and tiny entries; weights with zero and negative scales."""
    n, k = 24, 1024
    raw = synth.make_blocks("Q4_K", n, k, seed=2).reshape(-1, 144)
    raw[::5, 0:2] = 0                                      # d = 0 blocks
    raw[1::7, 1] |= 0x80                                   # negative d
    raw = raw.reshape(-1)
    x = synth.make_x(k, seed=3)
    x[::13] = 0.0
    x[5] = 3.0e4
    x[7] = 1.0e-30
    check("Q4_K", raw, x, n, k, gpu_matmul("Q4_K", x, raw, n, k))


@pytest.mark.parametrize("q", QS)
def test_gemv_k_zero_and_n_zero(frq, q):
    assert np.array_equal(gpu_matmul(q, np.zeros(0, np.float32), np.zeros(0, np.uint8), 5, 0), np.zeros(5, np.float32))
    be = synth.BLOCK[q][1]
    assert gpu_matmul(q, np.ones(be, np.float32), np.zeros(0, np.uint8), 0, be).shape == (0,)


@pytest.mark.parametrize("q,n,k", [("Q4_K", 300, 18944), ("Q4_K", 600, 3584), ("Q6_K", 300, 3584), ("Q8_0", 500, 896),
                                   ("Q1_0", 300, 4096)])
def test_launch_geometry_sweep(frq, q, n, k):
    """Every supported geometry (work unit, rows per workgroup, unroll) gives a
    result within tolerance; geometries that share a work unit give identical bits."""
    raw = synth.make_blocks(q, n, k, seed=5)
    x = synth.make_x(k, seed=6)
    y64, absw = G.matmul_f64(q, x, raw, n, k), G.abs_matmul_f64(q, x, raw, n, k)
    w = device.DeviceBuffer.from_host(raw)
    xd = device.DeviceBuffer.from_host(x)
    yd = device.DeviceBuffer(n * 4)
    by_cpl = {}
    for cpl in (1, 2, 4):
        for rows in (1, 3, 7, 8, 16, 32):
            for unroll in (4, 8):
                try:
                    plan = device.gemv_tuned(q, w, xd, yd, n, k, cpl=cpl, rows_per_wg=rows, unroll=unroll)
                except RuntimeError:
                    continue                         # work unit not valid for this format / k
                device.synchronize()
                y = yd.to_host(np.float32)
                assert_matvec_close(y, y64, absw, what=f"{plan}")
                if plan["cpl"] in by_cpl:
                    assert bits_equal(y, by_cpl[plan["cpl"]]), plan
                else:
                    by_cpl[plan["cpl"]] = y
    assert by_cpl


def test_resident_weights_match_host_path(backend):
    n, k = 333, 3584
    raw = synth.make_blocks("Q4_K", n, k, seed=8)
    x = synth.make_x(k, seed=9)
    w = backend.upload(raw)
    assert bits_equal(backend.matmul_q4k(x, w, n, k), backend.matmul_q4k(x, raw, n, k))
    xs = synth.make_x(k, seed=10, batch=4)
    assert bits_equal(backend.matmul_q4k(xs, w, n, k), backend.matmul_q4k(xs, raw, n, k))
