"""Prefill GEMM on the matrix cores (bf16 MFMA), Q4_K / Q6_K / Q8_0 weights,
against the oracle.

Contract (written here, checked below):
  * against fp64 X . bf16(W)^T, with W the exact fp32 dequant (oracle) rounded
    to bf16 nearest-even: within MATVEC_RTOL (1e-5) normwise and
    componentwise -- the kernel adds only fp32 accumulation error;
  * against fp64 X . W^T with the exact fp32 W: normwise within
    BF16_W_RTOL = 1e-2 -- the bf16 rounding of W (2^-9 relative per weight)
    is the only intended loss.
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import assert_matvec_close, bits_equal
from flatrun_amd import NativeBackend, _C, _lib, synth
from oracle import gguf_np as G

pytestmark = pytest.mark.gpu

BF16_W_RTOL = 1e-2


def bf16_round(a: np.ndarray) -> np.ndarray:
    """float32 -> nearest-even bf16 -> float32 (numpy, for the reference side)."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32)
    r = (u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) & np.uint32(0xFFFF0000)
    return r.view(np.float32)


def make_case(m, n, k, seed, q="Q4_K"):
    raw = synth.make_blocks(q, n, k, seed=seed)
    x = np.random.default_rng(seed + 1).standard_normal((m, k)).astype(np.float32)
    return raw, bf16_round(x)


def check(y, raw, xb, n, k, q="Q4_K"):
    w = G.DEQUANT[q](raw, (n, k)).astype(np.float32)
    wb = bf16_round(w).astype(np.float64)
    x64 = xb.astype(np.float64)
    ref = x64 @ wb.T
    absw = np.abs(x64) @ np.abs(wb).T
    assert_matvec_close(y.reshape(-1), ref.reshape(-1), absw.reshape(-1), what=f"{q} gemm {xb.shape[0]}x{n}x{k} vs bf16(W)")
    exact = x64 @ w.astype(np.float64).T
    err = np.max(np.abs(y - exact)) / np.max(np.abs(exact))
    assert err <= BF16_W_RTOL, f"gemm vs exact W: normwise {err:.3e} > {BF16_W_RTOL}"


@pytest.mark.parametrize("m,n,k", [(1, 1, 256), (5, 37, 512), (256, 128, 256), (300, 200, 1024), (513, 130, 768),
                                   (64, 1000, 4096)])
def test_gemm_shapes(frq, m, n, k):
    raw, xb = make_case(m, n, k, seed=m + n + k)
    y = _C.matmul_q4_k_bf16(xb, raw, n, k)
    assert y.shape == (m, n) and y.dtype == np.float32
    check(y, raw, xb, n, k)


@pytest.mark.parametrize("q", ["Q6_K", "Q8_0"])
@pytest.mark.parametrize("m,n,k", [(1, 1, 256), (5, 37, 512), (300, 200, 1024), (513, 130, 768), (64, 1000, 4096)])
def test_gemm_other_formats(frq, q, m, n, k):
    raw, xb = make_case(m, n, k, seed=m + 2 * n + k, q=q)
    y = _C.matmul_bf16(q, xb, raw, n, k)
    assert y.shape == (m, n)
    check(y, raw, xb, n, k, q=q)


def test_gemm_q8_0_k_multiple_of_128(frq):
    m, n, k = 9, 33, 128 * 3
    raw, xb = make_case(m, n, k, seed=3, q="Q8_0")
    check(_C.matmul_q8_0_bf16(xb, raw, n, k), raw, xb, n, k, q="Q8_0")
    with pytest.raises(RuntimeError):
        _C.matmul_q8_0_bf16(np.zeros((2, 320), np.float32), np.zeros(33 * 10 * 34, np.uint8), 33, 320)


def test_gemm_llama_down_q6_k(frq):
    """Llama-3-8B prefill down projection: Y[512 x 4096] = X[512 x 14336] . W^T, W Q6_K."""
    m, n, k = 512, 4096, 14336
    raw, xb = make_case(m, n, k, seed=12, q="Q6_K")
    check(_C.matmul_q6_k_bf16(xb, raw, n, k), raw, xb, n, k, q="Q6_K")


def test_gemm_resident_weight_q6_k(frq):
    m, n, k = 17, 96, 512
    raw, xb = make_case(m, n, k, seed=19, q="Q6_K")
    nb = NativeBackend()
    assert bits_equal(nb.matmul_q6k_bf16(xb, nb.upload(raw), n, k), nb.matmul_q6k_bf16(xb, raw, n, k))


def test_gemm_prefill_config(frq):
    """The prefill workload itself: Y[512 x 14336] = X[512 x 4096] . W^T."""
    m, n, k = 512, 14336, 4096
    raw, xb = make_case(m, n, k, seed=11)
    check(_C.matmul_q4_k_bf16(xb, raw, n, k), raw, xb, n, k)


def test_gemm_bf16_bits_input_and_1d(frq):
    m, n, k = 3, 70, 512
    raw, xb = make_case(m, n, k, seed=4)
    y = _C.matmul_q4_k_bf16(xb, raw, n, k)
    assert bits_equal(_C.matmul_q4_k_bf16(_C.to_bf16_bits(xb), raw, n, k), y)
    assert bits_equal(_C.matmul_q4_k_bf16(xb[1], raw, n, k), y[1])


def test_gemm_resident_weight_matches_host_path(frq):
    m, n, k = 40, 300, 1024
    raw, xb = make_case(m, n, k, seed=9)
    nb = NativeBackend()
    dw = nb.upload(raw)
    assert bits_equal(nb.matmul_q4k_bf16(xb, dw, n, k), nb.matmul_q4k_bf16(xb, raw, n, k))


def test_gemm_edges_and_errors(frq):
    assert _C.matmul_q4_k_bf16(np.zeros((0, 256), np.float32), np.zeros(144 * 3, np.uint8), 3, 256).shape == (0, 3)
    assert np.array_equal(_C.matmul_q4_k_bf16(np.zeros((2, 0), np.float32), np.zeros(0, np.uint8), 4, 0),
                          np.zeros((2, 4), np.float32))
    with pytest.raises(RuntimeError):
        _C.matmul_q4_k_bf16(np.zeros((2, 300), np.float32), np.zeros(144, np.uint8), 1, 300)
    with pytest.raises(RuntimeError):
        _C.matmul_q4_k_bf16(np.zeros((2, 256), np.float32), np.zeros(100, np.uint8), 1, 256)
    assert _lib.lib().frq_dev_gemm_q4_k_bf16(None, 144, None, None, 1, 1, 256, None) != 0


def test_gemm_split_k_deterministic_and_shared_scratch(frq):
    """Shapes with few output tiles split K (512 x 1024 x 4096: 8 splits);
    the partial planes are added in split order, so repeated calls give the
    same bits, also when other split GEMMs, graph replays and split-K GEMVs
    (which share the scratch) run in between."""
    from flatrun_amd import device

    m, n, k = 512, 1024, 4096
    raw, xb = make_case(m, n, k, seed=21)
    y0 = _C.matmul_q4_k_bf16(xb, raw, n, k)
    check(y0, raw, xb, n, k)
    raw2, xb2 = make_case(300, 200, 1024, seed=22, q="Q6_K")
    wg = synth.make_blocks("Q4_K", 8, 65536, seed=23)               # split-K GEMV (rows beyond one workgroup)
    xg = synth.make_x(65536, seed=24)
    for _ in range(3):
        assert bits_equal(_C.matmul_q4_k_bf16(xb, raw, n, k), y0)
        check(_C.matmul_bf16("Q6_K", xb2, raw2, 200, 1024), raw2, xb2, 200, 1024, q="Q6_K")
        _C.matmul_q4_k(xg, wg, 8, 65536)
    w = device.DeviceBuffer.from_host(raw)
    xd = device.DeviceBuffer.from_host(_C.to_bf16_bits(xb))
    yd = device.DeviceBuffer(m * n * 4)
    s = device.Stream()
    try:
        device.gemm_bf16("Q4_K", w, xd, yd, m, n, k, stream=s, w_bytes=raw.nbytes)
        s.synchronize()
        assert bits_equal(yd.to_host(np.float32).reshape(m, n), y0)
        with device.Graph.capture(s) as cap:
            device.gemm_bf16("Q4_K", w, xd, yd, m, n, k, stream=s, w_bytes=raw.nbytes)
        for _ in range(3):
            _lib.check(_lib.lib().frq_memcpy_h2d(yd.ptr, np.full(m * n, np.nan, np.float32).ctypes.data, m * n * 4))
            cap.launch(s)
            s.synchronize()
            assert bits_equal(yd.to_host(np.float32).reshape(m, n), y0)
        cap.destroy()
    finally:
        w.free()
        xd.free()
        yd.free()
        s.destroy()
