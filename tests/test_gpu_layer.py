"""DecoderProjections (flatrun_amd.layer): a decoder block's projection chain
with every activation on the device, at the Llama-3-8B shapes (the Q4_K_M
projection mix), and the SiLU·mul kernel (frq_dev_silu_mul).

Each stage is checked against the oracle on the stage's own device input
(downloaded): q|k|v, o, gate|up and down within the matvec contract (1e-5 of
fp64, normwise and componentwise); SiLU·mul against fp64 SiLU(g)·u (8 ulp of
the result: five fp32 roundings after an exp within 1-2 ulp) and against the
forwarder's own fp32 NumPy chain (model/qwen2.py:1703-1740) within 4 ulp.
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import assert_matvec_close
from flatrun_amd import _lib, device, synth
from flatrun_amd.layer import DecoderProjections
from oracle import gguf_np as G

pytestmark = pytest.mark.gpu

LLAMA = {"q": ("Q4_K", 4096, 4096), "k": ("Q4_K", 1024, 4096), "v": ("Q6_K", 1024, 4096),
         "o": ("Q4_K", 4096, 4096), "gate": ("Q4_K", 14336, 4096), "up": ("Q4_K", 14336, 4096),
         "down": ("Q6_K", 4096, 14336)}


def numpy_silu_mul(g, u):
    """The forwarder's chain, fp32 in place (qwen2.py:1725-1740)."""
    g = g.astype(np.float32)
    e = np.empty_like(g)
    with np.errstate(over="ignore", invalid="ignore"):
        np.exp(-g, out=e)
        e += np.float32(1.0)
        np.reciprocal(e, out=e)
        np.multiply(e, g, out=e)
        np.multiply(e, u.astype(np.float32), out=e)
    return e


def exact_silu_mul(g, u):
    g64, u64 = g.astype(np.float64), u.astype(np.float64)
    with np.errstate(over="ignore"):
        return g64 / (1.0 + np.exp(-g64)) * u64


def ulps(a, b):
    """|a - b| in units of the last place of b (fp32), elementwise."""
    b32 = b.astype(np.float32)
    sp = np.abs(np.spacing(b32)).astype(np.float64)
    return np.abs(a.astype(np.float64) - b.astype(np.float64)) / sp


def check_silu(act, g, u):
    ex = exact_silu_mul(g, u)
    tiny = np.abs(ex) < 1e-30          # exp(-g) past the fp32 range: 0 * g, as in NumPy
    assert np.all(np.abs(act[tiny]) <= 1e-30)
    big = ~tiny
    assert np.max(ulps(act[big], ex[big]), initial=0) <= 8, "silu_mul vs fp64"
    ref32 = numpy_silu_mul(g, u)
    assert np.max(ulps(act[big], ref32[big]), initial=0) <= 4, "silu_mul vs the NumPy chain"


@pytest.fixture(scope="module")
def llama_layer(frq):
    host = {name: synth.make_blocks(q, n, k, seed=500 + i) for i, (name, (q, n, k)) in enumerate(LLAMA.items())}
    dev = {name: device.DeviceBuffer.from_host(raw) for name, raw in host.items()}
    yield host, dev
    for b in dev.values():
        b.free()


@pytest.mark.parametrize("seq", [1, 4])
def test_decoder_chain_against_oracle(llama_layer, seq):
    host, dev = llama_layer
    weights = {name: (q, dev[name], n, k, host[name].nbytes) for name, (q, n, k) in LLAMA.items()}
    s = device.Stream()
    x_host = synth.make_x(4096, seed=7, batch=seq if seq > 1 else None).reshape(seq, 4096)
    x = device.DeviceBuffer.from_host(x_host)
    attn = device.DeviceBuffer(4 * seq * 4096)
    dp = DecoderProjections(weights, max_seq=8, stream=s)
    try:
        def attention(qkv, n_rows):      # stand-in: the q part of each row
            for r in range(n_rows):
                device.copy(attn.ptr + 4 * 4096 * r, qkv.ptr + 4 * dp.qkv_n * r, 4 * 4096, stream=s)
            return attn

        out = dp.forward(x, seq, attention=attention, post_attention=lambda o_out, n_rows: o_out)
        s.synchronize()
        qkv = dp.qkv.to_host(np.float32)[: seq * dp.qkv_n].reshape(seq, dp.qkv_n)
        o_out = dp.o_out.to_host(np.float32)[: seq * 4096].reshape(seq, 4096)
        gateup = dp.gateup.to_host(np.float32)[: seq * 2 * 14336].reshape(seq, 2 * 14336)
        act = dp.act.to_host(np.float32)[: seq * 14336].reshape(seq, 14336)
        mlp = out.to_host(np.float32)[: seq * 4096].reshape(seq, 4096)

        def close(name, xin, got):
            q, n, k = LLAMA[name]
            y64 = G.matmul_f64(q, xin, host[name], n, k)
            a64 = G.abs_matmul_f64(q, xin, host[name], n, k)
            for r in range(seq):
                assert_matvec_close(got[r], y64[r], a64[r], what=f"{name} row {r}")

        close("q", x_host, qkv[:, :4096])
        close("k", x_host, qkv[:, 4096:5120])
        close("v", x_host, qkv[:, 5120:6144])
        close("o", qkv[:, :4096].copy(), o_out)
        close("gate", o_out, gateup[:, :14336])
        close("up", o_out, gateup[:, 14336:])
        check_silu(act, gateup[:, :14336], gateup[:, 14336:])
        close("down", act, mlp)
    finally:
        dp.close()
        x.free()
        attn.free()
        s.destroy()


def test_silu_mul_special_values_and_strides(frq):
    """Special g (zeros, tiny, the exp overflow edge, infinities, NaN) and
    strided rows (ld_in > 2 inter, ld_out > inter): the padding is left
    untouched."""
    inter, rows, ld_in, ld_out = 37, 3, 2 * 37 + 5, 37 + 3
    g_special = np.array([0.0, -0.0, 1e-30, -1e-30, 1.0, -1.0, 20.0, -20.0, 88.0, -88.0, 89.0, -89.0, 100.0, -100.0,
                          1e30, -1e30, np.inf, -np.inf, np.nan], np.float32)
    rng = np.random.default_rng(3)
    g = rng.standard_normal((rows, inter)).astype(np.float32) * 8
    g[0, : g_special.size] = g_special
    u = rng.standard_normal((rows, inter)).astype(np.float32)
    u[1, :5] = [0.0, np.inf, -1e30, 1e-30, 3.0]
    buf = np.full((rows, ld_in), 7.0, np.float32)
    buf[:, :inter], buf[:, inter:2 * inter] = g, u
    gin = device.DeviceBuffer.from_host(buf)
    out = device.DeviceBuffer.from_host(np.full((rows, ld_out), -5.0, np.float32))
    try:
        device.silu_mul(gin, out, rows, inter, ld_in=ld_in, ld_out=ld_out)
        device.synchronize()
        got = out.to_host(np.float32).reshape(rows, ld_out)
        assert np.all(got[:, inter:] == -5.0)
        act = got[:, :inter]
        ref = numpy_silu_mul(g, u)
        fin = np.isfinite(ref) & np.isfinite(g) & np.isfinite(u) & (np.abs(g) < 1e29)
        assert np.array_equal(np.isnan(act), np.isnan(ref))
        assert np.array_equal(act[~fin & ~np.isnan(ref)], ref[~fin & ~np.isnan(ref)])
        check_silu(act[fin], g[fin], u[fin])
        assert act[0, 0] == 0.0 and act[0, 12] == np.float32(100.0) * u[0, 12]   # silu(0) = 0; silu(100) = 100
        assert act[0, 13] == 0.0                      # g = -100: exp(100) overflows, 1 / inf = 0
    finally:
        gin.free()
        out.free()


def test_silu_mul_rejects(frq):
    from flatrun_amd import _lib

    b = device.DeviceBuffer(1024)
    try:
        for args in [(b.ptr, 10, b.ptr, 5, 1, 6), (b.ptr, 12, b.ptr, 5, 1, 6), (0, 12, b.ptr, 6, 1, 6),
                     (b.ptr + 2, 12, b.ptr, 6, 1, 6)]:
            assert _lib.lib().frq_dev_silu_mul(*args, None) != 0
        assert _lib.lib().frq_dev_silu_mul(b.ptr, 12, b.ptr, 6, 0, 6, None) == 0     # no rows: nothing to do
    finally:
        b.free()


def _swiglu_pair(gq, uq, inter, k, batch, seed):
    g_raw = synth.make_blocks(gq, inter, k, seed=seed)
    u_raw = synth.make_blocks(uq, inter, k, seed=seed + 1)
    xs = synth.make_x(k, seed=seed + 2, batch=batch if batch > 1 else None).reshape(batch, k)
    bufs = [device.DeviceBuffer.from_host(g_raw), device.DeviceBuffer.from_host(u_raw),
            device.DeviceBuffer.from_host(xs)]
    out = [device.DeviceBuffer(4 * batch * 2 * inter) for _ in range(2)] + \
          [device.DeviceBuffer(4 * batch * inter) for _ in range(2)]
    try:
        wg, wu, x = bufs
        gu_f, gu_r, act_f, act_r = out
        nan = np.full(batch * 2 * inter, np.nan, np.float32)
        for b in (gu_f, gu_r):
            _lib.check(_lib.lib().frq_memcpy_h2d(b.ptr, nan.ctypes.data, nan.nbytes))
        device.gemv_swiglu((gq, wg, inter, g_raw.nbytes), (uq, wu, inter, u_raw.nbytes), x, k, gu_f, act_f,
                           batch=batch)
        device.gemv_group([(gq, wg, inter, gu_r.ptr, g_raw.nbytes), (uq, wu, inter, gu_r.ptr + 4 * inter, u_raw.nbytes)],
                          x, k, batch=batch, y_stride=2 * inter)
        device.silu_mul(gu_r, act_r, batch, inter)
        device.synchronize()
        return [b.to_host(np.float32) for b in out], (g_raw, u_raw, xs)
    finally:
        for b in bufs + out:
            b.free()


@pytest.mark.parametrize("gq,uq,inter,k,batch", [
    ("Q4_K", "Q4_K", 14336, 4096, 1), ("Q4_K", "Q4_K", 1000, 4096, 1), ("Q4_K", "Q4_K", 37, 2048, 1),
    ("Q4_K", "Q4_K", 18944, 3584, 1), ("Q4_K", "Q4_K", 300, 4096, 3), ("Q6_K", "Q4_K", 512, 4096, 1),
    ("Q4_K", "Q4_K", 5, 40960, 1),
])
def test_gemv_swiglu_matches_group_and_silu(frq, gq, uq, inter, k, batch):
    """frq_dev_gemv_swiglu gives the bits of the grouped gate|up launch plus
    frq_dev_silu_mul: fused (a Q4_K pair at batch 1, k covered by one
    workgroup, ragged last workgroup) and through those two calls (batch 3,
    a Q6_K gate, k beyond one workgroup); gate and up within the matvec
    contract."""
    (gu_f, gu_r, act_f, act_r), (g_raw, u_raw, xs) = _swiglu_pair(gq, uq, inter, k, batch, seed=inter + k)
    assert np.array_equal(gu_f.view(np.uint32), gu_r.view(np.uint32))
    assert np.array_equal(act_f.view(np.uint32), act_r.view(np.uint32))
    gu = gu_f.reshape(batch, 2 * inter)
    for name, raw, cols in (("gate", g_raw, slice(0, inter)), ("up", u_raw, slice(inter, 2 * inter))):
        q = gq if name == "gate" else uq
        y64 = G.matmul_f64(q, xs, raw, inter, k)
        a64 = G.abs_matmul_f64(q, xs, raw, inter, k)
        for r in range(batch):
            assert_matvec_close(gu[r, cols], y64[r], a64[r], what=f"{name} row {r}")


def test_gemv_swiglu_rejects(frq):
    raw = synth.make_blocks("Q4_K", 8, 256, seed=1)
    w = device.DeviceBuffer.from_host(raw)
    x = device.DeviceBuffer.from_host(synth.make_x(256, seed=2))
    y = device.DeviceBuffer(4 * 16)
    try:
        with pytest.raises(ValueError):         # up of another size
            device.gemv_swiglu(("Q4_K", w, 8, raw.nbytes), ("Q4_K", w, 4, raw.nbytes), x, 256, y, y)
        with pytest.raises(RuntimeError):       # weight byte size mismatch
            device.gemv_swiglu(("Q4_K", w, 8, raw.nbytes - 1), ("Q4_K", w, 8, raw.nbytes), x, 256, y, y)
        with pytest.raises(RuntimeError):       # null act
            device.gemv_swiglu(("Q4_K", w, 8, raw.nbytes), ("Q4_K", w, 8, raw.nbytes), x, 256, y, 0)
    finally:
        w.free()
        x.free()
        y.free()


def test_gemv_swiglu_fusable(frq):
    """The one-launch condition: a Q4_K pair, 16-byte aligned, k covered by
    one workgroup (8 lanes per block, k <= 32768)."""
    raw = synth.make_blocks("Q4_K", 4, 4096, seed=3)
    w = device.DeviceBuffer.from_host(raw)
    try:
        assert device.gemv_swiglu_fusable(("Q4_K", w), ("Q4_K", w), 4096)
        assert device.gemv_swiglu_fusable(("Q4_K", w), ("Q4_K", w), 32768)
        assert not device.gemv_swiglu_fusable(("Q4_K", w), ("Q4_K", w), 32768 + 256)
        assert not device.gemv_swiglu_fusable(("Q6_K", w), ("Q4_K", w), 4096)
        assert not device.gemv_swiglu_fusable(("Q4_K", w), ("Q4_K", w.ptr + 8), 4096)
    finally:
        w.free()
