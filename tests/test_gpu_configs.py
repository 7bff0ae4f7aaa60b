"""Every benchmark workload at its full size, through the same device path the
benchmark times (weights resident in HBM, default launch plan), against the
fp64 oracle (1e-5 normwise and componentwise, fp32 accumulation).

The Q6_K lm_head (152064 x 3584, 447 MB of blocks) would need a 4 GB fp64
dequant for a whole-matrix oracle; its rows are independent, so the oracle
is evaluated on a sample of rows (first, last, every row of three ragged
workgroup boundaries and 2000 random rows) cut from the same blocks.
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import assert_matvec_close, bits_equal
from flatrun_amd import NativeBackend, _lib, device, synth
from oracle import gguf_np as G

pytestmark = pytest.mark.gpu

CONFIGS = [("Q8_0", 4864, 896), ("Q4_K", 18944, 3584), ("Q4_K", 3584, 18944), ("Q1_0", 4096, 4096)]


def device_gemv(q, raw, x, n, k):
    w = device.DeviceBuffer.from_host(raw)
    xd = device.DeviceBuffer.from_host(x)
    yd = device.DeviceBuffer(4 * n)
    try:
        device.gemv(q, w, xd, yd, n, k)
        device.synchronize()
        return yd.to_host(np.float32)
    finally:
        w.free()
        xd.free()
        yd.free()


@pytest.mark.parametrize("q,n,k", CONFIGS)
def test_full_size_config(frq, q, n, k):
    raw = synth.make_blocks(q, n, k, seed=n ^ k)
    x = synth.make_x(k, seed=k + 7)
    y = device_gemv(q, raw, x, n, k)
    assert_matvec_close(y, G.matmul_f64(q, x, raw, n, k), G.abs_matmul_f64(q, x, raw, n, k),
                        what=f"{q} {n}x{k} full size")
    assert bits_equal(device_gemv(q, raw, x, n, k), y)          # launch after launch, same bits


def test_q6_k_lm_head_sampled_rows(frq):
    q, n, k = "Q6_K", 152064, 3584
    raw = synth.make_blocks(q, n, k, seed=5)
    x = synth.make_x(k, seed=6)
    y = device_gemv(q, raw, x, n, k)
    assert np.all(np.isfinite(y))
    row_bytes = synth.nbytes(q, 1, k)
    rng = np.random.default_rng(7)
    rows = np.unique(np.concatenate([[0, 1, n - 2, n - 1], np.arange(9500, 9510), np.arange(76030, 76040),
                                     rng.choice(n, 2000, replace=False)]))
    sub = raw.reshape(n, row_bytes)[rows].reshape(-1)
    m = len(rows)
    assert_matvec_close(y[rows], G.matmul_f64(q, x, sub, m, k), G.abs_matmul_f64(q, x, sub, m, k),
                        what="Q6_K lm_head sampled rows")


def test_llama_layer_grouped_full_size(frq):
    """One Llama-3-8B decoder layer (Q4_K_M mix) the way the fused decode step
    runs it: q|k|v and gate|up as grouped launches, o and down alone."""
    layer = [("q", "Q4_K", 4096, 4096), ("k", "Q4_K", 1024, 4096), ("v", "Q6_K", 1024, 4096),
             ("o", "Q4_K", 4096, 4096), ("gate", "Q4_K", 14336, 4096), ("up", "Q4_K", 14336, 4096),
             ("down", "Q6_K", 4096, 14336)]
    raws = {name: synth.make_blocks(q, n, k, seed=60 + i) for i, (name, q, n, k) in enumerate(layer)}
    spec = {name: (q, n, k) for name, q, n, k in layer}
    nb = NativeBackend()
    dev = {name: nb.upload(r) for name, r in raws.items()}
    x4 = synth.make_x(4096, seed=70)
    x14 = synth.make_x(14336, seed=71)
    for names in (("q", "k", "v"), ("gate", "up")):
        got = nb.matmul_fused(x4, [(spec[m][0], dev[m], spec[m][1]) for m in names], 4096)
        off = 0
        for m in names:
            q, n, k = spec[m]
            assert_matvec_close(got[off:off + n], G.matmul_f64(q, x4, raws[m], n, k),
                                G.abs_matmul_f64(q, x4, raws[m], n, k), what=f"layer {m}")
            off += n
    for m, x in (("o", x4), ("down", x14)):
        q, n, k = spec[m]
        got = nb.matmul_q6k(x, dev[m], n, k) if q == "Q6_K" else nb.matmul_q4k(x, dev[m], n, k)
        assert_matvec_close(got, G.matmul_f64(q, x, raws[m], n, k), G.abs_matmul_f64(q, x, raws[m], n, k),
                            what=f"layer {m}")


@pytest.mark.parametrize("q,n,k", [("Q8_0", 4864, 896), ("Q4_K", 18944, 3584), ("Q1_0", 4096, 4096),
                                   ("Q5_K", 18944, 3584), ("Q6_K", 152064, 3584)])
def test_full_size_dequant_word_for_word(frq, q, n, k):
    """Dequant at a benchmark config's full size (the lm_head: 545M outputs,
    2.2 GB of fp32), bit for bit and in place: every chunk of rows is copied
    back and compared word for word with the oracle's decode of the same
    rows, so a wrong element order fails as surely as a wrong value. The
    device-side XOR fold of all output words (the streaming read kernel)
    must also equal the oracle's."""
    raw = synth.make_blocks(q, n, k, seed=n + 3 * k)
    row_bytes = synth.nbytes(q, 1, k)
    w = device.DeviceBuffer.from_host(raw)
    y = device.DeviceBuffer(4 * n * k)
    out = device.DeviceBuffer(4 * device.READ_XOR_WORDS)
    decode = getattr(G, "dequant_" + q.lower())
    try:
        device.dequant(q, w, y, n * k)
        device.read_xor(y, 4 * n * k, out)
        device.synchronize()
        gpu_fold = int(np.bitwise_xor.reduce(out.to_host(np.uint32)))
        rows = max(1, (1 << 24) // k)
        host_fold = 0
        got = np.empty(rows * k, np.uint32)
        for r0 in range(0, n, rows):
            r1 = min(n, r0 + rows)
            ref = decode(raw[r0 * row_bytes:r1 * row_bytes], (r1 - r0) * k).view(np.uint32)
            host_fold ^= int(np.bitwise_xor.reduce(ref))
            part = got[:(r1 - r0) * k]
            _lib.check(_lib.lib().frq_memcpy_d2h(part.ctypes.data, y.ptr + 4 * r0 * k, part.nbytes))
            if not np.array_equal(part, ref):
                bad = int(np.flatnonzero(part != ref)[0])
                raise AssertionError(f"{q} {n}x{k}: first differing element at row {r0 + bad // k}, "
                                     f"column {bad % k}: {part[bad]:#010x} != {ref[bad]:#010x}")
        assert gpu_fold == host_fold, (q, n, k, hex(gpu_fold), hex(host_fold))
    finally:
        w.free()
        y.free()
        out.free()
