"""GGUF file -> HBM residency (flatrun_amd.gguf.ResidentModel) on the GPU.

Contract: every resident tensor holds exactly the file's bytes (read back
D2H), at a 256-byte aligned arena offset; matvecs through the resident
views equal the host-buffer path bit for bit (same kernels, same inputs),
and the dequant of a resident tensor equals the oracle bit for bit.
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import bits_equal
from flatrun_amd import DeviceWeight, NativeBackend, _lib, device, gguf, synth
from oracle import gguf_np as G

pytestmark = pytest.mark.gpu

MODEL = [  # (gguf name, qtype, n, k)
    ("blk.0.attn_q.weight", "Q4_K", 96, 1024),
    ("blk.0.attn_v.weight", "Q6_K", 64, 768),
    ("blk.0.ffn_down.weight", "Q8_0", 48, 896),
    ("blk.0.ffn_gate.weight", "Q5_K", 40, 512),
    ("blk.0.ffn_up.weight", "Q1_0", 33, 1152),
    ("output.weight", "Q6_K", 130, 256),
]


@pytest.fixture()
def model_file(tmp_path):
    tensors, raws = [], {}
    for i, (name, q, n, k) in enumerate(MODEL):
        raw = synth.make_blocks(q, n, k, seed=100 + i)
        raws[name] = raw
        tensors.append((name, (n, k), q, raw.tobytes()))
    norm = np.linspace(-1, 1, 1024, dtype=np.float32)
    tensors.insert(1, ("blk.0.attn_norm.weight", (1024,), "F32", norm.tobytes()))
    p = tmp_path / "m.gguf"
    gguf.write_gguf(p, tensors, {"general.architecture": "llama"})
    return p, raws, norm


def hf(name: str) -> str:
    return gguf.translate_gguf_name(name)


@pytest.mark.parametrize("staging", [1 << 12, 3 * 1000 + 8, 64 << 20])
def test_resident_bytes_match_file(frq, model_file, staging):
    """Small staging slots split tensors over many chunks (odd sizes too)."""
    p, raws, norm = model_file
    with gguf.ResidentModel(p, staging_bytes=staging) as m:
        assert set(m.names()) == {hf(n) for n, *_ in MODEL} | {hf("blk.0.attn_norm.weight")}
        for name, q, n, k in MODEL:
            w = m[hf(name)]
            assert isinstance(w, DeviceWeight) and w.qtype == q and w.shape == (n, k)
            assert w.offset % gguf.ARENA_ALIGN == 0 and w.nbytes == raws[name].nbytes
            back = np.empty(w.nbytes, np.uint8)
            _lib.check(_lib.lib().frq_memcpy_d2h(back.ctypes.data, w.data_ptr(), w.nbytes))
            assert np.array_equal(back, raws[name]), name
        wn = m[hf("blk.0.attn_norm.weight")]
        back = np.empty(1024, np.float32)
        _lib.check(_lib.lib().frq_memcpy_d2h(back.ctypes.data, wn.data_ptr(), 4096))
        assert np.array_equal(back, norm)
        assert m.nbytes == sum(r.nbytes for r in raws.values()) + 4096 and m.load_seconds > 0


def test_resident_matvec_equals_host_path(frq, model_file):
    p, raws, _ = model_file
    nb = NativeBackend()
    with nb.load_gguf(p) as m:
        for name, q, n, k in MODEL:
            x = synth.make_x(k, seed=k)
            xs = synth.make_x(k, seed=k + 1, batch=3)
            meth = getattr(nb, f"matmul_{q.lower()}") if q not in ("Q4_K",) else nb.matmul_q4k
            assert bits_equal(meth(x, m[hf(name)], n, k), meth(x, raws[name], n, k)), name
            assert bits_equal(meth(xs, m[hf(name)], n, k), meth(xs, raws[name], n, k)), name


def test_resident_dequant_equals_oracle(frq, model_file):
    p, raws, _ = model_file
    with gguf.ResidentModel(p, names=[hf(MODEL[0][0]), hf(MODEL[1][0])]) as m:
        assert len(m.names()) == 2
        for name, q, n, k in MODEL[:2]:
            y = device.DeviceBuffer(n * k * 4)
            try:
                device.dequant(q, m[hf(name)], y, n * k, w_bytes=m[hf(name)].nbytes)
                device.synchronize()
                assert bits_equal(y.to_host(np.float32).reshape(n, k), G.DEQUANT[q](raws[name], (n, k)))
            finally:
                y.free()


def test_view_bounds_and_missing(frq, model_file):
    p, _, _ = model_file
    with gguf.ResidentModel(p) as m:
        with pytest.raises(gguf.TensorNotFound):
            m["nope"]
        with pytest.raises(ValueError):
            DeviceWeight.view(m.arena, m.arena.nbytes - 4, 8)
    with pytest.raises(gguf.TensorNotFound):
        gguf.ResidentModel(p, names=["nope"])
