"""Layers of a GGUF file streamed to the GPU through the reference scheduler's
prefetch hook (flatrun_amd.streaming.SchedulerStream).

The scheduler here restates the call order of the reference's
``LayerScheduler`` (runtime/scheduler.py:222-262): for each layer, the
prefetch hook with the layer's descriptor, then the layer's handles, then the
forwarder's compute on them. Handles return what ``MmapTensorHandle.view``
returns (core/tensor.py:240-247): an array over ``mmap[a:b]``, a fresh copy
of the bytes per call. The forwarder stand-in multiplies x by every
quantized projection through ``NativeBackend.matmul_*``, as the reference's
forwarder does (model/qwen2.py:709, runtime/backend.py:270-277). Outputs must
equal, bit for bit, those of a backend without the stream (the host path),
for sequential decode steps (the plan wraps from the last layer to the
first), repeated layers and jumps (``step`` with any index); one layer is
checked against the fp64 oracle.
"""

from __future__ import annotations

import mmap
from dataclasses import dataclass

import numpy as np
import pytest

from conftest import assert_matvec_close, bits_equal
from flatrun_amd import NativeBackend, gguf, synth
from flatrun_amd.streaming import SchedulerStream
from oracle import gguf_np as G

pytestmark = pytest.mark.gpu

PROJ = [("attn_q", "Q4_K", 512, 1024), ("attn_k", "Q4_K", 128, 1024), ("attn_v", "Q6_K", 128, 1024),
        ("attn_output", "Q4_K", 1024, 512), ("ffn_gate", "Q4_K", 1536, 1024), ("ffn_up", "Q8_0", 1536, 1024),
        ("ffn_down", "Q6_K", 1024, 1536)]
N_LAYERS = 6


@dataclass
class Layer:                      # utils/types.py:124-138
    index: int
    tensor_names: tuple


class Handle:
    def __init__(self, mm, info):
        self._mm, self._info = mm, info

    def as_numpy(self):
        a = np.ndarray(shape=(self._info.nbytes,), dtype=np.uint8,
                       buffer=self._mm[self._info.offset:self._info.offset + self._info.nbytes])
        a.flags.writeable = False
        return a


class Scheduler:
    def __init__(self, layers, files):
        self._layers, self._files, self._hook = layers, files, None

    def set_prefetch_hook(self, hook):
        self._hook = hook

    def layer_count(self):
        return len(self._layers)

    def layer(self, i):
        return self._layers[i]

    def step(self, i, compute):
        layer = self._layers[i]
        if self._hook is not None:
            try:
                self._hook(layer)
            except Exception:
                pass                                  # prefetch failures never abort (scheduler.py:270-277)
        return compute(layer, {n: self._files(n) for n in layer.tensor_names})

    def run(self, compute):
        return [self.step(i, compute) for i in range(len(self._layers))]


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    path = tmp_path_factory.mktemp("sched") / "tiny_llama.gguf"
    tensors, host = [], {}
    for L in range(N_LAYERS):
        tensors.append((f"blk.{L}.attn_norm.weight", (1024,), "F32",
                        np.random.default_rng(L).standard_normal(1024).astype(np.float32).tobytes()))
        for i, (p, q, n, k) in enumerate(PROJ):
            raw = synth.make_blocks(q, n, k, seed=100 * L + i)
            host[(L, p)] = raw
            tensors.append((f"blk.{L}.{p}.weight", (n, k), q, raw.tobytes()))
    gguf.write_gguf(path, tensors, {"general.architecture": "llama", "llama.block_count": N_LAYERS})
    f = gguf.GGUFFile(path)
    fh = open(path, "rb")
    mm = mmap.mmap(fh.fileno(), 0, access=mmap.ACCESS_READ)
    names = {L: tuple(gguf.translate_gguf_name(f"blk.{L}.{p}.weight") for p in ["attn_norm"] + [x[0] for x in PROJ])
             for L in range(N_LAYERS)}
    layers = [Layer(L, names[L]) for L in range(N_LAYERS)]
    meta = {gguf.translate_gguf_name(f"blk.{L}.{p}.weight"): (L, p, q, n, k)
            for L in range(N_LAYERS) for p, q, n, k in PROJ}
    yield {"path": path, "file": f, "mm": mm, "layers": layers, "meta": meta, "host": host}
    mm.close()
    fh.close()
    f.close()


def _forwarder(backend, model, x):
    meth = {"Q4_K": backend.matmul_q4k, "Q6_K": backend.matmul_q6_k, "Q8_0": backend.matmul_q8_0}

    def compute(layer, handles):
        out = {}
        for name in layer.tensor_names:
            if name not in model["meta"]:
                continue                               # the norm: not a matmul
            L, p, q, n, k = model["meta"][name]
            out[p] = meth[q](x[:k], handles[name].as_numpy(), n, k)
        return layer.index, out
    return compute


def _handles(model):
    return lambda name: Handle(model["mm"], model["file"].info(name))


@pytest.mark.parametrize("depth", [1, 2, 3])
def test_scheduler_stream_equals_host_path(frq, model, depth):
    x = synth.make_x(1536, seed=3)
    plain = NativeBackend(weight_cache=False)
    sched_ref = Scheduler(model["layers"], _handles(model))
    want = dict(sched_ref.run(_forwarder(plain, model, x)))

    backend = NativeBackend(weight_cache=False)
    sched = Scheduler(model["layers"], _handles(model))
    st = SchedulerStream.bind(sched, model["path"], backend=backend, depth=depth, staging_bytes=1 << 16)
    try:
        assert st.depth == depth and st.slot_bytes >= sum(synth.nbytes(q, n, k) for _, q, n, k in PROJ)
        for rep in range(2):                           # two decode steps: the plan wraps around
            got = dict(sched.run(_forwarder(backend, model, x)))
            for L in range(N_LAYERS):
                for p, *_ in PROJ:
                    assert bits_equal(got[L][p], want[L][p]), (rep, L, p)
        assert st.error is None
        assert st.stats["hits"] == 2 * N_LAYERS * len(PROJ) and st.stats["misses"] == 0
        assert st.stats["restarts"] == 0
        # step() in any order: repeats and jumps plan again and stay exact
        compute = _forwarder(backend, model, x)
        for i in (3, 3, 1, 5, 0, 4, 2, 2, 5):
            L, out = sched.step(i, compute)
            for p, *_ in PROJ:
                assert bits_equal(out[p], want[L][p]), (i, p)
        assert st.stats["restarts"] >= 4 and st.stats["misses"] == 0
    finally:
        backend.attach_stream(None)
        st.close()


def test_scheduler_stream_oracle_and_foreign_weights(frq, model):
    """Layer 2 against the fp64 oracle; a weight that is not a tensor of the
    current layer (another layer's, or bytes from elsewhere) misses the
    stream and takes the host path."""
    x = synth.make_x(1536, seed=4)
    backend = NativeBackend(weight_cache=False)
    sched = Scheduler(model["layers"], _handles(model))
    st = SchedulerStream.bind(sched, model["file"], backend=backend, depth=2)
    try:
        L, out = sched.step(2, _forwarder(backend, model, x))
        for p, q, n, k in PROJ:
            raw = model["host"][(2, p)]
            assert_matvec_close(out[p], G.matmul_f64(q, x[:k], raw, n, k), G.abs_matmul_f64(q, x[:k], raw, n, k),
                                what=f"layer 2 {p}")
        misses = st.stats["misses"]
        other = model["host"][(4, "attn_q")]                # layer 4's bytes while layer 2 is current
        y = backend.matmul_q4k(x[:1024], other, 512, 1024)
        assert st.stats["misses"] == misses + 1
        assert bits_equal(y, NativeBackend(weight_cache=False).matmul_q4k(x[:1024], other, 512, 1024))
    finally:
        backend.attach_stream(None)
        st.close()
