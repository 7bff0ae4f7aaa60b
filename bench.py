"""Benchmark of the gfx950 GGUF matvec path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-suite]

Headline workload: Q4_K GEMV, W 3584 x 18944 (out x in; the Qwen2.5-7B
ffn_down shape), batch 1, fp32 x and y. One step = one fused dequant + matvec
launch over one weight copy. The raw blocks are resident in HBM before the
timed region, and steps rotate over >= 1 GiB of distinct weight copies so no
step is served from the 256 MB Infinity Cache.

Printed: ONE JSON line with
  value      effective GB/s over the whole timed region: K launches recorded
             once as a HIP graph and replayed back-to-back on one stream,
             bracketed by device syncs and HIP events on that stream;
             effective bytes per step = raw blocks + 4k (x) + 4n (y);
  roofline   the GEMV kernel against 8 TB/s HBM: achieved = effective bytes
             per launch / mean launch duration over the same timed region;
  eager_launch_us  mean time per launch when each launch is issued from
             Python one by one (host-bound for kernels this short);
  settle     the untimed burst (>= 20 ms of back-to-back launches) run before
             the warmup and the timed region, whatever --warmup says: the
             part raises its clocks over the first milliseconds of a burst;
  read_ceiling  the same weight copies read by the library's plain streaming
             read kernel, graph-replayed the same way: the time any kernel
             that reads those bytes once per launch needs here, and the
             GEMV's time over it;
  cpu_baseline  the reference's native scalar matmul (its own _C module built
             from its sources, 1 thread) on the same bytes, timed on the host
             for a bounded number of full-shape repetitions; plus the NumPy path;
  configs    every other benchmark workload (GB/s, mean kernel us, fraction of
             HBM peak; per GEMV config also the reference's CPU paths timed on
             this host: native 1 thread, row-parallel on every core, NumPy),
             the Llama-3-8B decode-step weight sweep (ms/step,
             graph replay and eager; resident and streamed), the fp32
             batched matvec at seq 4 / 32 / 512 (the re-prefill call), the
             prefill GEMM, the copy and read ceilings, and a GGUF file -> HBM
             load.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

from flatrun_amd import _lib, device, synth  # noqa: E402

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, published
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA, published
ROTATE_BYTES = 1 << 30         # >= 1 GiB of distinct copies per workload
SETTLE_MS = 20.0               # untimed back-to-back launches before every timed GEMV region


TRAFFIC_FILE = ROOT / "profiles" / "q4_k_gemv_3584x18944.traffic.json"


GEMM_COUNTERS_FILE = ROOT / "profiles" / "q4_k_gemm_bf16_512x14336x4096.counters.json"


def measured_mfma_util() -> float | None:
    """MFMA busy percentage of the prefill GEMM, from the committed rocprofv3
    SQ_VALU_MFMA_BUSY_CYCLES / GRBM_GUI_ACTIVE summary, if present."""
    try:
        return round(float(json.loads(GEMM_COUNTERS_FILE.read_text())["derived"]["mfma_util_pct"]), 1)
    except (OSError, KeyError, ValueError):
        return None


def measured_traffic() -> int | None:
    """HBM bytes per launch of the headline kernel, from the committed
    rocprofv3 FETCH_SIZE + WRITE_SIZE summary (copy-calibrated), if present."""
    try:
        return int(json.loads(TRAFFIC_FILE.read_text())["traffic_bytes"])
    except (OSError, KeyError, ValueError):
        return None


def effective_bytes(q: str, n: int, k: int, batch: int = 1) -> int:
    return synth.nbytes(q, n, k) + 4 * k * batch + 4 * n * batch


def graph_time(stream, launch, steps: int, warmup: int) -> float:
    """Seconds for `steps` calls launch(i) (i = warmup .. warmup + steps - 1)
    after `warmup` untimed ones. Two graphs, each replayed once after a device
    synchronization and bracketed by events: A = the warmup and the timed
    launches, B = the warmup launches alone. A - B is the time of exactly the
    `steps` timed launches: the fixed start of a graph replay on the device
    (~9 us here, which a timed region opened between two graphs would hold)
    and the host's submission are in both and cancel. HIP cannot time
    events recorded inside a graph."""
    def capture(count):
        with device.Graph.capture(stream) as cap:
            for i in range(count):
                launch(i)
        return cap.graph

    ga, gb = capture(warmup + steps), capture(warmup) if warmup else None
    e0, e1 = device.Event(), device.Event()

    def run(g):
        if g is None:
            return 0.0
        device.synchronize()
        e0.record(stream)
        g.launch(stream)
        e1.record(stream)
        e1.synchronize()
        return e0.elapsed_ms(e1) / 1e3

    tb = run(gb)
    ta = run(ga)
    device.synchronize()
    ga.destroy()
    if gb is not None:
        gb.destroy()
    e0.destroy()
    e1.destroy()
    return ta - tb


class GemvWorkload:
    """Rotating device copies of one seeded weight, x and y resident in HBM."""

    def __init__(self, q: str, n: int, k: int, seed: int, stream, rotate_bytes: int = ROTATE_BYTES,
                 kernel: int | None = None, batch: int = 1):
        self.q, self.n, self.k, self.kernel, self.batch = q, n, k, kernel, batch
        self.raw = synth.make_blocks(q, n, k, seed=seed)
        self.ncopies = max(2, math.ceil(rotate_bytes / self.raw.nbytes))
        self.w = [device.DeviceBuffer.from_host(self.raw) for _ in range(self.ncopies)]
        self.x_host = synth.make_x(k, seed=seed + 1, batch=batch if batch > 1 else None)
        self.x = device.DeviceBuffer.from_host(self.x_host)
        self.y = device.DeviceBuffer(4 * n * batch)
        self.stream = stream
        self.bytes = effective_bytes(q, n, k, batch)
        self.launch(0)                     # first launch allocates any per-stream scratch, outside graph capture
        device.synchronize()

    def launch(self, i: int) -> None:
        if self.kernel is None:
            device.gemv(self.q, self.w[i % self.ncopies], self.x, self.y, self.n, self.k, batch=self.batch,
                        stream=self.stream, w_bytes=self.raw.nbytes)
        else:
            device.gemv_tuned(self.q, self.w[i % self.ncopies], self.x, self.y, self.n, self.k, kernel=self.kernel,
                              stream=self.stream, w_bytes=self.raw.nbytes)

    def result(self) -> np.ndarray:
        device.synchronize()
        return self.y.to_host(np.float32)

    def graph(self, launches: int, start: int = 0) -> "device.Graph":
        """`launches` consecutive steps recorded as one HIP graph."""
        with device.Graph.capture(self.stream) as cap:
            for i in range(launches):
                self.launch(start + i)
        return cap.graph

    def settle(self, min_ms: float = SETTLE_MS, batch: int = 200) -> dict:
        """Untimed graph replays of `batch` launches until at least `min_ms`
        have run back to back: the part raises its clocks over the first
        milliseconds of a burst, so a short timed region right after idle
        reads slow. Independent of --warmup; returns what ran."""
        g = self.graph(batch)
        e0, e1 = device.Event(), device.Event()
        launches, ms = 0, 0.0
        e0.record(self.stream)
        while ms < min_ms and launches < 200 * batch:
            g.launch(self.stream)
            launches += batch
            e1.record(self.stream)
            e1.synchronize()
            ms = e0.elapsed_ms(e1)
        g.destroy()
        return {"launches": launches, "ms": round(ms, 3)}

    def time_throughput(self, steps: int, warmup: int) -> float:
        """Seconds for `steps` launches replayed back-to-back, after a settle
        burst (settle) and `warmup` untimed launches. Warmup, start event,
        the `steps` launches and end event are one HIP graph, replayed once
        after a device synchronization: the events bracket exactly the
        `steps` launches, with neither the host's submission nor the gap
        between two graphs inside (that gap, ~9 us here, spread over a short
        timed region of separately launched graphs, read as 0.45 us more per
        launch at 20 steps)."""
        self.settled = self.settle()
        return graph_time(self.stream, self.launch, steps, max(warmup, 1))

    def time_eager(self, steps: int) -> float:
        """Seconds for `steps` launches issued one by one from Python."""
        self.launch(0)
        device.synchronize()
        e0, e1 = device.Event(), device.Event()
        e0.record(self.stream)
        for i in range(steps):
            self.launch(i)
        e1.record(self.stream)
        e1.synchronize()
        return e0.elapsed_ms(e1) / 1e3

    def free(self) -> None:
        for b in self.w:
            b.free()
        self.x.free()
        self.y.free()


def cpu_baseline(work: GemvWorkload, y_gpu: np.ndarray, seconds: float) -> dict:
    """The reference's native matmul on the host (oracle/_ref, 1 thread) or, if
    that build is absent, the C restatement; plus the C restatement with rows
    split over every host core, and the NumPy path (BLAS)."""
    from oracle import gguf_np as G
    from oracle.loader import c_oracle, ref_C

    q, n, k, raw, x = work.q, work.n, work.k, work.raw, work.x_host
    R = ref_C()
    if R is not None:
        fn = getattr(R, f"matmul_{q.lower()}")
        kind, what = "reference", f"reference _C.matmul_{q.lower()} (src/flatrun_native, scalar x86, 1 thread)"
        run = lambda: fn(x, raw, n, k)  # noqa: E731
    else:
        kind, what = "port", f"C restatement of the reference scalar matmul_{q.lower()} (1 thread)"
        run = lambda: c_oracle().matmul(q, x, raw, n, k, threads=1)  # noqa: E731
    y_ref = run()
    reps, t0 = 0, time.perf_counter()
    while True:
        run()
        reps += 1
        el = time.perf_counter() - t0
        if el >= seconds or reps >= 200:
            break
    gbs = work.bytes * reps / el / 1e9
    # the C restatement with rows split over every host core: the reference's
    # row-parallel matmul_q4_k_mt (q4_k.h:464-511) is built on NEON only
    cores = os.cpu_count() or 1
    co = c_oracle()
    y_mt = co.matmul(q, x, raw, n, k, threads=cores)
    reps_mt, t0 = 0, time.perf_counter()
    while True:
        co.matmul(q, x, raw, n, k, threads=cores)
        reps_mt += 1
        el_mt = time.perf_counter() - t0
        if el_mt >= min(seconds, 3.0) or reps_mt >= 200:
            break
    # NumPy path of the reference (dequant + BLAS matvec), all host cores
    t0 = time.perf_counter()
    y_np = G.matmul_numpy(q, x, raw, n, k)
    t_np = time.perf_counter() - t0
    err = float(np.max(np.abs(y_gpu - y_ref)) / np.max(np.abs(y_ref)))
    err_np = float(np.max(np.abs(y_gpu - y_np)) / np.max(np.abs(y_np)))
    return {
        "value": round(gbs, 4), "unit": "GB/s", "cores": 1, "kind": kind,
        "sample": f"{q} GEMV {n}x{k} b1, full shape x {reps} reps ({el:.1f} s): {what}",
        "ms_per_step": round(el / reps * 1e3, 3),
        "row_parallel": {"value": round(work.bytes * reps_mt / el_mt / 1e9, 4), "unit": "GB/s",
                         "ms_per_step": round(el_mt / reps_mt * 1e3, 3), "cores": cores, "kind": "port",
                         "what": f"C restatement of matmul_{q.lower()}, rows split over {cores} threads",
                         "max_rel_err_vs_gpu": float(np.max(np.abs(y_gpu - y_mt)) / np.max(np.abs(y_mt)))},
        "numpy_path": {"value": round(work.bytes / t_np / 1e9, 4), "unit": "GB/s", "ms_per_step": round(t_np * 1e3, 2),
                       "cores": os.cpu_count(), "what": "dequant_q4_k restatement + numpy BLAS matvec"},
        "gpu_vs_cpu_max_rel_err": err, "gpu_vs_numpy_max_rel_err": err_np,
    }


def cpu_rates(q: str, n: int, k: int, raw: np.ndarray, x: np.ndarray, nbytes: int, budget_s: float = 1.0) -> dict:
    """The reference's CPU paths on one benchmark config, timed on this host
    beside the GPU figure: its native matmul (the reference's own _C built
    from its sources, scalar x86, 1 thread; Q8_0, Q4_K and Q6_K only), the C
    restatement with rows split over every host core (same formats), and the
    NumPy path (dequant + BLAS matvec on all cores; skipped above 10^8
    weights, where the fp32 dequant alone takes tens of seconds). Each runs
    for about `budget_s`, at least one call after one warm call."""
    from oracle import gguf_np as G
    from oracle.loader import c_oracle, ref_C

    cores = os.cpu_count() or 1

    def rate(fn) -> dict:
        fn()
        reps, t0 = 0, time.perf_counter()
        while True:
            fn()
            reps += 1
            el = time.perf_counter() - t0
            if el >= budget_s or reps >= 50:
                break
        return {"gbs": round(nbytes * reps / el / 1e9, 4), "ms_per_call": round(el / reps * 1e3, 3)}

    out = {}
    R = ref_C()
    if R is not None and hasattr(R, f"matmul_{q.lower()}"):
        fn = getattr(R, f"matmul_{q.lower()}")
        out["reference_native_1_thread"] = rate(lambda: fn(x, raw, n, k))
    if q in ("Q8_0", "Q4_K", "Q6_K"):
        co = c_oracle()
        out["row_parallel"] = dict(rate(lambda: co.matmul(q, x, raw, n, k, threads=cores)), cores=cores)
    if n * k <= 10**8:
        out["numpy"] = dict(rate(lambda: G.matmul_numpy(q, x, raw, n, k)), cores=cores)
    return out


# (name, quant, out, in, kernel): kernel None = the default device path
# (for these Q4_K shapes the element-wise fp32 kernel: dequant and dot in one
# pass); GEMV_MX forces the matrix-core kernel beside it
SUITE = [
    ("q8_0_4864x896", "Q8_0", 4864, 896, None),
    ("q4_k_18944x3584", "Q4_K", 18944, 3584, None),
    ("q4_k_3584x18944", "Q4_K", 3584, 18944, None),
    ("q4_k_3584x18944_matrix_cores", "Q4_K", 3584, 18944, _lib.GEMV_MX),
    ("q4_k_18944x3584_matrix_cores", "Q4_K", 18944, 3584, _lib.GEMV_MX),
    ("q6_k_152064x3584", "Q6_K", 152064, 3584, None),
    ("q1_0_4096x4096", "Q1_0", 4096, 4096, None),
]

# Llama-3-8B Q4_K_M projection mix: (name, quant, out, in)
LLAMA_LAYER = [
    ("q", "Q4_K", 4096, 4096), ("k", "Q4_K", 1024, 4096), ("v", "Q6_K", 1024, 4096), ("o", "Q4_K", 4096, 4096),
    ("gate", "Q4_K", 14336, 4096), ("up", "Q4_K", 14336, 4096), ("down", "Q6_K", 4096, 14336),
]


def run_suite(stream, steps: int, only: set | None = None, cpu: bool = True) -> dict:
    out = {}

    def want(name: str) -> bool:
        return not only or name in only

    for idx, (name, q, n, k, kernel) in enumerate(SUITE):
        if not want(name):
            continue
        w = GemvWorkload(q, n, k, seed=100 + idx, stream=stream, kernel=kernel)
        # after the settle burst: 200 untimed launches, then `steps` (>= 500)
        # timed ones, two graphs differenced (graph_time)
        t = w.time_throughput(steps, warmup=200)
        te = w.time_eager(min(steps, 200))
        tk = t / steps
        out[name] = {"gbs": round(w.bytes / tk / 1e9, 1), "kernel_us": round(tk * 1e6, 2),
                     "frac_hbm": round(w.bytes / tk / 1e9 / HBM_PEAK_GBS, 4),
                     "eager_us_per_launch": round(te / min(steps, 200) * 1e6, 2), "effective_bytes": w.bytes}
        if kernel is None and cpu:
            out[name]["cpu"] = cpu_rates(q, n, k, w.raw, w.x_host, w.bytes)
        w.free()
    extra = [("llama3_8b_decode_resident", lambda: decode_sweep_resident(stream, steps=max(3, min(steps // 50, 20)),
                                                                         cpu_baseline_on=cpu)),
             ("llama3_8b_decode_streamed", lambda: decode_sweep_streamed(stream)),
             ("llama3_8b_decode_scheduler_hook", lambda: decode_scheduler_hook(stream)),
             ("prefill_gemm_q4_k_bf16_512x14336x4096", lambda: prefill_gemm(stream, cpu_baseline_on=cpu)),
             ("llama3_8b_prefill_layer_512", lambda: prefill_layer(stream)),
             ("batched_f32_q4_k_3584x18944", lambda: batched_f32(stream, cpu_baseline_on=cpu)),
             ("dequant", lambda: dequant_suite(stream)),
             ("copy_ceiling", lambda: copy_ceiling(stream)),
             ("read_ceiling_447MB", lambda: read_ceiling(stream, synth.nbytes("Q6_K", 152064, 3584), reps=50)),
             ("gguf_load_llama3_8b_4_layers", lambda: gguf_load(stream)),
             ("host_path_q4_k_3584x18944", host_path_rate),
             ("drop_in_host_call_q4_k_3584x18944", drop_in_host_call)]
    for name, fn in extra:
        if want(name):
            out[name] = fn()
    return out


GGUF_PROJ = {"q": "attn_q", "k": "attn_k", "v": "attn_v", "o": "attn_output", "gate": "ffn_gate", "up": "ffn_up",
             "down": "ffn_down"}


def gguf_load(stream, layers: int = 4) -> dict:
    """A synthetic Llama-3-8B-shaped GGUF file (``layers`` decoder layers, the
    Q4_K_M projection mix, llama.cpp tensor names) written to a temporary
    directory, then loaded by ResidentModel: parse + mmap + page cache ->
    pinned -> HBM. The file was just written, so its pages are in the page
    cache (a cold disk read would add the disk's own rate). One decode step
    over the loaded tensors checks that they serve the GEMVs."""
    import tempfile

    from flatrun_amd import gguf

    host = {name: synth.make_blocks(q, n, k, seed=i) for i, (name, q, n, k) in enumerate(LLAMA_LAYER)}
    tensors = [(f"blk.{L}.{GGUF_PROJ[name]}.weight", (n, k), q, host[name].tobytes())
               for L in range(layers) for name, q, n, k in LLAMA_LAYER]
    with tempfile.TemporaryDirectory() as d:
        path = Path(d) / "llama3_8b_layers.gguf"
        gguf.write_gguf(path, tensors, {"general.architecture": "llama", "llama.block_count": layers})
        t0 = time.perf_counter()
        f = gguf.GGUFFile(path)
        t_parse = time.perf_counter() - t0
        m = gguf.ResidentModel(f, stream=stream)
        kmax = max(k for *_, k in LLAMA_LAYER)
        nmax = max(n for _, _, n, _ in LLAMA_LAYER)
        x = device.DeviceBuffer.from_host(synth.make_x(kmax, seed=5))
        y = device.DeviceBuffer(4 * nmax)
        for L in range(layers):
            for name, q, n, k in LLAMA_LAYER:
                w = m[gguf.translate_gguf_name(f"blk.{L}.{GGUF_PROJ[name]}.weight")]
                device.gemv(q, w, x, y, n, k, stream=stream, w_bytes=w.nbytes)
        device.synchronize()
        finite = bool(np.isfinite(y.to_host(np.float32)).all())
        out = {"layers": layers, "bytes": m.nbytes, "parse_ms": round(t_parse * 1e3, 2),
               "load_ms": round(m.load_seconds * 1e3, 1), "load_gbs": round(m.load_gbs, 2),
               "decode_step_outputs_finite": finite,
               "note": "warm page cache; staging 2 x 64 MiB pinned, 8 host copy threads"}
        x.free()
        y.free()
        m.close()
        f.close()
    return out


def decode_sweep_streamed(stream, layers: int = 32, depth: int = 3, steps: int = 2) -> dict:
    """All 32 layers' raw blocks in pinned host memory; one step streams every
    layer through a ring of `depth` device slots (copy stream) while the
    compute stream runs each layer's 7 GEMVs as soon as its copy lands."""
    from flatrun_amd.streaming import LayerStreamer

    st = LayerStreamer([(n_, q, n, k) for n_, q, n, k in LLAMA_LAYER], layers, depth=depth)
    host = {name: synth.make_blocks(q, n, k, seed=i) for i, (name, q, n, k) in enumerate(LLAMA_LAYER)}
    for L in range(layers):
        st.fill(L, host)
    kmax = max(k for *_, k in LLAMA_LAYER)
    nmax = max(n for _, _, n, _ in LLAMA_LAYER)
    x = device.DeviceBuffer.from_host(synth.make_x(kmax, seed=5))
    y = device.DeviceBuffer(4 * nmax)
    st.step(x, y, stream)
    device.synchronize()
    e0, e1 = device.Event(), device.Event()
    e0.record(stream)
    for _ in range(steps):
        st.step(x, y, stream)
    e1.record(stream)
    e1.synchronize()
    ms = e0.elapsed_ms(e1) / steps
    total = st.layer_bytes * layers
    st.close()
    x.free()
    y.free()
    return {"ms_per_step": round(ms, 3), "weight_bytes_per_step": total, "ring_slots": depth,
            "h2d_gbs": round(total / (ms / 1e3) / 1e9, 2),
            "note": "pinned host -> device over PCIe, overlapped with the GEMVs of earlier layers"}


def decode_scheduler_hook(stream, layers: int = 8, depth: int = 3, passes: int = 3) -> dict:
    """The reference scheduler's prefetch-hook path at Llama-3-8B shapes:
    a synthetic GGUF of `layers` decoder layers (the Q4_K_M mix, 139 MB per
    layer), bound through SchedulerStream (ring of `depth` device slots fed
    from the file mapping through two pinned staging slots). A restatement of
    LayerScheduler's call order (runtime/scheduler.py:222-242, 270-319) runs
    `passes` sweeps over the layers: per layer the hook, then the forwarder's
    seven projections through NativeBackend.matmul_* on host x (1-D), each
    weight handed over as the handle returns it. Two handles:
      copying    the reference's MmapTensorHandle.view (core/tensor.py:227-250):
                 an array over mmap[a:b], a fresh bytes copy per call, so every
                 call pays that copy and a content hash to find the weight;
      zero-copy  a view of the mapping itself (np.frombuffer), keyed once.
    Reported per layer and scaled to the 32 layers of a decode step."""
    import mmap as _mmap
    import tempfile

    from flatrun_amd import NativeBackend, gguf, residency
    from flatrun_amd.streaming import SchedulerStream

    host = {name: synth.make_blocks(q, n, k, seed=i) for i, (name, q, n, k) in enumerate(LLAMA_LAYER)}
    meth = {"Q4_K": "matmul_q4k", "Q6_K": "matmul_q6k", "Q8_0": "matmul_q8_0"}
    xs = {k: synth.make_x(k, seed=k) for k in {k for *_, k in LLAMA_LAYER}}
    out = {"layers_in_file": layers, "ring_slots": depth, "passes": passes}
    with tempfile.TemporaryDirectory() as d:
        path = Path(d) / "llama3_8b_layers.gguf"
        stored = {L: [f"blk.{L}.{GGUF_PROJ[nm]}.weight" for nm, *_ in LLAMA_LAYER] for L in range(layers)}
        gguf.write_gguf(path, [(stored[L][i], (n, k), q, host[nm].tobytes()) for L in range(layers)
                               for i, (nm, q, n, k) in enumerate(LLAMA_LAYER)],
                        {"general.architecture": "llama", "llama.block_count": layers})
        names = {L: [gguf.translate_gguf_name(t) for t in stored[L]] for L in range(layers)}   # the reader's names
        f = gguf.GGUFFile(path)
        fd = open(path, "rb")
        mm = _mmap.mmap(fd.fileno(), 0, access=_mmap.ACCESS_READ)
        infos = {nm: f.info(nm) for L in range(layers) for nm in names[L]}

        def copying(nm):
            i = infos[nm]
            a = np.ndarray(shape=(i.nbytes,), dtype=np.uint8, buffer=mm[i.offset:i.offset + i.nbytes])
            a.flags.writeable = False
            return a

        def zero_copy(nm):
            i = infos[nm]
            return np.frombuffer(mm, dtype=np.uint8, count=i.nbytes, offset=i.offset)

        class _Layer:                                    # utils/types.py:124-138
            def __init__(self, index, tensor_names):
                self.index, self.tensor_names = index, tensor_names

        lay = [_Layer(L, tuple(names[L])) for L in range(layers)]
        for label, handle in (("copying", copying), ("zero_copy", zero_copy)):
            nb = NativeBackend()
            st = SchedulerStream(f, lay, depth=depth)
            nb.attach_stream(st)
            hook = st.hook

            def run_layer(L):
                hook(lay[L])
                for (nm, q, n, k), tname in zip(LLAMA_LAYER, names[L]):
                    getattr(nb, meth[q])(xs[k], handle(tname), n, k)

            for L in range(layers):                      # one untimed pass: caches, keys, pipeline
                run_layer(L)
            t0 = time.perf_counter()
            for _ in range(passes):
                for L in range(layers):
                    run_layer(L)
            dt = (time.perf_counter() - t0) / (passes * layers)
            stats = dict(st.stats)
            nb.attach_stream(None)
            st.close()
            # what the copy and the hash cost alone, per layer
            t0 = time.perf_counter()
            arrs = [handle(tname) for tname in names[0]]
            t_handle = time.perf_counter() - t0
            t0 = time.perf_counter()
            for arr in arrs:
                residency.content_key(arr)
            t_hash = time.perf_counter() - t0
            del arrs, arr
            layer_bytes = sum(infos[t].nbytes for t in names[0])
            out[label] = {"ms_per_layer": round(dt * 1e3, 3), "ms_per_step_32_layers": round(dt * 32e3, 1),
                          "h2d_gbs_effective": round(layer_bytes / dt / 1e9, 2),
                          "handle_ms_per_layer": round(t_handle * 1e3, 3),
                          "hash_ms_per_layer": round(t_hash * 1e3, 3),
                          "hash_ms_per_step_32_layers": round(t_hash * 32e3, 1),
                          "lookups_hit": stats["hits"], "lookups_missed": stats["misses"],
                          "layers_streamed": stats["layers_streamed"]}
        out["layer_bytes"] = layer_bytes
        out["note"] = ("host x and y per call (the drop-in call shape); copying handles pay the mmap[a:b] copy "
                       "and the content hash on every call, zero-copy handles neither")
        try:
            mm.close()
        except BufferError:
            pass                    # a view still alive: the mapping goes with it
        fd.close()
        f.close()
    return out


def prefill_gemm(stream, m: int = 512, n: int = 14336, k: int = 4096, reps: int = 200,
                 cpu_baseline_on: bool = True) -> dict:
    """Q4_K prefill GEMM on the matrix cores, Y[m, n] = X[m, k] (bf16) . W^T,
    W rotated over 8 distinct copies (264 MB, beyond the Infinity Cache).
    `reps` launches per graph (~16 ms at 200): a graph of 20 (2 ms) reads
    15 % slower, before the part settles."""
    from flatrun_amd import _C

    raw = synth.make_blocks("Q4_K", n, k, seed=31)
    x = _C.to_bf16_bits(np.random.default_rng(32).standard_normal((m, k)).astype(np.float32))
    ws = [device.DeviceBuffer.from_host(raw) for _ in range(8)]
    xd, yd = device.DeviceBuffer.from_host(x), device.DeviceBuffer(4 * m * n)
    device.gemm_q4k_bf16(ws[0], xd, yd, m, n, k, stream=stream, w_bytes=raw.nbytes)   # any scratch before capture
    stream.synchronize()
    with device.Graph.capture(stream) as cap:
        for i in range(reps):
            device.gemm_q4k_bf16(ws[i % len(ws)], xd, yd, m, n, k, stream=stream, w_bytes=raw.nbytes)
    cap.launch(stream)
    device.synchronize()
    e0, e1 = device.Event(), device.Event()
    e0.record(stream)
    cap.launch(stream)
    e1.record(stream)
    e1.synchronize()
    us = e0.elapsed_ms(e1) / reps * 1e3
    cap.destroy()
    for b in ws:
        b.free()
    xd.free()
    yd.free()
    flop = 2 * m * n * k
    out = {"us": round(us, 2), "tflops": round(flop / us / 1e6, 1), "flop": flop,
           "frac_bf16_peak": round(flop / us / 1e6 / BF16_PEAK_TFLOPS, 4), "peak_tflops": BF16_PEAK_TFLOPS,
           "mfma_busy_pct_profiled": measured_mfma_util()}
    if cpu_baseline_on:
        # the reference prefills with matmul_q4_k_batched: one scalar GEMV per
        # token (_C.cpp:154-197); 4 of the 512 fp32 token rows, scaled
        from oracle.loader import ref_C

        R = ref_C()
        if R is not None:
            xs = np.random.default_rng(33).standard_normal((4, k)).astype(np.float32)
            t0 = time.perf_counter()
            R.matmul_q4_k_batched(xs, raw, n, k)
            out["cpu"] = {"reference_native_batched_1_thread_ms": round((time.perf_counter() - t0) * m / 4 * 1e3, 1),
                          "sample": f"4 of {m} token rows timed, scaled to {m}"}
    return out


def batched_f32(stream, q: str = "Q4_K", n: int = 3584, k: int = 18944, seqs=(2, 4, 32, 512),
                cpu_baseline_on: bool = True) -> dict:
    """The fp32 batched matvec (frq_dev_gemv with batch = seq rows of x), the
    shape of the reference CLI's re-prefill: every generated token multiplies
    the whole sequence so far by each weight (matmul_<q>_batched, one fp32
    matvec per row). One matrix-core GEMM launch reads W once per tile of x
    rows. Per seq: mean launch time over a graph-replayed region (weight
    copies rotated past the Infinity Cache), effective GB/s (W once + x + y),
    GFLOP/s (2 seq n k), and the time of seq single-row launches for
    comparison (two to six rows run the small-M matvec, W read once per two
    or three rows); cpu: the reference's native batched matmul (1 thread) on
    2 rows, scaled to seq."""
    single = GemvWorkload(q, n, k, seed=300, stream=stream)
    t1 = single.time_throughput(500, warmup=200) / 500
    single.free()
    out = {"shape": f"{q} {n}x{k}", "single_row_us": round(t1 * 1e6, 2)}
    for seq in seqs:
        steps = 200 if seq <= 32 else 40
        w = GemvWorkload(q, n, k, seed=300 + seq, stream=stream, batch=seq)
        t = w.time_throughput(steps, warmup=20) / steps
        out[f"seq{seq}"] = {"us": round(t * 1e6, 2), "gbs": round(w.bytes / t / 1e9, 1),
                            "gflops": round(2 * seq * n * k / t / 1e9, 1),
                            "seq_single_row_launches_us": round(seq * t1 * 1e6, 1),
                            "speedup_vs_single_rows": round(seq * t1 / t, 2)}
        w.free()
    if cpu_baseline_on:
        from oracle.loader import ref_C

        R = ref_C()
        if R is not None:
            raw = synth.make_blocks(q, n, k, seed=301)
            xs = synth.make_x(k, seed=302, batch=2)
            t0 = time.perf_counter()
            getattr(R, f"matmul_{q.lower()}_batched")(xs, raw, n, k)
            per_row = (time.perf_counter() - t0) / 2
            out["cpu"] = {"reference_native_batched_1_thread_ms_per_row": round(per_row * 1e3, 2),
                          "sample": "2 rows timed; the reference's batched loop is one matvec per row"}
    return out


def drop_in_host_call(q: str = "Q4_K", n: int = 3584, k: int = 18944, reps: int = 20) -> dict:
    """The one-line drop-in (NativeBackend.matmul_q4k(x, raw, n, k) on host
    arrays), per call, median ms of `reps`, with the weight read from a file
    mapping as the reference's forwarder reads it:
      copy_view     what MmapTensorHandle.view returns (core/tensor.py:240-247):
                    an array over ``mmap[a:b]``, a fresh bytes copy per call
                    (the copy is timed inside the call, as the forwarder pays it);
      zero_copy     an array over ``memoryview(mmap)[a:b]`` (no copy; file-backed);
    each without the weight cache (the weight crosses PCIe every call) and
    with it (content key: a hash of the copy per call, or once for the
    file-backed view). ``handle_copy_ms`` is the reference's copy alone."""
    import mmap
    import tempfile

    from flatrun_amd import NativeBackend

    raw = synth.make_blocks(q, n, k, seed=41)
    x = synth.make_x(k, seed=42)
    meth = {"Q4_K": "matmul_q4k", "Q6_K": "matmul_q6_k", "Q8_0": "matmul_q8_0"}[q]
    nb = raw.nbytes

    def med(fn) -> float:
        fn()
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return round(float(np.median(ts)) * 1e3, 3)

    out = {"shape": f"{q} {n}x{k}", "weight_bytes": nb}
    with tempfile.TemporaryDirectory() as d:
        path = Path(d) / "w.bin"
        path.write_bytes(raw.tobytes())
        with open(path, "rb") as fh:
            mm = mmap.mmap(fh.fileno(), 0, access=mmap.ACCESS_READ)

            def copy_view():
                a = np.ndarray(shape=(nb,), dtype=np.uint8, buffer=mm[0:nb])
                a.flags.writeable = False
                return a

            def zero_view():
                a = np.ndarray(shape=(nb,), dtype=np.uint8, buffer=memoryview(mm)[0:nb])
                a.flags.writeable = False
                return a

            out["handle_copy_ms"] = med(lambda: mm[0:nb])
            for cache in (False, True):
                be = NativeBackend(weight_cache="4G" if cache else False)
                for vname, view in (("copy_view", copy_view), ("zero_copy", zero_view)):
                    out[f"{vname}_{'cached' if cache else 'uncached'}_ms"] = med(
                        lambda: getattr(be, meth)(x, view(), n, k))
                if cache:
                    st = be.cache_stats()
                    out["cache_hits"], out["cache_misses"] = st["hits"], st["misses"]
                    be._cache.clear()
            mm.close()
    return out


def prefill_layer(stream, m: int = 512, reps: int = 20) -> dict:
    """One Llama-3-8B decoder layer's projections at prefill, Y = X . W^T for
    the Q4_K_M mix (q, k, o, gate, up Q4_K; v, down Q6_K), X [512 x in] bf16:
    seven bf16-MFMA GEMMs (shapes with few output tiles split K), captured as
    one graph and replayed. `grouped`: the same seven products with q|k|v and
    gate|up as frq_dev_gemm_bf16_group launches into concatenated outputs
    ([512 x 6144], [512 x 28672]; K split for each group's tile count), four
    GEMM launches."""
    from flatrun_amd import _C

    host = {name: synth.make_blocks(q, n, k, seed=40 + i) for i, (name, q, n, k) in enumerate(LLAMA_LAYER)}
    dev = {name: device.DeviceBuffer.from_host(host[name]) for name, *_ in LLAMA_LAYER}
    kmax = max(k for *_, k in LLAMA_LAYER)
    nmax = max(n for _, _, n, _ in LLAMA_LAYER)
    x = _C.to_bf16_bits(np.random.default_rng(41).standard_normal((m, kmax)).astype(np.float32))
    xd = device.DeviceBuffer.from_host(x)
    yd = device.DeviceBuffer(4 * m * 2 * nmax)
    groups = [["q", "k", "v"], ["o"], ["gate", "up"], ["down"]]
    shape = {name: (q, n, k) for name, q, n, k in LLAMA_LAYER}

    def layer():
        for name, q, n, k in LLAMA_LAYER:
            device.gemm_bf16(q, dev[name], xd, yd, m, n, k, stream=stream, w_bytes=host[name].nbytes)

    def layer_grouped():
        for names in groups:
            if len(names) == 1:
                q, n, k = shape[names[0]]
                device.gemm_bf16(q, dev[names[0]], xd, yd, m, n, k, stream=stream, w_bytes=host[names[0]].nbytes)
                continue
            ns = [shape[nm][1] for nm in names]
            offs = np.concatenate([[0], np.cumsum(ns)[:-1]])
            device.gemm_bf16_group([(shape[nm][0], dev[nm], shape[nm][1], yd.ptr + 4 * int(o), host[nm].nbytes)
                                    for nm, o in zip(names, offs)], xd, m, shape[names[0]][2], y_stride=sum(ns),
                                   stream=stream)

    def timed(fn):
        fn()                                  # split-K scratch exists before capture
        stream.synchronize()
        with device.Graph.capture(stream) as cap:
            for _ in range(reps):
                fn()
        cap.launch(stream)
        device.synchronize()
        e0, e1 = device.Event(), device.Event()
        e0.record(stream)
        cap.launch(stream)
        e1.record(stream)
        e1.synchronize()
        cap.destroy()
        return e0.elapsed_ms(e1) / reps * 1e3

    us = timed(layer)
    us_g = timed(layer_grouped)
    for b in dev.values():
        b.free()
    xd.free()
    yd.free()
    flop = sum(2 * m * n * k for _, _, n, k in LLAMA_LAYER)
    return {"us_per_layer": round(us, 1), "tflops": round(flop / us / 1e6, 1), "flop": flop, "gemms": len(LLAMA_LAYER),
            "frac_bf16_peak": round(flop / us / 1e6 / BF16_PEAK_TFLOPS, 4),
            "grouped": {"us_per_layer": round(us_g, 1), "tflops": round(flop / us_g / 1e6, 1), "gemm_launches": 4,
                            "frac_bf16_peak": round(flop / us_g / 1e6 / BF16_PEAK_TFLOPS, 4)},
            "note": "X 512 tokens (bf16); W resident raw blocks; the reference re-dequantizes W per token"}


DEQUANT_SUITE = [("Q8_0", 4864, 896), ("Q4_K", 18944, 3584), ("Q5_K", 18944, 3584), ("Q6_K", 152064, 3584),
                 ("Q8_0", 18944, 3584), ("Q1_0", 18944, 3584), ("Q4_0", 18944, 3584), ("Q5_0", 18944, 3584),
                 ("Q5_1", 18944, 3584)]


# fp16-output dequant (dequant_handle's default dtype): the big shapes
DEQUANT_F16_SUITE = [("Q4_K", 18944, 3584), ("Q6_K", 152064, 3584)]


def dequant_suite(stream, reps: int = 100) -> dict:
    """Block dequant to fp32 at the workload shapes, and every format at
    18944 x 3584: algorithmic bytes = raw blocks read + 4 n k written
    (2 n k for the fp16 lines, `_f16`), timed as a graph of at least `reps`
    launches. Weight copies and outputs rotate independently, each set over
    >= 1 GiB, so no launch finds its weights or its output in the 256 MB
    last-level cache. (A rotation over (weight, output) pairs is not enough:
    the outputs are written with non-temporal stores, which do not evict the
    weights from that cache, and the weights of a few pairs fit in it.)"""
    out = {}
    cases = [(q, n, k, 4) for q, n, k in DEQUANT_SUITE] + [(q, n, k, 2) for q, n, k in DEQUANT_F16_SUITE]
    for q, n, k, osz in cases:
        raw = synth.make_blocks(q, n, k, seed=50)
        nw = max(2, math.ceil(ROTATE_BYTES / raw.nbytes))
        ny = max(2, math.ceil(ROTATE_BYTES / (osz * n * k)))
        ws = [device.DeviceBuffer.from_host(raw) for _ in range(nw)]
        ys = [device.DeviceBuffer(osz * n * k) for _ in range(ny)]
        reps_q = max(reps, nw, ny)
        step = device.dequant if osz == 4 else device.dequant_f16
        us = graph_time(stream, lambda i: step(q, ws[i % nw], ys[i % ny], n * k, stream=stream,
                                                   w_bytes=raw.nbytes), reps_q, reps_q) / reps_q * 1e6
        for b in ws + ys:
            b.free()
        nbytes = raw.nbytes + osz * n * k
        out[f"{q.lower()}_{n}x{k}" + ("_f16" if osz == 2 else "")] = {
                                       "us": round(us, 2), "gbs": round(nbytes / us / 1e3, 1),
                                       "frac_hbm": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4),
                                       "algorithmic_bytes": nbytes, "weights_rotated": nw, "outputs_rotated": ny}
    return out


def copy_ceiling(stream, mib: int = 512, reps: int = 20) -> dict:
    """The library's plain streaming copy (16 B per lane, read + write) over
    `mib` MiB, replayed from a graph: the practical HBM ceiling to compare
    the GEMV against."""
    nbytes = mib << 20
    src, dst = device.DeviceBuffer(nbytes), device.DeviceBuffer(nbytes)
    ms = graph_time(stream, lambda i: device.copy(dst, src, nbytes, stream=stream), reps, reps) / reps * 1e3
    src.free()
    dst.free()
    return {"bytes_moved": 2 * nbytes, "us": round(ms * 1e3, 2), "gbs": round(2 * nbytes / (ms / 1e3) / 1e9, 1)}


def read_ceiling(stream, nbytes: int, reps: int = 200, bufs=None) -> dict:
    """The library's plain streaming read (16 B per lane, XOR-folded, one word
    written per workgroup) of `nbytes`, one distinct buffer per launch out of
    >= 1 GiB (`bufs`, or fresh ones), replayed from a graph like the GEMV:
    the practical ceiling for a kernel that reads `nbytes` once per launch."""
    nbytes = nbytes // 16 * 16
    own = bufs is None
    if own:
        bufs = [device.DeviceBuffer(nbytes) for _ in range(max(2, math.ceil(ROTATE_BYTES / nbytes)))]
    out = device.DeviceBuffer(4 * device.READ_XOR_WORDS)
    reps = max(reps, len(bufs))
    us = graph_time(stream, lambda i: device.read_xor(bufs[i % len(bufs)], nbytes, out, stream=stream),
                    reps, reps) / reps * 1e6
    out.free()
    if own:
        for b in bufs:
            b.free()
    return {"bytes": nbytes, "buffers_rotated": len(bufs), "us": round(us, 2), "gbs": round(nbytes / us / 1e3, 1),
            "frac_hbm": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4)}


def host_path_rate(reps: int = 20) -> dict:
    """The reference-shaped host entry point (_C.matmul_q4_k: numpy in, numpy
    out, weight and x copied host -> device on every call): PCIe-inclusive."""
    from flatrun_amd import _C

    q, n, k = "Q4_K", 3584, 18944
    raw = synth.make_blocks(q, n, k, seed=7)
    x = synth.make_x(k, seed=8)
    _C.matmul_q4_k(x, raw, n, k)
    t0 = time.perf_counter()
    for _ in range(reps):
        _C.matmul_q4_k(x, raw, n, k)
    dt = (time.perf_counter() - t0) / reps
    return {"ms_per_call": round(dt * 1e3, 3), "gbs": round(effective_bytes(q, n, k) / dt / 1e9, 2),
            "note": "pageable host buffers; includes the H2D copy of the raw weight bytes every call"}


def decode_step_cpu(host: dict, layers: int = 32) -> dict:
    """The reference's CPU paths on one Llama-3-8B layer's seven projections
    (the same seeded blocks), timed once each and scaled to 32 layers: its
    native matmuls (1 thread) and the C restatement on every host core."""
    from oracle.loader import c_oracle, ref_C

    cores = os.cpu_count() or 1
    R, co = ref_C(), c_oracle()
    xs = {k: synth.make_x(k, seed=5) for k in {k for *_, k in LLAMA_LAYER}}
    out = {"sample": "one layer's 7 projections timed once, x 32 layers"}
    if R is not None:
        t0 = time.perf_counter()
        for name, q, n, k in LLAMA_LAYER:
            getattr(R, f"matmul_{q.lower()}")(xs[k], host[name], n, k)
        out["reference_native_1_thread_ms_per_step"] = round((time.perf_counter() - t0) * layers * 1e3, 1)
    t0 = time.perf_counter()
    for name, q, n, k in LLAMA_LAYER:
        co.matmul(q, xs[k], host[name], n, k, threads=cores)
    out["row_parallel_ms_per_step"] = round((time.perf_counter() - t0) * layers * 1e3, 1)
    out["row_parallel_cores"] = cores
    return out


def decode_sweep_resident(stream, steps: int, layers: int = 32, cpu_baseline_on: bool = True) -> dict:
    """All 32 layers' raw blocks resident in HBM; one step = 224 GEMVs."""
    host = {name: synth.make_blocks(q, n, k, seed=i) for i, (name, q, n, k) in enumerate(LLAMA_LAYER)}
    dev = [{name: device.DeviceBuffer.from_host(host[name]) for name, *_ in LLAMA_LAYER} for _ in range(layers)]
    kmax = max(k for *_, k in LLAMA_LAYER)
    nmax = max(n for _, _, n, _ in LLAMA_LAYER)
    x = device.DeviceBuffer.from_host(synth.make_x(kmax, seed=5))
    y = device.DeviceBuffer(4 * nmax)
    total = sum(synth.nbytes(q, n, k) for _, q, n, k in LLAMA_LAYER) * layers

    def step():
        for L in range(layers):
            for name, q, n, k in LLAMA_LAYER:
                device.gemv(q, dev[L][name], x, y, n, k, stream=stream, w_bytes=host[name].nbytes)

    spec = {name: (q, n) for name, q, n, _ in LLAMA_LAYER}
    ycat = device.DeviceBuffer(4 * (2 * 14336 + 6144))

    def group(L, names, k):
        parts, off = [], 0
        for nm in names:
            q, n = spec[nm]
            parts.append((q, dev[L][nm], n, ycat.ptr + 4 * off, host[nm].nbytes))
            off += n
        return parts, k

    groups = [[group(L, ("q", "k", "v"), 4096), group(L, ("o",), 4096), group(L, ("gate", "up"), 4096),
               group(L, ("down",), 14336)] for L in range(layers)]

    def step_fused():
        # the forwarder's launch pattern with shared-x fusion: q|k|v, o, gate|up, down
        for L in range(layers):
            for parts, k in groups[L]:
                device.gemv_group(parts, x, k, stream=stream)

    def timed(run) -> float:
        run()
        device.synchronize()
        e0, e1 = device.Event(), device.Event()
        e0.record(stream)
        for _ in range(steps):
            run()
        e1.record(stream)
        e1.synchronize()
        return e0.elapsed_ms(e1) / steps

    ms_eager = timed(step)
    with device.Graph.capture(stream) as cap:
        step()
    ms = timed(lambda: cap.launch(stream))
    cap.destroy()
    with device.Graph.capture(stream) as capf:
        step_fused()
    ms_f = timed(lambda: capf.launch(stream))
    capf.destroy()
    fused_ok = all(device.gemv_group_fusable([(p[0], p[1]) for p in parts], k)
                   for parts, k in groups[0] if len(parts) > 1)
    ycat.free()
    # the forwarder's chain with resident activations (flatrun_amd.layer):
    # q|k|v -> o (on the q part) -> gate|up and SiLU.mul -> down, per layer
    from flatrun_amd.layer import DecoderProjections

    drivers = [DecoderProjections({nm: (spec[nm][0], dev[L][nm], spec[nm][1], kk, host[nm].nbytes)
                                   for nm, _, _, kk in LLAMA_LAYER}, max_seq=1, stream=stream)
               for L in range(layers)]

    def step_driver():
        for L, dp in enumerate(drivers):
            qkv = dp.qkv_proj(x)
            dp.mlp(dp.o_proj(qkv))          # seq 1: the q part leads each qkv row

    k_gate = {nm: kk for nm, _, _, kk in LLAMA_LAYER}["gate"]
    mlp_fused = all(device.gemv_swiglu_fusable((spec["gate"][0], dev[L]["gate"]), (spec["up"][0], dev[L]["up"]),
                                               k_gate) for L in range(layers))
    with device.Graph.capture(stream) as capd:
        step_driver()
    ms_d = timed(lambda: capd.launch(stream))
    capd.destroy()
    for dp in drivers:
        dp.close()
    for d in dev:
        for b in d.values():
            b.free()
    cpu = decode_step_cpu(host) if cpu_baseline_on else None
    return {"ms_per_step": round(ms, 4), "ms_per_step_eager": round(ms_eager, 4), "weight_bytes_per_step": total,
            **({"cpu": cpu} if cpu else {}),
            "gemvs_per_step": layers * len(LLAMA_LAYER), "gbs": round(total / (ms / 1e3) / 1e9, 1),
            "floor_ms_at_8TBs": round(total / 8e12 * 1e3, 4),
            "fused_shared_x": {"ms_per_step": round(ms_f, 4), "launches_per_step": layers * 4,
                               "gbs": round(total / (ms_f / 1e3) / 1e9, 1), "groups_fused": fused_ok,
                               "note": "q|k|v and gate|up as one grouped launch each"},
            "decoder_chain_resident": {"ms_per_step": round(ms_d, 4),
                                       "launches_per_step": layers * (4 if mlp_fused else 5),
                                       "gbs": round(total / (ms_d / 1e3) / 1e9, 1), "mlp_fused": mlp_fused,
                                       "note": "DecoderProjections per layer: q|k|v grouped, o on the q part, "
                                               "gate|up and SiLU.mul in one launch (frq_dev_gemv_swiglu), "
                                               "down; activations resident, one graph per step"}}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=1000)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-suite", action="store_true")
    ap.add_argument("--configs", default="",
                    help="comma-separated subset of the other workloads to run (names as in the output's configs)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="after the headline, run the library's streaming copy 20 times over MIB MiB "
                         "(reference traffic for rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs)")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: measures one GPU (the matvec path is single-device); "
              f"--gpus {a.gpus} is not supported", file=sys.stderr)
        return 2
    _lib.lib()
    if _lib.device_count() <= 0:
        print("bench.py: no HIP device visible", file=sys.stderr)
        return 1
    _lib.check(_lib.lib().frq_set_device(0))
    stream = device.Stream()

    q, n, k = "Q4_K", 3584, 18944
    work = GemvWorkload(q, n, k, seed=2024, stream=stream)
    work.launch(0)
    y_gpu = work.result()
    t = work.time_throughput(a.steps, a.warmup)
    t_kernel = t / a.steps                      # mean launch duration over the timed region
    t_eager = work.time_eager(min(a.steps, 500)) / min(a.steps, 500)
    value = work.bytes * a.steps / t / 1e9
    achieved = work.bytes / t_kernel / 1e9
    rec = {
        "metric": "Q4_K GEMV GB/s (% HBM peak) @3584x18944 b1; ms per 8B decode step",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(t / a.steps * 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32 (Q4_K weights)",
        "data": "synthetic: seeded GGUF Q4_K blocks (d, dmin ~ U[1e-4, 5e-3], 6-bit scales/mins U[0,63], "
                "q U[0,15]), x ~ N(0,1)",
        "config": {"workload": "Q4_K GEMV W[3584 x 18944] (out x in) . x[18944], batch 1",
                   "effective_bytes_per_step": work.bytes, "weight_copies_rotated": work.ncopies,
                   "rotation_bytes": work.ncopies * work.raw.nbytes},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
                     "kernel_us": round(t_kernel * 1e6, 3)},
        "eager_launch_us": round(t_eager * 1e6, 3),
        "settle": work.settled,
    }
    # the same weight copies read by a plain streaming kernel: what any kernel
    # reading these bytes once per launch can reach on this part
    rc = read_ceiling(stream, work.raw.nbytes, reps=min(a.steps, 1000), bufs=work.w)
    rc["gemv_time_over_read_time"] = round(t_kernel * 1e6 / rc["us"], 3)
    rec["read_ceiling"] = rc
    if a.copy_calibration > 0:
        nbytes = a.copy_calibration << 20
        src, dst = device.DeviceBuffer(nbytes), device.DeviceBuffer(nbytes)
        for _ in range(20):
            device.copy(dst, src, nbytes, stream=stream)
        device.synchronize()
        src.free()
        dst.free()
    if not a.no_suite:
        only = {c for c in a.configs.split(",") if c}
        rec["configs"] = run_suite(stream, steps=500, only=only, cpu=not a.no_cpu)
        if "llama3_8b_decode_resident" in rec["configs"]:
            rec["decode_step_ms_resident"] = rec["configs"]["llama3_8b_decode_resident"]["ms_per_step"]
    if not a.no_cpu:
        rec["cpu_baseline"] = cpu_baseline(work, y_gpu, a.cpu_seconds)
    work.free()
    print(json.dumps(rec), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
