"""Layer weights streamed from pinned host memory, H2D overlapped with compute.

The reference's layer scheduler acquires a layer, computes it and releases it
synchronously (``LayerScheduler.run / _acquire_layer / _release_layer``,
``runtime/scheduler.py:222-325``); its prefetch hook is a no-op
(``_maybe_prefetch``, ``scheduler.py:191-198,270-277``), so the weights of the
next layer are not read until the current one is done. For a model that does
not fit (or is not kept) in HBM, this module keeps every layer's raw GGUF
blocks in pinned host memory and runs a ring of ``depth`` device slots:

* a copy stream fills slot ``L % depth`` with layer L (one ``hipMemcpyAsync``
  of the whole layer) once the compute stream has released that slot, i.e.
  finished layer ``L - depth``;
* the compute stream waits for the copy of layer L, runs its GEMVs from the
  slot, and records that the slot is free again.

Both streams are fed by the host without blocking, so while layer L computes,
layers L+1 .. L+depth-1 are already in flight over PCIe. The per-step time
is then bounded by the H2D bandwidth (4.44 GB per Llama-3-8B step), not by
copy + compute in series.
"""

from __future__ import annotations

import os
import threading
from concurrent.futures import ThreadPoolExecutor
from dataclasses import dataclass

import numpy as np

from . import device, synth

ALIGN = 256


def _align(n: int) -> int:
    return (n + ALIGN - 1) // ALIGN * ALIGN


class StagedCopier:
    """Host bytes -> device memory through two pinned staging slots.

    A source (a zero-copy view of the file mapping, i.e. page-cache bytes) is
    cut into chunks of ``staging_bytes``; ``threads`` host threads copy a
    chunk into a free slot (numpy releases the GIL for the copy) and the
    slot goes to the device with hipMemcpyAsync on the caller's stream, so
    the host copy of chunk i + 1 overlaps the DMA of chunk i. A slot is
    refilled only after its previous transfer has finished (an event per
    slot). Host memory held: 2 x staging_bytes of pinned memory."""

    def __init__(self, staging_bytes: int = 64 << 20, threads: int | None = None):
        self.staging = max(int(staging_bytes), 1 << 16)
        self.threads = min(8, os.cpu_count() or 1) if threads is None else max(1, int(threads))
        self._slots = [device.PinnedBuffer(self.staging) for _ in range(2)]
        self._done = [device.Event() for _ in range(2)]
        self._used = [False, False]
        self._k = 0
        self._pool = ThreadPoolExecutor(max_workers=self.threads, thread_name_prefix="frq-stage")

    def _fill(self, dst: np.ndarray, src: np.ndarray) -> None:
        parts = max(1, min(self.threads, src.size >> 20))
        step = (src.size + parts - 1) // parts
        list(self._pool.map(lambda i: np.copyto(dst[i * step:(i + 1) * step], src[i * step:(i + 1) * step]),
                            range(parts)))

    def copy(self, dst_ptr: int, src: np.ndarray, stream) -> None:
        """Enqueue src (1-D uint8) -> device address dst_ptr on `stream`;
        returns once the last chunk is staged (the DMA may still run)."""
        src = src.reshape(-1)
        pos, n = 0, int(src.size)
        while pos < n:
            m = min(self.staging, n - pos)
            s = self._k & 1
            if self._used[s]:
                self._done[s].synchronize()          # the slot's previous transfer has finished
            self._fill(self._slots[s].array[:m], src[pos:pos + m])
            device.memcpy_h2d_async(dst_ptr + pos, self._slots[s].ptr, m, stream=stream)
            self._done[s].record(stream)
            self._used[s] = True
            pos += m
            self._k += 1

    def close(self) -> None:
        for s, used in enumerate(self._used):
            if used:
                self._done[s].synchronize()
        self._pool.shutdown()
        for e in self._done:
            e.destroy()
        for p in self._slots:
            p.free()
        self._slots, self._done = [], []


@dataclass(frozen=True)
class TensorSlot:
    name: str
    qtype: str
    n: int
    k: int
    offset: int       # byte offset inside a layer
    nbytes: int


def plan_layer(tensors) -> tuple[list[TensorSlot], int]:
    """Places the tensors of one layer at ALIGN-byte offsets; returns the
    slots and the layer's byte size."""
    out, off = [], 0
    for name, q, n, k in tensors:
        nb = synth.nbytes(q, n, k)
        out.append(TensorSlot(name, q, int(n), int(k), off, nb))
        off += (nb + ALIGN - 1) // ALIGN * ALIGN
    return out, off


class LayerStreamer:
    """``n_layers`` layers of the same tensor layout, resident in pinned host
    memory, streamed through ``depth`` device slots."""

    def __init__(self, tensors, n_layers: int, depth: int = 3):
        if n_layers <= 0 or depth <= 0:
            raise ValueError("n_layers and depth must be positive")
        self.slots, self.layer_bytes = plan_layer(tensors)
        self.n_layers, self.depth = int(n_layers), int(min(depth, n_layers))
        self.host = device.PinnedBuffer(self.layer_bytes * self.n_layers)
        self.dev = [device.DeviceBuffer(self.layer_bytes) for _ in range(self.depth)]
        self.copy_stream = device.Stream()
        self.ready = [device.Event() for _ in range(self.depth)]
        self.free_ = [device.Event() for _ in range(self.depth)]

    # -------------------------------------------------------------- host side
    def host_tensor(self, layer: int, name: str) -> np.ndarray:
        """Writable uint8 view of one tensor's raw blocks in pinned memory."""
        s = next(t for t in self.slots if t.name == name)
        base = layer * self.layer_bytes + s.offset
        return self.host.array[base: base + s.nbytes]

    def fill(self, layer: int, blocks: dict) -> None:
        for name, raw in blocks.items():
            self.host_tensor(layer, name)[:] = np.asarray(raw, dtype=np.uint8).reshape(-1)

    # ------------------------------------------------------------ device side
    def step(self, x, y, compute_stream, y_stride: int = 0) -> None:
        """Enqueues one pass over all layers: every tensor's GEMV with input
        ``x`` (fp32, at least max k elements). Tensor t of layer L writes
        ``y + (L * len(tensors) + t) * y_stride`` bytes (``y_stride`` 0: all
        write ``y``). Returns after enqueueing; synchronise on
        ``compute_stream``."""
        xa, ya = device._addr(x), device._addr(y)
        for layer in range(self.n_layers):
            d = layer % self.depth
            self.copy_stream.wait(self.free_[d])               # slot released by layer - depth
            device.memcpy_h2d_async(self.dev[d].ptr, self.host.ptr + layer * self.layer_bytes,
                                    self.layer_bytes, self.copy_stream)
            self.ready[d].record(self.copy_stream)
            compute_stream.wait(self.ready[d])
            for t, s in enumerate(self.slots):
                yo = ya + (layer * len(self.slots) + t) * y_stride
                device.gemv(s.qtype, self.dev[d].ptr + s.offset, xa, yo, s.n, s.k, stream=compute_stream,
                            w_bytes=s.nbytes)
            self.free_[d].record(compute_stream)

    def close(self) -> None:
        for b in self.dev:
            b.free()
        self.host.free()
        for e in self.ready + self.free_:
            e.destroy()
        self.copy_stream.destroy()


def _layer_entry(item, position: int) -> tuple[object, list[str]]:
    """(layer key, tensor names) of a LayerDescriptor-like object (``.index``,
    ``.tensor_names``; runtime/scheduler.py), an (index, names) pair, or a
    plain list of names (key = its position)."""
    if hasattr(item, "tensor_names"):
        return getattr(item, "index", position), list(item.tensor_names)
    if isinstance(item, tuple) and len(item) == 2 and not isinstance(item[1], str):
        return item[0], list(item[1])
    return position, list(item)


class _Plan:
    """Which layer each ring entry holds, for SchedulerStream (no device
    calls; the caller holds its lock).

    Entries t = 0, 1, 2, ... are layer positions in streaming order; entry t
    lives in slot t % depth. ``cur`` is the entry being computed,
    ``claimed`` / ``done`` count the entries the worker has taken / finished,
    entries < ``released + 1`` are computed. The worker may take entry t
    once t - depth <= released (the slot's previous entry is computed) and
    the plan reaches t; the plan always reaches cur + depth - 1, continuing
    with the next positions and wrapping from the last layer to the first."""

    def __init__(self, n_layers: int, depth: int):
        self.n, self.depth = int(n_layers), int(depth)
        self.seq: list[int] = []
        self.cur = None
        self.claimed = self.done = 0
        self.released = -1
        self.restarts = 0

    def is_jump(self, p: int) -> bool:
        """True if a hook for position p neither repeats the current layer nor
        continues the plan (the next planned position, or the position after
        the current one): the worker must then finish its claimed entries
        before :meth:`advance`."""
        if self.cur is None:
            return True
        if self.seq[self.cur] == p:
            return False
        nxt = self.cur + 1
        if nxt < len(self.seq):
            return self.seq[nxt] != p
        return p != (self.seq[self.cur] + 1) % self.n

    def advance(self, p: int) -> list[int]:
        """The hook for position p: returns the entries released by it."""
        if self.cur is not None and self.seq[self.cur] == p:
            pass                                            # the same layer again
        elif not self.is_jump(p):
            if self.cur + 1 == len(self.seq):
                self.seq.append(p)
            self.cur += 1
        else:
            if self.done != self.claimed:
                raise RuntimeError("plan restarted while the worker holds entries")
            del self.seq[self.claimed:]
            self.seq.append(p)
            if self.cur is not None:
                self.restarts += 1
            self.cur = len(self.seq) - 1
        rel = list(range(max(self.released + 1, self.cur - self.depth), self.cur))
        self.released = max(self.released, self.cur - 1)
        while len(self.seq) < self.cur + self.depth:
            self.seq.append((self.seq[-1] + 1) % self.n)
        return rel

    def claimable(self) -> bool:
        return self.claimed < len(self.seq) and self.claimed - self.depth <= self.released

    def claim(self) -> tuple[int, int]:
        t = self.claimed
        self.claimed += 1
        return t, self.seq[t]


class SchedulerStream:
    """The layers of a GGUF file streamed to the GPU ahead of the reference's
    layer scheduler, through its prefetch hook.

    ``LayerScheduler`` (runtime/scheduler.py) calls its prefetch hook with
    each layer's descriptor right before acquiring that layer
    (``_maybe_prefetch``, scheduler.py:191-198, 270-277, from ``run`` and
    ``step``), then runs the forwarder on the layer's handles, whose
    projections reach the backend's matmuls as host arrays. Bound with
    :meth:`bind` (``set_prefetch_hook(stream.hook)`` plus the backend's
    ``attach_stream``), this class keeps the current layer and the next
    ``depth - 1`` layers of the execution order (wrapping from the last layer
    to the first: the next decode step) in a ring of ``depth`` device slots:

    * a worker thread streams each layer's quantized tensors from the file
      mapping (zero-copy views, ``GGUFFile.raw``) through two pinned staging
      slots (:class:`StagedCopier`) on a copy stream into the layer's slot,
      once the layer that last used the slot is released (the hook for a
      later layer: the scheduler computes layers one at a time and the
      backend's matmuls return only when their results are on the host);
    * the backend's matmul looks its weight up by content
      (:func:`flatrun_amd.residency.content_key`: the reference hands over
      fresh copies of the mapping's bytes) among the current layer's
      tensors, waits for that layer's copy and computes from the slot.
      Weights not streamed (other layers' tensors, the embedding, the LM
      head, anything not quantized) go the backend's usual way.

    A hook call for a layer other than the planned next one (``step`` with
    an arbitrary index) restarts the plan at that layer. Host memory held:
    the two staging slots; device memory: ``depth`` slots of the largest
    layer. One scheduler drives a stream at a time."""

    def __init__(self, gguf, layers, *, depth: int = 3, staging_bytes: int = 64 << 20,
                 copy_threads: int | None = None):
        from . import DeviceWeight
        from .gguf import GGUFFile

        self._DeviceWeight = DeviceWeight
        own = not isinstance(gguf, GGUFFile)
        self.file = GGUFFile(gguf) if own else gguf
        self._own_file = own
        self._slots, self._ready, self._free = [], [], []
        self._copier = None
        self._copy = None
        self._thread = None
        try:
            self._layers = []       # (layer key, [(name, offset, nbytes)], bytes) in execution order
            for p, item in enumerate(layers):
                key, names = _layer_entry(item, p)
                plan, off = [], 0
                for name in names:
                    if name not in self.file:
                        continue
                    info = self.file.info(name)
                    if info.quantization is None:
                        continue
                    plan.append((name, off, info.nbytes))
                    off += _align(info.nbytes)
                self._layers.append((key, plan, off))
            if not self._layers:
                raise ValueError("SchedulerStream needs at least one layer")
            self._pos = {key: p for p, (key, _, _) in enumerate(self._layers)}
            self._sizes = [frozenset(nb for _, _, nb in plan) for _, plan, _ in self._layers]
            self.slot_bytes = max(ALIGN, max(b for _, _, b in self._layers))
            self.depth = max(1, min(int(depth), len(self._layers)))
            self._slots = [device.DeviceBuffer(self.slot_bytes) for _ in range(self.depth)]
            self._ready = [device.Event() for _ in range(self.depth)]
            self._free = [device.Event() for _ in range(self.depth)]
            for e in self._free:
                e.record(None)
            self._copy = device.Stream()
            self._copier = StagedCopier(staging_bytes, copy_threads)
        except BaseException:
            self.close()
            raise
        self._keys: dict[str, tuple] = {}   # tensor name -> content key, computed once
        self._cv = threading.Condition()
        self._plan = _Plan(len(self._layers), self.depth)
        self._pub: dict[int, dict] = {}  # entry -> {content key: DeviceWeight}
        self._closed = False
        self.error = None
        self.stats = {"layers_streamed": 0, "bytes_streamed": 0, "hits": 0, "misses": 0, "restarts": 0}
        self._thread = threading.Thread(target=self._worker, name="frq-layer-stream", daemon=True)
        self._thread.start()

    @classmethod
    def bind(cls, scheduler, gguf, backend=None, **kw) -> "SchedulerStream":
        """A stream over ``scheduler``'s layers (``layer_count`` / ``layer``,
        scheduler.py:245-249) installed as its prefetch hook
        (``set_prefetch_hook``, scheduler.py:191-198) and, given the
        flatrun_amd backend, attached to it."""
        layers = [scheduler.layer(i) for i in range(scheduler.layer_count())]
        st = cls(gguf, layers, **kw)
        scheduler.set_prefetch_hook(st.hook)
        if backend is not None:
            backend.attach_stream(st)
        return st

    # ------------------------------------------------------------ scheduler
    def hook(self, layer) -> None:
        """The prefetch hook: `layer` (a descriptor with ``.index``, or the
        key given at construction) is about to be computed."""
        p = self._pos.get(getattr(layer, "index", layer))
        if p is None:
            return
        with self._cv:
            if self._closed:
                return
            pl = self._plan
            if pl.is_jump(p):            # plan again from p once the worker's copies are enqueued
                while pl.done < pl.claimed and self.error is None:
                    self._cv.wait()
                if self.error is not None:
                    return
            for t in pl.advance(p):
                # computed entries: their slots may be refilled once the null
                # stream (the backend's matmuls) has passed this point
                self._free[t % self.depth].record(None)
            self.stats["restarts"] = pl.restarts
            self._cv.notify_all()

    # ------------------------------------------------------------- backend
    def lookup(self, raw: np.ndarray):
        """The device copy of host weight `raw` if it is a tensor of the
        current layer (after that layer's copy has finished), else None.
        A weight whose byte count no tensor of the current layer has (the
        embedding, the LM head, another layer's odd-sized tensor) returns
        None before any hashing; the others are identified by content."""
        from .residency import content_key

        with self._cv:
            if self._plan.cur is None or self._closed:
                return None
            p = self._plan.seq[self._plan.cur] if self._plan.cur < len(self._plan.seq) else None
        if p is not None and int(raw.nbytes) not in self._sizes[p]:
            with self._cv:
                self.stats["misses"] += 1
            return None
        key = content_key(raw.reshape(-1))
        with self._cv:
            t = self._plan.cur
            while self._plan.done <= t and self.error is None and not self._closed:
                self._cv.wait()
            ent = self._pub.get(t)
            dw = ent.get(key) if ent is not None else None
            self.stats["hits" if dw is not None else "misses"] += 1
            ev = self._ready[t % self.depth] if dw is not None else None
        if ev is not None:
            ev.synchronize()
        return dw

    # -------------------------------------------------------------- worker
    def _worker(self) -> None:
        from .residency import digest

        try:
            while True:
                with self._cv:
                    while not self._closed and not self._plan.claimable():
                        self._cv.wait()
                    if self._closed:
                        return
                    t, p = self._plan.claim()
                    self._pub.pop(t - self.depth, None)     # the slot's previous layer leaves the lookups
                d = t % self.depth
                _, plan, nbytes = self._layers[p]
                self._copy.wait(self._free[d])
                base = self._slots[d]
                entries = {}
                for name, off, nb in plan:
                    src = self.file.raw(name)
                    self._copier.copy(base.ptr + off, src, self._copy)
                    key = self._keys.get(name)
                    if key is None:
                        key = self._keys[name] = (int(src.nbytes), digest(src))
                    info = self.file.info(name)
                    entries[key] = self._DeviceWeight.view(base, off, nb, qtype=info.type_name, shape=info.shape,
                                                           name=name)
                self._ready[d].record(self._copy)
                with self._cv:
                    self._pub[t] = entries
                    self._plan.done = t + 1
                    self.stats["layers_streamed"] += 1
                    self.stats["bytes_streamed"] += sum(nb for _, _, nb in plan)
                    self._cv.notify_all()
        except BaseException as e:      # surfaced through .error; lookups then miss
            with self._cv:
                self.error = e
                self._cv.notify_all()

    def close(self) -> None:
        if getattr(self, "_cv", None) is not None:
            with self._cv:
                self._closed = True
                self._cv.notify_all()
        if self._thread is not None:
            self._thread.join()
            self._thread = None
        if self._copy is not None:
            self._copy.synchronize()
        if self._copier is not None:
            self._copier.close()
            self._copier = None
        for b in self._slots:
            b.free()
        for e in self._ready + self._free:
            e.destroy()
        self._slots, self._ready, self._free = [], [], []
        if self._copy is not None:
            self._copy.destroy()
            self._copy = None
        if self._own_file and self.file is not None:
            self.file.close()
        self.file = None

    def __enter__(self) -> "SchedulerStream":
        return self

    def __exit__(self, *exc) -> None:
        self.close()
