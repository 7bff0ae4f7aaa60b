"""Identity of host weight buffers, for device copies reused across calls.

The reference's forwarder hands the backend ``handle.as_numpy()`` for every
projection (model/qwen2.py:709, runtime/backend.py:251-257). For an mmap
handle that array is NOT a view of the file mapping: ``MmapTensorHandle.view``
(core/tensor.py:227-267) slices an ``mmap.mmap``, and slicing an mmap returns
``bytes`` -- a fresh copy at a fresh address on every call. A device copy
keyed by the array's address would therefore never be found again, and
holding the array to keep its address valid would pin a host copy of every
weight. So a weight is identified by its content:

  key = (nbytes, 128-bit xxh3 of the bytes)    (hashlib.blake2b-128 where the
                                                xxhash module is missing)

in one pass (about 15 GB/s on one core here; the module holds the GIL, so
splitting the pass over threads gains nothing). Arrays whose memory belongs
to a file mapping that they keep alive (``np.frombuffer(mmap)``,
``np.memmap``, a zero-copy view through ``memoryview(mmap)``) have a stable
address for as long as they live, so their key is computed once and then
found by (address, nbytes) while a reference to the array is held -- no
per-call hash. The hash is not cryptographic: the key identifies weights
of a model file the caller loads, not bytes chosen by an adversary to
collide.
"""

from __future__ import annotations

import collections
import hashlib
import mmap
import threading
import weakref

import numpy as np

try:
    import xxhash as _xxhash
except ImportError:          # pragma: no cover - the image ships xxhash
    _xxhash = None


def digest(raw: np.ndarray) -> bytes:
    """128-bit digest of a contiguous array's bytes."""
    flat = np.ascontiguousarray(raw).reshape(-1).view(np.uint8)
    if _xxhash is not None:
        return _xxhash.xxh3_128_digest(flat)
    return hashlib.blake2b(flat, digest_size=16).digest()


def _backing_mmap(raw: np.ndarray):
    """The ``mmap.mmap`` whose memory the array views and keeps alive
    (through ``.base`` / ``memoryview.obj`` links), else None."""
    o = raw
    for _ in range(16):
        o = o.obj if isinstance(o, memoryview) else getattr(o, "base", None)
        if o is None:
            return None
        if isinstance(o, mmap.mmap):
            return o
    return None


def file_backed(raw: np.ndarray) -> bool:
    """True when the array's memory belongs to an ``mmap.mmap`` that the
    array keeps alive."""
    return _backing_mmap(raw) is not None


class KeyMemo:
    """Content keys of file-backed arrays by (mapping, offset, nbytes).

    The memo holds no array and no mapping: entries are grouped per mapping
    in a weak-keyed table, so a mapping closed and collected takes its
    entries with it, and closing a GGUF file is never blocked by the memo.
    While an array over a mapping lives, the mapping cannot be closed, so the
    bytes at an offset are the bytes that were hashed -- provided the file
    is not rewritten on disk while it is mapped (a shared mapping shows such
    writes, and the memo would then serve the old key). At most `limit`
    entries per mapping, least recently used out."""

    def __init__(self, limit: int = 4096):
        self.limit = int(limit)
        self._m: "weakref.WeakKeyDictionary[mmap.mmap, collections.OrderedDict]" = weakref.WeakKeyDictionary()
        self._lock = threading.Lock()

    def key(self, raw: np.ndarray) -> tuple[int, bytes]:
        flat = raw.reshape(-1)
        mm = _backing_mmap(raw) if flat.nbytes and not raw.flags.writeable else None
        if mm is None:
            return (int(flat.nbytes), digest(flat))
        probe = np.frombuffer(mm, np.uint8, count=1)     # the mapping's base address (a transient export)
        at = (int(flat.ctypes.data) - int(probe.ctypes.data), int(flat.nbytes))
        del probe
        with self._lock:
            table = self._m.get(mm)
            hit = table.get(at) if table is not None else None
            if hit is not None:
                table.move_to_end(at)
                return hit
        k = (int(flat.nbytes), digest(flat))
        with self._lock:
            table = self._m.setdefault(mm, collections.OrderedDict())
            table[at] = k
            while len(table) > self.limit:
                table.popitem(last=False)
        return k

    def entries(self) -> int:
        with self._lock:
            return sum(len(t) for t in self._m.values())


_memo = KeyMemo()


def content_key(raw: np.ndarray) -> tuple[int, bytes]:
    """(nbytes, digest) of a host weight array; see the module docstring."""
    return _memo.key(raw)


class WeightCache:
    """Device copies of host weights by content key, least recently used out.

    No host memory is held for an entry: the key is the content, so a host
    buffer freed and reused for other bytes gets another key."""

    def __init__(self, capacity: int):
        self.capacity = int(capacity)
        self.bytes = 0
        self.hits = self.misses = 0
        self._entries: collections.OrderedDict = collections.OrderedDict()

    def lookup(self, raw: np.ndarray, upload, held=()):
        """The resident copy of `raw`, made by ``upload(raw)`` on a miss;
        None if `raw` is empty or larger than the whole cache, or if the
        entries in `held` leave no room for it.

        Eviction frees device memory at once. `held` names the entries the
        caller has already looked up for a launch it has not run yet (the
        parts of a grouped call): they are never evicted here, so a group
        whose parts together exceed the capacity caches what fits and the
        caller uploads the rest for that call alone."""
        flat = raw.reshape(-1)
        if flat.nbytes == 0 or flat.nbytes > self.capacity:
            return None
        key = content_key(flat)
        hit = self._entries.get(key)
        if hit is not None:
            self._entries.move_to_end(key)
            self.hits += 1
            return hit
        self.misses += 1
        keep = {id(h) for h in held if h is not None}
        if self.bytes + flat.nbytes > self.capacity:
            for old_key in list(self._entries):               # least recently used first
                if self.bytes + flat.nbytes <= self.capacity:
                    break
                old = self._entries[old_key]
                if id(old) in keep:
                    continue
                del self._entries[old_key]
                self.bytes -= old.nbytes
                old.buffer.free()
            if self.bytes + flat.nbytes > self.capacity:
                return None
        dw = upload(flat)
        self._entries[key] = dw
        self.bytes += flat.nbytes
        return dw

    def __len__(self) -> int:
        return len(self._entries)

    def clear(self) -> None:
        for dw in self._entries.values():
            dw.buffer.free()
        self._entries.clear()
        self.bytes = 0
