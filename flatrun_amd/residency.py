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


def file_backed(raw: np.ndarray) -> bool:
    """True when the array's memory belongs to an ``mmap.mmap`` that the
    array keeps alive (through ``.base`` / ``memoryview.obj`` links)."""
    o = raw
    for _ in range(16):
        o = o.obj if isinstance(o, memoryview) else getattr(o, "base", None)
        if o is None:
            return False
        if isinstance(o, mmap.mmap):
            return True
    return False


class KeyMemo:
    """Content keys of file-backed arrays by (address, nbytes). Each entry
    holds its array, so the mapping behind an address stays in place (and
    holds those bytes) while the entry lives; at most `limit` entries, least
    recently used out."""

    def __init__(self, limit: int = 4096):
        self.limit = int(limit)
        self._m: collections.OrderedDict = collections.OrderedDict()
        self._lock = threading.Lock()

    def key(self, raw: np.ndarray) -> tuple[int, bytes]:
        flat = raw.reshape(-1)
        if flat.nbytes and not raw.flags.writeable and file_backed(raw):
            addr = (int(flat.ctypes.data), int(flat.nbytes))
            with self._lock:
                hit = self._m.get(addr)
                if hit is not None:
                    self._m.move_to_end(addr)
                    return hit[1]
            k = (int(flat.nbytes), digest(flat))
            with self._lock:
                self._m[addr] = (raw, k)
                while len(self._m) > self.limit:
                    self._m.popitem(last=False)
            return k
        return (int(flat.nbytes), digest(flat))


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

    def lookup(self, raw: np.ndarray, upload):
        """The resident copy of `raw`, made by ``upload(raw)`` on a miss;
        None if `raw` is empty or larger than the whole cache."""
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
        while self._entries and self.bytes + flat.nbytes > self.capacity:
            _, old = self._entries.popitem(last=False)
            self.bytes -= old.nbytes
            old.buffer.free()
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
