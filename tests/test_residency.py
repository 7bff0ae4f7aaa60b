"""Host logic of weight identity (flatrun_amd.residency) and of the
scheduler stream's plan (flatrun_amd.streaming._Plan); no GPU needed."""

from __future__ import annotations

import mmap

import numpy as np
import pytest

from flatrun_amd import residency
from flatrun_amd.streaming import _Plan


@pytest.fixture
def mapped(tmp_path):
    data = np.random.default_rng(0).integers(0, 256, 3 << 20, dtype=np.uint8)
    p = tmp_path / "w.bin"
    p.write_bytes(data.tobytes())
    f = open(p, "rb")
    mm = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
    yield data, mm, p
    mm.close()
    f.close()


def test_reference_handle_views_are_copies(mapped):
    """What MmapTensorHandle.view does (core/tensor.py:240-247): an ndarray
    over ``mmap[a:b]``, which is bytes -- a new buffer per call."""
    data, mm, _ = mapped
    a = np.ndarray(shape=(1000,), dtype=np.uint8, buffer=mm[64:1064])
    b = np.ndarray(shape=(1000,), dtype=np.uint8, buffer=mm[64:1064])
    assert a.ctypes.data != b.ctypes.data
    assert not residency.file_backed(a)
    assert residency.content_key(a) == residency.content_key(b) == residency.content_key(data[64:1064].copy())


def test_file_backed_detection(mapped):
    data, mm, path = mapped
    assert residency.file_backed(np.frombuffer(mm, dtype=np.uint8, count=100, offset=8))
    assert residency.file_backed(np.ndarray(shape=(10,), dtype=np.uint8, buffer=memoryview(mm)[8:18]))
    assert residency.file_backed(np.memmap(path, dtype=np.uint8, mode="r")[5:50])
    assert residency.file_backed(np.frombuffer(mm, dtype=np.uint8).reshape(-1, 1024)[3:7])
    assert not residency.file_backed(data)
    assert not residency.file_backed(data[10:20])


def test_digest_content_and_order():
    rng = np.random.default_rng(1)
    c = 1 << 20
    big = rng.integers(0, 256, 3 * c + 1234, dtype=np.uint8)
    k0 = residency.content_key(big)
    assert k0 == residency.content_key(big.copy()) and k0[0] == big.size
    swapped = np.concatenate([big[c:2 * c], big[:c], big[2 * c:]])
    assert residency.content_key(swapped) != k0                  # order is part of the digest
    flip = big.copy()
    flip[-1] ^= 1
    assert residency.content_key(flip) != k0
    assert residency.content_key(big[:-1]) != k0                 # the size is part of the key
    small = rng.integers(0, 256, 1000, dtype=np.uint8)
    assert residency.content_key(small) != residency.content_key(small[::-1].copy())


def test_key_memo_hashes_file_backed_views_once(mapped, monkeypatch):
    _, mm, _ = mapped
    calls = []
    real = residency.digest
    monkeypatch.setattr(residency, "digest", lambda a: calls.append(a.nbytes) or real(a))
    memo = residency.KeyMemo(limit=2)
    v = np.frombuffer(mm, dtype=np.uint8, count=4096, offset=0)
    k1, k2 = memo.key(v), memo.key(np.frombuffer(mm, dtype=np.uint8, count=4096, offset=0))
    assert k1 == k2 and calls == [4096]                     # same (address, size): hashed once
    copy = np.ndarray(shape=(4096,), dtype=np.uint8, buffer=mm[0:4096])
    assert memo.key(copy) == k1 and memo.key(copy) == k1 and calls == [4096] * 3   # copies: every call
    for off in (4096, 8192, 12288):                          # LRU bound
        memo.key(np.frombuffer(mm, dtype=np.uint8, count=4096, offset=off))
    assert memo.entries() == 2


def test_key_memo_holds_no_mapping(tmp_path):
    """The memo keeps neither the arrays nor their mapping: once the views
    are gone the file closes (a GGUF file's close is not blocked), and a
    collected mapping takes its entries with it."""
    import gc

    p = tmp_path / "m.bin"
    p.write_bytes(bytes(range(256)) * 64)
    f = open(p, "rb")
    mm = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
    memo = residency.KeyMemo()
    v = np.frombuffer(mm, dtype=np.uint8, count=1024, offset=2048)
    k = memo.key(v)
    assert k == (1024, residency.digest(np.frombuffer(bytes(range(256)) * 4, dtype=np.uint8)))
    assert memo.entries() == 1
    del v
    mm.close()                                               # no BufferError: nothing of the memo holds it
    f.close()
    del mm
    gc.collect()
    assert memo.entries() == 0


class _FakeBuf:
    def __init__(self):
        self.freed = False

    def free(self):
        self.freed = True


class _FakeDW:
    def __init__(self, raw):
        self.nbytes = raw.nbytes
        self.buffer = _FakeBuf()


def test_weight_cache_by_content():
    rng = np.random.default_rng(2)
    a, b, c = (rng.integers(0, 256, 1000, dtype=np.uint8) for _ in range(3))
    cache = residency.WeightCache(2000)
    da = cache.lookup(a, _FakeDW)
    assert cache.lookup(a.copy(), _FakeDW) is da                # fresh copy of the same bytes: a hit
    a2 = a.copy()
    a2.flags.writeable = False
    assert cache.lookup(a2, _FakeDW) is da
    assert (cache.hits, cache.misses, len(cache)) == (2, 1, 1)
    db = cache.lookup(b, _FakeDW)
    cache.lookup(a, _FakeDW)                                     # a most recent
    cache.lookup(c, _FakeDW)                                     # evicts b
    assert db.buffer.freed and not da.buffer.freed and len(cache) == 2 and cache.bytes == 2000
    assert cache.lookup(np.zeros(3000, np.uint8), _FakeDW) is None   # larger than the cache
    assert cache.lookup(np.zeros(0, np.uint8), _FakeDW) is None
    cache.clear()
    assert da.buffer.freed and len(cache) == 0 and cache.bytes == 0


def test_weight_cache_keeps_held_entries():
    """A grouped call looks up each part before its one launch: a later
    part's lookup must not evict (free) an earlier part of the same call,
    even when the parts together exceed the capacity; it then returns None
    (the caller uploads that part for the call alone) and frees nothing."""
    rng = np.random.default_rng(3)
    a, b, c = (rng.integers(0, 256, 1000, dtype=np.uint8) for _ in range(3))
    cache = residency.WeightCache(1500)
    da = cache.lookup(a, _FakeDW)
    assert cache.lookup(b, _FakeDW, held=[da]) is None          # no room beside the held entry
    assert not da.buffer.freed and len(cache) == 1 and cache.bytes == 1000
    db = cache.lookup(b, _FakeDW)                               # nothing held: a is evicted
    assert da.buffer.freed and len(cache) == 1
    cache2 = residency.WeightCache(2500)
    d1, d2 = cache2.lookup(a, _FakeDW), cache2.lookup(b, _FakeDW)
    d3 = cache2.lookup(c, _FakeDW, held=[d1])                   # evicts the unheld b, keeps a
    assert d3 is not None and not d1.buffer.freed and d2.buffer.freed and cache2.bytes == 2000
    assert db is not None


def _drive(plan, p):
    """A hook call; the worker is assumed idle (done == claimed)."""
    return plan.advance(p)


def _work(plan):
    out = []
    while plan.claimable():
        out.append(plan.claim())
    plan.done = plan.claimed
    return out


def test_plan_sequential_and_wrap():
    pl = _Plan(n_layers=5, depth=3)
    assert pl.is_jump(0) and _drive(pl, 0) == []
    assert pl.seq == [0, 1, 2] and _work(pl) == [(0, 0), (1, 1), (2, 2)]
    assert not pl.is_jump(1)
    assert _drive(pl, 1) == [0]                    # layer 0 computed: its slot is released
    assert _work(pl) == [(3, 3)]                   # entry 3 reuses slot 0
    for p in (2, 3, 4):
        _drive(pl, p)
        _work(pl)
    assert pl.seq == [0, 1, 2, 3, 4, 0, 1]         # the next decode step is prefetched
    assert not pl.is_jump(0)
    assert _drive(pl, 0) == [4] and pl.cur == 5 and pl.restarts == 0
    assert pl.claimed == 7                          # cur + depth - 1 = 7 entries claimed before
    assert _work(pl) == [(7, 2)]


def test_plan_slot_never_reused_before_release():
    pl = _Plan(n_layers=8, depth=2)
    _drive(pl, 0)
    assert _work(pl) == [(0, 0), (1, 1)]
    assert not pl.claimable()                      # entry 2 would overwrite layer 0's slot
    _drive(pl, 1)
    assert _work(pl) == [(2, 2)]
    for step in range(40):
        p = pl.seq[pl.cur + 1]
        for t in range(pl.claimed):
            # every claimed entry's slot predecessor is released
            assert t - pl.depth <= pl.released
        _drive(pl, p)
        _work(pl)
        assert pl.claimed <= pl.cur + pl.depth


def test_plan_jump_and_repeat():
    pl = _Plan(n_layers=6, depth=3)
    _drive(pl, 0)
    _work(pl)
    assert _drive(pl, 0) == [] and pl.cur == 0     # the same layer again: nothing changes
    assert pl.is_jump(4)
    rel = _drive(pl, 4)                            # step(4): plan again from layer 4
    assert pl.restarts == 1 and pl.seq[pl.cur] == 4 and pl.cur == 3
    assert rel == [0, 1, 2] and pl.released == 2   # prefetched, never used: released
    assert pl.seq[3:6] == [4, 5, 0]
    assert _work(pl) == [(3, 4), (4, 5), (5, 0)]
    pl.claimed += 1                                # a worker in the middle of an entry
    with pytest.raises(RuntimeError):
        pl.advance(2)


def test_plan_depth_one_continues():
    """depth 1 holds only the current layer: the next position still
    continues the plan (no restart), and its slot is released first."""
    pl = _Plan(n_layers=3, depth=1)
    _drive(pl, 0)
    assert _work(pl) == [(0, 0)]
    for i in range(1, 7):
        assert not pl.is_jump(i % 3)
        assert _drive(pl, i % 3) == [i - 1]
        assert _work(pl) == [(i, i % 3)]
    assert pl.restarts == 0 and pl.seq == [0, 1, 2, 0, 1, 2, 0]
    assert pl.is_jump(2)


def test_plan_single_layer_stays_resident():
    pl = _Plan(n_layers=1, depth=1)
    _drive(pl, 0)
    _work(pl)
    for _ in range(5):
        assert _drive(pl, 0) == [] and not pl.claimable()
    assert pl.claimed == 1 and pl.restarts == 0
