"""The snapshot store's bookkeeping on the CPU (no tensors touched): cumulative chunk keys, the first-fit row
allocator, and the reference's eviction rule (state_cache.py:95-104): only leaves go, least recently used first, so
every snapshot's ancestors stay; a resumed path is never evicted to make room for its own child."""
import hashlib

import pytest
import torch

from opendecider_amd.state_cache import RangeAllocator, SnapshotTree, chunk_keys


def test_chunk_keys_are_cumulative_and_type_consistent():
    keys = chunk_keys(["a", "bc", "d"])
    h = hashlib.sha1()
    for c in ["a", "bc", "d"]:
        h.update(hashlib.sha1(c.encode()).digest())
    assert keys[-1] == h.hexdigest() and len(set(keys)) == 3
    assert chunk_keys(["a", "bc"]) == keys[:2]                      # a prefix's keys are the prefix of the keys
    assert chunk_keys(["ab", "c", "d"])[-1] != keys[-1]             # chunk boundaries matter
    t = [torch.tensor([1, 2, 3]), torch.tensor([4])]
    assert chunk_keys(t) == chunk_keys([x.to(torch.int32) for x in t])


def test_range_allocator_first_fit_and_coalescing():
    r = RangeAllocator(100)
    a, b, c = r.alloc(30), r.alloc(30), r.alloc(30)
    assert (a, b, c) == (0, 30, 60) and r.alloc(20) is None and r.free_rows() == 10
    r.release(b, 30)
    assert r.alloc(40) is None and r.alloc(25) == 30               # first fit inside the hole
    r.release(a, 30)
    r.release(30, 25)
    assert r.free == [(0, 60), (90, 10)]                           # coalesced back into one run
    with pytest.raises(ValueError):
        r.release(10, 5)                                           # a double free overlaps a free run


def test_eviction_takes_lru_leaves_and_keeps_ancestors():
    t = SnapshotTree(100)
    root = t.add("r", None, 40)                                    # rows 0..39
    a = t.add("a", root, 60)                                       # 20 own rows
    b = t.add("b", root, 70)                                       # 30 own rows
    assert root.children == 2 and t.rows.free_rows() == 10
    t.touch(a)                                                     # b is now the least recently used leaf
    c = t.add("c", a, 85)                                          # needs 25 rows: evicts b (LRU leaf), not root
    assert "b" not in t and "r" in t and c.start == 60
    assert root.children == 1 and a.children == 1
    with pytest.raises(MemoryError):                               # only c is evictable, and c's path is protected
        t.add("d", c, 130)
    assert "c" in t and "a" in t and "r" in t                      # the failed add evicted nothing on the path
    assert t.deepest(["r", "a", "c", "zz"]) == 2 and t.deepest(["x"]) == -1
    t.remove(c)
    t.remove(a)
    assert root.children == 0 and t.rows.free_rows() == 60
