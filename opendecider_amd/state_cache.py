"""Snapshots of growing int8 states with exact resume: the snapshot core of the reference's PrefixCache
(src/opendecider/state_cache.py:32-124) on an append-only device arena.

A snapshot marks a prefix boundary of a state and stores the int8 K/V (bytes and fp32 scales, every layer) of ITS OWN
tokens only, a delta over its parent (state_cache.py:68-93). A request resumes from its deepest cached prefix: the
deltas along the snapshot's path are copied back into a working StateKV and only the rest is prefilled. Only leaves
are evicted, least recently used first, so every snapshot's ancestors stay present (state_cache.py:95-104).

Different from the reference on purpose: the reference restores by dequantizing every delta, concatenating and
quantizing again (state_cache.py:106-124 and the pack at :154); here the stored bytes go back unchanged, so a resumed
state is bit-identical to the one the snapshot was taken from. Taking and restoring are one kernel launch each
(od_kv_copy_rows) for all layers, K and V.

Storage: one arena per store, q int8 (2 L, Hkv, cap, D) and scale fp32 (2 L, Hkv, cap), the layout of one state of a
StateKV; a snapshot owns a run of arena rows, handed out first-fit from a free list. The attention reads the working
StateKV, never the arena.
"""
from __future__ import annotations

import hashlib
import time
from collections import OrderedDict
from dataclasses import dataclass, field

import torch

from . import kernels
from .kv_cache import StateKV


def chunk_keys(chunks) -> list[str]:
    """Cumulative content keys: keys[i] identifies chunks[:i+1] (each chunk a str, bytes or a 1-D token-id tensor);
    the reference's scheme (state_cache.py:51-57): a running SHA-1 over the chunks' own SHA-1 digests."""
    keys, h = [], hashlib.sha1()
    for c in chunks:
        if isinstance(c, torch.Tensor):
            c = c.detach().to("cpu", torch.int64).contiguous().numpy().tobytes()
        elif isinstance(c, str):
            c = c.encode()
        h.update(hashlib.sha1(c).digest())
        keys.append(h.copy().hexdigest())
    return keys


class RangeAllocator:
    """First-fit allocator of row runs in [0, capacity), with coalescing frees."""

    def __init__(self, capacity: int):
        self.capacity = capacity
        self.free = [(0, capacity)]                  # sorted disjoint (start, length)

    def alloc(self, n: int) -> int | None:
        for i, (s, ln) in enumerate(self.free):
            if ln >= n:
                if ln == n:
                    del self.free[i]
                else:
                    self.free[i] = (s + n, ln - n)
                return s
        return None

    def release(self, start: int, n: int) -> None:
        if n == 0:
            return
        runs = sorted(self.free + [(start, n)])
        merged = []
        for s, ln in runs:
            if merged and merged[-1][0] + merged[-1][1] > s:
                raise ValueError(f"RangeAllocator: run ({start}, {n}) overlaps a free run")
            if merged and merged[-1][0] + merged[-1][1] == s:
                merged[-1] = (merged[-1][0], merged[-1][1] + ln)
            else:
                merged.append((s, ln))
        self.free = merged

    def free_rows(self) -> int:
        return sum(ln for _, ln in self.free)


@dataclass(eq=False)                                 # identity semantics: snapshots go into sets
class Snapshot:
    key: str
    parent: "Snapshot | None"
    n_tokens: int                                    # tokens of the state up to this boundary
    start: int                                       # arena row of this snapshot's first own token
    children: int = 0
    last_used: float = field(default_factory=time.monotonic)

    @property
    def n0(self) -> int:
        """Tokens before this snapshot's own ones (its parent's boundary)."""
        return self.parent.n_tokens if self.parent is not None else 0

    @property
    def n_own(self) -> int:
        return self.n_tokens - self.n0

    def path(self) -> list["Snapshot"]:
        """Root first."""
        out, s = [], self
        while s is not None:
            out.append(s)
            s = s.parent
        return out[::-1]


class SnapshotTree:
    """The bookkeeping of a snapshot store, independent of any tensor: keys, parents, children counts, LRU order
    (state_cache.py:32-48,95-104) and arena rows."""

    def __init__(self, capacity_rows: int):
        self.snaps: OrderedDict[str, Snapshot] = OrderedDict()   # least recently used first
        self.rows = RangeAllocator(capacity_rows)

    def __contains__(self, key: str) -> bool:
        return key in self.snaps

    def __len__(self) -> int:
        return len(self.snaps)

    def deepest(self, keys: list[str]) -> int:
        """Index of the last key present, or -1."""
        return next((i for i in range(len(keys) - 1, -1, -1) if keys[i] in self.snaps), -1)

    def touch(self, snap: Snapshot) -> None:
        for p in snap.path():
            self.snaps.move_to_end(p.key)
            p.last_used = time.monotonic()

    def evict_one(self, protect=()) -> Snapshot | None:
        """Drop the least recently used leaf not in `protect`; returns it (None if there is none)."""
        leaf = next((s for s in self.snaps.values() if s.children == 0 and s not in protect), None)
        if leaf is not None:
            self.remove(leaf)
        return leaf

    def remove(self, snap: Snapshot) -> None:
        if snap.children:
            raise ValueError(f"snapshot {snap.key[:8]} has children")
        del self.snaps[snap.key]
        self.rows.release(snap.start, snap.n_own)
        if snap.parent is not None:
            snap.parent.children -= 1

    def add(self, key: str, parent: Snapshot | None, n_tokens: int) -> Snapshot:
        """Allocate arena rows for a new snapshot, evicting LRU leaves (never `parent`'s path) as needed."""
        if key in self.snaps:
            raise KeyError(f"snapshot {key[:8]} exists")
        n0 = parent.n_tokens if parent is not None else 0
        n = n_tokens - n0
        if n < 0:
            raise ValueError(f"snapshot at {n_tokens} tokens lies before its parent's boundary {n0}")
        protect = set(parent.path()) if parent is not None else set()
        start = self.rows.alloc(n)
        while start is None:
            if self.evict_one(protect) is None:
                raise MemoryError(f"snapshot store: no room for {n} rows ({self.rows.free_rows()} free, fragmented "
                                  f"or held by the resumed path)")
            start = self.rows.alloc(n)
        s = Snapshot(key, parent, n_tokens, start)
        if parent is not None:
            parent.children += 1
        self.snaps[key] = s
        return s


class Int8PrefixCache:
    """Snapshots of one-state int8 K/V on an arena of `capacity_rows` token rows (every layer, K and V).

    take(state, b, key, parent, n_tokens)  copies state b's rows parent.n_tokens .. n_tokens into a new snapshot
    restore(snap, state, b)                 writes the snapshot's path back into state b, sets the state's length
    encode(dec, chunks, state)              the reference's resume-then-prefill flow (state_cache.py:127-163) on
                                            token-id chunks: restore the deepest cached prefix, prefill the rest,
                                            snapshot the end; returns the number of tokens served from the store
    """

    def __init__(self, n_layers: int, n_heads: int, head_dim: int, capacity_rows: int, device):
        self.q = torch.zeros(2 * n_layers, n_heads, capacity_rows, head_dim, dtype=torch.int8, device=device)
        self.scale = torch.zeros(2 * n_layers, n_heads, capacity_rows, dtype=torch.float32, device=device)
        self.tree = SnapshotTree(capacity_rows)
        self.stats = {"hit_tokens": 0, "new_tokens": 0, "requests": 0}

    def _check(self, state: StateKV) -> None:
        if state.q.shape[0] != self.q.shape[0] or state.q.shape[2] != self.q.shape[1] or \
                state.q.shape[4] != self.q.shape[3]:
            raise ValueError("Int8PrefixCache: the state's layers / heads / head_dim differ from the store's")

    def take(self, state: StateKV, b: int, key: str, parent: Snapshot | None, n_tokens: int) -> Snapshot:
        self._check(state)
        if n_tokens > state.length:
            raise ValueError(f"snapshot at {n_tokens} tokens but the state holds {state.length}")
        snap = self.tree.add(key, parent, n_tokens)
        sq, ss = state.state(b)
        kernels.kv_copy_rows(sq, ss, self.q, self.scale, [(snap.n0, snap.start, snap.n_own)])
        return snap

    def restore(self, snap: Snapshot, state: StateKV, b: int) -> None:
        self._check(state)
        if snap.n_tokens > state.capacity:
            raise ValueError(f"snapshot of {snap.n_tokens} tokens exceeds the state's capacity {state.capacity}")
        path = snap.path()
        dq, ds = state.state(b)
        kernels.kv_copy_rows(self.q, self.scale, dq, ds, [(p.start, p.n0, p.n_own) for p in path])
        state.set_length(snap.n_tokens)
        self.tree.touch(snap)

    def lookup(self, keys: list[str]) -> tuple[int, Snapshot | None]:
        i = self.tree.deepest(keys)
        return i, (self.tree.snaps[keys[i]] if i >= 0 else None)

    def encode(self, dec, chunks: list[torch.Tensor], state: StateKV, piece: int = 256) -> int:
        """chunks: 1-D token-id tensors on the GPU (the content of one state, in order). The state (batch 1) ends up
        holding all of them; the tokens up to the deepest cached chunk boundary come from the store, the rest are
        prefilled (pieces of at most `piece` tokens on top of a non-empty cache) and snapshotted at the end."""
        if state.q.shape[1] != 1:
            raise ValueError("Int8PrefixCache.encode: one state per call (batch 1)")
        keys = chunk_keys(chunks)
        ends = torch.cumsum(torch.tensor([int(c.numel()) for c in chunks]), 0).tolist()
        hit, snap = self.lookup(keys)
        if snap is not None:
            self.restore(snap, state, 0)
        else:
            state.set_length(0)
        n_cached = snap.n_tokens if snap is not None else 0
        if hit < len(chunks) - 1:
            ids = torch.cat([c.reshape(-1) for c in chunks[hit + 1:]]).view(1, -1)
            pos = 0
            while pos < ids.shape[1]:
                n = ids.shape[1] - pos if state.length == 0 else min(piece, ids.shape[1] - pos)
                dec.prefill(ids[:, pos:pos + n], state)
                pos += n
            self.take(state, 0, keys[-1], snap, ends[-1])
        self.stats["requests"] += 1
        self.stats["hit_tokens"] += n_cached
        self.stats["new_tokens"] += ends[-1] - n_cached
        return n_cached

    def nbytes(self) -> int:
        return self.q.numel() + self.scale.numel() * 4
