"""Append-only int8 KV cache for a growing shared state.

Replaces the reference's incremental-state storage on the scoring path: PrefixCache._take quantizes ONLY the new
tokens' K/V slice (src/opendecider/state_cache.py:79) and PackedCache.pack quantizes a whole cache
(src/opendecider/backbone.py:446), both through Int8Tensor.quantize (src/opendecider/quant.py:36-41). With one
scale per (token, head), quantizing a slice gives the same bytes as quantizing the whole tensor, so appending new
rows in place is byte-identical to re-packing, and nothing is ever dequantized or re-quantized (the reference's
restore path concatenates dequantized deltas and re-packs, state_cache.py:116,154).

Layout in HBM: q int8 (B, Hkv, cap, D) and scale fp32 (B, Hkv, cap), token-contiguous per head, so the attention
kernel streams one (state, head) as a single contiguous slab.
"""
from __future__ import annotations

import itertools

import torch

from . import kernels
from .quant import Int8Tensor

# Cache versions come from one process-wide counter: every new cache and every write takes a value no other cache
# has held, so a (generation) key can never match a different cache, even one that reuses a freed cache's id().
_GENERATIONS = itertools.count(1)


class Int8KVCache:
    def __init__(self, batch: int, n_heads: int, head_dim: int, capacity: int, device, dtype=torch.bfloat16):
        self.q = torch.zeros(batch, n_heads, capacity, head_dim, dtype=torch.int8, device=device)
        self.scale = torch.zeros(batch, n_heads, capacity, dtype=torch.float32, device=device)
        self.length = 0
        self.dtype = dtype
        # a fresh value on every write through this package (derived data, e.g. block images, keys on it); unique
        # across caches, so a new cache never looks like an old one
        self.generation = next(_GENERATIONS)

    @classmethod
    def from_tensors(cls, q: torch.Tensor, scale: torch.Tensor, dtype=torch.bfloat16) -> "Int8KVCache":
        """A cache over existing buffers q int8 (B, Hkv, cap, D) and scale fp32 (B, Hkv, cap), both contiguous."""
        if q.dtype != torch.int8 or scale.dtype != torch.float32 or scale.shape != q.shape[:3]:
            raise TypeError("Int8KVCache.from_tensors: q int8 (B, H, cap, D) with fp32 scales (B, H, cap)")
        if not (q.is_contiguous() and scale.is_contiguous()):
            raise ValueError("Int8KVCache.from_tensors: buffers must be contiguous")
        c = cls.__new__(cls)
        c.q, c.scale, c.length, c.dtype, c.generation = q, scale, 0, dtype, next(_GENERATIONS)
        return c

    def touch(self) -> None:
        """Mark the bytes as changed (call after writing q / scale directly)."""
        self.generation = next(_GENERATIONS)

    @property
    def capacity(self) -> int:
        return self.q.shape[2]

    def append(self, x: torch.Tensor) -> None:
        """Quantize x (B, Hkv, n, D) bf16 per (token, head) and append it after the current tokens."""
        n = x.shape[2]
        if self.length + n > self.capacity:
            raise ValueError(f"Int8KVCache: {self.length} + {n} tokens exceed the capacity {self.capacity}")
        kernels.kv_quant_append(x, self.q, self.scale, self.length)
        self.length += n
        self.touch()

    def as_int8_tensor(self) -> Int8Tensor:
        """The filled part as an Int8Tensor (views, no copy): q (B, Hkv, T, D), scale (B, Hkv, T, 1) fp32."""
        T = self.length
        return Int8Tensor(self.q[:, :, :T], self.scale[:, :, :T, None], self.dtype)

    def nbytes(self) -> int:
        return self.q.numel() + self.scale.numel() * 4


class StateKV:
    """Every layer's K and V caches of `batch` states in one allocation: q int8 (2 L, B, Hkv, cap, D) and scale fp32
    (2 L, B, Hkv, cap), matrix 2 l being layer l's K and 2 l + 1 its V. Indexing and iteration give the per-layer
    (K, V) Int8KVCache pairs (views), so it stands wherever the decoder takes a list of cache pairs; one state's rows
    of every layer are then reachable at one matrix stride, which lets one launch copy them all
    (kernels.kv_copy_rows)."""

    def __init__(self, n_layers: int, batch: int, n_heads: int, head_dim: int, capacity: int, device,
                 dtype=torch.bfloat16):
        self.q = torch.zeros(2 * n_layers, batch, n_heads, capacity, head_dim, dtype=torch.int8, device=device)
        self.scale = torch.zeros(2 * n_layers, batch, n_heads, capacity, dtype=torch.float32, device=device)
        self.pairs = [(Int8KVCache.from_tensors(self.q[2 * li], self.scale[2 * li], dtype),
                       Int8KVCache.from_tensors(self.q[2 * li + 1], self.scale[2 * li + 1], dtype))
                      for li in range(n_layers)]

    def __len__(self) -> int:
        return len(self.pairs)

    def __getitem__(self, li):
        return self.pairs[li]

    def __iter__(self):
        return iter(self.pairs)

    @property
    def capacity(self) -> int:
        return self.q.shape[3]

    @property
    def length(self) -> int:
        n = {c.length for pair in self.pairs for c in pair}
        if len(n) != 1:
            raise RuntimeError(f"StateKV: layers hold different lengths {sorted(n)}")
        return n.pop()

    def set_length(self, n: int) -> None:
        if not 0 <= n <= self.capacity:
            raise ValueError(f"StateKV: length {n} outside [0, {self.capacity}]")
        for pair in self.pairs:
            for c in pair:
                c.length = n
                c.touch()

    def state(self, b: int):
        """State b of every layer: q (2 L, Hkv, cap, D) and scale (2 L, Hkv, cap) views."""
        return self.q[:, b], self.scale[:, b]

    def nbytes(self) -> int:
        return self.q.numel() + self.scale.numel() * 4


class GDNState:
    """A Gated DeltaNet layer's state of `batch` sequences, the counterpart of an attention layer's K/V cache (the
    reference keeps it per row in the HF cache's conv_states / recurrent_states, src/opendecider/backbone.py:256-289,
    529-571): conv (B, 3, C) bf16, the last 3 pre-conv inputs of the projection's qkv block, and rec (B, n_v, dk, dv)
    fp32, the recurrent state. length counts the tokens absorbed. Option rows read these in place, one shared state
    per request, never a per-row copy."""

    def __init__(self, conv: torch.Tensor, rec: torch.Tensor):
        self.conv, self.rec, self.length = conv, rec, 0

    @property
    def batch(self) -> int:
        return self.conv.shape[0]


class HybridState:
    """Every layer's state of `batch` sequences for a hybrid stack: the attention layers' int8 K/V caches (one
    StateKV) and the Gated DeltaNet layers' GDNState (two allocations: conv and rec of every GDN layer). Indexing by
    layer gives a (K, V) Int8KVCache pair or a GDNState, so it stands wherever the decoder takes per-layer states."""

    def __init__(self, gdn_layers: list, batch: int, n_kv_heads: int, head_dim: int, capacity: int, conv_dim: int,
                 n_v: int, dk: int, dv: int, device):
        n_gdn = sum(1 for g in gdn_layers if g)
        n_attn = len(gdn_layers) - n_gdn
        self.kv = StateKV(n_attn, batch, n_kv_heads, head_dim, capacity, device) if n_attn else None
        self.conv = torch.zeros(n_gdn, batch, 3, conv_dim, dtype=torch.bfloat16, device=device)
        self.rec = torch.zeros(n_gdn, batch, n_v, dk, dv, dtype=torch.float32, device=device)
        self.items, ai, gi = [], 0, 0
        for g in gdn_layers:
            if g:
                self.items.append(GDNState(self.conv[gi], self.rec[gi]))
                gi += 1
            else:
                self.items.append(self.kv[ai])
                ai += 1

    def __len__(self) -> int:
        return len(self.items)

    def __getitem__(self, li):
        return self.items[li]

    def __iter__(self):
        return iter(self.items)

    @property
    def capacity(self) -> int | None:
        return None if self.kv is None else self.kv.capacity

    @property
    def length(self) -> int:
        n = {it.length for it in self.items if isinstance(it, GDNState)}
        if self.kv is not None:
            n.add(self.kv.length)
        if len(n) != 1:
            raise RuntimeError(f"HybridState: layers hold different lengths {sorted(n)}")
        return n.pop()

    def nbytes(self) -> int:
        return (0 if self.kv is None else self.kv.nbytes()) + self.conv.numel() * 2 + self.rec.numel() * 4
