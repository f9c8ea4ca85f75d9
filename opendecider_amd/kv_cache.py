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

import torch

from . import kernels
from .quant import Int8Tensor


class Int8KVCache:
    def __init__(self, batch: int, n_heads: int, head_dim: int, capacity: int, device, dtype=torch.bfloat16):
        self.q = torch.zeros(batch, n_heads, capacity, head_dim, dtype=torch.int8, device=device)
        self.scale = torch.zeros(batch, n_heads, capacity, dtype=torch.float32, device=device)
        self.length = 0
        self.dtype = dtype

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

    def as_int8_tensor(self) -> Int8Tensor:
        """The filled part as an Int8Tensor (views, no copy): q (B, Hkv, T, D), scale (B, Hkv, T, 1) fp32."""
        T = self.length
        return Int8Tensor(self.q[:, :, :T], self.scale[:, :, :T, None], self.dtype)

    def nbytes(self) -> int:
        return self.q.numel() + self.scale.numel() * 4
