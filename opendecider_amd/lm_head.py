"""The LM head's token log-probs over a frozen int8 or Q4_0 vocabulary table (the option-token LM feature).

Mirrors src/opendecider/quant.py:183-246 (Int8Embedding: the frozen int8 table, per-row absmax scales stored in the
weight's dtype, dequant_rows, lookup; Q4Table: llama.cpp's Q4_0 layout) and src/opendecider/backbone.py:164-178 (Backbone.token_logprob: log
softmax(h @ W^T)[tok] with the normaliser over the whole vocabulary). The log-prob runs as one pass of
od_lm_head_logprob over the table: the reference's vocabulary chunks and row blocks only bound its memory, so they
are accepted and do not change the result.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from . import kernels


class Int8Table(nn.Module):
    """A frozen int8 table of V rows of K values (an embedding or an LM head): qweight int8 (V, K) and scale (V, 1)
    in the source weight's dtype (quant.py:189-194). Built from float rows with the reference's formula, or from an
    existing (qweight, scale) pair (from_quantized)."""

    def __init__(self, weight: torch.Tensor | None = None, *, qweight=None, scale=None):
        super().__init__()
        if weight is not None:
            w = weight.detach().float()
            s = w.abs().amax(1, keepdim=True).clamp_min(1e-8) / 127.0
            qweight = torch.round(w / s).clamp_(-127, 127).to(torch.int8)
            scale = s.to(weight.dtype)
        if qweight is None or scale is None:
            raise ValueError("Int8Table needs float rows or (qweight, scale)")
        self.register_buffer("qweight", qweight)
        self.register_buffer("scale", scale.reshape(-1, 1))
        self.num_embeddings, self.embedding_dim = qweight.shape
        self.in_features, self.out_features = self.embedding_dim, self.num_embeddings
        self.padding_idx = None

    @classmethod
    def from_quantized(cls, qweight: torch.Tensor, scale: torch.Tensor) -> "Int8Table":
        return cls(qweight=qweight, scale=scale)

    @property
    def weight(self) -> torch.Tensor:
        return self.qweight.to(self.scale.dtype) * self.scale

    def dequant_rows(self, idx, dtype=torch.bfloat16) -> torch.Tensor:
        return self.qweight[idx].to(dtype) * self.scale[idx].to(dtype)

    def forward(self, ids: torch.Tensor) -> torch.Tensor:
        return self.qweight[ids].to(self.scale.dtype) * self.scale[ids]


class Q4Table(nn.Module):
    """A frozen Q4_0 table (quant.py:206-246): blocks of 32 values along a row, one fp16 scale d per block,
    w = (q - 8) d with q in 0..15 (a block's positions 0-15 in the low nibbles of its 16 bytes, 16-31 in the high
    ones), 4.5 bits per value. Quantized from float rows with the reference's round-to-nearest formula (values that
    came from a Q4_0 tensor come back exactly)."""

    def __init__(self, w: torch.Tensor | None = None, *, qs=None, d=None):
        super().__init__()
        if w is not None:
            N, K = w.shape
            if K % 32:
                raise ValueError("Q4Table needs rows whose length is a multiple of 32")
            qs_parts, d_parts = [], []
            for a in range(0, N, 16384):  # bounded float32 temporaries
                b = w[a:a + 16384].float().view(-1, K // 32, 32)
                idx = b.abs().argmax(-1, keepdim=True)
                dd = b.gather(-1, idx) / -8
                inv = torch.where(dd != 0, 1 / dd, torch.zeros_like(dd))
                q = torch.clamp(torch.floor(b * inv + 8.5), 0, 15).to(torch.uint8)
                qs_parts.append((q[..., :16] | (q[..., 16:] << 4)).view(b.shape[0], K // 2))
                d_parts.append(dd.squeeze(-1).to(torch.float16))
            qs, d = torch.cat(qs_parts), torch.cat(d_parts)
        if qs is None or d is None:
            raise ValueError("Q4Table needs float rows or (qs, d)")
        self.register_buffer("qs", qs)
        self.register_buffer("d", d)
        self.num_embeddings, self.embedding_dim = qs.shape[0], qs.shape[1] * 2
        self.in_features, self.out_features = self.embedding_dim, self.num_embeddings
        self.padding_idx = None

    def dequant_rows(self, idx, dtype=torch.bfloat16) -> torch.Tensor:
        q = self.qs[idx]
        n, K = q.shape[0], self.embedding_dim
        q = q.view(n, K // 32, 16)
        v = torch.cat([q & 15, q >> 4], -1).to(dtype) - 8
        return (v * self.d[idx].to(dtype).unsqueeze(-1)).view(n, K)

    @property
    def weight(self) -> torch.Tensor:
        return self.dequant_rows(slice(None), torch.bfloat16)

    def forward(self, ids: torch.Tensor) -> torch.Tensor:
        return self.dequant_rows(ids.reshape(-1), torch.bfloat16).view(*ids.shape, self.embedding_dim)


@torch.no_grad()
def token_logprob(table, h: torch.Tensor, tok: torch.Tensor, chunk: int = 32768,
                  max_block_bytes: int = 1 << 30) -> torch.Tensor:
    """log softmax(h @ W^T)[tok] per row of h (n, K), W the rows of an Int8Table or a Q4Table
    (Backbone.token_logprob, backbone.py:164-178): the normaliser from the bf16 logits of bf16(h) against the
    bf16-dequantized rows, the target term (h.float() * row(tok)).sum(-1) in fp32. `chunk` and `max_block_bytes`
    bound the reference's temporaries; the kernel keeps none, so they are accepted and ignored. Returns fp32 (n,)."""
    if isinstance(table, Q4Table):
        return kernels.lm_head_logprob_q4(h, table.qs, table.d, tok)
    if table.scale.dtype != torch.bfloat16:
        raise TypeError("the kernel reads bf16 table scales (a bf16 model's Int8Embedding / Int8Linear)")
    return kernels.lm_head_logprob(h, table.qweight, table.scale, tok)
