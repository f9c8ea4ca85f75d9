"""The LM head's token log-probs over a frozen int8 vocabulary table (the option-token LM feature).

Mirrors src/opendecider/quant.py:183-203 (Int8Embedding: the frozen int8 table, per-row absmax scales stored in the
weight's dtype, dequant_rows, lookup) and src/opendecider/backbone.py:164-178 (Backbone.token_logprob: log
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


@torch.no_grad()
def token_logprob(table: Int8Table, h: torch.Tensor, tok: torch.Tensor, chunk: int = 32768,
                  max_block_bytes: int = 1 << 30) -> torch.Tensor:
    """log softmax(h @ W^T)[tok] per row of h (n, K), W the table's rows (Backbone.token_logprob,
    backbone.py:164-178): the normaliser from the bf16 logits of bf16(h) against the bf16-dequantized rows, the
    target term (h.float() * row(tok)).sum(-1) in fp32. `chunk` and `max_block_bytes` bound the reference's
    temporaries; the kernel keeps none, so they are accepted and ignored. Returns fp32 (n,)."""
    if table.scale.dtype != torch.bfloat16:
        raise TypeError("the kernel reads bf16 table scales (a bf16 model's Int8Embedding / Int8Linear)")
    return kernels.lm_head_logprob(h, table.qweight, table.scale, tok)
