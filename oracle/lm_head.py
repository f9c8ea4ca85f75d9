"""CPU oracle for the LM-head token log-prob over a quantized vocabulary table. TEST INFRASTRUCTURE ONLY (see
oracle/__init__.py).

Restates Backbone.token_logprob (src/opendecider/backbone.py:164-178) on the frozen tables of
src/opendecider/quant.py: Int8Embedding (quant.py:183-203; Int8Linear's rows, quant.py:122-132,159-161, have the
same form) and Q4Table (quant.py:206-246).

    log p(tok | h) = sum_k float(h_k) * float(row(tok)_k)  -  logsumexp_v bf16(bf16(h) . bf16row(v))

where bf16row(v) = bf16(q_v,k * s_v) is the table row dequantized in bf16 (dequant_rows(idx, bfloat16): a bf16
product), the logits are the bf16 result of a bf16 matmul (accumulated in fp32, rounded once to bf16), and the
normaliser is accumulated over vocabulary chunks with logaddexp in fp32. The target term uses the float32 row and
float32 h (backbone.py:178). Both forms are written out below with their roundings explicit.
"""
from __future__ import annotations

import torch

BF16 = torch.bfloat16


def int8_table(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Int8Embedding.__init__ (quant.py:189-194): per-row absmax over the float32 weight, scale = max|w| clamped to
    >= 1e-8, / 127; q = round-half-even(w / scale) clamped to [-127, 127]; the scale is stored in the weight's dtype.
    Returns (qweight int8 (V, K), scale (V,) in w.dtype)."""
    wf = w.detach().to("cpu").float()
    scale = wf.abs().amax(1, keepdim=True).clamp_min(1e-8) / 127.0
    q = torch.round(wf / scale).clamp_(-127, 127).to(torch.int8)
    return q, scale.squeeze(1).to(w.dtype)


def int8_rows(q: torch.Tensor, scale: torch.Tensor, idx, dtype: torch.dtype) -> torch.Tensor:
    """Int8Embedding.dequant_rows (quant.py:202-203): q[idx].to(dtype) * scale[idx].to(dtype), rounded in dtype."""
    return q[idx].to(dtype) * scale[idx].to(dtype).unsqueeze(-1)


def q4_table(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Q4Table.__init__ (quant.py:213-229): blocks of 32 along a row; d = (signed value of largest magnitude) / -8
    (fp16 stored); q = clamp(floor(w / d + 8.5), 0, 15) with 1/d (0 for d == 0); positions 0-15 of a block in the low
    nibbles of its 16 bytes, 16-31 in the high nibbles. Returns (qs uint8 (V, K/2), d fp16 (V, K/32))."""
    N, K = w.shape
    b = w.detach().to("cpu").float().view(N, K // 32, 32)
    idx = b.abs().argmax(-1, keepdim=True)
    mx = b.gather(-1, idx)
    d = mx / -8
    inv = torch.where(d != 0, 1 / d, torch.zeros_like(d))
    q = torch.clamp(torch.floor(b * inv + 8.5), 0, 15).to(torch.uint8)
    qs = (q[..., :16] | (q[..., 16:] << 4)).view(N, K // 2)
    return qs, d.squeeze(-1).to(torch.float16)


def q4_rows(qs: torch.Tensor, d: torch.Tensor, idx, dtype: torch.dtype) -> torch.Tensor:
    """Q4Table.dequant_rows (quant.py:231-237): ((q - 8) in dtype) * d.to(dtype), rounded in dtype."""
    q = qs[idx]
    n, K = q.shape[0], q.shape[1] * 2
    q = q.view(n, K // 32, 16)
    v = torch.cat([q & 15, q >> 4], -1).to(dtype) - 8
    return (v * d[idx].to(dtype).unsqueeze(-1)).view(n, K)


def bf16_logits(h: torch.Tensor, rows_bf16: torch.Tensor) -> torch.Tensor:
    """(bf16(h) @ rows.T) as a bf16 matmul returns it: exact products of the bf16 operands accumulated in float32
    (here in float64, then rounded to float32), rounded once to bf16; returned as float32."""
    acc = h.to(BF16).double() @ rows_bf16.double().t()
    return acc.float().to(BF16).float()


def token_logprob(h: torch.Tensor, rows, V: int, tok: torch.Tensor, chunk: int = 32768) -> torch.Tensor:
    """Backbone.token_logprob (backbone.py:164-178). `rows(idx, dtype)` is the table's dequant_rows, V its size.
    The normaliser: for each vocabulary chunk, logsumexp of the chunk's bf16 logits (float32), merged into the
    running value with logaddexp (float32). The target term: (float(h) * rows(tok, float32)).sum(-1) in float32."""
    h = h.detach().to("cpu")
    lse = torch.full((h.shape[0],), -float("inf"))
    for a in range(0, V, chunk):
        lg = bf16_logits(h, rows(slice(a, min(a + chunk, V)), BF16))
        lse = torch.logaddexp(lse, torch.logsumexp(lg, dim=-1))
    return (h.float() * rows(tok.to("cpu").long(), torch.float32)).sum(-1) - lse
