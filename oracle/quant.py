"""CPU oracle for the int8 quantizers and the W8A8 linear. TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Every function restates a formula of src/opendecider/quant.py in plain torch CPU arithmetic, with the float32
operation order written out so that a GPU kernel can be held to it bit for bit.
"""
from __future__ import annotations

import torch

QMAX = 127.0
EPS = 1e-8


def quantize_rows(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Int8Tensor.quantize (quant.py:36-41): one symmetric scale per row over the last dim.

    xf = x.float(); scale = max|xf| clamped to >= 1e-8, divided by 127 (IEEE fp32 division);
    q = round-half-even(xf / scale) (IEEE fp32 division), clamped to [-127, 127], int8.
    Returns (q int8, same shape as x; scale fp32, shape[:-1] + (1,)). The reference stores the scale in x.dtype when
    x is not fp32 (quant.py:41); the fp32 value returned here is the one that produced q, and it is what the KV
    cache and the W8A8 path store."""
    xf = x.detach().to("cpu").float()
    scale = xf.abs().amax(-1, keepdim=True).clamp_min(EPS) / QMAX
    q = torch.round(xf / scale).clamp_(-QMAX, QMAX).to(torch.int8)
    return q, scale


def dequantize(q: torch.Tensor, scale: torch.Tensor, dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Int8Tensor.dequantize (quant.py:43-45): q.to(dtype) * scale.to(dtype), the product rounded in `dtype`."""
    return q.to(dtype) * scale.to(dtype)


def quantize_weight(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Int8Linear weight quantization (quant.py:124-126): per output channel (row of the (out, in) weight), the same
    formula as quantize_rows. Returns (qweight int8 (N, K), scale fp32 (N,))."""
    q, s = quantize_rows(w)
    return q, s.squeeze(-1)


def smooth_input(x: torch.Tensor, inv_s: torch.Tensor) -> torch.Tensor:
    """SmoothedLinear.forward's input (quant.py:325,329): x * inv_s.to(x.dtype), the product rounded to x.dtype
    (bf16: float product then round-to-nearest-even)."""
    return x * inv_s.to(x.dtype)


def act_quant(x: torch.Tensor, inv_s: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Dynamic per-token activation quantization ahead of the W8A8 GEMM: optional SmoothQuant input scaling
    (quant.py:329), then the Int8Tensor formula per token (quant.py:38-40). x (..., K) bf16.
    Returns (xq int8 (..., K), sx fp32 (...,))."""
    if inv_s is not None:
        x = smooth_input(x, inv_s)
    q, s = quantize_rows(x)
    return q, s.squeeze(-1)


def int_gemm(a: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """int8 A (M, K) x int8 W (N, K) (nn.Linear layout) -> exact int32 accumulators (M, N), with torch's CPU
    int8 x int8 -> int32 matmul. |acc| <= 127^2 K stays below 2^31 for K < 133,144, so int32 accumulation is exact
    (pinned against an int64 matmul and scalar loops in tests/test_oracle_quant.py)."""
    assert a.dtype == torch.int8 and w.dtype == torch.int8 and a.shape[-1] == w.shape[-1]
    assert a.shape[-1] < 133_144
    a2 = a.detach().to("cpu").reshape(-1, a.shape[-1]).contiguous()
    acc = torch._int_mm(a2, w.detach().to("cpu").t().contiguous())
    return acc.reshape(*a.shape[:-1], w.shape[0])


def w8a8_epilogue(acc: torch.Tensor, sx: torch.Tensor, sw: torch.Tensor, bias: torch.Tensor | None = None,
                  residual: torch.Tensor | None = None, out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """Dequant epilogue: fp32 ((float(acc) * sx[m]) * sw[n]) (+ float(bias[n])) (+ float(residual[m, n])), then
    rounded once to out_dtype. float(acc) rounds to nearest even (exact below 2^24)."""
    y = acc.float() * sx.float()[..., None]
    y = y * sw.float()
    if bias is not None:
        y = y + bias.float()
    if residual is not None:
        y = y + residual.float()
    return y.to(out_dtype)


def w8a8_linear(x: torch.Tensor, wq: torch.Tensor, sw: torch.Tensor, bias: torch.Tensor | None = None,
                inv_s: torch.Tensor | None = None, residual: torch.Tensor | None = None):
    """The whole W8A8 linear: act_quant -> int_gemm -> w8a8_epilogue. Returns (out bf16, acc int32, xq, sx)."""
    xq, sx = act_quant(x, inv_s)
    acc = int_gemm(xq, wq)
    return w8a8_epilogue(acc, sx, sw, bias, residual), acc, xq, sx


def int8_linear_dequant(x: torch.Tensor, wq: torch.Tensor, scale: torch.Tensor, bias: torch.Tensor | None = None):
    """Int8Linear.forward's unfused path (quant.py:156-157): F.linear(x, q.to(dt) * s.to(dt), bias) in x.dtype.
    This is the reference's CPU linear path (its fused kernels are a no-op on CPU, quant.py:441-442)."""
    dt = x.dtype
    w = wq.to(dt) * scale.reshape(-1, 1).to(dt)
    return torch.nn.functional.linear(x, w, None if bias is None else bias.to(dt))


def smooth_fold(w: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
    """smooth_a8w8_'s weight fold (quant.py:343-344): W' = (W.float() * s[None, :]).to(W.dtype)."""
    return (w.float() * s.float()[None, :]).to(w.dtype)


def smooth_inv(s: torch.Tensor) -> torch.Tensor:
    """SmoothedLinear's stored input scale (quant.py:325): (1.0 / s).to(bfloat16)."""
    return (1.0 / s).to(torch.bfloat16)


def smooth_scales(amax_x: torch.Tensor, w: torch.Tensor, alpha: float = 0.5) -> torch.Tensor:
    """smooth_scales (quant.py:353-356): s_j = max|X_j|^alpha / max|W_:,j|^(1-alpha), clamped to [1e-3, 1e3]."""
    aw = w.abs().amax(0).float().clamp(min=1e-5)
    return (amax_x.float().clamp(min=1e-5) ** alpha / aw ** (1 - alpha)).clamp(1e-3, 1e3)
