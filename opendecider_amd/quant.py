"""int8 tensors, int8 / W8A8 linears and their installers, on the MI355X kernels.

Drop-in for the quantized-scoring part of src/opendecider/quant.py: the same class and function names, argument
meanings, attributes and return values, with the arithmetic moved to the HIP library:
  * Int8Tensor.quantize          -> od_act_quant (per-row absmax int8, bit-exact with quant.py:38-40)
  * W8A8Linear (GemLite A8W8)    -> od_act_quant (+ fused SmoothQuant input scale) + od_w8a8_gemm (int8 MFMA)
  * Int8Linear._fused slot       -> the same W8A8 path on the layer's own int8 weights (fast_int8_kernels_)
Load-time weight preparation (Int8Linear(lin), W8A8Linear.from_linear, the SmoothQuant fold) is done by the same
kernel on the GPU, and by the same formula in torch when a model is still being built on the CPU. The forward
paths of W8A8Linear and of the fused slot run only on the GPU and raise otherwise.
"""
from __future__ import annotations

import os
from dataclasses import dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import kernels


# ---------------------------------------------------------------- int8 tensors (caches)
@dataclass
class Int8Tensor:
    """int8 values + one scale per row over the last dim (per token, per head for K/V): quant.py:30-58."""
    q: torch.Tensor          # int8, same shape as the original
    scale: torch.Tensor      # shape[:-1] + (1,)
    dtype: torch.dtype

    @classmethod
    def quantize(cls, x: torch.Tensor, scale_dtype: torch.dtype | None = None) -> "Int8Tensor":
        """quant.py:36-41 on the GPU. The scale is stored like the reference (x.dtype, fp32 for fp32 input) unless
        scale_dtype is given; the KV caches of this package keep it in fp32 (the value that produced q)."""
        if x.dtype == torch.bfloat16:
            q, s = kernels.act_quant(x)
        elif x.dtype in (torch.float32, torch.float16, torch.float64):
            q, s = kernels.act_quant_float(x)
        else:
            raise TypeError(f"Int8Tensor.quantize: floating-point input expected, got {x.dtype}")
        q = q.view(x.shape)
        s = s.view(*x.shape[:-1], 1)
        sd = scale_dtype or (x.dtype if x.dtype != torch.float32 else torch.float32)
        return cls(q, s.to(sd), x.dtype)

    def dequantize(self, dtype: torch.dtype | None = None) -> torch.Tensor:
        dt = dtype or self.dtype
        return self.q.to(dt) * self.scale.to(dt)

    @property
    def shape(self):
        return self.q.shape

    def nbytes(self) -> int:
        return self.q.numel() + self.scale.numel() * self.scale.element_size()

    def to(self, device) -> "Int8Tensor":
        return Int8Tensor(self.q.to(device), self.scale.to(device), self.dtype)

    def index_select(self, dim: int, idx: torch.Tensor) -> "Int8Tensor":
        return Int8Tensor(self.q.index_select(dim, idx), self.scale.index_select(dim, idx), self.dtype)


def kv_mode(cfg) -> str | bool:
    """Cache quantization from a backbone config: False | "int8" (quant.py:100-102; int4 is not built here)."""
    return cfg.kv_quant if cfg.kv_quant == "int8" else False


def maybe_quantize(x: torch.Tensor, enabled):
    """quant.py:105-109 for int8: False/None keeps x, True or "int8" quantizes."""
    if not enabled:
        return x
    if enabled == "int4":
        raise NotImplementedError("int4 caches are outside the MI355X int8 path")
    return Int8Tensor.quantize(x)


def materialize(x, dtype: torch.dtype | None = None) -> torch.Tensor:
    if isinstance(x, Int8Tensor):
        return x.dequantize(dtype)
    return x if dtype is None else x.to(dtype)


def _quantize_rows_host(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-row int8 quantization for load-time weight preparation: the kernel on the GPU; the same formula
    (quant.py:124-126) in torch for a model still on the CPU. Returns (q int8, scale fp32 (rows, 1))."""
    if w.is_cuda and w.dtype == torch.bfloat16:
        q, s = kernels.act_quant(w)
        return q.view(w.shape), s.view(-1, 1)
    wf = w.float()
    s = wf.abs().amax(1, keepdim=True).clamp_min(1e-8) / 127.0
    return torch.round(wf / s).clamp_(-127, 127).to(torch.int8), s


# ---------------------------------------------------------------- int8 weights
class Int8Linear(nn.Module):
    """Frozen int8 linear with per-output-channel absmax scales (quant.py:119-164). Unfused, forward is the
    reference's dequantize + F.linear; fast_int8_kernels_ attaches the W8A8 HIP path in the `_fused` slot."""

    def __init__(self, lin: nn.Linear):
        super().__init__()
        q, s = _quantize_rows_host(lin.weight.data)
        self.register_buffer("qweight", q)
        self.register_buffer("scale", s.to(lin.weight.dtype))
        if lin.bias is not None:
            self.register_buffer("bias", lin.bias.data.clone())
        else:
            self.bias = None
        self.in_features, self.out_features = lin.in_features, lin.out_features

    @property
    def weight(self) -> torch.Tensor:
        if self.__dict__.get("_dq") is not None:
            return self._dq
        if self.__dict__.get("_fused") is not None:
            return self._fused.dense_weight().t()
        return self.qweight.to(self.scale.dtype) * self.scale

    def materialize(self, dtype: torch.dtype) -> None:
        self.__dict__["_dq"] = (self.qweight.to(dtype) * self.scale.to(dtype)).detach()
        self.qweight = torch.empty(0, dtype=torch.int8, device=self.qweight.device)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        fused = self.__dict__.get("_fused")
        if fused is not None:
            return fused(x)
        dq = self.__dict__.get("_dq")
        if dq is not None and dq.dtype == x.dtype:
            return F.linear(x, dq, None if self.bias is None else self.bias.to(x.dtype))
        return F.linear(x, self.qweight.to(x.dtype) * self.scale.to(x.dtype),
                        None if self.bias is None else self.bias.to(x.dtype))

    def dequant_rows(self, idx, dtype=torch.bfloat16) -> torch.Tensor:
        return self.qweight[idx].to(dtype) * self.scale[idx].to(dtype)

    def extra_repr(self) -> str:
        return f"in={self.in_features}, out={self.out_features}, int8 weight-only"


def quantize_int8_(module: nn.Module, skip: tuple[str, ...] = ()) -> nn.Module:
    """Replace every nn.Linear under `module` in place with Int8Linear (quant.py:256-267; embeddings stay)."""
    for name, child in list(module.named_children()):
        if name in skip:
            continue
        if isinstance(child, nn.Linear):
            setattr(module, name, Int8Linear(child))
        else:
            quantize_int8_(child, skip)
    return module


# ---------------------------------------------------------------- W8A8 on int8 MFMA
def _pad16(k: int) -> int:
    return (k + 15) // 16 * 16


class W8A8Linear(nn.Module):
    """W8A8 linear: per-token dynamic int8 activations x per-output-channel int8 weights, int32 accumulation, bf16
    dequant epilogue, on the MI355X (od_act_quant + od_w8a8_gemm). Takes the place of GemLite's
    A8W8_int8_dynamic layer (quant.py:302-314) and of Int8GemLite in Int8Linear's `_fused` slot (quant.py:375-409).

    Buffers: qweight int8 (out, in padded to a multiple of 16 with zero columns), w_scale fp32 (out,), bias (bf16 or
    None), inv_s (bf16 (in,) SmoothQuant input scale folded into the activation quantizer, or None)."""

    def __init__(self, qweight: torch.Tensor, w_scale: torch.Tensor, bias: torch.Tensor | None = None,
                 in_features: int | None = None, inv_s: torch.Tensor | None = None,
                 scale_dtype: torch.dtype = torch.bfloat16):
        super().__init__()
        self.scale_dtype = scale_dtype  # dtype of the dense weight handed out by dense_weight()
        N, K = qweight.shape
        self.in_features = K if in_features is None else in_features
        self.out_features = N
        Kp = _pad16(self.in_features)
        if K != Kp:
            qweight = torch.cat([qweight, qweight.new_zeros(N, Kp - K)], 1)
        self.register_buffer("qweight", qweight.contiguous())
        self.register_buffer("w_scale", w_scale.reshape(N).float().contiguous())
        self.register_buffer("bias", None if bias is None else bias.to(torch.bfloat16).contiguous())
        self.register_buffer("inv_s", None if inv_s is None else inv_s.to(torch.bfloat16).contiguous())

    @classmethod
    def from_linear(cls, lin: nn.Linear, s: torch.Tensor | None = None) -> "W8A8Linear":
        """Quantize lin's weight per output channel (quant.py:124-126), after the SmoothQuant fold W * s per input
        channel when s is given (quant.py:343-344); the layer then applies bf16(1 / s) to its input
        (quant.py:325, 329), fused into the activation quantizer."""
        w = lin.weight.data
        if s is not None:
            s = s.to(w.device, torch.float32)
            w = (w.float() * s[None, :]).to(w.dtype)
        q, sc = _quantize_rows_host(w)
        inv = None if s is None else (1.0 / s).to(torch.bfloat16)
        return cls(q, sc.reshape(-1), None if lin.bias is None else lin.bias.data, lin.in_features, inv)

    @classmethod
    def from_int8(cls, m: "Int8Linear") -> "W8A8Linear":
        """The SAME int8 weights as an Int8Linear; the weight scale is its stored scale (so dense_weight() equals
        Int8Linear.weight exactly)."""
        return cls(m.qweight, m.scale.float().reshape(-1), m.bias, m.in_features, scale_dtype=m.scale.dtype)

    def dense_weight(self) -> torch.Tensor:
        """(in, out) dense weight, q * scale in the scale's reference dtype (Int8GemLite.dense_weight, quant.py:385)."""
        q = self.qweight[:, : self.in_features]
        return (q.to(self.scale_dtype) * self.w_scale.to(self.scale_dtype)[:, None]).t()

    def forward(self, x: torch.Tensor, residual: torch.Tensor | None = None) -> torch.Tensor:
        if not x.is_cuda:
            raise RuntimeError("W8A8Linear runs on the MI355X only (no CPU path)")
        lead = x.shape[:-1]
        xb = x if x.dtype == torch.bfloat16 else x.to(torch.bfloat16)
        xq, sx = kernels.act_quant(xb, self.inv_s, ld=self.qweight.shape[1])
        res = None if residual is None else residual.reshape(-1, self.out_features)
        y = kernels.w8a8_gemm(xq, sx, self.qweight, self.w_scale, self.bias, res)
        y = y.view(*lead, self.out_features)
        return y if x.dtype == torch.bfloat16 else y.to(x.dtype)

    def extra_repr(self) -> str:
        return f"in={self.in_features}, out={self.out_features}, W8A8 int8 MFMA" + (
            ", smoothed" if self.inv_s is not None else "")


def gemlite_a8w8_(module: nn.Module) -> nn.Module:
    """Replace every nn.Linear under `module` with W8A8Linear (the reference's gemlite_a8w8_, quant.py:302-314)."""
    for name, child in list(module.named_children()):
        if isinstance(child, nn.Linear):
            setattr(module, name, W8A8Linear.from_linear(child))
        else:
            gemlite_a8w8_(child)
    return module


w8a8_ = gemlite_a8w8_


class SmoothedLinear(nn.Module):
    """y = inner(x / s) with inner holding W * s (SmoothQuant, arXiv:2211.10438; quant.py:317-329). With a
    W8A8Linear inner the division is fused into its activation quantizer; other inner modules get the reference's
    elementwise x * inv_s."""

    def __init__(self, inner: nn.Module, s: torch.Tensor):
        super().__init__()
        self.inner = inner
        self.register_buffer("inv_s", (1.0 / s).to(torch.bfloat16))
        self.in_features, self.out_features = inner.in_features, inner.out_features

    def forward(self, x):
        if isinstance(self.inner, W8A8Linear) and self.inner.inv_s is not None:
            return self.inner(x)
        return self.inner(x * self.inv_s.to(x.dtype))


@torch.no_grad()
def smooth_a8w8_(module: nn.Module, scales: dict, prefix: str = "") -> nn.Module:
    """Every nn.Linear under `module` whose name (relative to it) has a scale vector: W *= s per input channel, then
    W8A8, wrapped in SmoothedLinear; linears without scales get plain W8A8 (quant.py:332-350)."""
    for name, child in list(module.named_children()):
        full = f"{prefix}{name}"
        if isinstance(child, nn.Linear):
            s = scales.get(full)
            q = W8A8Linear.from_linear(child, s)
            setattr(module, name, q if s is None else SmoothedLinear(q, s.to(q.qweight.device, torch.float32)))
        else:
            smooth_a8w8_(child, scales, f"{full}.")
    return module


def smooth_scales(amax_x: torch.Tensor, W: torch.Tensor, alpha: float = 0.5) -> torch.Tensor:
    """SmoothQuant per-input-channel scales s_j = max|X_j|^alpha / max|W_:,j|^(1-alpha), clamped (quant.py:353-356).
    A calibration-time helper (not on the scoring path)."""
    aw = W.abs().amax(0).float().clamp(min=1e-5)
    return (amax_x.float().clamp(min=1e-5) ** alpha / aw ** (1 - alpha)).clamp(1e-3, 1e3)


# ---------------------------------------------------------------- fused int8 inference GEMMs (same weights)
def int8_to_w8a8_(module: nn.Module) -> int:
    """Give every (non-materialized) Int8Linear under `module` a W8A8Linear on the SAME int8 weights in its `_fused`
    slot and free its own int8 copy; the Int8Linear objects (and forward hooks on them) stay in place
    (int8_to_gemlite_, quant.py:398-409). Returns the count."""
    n = 0
    for m in module.modules():
        if isinstance(m, Int8Linear) and m.qweight.numel() and m.__dict__.get("_dq") is None:
            m.__dict__["_fused"] = W8A8Linear.from_int8(m)
            m.qweight = torch.empty(0, dtype=torch.int8, device=m.qweight.device)
            n += 1
    return n


def fast_int8_kernels_(backbone) -> int:
    """Inference loaders: run the Int8Linear layers of `backbone.lm.layers` on the W8A8 MI355X kernels
    (quant.py:437-453). OPENDECIDER_INT8_GEMM=dequant, or a backbone not on the GPU, keeps the dequantize path and
    returns 0. Returns the number of layers given the fused path."""
    if os.environ.get("OPENDECIDER_INT8_GEMM", "auto") == "dequant" or backbone.device.type != "cuda":
        return 0
    if not any(isinstance(m, Int8Linear) for m in backbone.lm.layers.modules()):
        return 0
    n = int8_to_w8a8_(backbone.lm.layers)
    torch.cuda.empty_cache()
    return n
