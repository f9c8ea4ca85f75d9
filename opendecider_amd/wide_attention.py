"""wide_attention: flash attention whose query/key width may exceed the value width, behind the reference's
signature (src/opendecider/wide_attention.py:70-91), on the od_wide_attn HIP kernel.

    out = wide_attention(q (B,H,T,Dk), k (B,G,S,Dk), v (B,G,S,Dv), scale, kvalid=None (B,S) bool)

Queries are the last T of the S positions (causal with offset S - T). The Triton tuning arguments (BM, BN, BD,
num_warps, num_stages) are accepted and ignored: the kernel's tiling is fixed for gfx950 (128 query slots x 64
keys per block)."""
from __future__ import annotations

import torch
import torch.nn.functional as F

from . import kernels


def wide_attention(q, k, v, scale: float, kvalid=None, causal: bool = True, return_lse: bool = False, BM: int = 64,
                   BN: int = 64, BD: int = 32, num_warps: int = 4, num_stages: int = 2):
    """causal=False: every query sees every (valid) key. return_lse: also the (B, H, T) fp32 log-sum-exp of the
    scaled scores (natural log), to merge with attention over other keys. bf16 inputs; Dv in {64, 128, 256};
    Dk up to 512 (a Dk that is not a multiple of 8 is zero-padded, which leaves every score unchanged). The scale
    must be positive and finite (the kernel takes each block's max on the unscaled scores); the softmax scale
    Dk^-0.5 the reference passes always is."""
    B, H, T, DK = q.shape
    G, S, DV = k.shape[1], k.shape[2], v.shape[-1]
    rep = H // G
    assert H % G == 0 and v.shape[2] == S and DV in (64, 128, 256) and BM % rep == 0
    if q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16:
        raise TypeError("wide_attention: q, k and v must be bf16")
    if DK > 512:
        raise ValueError(f"wide_attention: head width {DK} above 512 is not supported")
    if not 0.0 < float(scale) < float("inf"):
        raise ValueError(f"wide_attention: the scale must be positive and finite, got {scale}")
    if DK % 8:
        pad = 8 - DK % 8
        q, k = F.pad(q, (0, pad)), F.pad(k, (0, pad))
    return kernels.wide_attn(q, k, v, scale, kvalid=kvalid, causal=causal, return_lse=return_lse)
