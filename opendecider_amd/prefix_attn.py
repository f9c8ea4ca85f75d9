"""Shared-prefix (Hydragen) attention for branched option rows on the MI355X.

Drop-in for the op at the centre of src/opendecider/prefix_attn.py: `_split_attention` (prefix_attn.py:43-76), its
per-state loop in `_forward` (prefix_attn.py:118-128) and the per-layer dequantized copy of the state's K/V made by
`shared_prefix_attention` (prefix_attn.py:145-149). An int8 state (Int8Tensor) goes to the branched kernel as it is
stored, with its per-(token, head) scales, and one launch covers every row: prefix partial, own causal partial and
their log-sum-exp merge, the state dequantized in registers as the reference materializes it (bf16(q * bf16(s))).
A dense bf16 prefix, as the reference's _forward passes it (prefix_attn.py:127), is written into the same block
images (od_attn_stage_bf16) and attended by the same one-softmax kernel.
"""
from __future__ import annotations

import torch

from . import kernels
from .quant import Int8Tensor


def _state_parts(K, V):
    """(kq, ks, vq, vs) from Int8Tensor states (Hkv, T, D) or (Ns, Hkv, T, D) with scales (..., 1) (fp32, or the
    reference's bf16 stored scale, whose value is exact in fp32)."""
    kq, vq = K.q, V.q
    ks, vs = K.scale.float(), V.scale.float()
    if kq.dim() == 3:
        kq, vq, ks, vs = kq[None], vq[None], ks[None], vs[None]
    return kq.contiguous(), ks.reshape(kq.shape[:3]).contiguous(), vq.contiguous(), vs.reshape(vq.shape[:3]).contiguous()


def _split_attention(q, k, v, Kp, Vp, pm, scale, dequant: str = "bf16"):
    """Hydragen split for rows continuing ONE shared prefix (prefix_attn.py:43-76): q (n, Hq, t, D) attends the
    prefix Kp/Vp ((Hkv, T, D); pm (T,) real keys or None) and its own row's k/v (n, Hkv, t, D) causally; the two
    softmax parts are merged by their log-sum-exp. Kp/Vp are either Int8Tensor (the int8 state read directly,
    dequantized as `dequant` says: "bf16" is the reference's materialize, "fp32" the exact q * s) or dense bf16
    tensors as the reference's caller passes them (prefix_attn.py:127). Returns (n, Hq, t, D) in v.dtype."""
    if isinstance(Kp, Int8Tensor) and isinstance(Vp, Int8Tensor):
        kq, ks, vq, vs = _state_parts(Kp, Vp)
        kvalid = None if pm is None else pm.reshape(1, -1)
        out = kernels.branched_attn(q, k, v, kq, ks, vq, vs, scale, kvalid=kvalid, length=kq.shape[2],
                                    dequant=dequant)
        return out.to(v.dtype)
    if isinstance(Kp, Int8Tensor) or isinstance(Vp, Int8Tensor):
        raise TypeError("_split_attention: Kp and Vp must both be Int8Tensor or both dense tensors")
    T = Kp.shape[1]
    kvalid = None if pm is None else pm.reshape(1, T).to(torch.uint8).contiguous()
    img = kernels.stage_state_bf16(Kp[None], Vp[None], T, scale, kvalid)
    return kernels.branched_attn_images(q, k, v, img, 1, T, scale).to(v.dtype)


split_attention = _split_attention


def group_rows(row_state: torch.Tensor, n_states: int, max_rows: int | None = None):
    """Rows in any state order -> the grouped layout the one-launch kernels take. row_state (R,) integer device
    tensor, row i reads state row_state[i] (the reference's `rows`, prefix_attn.py:103-117,152-154). Returns
    (order, row_start, max_rows): order (R,) int64 lists the rows grouped by state, stably (rows of one state keep
    their relative order); row_start int32 (n_states + 1,) the groups' offsets in `order`; max_rows the largest
    group. All on the device with no host sync when max_rows is given (a caller that captures a graph knows it);
    otherwise one host read, which also checks that every state index lies in [0, n_states)."""
    rs = row_state.reshape(-1).to(torch.int64)
    order = torch.argsort(rs, stable=True)
    # row_start[s] = number of rows whose state is below s (searchsorted on the sorted states)
    bounds = torch.arange(n_states + 1, dtype=torch.int64, device=rs.device)
    row_start = torch.searchsorted(rs.index_select(0, order), bounds).to(torch.int32)
    if max_rows is None:
        counts = row_start[1:] - row_start[:-1]
        lo, hi, mr = torch.stack([rs.min(), rs.max(), counts.max().to(torch.int64)]).tolist() if rs.numel() else (0, 0, 0)
        if lo < 0 or hi >= n_states:
            raise ValueError(f"row_state values must lie in [0, {n_states}), got [{lo}, {hi}]")
        max_rows = int(mr)
    return order, row_start, int(max_rows)


def split_attention_int8(q, k, v, Kq, Ks, Vq, Vs, pm, scale, row_counts=None, return_lse: bool = False,
                         dequant: str = "bf16", row_state=None, max_rows: int | None = None):
    """The batched form: rows of several states in one launch. q (R, Hq, t, D); k/v (R, Hkv, t, D); Kq/Vq int8
    (Ns, Hkv, T, D) or (Hkv, T, D); Ks/Vs fp32 (Ns, Hkv, T[, 1]); pm (Ns, T) bool or None; dequant as
    _split_attention. Which rows read which state, one of:
      * row_counts: how many consecutive rows belong to each state (rows grouped by state);
      * row_state: (R,) integer device tensor, row i reads state row_state[i], rows in any order (the reference's
        `rows`, prefix_attn.py:152-154); the rows are grouped on the device (group_rows), attended in one launch and
        returned in the caller's order. max_rows: the largest number of rows of one state, when the caller knows it
        (no host sync; the state indices are then trusted to lie in [0, Ns));
      * neither: one state."""
    if Kq.dim() == 3:
        Kq, Vq, Ks, Vs = Kq[None], Vq[None], Ks[None], Vs[None]
    Ks = Ks.float().reshape(Kq.shape[:3]).contiguous()
    Vs = Vs.float().reshape(Vq.shape[:3]).contiguous()
    length = Kq.shape[2] if pm is None else None
    if row_state is None:
        return kernels.branched_attn(q, k, v, Kq.contiguous(), Ks, Vq.contiguous(), Vs, scale, kvalid=pm,
                                     row_counts=row_counts, length=length, return_lse=return_lse, dequant=dequant)
    if row_counts is not None:
        raise ValueError("split_attention_int8: give row_counts or row_state, not both")
    if row_state.numel() != q.shape[0]:
        raise ValueError("split_attention_int8: row_state must have one entry per row")
    order, row_start, max_rows = group_rows(row_state.to(q.device), Kq.shape[0], max_rows)
    res = kernels.branched_attn(q.index_select(0, order), k.index_select(0, order), v.index_select(0, order),
                                Kq.contiguous(), Ks, Vq.contiguous(), Vs, scale, kvalid=pm, length=length,
                                row_start=row_start, max_rows=max_rows, return_lse=return_lse, dequant=dequant)
    out_g, lse_g = res if return_lse else (res, None)
    out = torch.empty_like(out_g).index_copy_(0, order, out_g)
    if not return_lse:
        return out
    return out, torch.empty_like(lse_g).index_copy_(0, order, lse_g)
