"""CPU oracle for the wide flash attention contract and the branched (Hydragen) option-row attention.
TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Conventions followed (reference file:line):
  * wide_attention (wide_attention.py:13-91): q (B,H,T,Dk), k (B,G,S,Dk), v (B,G,S,Dv), GQA with head h reading
    KV group h // (H // G) (:23-25); queries are the LAST T of the S key positions, so query t sits at position
    t + S - T (:26) and under causal=True sees keys 0..t+S-T (:49); kvalid (B,S) masks keys (:50-52); a query
    row with no visible key returns 0 (:62) and LSE -inf (:65-67); LSE is the natural log of the sum of
    exp(scale * q.k) over visible keys (:65-67).
  * _split_attention (prefix_attn.py:43-76): every row's queries attend the shared prefix Kp/Vp (Hkv, T, D) under
    the key mask pm (T,), and the row's own k/v causally (tril over the row's t tokens, :71); the two softmax
    parts are merged by their log-sum-exp (:74-76). The CPU branch (:58-73) computes in fp32 with einsum; where
    every prefix key is masked that branch yields NaN (softmax of an all -inf row), while the CUDA branch yields
    the own part only (wide_attention's empty-row rule). This oracle follows the CUDA branch's rule.
  * int8 state (quant.py:43-45, prefix_attn.py:145-149): the reference dequantizes the state K/V once per layer,
    q.to(bf16) * scale.to(bf16). `dequant="bf16"` restates that exactly; `dequant="fp32"` uses q * scale in fp32,
    which is what a kernel that folds the fp32 scales into the scores computes.
"""
from __future__ import annotations

import contextlib
import math

import torch

NEG_INF = float("-inf")


def _f(x, dt):
    return x.detach().to("cpu").to(dt)


def attention(q, k, v, scale: float, kvalid=None, causal: bool = True, dtype=torch.float32, chunk: int = 1 << 24):
    """wide_attention's contract (wide_attention.py:70-91) as plain softmax attention.
    Returns (o (B,H,T,Dv) `dtype`, lse (B,H,T) `dtype`)."""
    B, H, T, _ = q.shape
    G, S, Dv = k.shape[1], k.shape[2], v.shape[-1]
    rep = H // G
    assert H % G == 0 and v.shape[2] == S
    qf, kf, vf = _f(q, dtype), _f(k, dtype).repeat_interleave(rep, 1), _f(v, dtype).repeat_interleave(rep, 1)
    ok = torch.ones(T, S, dtype=torch.bool)
    if causal:
        ok = torch.arange(S)[None, :] <= (torch.arange(T)[:, None] + (S - T))
    o = torch.zeros(B, H, T, Dv, dtype=dtype)
    lse = torch.full((B, H, T), NEG_INF, dtype=dtype)
    per = max(1, chunk // max(1, H * T * S))
    for b0 in range(0, B, per):
        b1 = min(B, b0 + per)
        s = torch.einsum("bhtd,bhsd->bhts", qf[b0:b1], kf[b0:b1]) * scale
        m = ok[None, None].expand(b1 - b0, H, T, S)
        if kvalid is not None:
            m = m & _f(kvalid[b0:b1], torch.bool)[:, None, None, :]
        s = s.masked_fill(~m, NEG_INF)
        l_ = torch.logsumexp(s, -1)
        p = torch.exp(s - torch.where(torch.isfinite(l_), l_, torch.zeros_like(l_))[..., None])
        p = torch.where(m, p, torch.zeros_like(p))
        o[b0:b1] = p @ vf[b0:b1]
        lse[b0:b1] = l_
    return o, lse


def wide_attention_blocked(q, k, v, scale: float, kvalid=None, causal: bool = True, block: int = 64,
                           with_bound: bool = False):
    """_wide_fwd (wide_attention.py:13-67) step by step in fp32, one key block of `block` keys at a time:
    s = (q.k) * scale * log2(e) with masked keys at -inf (:46-53), m_new = max(m, rowmax s) (:54), m_safe = 0 where
    m_new = -inf (:55), p = exp2(s - m_safe) (:56), alpha = exp2(m - m_safe) (:57), l = l alpha + sum p (:58),
    acc = acc alpha + bf16(p) @ v (:60, p.to(v.dtype) with bf16 v), out = acc / (l or 1) (:62), lse =
    (m + log2 l) ln 2 (:66). The kernel under test runs the same blocking (64 keys), so the bf16 rounding of p
    happens against the same running max. Returns (o (B,H,T,Dv) fp32, lse (B,H,T) fp32) and, with with_bound,
    the per-element bound 2^-7 (sum_j p_j |v_j|) / l on how far an implementation of the same algorithm can move
    when each bf16(p_j) lands on the neighbouring bf16 value (one ulp, at most 2^-7 p_j), e.g. because its exp2
    differs in the last bit."""
    B, H, T, _ = q.shape
    G, S, Dv = k.shape[1], k.shape[2], v.shape[-1]
    rep = H // G
    assert H % G == 0 and v.shape[2] == S
    qf = _f(q, torch.float32)
    kf = _f(k, torch.float32).repeat_interleave(rep, 1)
    vb = _f(v, torch.float32).repeat_interleave(rep, 1)
    c = scale * 1.4426950408889634
    pos = torch.arange(T)[:, None] + (S - T)
    m = torch.full((B, H, T), NEG_INF)
    l_ = torch.zeros(B, H, T)
    acc = torch.zeros(B, H, T, Dv)
    acc_abs = torch.zeros(B, H, T, Dv)
    for n0 in range(0, S, block):
        n1 = min(S, n0 + block)
        s = torch.einsum("bhtd,bhsd->bhts", qf, kf[:, :, n0:n1]) * c
        ok = torch.ones(T, n1 - n0, dtype=torch.bool)
        if causal:
            ok = torch.arange(n0, n1)[None, :] <= pos
        okb = ok[None, None].expand(B, H, T, n1 - n0)
        if kvalid is not None:
            okb = okb & _f(kvalid[:, n0:n1], torch.bool)[:, None, None, :]
        s = torch.where(okb, s, torch.full_like(s, NEG_INF))
        m_new = torch.maximum(m, s.amax(-1))
        m_safe = torch.where(m_new == NEG_INF, torch.zeros_like(m_new), m_new)
        p = torch.exp2(s - m_safe[..., None])
        alpha = torch.exp2(m - m_safe)
        l_ = l_ * alpha + p.sum(-1)
        acc = acc * alpha[..., None] + p.to(torch.bfloat16).float() @ vb[:, :, n0:n1]
        if with_bound:
            acc_abs = acc_abs * alpha[..., None] + p @ vb[:, :, n0:n1].abs()
        m = m_new
    den = torch.where(l_ == 0, torch.ones_like(l_), l_)[..., None]
    out = acc / den
    lse = (m + torch.log2(l_)) * 0.6931471805599453
    if with_bound:
        return out, lse, 2.0 ** -7 * acc_abs / den
    return out, lse


@contextlib.contextmanager
def reference_gpu_arithmetic():
    """Within this context every softmax attention of the oracle (split_attention's prefix and own parts, hence
    branched_attention, two_level_attention and the prefill's causal attention) runs as the reference's CUDA path
    computes it: _split_attention's two wide_attention calls (prefix_attn.py:50-57), i.e. the flash kernel's blocked
    online softmax with P rounded to bf16 before P.V (wide_attention.py:54-62, restated by wide_attention_blocked),
    instead of its CPU branch's one-shot fp32 softmax (prefix_attn.py:58-73). How far the two disagree end to end is
    the spread between the reference's own GPU and CPU paths."""
    global attention
    cpu = attention

    def blocked(q, k, v, scale: float, kvalid=None, causal: bool = True, dtype=torch.float32, chunk: int = 1 << 24):
        o, lse = wide_attention_blocked(q, k, v, scale, kvalid, causal)
        return o.to(dtype), lse.to(dtype)

    attention = blocked
    try:
        yield
    finally:
        attention = cpu


def lse_merge(o_p, l_p, o_o, l_o):
    """The exact merge of two softmax partials (prefix_attn.py:74-76): m = max(l_p, l_o), w = exp(l - m),
    out = (o_p w_p + o_o w_o) / (w_p + w_o). Both parts empty -> 0 output. Returns (out, merged lse)."""
    m = torch.maximum(l_p, l_o)
    m_safe = torch.where(torch.isfinite(m), m, torch.zeros_like(m))
    wp, wo = torch.exp(l_p - m_safe), torch.exp(l_o - m_safe)
    den = wp + wo
    out = (o_p * wp[..., None] + o_o * wo[..., None]) / torch.where(den > 0, den, torch.ones_like(den))[..., None]
    lse = torch.where(den > 0, m_safe + torch.log(torch.where(den > 0, den, torch.ones_like(den))),
                      torch.full_like(den, NEG_INF))
    return out, lse


def split_attention(q, k, v, Kp, Vp, pm, scale: float, dtype=torch.float32):
    """_split_attention (prefix_attn.py:43-76) for rows continuing ONE shared prefix.
    q (n,Hq,t,D), k/v (n,Hkv,t,D), Kp/Vp (Hkv,T,D), pm (T,) bool or None. Returns (out (n,Hq,t,D), lse (n,Hq,t))
    in `dtype` (the reference casts out to v.dtype at the end, :76)."""
    n, Hq, t, D = q.shape
    Hkv, T = Kp.shape[0], Kp.shape[1]
    # prefix part: all rows' queries against the prefix, no causal mask (prefix_attn.py:52-55 / 60-69)
    qs = q.transpose(0, 1).reshape(1, Hq, n * t, D)
    kv = None if pm is None else pm.reshape(1, T)
    o_p, l_p = attention(qs, Kp[None], Vp[None], scale, kv, causal=False, dtype=dtype)
    o_p = o_p.reshape(Hq, n, t, -1).transpose(0, 1)
    l_p = l_p.reshape(Hq, n, t).transpose(0, 1)
    # own part: each row's queries against its own t keys, causal (prefix_attn.py:56 / 70-73)
    o_o, l_o = attention(q, k, v, scale, None, causal=True, dtype=dtype)
    return lse_merge(o_p, l_p, o_o, l_o)


def dequant_state(kq, ks, mode: str = "fp32"):
    """State K or V from int8 + per-(token, head) scale. mode "fp32": q * s in fp32. mode "bf16": the reference's
    materialize, q.to(bf16) * s.to(bf16) rounded to bf16 (quant.py:45), returned as fp32 values."""
    ks = ks.detach().to("cpu")
    if ks.dim() == kq.dim() - 1:
        ks = ks[..., None]
    if mode == "fp32":
        return kq.detach().to("cpu").float() * ks.float()
    if mode == "bf16":
        return (kq.detach().to("cpu").to(torch.bfloat16) * ks.to(torch.bfloat16)).float()
    raise ValueError(mode)


def branched_attention(q, k_own, v_own, Kp, Vp, scale: float, kvalid=None, row_state=None, dtype=torch.float32):
    """_forward's per-state loop (prefix_attn.py:118-128) around _split_attention, for rows of several states.
    q (R,Hq,t,D); k_own/v_own (R,Hkv,t,D); Kp/Vp (Ns,Hkv,T,D) float; kvalid (Ns,T) bool or None; row_state (R,)
    int (state of each row; None -> every row reads state 0). Returns (out (R,Hq,t,D), lse (R,Hq,t))."""
    R, Hq, t, D = q.shape
    rs = torch.zeros(R, dtype=torch.long) if row_state is None else row_state.detach().to("cpu").long()
    out = torch.zeros(R, Hq, t, Vp.shape[-1], dtype=dtype)
    lse = torch.zeros(R, Hq, t, dtype=dtype)
    for s in torch.unique(rs).tolist():
        r = (rs == s).nonzero().squeeze(1)
        pm = None if kvalid is None else kvalid[s].detach().to("cpu").bool()
        o, l_ = split_attention(q[r], k_own[r], v_own[r], Kp[s], Vp[s], pm, scale, dtype)
        out[r], lse[r] = o, l_
    return out, lse


def branched_attention_int8(q, k_own, v_own, kq, ks, vq, vs, scale: float, kvalid=None, row_state=None,
                            dequant: str = "bf16", dtype=torch.float32):
    """The int8-state branched attention: the state K/V are dequantized (dequant_state; "bf16" is the reference's
    materialize, prefix_attn.py:145-149, and the default) and passed to branched_attention. kq/vq (Ns,Hkv,T,D) int8;
    ks/vs (Ns,Hkv,T) fp32."""
    Kp = dequant_state(kq, ks, dequant).to(dtype)
    Vp = dequant_state(vq, vs, dequant).to(dtype)
    return branched_attention(q, k_own, v_own, Kp, Vp, scale, kvalid, row_state, dtype)


def two_level_attention(q, k_own, v_own, kq, ks, vq, vs, Kq2, Vq2, qmask, scale: float, row_group, group_state,
                        dequant: str = "bf16", dtype=torch.float32):
    """The question-cache attention (prefix_attn.py:94-99 then _split_attention): the rows of question g attend the
    prefix [its state's K/V ; question g's own K/V] (state_of_group = group_state[g]; the int8 state dequantized as
    dequant_state; the question K/V dense, pads masked by qmask (G, T2)) and their own tokens causally, merged by
    LSE. q (R,Hq,t,D); k_own/v_own (R,Hkv,t,D); kq/vq (Ns,Hkv,T,D) int8, ks/vs (Ns,Hkv,T); Kq2/Vq2 (G,Hkv,T2,D);
    row_group (R,) int. Returns (out (R,Hq,t,D), lse (R,Hq,t))."""
    Kp = dequant_state(kq, ks, dequant)
    Vp = dequant_state(vq, vs, dequant)
    R, Hq, t, D = q.shape
    rg = row_group.detach().to("cpu").long()
    out = torch.zeros(R, Hq, t, Vp.shape[-1], dtype=dtype)
    lse = torch.zeros(R, Hq, t, dtype=dtype)
    T = Kp.shape[2]
    for gi in torch.unique(rg).tolist():
        r = (rg == gi).nonzero().squeeze(1)
        s = int(group_state[gi])
        K = torch.cat([Kp[s], _f(Kq2[gi], torch.float32)], 1).to(dtype)
        V = torch.cat([Vp[s], _f(Vq2[gi], torch.float32)], 1).to(dtype)
        pm = torch.cat([torch.ones(T, dtype=torch.bool), _f(qmask[gi], torch.bool)])
        o, l_ = split_attention(q[r], k_own[r], v_own[r], K, V, pm, scale, dtype)
        out[r], lse[r] = o, l_
    return out, lse


def brute_force_attention(q, k, v, scale: float, allowed):
    """Scalar float64 softmax attention for tiny shapes: q (Tq, D), k (Tk, D), v (Tk, Dv), allowed[i][j] bool.
    Returns (out (Tq, Dv) float64, lse (Tq,) float64). Used only to pin the vectorised oracle."""
    Tq, Tk = len(q), len(k)
    qd = q.double().tolist()
    kd = k.double().tolist()
    vd = v.double().tolist()
    out, lses = [], []
    for i in range(Tq):
        sc = [sum(a * b for a, b in zip(qd[i], kd[j])) * scale if allowed[i][j] else None for j in range(Tk)]
        vis = [x for x in sc if x is not None]
        if not vis:
            out.append([0.0] * len(vd[0]))
            lses.append(NEG_INF)
            continue
        mx = max(vis)
        w = [math.exp(x - mx) if x is not None else 0.0 for x in sc]
        z = sum(w)
        out.append([sum(w[j] * vd[j][c] for j in range(Tk)) / z for c in range(len(vd[0]))])
        lses.append(mx + math.log(z))
    return torch.tensor(out, dtype=torch.float64), torch.tensor(lses, dtype=torch.float64)
