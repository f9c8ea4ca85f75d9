"""CPU oracle of the decision-forward harness: a dense 9B-class decoder (Qwen3-style layer: RMSNorm, fused QKV,
per-head q/k RMSNorm, rotary embedding, GQA attention, output projection, SwiGLU MLP) whose linears are W8A8 and
whose attention is the branched option-row attention over int8 state K/V, followed by the option readout (mean-pool
each option row, one logit per row, a learned 'none' logit, log-softmax per request).
TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

This layer is the harness that carries the path, not a reference function: the reference runs the same steps inside
HF Qwen3.5 modules (src/opendecider/prefix_attn.py:79-131 for the attention layer, the W8A8 linears in every
nn.Linear slot, decision logits + 'none' at src/opendecider/v3.py:639-643,701-709 and softmax at
src/opendecider/decider.py:255-257). Rounding follows torch bf16 module arithmetic: every elementwise product of
bf16 tensors rounds to bf16 once.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import attention as oa
from . import quant as oq


@dataclass
class DecoderConfig:
    hidden: int = 4096
    ffn: int = 12288
    n_heads: int = 32
    n_kv_heads: int = 8
    head_dim: int = 128
    n_layers: int = 36
    vocab: int = 151936
    eps: float = 1e-6
    theta: float = 1e6
    gated: bool = False  # Qwen3.5's output gate: q_proj gives each head's q and gate (prefix_attn.py:84-85,130)
    # Qwen3.5's hybrid stack (the backbone's layer_types, src/opendecider/backbone.py:75,270; transformers'
    # Qwen3_5TextConfig): with an interval n > 0, layer i is full attention when (i + 1) % n == 0, a Gated DeltaNet
    # layer otherwise (oracle/gdn.py); 0 keeps every layer full attention.
    full_attention_interval: int = 0
    lin_k_heads: int = 16
    lin_v_heads: int = 32
    lin_k_dim: int = 128
    lin_v_dim: int = 128
    conv_kernel: int = 4
    # Qwen3.5's attention geometry (transformers' Qwen3_5TextConfig / Qwen3_5Attention): rotary embedding on the first
    # rot_dim dims of each head only (partial_rotary_factor 0.25 of head_dim 256; 0 = the whole head), and every
    # RMSNorm of the decoder (input / post-attention / q / k / final) zero-centred, Qwen3_5RMSNorm's
    # (x * r) * (1 + w), instead of w * bf16(x * r).
    rot_dim: int = 0
    norm_offset: bool = False

    @property
    def rotary_dims(self) -> int:
        return self.rot_dim or self.head_dim

    @property
    def qkv_out(self) -> int:
        return (self.n_heads * (2 if self.gated else 1) + 2 * self.n_kv_heads) * self.head_dim

    def is_gdn(self, li: int) -> bool:
        n = self.full_attention_interval
        return n > 0 and (li + 1) % n != 0

    @property
    def gdn(self):
        from .gdn import GDNConfig
        return GDNConfig(hidden=self.hidden, n_k_heads=self.lin_k_heads, n_v_heads=self.lin_v_heads,
                         dk=self.lin_k_dim, dv=self.lin_v_dim, conv=self.conv_kernel, eps=self.eps)


def make_weights(cfg: DecoderConfig, seed: int = 0, device="cpu", layers: int | None = None, smooth: bool = True):
    """Random-init weights of the decoder (bf16, N(0, 0.02) linears, norms near 1) and SmoothQuant factors
    s ~ U(0.5, 2) per linear input. Deterministic for a seed and device. Returns a dict."""
    g = torch.Generator(device=device).manual_seed(seed)
    bf = torch.bfloat16
    H, F, D = cfg.hidden, cfg.ffn, cfg.head_dim

    def lin(n, k):
        return (torch.randn(n, k, generator=g, device=device) * 0.02).to(bf)

    def norm(n):  # near 1 as applied: 1 + w with the zero-centred weights
        return ((0.0 if cfg.norm_offset else 1.0) + 0.1 * torch.randn(n, generator=g, device=device)).to(bf)

    def sm(n):
        return (torch.rand(n, generator=g, device=device) * 1.5 + 0.5) if smooth else None

    out = {"layers": []}
    for li in range(cfg.n_layers if layers is None else layers):
        if cfg.is_gdn(li):  # a GDN token mixer (oracle/gdn.py) with the same norms and MLP
            from .gdn import make_gdn_weights
            lw = {"ln1": norm(H), "ln2": norm(H)}
            lw.update(make_gdn_weights(cfg.gdn, g, device, smooth))
            lw.update({"wgu": lin(2 * F, H), "wdown": lin(H, F), "s_gu": sm(H), "s_down": sm(F)})
            out["layers"].append(lw)
            continue
        out["layers"].append({
            "ln1": norm(H), "ln2": norm(H), "q_norm": norm(D), "k_norm": norm(D),
            "wqkv": lin(cfg.qkv_out, H), "wo": lin(H, cfg.n_heads * D), "wgu": lin(2 * F, H), "wdown": lin(H, F),
            "s_qkv": sm(H), "s_o": sm(cfg.n_heads * D), "s_gu": sm(H), "s_down": sm(F),
        })
    out["final_norm"] = norm(H)
    out["head"] = (torch.randn(H, generator=g, device=device) / H ** 0.5).float()
    out["none_logit"] = torch.zeros((), device=device)
    return out


def make_embedding(cfg: DecoderConfig, seed: int = 0, device="cpu"):
    g = torch.Generator(device=device).manual_seed(seed + 7919)
    return torch.randn(cfg.vocab, cfg.hidden, generator=g, device=device).to(torch.bfloat16)


def quantize_linear(w: torch.Tensor, s: torch.Tensor | None):
    """SmoothQuant fold W * s (quant.py:343-344), per-channel int8 (quant.py:124-126), bf16(1/s) (quant.py:325)."""
    if s is not None:
        w = oq.smooth_fold(w, s)
    q, sw = oq.quantize_weight(w)
    return q, sw, None if s is None else oq.smooth_inv(s)


def rope_tables(cfg: DecoderConfig, n_pos: int):
    """cos/sin bf16 tables [n_pos, R/2] over the R = cfg.rotary_dims rotated dims: inv_freq = 1 / theta^(2i/R), angle
    = pos * inv_freq in fp32 (transformers' default rope parameters take dim = head_dim * partial_rotary_factor)."""
    D = cfg.rotary_dims
    inv_freq = 1.0 / (cfg.theta ** (torch.arange(0, D, 2, dtype=torch.int64).float() / D))
    ang = torch.arange(n_pos, dtype=torch.float32)[:, None] * inv_freq[None, :]
    return ang.cos().to(torch.bfloat16), ang.sin().to(torch.bfloat16)


def rms_factor(x: torch.Tensor, eps: float) -> torch.Tensor:
    """r = 1 / sqrt(mean(x^2) + eps) over the last dim, the HF RMSNorm factor (fp32 in the reference:
    torch.rsqrt(x.float().pow(2).mean(-1) + eps)), evaluated in float64 and rounded once to fp32: the correctly
    rounded value of that expression (the reference's fp32 evaluation lands within a few fp32 ulps of it). The
    squares of bf16 / fp32 inputs are exact in float64 and their sum is exact unless the row spans more than ~25
    binades, so the result does not depend on the summation order; eps enters as the fp32 value the reference adds."""
    xd = x.detach().to("cpu").double()
    ms = (xd * xd).sum(-1, keepdim=True) / xd.shape[-1]
    eps32 = float(torch.tensor(eps, dtype=torch.float32))
    return (1.0 / torch.sqrt(ms + eps32)).float()


def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float, offset: bool = False) -> torch.Tensor:
    """w * bf16(x * r) in bf16 (the HF RMSNorm arithmetic: x * r in fp32, rounded to bf16, times the bf16 weight,
    rounded again), r = rms_factor(x). offset: Qwen3.5's zero-centred norm (transformers' Qwen3_5RMSNorm.forward:
    output = norm(x.float()) * (1.0 + weight.float()), then .type_as(x)): (x * r) * (1 + w) with the sum and both
    products in fp32, rounded once to bf16."""
    xf = x.float()
    if offset:
        return ((xf * rms_factor(xf, eps)) * (1.0 + w.float())).to(torch.bfloat16)
    return w * (xf * rms_factor(xf, eps)).to(torch.bfloat16)


def qk_norm_rope(qkv: torch.Tensor, cfg: DecoderConfig, q_w, k_w, cos, sin, pos) -> torch.Tensor:
    """Per-head RMSNorm of the q and k heads of qkv (M, qkv_out) (zero-centred with cfg.norm_offset), then
    rotate_half RoPE on the first R = cfg.rotary_dims dims of each head, the other D - R passing through (transformers'
    apply_rotary_pos_emb for a table narrower than the head: q_embed = cat((q_rot * cos) + (rotate_half(q_rot) *
    sin), q_pass)); v untouched."""
    M = qkv.shape[0]
    D, Hq, Hk = cfg.head_dim, cfg.n_heads, cfg.n_kv_heads
    R = cfg.rotary_dims
    L = R // 2
    out = qkv.clone()
    c = cos[pos].repeat(1, 2)[:, None, :]            # (M, 1, R), halves shared
    s = sin[pos].repeat(1, 2)[:, None, :]
    for lo, nh, w in ((0, Hq, q_w), (Hq * D, Hk, k_w)):
        x = qkv[:, lo:lo + nh * D].reshape(M, nh, D)
        n = rmsnorm(x, w, cfg.eps, cfg.norm_offset)
        nr = n[..., :R]
        rot = torch.cat([-nr[..., L:], nr[..., :L]], -1)
        out[:, lo:lo + nh * D] = torch.cat([(nr * c) + (rot * s), n[..., R:]], -1).reshape(M, nh * D)
    return out


def silu_bf16(g: torch.Tensor) -> torch.Tensor:
    """bf16(silu(g)) for bf16 g, with silu(g) = g / (1 + exp(-g)) evaluated in float64 and rounded once to fp32
    before the bf16 rounding: the reference's F.silu on a bf16 tensor computes g / (1 + exp(-g)) in fp32 and rounds
    to bf16; this is that fp32 value correctly rounded. g has 65536 possible values, so the function is a table
    that a kernel can be checked against exhaustively."""
    gd = g.double()
    return (gd / (1.0 + torch.exp(-gd))).float().to(torch.bfloat16)


def sigmoid_bf16(g: torch.Tensor) -> torch.Tensor:
    """bf16(sigmoid(g)) for bf16 g, sigmoid(g) = 1 / (1 + exp(-g)) evaluated in float64 and rounded once to fp32
    before the bf16 rounding (torch's sigmoid on a bf16 tensor computes in fp32 and rounds to bf16)."""
    gd = g.double()
    return (1.0 / (1.0 + torch.exp(-gd))).float().to(torch.bfloat16)


def split_qkv(qkv: torch.Tensor, cfg: DecoderConfig):
    """The fused projection's output in the reference's layout -> (q|k|v (M, (Hq + 2 Hkv) D), gate (M, Hq D) or
    None). Gated: q_proj's rows hold each head's q then its gate, (Hq, 2D) per token (prefix_attn.py:84-85), then
    k_proj's and v_proj's rows."""
    if not cfg.gated:
        return qkv, None
    M = qkv.shape[0]
    D, Hq = cfg.head_dim, cfg.n_heads
    qg = qkv[:, :2 * Hq * D].reshape(M, Hq, 2 * D)
    q, gate = qg[..., :D].reshape(M, Hq * D), qg[..., D:].reshape(M, Hq * D)
    return torch.cat([q, qkv[:, 2 * Hq * D:]], 1), gate


def output_gate(attn: torch.Tensor, gate: torch.Tensor | None) -> torch.Tensor:
    """o * sigmoid(gate) (prefix_attn.py:130): the bf16 product of the attention output and bf16(sigmoid(gate))."""
    return attn if gate is None else attn * sigmoid_bf16(gate)


def swiglu(gu: torch.Tensor, F: int) -> torch.Tensor:
    """bf16(bf16(silu(g)) * u) with g = gu[:, :F], u = gu[:, F:] (torch's bf16 product: fp32 product, one
    rounding)."""
    return silu_bf16(gu[:, :F]) * gu[:, F:]


def _layer_tail(h, attn, qlin, lw, cfg: DecoderConfig, o_proj: str = "wo"):
    """O projection (o_proj: "wo", or a GDN layer's "wout") + residual, RMSNorm, gate+up, SwiGLU, down + residual
    (each linear W8A8 with its fused activation quantizer)."""
    q, sw, inv = qlin[o_proj]
    h, _, _, _ = oq.w8a8_linear(attn, q, sw, inv_s=inv, residual=h)
    x = rmsnorm(h, lw["ln2"], cfg.eps, cfg.norm_offset)
    q, sw, inv = qlin["wgu"]
    gu, _, _, _ = oq.w8a8_linear(x, q, sw, inv_s=inv)
    a = swiglu(gu, cfg.ffn)
    q, sw, inv = qlin["wdown"]
    h, _, _, _ = oq.w8a8_linear(a, q, sw, inv_s=inv, residual=h)
    return h


def layer_forward(h, lw, qlin, cfg: DecoderConfig, state_k, state_v, R: int, t: int, pos, cos, sin,
                  row_state=None, kvalid=None, attn_hook=None, dequant: str = "bf16", attn_dtype=torch.float32,
                  capture=None, two_level=None):
    """One decoder layer over the option-row tokens h (M = R * t, hidden) bf16. qlin: {name: (q, sw, inv_s)}.
    state_k/state_v: (kq int8 (Ns, Hkv, T, D), ks fp32 (Ns, Hkv, T)) of this layer. attn_hook, if given, maps the
    bf16 attention output (M, Hq D) to the tensor used downstream (sensitivity studies). dequant: how the int8 state
    becomes K/V ("bf16": the reference's materialize, q.to(bf16) * s.to(bf16), prefix_attn.py:145-149; "fp32": q * s
    exact); attn_dtype: the attention's arithmetic (fp32 as the reference's CPU branch, or float64 to measure how
    much the result depends on the accumulation). capture: a list that receives this layer's (k, v) (R, Hkv, t, D)
    bf16 after q/k norm + RoPE (the question pass's capture, prefix_attn.py:92-93). two_level: (Kq2, Vq2, qmask,
    row_group, group_state) to attend the two-level prefix instead (prefix_attn.py:94-99). Returns the new h."""
    D, Hq, Hk = cfg.head_dim, cfg.n_heads, cfg.n_kv_heads
    x = rmsnorm(h, lw["ln1"], cfg.eps, cfg.norm_offset)
    q, sw, inv = qlin["wqkv"]
    qkv, _, _, _ = oq.w8a8_linear(x, q, sw, inv_s=inv)
    qkv, gate = split_qkv(qkv, cfg)
    qkv = qk_norm_rope(qkv, cfg, lw["q_norm"], lw["k_norm"], cos, sin, pos)
    qh = qkv[:, :Hq * D].reshape(R, t, Hq, D).transpose(1, 2)
    kh = qkv[:, Hq * D:(Hq + Hk) * D].reshape(R, t, Hk, D).transpose(1, 2)
    vh = qkv[:, (Hq + Hk) * D:].reshape(R, t, Hk, D).transpose(1, 2)
    if capture is not None:
        capture.append((kh.contiguous(), vh.contiguous()))
    if two_level is not None:
        Kq2, Vq2, qmask, row_group, group_state = two_level
        o, _ = oa.two_level_attention(qh, kh, vh, state_k[0], state_k[1], state_v[0], state_v[1], Kq2, Vq2, qmask,
                                      D ** -0.5, row_group, group_state, dequant=dequant, dtype=attn_dtype)
    else:
        o, _ = oa.branched_attention_int8(qh, kh, vh, state_k[0], state_k[1], state_v[0], state_v[1], D ** -0.5,
                                          kvalid, row_state, dequant=dequant, dtype=attn_dtype)
    attn = o.to(torch.bfloat16).transpose(1, 2).reshape(R * t, Hq * D)
    if attn_hook is not None:
        attn = attn_hook(attn)
    return _layer_tail(h, output_gate(attn, gate), qlin, lw, cfg)


def prefill_forward(ids, weights, embed, cfg: DecoderConfig, state_kv=None, n0: int = 0, kvalid=None,
                    attn_hook=None, dequant: str = "bf16", attn_dtype=torch.float32, gdn_dtype=torch.float64):
    """State pass over S new tokens of each of B states (ids (B, S)) appended after n0 cached tokens.
    n0 = 0: causal attention among the new tokens on their bf16 K/V (exact softmax attention, the contract of the
    backbone's attention on the state, wide_attention.py:70-91). n0 > 0: the new tokens attend the cached int8 state
    (state_kv[l] = ((kq, ks), (vq, vs)) of length n0) and themselves causally, merged by LSE (one row per state,
    prefix_attn.py:43-76). Then only the new tokens' K/V are quantized per (token, head) and appended
    (state_cache.py:79, quant.py:36-41). A GDN layer continues each state's conv and recurrent state (zeros at
    n0 = 0) and returns the new ones in its slot. dequant / attn_dtype as layer_forward. Returns (h (B S, hidden)
    bf16, the per-layer state K/V of length n0 + S, (conv, rec) for GDN layers)."""
    B, S = ids.shape
    D, Hq, Hk = cfg.head_dim, cfg.n_heads, cfg.n_kv_heads
    h = embed[ids.reshape(-1)]
    pos = (n0 + torch.arange(S)).repeat(B)
    cos, sin = rope_tables(cfg, n0 + S)
    out_kv = []
    for li, lw in enumerate(weights["layers"]):
        qlin = quantize_layer(lw)
        if cfg.is_gdn(li):  # state i continues its own conv / recurrent state (or starts from zeros)
            if kvalid is not None:
                raise ValueError("prefill_forward: key masks are not defined for GDN layers")
            conv, rec = (None, None) if n0 == 0 else state_kv[li]
            h, conv, rec = gdn_layer_forward(h, lw, qlin, cfg, B, S, conv, rec, None, gdn_dtype)
            out_kv.append((conv, rec))
            continue
        x = rmsnorm(h, lw["ln1"], cfg.eps, cfg.norm_offset)
        q, sw, inv = qlin["wqkv"]
        qkv, _, _, _ = oq.w8a8_linear(x, q, sw, inv_s=inv)
        qkv, gate = split_qkv(qkv, cfg)
        qkv = qk_norm_rope(qkv, cfg, lw["q_norm"], lw["k_norm"], cos, sin, pos)
        qh = qkv[:, :Hq * D].reshape(B, S, Hq, D).transpose(1, 2)
        kh = qkv[:, Hq * D:(Hq + Hk) * D].reshape(B, S, Hk, D).transpose(1, 2)
        vh = qkv[:, (Hq + Hk) * D:].reshape(B, S, Hk, D).transpose(1, 2)
        if n0 == 0:
            o, _ = oa.attention(qh, kh, vh, D ** -0.5, kvalid, causal=True, dtype=attn_dtype)
        else:
            (kq, ks), (vq, vs) = state_kv[li]
            o, _ = oa.branched_attention_int8(qh, kh, vh, kq, ks, vq, vs, D ** -0.5, kvalid, torch.arange(B),
                                              dequant=dequant, dtype=attn_dtype)
        attn = o.to(torch.bfloat16).transpose(1, 2).reshape(B * S, Hq * D)
        if attn_hook is not None:
            attn = attn_hook(attn)
        kq_new, ks_new = oq.quantize_rows(kh.contiguous())
        vq_new, vs_new = oq.quantize_rows(vh.contiguous())
        ks_new, vs_new = ks_new[..., 0], vs_new[..., 0]
        if n0 > 0:
            (kq, ks), (vq, vs) = state_kv[li]
            kq_new, ks_new = torch.cat([kq, kq_new], 2), torch.cat([ks, ks_new], 2)
            vq_new, vs_new = torch.cat([vq, vq_new], 2), torch.cat([vs, vs_new], 2)
        out_kv.append(((kq_new, ks_new), (vq_new, vs_new)))
        h = _layer_tail(h, output_gate(attn, gate), qlin, lw, cfg)
    return h, out_kv


def quantize_layer(lw):
    names = ("win", "wout", "wgu", "wdown") if "win" in lw else ("wqkv", "wo", "wgu", "wdown")
    return {k: quantize_linear(lw[k], lw["s_" + k[1:]]) for k in names}


def gdn_layer_forward(h, lw, qlin, cfg: DecoderConfig, S: int, L: int, conv_state=None, rec_state=None,
                      seq_state=None, dtype=torch.float64, seq_len=None):
    """One Gated DeltaNet layer over S sequences of L tokens (h (S L, hidden) bf16): RMSNorm, the GDN token mixer
    (oracle/gdn.py's gdn_mixer: in_proj, conv + SiLU, l2norm, gates, gated delta rule, gated RMSNorm) continuing
    the states conv_state / rec_state (seq_state: each sequence's state; None: sequence i continues state i; None
    states: fresh sequences), out_proj + residual, then the MLP as in an attention layer. Returns (h, new conv states
    (S, 3, C), new recurrent states (S, n_v, dk, dv) fp32)."""
    from .gdn import gdn_mixer
    x = rmsnorm(h, lw["ln1"], cfg.eps, cfg.norm_offset)
    out, conv, rec = gdn_mixer(x, lw, qlin, cfg.gdn, S, L, conv_state, rec_state, seq_state, dtype, seq_len)
    return _layer_tail(h, out, qlin, lw, cfg, "wout"), conv, rec


def readout(h, final_norm, head, none_logit, cfg: DecoderConfig, B: int, n_opt: int, t: int,
            temperature: float = 1.0, pool_last: int | None = None):
    """Mean-pool each option row's final-normed hidden states (its last pool_last tokens when given: the option's
    own tokens of a row that also carries its question), one logit per row (pooled . head), append the 'none' logit,
    divide by the decision temperature (the reference's softmax(logits / T), decider.py:255-257) and log-softmax per
    request. Returns (B, n_opt + 1) fp32 log-probabilities."""
    hf = rmsnorm(h, final_norm, cfg.eps, cfg.norm_offset).float().reshape(B, n_opt, t, -1)
    hf = (hf if pool_last is None else hf[:, :, t - pool_last:]).mean(2)
    logits = hf @ head.float()
    logits = torch.cat([logits, none_logit.float().expand(B, 1)], 1)
    return torch.log_softmax(logits / temperature, -1)


def nudge_bf16(x: torch.Tensor, frac: float, seed: int) -> torch.Tensor:
    """x (bf16) with a seeded `frac` of its elements moved by one bf16 step up or down: a perturbation the size of
    one rounding difference, used to measure how strongly the forward amplifies rounding noise."""
    g = torch.Generator().manual_seed(seed)
    bits = x.contiguous().view(torch.int16)
    flip = ((torch.rand(bits.shape, generator=g) < frac) & (x.contiguous() != 0)).to(torch.int16)  # zeros stay
    sign = (torch.randint(0, 2, bits.shape, generator=g) * 2 - 1).to(torch.int16)
    return (bits + flip * sign).view(torch.bfloat16)


def decision_forward(ids, weights, embed, cfg: DecoderConfig, state_kv, T: int, kvalid=None, attn_hook=None,
                     dequant: str = "bf16", attn_dtype=torch.float32, temperature: float | None = None,
                     pool_last: int | None = None, gdn_dtype=torch.float64):
    """Option-row scoring pass: ids (B, n_opt, t) token ids; state_kv[l] = ((kq, ks), (vq, vs)) per layer for the
    B cached states of length T (for a GDN layer: (conv (B, 3, C) bf16, rec (B, n_v, dk, dv) fp32)). dequant /
    attn_dtype as layer_forward, temperature as readout (None: the weights' "temperature", 1 if absent), gdn_dtype
    the GDN recurrence's arithmetic (float64: the value an fp32 evaluation approximates). Returns (B, n_opt + 1)
    log-probabilities."""
    if temperature is None:
        temperature = float(weights.get("temperature", 1.0))
    B, n_opt, t = ids.shape
    R = B * n_opt
    h = embed[ids.reshape(-1)]
    pos = (T + torch.arange(t)).repeat(R)
    cos, sin = rope_tables(cfg, T + t)
    row_state = torch.arange(B).repeat_interleave(n_opt)
    for li, lw in enumerate(weights["layers"]):
        if cfg.is_gdn(li):  # state_kv[li] = (conv states, recurrent states); rows read their request's, in place
            h, _, _ = gdn_layer_forward(h, lw, quantize_layer(lw), cfg, R, t, state_kv[li][0], state_kv[li][1],
                                        row_state, gdn_dtype)
            continue
        h = layer_forward(h, lw, quantize_layer(lw), cfg, state_kv[li][0], state_kv[li][1], R, t, pos, cos, sin,
                          row_state, kvalid, attn_hook, dequant, attn_dtype)
    return readout(h, weights["final_norm"], weights["head"], weights["none_logit"], cfg, B, n_opt, t, temperature,
                   pool_last)


def question_forward(ids_q, weights, embed, cfg: DecoderConfig, state_kv, T: int, group_state, attn_dtype=torch.float32,
                     qlen=None, gdn_dtype=torch.float64):
    """The question pass of the question cache (v3.py:446-534, the capture of prefix_attn.py:92-93): question g's
    Lq tokens (ids_q (G, Lq), right-padded), at positions T .. T + Lq - 1 after its state group_state[g], attend that
    state's int8 K/V and themselves causally through every layer. Pads come after the real tokens, so no real token
    sees them; they are masked as keys by the rows. A Gated DeltaNet layer continues the question's state
    (state_kv[l] = (conv, rec) of the states) over its real tokens qlen[g] as the reference's batched question pass
    does (Backbone.padded_continuation, v3.py:494-497): pads leave the recurrent state unchanged and the new conv
    state ends at the last real token. Returns per layer [(K, V) (G, Hkv, Lq, D) bf16] or, for a GDN layer, the
    questions' (conv (G, 3, C), rec (G, Hv, dk, dv)) states."""
    G, Lq = ids_q.shape
    h = embed[ids_q.reshape(-1)]
    pos = (T + torch.arange(Lq)).repeat(G)
    cos, sin = rope_tables(cfg, T + Lq)
    gs = torch.as_tensor(group_state).long()
    out = []
    for li, lw in enumerate(weights["layers"]):
        if cfg.is_gdn(li):
            if qlen is None:
                raise ValueError("question_forward: a GDN layer needs the questions' real lengths (qlen)")
            h, conv, rec = gdn_layer_forward(h, lw, quantize_layer(lw), cfg, G, Lq, state_kv[li][0], state_kv[li][1],
                                             gs, gdn_dtype, seq_len=qlen)
            out.append((conv, rec))
            continue
        h = layer_forward(h, lw, quantize_layer(lw), cfg, state_kv[li][0], state_kv[li][1], G, Lq, pos, cos, sin,
                          gs, attn_dtype=attn_dtype, capture=out)
    return out


def qcache_decision_forward(ids_o, weights, embed, cfg: DecoderConfig, state_kv, T: int, q_kv, qlen, group_state,
                            attn_dtype=torch.float32, temperature: float | None = None, gdn_dtype=torch.float64):
    """Option rows over the question cache: ids_o (G, n_opt, t); the rows of question g start right after their
    question's last real token (position T + qlen[g], v3.py:520) and attend [state group_state[g] ; question g's K/V
    from question_forward, keys past qlen[g] masked] + their own tokens causally (prefix_attn.py:94-99); in a GDN
    layer they continue their question's (conv, rec) state from question_forward. Returns (G, n_opt + 1)
    log-probabilities."""
    if temperature is None:
        temperature = float(weights.get("temperature", 1.0))
    G, n_opt, t = ids_o.shape
    R = G * n_opt
    qlen = torch.as_tensor(qlen).long()
    Lq = next(kv[0].shape[2] for li, kv in enumerate(q_kv) if not cfg.is_gdn(li))
    row_group = torch.arange(G).repeat_interleave(n_opt)
    pos = (T + qlen[row_group][:, None] + torch.arange(t)[None, :]).reshape(-1)
    qmask = torch.arange(Lq)[None, :] < qlen[:, None]
    cos, sin = rope_tables(cfg, T + Lq + t)
    gs = torch.as_tensor(group_state).long()
    h = embed[ids_o.reshape(-1)]
    for li, lw in enumerate(weights["layers"]):
        if cfg.is_gdn(li):
            h, _, _ = gdn_layer_forward(h, lw, quantize_layer(lw), cfg, R, t, q_kv[li][0], q_kv[li][1], row_group,
                                        gdn_dtype)
            continue
        Kq2, Vq2 = q_kv[li]
        h = layer_forward(h, lw, quantize_layer(lw), cfg, state_kv[li][0], state_kv[li][1], R, t, pos, cos, sin,
                          attn_dtype=attn_dtype, two_level=(Kq2, Vq2, qmask, row_group, gs))
    return readout(h, weights["final_norm"], weights["head"], weights["none_logit"], cfg, G, n_opt, t, temperature)
