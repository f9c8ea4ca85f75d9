"""CPU oracle of the Gated DeltaNet (linear-attention) layer of the Qwen3.5 hybrid backbone. TEST INFRASTRUCTURE ONLY
(see oracle/__init__.py).

The reference runs these layers inside HF transformers' Qwen3.5 modules (the reference pins transformers>=5.2,
pyproject.toml:8; the algorithm below is read from transformers 5.15.0, models/qwen3_5/modeling_qwen3_5.py:
Qwen3_5GatedDeltaNet.forward, causal_conv1d_fn / causal_conv1d_update, l2norm, torch_recurrent_gated_delta_rule,
torch_chunk_gated_delta_rule, Qwen3_5RMSNormGated), through the reference's continuation / state paths
(src/opendecider/backbone.py:256-289, src/opendecider/skipkv.py:208-231). Branch rows continue a shared prefix
state; the reference copies that state per row, and docs/branched_shared_prefix_math.md:16-37 shows the rows need
only read it. Per token of a sequence, per value head (state S in R^{dk x dv}, fp32):

    qkv = in_proj(x); conv (kernel 4, depthwise, causal, continuing the previous 3 inputs) + SiLU -> q, k, v
    q, k <- l2norm(q), l2norm(k) (bf16 arithmetic); beta = sigmoid(b); g = -exp(A_log) softplus(a + dt_bias)
    S <- S e^g ; kv = S^T k ; delta = (v - kv) beta ; S <- S + k delta^T ; o = S^T (q / sqrt(dk))
    out = RMSNormGated(o, z) = bf16(bf16(w * bf16(o * rms(o))) * silu(z)); h += out_proj(out)

Rounding follows the torch module arithmetic on bf16 tensors (each bf16 elementwise op rounds once); where torch's
own evaluation order is not defined (sums), the oracle takes the exact (float64) value rounded once, so that a
kernel can match it bit for bit: the conv, the l2norm, the gates and the gated norm are bit-exact targets, the
recurrence (fp32 state, reductions in hardware order) a tolerance target.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import quant as oq


@dataclass
class GDNConfig:
    hidden: int = 4096
    n_k_heads: int = 16
    n_v_heads: int = 32
    dk: int = 128
    dv: int = 128
    conv: int = 4
    eps: float = 1e-6

    @property
    def key_dim(self) -> int:
        return self.n_k_heads * self.dk

    @property
    def value_dim(self) -> int:
        return self.n_v_heads * self.dv

    @property
    def conv_dim(self) -> int:
        return 2 * self.key_dim + self.value_dim

    @property
    def proj_out(self) -> int:
        # one fused input projection: [qkv (conv_dim) | z (value_dim) | b (n_v) | a (n_v)]
        return self.conv_dim + self.value_dim + 2 * self.n_v_heads


def make_gdn_weights(cfg: GDNConfig, g: torch.Generator, device="cpu", smooth: bool = True) -> dict:
    """Random-init weights of one GDN layer: the fused input projection (the reference's in_proj_qkv, in_proj_z,
    in_proj_b, in_proj_a rows stacked) and out_proj N(0, 0.02); conv weights N(0, 0.3); A = U(0.5, 16) (A_log =
    log A, HF's init range) and dt_bias ~ 1 + 0.1 N(0, 1), both stored in bf16 as a bf16 model holds them; the
    gated norm's weight near 1; SmoothQuant factors U(0.5, 2) per linear input."""
    bf = torch.bfloat16
    H = cfg.hidden
    A = torch.rand(cfg.n_v_heads, generator=g, device=device) * 15.5 + 0.5
    return {
        "win": (torch.randn(cfg.proj_out, H, generator=g, device=device) * 0.02).to(bf),
        "conv_w": (torch.randn(cfg.conv_dim, cfg.conv, generator=g, device=device) * 0.3).to(bf),
        "A_log": torch.log(A).to(bf),
        "dt_bias": (1.0 + 0.1 * torch.randn(cfg.n_v_heads, generator=g, device=device)).to(bf),
        "gnorm": (1.0 + 0.1 * torch.randn(cfg.dv, generator=g, device=device)).to(bf),
        "wout": (torch.randn(H, cfg.value_dim, generator=g, device=device) * 0.02).to(bf),
        "s_in": (torch.rand(H, generator=g, device=device) * 1.5 + 0.5) if smooth else None,
        "s_out": (torch.rand(cfg.value_dim, generator=g, device=device) * 1.5 + 0.5) if smooth else None,
    }


def split_proj(proj: torch.Tensor, cfg: GDNConfig):
    """(M, proj_out) -> qkv (M, conv_dim), z (M, value_dim), b (M, n_v), a (M, n_v)."""
    c, v = cfg.conv_dim, cfg.value_dim
    return proj[:, :c], proj[:, c:c + v], proj[:, c + v:c + v + cfg.n_v_heads], proj[:, c + v + cfg.n_v_heads:]


def conv_silu(x: torch.Tensor, w: torch.Tensor, state: torch.Tensor | None, lens=None):
    """Causal depthwise conv over the sequence axis + SiLU (causal_conv1d_fn / causal_conv1d_update with SiLU).
    x (S, L, C) bf16 pre-conv inputs of S sequences; w (C, K) bf16; state (S, K-1, C) bf16: the previous K-1 inputs
    of each sequence (None: zeros, a fresh sequence). y[t, c] = sum_j w[c, j] full[t + j, c] over full = [state ; x],
    taken exactly (float64) and rounded once to bf16 (torch's bf16 conv accumulates in fp32 and rounds), then
    bf16(silu(y)). Returns (y (S, L, C) bf16, the new state: the last K-1 inputs of [state ; x]; with lens (S,), the
    real lengths of right-padded sequences, the K-1 inputs ending at each sequence's last real token, the gather of
    Backbone.padded_continuation, src/opendecider/backbone.py:284-289)."""
    S, L, C = x.shape
    K = w.shape[1]
    if state is None:
        state = torch.zeros(S, K - 1, C, dtype=x.dtype)
    full = torch.cat([state.to(x.dtype), x], 1).double()
    wd = w.double()
    y = torch.zeros(S, L, C, dtype=torch.float64)
    for j in range(K):
        y += full[:, j:j + L, :] * wd[:, j]
    y = y.float().to(torch.bfloat16)
    from .decoder import silu_bf16
    if lens is None:
        return silu_bf16(y), full[:, L:, :].to(x.dtype)
    idx = torch.as_tensor(lens).long()[:, None] + torch.arange(K - 1)[None, :]
    return silu_bf16(y), torch.stack([full[s, idx[s]] for s in range(S)]).to(x.dtype)


def l2norm_bf16(x: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """transformers' l2norm on a bf16 tensor (x * rsqrt((x * x).sum(-1) + eps)) in torch's bf16 arithmetic: the
    squares rounded to bf16, their sum (exact, rounded once to bf16), + eps rounded to bf16, rsqrt rounded to bf16,
    the product rounded to bf16."""
    xf = x.float()
    sq = (xf * xf).to(torch.bfloat16)
    s = sq.double().sum(-1, keepdim=True).float().to(torch.bfloat16)
    den = (s.float() + torch.tensor(eps, dtype=torch.float32)).to(torch.bfloat16)
    inv = (1.0 / torch.sqrt(den.double())).float().to(torch.bfloat16)
    return (xf * inv.float()).to(torch.bfloat16)


def _f32(x: torch.Tensor) -> torch.Tensor:
    return x.float()


def gates(a: torch.Tensor, b: torch.Tensor, A_log: torch.Tensor, dt_bias: torch.Tensor):
    """beta = bf16(sigmoid(b)) (b.sigmoid() on bf16) and g = -exp(A_log) * softplus(a + dt_bias) in fp32 (the
    reference upcasts a, A_log and dt_bias), each fp32 operation correctly rounded (float64, rounded to fp32);
    softplus(x) = x above 20 (torch's threshold), else log1p(exp(x)). Returns (g fp32, beta fp32 holding bf16
    values)."""
    from .decoder import sigmoid_bf16
    beta = sigmoid_bf16(b).float()
    e = torch.exp(A_log.double()).float()
    x = (a.double() + dt_bias.double()).float()
    xd = x.double()
    sp = torch.where(xd > 20.0, xd, torch.log1p(torch.exp(xd))).float()
    g = (-(e.double() * sp.double())).float()
    return g, beta


def recurrence(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, g: torch.Tensor, beta: torch.Tensor,
               init: torch.Tensor | None, dtype=torch.float64):
    """The gated delta rule, token by token (torch_recurrent_gated_delta_rule with the l2norm already applied).
    q, k (S, L, Hv, dk) bf16 (already repeated to the value heads), v (S, L, Hv, dv) bf16, g, beta (S, L, Hv) fp32,
    init (S, Hv, dk, dv) fp32 or None (zeros). Arithmetic in `dtype` (float64: the value the fp32 reference and a
    kernel approximate; float32: the reference's own). Returns (o (S, L, Hv, dv) bf16, final state (S, Hv, dk, dv)
    in dtype)."""
    S_, L, Hv, dk = q.shape
    dv = v.shape[-1]
    # query * (1 / sqrt(dk)) in fp32, as the reference scales the upcast query
    qd = (q.float() * torch.tensor(1.0 / dk ** 0.5, dtype=torch.float32)).to(dtype)
    kd, vd = k.to(dtype), v.to(dtype)
    gd, bd = g.to(dtype), beta.to(dtype)
    st = torch.zeros(S_, Hv, dk, dv, dtype=dtype) if init is None else init.to(dtype).clone()
    out = torch.zeros(S_, L, Hv, dv, dtype=dtype)
    for t in range(L):
        st = st * torch.exp(gd[:, t])[..., None, None]
        kv = (st * kd[:, t, :, :, None]).sum(-2)
        delta = (vd[:, t] - kv) * bd[:, t, :, None]
        st = st + kd[:, t, :, :, None] * delta[:, :, None, :]
        out[:, t] = (st * qd[:, t, :, :, None]).sum(-2)
    return out.float().to(torch.bfloat16), st


def chunked_recurrence(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, g: torch.Tensor, beta: torch.Tensor,
                       init: torch.Tensor | None, chunk: int = 32):
    """The same gated delta rule in the chunked (WY) form that transformers' torch_chunk_gated_delta_rule evaluates
    and od_gdn_recurrence_chunked implements, in float64: per chunk with gamma = cumsum(g) and S_0 the state at its
    start, A_ij = beta_i e^{gamma_i - gamma_j} k_i.k_j (j < i), T = (I + A)^{-1} diag(beta),
    delta = T V - T diag(e^gamma) K S_0, O = diag(e^gamma) Q~ S_0 + (Q~ K^T o D) delta (D_ij = e^{gamma_i - gamma_j},
    j <= i), S_C = e^{gamma_C} S_0 + K^T diag(e^{gamma_C - gamma}) delta. Arguments as recurrence; returns (o bf16,
    final state float64). Equal to the token-by-token recurrence up to float64 rounding (the algebra the kernel
    relies on)."""
    S_, L, Hv, dk = q.shape
    dv = v.shape[-1]
    qd = (q.float() * torch.tensor(1.0 / dk ** 0.5, dtype=torch.float32)).double()
    kd, vd, gd, bd = k.double(), v.double(), g.double(), beta.double()
    st = torch.zeros(S_, Hv, dk, dv, dtype=torch.float64) if init is None else init.double().clone()
    out = torch.zeros(S_, L, Hv, dv, dtype=torch.float64)
    for c0 in range(0, L, chunk):
        sl = slice(c0, min(L, c0 + chunk))
        K, Q, V = kd[:, sl].transpose(1, 2), qd[:, sl].transpose(1, 2), vd[:, sl].transpose(1, 2)  # (S, H, C, d)
        gam = torch.cumsum(gd[:, sl].transpose(1, 2), -1)                                          # (S, H, C)
        bb = bd[:, sl].transpose(1, 2)
        n = K.shape[2]
        D = torch.exp(gam[..., :, None] - gam[..., None, :])
        A = torch.tril(bb[..., :, None] * D * (K @ K.transpose(-1, -2)), -1)
        T = torch.linalg.solve_triangular(torch.eye(n, dtype=torch.float64) + A, torch.diag_embed(bb), upper=False,
                                          unitriangular=True)
        delta = T @ V - T @ (torch.exp(gam)[..., None] * (K @ st))
        P = torch.tril((Q @ K.transpose(-1, -2)) * D)
        out[:, sl] = (torch.exp(gam)[..., None] * (Q @ st) + P @ delta).transpose(1, 2)
        dec = torch.exp(gam[..., -1:] - gam)
        st = torch.exp(gam[..., -1])[..., None, None] * st + K.transpose(-1, -2) @ (dec[..., None] * delta)
    return out.float().to(torch.bfloat16), st


def silu_f32(z: torch.Tensor) -> torch.Tensor:
    """F.silu in fp32 on fp32 inputs, correctly rounded (float64, rounded once)."""
    zd = z.double()
    return (zd / (1.0 + torch.exp(-zd))).float()


def gated_norm(o: torch.Tensor, z: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """Qwen3_5RMSNormGated per value head: bf16(bf16(w * bf16(o * r)) * silu(z.float())), r = 1 / sqrt(mean(o^2) +
    eps) correctly rounded to fp32 (decoder.rms_factor). o, z (M, Hv, dv) bf16, w (dv,) bf16. Returns (M, Hv, dv)
    bf16."""
    from .decoder import rms_factor
    of = o.float()
    hn = (of * rms_factor(of, eps)).to(torch.bfloat16)
    hw = (w.float() * hn.float()).to(torch.bfloat16)
    return (hw.float() * silu_f32(z.float())).to(torch.bfloat16)


def gdn_mixer(x: torch.Tensor, lw: dict, qlin: dict, cfg: GDNConfig, S: int, L: int, conv_state=None,
              rec_state=None, seq_state=None, dtype=torch.float64, seq_len=None):
    """The GDN token mixer over S sequences of L tokens each (x (S L, hidden) bf16, the ln1-normed input):
    projection, conv + SiLU, l2norm, gates, recurrence, gated norm. conv_state (Ns, K-1, conv_dim) bf16 and
    rec_state (Ns, Hv, dk, dv) fp32 are the states the sequences continue (seq_state (S,): each sequence's state
    index; None: sequence i continues state i; conv_state / rec_state None: fresh sequences). seq_len (S,): real
    lengths of right-padded sequences, the reference's Backbone.padded_continuation (backbone.py:256-289): the
    in_proj outputs a and b are set to -inf at the pads (so g = -exp(A) softplus(-inf) = -0 and beta = sigmoid(-inf)
    = 0 and the recurrent state passes through), and the new conv state is re-gathered at each real end. Returns (the
    gated-norm output (S L, value_dim) bf16, new conv states (S, K-1, conv_dim), new recurrent states (S, Hv, dk,
    dv))."""
    M = S * L
    q8, sw, inv = qlin["win"]
    proj, _, _, _ = oq.w8a8_linear(x, q8, sw, inv_s=inv)
    qkv, z, b, a = split_proj(proj, cfg)
    if seq_len is not None:
        keep = (torch.arange(L)[None, :] < torch.as_tensor(seq_len).long()[:, None]).reshape(M, 1)
        ninf = torch.full((), -float("inf"), dtype=a.dtype)
        a, b = torch.where(keep, a, ninf), torch.where(keep, b, ninf)
    idx = torch.arange(S) if seq_state is None else torch.as_tensor(seq_state).long()
    cs = None if conv_state is None else conv_state[idx]
    y, new_conv = conv_silu(qkv.reshape(S, L, cfg.conv_dim), lw["conv_w"], cs, seq_len)
    y = y.reshape(M, cfg.conv_dim)
    kd = cfg.key_dim
    q = l2norm_bf16(y[:, :kd].reshape(M, cfg.n_k_heads, cfg.dk), cfg.eps)
    k = l2norm_bf16(y[:, kd:2 * kd].reshape(M, cfg.n_k_heads, cfg.dk), cfg.eps)
    v = y[:, 2 * kd:].reshape(M, cfg.n_v_heads, cfg.dv)
    rep = cfg.n_v_heads // cfg.n_k_heads
    q = q.repeat_interleave(rep, dim=1)
    k = k.repeat_interleave(rep, dim=1)
    g, beta = gates(a, b, lw["A_log"], lw["dt_bias"])
    init = None if rec_state is None else rec_state[idx]
    o, st = recurrence(q.reshape(S, L, cfg.n_v_heads, cfg.dk), k.reshape(S, L, cfg.n_v_heads, cfg.dk),
                       v.reshape(S, L, cfg.n_v_heads, cfg.dv), g.reshape(S, L, -1), beta.reshape(S, L, -1), init,
                       dtype)
    out = gated_norm(o.reshape(M, cfg.n_v_heads, cfg.dv), z.reshape(M, cfg.n_v_heads, cfg.dv), lw["gnorm"], cfg.eps)
    return out.reshape(M, cfg.value_dim), new_conv, st.float()


def quantize_gdn(lw: dict) -> dict:
    from .decoder import quantize_linear
    return {"win": quantize_linear(lw["win"], lw["s_in"]), "wout": quantize_linear(lw["wout"], lw["s_out"])}
