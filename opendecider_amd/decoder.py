"""Decision-forward harness on the MI355X: a dense 9B-class decoder whose linears are W8A8 (int8 MFMA), whose
option-row attention is the branched kernel over int8 state K/V, with the option readout on top.

This is the backbone stand-in that carries the path (the reference runs the same per-layer steps inside HF Qwen3.5
modules: the W8A8 linears in every nn.Linear slot, src/opendecider/prefix_attn.py:79-131 for the attention layer,
option logits + 'none' in src/opendecider/v3.py:639-643,701-709 and the softmax in src/opendecider/decider.py:255-257).
State prefill (prefill): the same layer with causal wide_attention over the new tokens' bf16 K/V (or, for a record
appended to a cached state, the branched kernel over the int8 cache + the record's own tokens), the new K/V quantized
into per-layer int8 caches by od_kv_quant_append. Scoring (score), per layer, for the M = rows x tokens option-row
tokens:
    od_rmsnorm_quant -> od_w8a8_gemm (QKV) -> od_qk_norm_rope -> od_branched_attn -> od_act_quant
    -> od_w8a8_gemm (O, + residual) -> od_rmsnorm_quant -> od_w8a8_gemm_swiglu (gate+up with SwiGLU in the
    epilogue; gate and up weight rows interleaved) -> od_act_quant -> od_w8a8_gemm (down, + residual)
All activations live in preallocated HBM buffers; nothing allocates or synchronizes inside a forward, so the whole
forward can be captured in one HIP graph.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch

from . import kernels
from .kv_cache import GDNState, HybridState, Int8KVCache, StateKV


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
    # The Qwen3.5 hybrid stack: with an interval n > 0, layer i is full attention when (i + 1) % n == 0 and a Gated
    # DeltaNet (linear-attention) layer otherwise (the backbone's layer_types, src/opendecider/backbone.py:75,270);
    # 0 keeps every layer full attention. The GDN dims are Qwen3.5's (16 key heads, 32 value heads, 128 / 128).
    full_attention_interval: int = 0
    lin_k_heads: int = 16
    lin_v_heads: int = 32
    lin_k_dim: int = 128
    lin_v_dim: int = 128
    conv_kernel: int = 4
    # Qwen3.5's attention geometry (transformers' Qwen3_5TextConfig / Qwen3_5Attention): rotary embedding on the first
    # rot_dim dims of each head (partial_rotary_factor 0.25 of head_dim 256; 0 = the whole head), and every RMSNorm of
    # the decoder (input / post-attention / q / k / final) zero-centred: Qwen3_5RMSNorm's (x * r) * (1 + w).
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
    def lin_key(self) -> int:
        return self.lin_k_heads * self.lin_k_dim

    @property
    def lin_value(self) -> int:
        return self.lin_v_heads * self.lin_v_dim

    @property
    def lin_conv(self) -> int:
        return 2 * self.lin_key + self.lin_value

    @property
    def lin_proj(self) -> int:
        """The GDN input projection's rows: [qkv (lin_conv) | z (lin_value) | b (n_v) | a (n_v)]."""
        return self.lin_conv + self.lin_value + 2 * self.lin_v_heads


def rope_tables(cfg: DecoderConfig, n_pos: int):
    """cos/sin bf16 tables [n_pos, R/2] over the R = cfg.rotary_dims rotated dims: inv_freq = 1 / theta^(2i/R),
    angle = pos * inv_freq in fp32 (computed on the host, as the rotary-embedding module of the backbone does)."""
    D = cfg.rotary_dims
    inv_freq = 1.0 / (cfg.theta ** (torch.arange(0, D, 2, dtype=torch.int64).float() / D))
    ang = torch.arange(n_pos, dtype=torch.float32)[:, None] * inv_freq[None, :]
    return ang.cos().to(torch.bfloat16), ang.sin().to(torch.bfloat16)


class QLinear:
    """One W8A8 linear's device tensors: int8 weight (out, in), fp32 per-output-channel scale, bf16 1/s."""

    def __init__(self, w: torch.Tensor, s: torch.Tensor | None, device):
        w = w.to(device)
        inv = None
        if s is not None:
            # fold W * s per input channel in fp32, round to bf16 (quant.py:343-344); bf16(1/s) (quant.py:325)
            w = (w.float() * s.to(device, torch.float32)[None, :]).to(torch.bfloat16)
            inv = (1.0 / s.float().cpu()).to(torch.bfloat16).to(device)
        q, sc = kernels.act_quant(w.to(torch.bfloat16))
        self.q, self.scale, self.inv_s = q, sc, inv
        self.out_features, self.in_features = q.shape


def random_layer_weights(cfg: DecoderConfig, g: torch.Generator, device, smooth: bool = True) -> dict:
    """One layer of random-init bf16 weights (linears N(0, 0.02), norms near 1) and SmoothQuant factors
    s ~ U(0.5, 2) per linear input, generated on `device`."""
    bf = torch.bfloat16
    H, F, D = cfg.hidden, cfg.ffn, cfg.head_dim

    def lin(n, k):
        return (torch.randn(n, k, generator=g, device=device) * 0.02).to(bf)

    def norm(n):  # near 1 as applied: 1 + w with the zero-centred weights
        return ((0.0 if cfg.norm_offset else 1.0) + 0.1 * torch.randn(n, generator=g, device=device)).to(bf)

    def sm(n):
        return (torch.rand(n, generator=g, device=device) * 1.5 + 0.5) if smooth else None

    return {"ln1": norm(H), "ln2": norm(H), "q_norm": norm(D), "k_norm": norm(D),
            "wqkv": lin(cfg.qkv_out, H), "wo": lin(H, cfg.n_heads * D), "wgu": lin(2 * F, H), "wdown": lin(H, F),
            "s_qkv": sm(H), "s_o": sm(cfg.n_heads * D), "s_gu": sm(H), "s_down": sm(F)}


def random_gdn_layer_weights(cfg: DecoderConfig, g: torch.Generator, device, smooth: bool = True) -> dict:
    """One Gated DeltaNet layer of random-init weights: the fused input projection [qkv | z | b | a] and out_proj
    N(0, 0.02), conv N(0, 0.3), A = U(0.5, 16) (A_log = log A) and dt_bias ~ 1 + 0.1 N(0, 1) in bf16, the gated
    norm's weight near 1, the MLP as in an attention layer, SmoothQuant factors U(0.5, 2) per linear input."""
    bf = torch.bfloat16
    H, F = cfg.hidden, cfg.ffn

    def lin(n, k):
        return (torch.randn(n, k, generator=g, device=device) * 0.02).to(bf)

    def norm(n):  # near 1 as applied: 1 + w with the zero-centred weights
        return ((0.0 if cfg.norm_offset else 1.0) + 0.1 * torch.randn(n, generator=g, device=device)).to(bf)

    def sm(n):
        return (torch.rand(n, generator=g, device=device) * 1.5 + 0.5) if smooth else None

    A = torch.rand(cfg.lin_v_heads, generator=g, device=device) * 15.5 + 0.5
    return {"ln1": norm(H), "ln2": norm(H), "win": lin(cfg.lin_proj, H),
            "conv_w": (torch.randn(cfg.lin_conv, cfg.conv_kernel, generator=g, device=device) * 0.3).to(bf),
            "A_log": torch.log(A).to(bf), "dt_bias": (1.0 + 0.1 * torch.randn(cfg.lin_v_heads, generator=g,
                                                                            device=device)).to(bf),
            "gnorm": norm(cfg.lin_v_dim), "wout": lin(H, cfg.lin_value), "wgu": lin(2 * F, H), "wdown": lin(H, F),
            "s_in": sm(H), "s_out": sm(cfg.lin_value), "s_gu": sm(H), "s_down": sm(F)}


def random_decoder(cfg: DecoderConfig, seed: int = 0, device="cuda", max_pos: int = 65536) -> "DenseDecoder":
    """A random-init decoder of `cfg` built layer by layer on the GPU (bf16 weights are quantized and dropped one
    layer at a time). The embedding is random bf16 (vocab x hidden)."""
    g = torch.Generator(device=device).manual_seed(seed)
    H = cfg.hidden
    head = {"final_norm": ((0.0 if cfg.norm_offset else 1.0) + 0.1 * torch.randn(H, generator=g, device=device)
                           ).to(torch.bfloat16),
            "head": torch.randn(H, generator=g, device=device) / H ** 0.5,
            "none_logit": torch.zeros((), device=device), "layers": []}
    dec = DenseDecoder(cfg, head, None, device, max_pos)
    for li in range(cfg.n_layers):
        dec.add_layer((random_gdn_layer_weights if cfg.is_gdn(li) else random_layer_weights)(cfg, g, device))
    dec.embed = torch.randn(cfg.vocab, H, generator=g, device=device).to(torch.bfloat16)
    return dec


class DenseDecoder:
    """Weights from a dict (oracle.decoder.make_weights layout) on any device; quantized on the GPU."""

    def __init__(self, cfg: DecoderConfig, weights: dict, embed: torch.Tensor | None, device="cuda",
                 max_pos: int = 65536):
        self.cfg, self.dev = cfg, torch.device(device)
        self.layers = []
        for lw in weights["layers"]:
            self.add_layer(lw)
        self.final_norm = weights["final_norm"].to(self.dev)
        self.head = weights["head"].to(self.dev).float()
        self.none_logit = weights["none_logit"].to(self.dev).float()
        self.embed = None if embed is None else embed.to(self.dev)
        cos, sin = rope_tables(cfg, max_pos)
        self.cos, self.sin = cos.to(self.dev), sin.to(self.dev)
        self.temperature = float(weights.get("temperature", 1.0))
        self._eps32 = float(torch.tensor(cfg.eps, dtype=torch.float32))
        self._ws = {}
        self._rows = {}
        self._images = {}  # layer -> (key, block images of that layer's state K/V)

    def qkv_rows(self) -> torch.Tensor | None:
        """Gated: the row order that takes the fused projection from the reference's layout (q_proj's per-head
        [q_h; gate_h], then k_proj, v_proj) to [q (Hq D); k; v; gate (Hq D)], so that q and k keep their places for
        the q/k norm + RoPE kernels and the gate is one contiguous block (a row permutation: per-row quantization
        is unchanged). None when not gated."""
        cfg = self.cfg
        if not cfg.gated:
            return None
        D, Hq, Hk = cfg.head_dim, cfg.n_heads, cfg.n_kv_heads
        heads = torch.arange(Hq)[:, None] * 2 * D
        q_rows = (heads + torch.arange(D)[None, :]).reshape(-1)
        g_rows = (heads + D + torch.arange(D)[None, :]).reshape(-1)
        kv_rows = 2 * Hq * D + torch.arange(2 * Hk * D)
        return torch.cat([q_rows, kv_rows, g_rows])

    def add_layer(self, lw: dict) -> None:
        if self.cfg.is_gdn(len(self.layers)):
            self._add_gdn_layer(lw)
            return
        L = {k: lw[k].to(self.dev) for k in ("ln1", "ln2", "q_norm", "k_norm")}
        L["gdn"] = False
        rows = self.qkv_rows()
        wqkv = lw["wqkv"] if rows is None else lw["wqkv"][rows.to(lw["wqkv"].device)]
        L["qkv"] = QLinear(wqkv, lw.get("s_qkv"), self.dev)
        for name in ("o", "down"):
            L[name] = QLinear(lw["w" + name], lw.get("s_" + name), self.dev)
        # gate and up rows interleaved for the SwiGLU GEMM (a row permutation: per-row quantization is unchanged)
        L["gu"] = QLinear(kernels.interleave_gate_up(lw["wgu"]), lw.get("s_gu"), self.dev)
        self.layers.append(L)

    def _add_gdn_layer(self, lw: dict) -> None:
        """A Gated DeltaNet layer: the fused input projection padded with zero rows to a multiple of 8 outputs (16-byte
        rows for od_gdn_prep; a zero row quantizes to q = 0 and outputs 0), out_proj, the MLP."""
        cfg = self.cfg
        if cfg.conv_kernel != 4:
            raise ValueError("GDN layers: the conv kernel must be 4 (Qwen3.5's)")
        L = {k: lw[k].to(self.dev).contiguous() for k in ("ln1", "ln2", "conv_w", "A_log", "dt_bias", "gnorm")}
        L["gdn"] = True
        win = lw["win"]
        pad = -win.shape[0] % 8
        if pad:
            win = torch.cat([win, torch.zeros(pad, win.shape[1], dtype=win.dtype, device=win.device)])
        L["win"] = QLinear(win, lw.get("s_in"), self.dev)
        L["wout"] = QLinear(lw["wout"], lw.get("s_out"), self.dev)
        L["down"] = QLinear(lw["wdown"], lw.get("s_down"), self.dev)
        L["gu"] = QLinear(kernels.interleave_gate_up(lw["wgu"]), lw.get("s_gu"), self.dev)
        self.layers.append(L)

    @property
    def hybrid(self) -> bool:
        return any(L["gdn"] for L in self.layers)

    # ---------------------------------------------------------------- buffers
    def workspace(self, M: int):
        """Activation buffers for M tokens (kept per M: a decision runs a state prefill and the option rows)."""
        if M in self._ws:
            return self._ws[M]
        cfg, d = self.cfg, self.dev
        bf = torch.bfloat16
        kmax = max(cfg.hidden, cfg.ffn, cfg.n_heads * cfg.head_dim, cfg.lin_value if self.hybrid else 0)
        self._ws[M] = {
            "M": M,
            "h": [torch.empty(M, cfg.hidden, dtype=bf, device=d) for _ in range(2)],
            "xq": torch.empty(M, (kmax + 15) // 16 * 16, dtype=torch.int8, device=d),
            "sx": torch.empty(M, dtype=torch.float32, device=d),
            "qkv": torch.empty(M, cfg.qkv_out, dtype=bf, device=d),
            "attn": torch.empty(M, cfg.n_heads * cfg.head_dim, dtype=bf, device=d),
            "hmlp": torch.empty(M, cfg.ffn, dtype=bf, device=d),
        }
        if self.hybrid:  # the GDN layers' buffers: projection, conv outputs, gates, recurrence output
            nv = cfg.lin_v_heads
            self._ws[M].update({
                "proj": torch.empty(M, self.layers[self._first_gdn()]["win"].out_features, dtype=bf, device=d),
                "gqk": torch.empty(M, 2 * cfg.lin_key, dtype=bf, device=d),
                "gv": torch.empty(M, cfg.lin_value, dtype=bf, device=d),
                "gg": torch.empty(M, nv, dtype=torch.float32, device=d),
                "gbeta": torch.empty(M, nv, dtype=torch.float32, device=d),
                "go": torch.empty(M, cfg.lin_value, dtype=bf, device=d),
            })
        return self._ws[M]

    def _first_gdn(self) -> int:
        return next(i for i, L in enumerate(self.layers) if L["gdn"])

    def new_state_caches(self, batch: int, capacity: int):
        """Empty per-layer states for `batch` states of up to `capacity` tokens: the (K, V) int8 caches in one
        allocation (StateKV), or for a hybrid stack a HybridState (K/V caches of the attention layers, conv and
        recurrent states of the GDN layers)."""
        cfg = self.cfg
        if not self.hybrid:
            return StateKV(len(self.layers), batch, cfg.n_kv_heads, cfg.head_dim, capacity, self.dev)
        return HybridState([L["gdn"] for L in self.layers], batch, cfg.n_kv_heads, cfg.head_dim, capacity,
                           cfg.lin_conv, cfg.lin_v_heads, cfg.lin_k_dim, cfg.lin_v_dim, self.dev)

    @staticmethod
    def state_length(states) -> int:
        """Tokens held by the states (every layer holds the same number)."""
        s0 = states[0]
        return s0.length if isinstance(s0, GDNState) else s0[0].length

    @staticmethod
    def state_count(states) -> int:
        """States held per layer."""
        s0 = states[0]
        return s0.batch if isinstance(s0, GDNState) else s0[0].q.shape[0]

    # ---------------------------------------------------------------- forward
    def _attn_in(self, li: int, h: torch.Tensor, ws: dict, pos: torch.Tensor, append=None) -> torch.Tensor:
        """RMSNorm + quantize, W8A8 QKV GEMM, q/k norm + RoPE (in place): the layer's qkv (M, qkv_out) bf16.
        append = (B, S, K cache, V cache): the same pass also appends the tokens' int8 K/V to the caches."""
        cfg, L = self.cfg, self.layers[li]
        kernels.rmsnorm_quant(h, L["ln1"], cfg.eps, L["qkv"].inv_s, ws["xq"][:, :cfg.hidden], ws["sx"],
                              offset=cfg.norm_offset)
        qkv = kernels.w8a8_gemm(ws["xq"][:, :cfg.hidden], ws["sx"], L["qkv"].q, L["qkv"].scale, out=ws["qkv"])
        if append is None:
            kernels.qk_norm_rope(qkv, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, L["q_norm"], L["k_norm"], self.cos,
                                 self.sin, pos, cfg.eps, cfg.rotary_dims, cfg.norm_offset)
        else:
            B, S, cache_k, cache_v = append
            kernels.qk_norm_rope_kv_append(qkv, B, S, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, L["q_norm"],
                                           L["k_norm"], self.cos, self.sin, pos, cfg.eps, cache_k, cache_v,
                                           cfg.rotary_dims, cfg.norm_offset)
        return qkv

    def _heads(self, qkv: torch.Tensor, ws: dict, R: int, t: int):
        """(R, heads, t, D) views of q, k, v in the qkv buffer and of the attention output buffer."""
        cfg = self.cfg
        D, Hq, Hk = cfg.head_dim, cfg.n_heads, cfg.n_kv_heads
        q = qkv[:, :Hq * D].view(R, t, Hq, D).transpose(1, 2)
        k = qkv[:, Hq * D:(Hq + Hk) * D].view(R, t, Hk, D).transpose(1, 2)
        v = qkv[:, (Hq + Hk) * D:(Hq + 2 * Hk) * D].view(R, t, Hk, D).transpose(1, 2)
        attn = ws["attn"].view(R, t, Hq, D).transpose(1, 2)
        return q, k, v, attn

    def _attn_out_mlp(self, li: int, h: torch.Tensor, h_out: torch.Tensor, ws: dict) -> torch.Tensor:
        """Quantize the attention output, W8A8 O GEMM + residual (into h_out), RMSNorm + quantize, gate+up GEMM with
        SwiGLU in its epilogue, quantize, down GEMM + residual (back into h)."""
        cfg, L = self.cfg, self.layers[li]
        xq, sx = ws["xq"], ws["sx"]
        hd = cfg.n_heads * cfg.head_dim
        if cfg.gated:  # o * sigmoid(gate) fused into o_proj's input quantizer (prefix_attn.py:130)
            gate = ws["qkv"][:, (cfg.n_heads + 2 * cfg.n_kv_heads) * cfg.head_dim:]
            kernels.gate_act_quant(ws["attn"], gate, L["o"].inv_s, xq=xq[:, :hd], sx=sx)
        else:
            kernels.act_quant(ws["attn"], L["o"].inv_s, xq=xq[:, :hd], sx=sx)
        kernels.w8a8_gemm(xq[:, :hd], sx, L["o"].q, L["o"].scale, residual=h, out=h_out)
        return self._mlp(li, h, h_out, ws)

    def _mlp(self, li: int, h: torch.Tensor, h_out: torch.Tensor, ws: dict) -> torch.Tensor:
        """The MLP half of a layer on the mid residual h_out: RMSNorm + quantize, gate+up GEMM with SwiGLU in its
        epilogue, quantize, down GEMM + residual (into h)."""
        cfg, L = self.cfg, self.layers[li]
        xq, sx = ws["xq"], ws["sx"]
        kernels.rmsnorm_quant(h_out, L["ln2"], cfg.eps, L["gu"].inv_s, xq[:, :cfg.hidden], sx, offset=cfg.norm_offset)
        hm = kernels.w8a8_gemm_swiglu(xq[:, :cfg.hidden], sx, L["gu"].q, L["gu"].scale, out=ws["hmlp"])
        kernels.act_quant(hm, L["down"].inv_s, xq=xq[:, :cfg.ffn], sx=sx)
        kernels.w8a8_gemm(xq[:, :cfg.ffn], sx, L["down"].q, L["down"].scale, residual=h_out, out=h)
        return h

    def gdn_layer(self, li: int, h: torch.Tensor, h_out: torch.Tensor, ws: dict, st: GDNState, S: int, L: int,
                  seq_state=None, prefill: bool = False, conv_tmp=None, continue_into=None) -> torch.Tensor:
        """One Gated DeltaNet layer over S sequences of L tokens (Qwen3_5GatedDeltaNet.forward's steps, the token
        mixer of src/opendecider/backbone.py's linear_attention layers):
            od_rmsnorm_quant -> od_w8a8_gemm (in_proj: [qkv | z | b | a]) -> od_gdn_prep (conv + SiLU, l2norm,
            gates) -> od_gdn_recurrence -> od_gdn_norm_quant (gated RMSNorm + out_proj's quantizer)
            -> od_w8a8_gemm (out_proj, + residual) -> the MLP.
        Scoring (prefill False): sequence i is option row i and continues state seq_state[i] (int32 (S,) on the
        GPU): its conv window starts from that state's last 3 inputs and its recurrence from that state's fp32 S0,
        both read in place (no per-row copy of the state, docs/branched_shared_prefix_math.md:16-37); the rows are
        terminal, nothing is written back. Prefill (prefill True, S = the states' batch): sequence i continues state
        i (or starts from zeros when st.length is 0) and its new conv window and final recurrent state are written
        back (the conv window through conv_tmp (S, 3, C) when continuing, since other tokens still read the old
        one). continue_into = (GDNState of S sequences, seq_len int32 (S,)): the question pass; sequence i continues
        state seq_state[i] over its seq_len[i] real tokens (right pads leave the state unchanged, the reference's
        padded continuation, backbone.py:256-289) and its conv window and final state go to that GDNState."""
        cfg, Ly = self.cfg, self.layers[li]
        H, nk, nv, dk, dv = cfg.hidden, cfg.lin_k_heads, cfg.lin_v_heads, cfg.lin_k_dim, cfg.lin_v_dim
        M = S * L
        xq, sx = ws["xq"], ws["sx"]
        kernels.rmsnorm_quant(h, Ly["ln1"], cfg.eps, Ly["win"].inv_s, xq[:, :H], sx, offset=cfg.norm_offset)
        proj = kernels.w8a8_gemm(xq[:, :H], sx, Ly["win"].q, Ly["win"].scale, out=ws["proj"])
        bufs = (ws["gqk"], ws["gv"], ws["gg"], ws["gbeta"])
        if continue_into is not None:
            qst, seq_len = continue_into
            kernels.gdn_prep(proj, Ly["conv_w"], Ly["A_log"], Ly["dt_bias"], S, L, nk, nv, dk, dv, conv_in=st.conv,
                             seq_state=seq_state, conv_out=qst.conv, out=bufs, seq_len=seq_len)
            kernels.gdn_recurrence(*bufs, S, L, nk, nv, dk, dv, init=st.rec, seq_state=seq_state, final=qst.rec,
                                   out=ws["go"])
        elif prefill:
            fresh = st.length == 0
            conv_out = st.conv[:S] if fresh else conv_tmp
            kernels.gdn_prep(proj, Ly["conv_w"], Ly["A_log"], Ly["dt_bias"], S, L, nk, nv, dk, dv,
                             conv_in=None if fresh else st.conv, conv_out=conv_out, out=bufs)
            kernels.gdn_recurrence(*bufs, S, L, nk, nv, dk, dv, init=None if fresh else st.rec[:S],
                                   final=st.rec[:S], out=ws["go"])
            if not fresh:
                st.conv[:S].copy_(conv_tmp)
        else:
            kernels.gdn_prep(proj, Ly["conv_w"], Ly["A_log"], Ly["dt_bias"], S, L, nk, nv, dk, dv, conv_in=st.conv,
                             seq_state=seq_state, out=bufs)
            kernels.gdn_recurrence(*bufs, S, L, nk, nv, dk, dv, init=st.rec, seq_state=seq_state, out=ws["go"])
        C, V = cfg.lin_conv, cfg.lin_value
        kernels.gdn_norm_quant(ws["go"], proj[:, C:C + V], Ly["gnorm"], cfg.eps, nv, dv, Ly["wout"].inv_s,
                               xq=xq[:, :V], sx=sx)
        kernels.w8a8_gemm(xq[:, :V], sx, Ly["wout"].q, Ly["wout"].scale, residual=h, out=h_out)
        return self._mlp(li, h, h_out, ws)

    def state_images(self, li: int, state_k: Int8KVCache, state_v: Int8KVCache):
        """Layer li's block images of the cached states (od_attn_stage), built once and reused by every scoring pass
        until the caches change (their generations or length move; generations are unique across caches, so a new
        state never hits the images of a freed one). Only for an unmasked state."""
        cfg = self.cfg
        key = (id(state_k), id(state_v), state_k.generation, state_v.generation, state_k.length)
        hit = self._images.get(li)
        if hit is not None and hit[0] == key:
            return hit[1]
        img = kernels.stage_state(state_k.q, state_k.scale, state_v.q, state_v.scale, state_k.length,
                                  cfg.head_dim ** -0.5, out=None if hit is None else hit[1])
        self._images[li] = (key, img)
        return img

    def layer(self, li: int, h: torch.Tensor, h_out: torch.Tensor, ws: dict, state_k: Int8KVCache,
              state_v: Int8KVCache, R: int, t: int, pos: torch.Tensor, row_start, max_rows: int, kvalid=None):
        """One layer over R option rows of t tokens that attend their state's int8 K/V and themselves. When the
        staged path applies (enough slot tiles per (state, head)) and the state is unmasked, the state's block images
        come from state_images (built once per state version, not per pass)."""
        cfg = self.cfg
        D = cfg.head_dim
        qkv = self._attn_in(li, h, ws, pos)
        q, k, v, attn = self._heads(qkv, ws, R, t)
        img = None
        if kvalid is None and state_k.length > 0 and kernels.uses_staging(max_rows, t, cfg.n_heads, cfg.n_kv_heads):
            img = self.state_images(li, state_k, state_v)
        kernels.branched_attn(q, k, v, state_k.q, state_k.scale, state_v.q, state_v.scale, D ** -0.5, kvalid=kvalid,
                              length=state_k.length, out=attn, row_start=row_start, max_rows=max_rows, images=img)
        return self._attn_out_mlp(li, h, h_out, ws)  # the output goes back into h (h_out held the mid residual)

    def prefill_layer(self, li: int, h: torch.Tensor, h_out: torch.Tensor, ws: dict, cache_k: Int8KVCache,
                      cache_v: Int8KVCache, B: int, S: int, pos: torch.Tensor, kvalid=None, row_start=None):
        """One layer over S new state tokens of each of B states, appended after the cache's current n0 tokens.
        n0 = 0: causal attention among the new tokens on bf16 K/V (wide_attention), as the backbone's state pass.
        n0 > 0 (an appended record, S <= 256): the new tokens attend the cached int8 state and themselves causally
        (the branched kernel with one row per state). Only the new tokens' K/V are quantized and appended
        (state_cache.py:79), in the same pass as the q/k norm + RoPE; the attention reads the cache's first n0 tokens
        only."""
        D = self.cfg.head_dim
        n0 = cache_k.length
        if S > 256 and n0 > 0:
            raise ValueError(f"prefill: an appended record of {S} tokens exceeds 256 (append it in pieces)")
        qkv = self._attn_in(li, h, ws, pos, append=(B, S, cache_k, cache_v))
        q, k, v, attn = self._heads(qkv, ws, B, S)
        if n0 == 0:
            kernels.wide_attn(q, k, v, D ** -0.5, kvalid=kvalid, causal=True, out=attn)
        else:
            rs, mr = (None, 1) if B == 1 else (row_start, 1)  # one row (the record) per state
            kernels.branched_attn(q, k, v, cache_k.q, cache_k.scale, cache_v.q, cache_v.scale, D ** -0.5,
                                  kvalid=kvalid, length=n0, out=attn, row_start=rs, max_rows=mr)
        return self._attn_out_mlp(li, h, h_out, ws)

    def prefill(self, ids: torch.Tensor, caches: list, kvalid=None) -> torch.Tensor:
        """ids (B, S) state token ids on the GPU, appended to the B states held in caches[l] = (K, V) (all layers at
        the same length n0). kvalid: (B, S) key mask of the new tokens (first prefill) or (B, n0) of the cached
        ones (an appended record). Returns the new tokens' final hidden states (B S, hidden)."""
        B, S = ids.shape
        n0 = self.state_length(caches)
        if n0 + S > self.cos.shape[0]:
            raise ValueError(f"positions up to {n0 + S} exceed the rotary tables ({self.cos.shape[0]})")
        conv_tmp = None
        if self.hybrid:
            if kvalid is not None:
                raise ValueError("prefill: key masks are not supported with GDN layers (every token enters the "
                                 "recurrent state)")
            if self.state_count(caches) != B:
                raise ValueError(f"prefill: {B} sequences for {self.state_count(caches)} states")
            if n0 > 0:
                conv_tmp = self._conv_tmp(B)
        ws = self.workspace(B * S)
        h, mid = ws["h"]
        h.copy_(self.embed.index_select(0, ids.reshape(-1)))
        pos, row_start = self.prefill_layout(n0, B, S)
        for li in range(len(self.layers)):
            if self.layers[li]["gdn"]:
                self.gdn_layer(li, h, mid, ws, caches[li], B, S, prefill=True, conv_tmp=conv_tmp)
            else:
                self.prefill_layer(li, h, mid, ws, caches[li][0], caches[li][1], B, S, pos, kvalid, row_start)
        for st in caches:
            if isinstance(st, GDNState):
                st.length = n0 + S
        return h

    def _conv_tmp(self, B: int) -> torch.Tensor:
        key = ("conv_tmp", B)
        if key not in self._rows:
            self._rows[key] = torch.empty(B, 3, self.cfg.lin_conv, dtype=torch.bfloat16, device=self.dev)
        return self._rows[key]

    def row_states(self, B: int, n_opt: int) -> torch.Tensor | None:
        """Each option row's state index (int32 on the GPU, built once per shape) for the GDN layers; None for a
        stack without them."""
        if not self.hybrid:
            return None
        key = ("row_state", B, n_opt)
        if key not in self._rows:
            self._rows[key] = torch.arange(B, dtype=torch.int32).repeat_interleave(n_opt).to(self.dev)
        return self._rows[key]

    def rows_forward(self, h0: torch.Tensor, states: list, R: int, t: int, pos: torch.Tensor, row_start, max_rows,
                     kvalid=None, row_state=None) -> torch.Tensor:
        """Option-row tokens h0 (M = R t, hidden) bf16 through every layer; states[l] = (K cache, V cache), or a
        GDNState for a GDN layer (row_state: each row's state index, int32 (R,) on the GPU)."""
        if self.hybrid and (row_state is None or kvalid is not None):
            raise ValueError("rows_forward: GDN layers need row_state and take no key mask")
        ws = self.workspace(h0.shape[0])
        h, mid = ws["h"]
        h.copy_(h0)
        for li in range(len(self.layers)):
            if self.layers[li]["gdn"]:
                self.gdn_layer(li, h, mid, ws, states[li], R, t, row_state)
            else:
                self.layer(li, h, mid, ws, states[li][0], states[li][1], R, t, pos, row_start, max_rows, kvalid)
        return h

    def question_pass(self, ids_q: torch.Tensor, qlen, states, group_state) -> "QuestionCache":
        """The question pass of the question cache (v3.py:446-534): question g's tokens (ids_q (G, Lq) on the GPU,
        right-padded; qlen its real lengths) at positions T .. T + Lq - 1 after its state group_state[g] attend that
        state's int8 K/V and themselves causally through every layer (the branched kernel, one row per question), and
        each layer's question K/V (bf16, after q/k norm + RoPE; prefix_attn.py:92-93's capture) are written straight
        into block images (od_attn_stage_bf16, keys past qlen[g] masked): the second prefix level the option rows
        read. Questions must be grouped by state (group_state non-decreasing). On a hybrid stack each Gated DeltaNet
        layer continues question g's state over its qlen[g] real tokens as the reference's batched question pass does
        (Backbone.padded_continuation, v3.py:494-497: pads leave the recurrent state unchanged, the conv window ends
        at the last real token) into a per-question state that the option rows then continue."""
        cfg = self.cfg
        G, Lq = ids_q.shape
        gs = [int(s) for s in group_state]
        qlen = [int(n) for n in qlen]
        if len(gs) != G or len(qlen) != G or any(b < a for a, b in zip(gs, gs[1:])):
            raise ValueError("question_pass: one state per question, questions grouped by state")
        if any(not 1 <= n <= Lq for n in qlen) or Lq > 256:
            raise ValueError("question_pass: 1 <= qlen <= Lq <= 256")
        T = self.state_length(states)
        Ns = self.state_count(states)
        if T + Lq > self.cos.shape[0]:
            raise ValueError(f"question_pass: positions up to {T + Lq} exceed the rotary tables ({self.cos.shape[0]})")
        if min(gs) < 0 or max(gs) >= Ns:
            raise ValueError(f"question_pass: group_state outside [0, {Ns})")
        ws = self.workspace(G * Lq)
        h, mid = ws["h"]
        h.copy_(self.embed.index_select(0, ids_q.reshape(-1)))
        pos = (T + torch.arange(Lq, dtype=torch.int32)).repeat(G).to(self.dev)
        row_start, max_rows = kernels.row_start_of([gs.count(s) for s in range(Ns)], self.dev)
        qmask = (torch.arange(Lq)[None, :] < torch.tensor(qlen)[:, None]).to(torch.uint8).to(self.dev)
        D = cfg.head_dim
        images, gdn = [], {}
        gs_dev = torch.tensor(gs, dtype=torch.int32).to(self.dev)
        qlen_dev = torch.tensor(qlen, dtype=torch.int32).to(self.dev)
        for li in range(len(self.layers)):
            if self.layers[li]["gdn"]:
                src = states[li]
                qst = GDNState(torch.empty(G, *src.conv.shape[1:], dtype=src.conv.dtype, device=self.dev),
                               torch.empty(G, *src.rec.shape[1:], dtype=src.rec.dtype, device=self.dev))
                qst.length = T + Lq
                self.gdn_layer(li, h, mid, ws, src, G, Lq, seq_state=gs_dev, continue_into=(qst, qlen_dev))
                images.append(None)
                gdn[li] = qst
                continue
            state_k, state_v = states[li]
            qkv = self._attn_in(li, h, ws, pos)
            q, k, v, attn = self._heads(qkv, ws, G, Lq)
            img = None
            if state_k.length > 0 and kernels.uses_staging(max_rows, Lq, cfg.n_heads, cfg.n_kv_heads):
                img = self.state_images(li, state_k, state_v)
            kernels.branched_attn(q, k, v, state_k.q, state_k.scale, state_v.q, state_v.scale, D ** -0.5,
                                  length=state_k.length, out=attn, row_start=row_start, max_rows=max_rows,
                                  images=img)
            images.append(kernels.stage_state_bf16(k, v, Lq, D ** -0.5, qmask))
            self._attn_out_mlp(li, h, mid, ws)
        return QuestionCache(images, Lq, qlen, gs, gs_dev, T, gdn)

    def score_qcache(self, ids_o: torch.Tensor, qc: "QuestionCache", states) -> torch.Tensor:
        """Option rows over the question cache: ids_o (G, n_opt, t) on the GPU; the rows of question g start right
        after its last real token (position T + qlen[g], v3.py:520) and attend [state group_state[g] ; question g's
        K/V] and their own tokens (od_branched_attn_staged2); in a Gated DeltaNet layer they continue their
        question's state from the question pass, read in place. Returns (G, n_opt + 1) log-probabilities."""
        cfg = self.cfg
        G, n_opt, t = ids_o.shape
        if G != len(qc.qlen):
            raise ValueError("score_qcache: one group of option rows per question")
        T = self.state_length(states)
        if T != qc.T:
            raise ValueError("score_qcache: the states changed since the question pass")
        R = G * n_opt
        if T + max(qc.qlen) + t > self.cos.shape[0]:
            raise ValueError(f"score_qcache: positions up to {T + max(qc.qlen) + t} exceed the rotary tables")
        key = ("qcache", T, tuple(qc.qlen), n_opt, t)
        if key not in self._rows:
            pos = torch.cat([T + n + torch.arange(t, dtype=torch.int32) for n in qc.qlen for _ in range(n_opt)])
            row_q = torch.arange(G, dtype=torch.int32).repeat_interleave(n_opt)
            self._rows[key] = (pos.to(self.dev), *kernels.row_start_of([n_opt] * G, self.dev), row_q.to(self.dev))
        pos, row_start, max_rows, row_q = self._rows[key]
        ws = self.workspace(R * t)
        h, mid = ws["h"]
        h.copy_(self.embed.index_select(0, ids_o.reshape(-1)))
        Ns = self.state_count(states)
        D = cfg.head_dim
        for li in range(len(self.layers)):
            if self.layers[li]["gdn"]:  # row r continues question r // n_opt's state
                self.gdn_layer(li, h, mid, ws, qc.gdn[li], R, t, seq_state=row_q)
                continue
            state_k, state_v = states[li]
            qkv = self._attn_in(li, h, ws, pos)
            q, k, v, attn = self._heads(qkv, ws, R, t)
            img = self.state_images(li, state_k, state_v) if T > 0 else None
            kernels.branched_attn_two_level(q, k, v, img, Ns, T, qc.images[li], qc.Lq, D ** -0.5,
                                            group_state=qc.group_state, row_start=row_start, max_rows=max_rows,
                                            out=attn)
            self._attn_out_mlp(li, h, mid, ws)
        return self.readout(h, G, n_opt, t)

    def readout(self, h: torch.Tensor, B: int, n_opt: int, t: int, pool_last: int | None = None) -> torch.Tensor:
        """Mean-pool each option row's final-normed hidden states (the last pool_last tokens of each row when
        given: the option's own tokens of a row that carries its question too), one logit per row, the 'none' logit
        appended,
        divided by the decision temperature (softmax(logits / T), decider.py:255-257), log-softmax per request:
        (B, n_opt + 1) fp32. The RMSNorm factor is the correctly rounded one (a float64 mean of squares, as
        od_rmsnorm_quant computes it); with cfg.norm_offset the zero-centred norm bf16((h * r) * (1 + w))."""
        hf = h.float()
        hd = hf.double()
        r = (1.0 / torch.sqrt((hd * hd).sum(-1, keepdim=True) / hd.shape[-1] + self._eps32)).float()
        if self.cfg.norm_offset:
            hn = ((hf * r) * (1.0 + self.final_norm.float())).to(torch.bfloat16).float()
        else:
            hn = (self.final_norm * (hf * r).to(torch.bfloat16)).float()
        hn = hn.view(B, n_opt, t, -1)
        pooled = (hn if pool_last is None else hn[:, :, t - pool_last:]).mean(2)
        logits = torch.cat([pooled @ self.head, self.none_logit.expand(B, 1)], 1)
        return torch.log_softmax(logits / self.temperature, -1)

    def positions(self, T: int, R: int, t: int) -> torch.Tensor:
        if T + t > self.cos.shape[0]:
            raise ValueError(f"positions up to {T + t} exceed the rotary tables ({self.cos.shape[0]})")
        return (T + torch.arange(t, dtype=torch.int32)).repeat(R).to(self.dev)

    def score(self, ids: torch.Tensor, states: list, kvalid=None, pool_last: int | None = None) -> torch.Tensor:
        """ids (B, n_opt, t) option-row token ids on the GPU; states[l] = (K, V) Int8KVCache of the B cached
        states. Returns (B, n_opt + 1) log-probabilities over the options and 'none'."""
        B, n_opt, t = ids.shape
        R = B * n_opt
        T = self.state_length(states)
        h0 = self.embed.index_select(0, ids.reshape(-1))
        pos, row_start, max_rows = self.row_layout(T, B, n_opt, t)
        h = self.rows_forward(h0, states, R, t, pos, row_start, max_rows, kvalid, self.row_states(B, n_opt))
        return self.readout(h, B, n_opt, t, pool_last)

    def prefill_layout(self, n0: int, B: int, S: int):
        """Device positions of a state pass appending S tokens at n0 to B states, and the one-row-per-state offsets
        (None for a first prefill or one state), built once per shape so that a prefill makes no host-to-device
        copy."""
        key = ("prefill", n0, B, S)
        if key not in self._rows:
            pos = (n0 + torch.arange(S, dtype=torch.int32)).repeat(B).to(self.dev)
            row_start = kernels.row_start_of([1] * B, self.dev)[0] if (n0 > 0 and B > 1) else None
            self._rows[key] = (pos, row_start)
        return self._rows[key]

    def capture_scoring(self, states, B: int, n_opt: int, t: int, kvalid=None):
        """A HIP graph of every layer of a scoring pass over `states` for B requests x n_opt options x t tokens
        (every kernel launch of the pass recorded once, deploy.py:1-14's static mode). Returns run(ids) -> (B,
        n_opt + 1) log-probabilities: it copies the rows' embeddings into the graph's input buffer, replays the graph
        and reads out. The graph holds the addresses of the states' K/V, their block images, the row layout and the
        activation buffers: re-capture after the states change (append, restore)."""
        cfg = self.cfg
        R = B * n_opt
        T = self.state_length(states)
        pos, row_start, max_rows = self.row_layout(T, B, n_opt, t)
        row_state = self.row_states(B, n_opt)
        h0 = torch.zeros(R * t, cfg.hidden, dtype=torch.bfloat16, device=self.dev)
        side = torch.cuda.Stream(self.dev)  # warm-up off the capture: block images, module loads
        side.wait_stream(torch.cuda.current_stream(self.dev))
        with torch.cuda.stream(side):
            self.rows_forward(h0, states, R, t, pos, row_start, max_rows, kvalid, row_state)
        torch.cuda.current_stream(self.dev).wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            h = self.rows_forward(h0, states, R, t, pos, row_start, max_rows, kvalid, row_state)

        def run(ids: torch.Tensor) -> torch.Tensor:
            if tuple(ids.shape) != (B, n_opt, t):
                raise ValueError(f"captured for ids of shape {(B, n_opt, t)}, got {tuple(ids.shape)}")
            h0.copy_(self.embed.index_select(0, ids.reshape(-1)))
            graph.replay()
            return self.readout(h, B, n_opt, t)

        run.graph = graph
        return run

    def row_layout(self, T: int, B: int, n_opt: int, t: int):
        """Device positions and per-state row offsets of a scoring pass, built once per shape: a host-to-device
        copy per pass would wait for the previous pass to drain the stream."""
        key = (T, B, n_opt, t)
        if key not in self._rows:
            pos = self.positions(T, B * n_opt, t)
            row_start, max_rows = kernels.row_start_of([n_opt] * B, self.dev)
            self._rows[key] = (pos, row_start, max_rows)
        return self._rows[key]


@dataclass
class QuestionCache:
    """The question cache of a question pass: per layer, the block images of every question's K/V (the second prefix
    level), the padded length Lq, the real lengths, each question's state, and the state length it was built on."""
    images: list
    Lq: int
    qlen: list
    gs: list
    group_state: torch.Tensor
    T: int
    gdn: dict = field(default_factory=dict)  # a hybrid stack's per-question GDNState of each Gated DeltaNet layer
