"""Tolerances shared by the parity tests.

The path's bar for floating-point outputs is 2e-3 relative against the oracle's fp32 result. A bf16 output cannot
agree elementwise with an fp32 value to better than its own rounding (up to 2^-9 relative, and two candidate
roundings differ by 2^-8), so the bar is checked in three forms:
  * norm-relative, whole tensor:     ||out - ref||_2 <= 2e-3 ||ref||_2
  * norm-relative, every slice along dim 0 (one option row, one token row, ...)
  * elementwise:                     |out - ref| <= 2^-8 |ref| + 2e-3 rms(ref)
    (one bf16 step at the element's own magnitude, plus 2e-3 of the tensor's rms for the kernel's own error)
Probabilities are held to 1e-4 absolute. Integer and byte outputs are compared exactly.
"""
import torch

REL = 2e-3
PROB_ABS = 1e-4
BF16_STEP = 2.0 ** -8


def rel_err(out: torch.Tensor, ref: torch.Tensor) -> float:
    out, ref = out.detach().double().cpu(), ref.detach().double().cpu()
    return ((out - ref).norm() / ref.norm().clamp_min(1e-300)).item()


def error_stats(out: torch.Tensor, ref: torch.Tensor) -> dict:
    out, ref = out.detach().double().cpu(), ref.detach().double().cpu()
    d = (out - ref).abs()
    rms = ref.pow(2).mean().sqrt().clamp_min(1e-300)
    return {
        "norm_rel": ((out - ref).norm() / ref.norm().clamp_min(1e-300)).item(),
        "max_abs_over_rms": (d.max() / rms).item(),
        "elem_ratio": (d / (BF16_STEP * ref.abs() + REL * rms)).max().item(),  # <= 1 passes
    }


def assert_close_rel(out: torch.Tensor, ref: torch.Tensor, rel: float = REL, what: str = "", elem_steps: int = 1) -> dict:
    """The three forms above; elem_steps widens the elementwise form to that many bf16 steps of |ref| (used where
    the algorithm itself rounds an intermediate to bf16, so a last-bit difference upstream can flip that rounding)."""
    out, ref = out.detach().double().cpu(), ref.detach().double().cpu()
    assert out.shape == ref.shape, (what, out.shape, ref.shape)
    assert torch.isfinite(out).all(), f"{what}: non-finite values"
    st = error_stats(out, ref)
    assert st["norm_rel"] <= rel, f"{what}: norm-relative error {st}"
    if out.dim() > 1 and out.shape[0] > 1:
        o2, r2 = out.reshape(out.shape[0], -1), ref.reshape(ref.shape[0], -1)
        per = ((o2 - r2).norm(dim=1) / r2.norm(dim=1).clamp_min(1e-300))
        st["worst_slice_norm_rel"] = per.max().item()
        assert st["worst_slice_norm_rel"] <= rel, f"{what}: a slice along dim 0 is beyond {rel}: {st}"
    rms = ref.pow(2).mean().sqrt()
    bad = (out - ref).abs() > elem_steps * BF16_STEP * ref.abs() + rel * rms
    assert not bad.any(), f"{what}: {int(bad.sum())} elements beyond {elem_steps} x 2^-8|ref| + {rel} rms: {st}"
    return st


def decoder_case(cfg_kw: dict, B: int, n_opt: int, t: int, T: int, temperature: float = 1.0):
    """The seeded decision-forward case shared by the GPU end-to-end tests and the CPU tests of their bar: random-init
    weights (seed 3) with the decision temperature, embedding (seed 3), per-layer int8 states of T tokens (source bf16
    N(0,1), seed 4) and option token ids (seed 5). Returns (cfg, weights, embedding, states, ids)."""
    from oracle import decoder as od
    from oracle import quant as oq
    cfg = od.DecoderConfig(**cfg_kw)
    w = od.make_weights(cfg, seed=3)
    w["temperature"] = temperature
    emb = od.make_embedding(cfg, seed=3)
    g = torch.Generator().manual_seed(4)
    states = []
    for _ in range(cfg.n_layers):
        kv = torch.randn(2, B, cfg.n_kv_heads, T, cfg.head_dim, generator=g).to(torch.bfloat16)
        kq, ks = oq.quantize_rows(kv[0])
        vq, vs = oq.quantize_rows(kv[1])
        states.append(((kq, ks[..., 0]), (vq, vs[..., 0])))
    ids = torch.randint(0, cfg.vocab, (B, n_opt, t), generator=torch.Generator().manual_seed(5))
    return cfg, w, emb, states, ids


def hybrid_states(cfg, B: int, T: int, seed: int = 4):
    """Per-layer states of B requests for a hybrid stack: int8 K/V of T tokens (bf16 N(0, 1) source) for the attention
    layers; a conv window (bf16 N(0, 1)) and a recurrent state (fp32 0.05 N(0, 1)) for the GDN layers."""
    from oracle import quant as oq
    g = torch.Generator().manual_seed(seed)
    gc = cfg.gdn
    out = []
    for li in range(cfg.n_layers):
        if cfg.is_gdn(li):
            out.append((torch.randn(B, 3, gc.conv_dim, generator=g).to(torch.bfloat16),
                        torch.randn(B, gc.n_v_heads, gc.dk, gc.dv, generator=g) * 0.05))
        else:
            kv = torch.randn(2, B, cfg.n_kv_heads, T, cfg.head_dim, generator=g).to(torch.bfloat16)
            kq, ks = oq.quantize_rows(kv[0])
            vq, vs = oq.quantize_rows(kv[1])
            out.append(((kq, ks[..., 0]), (vq, vs[..., 0])))
    return out
