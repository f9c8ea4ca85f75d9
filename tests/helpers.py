"""Tolerances shared by the parity tests.

Floating-point outputs are held to the path's stated bar, 2e-3 relative, in two forms:
  * norm-relative:  ||out - ref||_2 <= 2e-3 ||ref||_2
  * elementwise:    |out - ref| <= 2e-3 (|ref| + rms(ref))
`ref` is the oracle's fp32 value (before any bf16 rounding), so a bf16 output's own rounding (<= 2^-9 relative)
is inside the budget. Probabilities are held to 1e-4 absolute. Integer and byte outputs are compared exactly.
"""
import torch

REL = 2e-3
PROB_ABS = 1e-4


def rel_err(out: torch.Tensor, ref: torch.Tensor) -> float:
    out, ref = out.detach().double().cpu(), ref.detach().double().cpu()
    return ((out - ref).norm() / ref.norm().clamp_min(1e-30)).item()


def assert_close_rel(out: torch.Tensor, ref: torch.Tensor, rel: float = REL, what: str = ""):
    out, ref = out.detach().double().cpu(), ref.detach().double().cpu()
    assert out.shape == ref.shape, (what, out.shape, ref.shape)
    assert torch.isfinite(out).all(), f"{what}: non-finite values"
    e = rel_err(out, ref)
    assert e <= rel, f"{what}: norm-relative error {e:.3e} > {rel}"
    rms = ref.pow(2).mean().sqrt()
    bad = (out - ref).abs() > rel * (ref.abs() + rms)
    assert not bad.any(), (f"{what}: {int(bad.sum())} elements beyond {rel} (|ref| + rms); worst "
                           f"{((out - ref).abs() / (ref.abs() + rms)).max().item():.3e}")
    return e
