"""The int8 quantizer of the gfx950 kernels replaces the per-element IEEE division v / scale with a multiplication by
inv = RN(1 / scale), reads the integer out of v * inv + 1.5 * 2^23, and redoes the division only where v * inv lies
within 2^-15 of a half-integer. This restates those steps in numpy float32 (every operation one IEEE rounding, as
on the device) and checks them against the oracle's quantizer (oracle/quant.py quantize_rows, IEEE division and
round half to even) on random rows over a wide range of magnitudes and on values placed a few ulps around the
decision points k + 0.5. A zero tolerance (no fallback) must fail, which shows the cases reach the boundary."""
import numpy as np
import torch

from oracle import quant as oq

F32 = np.float32
MAGIC = F32(12582912.0)                      # 1.5 * 2^23
TIE_EDGE = F32(0.5) - F32(2.0 ** -15)


def _device_steps(v: np.ndarray, scale: np.ndarray, edge: np.float32):
    inv = (F32(1.0) / scale).astype(F32)
    q = (v * inv).astype(F32)
    t = (q + MAGIC).astype(F32)
    d = (q - (t - MAGIC)).astype(F32)
    fast = (t.view(np.uint32) & 0xFF).astype(np.uint8).view(np.int8)
    exact = np.clip(np.rint((v / scale).astype(F32)), -127, 127).astype(np.int8)
    flagged = np.abs(d) >= edge
    return np.where(flagged, exact, fast), flagged


def _bf16(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(x).to(torch.bfloat16).float().numpy()


def test_division_free_quantizer_equals_ieee_division_random_rows():
    rng = np.random.default_rng(5)
    flagged_total = 0
    for it in range(6):
        x = rng.standard_normal((1024, 1024), dtype=F32) * np.exp(rng.uniform(-25, 25, (1024, 1))).astype(F32)
        x[:, :8] *= F32(20.0)                                   # outlier channels
        x = _bf16(x)
        q_ref, s_ref = oq.quantize_rows(torch.from_numpy(x))
        scale = s_ref.numpy().astype(F32)
        q, flagged = _device_steps(x, scale, TIE_EDGE)
        assert np.array_equal(q, q_ref.numpy())
        flagged_total += int(flagged.sum())
    assert flagged_total < 6 * 1024 * 1024 * 1e-3              # the division is rare


def test_division_free_quantizer_at_half_integer_boundaries():
    rng = np.random.default_rng(6)
    scale = np.exp(rng.uniform(-20, 6, (2048, 1))).astype(F32)
    h = rng.integers(-127, 127, (2048, 512)).astype(F32) + F32(0.5)
    base = (h * scale).astype(F32)
    v = (base.view(np.int32) + rng.integers(-40, 41, base.shape).astype(np.int32)).view(F32)
    exact = np.clip(np.rint((v / scale).astype(F32)), -127, 127).astype(np.int8)
    q, _ = _device_steps(v, scale, TIE_EDGE)
    assert np.array_equal(q, exact)
    q0, _ = _device_steps(v, scale, F32(1.0))                   # never flagged: the fast step alone
    assert not np.array_equal(q0, exact)
