"""Pins the quantization / W8A8 oracle (oracle/quant.py) against arithmetic that does not reuse its formula:
exact rational IEEE rounding, hand-derived known answers, bounds and invariants, brute-force integer loops, and the
reference's own SmoothQuant test restated (tests/test_int8_gemm.py:70-88 of the reference)."""
import json
import os
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import quant as oq

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


# ---------------------------------------------------------------- exact IEEE float32 helpers (independent of torch)
def _f32_round(fr: Fraction) -> np.float32:
    """Nearest float32 to the exact rational `fr`, ties to even, computed by exact comparison."""
    approx = np.float32(float(fr))
    cands = {approx, np.nextafter(approx, np.float32(np.inf)), np.nextafter(approx, np.float32(-np.inf))}
    best = None
    for c in sorted(cands, key=float):
        d = abs(Fraction(float(c)) - fr)
        if best is None or d < best[0]:
            best = (d, c)
        elif d == best[0]:                                    # tie: even mantissa
            if int(np.float32(c).view(np.uint32)) % 2 == 0:
                best = (d, c)
    return best[1]


def _round_half_even(fr: Fraction) -> int:
    fl = fr.numerator // fr.denominator
    rem = fr - fl
    if rem > Fraction(1, 2):
        return fl + 1
    if rem < Fraction(1, 2):
        return fl
    return fl if fl % 2 == 0 else fl + 1


def _brute_quantize_row(row: np.ndarray):
    """Per-element exact arithmetic: scale = fl32(max(|x|, 1e-8f) / 127), q = rne(fl32(x / scale)) clamped."""
    xs = [Fraction(float(np.float32(v))) for v in row]
    amax = max(abs(v) for v in xs)
    amax = max(amax, Fraction(float(np.float32(1e-8))))
    scale = _f32_round(amax / 127)
    qs = []
    for v in xs:
        quo = _f32_round(v / Fraction(float(scale)))
        qs.append(max(-127, min(127, _round_half_even(Fraction(float(quo))))))
    return qs, float(scale)


def test_quantize_matches_exact_ieee_brute_force():
    g = torch.Generator().manual_seed(11)
    x = torch.randn(6, 37, generator=g) * torch.logspace(-3, 2, 6)[:, None]
    x[2, 5] = 0.0
    x[3] *= 0.0                                                  # all-zero row -> clamp_min(1e-8) path
    q, s = oq.quantize_rows(x)
    for i in range(x.shape[0]):
        qs, sc = _brute_quantize_row(x[i].numpy())
        assert q[i].tolist() == qs
        assert s[i, 0].item() == sc


def test_quantize_known_answers():
    with open(os.path.join(GOLDEN, "quant_known_answers.json")) as f:
        cases = json.load(f)
    for c in cases:
        x = torch.tensor(c["x"], dtype=torch.float32)[None]
        q, s = oq.quantize_rows(x)
        assert q[0].tolist() == c["q"], c["name"]
        assert s[0, 0].item() == np.float32(c["scale"]), c["name"]


def test_quantize_bf16_input_and_bounds():
    g = torch.Generator().manual_seed(3)
    x = (torch.randn(64, 128, generator=g) * 3).to(torch.bfloat16)
    q, s = oq.quantize_rows(x)
    xf = x.float()
    # the absmax element of every row lands on +-127 and every element is within half a step
    assert (q.abs().amax(-1) == 127).all()
    assert ((q.float() * s - xf).abs() <= s / 2 + xf.abs() * 2.0 ** -21).all()   # half a step + fp32 ulps
    # reference round-trip bound (tests/test_components.py:11-17 of the reference)
    assert ((oq.dequantize(q, s) - xf).abs().max() <= xf.abs().amax() / 127 + 1e-6)


def test_quantize_slices_equal_whole():
    """Per-(token, head) scales: quantizing only the appended tokens gives the bytes of quantizing everything."""
    g = torch.Generator().manual_seed(5)
    x = torch.randn(2, 4, 96, 64, generator=g).to(torch.bfloat16)
    q_all, s_all = oq.quantize_rows(x)
    q_a, s_a = oq.quantize_rows(x[:, :, :70])
    q_b, s_b = oq.quantize_rows(x[:, :, 70:])
    assert torch.equal(torch.cat([q_a, q_b], 2), q_all) and torch.equal(torch.cat([s_a, s_b], 2), s_all)


def test_int_gemm_brute_force_and_closed_form():
    g = torch.Generator().manual_seed(7)
    a = torch.randint(-127, 128, (5, 48), generator=g, dtype=torch.int8)
    w = torch.randint(-127, 128, (7, 48), generator=g, dtype=torch.int8)
    acc = oq.int_gemm(a, w)
    for i in range(5):
        for j in range(7):
            assert acc[i, j].item() == sum(int(a[i, k]) * int(w[j, k]) for k in range(48))
    ones = torch.ones(3, 48, dtype=torch.int8)
    assert torch.equal(oq.int_gemm(ones, w), w.to(torch.int32).sum(1)[None].expand(3, 7))
    # the largest accumulator the 9B shapes can produce stays exact
    big = torch.full((2, 12288), 127, dtype=torch.int8)
    assert oq.int_gemm(big, -big)[0, 0].item() == -127 * 127 * 12288


@pytest.mark.parametrize("M,N,K", [(32, 64, 256), (1, 3, 16), (300, 70, 1040)])
def test_int_gemm_matches_int64_matmul(M, N, K):
    g = torch.Generator().manual_seed(8)
    a = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8)
    w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    ref = (a.to(torch.int64) @ w.to(torch.int64).t())
    assert torch.equal(oq.int_gemm(a, w).to(torch.int64), ref)


def test_epilogue_within_one_bf16_rounding_of_float64():
    g = torch.Generator().manual_seed(9)
    acc = torch.randint(-2**27, 2**27, (16, 24), generator=g, dtype=torch.int32)
    sx = torch.rand(16, generator=g) * 0.1
    sw = torch.rand(24, generator=g) * 2e-3 + 5e-4
    bias = torch.randn(24, generator=g).to(torch.bfloat16)
    y = oq.w8a8_epilogue(acc, sx, sw, bias).double()
    y64 = acc.double() * sx.double()[:, None] * sw.double()[None] + bias.double()[None]
    assert ((y - y64).abs() <= y64.abs() * 2.0 ** -8 + 1e-30).all()
    # operands are not transposed: row m uses sx[m], column n uses sw[n]
    sx2 = sx.clone()
    sx2[3] *= 2
    assert torch.equal(oq.w8a8_epilogue(acc, sx2, sw)[4], oq.w8a8_epilogue(acc, sx, sw)[4])
    assert not torch.equal(oq.w8a8_epilogue(acc, sx2, sw)[3], oq.w8a8_epilogue(acc, sx, sw)[3])


def test_w8a8_linear_close_to_float_linear():
    """W8A8 with outlier channels and SmoothQuant is a close approximation of the float linear."""
    g = torch.Generator().manual_seed(10)
    K, N = 256, 96
    x = torch.randn(40, K, generator=g)
    x[:, torch.randperm(K, generator=g)[:3]] *= 20
    x = x.to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    s = oq.smooth_scales(x.abs().amax(0), w, 0.5)
    wq, sw = oq.quantize_weight(oq.smooth_fold(w, s))
    out, acc, xq, sx = oq.w8a8_linear(x, wq, sw, inv_s=oq.smooth_inv(s))
    ref = x.float() @ w.float().t()
    assert ((out.float() - ref).norm() / ref.norm()).item() < 0.03


def test_smoothquant_wrapper_is_exact_math():
    """Restates the reference's test_smoothquant_wrapper_is_exact_math (test_int8_gemm.py:70-88)."""
    torch.manual_seed(0)
    lin = torch.nn.Linear(16, 8, bias=True).double()
    x = torch.randn(32, 16, dtype=torch.float64) * torch.logspace(-1, 2, 16, dtype=torch.float64)
    s = oq.smooth_scales(x.abs().amax(0), lin.weight.data, 0.5).double()
    assert torch.allclose(s, (x.abs().amax(0) ** 0.5 / lin.weight.abs().amax(0) ** 0.5).clamp(1e-3, 1e3), rtol=1e-4)
    w_folded = lin.weight.data * s[None, :]
    y = torch.nn.functional.linear(x * (1.0 / s), w_folded, lin.bias.data)
    assert torch.allclose(y, lin(x), atol=1e-10)
    xs = x / s
    assert xs.abs().amax(0).max() / xs.abs().amax(0).min() < x.abs().amax(0).max() / x.abs().amax(0).min()


def test_smooth_input_rounds_product_to_bf16():
    x = torch.tensor([[1.0, 3.0, -7.0]], dtype=torch.bfloat16)
    inv = torch.tensor([1 / 3, 1 / 3, 0.1], dtype=torch.float32)
    y = oq.smooth_input(x, inv.to(torch.bfloat16))
    exp = (x.float() * inv.to(torch.bfloat16).float()).to(torch.bfloat16)
    assert torch.equal(y, exp) and y.dtype == torch.bfloat16


def test_int8_linear_dequant_path():
    """Int8Linear's unfused path keeps the reference's relative error bound (test_components.py:20-26)."""
    torch.manual_seed(0)
    lin = torch.nn.Linear(64, 32)
    wq, s = oq.quantize_weight(lin.weight.data)
    x = torch.randn(10, 64)
    y = oq.int8_linear_dequant(x, wq, s, lin.bias.data)
    assert ((y - lin(x)).norm() / lin(x).norm()).item() < 0.01
