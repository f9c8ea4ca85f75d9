"""Seeded random shapes through the whole W8A8 linear (activation quantizer, GEMM, epilogue with bias and residual),
the LM-head log-prob and the branched attention, against the oracle: the fixed-shape tests pick the edges by hand,
these draw ragged M / N / V and K from the ranges each entry point accepts (K a multiple of 16 for the GEMM, of 64
for the LM head), and for the attention ragged state lengths, capacities, row counts per state (empty states
included), GQA groups 1-8, own-token counts up to 48 (rows whose (head, token) slots span two 128-slot tiles) and
key masks, so a tile-boundary case nobody listed still meets the bars: bit-exact int8 / int32 / bf16 for the linear,
|d log p| <= 1e-3 for the log-probs, the one-pass bar (2e-3 relative, LSE within 1e-4) for the attention, whose
direct path must give the staged path's bits."""
import pytest
import torch

from oracle import lm_head as ol
from oracle import quant as oq

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _shapes(seed, n, lo, hi):
    g = torch.Generator().manual_seed(seed)
    return [tuple(int(torch.randint(a, b + 1, (1,), generator=g)) for a, b in zip(lo, hi)) for _ in range(n)]


@pytest.mark.parametrize("M,N,K16", _shapes(101, 12, (1, 1, 1), (700, 900, 70)))
def test_w8a8_linear_random_shape(gpu_lib, M, N, K16):
    from opendecider_amd import kernels
    K = 16 * K16
    print(f"w8a8 linear M={M} N={N} K={K}", flush=True)
    g = torch.Generator().manual_seed(M * 7919 + N * 31 + K)
    x = (torch.randn(M, K, generator=g) * 2).to(torch.bfloat16)
    w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    sw = torch.rand(N, generator=g) * 1.5e-3 + 0.5e-3
    bias = torch.randn(N, generator=g).to(torch.bfloat16)
    res = torch.randn(M, N, generator=g).to(torch.bfloat16)
    xq, sx = kernels.act_quant(x.to(DEV))
    out, acc = kernels.w8a8_gemm(xq, sx, w.to(DEV), sw.to(DEV), bias=bias.to(DEV), residual=res.to(DEV),
                                 want_acc=True)
    rout, racc, rxq, rsx = oq.w8a8_linear(x, w, sw, bias=bias, residual=res)
    assert torch.equal(xq.cpu(), rxq) and torch.equal(sx.cpu(), rsx)
    assert torch.equal(acc.cpu(), racc)
    assert torch.equal(out.cpu(), rout)


@pytest.mark.parametrize("M,V,K64", _shapes(202, 8, (1, 1, 1), (600, 5000, 6)))
def test_lm_head_logprob_random_shape(gpu_lib, M, V, K64):
    from opendecider_amd import kernels
    K = 64 * K64
    print(f"lm head M={M} V={V} K={K}", flush=True)
    g = torch.Generator().manual_seed(M * 7919 + V * 31 + K)
    q, s = ol.int8_table((torch.randn(V, K, generator=g) * 0.05).to(torch.bfloat16))
    h = (torch.randn(M, K, generator=g) * 2).to(torch.bfloat16)
    tok = torch.randint(0, V, (M,), generator=g)
    got = kernels.lm_head_logprob(h.to(DEV), q.to(DEV), s.to(DEV), tok.to(DEV)).cpu()
    want = ol.token_logprob(h, lambda idx, dt: ol.int8_rows(q, s, idx, dt), V, tok)
    assert (got - want).abs().max().item() <= 1e-3


def _attn_cases(seed, n):
    g = torch.Generator().manual_seed(seed)
    r = lambda a, b: int(torch.randint(a, b + 1, (1,), generator=g))
    out = []
    for i in range(n):
        Ns = r(1, 3)
        counts = [r(0, 5) for _ in range(Ns)]
        counts[r(0, Ns - 1)] += 1
        Hkv = (2, 4, 8)[r(0, 2)]
        group = (1, 2, 4, 8)[r(0, 3 if Hkv <= 4 else 2)]
        T = r(0, 700)
        out.append(dict(seed=1000 + i, Ns=Ns, row_counts=counts, Hq=Hkv * group, Hkv=Hkv, t=r(1, 48),
                        D=(64, 128)[r(0, 1)], T=T, cap=T + r(0, 50), holes=T > 0 and r(0, 1) == 1))
    return out


@pytest.mark.parametrize("case", _attn_cases(303, 10), ids=lambda c: "Ns{Ns}-R{row_counts}-H{Hq}x{Hkv}-t{t}-D{D}-T{T}"
                         .format(**c).replace(" ", ""))
def test_branched_attention_random_shape(gpu_lib, case):
    """One pass (block images), the direct int8 path (the same bits) and a split over key ranges, against the
    oracle at the one-pass bar."""
    from test_gpu_attention import make_case, run_gpu, run_oracle
    from helpers import assert_close_rel
    print(f"attention {case}", flush=True)
    c = make_case(**case)
    ref, ref_lse = run_oracle(c)
    out, lse = run_gpu(c)
    assert_close_rel(out.float().cpu(), ref, what="one pass")
    assert (lse.cpu() - ref_lse).abs().max().item() <= 1e-4
    out_d, lse_d = run_gpu(c, staged=False)
    assert torch.equal(out_d, out) and torch.equal(lse_d, lse)
    n_split = 2 + case["seed"] % 7
    out_s, lse_s = run_gpu(c, n_split=n_split)
    assert_close_rel(out_s.float().cpu(), ref, what=f"split {n_split}")
    assert (lse_s.cpu() - ref_lse).abs().max().item() <= 1e-4
