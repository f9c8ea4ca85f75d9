"""GPU parity of the LM-head token log-prob (od_lm_head_logprob) against the oracle (oracle/lm_head.py).

Bar: log-probs within 1e-3 absolute of the oracle (they are natural logs of order -5 .. -15 at a 150k vocabulary;
the device and the oracle differ only in the fp32 accumulation order of each logit, which can move a bf16 rounding
of a logit, and in exp / log), which keeps the probabilities within the 2e-3 relative bar. Closed form: one-hot
rows over a table whose entries are exact in bf16 give the float64 log_softmax of a table column. Rows are
independent, so splitting the rows over calls changes no bit. A token id outside the vocabulary gives NaN.
"""
import pytest
import torch

from oracle import lm_head as ol

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(M, V, K, seed, h_dtype=torch.bfloat16, pow2=False):
    g = torch.Generator().manual_seed(seed)
    w = (torch.randn(V, K, generator=g) * 0.05).to(torch.bfloat16)
    q, s = ol.int8_table(w)
    if pow2:
        s = torch.exp2(torch.randint(-9, -4, (V,), generator=g).float()).to(torch.bfloat16)
    h = (torch.randn(M, K, generator=g) * 2.0).to(h_dtype)
    tok = torch.randint(0, V, (M,), generator=g)
    return h, q, s, tok


def _gpu(h, q, s, tok):
    from opendecider_amd import kernels
    return kernels.lm_head_logprob(h.to(DEV), q.to(DEV), s.to(DEV), tok.to(DEV)).cpu()


def _oracle(h, q, s, tok):
    return ol.token_logprob(h, lambda idx, dt: ol.int8_rows(q, s, idx, dt), q.shape[0], tok)


@pytest.mark.parametrize("M,V,K,h_dtype", [(37, 10007, 256, torch.bfloat16), (300, 4429, 128, torch.float32),
                                           (5, 1000, 64, torch.bfloat16), (513, 2304, 192, torch.bfloat16)])
def test_logprob_matches_oracle(gpu_lib, M, V, K, h_dtype):
    print(f"lm head M={M} V={V} K={K} {h_dtype}", flush=True)
    h, q, s, tok = _case(M, V, K, M + V, h_dtype)
    got, want = _gpu(h, q, s, tok), _oracle(h, q, s, tok)
    d = (got - want).abs().max().item()
    print(f"  max |d log p| {d:.2e}; log p range {want.min().item():.2f} .. {want.max().item():.2f}")
    assert d <= 1e-3
    pg, pw = got.double().exp(), want.double().exp()
    assert ((pg - pw).abs() <= torch.maximum(2e-3 * pw, torch.full_like(pw, 1e-4))).all()


def test_one_hot_closed_form(gpu_lib):
    M, V, K = 6, 3001, 64
    _, q, s, _ = _case(M, V, K, 3, pow2=True)
    col = q.double() * s.double()[:, None]
    h = torch.zeros(M, K, dtype=torch.bfloat16)
    ks = [0, 5, 17, 31, 40, 63]
    for i, k in enumerate(ks):
        h[i, k] = 1.0
    tok = torch.tensor([0, 1, 1500, 2999, 3000, 7])
    got = _gpu(h, q, s, tok).double()
    want = torch.stack([torch.log_softmax(col[:, k], 0)[t] for k, t in zip(ks, tok.tolist())])
    assert torch.allclose(got, want, atol=5e-6), (got - want).abs().max()


def test_rows_are_independent_bitwise(gpu_lib):
    h, q, s, tok = _case(700, 5000, 128, 9)
    a = _gpu(h, q, s, tok)
    b = torch.cat([_gpu(h[:123], q, s, tok[:123]), _gpu(h[123:], q, s, tok[123:])])
    assert torch.equal(a, b)


def test_bad_token_gives_nan_and_shapes(gpu_lib):
    from opendecider_amd import kernels
    h, q, s, tok = _case(8, 777, 64, 4)
    tok[3] = 777
    tok[5] = -1
    got = _gpu(h, q, s, tok)
    assert torch.isnan(got[3]) and torch.isnan(got[5]) and torch.isfinite(got[[0, 1, 2, 4, 6, 7]]).all()
    with pytest.raises(RuntimeError):  # K not a multiple of 64
        kernels.lm_head_logprob(torch.zeros(2, 96, dtype=torch.bfloat16, device=DEV),
                                torch.zeros(10, 96, dtype=torch.int8, device=DEV),
                                torch.ones(10, dtype=torch.bfloat16, device=DEV),
                                torch.zeros(2, dtype=torch.int64, device=DEV))


def test_module_api_and_full_vocab_rows(gpu_lib):
    """Int8Table + token_logprob (the Backbone.token_logprob interface) at a Qwen-size vocabulary and hidden size,
    against the oracle on a few rows."""
    from opendecider_amd import Int8Table, token_logprob
    V, K = 151936, 4096
    g = torch.Generator(device=DEV).manual_seed(11)
    w = (torch.randn(V, K, device=DEV, generator=g) * 0.03).to(torch.bfloat16)
    table = Int8Table(w)
    del w
    h = torch.randn(4, K, device=DEV, generator=g).to(torch.bfloat16)
    tok = torch.tensor([0, 1, 77777, V - 1], device=DEV)
    got = token_logprob(table, h, tok).cpu()
    q, s = table.qweight.cpu(), table.scale.cpu().reshape(-1)
    want = _oracle(h.cpu(), q, s, tok.cpu())
    assert (got - want).abs().max().item() <= 1e-3, (got, want)


# ---- Q4_0 tables (od_lm_head_logprob_q4)

def _q4_case(M, V, K, seed, h_dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(V, K, generator=g) * 0.05
    qs, d = ol.q4_table(w)
    h = (torch.randn(M, K, generator=g) * 2.0).to(h_dtype)
    tok = torch.randint(0, V, (M,), generator=g)
    return h, qs, d, tok


def _q4_gpu(h, qs, d, tok):
    from opendecider_amd import kernels
    return kernels.lm_head_logprob_q4(h.to(DEV), qs.to(DEV), d.to(DEV), tok.to(DEV)).cpu()


def _q4_oracle(h, qs, d, tok):
    return ol.token_logprob(h, lambda idx, dt: ol.q4_rows(qs, d, idx, dt), qs.shape[0], tok)


@pytest.mark.parametrize("M,V,K,h_dtype", [(37, 10007, 256, torch.bfloat16), (300, 4429, 128, torch.float32),
                                           (513, 2304, 192, torch.bfloat16)])
def test_q4_logprob_matches_oracle(gpu_lib, M, V, K, h_dtype):
    print(f"lm head q4 M={M} V={V} K={K} {h_dtype}", flush=True)
    h, qs, d, tok = _q4_case(M, V, K, M + V + 1, h_dtype)
    got, want = _q4_gpu(h, qs, d, tok), _q4_oracle(h, qs, d, tok)
    assert (got - want).abs().max().item() <= 1e-3
    pg, pw = got.double().exp(), want.double().exp()
    assert ((pg - pw).abs() <= torch.maximum(2e-3 * pw, torch.full_like(pw, 1e-4))).all()


def test_q4_one_hot_closed_form(gpu_lib):
    """One-hot h over a Q4 table whose block scales are powers of two (entries exact in bf16 and fp16): the float64
    log_softmax of a table column, at both nibble halves of a block."""
    g = torch.Generator().manual_seed(8)
    V, K = 900, 64
    qv = torch.randint(0, 16, (V, K // 32, 32), generator=g)
    qv[..., 3] = 0
    dd = torch.exp2(torch.randint(-10, -3, (V, K // 32, 1), generator=g).float())
    w = ((qv - 8).float() * dd).view(V, K)
    qs, d = ol.q4_table(w)
    ks = [0, 15, 16, 31, 40, 63]
    h = torch.zeros(len(ks), K, dtype=torch.bfloat16)
    for i, k in enumerate(ks):
        h[i, k] = 1.0
    tok = torch.tensor([0, 450, 899, 1, 2, 3])
    got = _q4_gpu(h, qs, d, tok).double()
    want = torch.stack([torch.log_softmax(w[:, k].double(), 0)[t] for k, t in zip(ks, tok.tolist())])
    assert torch.allclose(got, want, atol=5e-6), (got - want).abs().max()


def test_q4_module_api(gpu_lib):
    """Q4Table + token_logprob equals the kernel wrapper, and Q4Table's bytes are the oracle's."""
    from opendecider_amd import Q4Table, token_logprob
    g = torch.Generator().manual_seed(12)
    w = torch.randn(3000, 256, generator=g) * 0.05
    t = Q4Table(w.to(DEV))
    qs, d = ol.q4_table(w)
    assert torch.equal(t.qs.cpu(), qs) and torch.equal(t.d.cpu(), d)
    h = torch.randn(20, 256, generator=g).to(torch.bfloat16)
    tok = torch.randint(0, 3000, (20,), generator=g)
    assert torch.equal(token_logprob(t, h.to(DEV), tok.to(DEV)).cpu(), _q4_gpu(h, qs, d, tok))


def test_leading_dims_and_empty_rows(gpu_lib):
    """h (..., K) and tok (...) give log-probs of shape (...), the rows of a flattened call; zero rows give an empty
    result without a launch (both table formats)."""
    from opendecider_amd import kernels
    h, q, s, tok = _case(12, 3000, 128, 21)
    flat = _gpu(h, q, s, tok)
    got = kernels.lm_head_logprob(h.view(3, 4, 128).to(DEV), q.to(DEV), s.to(DEV), tok.view(3, 4).to(DEV)).cpu()
    assert got.shape == (3, 4) and torch.equal(got.reshape(-1), flat)
    e = kernels.lm_head_logprob(h[:0].to(DEV), q.to(DEV), s.to(DEV), tok[:0].to(DEV))
    assert e.shape == (0,)
    qs, d = ol.q4_table(q.float() * s.float()[:, None])
    e4 = kernels.lm_head_logprob_q4(h[:0].to(DEV), qs.to(DEV), d.to(DEV), tok[:0].to(DEV))
    assert e4.shape == (0,)
    g4 = kernels.lm_head_logprob_q4(h.view(2, 6, 128).to(DEV), qs.to(DEV), d.to(DEV), tok.view(2, 6).to(DEV)).cpu()
    assert torch.equal(g4.reshape(-1), _q4_gpu(h, qs, d, tok))
