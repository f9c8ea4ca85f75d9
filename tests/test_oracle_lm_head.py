"""Pins the LM-head log-prob oracle (oracle/lm_head.py) without retyping its formula: the reference's own chunk test
restated (tests/test_materialize.py:27-38 of the reference), a one-hot closed form (log p = log_softmax of a table
column, in float64), normalisation over the vocabulary, invariance under a permutation of the vocabulary, and the
reference's Q4 table tests restated (tests/test_q4table.py:7-39)."""
import math

import torch

from oracle import lm_head as ol
from oracle import quant as oq


def _table(V, K, seed, pow2_scale=False):
    g = torch.Generator().manual_seed(seed)
    q = torch.randint(-127, 128, (V, K), generator=g, dtype=torch.int8)
    if pow2_scale:  # rows q * 2^e are exact in bf16 (<= 8 significant bits)
        s = torch.exp2(torch.randint(-9, -4, (V,), generator=g).float()).to(torch.bfloat16)
    else:
        s = (torch.rand(V, generator=g) * 0.02 + 1e-3).to(torch.bfloat16)
    return q, s


def test_row_chunks_do_not_change_the_result():
    """The reference's test: the chunking of the vocabulary does not change the result (atol 1e-5)."""
    V, K = 10007, 64
    q, s = _table(V, K, 1)
    rows = lambda idx, dt: ol.int8_rows(q, s, idx, dt)
    g = torch.Generator().manual_seed(2)
    h = torch.randn(37, K, generator=g)
    tok = torch.randint(0, V, (37,), generator=g)
    a = ol.token_logprob(h, rows, V, tok)
    for chunk in (4096, 1000, 10007):
        b = ol.token_logprob(h, rows, V, tok, chunk=chunk)
        assert torch.allclose(a, b, atol=1e-5), chunk


def test_one_hot_rows_give_log_softmax_of_a_column():
    """h = e_k: every logit is the table entry (k) itself, exact in bf16 for power-of-two scales, so log p(tok) is
    the float64 log_softmax of column k at tok."""
    V, K = 3001, 32
    q, s = _table(V, K, 3, pow2_scale=True)
    rows = lambda idx, dt: ol.int8_rows(q, s, idx, dt)
    col = (q.double() * s.double()[:, None])                       # exact entries
    for k in (0, 7, 31):
        h = torch.zeros(5, K)
        h[:, k] = 1.0
        tok = torch.tensor([0, 1, 17, 2999, 3000])
        got = ol.token_logprob(h, rows, V, tok, chunk=512)
        want = torch.log_softmax(col[:, k], 0)[tok]
        assert torch.allclose(got.double(), want, atol=2e-6), (k, (got.double() - want).abs().max())


def test_probabilities_over_the_vocabulary_sum_to_one():
    """When every logit is exact in bf16 the target term equals the logit, so exp(log p) over every token sums to 1:
    entries in -3..3 times a power of two, and h with small integer weights, keep each dot product below 2^5 in
    units of the row's scale."""
    V, K = 700, 16
    q, s = _table(V, K, 4, pow2_scale=True)
    q = torch.remainder(q.to(torch.int32), 7).to(torch.int8) - 3
    rows = lambda idx, dt: ol.int8_rows(q, s, idx, dt)
    h = torch.tensor([[1.0, -2.0, 1.0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 1.0]])
    lp = ol.token_logprob(h.repeat(V, 1), rows, V, torch.arange(V), chunk=128)
    assert abs(torch.logsumexp(lp.double(), 0).item()) < 1e-5


def test_vocabulary_permutation():
    V, K = 2000, 48
    q, s = _table(V, K, 5)
    g = torch.Generator().manual_seed(6)
    h = torch.randn(9, K, generator=g)
    tok = torch.randint(0, V, (9,), generator=g)
    perm = torch.randperm(V, generator=g)
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(V)
    a = ol.token_logprob(h, lambda i, dt: ol.int8_rows(q, s, i, dt), V, tok, chunk=777)
    b = ol.token_logprob(h, lambda i, dt: ol.int8_rows(q[perm], s[perm], i, dt), V, inv[tok], chunk=777)
    assert torch.allclose(a, b, atol=1e-5)


def test_int8_table_is_the_row_quantizer():
    """Int8Embedding's table (quant.py:189-194) uses the Int8Tensor formula per row; the stored scale is bf16."""
    g = torch.Generator().manual_seed(7)
    w = (torch.randn(300, 96, generator=g) * 0.05).to(torch.bfloat16)
    q, s = ol.int8_table(w)
    rq, rs = oq.quantize_rows(w)
    assert torch.equal(q, rq) and s.dtype == torch.bfloat16
    assert torch.equal(s, rs.squeeze(1).to(torch.bfloat16))
    # dequant_rows in bf16 is the bf16 product of the two bf16 factors
    r = ol.int8_rows(q, s, slice(None), torch.bfloat16)
    assert torch.equal(r, (q.float() * s.float()[:, None]).to(torch.bfloat16))


def _q4_0_values(n=50, k=64, seed=0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randint(0, 16, (n, k // 32, 32), generator=g)
    q[..., 5] = 0
    d = (torch.rand(n, k // 32, 1, generator=g) * 0.02 + 1e-3).half().float()
    return ((q - 8).float() * d).view(n, k)


def test_q4_0_values_round_trip_exactly():
    w = _q4_0_values()
    qs, d = ol.q4_table(w)
    assert torch.equal(ol.q4_rows(qs, d, slice(None), torch.float32), w)


def test_q4_error_bound_and_bytes():
    g = torch.Generator().manual_seed(0)
    w = torch.randn(40, 96, generator=g)
    qs, d = ol.q4_table(w)
    err = (ol.q4_rows(qs, d, slice(None), torch.float32) - w).abs().view(40, 3, 32)
    dd = w.view(40, 3, 32).abs().amax(-1, keepdim=True) / 8
    assert (err <= dd + 1e-6).all() and err.mean() < (dd * 0.3).mean()
    assert qs.numel() + 2 * d.numel() == 40 * 96 // 2 + 40 * 3 * 2
    assert torch.equal(ol.q4_rows(qs, d, torch.tensor([5, 9]), torch.float32),
                       ol.q4_rows(qs, d, slice(None), torch.float32)[[5, 9]])


def test_q4_one_hot_closed_form():
    """One-hot h over a Q4 table whose entries are exact in bf16 (fp16 block scales that are powers of two)."""
    g = torch.Generator().manual_seed(8)
    V, K = 900, 64
    qv = torch.randint(0, 16, (V, K // 32, 32), generator=g)
    qv[..., 3] = 0
    d = torch.exp2(torch.randint(-10, -3, (V, K // 32, 1), generator=g).float())
    w = ((qv - 8).float() * d).view(V, K)
    qs, dd = ol.q4_table(w)
    rows = lambda idx, dt: ol.q4_rows(qs, dd, idx, dt)
    h = torch.zeros(3, K)
    h[:, 40] = 1.0
    tok = torch.tensor([0, 450, 899])
    got = ol.token_logprob(h, rows, V, tok, chunk=256)
    want = torch.log_softmax(w[:, 40].double(), 0)[tok]
    assert torch.allclose(got.double(), want, atol=2e-6)
    assert math.isfinite(got.sum().item())
