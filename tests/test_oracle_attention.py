"""Pins the attention oracle (oracle/attention.py): float64 brute-force softmax loops on tiny shapes, the LSE merge
against ONE softmax over the concatenated keys (the reference's math note, docs/branched_shared_prefix_math.md
:39-48), torch.logsumexp, permutation equivariance over option rows, and the empty-key-set rules of
wide_attention.py:62,65-67."""
import pytest
import torch

from oracle import attention as oa


def _rand(g, *shape):
    return torch.randn(*shape, generator=g)


@pytest.mark.parametrize("B,H,G,T,S,causal", [(1, 4, 2, 5, 5, True), (2, 4, 1, 3, 9, True), (1, 2, 2, 4, 7, False),
                                              (2, 6, 3, 1, 4, True)])
@pytest.mark.parametrize("masked", [False, True])
def test_attention_matches_brute_force(B, H, G, T, S, causal, masked):
    g = torch.Generator().manual_seed(B * 100 + T * 10 + S)
    D, Dv = 8, 6
    q, k, v = _rand(g, B, H, T, D), _rand(g, B, G, S, D), _rand(g, B, G, S, Dv)
    kvalid = None
    if masked:
        kvalid = torch.ones(B, S, dtype=torch.bool)
        kvalid[-1, : S // 2] = False
    o, lse = oa.attention(q, k, v, 0.37, kvalid, causal, dtype=torch.float64)
    rep = H // G
    for b in range(B):
        for h in range(H):
            allowed = [[(not causal or j <= i + S - T) and (kvalid is None or bool(kvalid[b, j])) for j in range(S)]
                       for i in range(T)]
            ob, lb = oa.brute_force_attention(q[b, h], k[b, h // rep], v[b, h // rep], 0.37, allowed)
            assert torch.allclose(o[b, h], ob, atol=1e-12)
            fin = torch.isfinite(lb)
            assert torch.equal(fin, torch.isfinite(lse[b, h]))
            assert torch.allclose(lse[b, h][fin], lb[fin], atol=1e-12)


def test_empty_rows_give_zero_and_neg_inf():
    g = torch.Generator().manual_seed(1)
    q, k, v = _rand(g, 1, 2, 3, 4), _rand(g, 1, 1, 5, 4), _rand(g, 1, 1, 5, 4)
    kvalid = torch.zeros(1, 5, dtype=torch.bool)
    o, lse = oa.attention(q, k, v, 0.5, kvalid, causal=False)
    assert torch.equal(o, torch.zeros_like(o)) and torch.isneginf(lse).all()


def test_lse_is_logsumexp_of_scaled_scores():
    g = torch.Generator().manual_seed(2)
    q, k, v = _rand(g, 2, 4, 6, 16), _rand(g, 2, 2, 11, 16), _rand(g, 2, 2, 11, 16)
    o, lse = oa.attention(q, k, v, 16 ** -0.5, causal=False, dtype=torch.float64)
    s = torch.einsum("bhtd,bhsd->bhts", q.double(), k.double().repeat_interleave(2, 1)) * 16 ** -0.5
    assert torch.allclose(lse, torch.logsumexp(s, -1), atol=1e-12)
    assert torch.allclose(o, torch.softmax(s, -1) @ v.double().repeat_interleave(2, 1), atol=1e-12)


def _one_softmax_split(q, k, v, Kp, Vp, pm, scale):
    """One softmax per query over [prefix keys ; own keys] with the split's mask, float64 brute force."""
    n, Hq, t, D = q.shape
    Hkv, T = Kp.shape[0], Kp.shape[1]
    rep = Hq // Hkv
    out = torch.zeros(n, Hq, t, Vp.shape[-1], dtype=torch.float64)
    lse = torch.zeros(n, Hq, t, dtype=torch.float64)
    for r in range(n):
        for h in range(Hq):
            kk = torch.cat([Kp[h // rep], k[r, h // rep]], 0)
            vv = torch.cat([Vp[h // rep], v[r, h // rep]], 0)
            allowed = [[(j < T and (pm is None or bool(pm[j]))) or (j >= T and j - T <= i) for j in range(T + t)]
                       for i in range(t)]
            out[r, h], lse[r, h] = oa.brute_force_attention(q[r, h], kk, vv, scale, allowed)
    return out, lse


@pytest.mark.parametrize("pm_kind", ["none", "holes", "all_masked"])
def test_split_merge_equals_one_softmax(pm_kind):
    g = torch.Generator().manual_seed(4)
    n, Hq, Hkv, t, T, D = 3, 4, 2, 4, 9, 8
    q, k, v = _rand(g, n, Hq, t, D), _rand(g, n, Hkv, t, D), _rand(g, n, Hkv, t, D)
    Kp, Vp = _rand(g, Hkv, T, D), _rand(g, Hkv, T, D)
    pm = None
    if pm_kind == "holes":
        pm = torch.ones(T, dtype=torch.bool)
        pm[[0, 1, 5]] = False
    elif pm_kind == "all_masked":
        pm = torch.zeros(T, dtype=torch.bool)
    out, lse = oa.split_attention(q, k, v, Kp, Vp, pm, 0.3, dtype=torch.float64)
    ref, ref_lse = _one_softmax_split(q, k, v, Kp, Vp, pm, 0.3)
    assert torch.allclose(out, ref, atol=1e-12) and torch.allclose(lse, ref_lse, atol=1e-12)


def test_split_rows_are_permutation_equivariant():
    g = torch.Generator().manual_seed(6)
    n, Hq, Hkv, t, T, D = 6, 4, 1, 3, 10, 8
    q, k, v = _rand(g, n, Hq, t, D), _rand(g, n, Hkv, t, D), _rand(g, n, Hkv, t, D)
    Kp, Vp = _rand(g, Hkv, T, D), _rand(g, Hkv, T, D)
    perm = torch.randperm(n, generator=g)
    out, _ = oa.split_attention(q, k, v, Kp, Vp, None, 0.3)
    out_p, _ = oa.split_attention(q[perm], k[perm], v[perm], Kp, Vp, None, 0.3)
    assert (out_p - out[perm]).abs().max().item() <= 1e-6


def test_branched_int8_rows_read_their_state():
    """row_state routes each row to its state: equal to running split_attention per state on dequantized K/V."""
    g = torch.Generator().manual_seed(7)
    Ns, R, Hq, Hkv, t, T, D = 2, 5, 4, 2, 3, 6, 8
    kq = torch.randint(-127, 128, (Ns, Hkv, T, D), generator=g, dtype=torch.int8)
    vq = torch.randint(-127, 128, (Ns, Hkv, T, D), generator=g, dtype=torch.int8)
    ks, vs = torch.rand(Ns, Hkv, T, generator=g) * 0.02, torch.rand(Ns, Hkv, T, generator=g) * 0.02
    q, k, v = _rand(g, R, Hq, t, D), _rand(g, R, Hkv, t, D), _rand(g, R, Hkv, t, D)
    rs = torch.tensor([1, 0, 1, 1, 0])
    out, lse = oa.branched_attention_int8(q, k, v, kq, ks, vq, vs, 0.3, row_state=rs, dequant="fp32")
    outb, _ = oa.branched_attention_int8(q, k, v, kq, ks, vq, vs, 0.3, row_state=rs)  # default: bf16 materialize
    for r in range(R):
        s = int(rs[r])
        Kb = (kq[s].to(torch.bfloat16) * ks[s][..., None].to(torch.bfloat16)).float()
        Vb = (vq[s].to(torch.bfloat16) * vs[s][..., None].to(torch.bfloat16)).float()
        ob, _ = oa.split_attention(q[r:r + 1], k[r:r + 1], v[r:r + 1], Kb, Vb, None, 0.3)
        assert torch.allclose(outb[r], ob[0], atol=1e-6)
        Kp = kq[s].float() * ks[s][..., None]
        Vp = vq[s].float() * vs[s][..., None]
        o1, l1 = oa.split_attention(q[r:r + 1], k[r:r + 1], v[r:r + 1], Kp, Vp, None, 0.3)
        assert torch.allclose(out[r], o1[0], atol=1e-6) and torch.allclose(lse[r], l1[0], atol=1e-6)


def test_bf16_dequant_is_the_reference_materialize():
    g = torch.Generator().manual_seed(8)
    kq = torch.randint(-127, 128, (2, 5, 8), generator=g, dtype=torch.int8)
    ks = torch.rand(2, 5, generator=g) * 0.03
    got = oa.dequant_state(kq, ks, "bf16")
    exp = (kq.to(torch.bfloat16) * ks[..., None].to(torch.bfloat16)).float()
    assert torch.equal(got, exp)
    assert torch.equal(oa.dequant_state(kq, ks, "fp32"), kq.float() * ks[..., None])


def test_two_level_attention_matches_brute_force():
    """The question-cache attention (two_level_attention) against scalar float64 softmax loops: every query of a row
    of question g sees all keys of its state, the unmasked keys of question g, and its own row's keys 0..i; GQA
    head h reads KV head h // (Hq / Hkv). Pads of a question are excluded; rows of two questions on one state."""
    g = torch.Generator().manual_seed(17)
    Ns, Hq, Hkv, T, T2, t, D = 2, 4, 2, 5, 4, 3, 8
    kq = torch.randint(-127, 128, (Ns, Hkv, T, D), generator=g, dtype=torch.int8)
    vq = torch.randint(-127, 128, (Ns, Hkv, T, D), generator=g, dtype=torch.int8)
    ks, vs = torch.rand(Ns, Hkv, T, generator=g) * 0.02, torch.rand(Ns, Hkv, T, generator=g) * 0.02
    group_state = [1, 1, 0]
    Kq2, Vq2 = _rand(g, 3, Hkv, T2, D), _rand(g, 3, Hkv, T2, D)
    qmask = torch.tensor([[1, 1, 1, 0], [1, 1, 1, 1], [1, 0, 0, 0]], dtype=torch.bool)
    row_group = torch.tensor([0, 0, 1, 2, 2])
    R = len(row_group)
    q, k, v = _rand(g, R, Hq, t, D), _rand(g, R, Hkv, t, D), _rand(g, R, Hkv, t, D)
    out, lse = oa.two_level_attention(q, k, v, kq, ks, vq, vs, Kq2, Vq2, qmask, 0.4, row_group, group_state,
                                      dequant="fp32", dtype=torch.float64)
    for r in range(R):
        gi = int(row_group[r])
        s = group_state[gi]
        for h in range(Hq):
            kv = h // (Hq // Hkv)
            Ks = kq[s, kv].double() * ks[s, kv][:, None].double()
            Vs = vq[s, kv].double() * vs[s, kv][:, None].double()
            keep = qmask[gi].nonzero().squeeze(1)
            K = torch.cat([Ks, Kq2[gi, kv][keep].double(), k[r, kv].double()])
            V = torch.cat([Vs, Vq2[gi, kv][keep].double(), v[r, kv].double()])
            n_pre = T + len(keep)
            allowed = [[j < n_pre or j - n_pre <= i for j in range(len(K))] for i in range(t)]
            o_bf, l_bf = oa.brute_force_attention(q[r, h], K, V, 0.4, allowed)
            assert torch.allclose(out[r, h], o_bf, atol=1e-9), (r, h)
            assert torch.allclose(lse[r, h], l_bf, atol=1e-9), (r, h)


# ---- wide_attention_blocked (the reference kernel's arithmetic, step by step)

def test_wide_blocked_pinned_by_exact_attention():
    """The blocked restatement differs from exact attention only by p's bf16 rounding: its LSE (a sum of unrounded
    p) matches the exact LSE to fp32 accuracy, and its output is within the bf16 rounding of p. A dropped rescale,
    a wrong causal offset or a missed mask moves either far beyond these bounds."""
    g = torch.Generator().manual_seed(0)
    B, H, G, T, S, DK, DV = 2, 4, 2, 37, 150, 40, 24
    q = torch.randn(B, H, T, DK, generator=g).to(torch.bfloat16)
    k = torch.randn(B, G, S, DK, generator=g).to(torch.bfloat16)
    v = torch.randn(B, G, S, DV, generator=g).to(torch.bfloat16)
    kv = torch.ones(B, S, dtype=torch.bool)
    kv[1, :50] = False
    for causal in (True, False):
        ob, lb, bound = oa.wide_attention_blocked(q, k, v, DK ** -0.5, kv, causal=causal, block=64, with_bound=True)
        oe, le = oa.attention(q, k, v, DK ** -0.5, kv, causal=causal)
        # rounding p to bf16 moves it by at most half an ulp, i.e. half the one-ulp flip bound
        assert ((ob - oe).abs() <= bound / 2 + 1e-6).all()
        fin = torch.isfinite(le)
        assert torch.equal(torch.isfinite(lb), fin)
        assert (lb[fin] - le[fin]).abs().max().item() < 1e-5
        assert ((ob - oe).norm() / oe.norm()).item() < 2e-3
        assert (ob - oe).abs().max().item() < 2e-2


def test_wide_blocked_matches_brute_force_on_tiny_case():
    g = torch.Generator().manual_seed(1)
    T, S, D = 3, 7, 8
    q = torch.randn(1, 1, T, D, generator=g).to(torch.bfloat16)
    k = torch.randn(1, 1, S, D, generator=g).to(torch.bfloat16)
    v = torch.randn(1, 1, S, D, generator=g).to(torch.bfloat16)
    kv = torch.tensor([[True, False, True, True, True, True, False]])
    allowed = [[kv[0, j].item() and j <= i + S - T for j in range(S)] for i in range(T)]
    ref, lref = oa.brute_force_attention(q[0, 0], k[0, 0], v[0, 0], D ** -0.5, allowed)
    ob, lb = oa.wide_attention_blocked(q, k, v, D ** -0.5, kv, causal=True, block=2)
    assert (lb[0, 0].double() - lref).abs().max().item() < 1e-5
    assert (ob[0, 0].double() - ref).abs().max().item() < 1e-2 * ref.abs().max().item()


def test_wide_blocked_empty_rows():
    q = torch.randn(1, 2, 4, 8).to(torch.bfloat16)
    k = torch.randn(1, 1, 5, 8).to(torch.bfloat16)
    v = torch.randn(1, 1, 5, 8).to(torch.bfloat16)
    kv = torch.zeros(1, 5, dtype=torch.bool)
    ob, lb = oa.wide_attention_blocked(q, k, v, 0.3, kv, causal=False)
    assert torch.count_nonzero(ob).item() == 0 and torch.isneginf(lb).all()


def test_reference_gpu_arithmetic_composes_the_blocked_kernel():
    """Inside oa.reference_gpu_arithmetic(), split_attention is the reference's CUDA composition (prefix_attn.py:
    50-57): the blocked flash kernel on the prefix (non-causal, key mask) and on the row's own keys (causal), merged
    by LSE; it stays within the blocked kernel's bf16-P flip bound of the exact fp32 result; and the CPU arithmetic
    is back afterwards."""
    g = torch.Generator().manual_seed(21)
    n, Hq, Hkv, t, D, T = 3, 8, 2, 5, 64, 150
    q = torch.randn(n, Hq, t, D, generator=g).bfloat16()
    k = torch.randn(n, Hkv, t, D, generator=g).bfloat16()
    v = torch.randn(n, Hkv, t, D, generator=g).bfloat16()
    Kp = torch.randn(Hkv, T, D, generator=g).bfloat16().float()
    Vp = torch.randn(Hkv, T, D, generator=g).bfloat16().float()
    pm = torch.rand(T, generator=g) > 0.2
    exact, lse_exact = oa.split_attention(q, k, v, Kp, Vp, pm, 0.125)
    with oa.reference_gpu_arithmetic():
        got, lse = oa.split_attention(q, k, v, Kp, Vp, pm, 0.125)
    assert oa.attention.__name__ == "attention"
    qs = q.transpose(0, 1).reshape(1, Hq, n * t, D)
    o_p, l_p, b_p = oa.wide_attention_blocked(qs, Kp[None], Vp[None], 0.125, pm[None], causal=False, with_bound=True)
    o_p, l_p = o_p.reshape(Hq, n, t, D).transpose(0, 1), l_p.reshape(Hq, n, t).transpose(0, 1)
    o_o, l_o, b_o = oa.wide_attention_blocked(q, k, v, 0.125, None, causal=True, with_bound=True)
    want, lse_want = oa.lse_merge(o_p, l_p, o_o, l_o)
    assert torch.equal(got, want) and torch.equal(lse, lse_want)
    bound = b_p.reshape(Hq, n, t, D).transpose(0, 1) + b_o
    assert ((got - exact).abs() <= bound + 1e-5).all()
    assert (lse - lse_exact).abs().max().item() <= 1e-5
    assert (got - exact).abs().max().item() > 0  # the bf16 rounding of P is there
