"""GPU parity of the Gated DeltaNet kernels against the oracle (oracle/gdn.py): od_gdn_prep and od_gdn_norm_quant
bit-exact (every open-order sum is exact on both sides), od_gdn_recurrence against the float64 recurrence within
one bf16 step per output (plus 2e-3 relative in norm) and its fp32 final state within 1e-5 relative."""
import pytest
import torch

from oracle import gdn as og
from oracle import quant as oq

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _bf(g, *shape, scale=1.0):
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16)


def _proj(g, M, n_k, n_v, dk, dv, pad=8):
    C = 2 * n_k * dk + n_v * dv
    P = C + n_v * dv + 2 * n_v
    pad += (-(P + pad)) % 8  # rows of 16-byte multiples, as the kernel requires
    p = _bf(g, M, P + pad)
    p[:, C + n_v * dv:] = _bf(g, M, 2 * n_v + pad, scale=3.0)  # b and a over a wider range
    return p


@pytest.mark.parametrize("S,L,n_k,n_v,with_state", [(2, 5, 2, 4, False), (3, 33, 2, 4, True), (4, 1, 2, 4, True),
                                                    (2, 2, 1, 2, True), (1, 70, 16, 32, False), (2, 24, 16, 32, True)])
def test_gdn_prep_bit_exact(gpu_lib, S, L, n_k, n_v, with_state):
    from opendecider_amd import kernels
    dk = dv = 128
    g = torch.Generator().manual_seed(S * 100 + L + n_k)
    C = 2 * n_k * dk + n_v * dv
    proj = _proj(g, S * L, n_k, n_v, dk, dv)
    conv_w = _bf(g, C, 4, scale=0.3)
    A_log = torch.log(torch.rand(n_v, generator=g) * 15.5 + 0.5).to(torch.bfloat16)
    dt = (1 + 0.1 * torch.randn(n_v, generator=g)).to(torch.bfloat16)
    n_states = 3
    conv_in = _bf(g, n_states, 3, C) if with_state else None
    seq = torch.randint(0, n_states, (S,), generator=g, dtype=torch.int32) if with_state else None
    if with_state and S > 1:
        seq[-1] = 7  # outside [0, n_states): reads zeros
    print(f"gdn_prep S={S} L={L} n_k={n_k} n_v={n_v} state={with_state}", flush=True)
    qk, v, gg, beta, co = kernels.gdn_prep(proj.to(DEV), conv_w.to(DEV), A_log.to(DEV), dt.to(DEV), S, L, n_k, n_v,
                                           dk, dv, None if conv_in is None else conv_in.to(DEV),
                                           None if seq is None else seq.to(DEV), conv_out=True)
    qkv_r, z_r, b_r, a_r = og.split_proj(proj[:, :C + n_v * dv + 2 * n_v], og.GDNConfig(n_k_heads=n_k, n_v_heads=n_v))
    cs = None
    if with_state:
        cs = torch.zeros(S, 3, C, dtype=torch.bfloat16)
        for i in range(S):
            if 0 <= int(seq[i]) < n_states:
                cs[i] = conv_in[int(seq[i])]
    y, new = og.conv_silu(qkv_r.reshape(S, L, C), conv_w, cs)
    y = y.reshape(S * L, C)
    kd = n_k * dk
    q_r = og.l2norm_bf16(y[:, :kd].reshape(-1, n_k, dk)).reshape(-1, kd)
    k_r = og.l2norm_bf16(y[:, kd:2 * kd].reshape(-1, n_k, dk)).reshape(-1, kd)
    g_r, beta_r = og.gates(a_r, b_r, A_log, dt)
    assert torch.equal(qk.cpu(), torch.cat([q_r, k_r], 1))
    assert torch.equal(v.cpu(), y[:, 2 * kd:])
    assert torch.equal(gg.cpu(), g_r) and torch.equal(beta.cpu(), beta_r)
    assert torch.equal(co.cpu(), new)


@pytest.mark.parametrize("S,L,n_k,n_v,lens", [(4, 11, 2, 4, [11, 6, 2, 0]), (3, 40, 16, 32, [40, 17, 1]),
                                               (2, 9, 2, 4, [3, 8])])
def test_gdn_prep_padded_sequences_bit_exact(gpu_lib, S, L, n_k, n_v, lens):
    """od_gdn_prep_ex with right-padded sequences (the reference's padded continuation): gates beta = 0, g = -0 at
    every pad (what b = a = -inf give), the conv window ending at each sequence's last real token (the state's own
    window for an empty one), everything at real positions as without padding; bit-exact against the oracle."""
    from opendecider_amd import kernels
    dk = dv = 128
    g = torch.Generator().manual_seed(S * 31 + L)
    C = 2 * n_k * dk + n_v * dv
    proj = _proj(g, S * L, n_k, n_v, dk, dv)
    conv_w = _bf(g, C, 4, scale=0.3)
    A_log = torch.log(torch.rand(n_v, generator=g) * 15.5 + 0.5).to(torch.bfloat16)
    dt = (1 + 0.1 * torch.randn(n_v, generator=g)).to(torch.bfloat16)
    conv_in = _bf(g, S, 3, C)
    seq_len = torch.tensor(lens, dtype=torch.int32)
    print(f"gdn_prep padded S={S} L={L} lens={lens}", flush=True)
    qk, v, gg, beta, co = kernels.gdn_prep(proj.to(DEV), conv_w.to(DEV), A_log.to(DEV), dt.to(DEV), S, L, n_k, n_v,
                                           dk, dv, conv_in.to(DEV), conv_out=True, seq_len=seq_len.to(DEV))
    cfg = og.GDNConfig(n_k_heads=n_k, n_v_heads=n_v)
    qkv_r, z_r, b_r, a_r = og.split_proj(proj[:, :C + n_v * dv + 2 * n_v], cfg)
    keep = (torch.arange(L)[None, :] < seq_len[:, None].long()).reshape(-1, 1)
    ninf = torch.full((), -float("inf"), dtype=torch.bfloat16)
    g_r, beta_r = og.gates(torch.where(keep, a_r, ninf), torch.where(keep, b_r, ninf), A_log, dt)
    y, new = og.conv_silu(qkv_r.reshape(S, L, C), conv_w, conv_in, lens)
    y = y.reshape(S * L, C)
    kd = n_k * dk
    real = keep[:, 0]
    q_r = og.l2norm_bf16(y[:, :kd].reshape(-1, n_k, dk)).reshape(-1, kd)
    k_r = og.l2norm_bf16(y[:, kd:2 * kd].reshape(-1, n_k, dk)).reshape(-1, kd)
    assert torch.equal(qk.cpu()[real], torch.cat([q_r, k_r], 1)[real])
    assert torch.equal(v.cpu()[real], y[real, 2 * kd:])
    assert torch.equal(gg.cpu().view(torch.int32), g_r.view(torch.int32))
    assert torch.equal(beta.cpu(), beta_r)
    assert (beta.cpu()[~real] == 0).all() and (gg.cpu()[~real] == 0).all()
    assert torch.equal(co.cpu(), new)


@pytest.mark.parametrize("chunked", [True, False])
def test_gdn_padded_continuation_keeps_each_state(gpu_lib, chunked):
    """The recurrence over right-padded sequences (gates from od_gdn_prep_ex) leaves each sequence's final state equal
    to that of its unpadded pass at its real length, and a sequence with no real token its initial state bit for
    bit."""
    from opendecider_amd import kernels
    dk = dv = 128
    n_k, n_v, S, L = 2, 4, 3, 37
    lens = [37, 12, 0]
    g = torch.Generator().manual_seed(77)
    C = 2 * n_k * dk + n_v * dv
    proj = _proj(g, S * L, n_k, n_v, dk, dv).to(DEV)
    conv_w = _bf(g, C, 4, scale=0.3).to(DEV)
    A_log = torch.log(torch.rand(n_v, generator=g) * 15.5 + 0.5).to(torch.bfloat16).to(DEV)
    dt = (1 + 0.1 * torch.randn(n_v, generator=g)).to(torch.bfloat16).to(DEV)
    conv_in = _bf(g, S, 3, C).to(DEV)
    init = (torch.randn(S, n_v, dk, dv, generator=g) * 0.05).to(DEV)
    print(f"gdn padded continuation chunked={chunked}", flush=True)
    qk, v, gg, beta, _ = kernels.gdn_prep(proj, conv_w, A_log, dt, S, L, n_k, n_v, dk, dv, conv_in,
                                          seq_len=torch.tensor(lens, dtype=torch.int32, device=DEV))
    _, fin = kernels.gdn_recurrence(qk, v, gg, beta, S, L, n_k, n_v, dk, dv, init=init, final=True, chunked=chunked)
    assert torch.equal(fin[2], init[2])
    for s_, n in enumerate(lens[:2]):
        rows = slice(s_ * L, s_ * L + n)
        qk1, v1, g1, b1, _ = kernels.gdn_prep(proj[rows].contiguous(), conv_w, A_log, dt, 1, n, n_k, n_v, dk, dv,
                                              conv_in[s_:s_ + 1])
        _, fin1 = kernels.gdn_recurrence(qk1, v1, g1, b1, 1, n, n_k, n_v, dk, dv, init=init[s_:s_ + 1].contiguous(),
                                         final=True, chunked=chunked)
        d = (fin[s_] - fin1[0]).abs().max().item()
        assert d <= 1e-5 * fin1.abs().max().item() + 1e-7, (s_, d)


def _rec_inputs(g, S, L, n_k, n_v, dk=128, dv=128):
    M = S * L
    q = og.l2norm_bf16(_bf(g, M, n_k, dk))
    k = og.l2norm_bf16(_bf(g, M, n_k, dk))
    v = _bf(g, M, n_v, dv)
    a, b = _bf(g, M, n_v, scale=2.0), _bf(g, M, n_v, scale=2.0)
    A_log = torch.log(torch.rand(n_v, generator=g) * 15.5 + 0.5).to(torch.bfloat16)
    dt = (1 + 0.1 * torch.randn(n_v, generator=g)).to(torch.bfloat16)
    gg, beta = og.gates(a, b, A_log, dt)
    return q, k, v, gg, beta


@pytest.mark.parametrize("chunked", [True, False])
@pytest.mark.parametrize("S,L,n_k,n_v,init,gmul", [(2, 1, 2, 4, False, 1), (2, 16, 2, 4, True, 1),
                                                   (3, 70, 2, 4, True, 1), (1, 33, 16, 32, False, 1),
                                                   (4, 24, 16, 32, True, 1), (2, 300, 2, 4, True, 1),
                                                   (2, 64, 2, 4, True, 40), (2, 96, 2, 4, True, 0.01)])
def test_gdn_recurrence_matches_float64(gpu_lib, S, L, n_k, n_v, init, gmul, chunked):
    """Both forms (the chunked one on bf16 MFMA, and token by token) against the float64 recurrence; gmul scales the
    log-decays (x40: most of the state vanishes within a token; x0.01: almost no decay over the sequence)."""
    from opendecider_amd import kernels
    dk = dv = 128
    g = torch.Generator().manual_seed(S * 1000 + L + n_v)
    q, k, v, gg, beta = _rec_inputs(g, S, L, n_k, n_v)
    gg = gg * gmul
    n_states = 3
    st0 = torch.randn(n_states, n_v, dk, dv, generator=g) * 0.5 if init else None
    seq = torch.randint(0, n_states, (S,), generator=g, dtype=torch.int32) if init else None
    print(f"gdn_recurrence S={S} L={L} n_k={n_k} n_v={n_v} init={init} gmul={gmul} chunked={chunked}", flush=True)
    qk = torch.cat([q.reshape(S * L, -1), k.reshape(S * L, -1)], 1)
    o, fs = kernels.gdn_recurrence(qk.to(DEV), v.reshape(S * L, -1).to(DEV), gg.to(DEV), beta.to(DEV), S, L, n_k,
                                   n_v, dk, dv, None if st0 is None else st0.to(DEV),
                                   None if seq is None else seq.to(DEV), final=True, chunked=chunked)
    rep = n_v // n_k
    init_r = None if st0 is None else st0[seq.long()]
    o_r, st_r = og.recurrence(q.repeat_interleave(rep, 1).reshape(S, L, n_v, dk),
                              k.repeat_interleave(rep, 1).reshape(S, L, n_v, dk), v.reshape(S, L, n_v, dv),
                              gg.reshape(S, L, n_v), beta.reshape(S, L, n_v), init_r, torch.float64)
    o_r = o_r.reshape(S * L, n_v * dv).float()
    got = o.cpu().float()
    d = (got - o_r).abs()
    assert (d <= o_r.abs() * 2.0 ** -7 + 1e-6).all(), d.max().item()
    assert (d.norm() / o_r.norm()).item() <= 2e-3
    assert torch.allclose(fs.cpu(), st_r.float(), rtol=1e-5, atol=1e-5 * st_r.abs().max().item())


@pytest.mark.parametrize("chunked", [True, False])
def test_gdn_recurrence_in_place_state_and_continuation(gpu_lib, chunked):
    """Running L1 tokens, then L2 more continuing the written state in place, equals one run over L1 + L2 tokens up
    to rounding: the split moves the chunk boundaries (and the token-by-token form's scalar decay factor is
    multiplied into the state there), so the states agree to 1e-5 and the outputs to one bf16 step."""
    from opendecider_amd import kernels
    S, n_k, n_v, L1, L2 = 2, 2, 4, 45, 50
    g = torch.Generator().manual_seed(5)
    q, k, v, gg, beta = _rec_inputs(g, S, L1 + L2, n_k, n_v)

    def part(lo, hi):
        sel = lambda x: x.reshape(S, L1 + L2, *x.shape[1:])[:, lo:hi].reshape(S * (hi - lo), *x.shape[1:])
        qk = torch.cat([sel(q).reshape(S * (hi - lo), -1), sel(k).reshape(S * (hi - lo), -1)], 1)
        return qk.to(DEV), sel(v).reshape(S * (hi - lo), -1).to(DEV), sel(gg).to(DEV), sel(beta).to(DEV)

    whole, fs_whole = kernels.gdn_recurrence(*part(0, L1 + L2), S, L1 + L2, n_k, n_v, 128, 128, final=True,
                                             chunked=chunked)
    o1, st = kernels.gdn_recurrence(*part(0, L1), S, L1, n_k, n_v, 128, 128, final=True, chunked=chunked)
    o2, st2 = kernels.gdn_recurrence(*part(L1, L1 + L2), S, L2, n_k, n_v, 128, 128, init=st, final=st,
                                     chunked=chunked)
    assert st2.data_ptr() == st.data_ptr()
    both = torch.cat([o1.reshape(S, L1, -1), o2.reshape(S, L2, -1)], 1).reshape(S * (L1 + L2), -1).float()
    whole = whole.float()
    assert ((both - whole).abs() <= whole.abs() * 2.0 ** -7 + 1e-6).all()
    assert (both != whole).float().mean().item() < 0.01
    assert torch.allclose(st2, fs_whole, rtol=1e-5, atol=1e-5 * fs_whole.abs().max().item())


def test_gdn_norm_quant_every_gate_value(gpu_lib):
    """The gate z takes every finite bf16 value (the fast fp32 SiLU product and its float64 fallback both run) under
    random o and weights: bytes and scales equal the oracle's."""
    from opendecider_amd import kernels
    M, n_v, dv = 16, 32, 128
    g = torch.Generator().manual_seed(17)
    bits = torch.arange(65536, dtype=torch.int32).to(torch.int16)
    zv = bits.view(torch.bfloat16)
    zv = zv[torch.isfinite(zv.float())]
    z = torch.cat([zv, zv[: M * n_v * dv - zv.numel()]]).reshape(M, n_v * dv)
    o = _bf(g, M, n_v * dv, scale=0.3)
    w = (1 + 0.1 * torch.randn(dv, generator=g)).to(torch.bfloat16)
    inv = (1.0 / (torch.rand(n_v * dv, generator=g) * 1.5 + 0.5)).to(torch.bfloat16)
    for smooth in (None, inv):
        xq, sx = kernels.gdn_norm_quant(o.to(DEV), z.to(DEV), w.to(DEV), 1e-6, n_v, dv,
                                        None if smooth is None else smooth.to(DEV))
        y = og.gated_norm(o.reshape(M, n_v, dv), z.reshape(M, n_v, dv), w, 1e-6).reshape(M, n_v * dv)
        rq, rs = oq.act_quant(y, smooth)
        assert torch.equal(sx.cpu(), rs) and torch.equal(xq.cpu(), rq)


@pytest.mark.parametrize("M,n_v,smooth", [(5, 4, False), (33, 4, True), (64, 32, True), (3, 2, False),
                                          (512, 32, True)])
def test_gdn_norm_quant_bit_exact(gpu_lib, M, n_v, smooth):
    from opendecider_amd import kernels
    dv = 128
    g = torch.Generator().manual_seed(M + n_v)
    o = _bf(g, M, n_v * dv, scale=0.3)
    if M > 2:
        o[1] = 0                                               # a zero row: r = 1 / sqrt(eps)
    zz = _bf(g, M, n_v * dv + 40, scale=2.0)[:, 24:24 + n_v * dv]   # a strided column slice, as from proj
    w = (1 + 0.1 * torch.randn(dv, generator=g)).to(torch.bfloat16)
    inv = (1.0 / (torch.rand(n_v * dv, generator=g) * 1.5 + 0.5)).to(torch.bfloat16) if smooth else None
    print(f"gdn_norm_quant M={M} n_v={n_v} smooth={smooth}", flush=True)
    zd = zz.to(DEV)
    xq, sx = kernels.gdn_norm_quant(o.to(DEV), zd, w.to(DEV), 1e-6, n_v, dv, None if inv is None else inv.to(DEV))
    y = og.gated_norm(o.reshape(M, n_v, dv), zz.reshape(M, n_v, dv), w, 1e-6).reshape(M, n_v * dv)
    rq, rs = oq.act_quant(y, inv)
    assert torch.equal(sx.cpu(), rs) and torch.equal(xq.cpu(), rq)
