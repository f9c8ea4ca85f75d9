"""Pins the Gated DeltaNet oracle (oracle/gdn.py) on the CPU: against transformers' own Qwen3.5 functions (the
third-party code the reference runs these layers through; transformers 5.15.0 here, the reference requires >=5.2),
against closed forms that hold whatever the implementation (no write: pure decay; continuation of a sequence equals
the whole sequence), and against decimal arithmetic where the oracle claims correct rounding."""
import decimal

import pytest
import torch

from oracle import gdn as og

mq = pytest.importorskip("transformers.models.qwen3_5.modeling_qwen3_5")


def _bf(g, *shape, scale=1.0):
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16)


def test_conv_silu_matches_causal_conv1d_fresh_and_continued():
    g = torch.Generator().manual_seed(0)
    S, L, C = 3, 29, 40
    x, w = _bf(g, S, L, C), _bf(g, C, 4, scale=0.3)
    state = _bf(g, S, 3, C)
    y, new = og.conv_silu(x, w, None)
    ref = mq.causal_conv1d_fn(x.transpose(1, 2), w, None, activation="silu").transpose(1, 2)
    assert torch.equal(y, ref)
    assert torch.equal(new, x[:, -3:])
    cs = state.transpose(1, 2).contiguous().clone()
    y2, new2 = og.conv_silu(x, w, state)
    ref2 = mq.causal_conv1d_update(x.transpose(1, 2).contiguous(), cs, w, None, activation="silu").transpose(1, 2)
    assert torch.equal(y2, ref2)
    assert torch.equal(new2, cs.transpose(1, 2))          # the reference's updated conv state
    # a 1- and a 2-token continuation keep the right tail of the previous state
    for L2 in (1, 2):
        _, n = og.conv_silu(x[:, :L2], w, state)
        assert torch.equal(n, torch.cat([state, x[:, :L2]], 1)[:, -3:])


def test_gates_match_the_reference_formula():
    g = torch.Generator().manual_seed(1)
    a, b = _bf(g, 50, 32, scale=3.0), _bf(g, 50, 32, scale=3.0)
    a[0, :4] = torch.tensor([25.0, -30.0, 19.875, 20.125])   # both sides of softplus' threshold
    A_log = torch.log(torch.rand(32, generator=g) * 15.5 + 0.5).to(torch.bfloat16)
    dt = (1 + 0.1 * torch.randn(32, generator=g)).to(torch.bfloat16)
    gg, beta = og.gates(a, b, A_log, dt)
    ref = -A_log.float().exp() * torch.nn.functional.softplus(a.float() + dt)
    assert ((gg - ref).abs() <= 2 * ref.abs() * 2.0 ** -23).all()       # within torch's fp32 exp / log1p ulps
    assert torch.equal(beta.to(torch.bfloat16), b.sigmoid())


def test_l2norm_bf16_is_the_reference_arithmetic_with_a_correctly_rounded_rsqrt():
    """Squares, sum, + eps and the product as torch's bf16 ops give them; the rsqrt correctly rounded (torch's CPU
    bf16 rsqrt is an approximation: where the two differ, the oracle's is the nearest bf16 to the exact value)."""
    g = torch.Generator().manual_seed(2)
    x = _bf(g, 4000, 16)
    got = og.l2norm_bf16(x)
    ref = mq.l2norm(x, dim=-1, eps=1e-6)
    diff = (got != ref).any(-1)
    assert diff.float().mean().item() < 0.01
    den = ((x.float() * x.float()).to(torch.bfloat16).double().sum(-1).float().to(torch.bfloat16).float()
           + torch.tensor(1e-6)).to(torch.bfloat16)
    decimal.getcontext().prec = 30
    for i in diff.nonzero().squeeze(1).tolist()[:40]:
        exact = 1 / decimal.Decimal(float(den[i])).sqrt()
        want = torch.tensor(float(exact)).to(torch.bfloat16)
        inv = (got[i].float() / x[i].float())[x[i] != 0]
        # every element's product used the same inv: recover it from the element with the largest |x|
        j = x[i].float().abs().argmax()
        assert torch.equal((x[i, j].float() * want.float()).to(torch.bfloat16), got[i, j]), (i, inv)


def test_recurrence_matches_transformers_recurrent_and_chunked():
    g = torch.Generator().manual_seed(3)
    S, L, H, dk, dv = 2, 70, 4, 32, 16
    q = og.l2norm_bf16(_bf(g, S, L, H, dk))
    k = og.l2norm_bf16(_bf(g, S, L, H, dk))
    v = _bf(g, S, L, H, dv)
    a, b = _bf(g, S, L, H), _bf(g, S, L, H)
    A_log = torch.log(torch.rand(H, generator=g) * 15.5 + 0.5).to(torch.bfloat16)
    dt = (1 + 0.1 * torch.randn(H, generator=g)).to(torch.bfloat16)
    gg, beta = og.gates(a, b, A_log, dt)
    init = torch.randn(S, H, dk, dv, generator=g)
    o, st = og.recurrence(q, k, v, gg, beta, init, torch.float64)
    o32, st32 = og.recurrence(q, k, v, gg, beta, init, torch.float32)
    ref_o, ref_st = mq.torch_recurrent_gated_delta_rule(q, k, v, gg, beta.to(torch.bfloat16), init, True)
    chk_o, chk_st = mq.torch_chunk_gated_delta_rule(q, k, v, gg, beta.to(torch.bfloat16), initial_state=init,
                                                    output_final_state=True)
    step = lambda t: t.float().abs() * 2.0 ** -7 + 1e-6
    for other in (ref_o, chk_o, o32):
        assert ((o.float() - other.float()).abs() <= step(o)).all()      # within one bf16 step
    assert torch.allclose(st.float(), ref_st, atol=1e-5) and torch.allclose(st.float(), chk_st, atol=1e-5)
    assert torch.equal(o32, ref_o)                                          # fp32 mode: the reference's own ops


@pytest.mark.parametrize("L,gmul", [(70, 1.0), (64, 30.0), (5, 0.01)])
def test_chunked_form_equals_the_recurrence(L, gmul):
    """The chunked (WY) form the MFMA kernel implements equals the token-by-token recurrence in float64 (state to
    1e-10, outputs bit for bit after the bf16 rounding but for ties), including chunks whose decay empties the state
    within a token (gmul 30) and a partial chunk."""
    g = torch.Generator().manual_seed(7)
    S, H, dk, dv = 2, 3, 16, 8
    q = og.l2norm_bf16(_bf(g, S, L, H, dk))
    k = og.l2norm_bf16(_bf(g, S, L, H, dk))
    v = _bf(g, S, L, H, dv)
    gg = -torch.rand(S, L, H, generator=g) * gmul
    beta = torch.rand(S, L, H, generator=g)
    init = torch.randn(S, H, dk, dv, generator=g)
    o, st = og.recurrence(q, k, v, gg, beta, init, torch.float64)
    oc, stc = og.chunked_recurrence(q, k, v, gg, beta, init, chunk=32)
    assert torch.allclose(stc, st, rtol=1e-10, atol=1e-12)
    assert (oc != o).float().mean().item() < 0.002
    assert ((oc.float() - o.float()).abs() <= o.float().abs() * 2.0 ** -8 + 1e-30).all()


def test_pure_decay_closed_form():
    """beta = 0 (no writes): S_t = exp(sum g) S_0 and o_t = exp(sum_{<=t} g) S_0^T q_t / sqrt(dk)."""
    g = torch.Generator().manual_seed(4)
    S, L, H, dk, dv = 1, 9, 2, 8, 4
    q = og.l2norm_bf16(_bf(g, S, L, H, dk))
    k = og.l2norm_bf16(_bf(g, S, L, H, dk))
    v = _bf(g, S, L, H, dv)
    gg = -torch.rand(S, L, H, generator=g)
    init = torch.randn(S, H, dk, dv, generator=g).double()
    o, st = og.recurrence(q, k, v, gg, torch.zeros(S, L, H), init.float(), torch.float64)
    cum = torch.cumsum(gg.double(), 1)
    assert torch.allclose(st, torch.exp(cum[:, -1])[..., None, None] * init.float().double(), rtol=1e-12)
    qs = (q.float() * torch.tensor(1 / dk ** 0.5)).double()
    want = torch.einsum("slh,shkv,slhk->slhv", torch.exp(cum), init.float().double(), qs)
    assert torch.allclose(o.float(), want.float().to(torch.bfloat16).float())


def test_continuation_equals_the_whole_sequence():
    """The branch-row identity behind a shared prefix state: a sequence run as [prefix] then [row] continuing the
    prefix's conv and recurrent states equals the whole [prefix ; row] run (float64 recurrence)."""
    cfg = og.GDNConfig(hidden=64, n_k_heads=2, n_v_heads=4, dk=16, dv=8)
    g = torch.Generator().manual_seed(5)
    lw = og.make_gdn_weights(cfg, g)
    qlin = og.quantize_gdn(lw)
    P, L = 11, 6
    x = _bf(g, P + L, cfg.hidden)
    whole, _, st_whole = og.gdn_mixer(x, lw, qlin, cfg, 1, P + L)
    pre, conv_s, rec_s = og.gdn_mixer(x[:P], lw, qlin, cfg, 1, P)
    row, _, st_row = og.gdn_mixer(x[P:], lw, qlin, cfg, 1, L, conv_state=conv_s, rec_state=rec_s)
    # the W8A8 projection quantizes per token, so token rows are independent of the split
    assert torch.equal(torch.cat([pre, row]), whole)
    assert torch.allclose(st_row, st_whole)


def test_gated_norm_matches_qwen3_5_rmsnorm_gated():
    g = torch.Generator().manual_seed(6)
    o, z = _bf(g, 300, 4, 64), _bf(g, 300, 4, 64, scale=2.0)
    w = (1 + 0.1 * torch.randn(64, generator=g)).to(torch.bfloat16)
    m = mq.Qwen3_5RMSNormGated(64, eps=1e-6)
    m.weight.data = w.clone()
    m = m.to(torch.bfloat16)
    ref = m(o.reshape(-1, 64), z.reshape(-1, 64)).reshape(o.shape)
    got = og.gated_norm(o, z, w, 1e-6)
    # the reference's fp32 rsqrt and silu are within a few ulps of the correctly rounded values the oracle uses
    d = (got.float() - ref.float()).abs()
    assert (d <= got.float().abs() * 2.0 ** -7 + 1e-30).all() and (got != ref).float().mean().item() < 0.01


def _gdn_stack(n_layers=2, interval=0, **kw):
    from oracle import decoder as od
    base = dict(hidden=64, ffn=96, n_heads=2, n_kv_heads=1, head_dim=32, n_layers=n_layers, vocab=300,
                lin_k_heads=2, lin_v_heads=4, lin_k_dim=16, lin_v_dim=8)
    base.update(kw)
    # interval > n_layers: every layer is a GDN layer
    cfg = od.DecoderConfig(full_attention_interval=interval or n_layers + 1, **base)
    return cfg, od.make_weights(cfg, seed=11), od.make_embedding(cfg, seed=11)


def test_hybrid_layer_types_follow_qwen3_5():
    from oracle import decoder as od
    cfg = od.DecoderConfig(n_layers=32, full_attention_interval=4)
    want = mq.Qwen3_5TextConfig().layer_types                    # transformers' own default stack
    assert ["linear_attention" if cfg.is_gdn(i) else "full_attention" for i in range(32)] == want
    assert not any(od.DecoderConfig(n_layers=8).is_gdn(i) for i in range(8))


def test_gdn_stack_prefill_in_pieces_equals_one_prefill():
    """A GDN-only stack: prefilling S1 tokens, then S2 more continuing the states, gives the same hidden states
    and the same conv / recurrent states as one prefill of S1 + S2 tokens (fp32 recurrence: the same operations in
    the same order, so bit for bit)."""
    from oracle import decoder as od
    cfg, w, emb = _gdn_stack()
    g = torch.Generator().manual_seed(12)
    ids = torch.randint(0, cfg.vocab, (2, 13), generator=g)
    h_all, st_all = od.prefill_forward(ids, w, emb, cfg, gdn_dtype=torch.float32)
    h1, st1 = od.prefill_forward(ids[:, :8], w, emb, cfg, gdn_dtype=torch.float32)
    h2, st2 = od.prefill_forward(ids[:, 8:], w, emb, cfg, state_kv=st1, n0=8, gdn_dtype=torch.float32)
    hw = h_all.reshape(2, 13, -1)
    assert torch.equal(torch.cat([h1.reshape(2, 8, -1), h2.reshape(2, 5, -1)], 1), hw)
    for (c, r), (ca, ra) in zip(st2, st_all):
        assert torch.equal(c, ca) and torch.equal(r, ra)


def test_gdn_stack_option_rows_equal_continuing_prefill():
    """Option rows read their request's state in place: a GDN-only stack's decision forward equals the readout of
    a prefill that continues each request's states with its option row (rows laid out one per state)."""
    from oracle import decoder as od
    cfg, w, emb = _gdn_stack()
    g = torch.Generator().manual_seed(13)
    B, n_opt, t, T = 2, 3, 5, 9
    _, st = od.prefill_forward(torch.randint(0, cfg.vocab, (B, T), generator=g), w, emb, cfg)
    ids = torch.randint(0, cfg.vocab, (B, n_opt, t), generator=g)
    lp = od.decision_forward(ids, w, emb, cfg, st, T)
    rep = [(c.repeat_interleave(n_opt, 0), r.repeat_interleave(n_opt, 0)) for c, r in st]
    h, _ = od.prefill_forward(ids.reshape(B * n_opt, t), w, emb, cfg, state_kv=rep, n0=T)
    ref = od.readout(h, w["final_norm"], w["head"], w["none_logit"], cfg, B, n_opt, t)
    assert torch.equal(lp, ref)


def test_hybrid_option_rows_depend_on_their_own_state():
    """In a hybrid stack (GDN, attention) each request's rows see only its own GDN state: perturbing request 1's
    recurrent state moves request 1's probabilities and leaves request 0's bit for bit."""
    from oracle import decoder as od
    cfg, w, emb = _gdn_stack(interval=2)
    assert cfg.is_gdn(0) and not cfg.is_gdn(1)
    g = torch.Generator().manual_seed(14)
    B, n_opt, t, T = 2, 3, 4, 7
    _, st = od.prefill_forward(torch.randint(0, cfg.vocab, (B, T), generator=g), w, emb, cfg)
    ids = torch.randint(0, cfg.vocab, (B, n_opt, t), generator=g)
    lp = od.decision_forward(ids, w, emb, cfg, st, T, temperature=1.0)
    conv, rec = st[0]
    rec2 = rec.clone()
    rec2[1] += torch.randn(rec[1].shape, generator=g)   # (a uniform scale would cancel in the gated norm)
    st2 = [(conv, rec2)] + st[1:]
    lp2 = od.decision_forward(ids, w, emb, cfg, st2, T, temperature=1.0)
    assert torch.equal(lp2[0], lp[0]) and not torch.equal(lp2[1], lp[1])


def test_padded_continuation_equals_one_unpadded_pass_per_sequence():
    """The reference's claim for Backbone.padded_continuation (backbone.py:257-263: features equal one unpadded pass
    per row): right-padded sequences continuing their states, with a and b set to -inf at the pads, give at every
    real position the outputs of each sequence run alone at its real length, and leave exactly that pass's conv and
    recurrent state (bit for bit: at a pad e^g = 1 and beta = 0, so the state is carried unchanged); a sequence with no
    real token leaves its state as it was."""
    from oracle import decoder as od
    cfg = og.GDNConfig(hidden=128, n_k_heads=2, n_v_heads=4, dk=128, dv=32)
    g = torch.Generator().manual_seed(21)
    lw = og.make_gdn_weights(cfg, g)
    qlin = og.quantize_gdn(lw)
    S, L = 4, 11
    lens = [11, 6, 2, 0]
    x = _bf(g, S * L, cfg.hidden)
    conv0 = _bf(g, S, 3, cfg.conv_dim)
    rec0 = torch.randn(S, cfg.n_v_heads, cfg.dk, cfg.dv, generator=g) * 0.05
    out, conv, rec = og.gdn_mixer(x, lw, qlin, cfg, S, L, conv0, rec0, seq_len=lens)
    out = out.reshape(S, L, -1)
    for s_, n in enumerate(lens):
        if n == 0:
            assert torch.equal(conv[s_], conv0[s_]) and torch.equal(rec[s_], rec0[s_])
            continue
        o1, c1, r1 = og.gdn_mixer(x.reshape(S, L, -1)[s_, :n], lw, qlin, cfg, 1, n, conv0[s_:s_ + 1],
                                  rec0[s_:s_ + 1])
        assert torch.equal(out[s_, :n].view(torch.int16), o1.view(torch.int16)), s_
        assert torch.equal(conv[s_], c1[0]) and torch.equal(rec[s_], r1[0]), s_
    # without the masking the pads would move the states
    _, conv_np, rec_np = og.gdn_mixer(x, lw, qlin, cfg, S, L, conv0, rec0)
    assert not torch.equal(rec_np[1], rec[1]) and not torch.equal(conv_np[1], conv[1])


def test_hybrid_question_cache_equals_rows_that_carry_the_question():
    """The question cache on the hybrid stack (a batched, right-padded question pass, v3.py:446-497): question g's
    real tokens continue every layer's state (GDN: the padded continuation above; attention: the captured K/V, pads
    masked), and option rows over that cache give the log-probabilities of rows that carry [question g's real tokens
    ; option] over state g, pooled over the option tokens (float64 attention and recurrence)."""
    from helpers import hybrid_states
    from oracle import decoder as od
    cfg = od.DecoderConfig(hidden=256, ffn=512, n_heads=4, n_kv_heads=2, head_dim=64, n_layers=4, vocab=500,
                           full_attention_interval=2, lin_k_heads=2, lin_v_heads=4, gated=True, rot_dim=16,
                           norm_offset=True)
    w = od.make_weights(cfg, seed=3)
    w["temperature"] = 24.0
    emb = od.make_embedding(cfg, seed=3)
    T = 40
    states = hybrid_states(cfg, 2, T)
    g = torch.Generator().manual_seed(22)
    qlen, Lq, n_opt, t = [9, 5], 9, 3, 4
    ids_q = torch.randint(0, 500, (2, Lq), generator=g)
    ids_o = torch.randint(0, 500, (2, n_opt, t), generator=g)
    q_kv = od.question_forward(ids_q, w, emb, cfg, states, T, [0, 1], attn_dtype=torch.float64, qlen=qlen)
    lp_qc = od.qcache_decision_forward(ids_o, w, emb, cfg, states, T, q_kv, qlen, [0, 1], attn_dtype=torch.float64)
    for q in range(2):
        # state q alone: ((kq, ks), (vq, vs)) of an attention layer, (conv, rec) of a GDN layer
        st_q = [tuple(tuple(x[q:q + 1] for x in e) for e in st) if isinstance(st[0], tuple) else
                tuple(x[q:q + 1] for x in st) for st in states]
        rows = torch.cat([ids_q[q, :qlen[q]][None, None, :].expand(1, n_opt, qlen[q]), ids_o[q:q + 1]], 2)
        lp_rows = od.decision_forward(rows, w, emb, cfg, st_q, T, attn_dtype=torch.float64, pool_last=t)
        assert (lp_qc[q] - lp_rows[0]).abs().max().item() <= 1e-6, q
