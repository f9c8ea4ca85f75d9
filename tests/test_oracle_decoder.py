"""Pins the decision-forward oracle (oracle/decoder.py) step by step against independent float64 math: RMSNorm's
closed form, RoPE as a complex rotation (norm preservation, relative-position property), SwiGLU, the readout's
normalisation, and option-order invariance of the whole forward."""
import math

import pytest
import torch

from oracle import decoder as od
from oracle import quant as oq


def test_rmsnorm_matches_float64_within_bf16_rounding():
    g = torch.Generator().manual_seed(0)
    x = (torch.randn(6, 64, generator=g) * 3).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(64, generator=g)).to(torch.bfloat16)
    y = od.rmsnorm(x, w, 1e-6).double()
    xd = x.double()
    ref = w.double() * xd / torch.sqrt(xd.pow(2).mean(-1, keepdim=True) + 1e-6)
    assert ((y - ref).abs() <= ref.abs() * 2.0 ** -7 + 1e-12).all()
    # closed form: a constant row normalises to sign * w
    c = torch.full((1, 64), -2.5, dtype=torch.bfloat16)
    assert torch.equal(od.rmsnorm(c, w, 0.0), (-w.float()).to(torch.bfloat16)[None])


def _qwen35_modules():
    return pytest.importorskip("transformers.models.qwen3_5.modeling_qwen3_5")


def test_zero_centred_rmsnorm_matches_transformers_qwen3_5_rmsnorm():
    """The offset convention against transformers' Qwen3_5RMSNorm (the norm of the reference's default backbone):
    with the module's normalisation given the oracle's r, the module's own (1 + w) product and cast give the oracle's
    bits; with its own fp32 mean / rsqrt it lands within one bf16 step on a few elements. The Llama-style product
    with 1 + w folded into the weight (w' * bf16(x * r), two roundings) is shown to differ, so the check can tell
    the conventions apart."""
    mq = _qwen35_modules()
    g = torch.Generator().manual_seed(11)
    K = 256
    x = (torch.randn(64, K, generator=g) * 3).to(torch.bfloat16)
    w = (0.1 * torch.randn(K, generator=g)).to(torch.bfloat16)
    m = mq.Qwen3_5RMSNorm(K, eps=1e-6).to(torch.bfloat16)
    with torch.no_grad():
        m.weight.copy_(w)
    ours = od.rmsnorm(x, w, 1e-6, offset=True)
    own = m(x)
    d = (own.view(torch.int16).int() - ours.view(torch.int16).int()).abs()
    assert d.max().item() <= 1 and (d > 0).float().mean().item() < 0.02
    m._norm = lambda t: t * od.rms_factor(t, m.eps)     # the module's arithmetic around the oracle's r
    assert torch.equal(m(x).view(torch.int16), ours.view(torch.int16))
    folded = od.rmsnorm(x, (1.0 + w.float()).to(torch.bfloat16), 1e-6)
    assert not torch.equal(folded.view(torch.int16), ours.view(torch.int16))


def test_partial_rotary_matches_transformers_qwen3_5():
    """Qwen3.5's partial rotary (64 of 256 dims) against transformers: the oracle's cos/sin tables equal
    Qwen3_5TextRotaryEmbedding's (bf16, halves repeated) and qk_norm_rope equals apply_rotary_pos_emb applied to
    the oracle's zero-centred q/k norms, bit for bit; the 192 unrotated dims keep the normed values."""
    mq = _qwen35_modules()
    cfg = od.DecoderConfig(hidden=1024, n_heads=4, n_kv_heads=2, head_dim=256, rot_dim=64, norm_offset=True)
    tcfg = mq.Qwen3_5TextConfig(head_dim=256, num_attention_heads=4, num_key_value_heads=2, hidden_size=1024,
                                rope_parameters={"rope_type": "default", "rope_theta": cfg.theta,
                                                 "partial_rotary_factor": 0.25})
    pos = torch.tensor([0, 1, 2, 7, 300, 4095, 20000, 32767])
    M = pos.numel()
    cos_t, sin_t = mq.Qwen3_5TextRotaryEmbedding(tcfg)(torch.zeros(1, dtype=torch.bfloat16), pos[None])
    cos, sin = od.rope_tables(cfg, 32768)
    assert cos.shape == (32768, 32)
    assert torch.equal(cos_t[0], cos[pos].repeat(1, 2)) and torch.equal(sin_t[0], sin[pos].repeat(1, 2))
    g = torch.Generator().manual_seed(12)
    qkv = (torch.randn(M, cfg.qkv_out, generator=g) * 2).to(torch.bfloat16)
    qw, kw = ((0.1 * torch.randn(256, generator=g)).to(torch.bfloat16) for _ in range(2))
    out = od.qk_norm_rope(qkv, cfg, qw, kw, cos, sin, pos)
    D = 256
    qn = od.rmsnorm(qkv[:, :4 * D].reshape(M, 4, D), qw, cfg.eps, True)
    kn = od.rmsnorm(qkv[:, 4 * D:6 * D].reshape(M, 2, D), kw, cfg.eps, True)
    qe, ke = mq.apply_rotary_pos_emb(qn.transpose(0, 1)[None], kn.transpose(0, 1)[None], cos_t, sin_t)
    assert torch.equal(out[:, :4 * D].view(torch.int16), qe[0].transpose(0, 1).reshape(M, 4 * D).view(torch.int16))
    assert torch.equal(out[:, 4 * D:6 * D].view(torch.int16),
                       ke[0].transpose(0, 1).reshape(M, 2 * D).view(torch.int16))
    assert torch.equal(out[:, :4 * D].reshape(M, 4, D)[..., 64:], qn[..., 64:])
    assert torch.equal(out[:, 6 * D:], qkv[:, 6 * D:])
    # a full-head rotation (the dense configs' convention) is a different function on these heads
    full = od.qk_norm_rope(qkv, od.DecoderConfig(**{**cfg.__dict__, "rot_dim": 0}), qw, kw,
                           *od.rope_tables(od.DecoderConfig(head_dim=256), 32768), pos)
    assert not torch.equal(full.view(torch.int16), out.view(torch.int16))


def _rope64(x, pos, cfg):
    """Independent float64 RoPE: pairs (x_i, x_{i+D/2}) rotated by pos * theta^(-2i/D) as complex numbers."""
    D = x.shape[-1]
    L = D // 2
    i = torch.arange(L, dtype=torch.float64)
    ang = pos[:, None].double() * cfg.theta ** (-2 * i / D)
    z = torch.complex(x[..., :L].double(), x[..., L:].double()) * torch.exp(1j * ang)[:, None, :]
    return torch.cat([z.real, z.imag], -1)


def test_qk_norm_rope_is_a_rotation_of_the_normed_heads():
    cfg = od.DecoderConfig(hidden=256, n_heads=4, n_kv_heads=2, head_dim=64)
    g = torch.Generator().manual_seed(1)
    M = 10
    qkv = torch.randn(M, cfg.qkv_out, generator=g).to(torch.bfloat16)
    qw, kw = torch.ones(64, dtype=torch.bfloat16), (1 + 0.1 * torch.randn(64, generator=g)).to(torch.bfloat16)
    pos = torch.tensor([0, 1, 2, 5, 77, 1000, 4095, 4096, 20000, 32767])
    cos, sin = od.rope_tables(cfg, 32768)
    out = od.qk_norm_rope(qkv, cfg, qw, kw, cos, sin, pos)
    D = 64
    qn = od.rmsnorm(qkv[:, :4 * D].reshape(M, 4, D), qw, cfg.eps)
    ref = _rope64(qn, pos, cfg)
    got = out[:, :4 * D].reshape(M, 4, D).double()
    assert (got - ref).abs().max().item() < 0.05                      # bf16 tables and products
    # a rotation keeps each pair's norm (within bf16 rounding) and leaves v untouched
    nr = lambda t: (t[..., :32] ** 2 + t[..., 32:] ** 2).sqrt()
    assert ((nr(got) - nr(qn.double())).abs() <= nr(qn.double()) * 0.02 + 1e-3).all()
    assert torch.equal(out[:, 6 * D:], qkv[:, 6 * D:])


def test_rope_scores_depend_on_relative_position_only():
    """q_m . k_n after RoPE equals q_{m+d} . k_{n+d} (float64 restatement of the same rotation)."""
    cfg = od.DecoderConfig(head_dim=128)
    g = torch.Generator().manual_seed(2)
    q, k = torch.randn(1, 1, 128, generator=g), torch.randn(1, 1, 128, generator=g)
    s1 = (_rope64(q, torch.tensor([10]), cfg) * _rope64(k, torch.tensor([3]), cfg)).sum()
    s2 = (_rope64(q, torch.tensor([5010]), cfg) * _rope64(k, torch.tensor([5003]), cfg)).sum()
    assert abs(s1.item() - s2.item()) < 1e-9


def test_swiglu_matches_float64():
    g = torch.Generator().manual_seed(3)
    gu = (torch.randn(5, 2 * 48, generator=g) * 4).to(torch.bfloat16)
    y = od.swiglu(gu, 48).double()
    gd, ud = gu[:, :48].double(), gu[:, 48:].double()
    ref = gd / (1 + torch.exp(-gd)) * ud
    assert ((y - ref).abs() <= ref.abs() * 2.0 ** -7 + 1e-6).all()


def test_readout_normalises_and_appends_none():
    cfg = od.DecoderConfig(hidden=32)
    g = torch.Generator().manual_seed(4)
    h = torch.randn(2 * 3 * 4, 32, generator=g).to(torch.bfloat16)
    head = torch.randn(32, generator=g)
    lp = od.readout(h, torch.ones(32, dtype=torch.bfloat16), head, torch.tensor(0.3), cfg, 2, 3, 4)
    assert lp.shape == (2, 4)
    assert torch.allclose(lp.exp().sum(-1), torch.ones(2), atol=1e-6)
    # the none logit is the last entry: its log-prob is 0.3 - logsumexp(all logits)
    hf = od.rmsnorm(h, torch.ones(32, dtype=torch.bfloat16), cfg.eps).double().reshape(2, 3, 4, 32).mean(2)
    logits = torch.cat([hf @ head.double(), torch.full((2, 1), 0.3, dtype=torch.float64)], 1)
    assert torch.allclose(lp[:, 3].double(), 0.3 - torch.logsumexp(logits, 1), atol=1e-5)
    assert torch.allclose(lp.double(), torch.log_softmax(logits, 1), atol=1e-5)


def _tiny_states(cfg, B, T, layers, seed):
    from oracle import quant as oq
    g = torch.Generator().manual_seed(seed)
    out = []
    for _ in range(layers):
        kv = torch.randn(2, B, cfg.n_kv_heads, T, cfg.head_dim, generator=g).to(torch.bfloat16)
        kq, ks = oq.quantize_rows(kv[0])
        vq, vs = oq.quantize_rows(kv[1])
        out.append(((kq, ks[..., 0]), (vq, vs[..., 0])))
    return out


def test_decision_forward_is_option_order_invariant():
    cfg = od.DecoderConfig(hidden=128, ffn=256, n_heads=4, n_kv_heads=2, head_dim=32, n_layers=2, vocab=97)
    w = od.make_weights(cfg, seed=5)
    emb = od.make_embedding(cfg, seed=5)
    B, n_opt, t, T = 2, 5, 3, 20
    states = _tiny_states(cfg, B, T, cfg.n_layers, 6)
    ids = torch.randint(0, cfg.vocab, (B, n_opt, t), generator=torch.Generator().manual_seed(7))
    lp = od.decision_forward(ids, w, emb, cfg, states, T)
    perm = torch.tensor([3, 0, 4, 1, 2])
    lp_p = od.decision_forward(ids[:, perm], w, emb, cfg, states, T)
    assert (lp_p[:, :n_opt] - lp[:, perm]).abs().max().item() <= 1e-6
    assert (lp_p[:, n_opt] - lp[:, n_opt]).abs().max().item() <= 1e-6
    assert torch.allclose(lp.exp().sum(-1), torch.ones(B), atol=1e-5)


# ---- state prefill (prefill_forward)

def _tiny():
    cfg = od.DecoderConfig(hidden=64, ffn=128, n_heads=4, n_kv_heads=2, head_dim=16, n_layers=2, vocab=97)
    return cfg, od.make_weights(cfg, seed=11), od.make_embedding(cfg, seed=11)


def test_prefill_is_causal():
    """A state token's hidden state depends only on the tokens before it: prefilling a prefix of the ids gives the
    same hidden states for that prefix as prefilling all of them."""
    cfg, w, emb = _tiny()
    ids = torch.randint(0, cfg.vocab, (2, 20), generator=torch.Generator().manual_seed(1))
    h_all, kv_all = od.prefill_forward(ids, w, emb, cfg)
    h_pre, kv_pre = od.prefill_forward(ids[:, :13], w, emb, cfg)
    hs = h_all.reshape(2, 20, -1)[:, :13].reshape(26, -1)
    assert ((hs.float() - h_pre.float()).abs() <= 1e-2 * h_pre.float().abs().max()).all()
    for (k1, _), (k2, _) in zip(kv_all, kv_pre):
        d = (k1[0][:, :, :13].int() - k2[0].int()).abs()
        assert d.max().item() <= 1 and (d > 0).float().mean().item() < 0.01


def test_prefill_append_keeps_cache_and_positions():
    """An appended record leaves the cached tokens' bytes untouched, grows every layer's cache by the record's
    length, and its layer-0 keys are the ones computed at positions n0 .. n0 + S - 1 (RoPE continues the state)."""
    cfg, w, emb = _tiny()
    g = torch.Generator().manual_seed(2)
    ids0 = torch.randint(0, cfg.vocab, (2, 17), generator=g)
    rec = torch.randint(0, cfg.vocab, (2, 9), generator=g)
    _, kv0 = od.prefill_forward(ids0, w, emb, cfg)
    _, kv1 = od.prefill_forward(rec, w, emb, cfg, state_kv=kv0, n0=17)
    for ((kq0, ks0), (vq0, vs0)), ((kq1, ks1), (vq1, vs1)) in zip(kv0, kv1):
        assert kq1.shape[2] == 26 and vs1.shape[2] == 26
        assert torch.equal(kq1[:, :, :17], kq0) and torch.equal(vq1[:, :, :17], vq0)
        assert torch.equal(ks1[:, :, :17], ks0) and torch.equal(vs1[:, :, :17], vs0)
    # layer 0 keys of the record, recomputed directly at positions 17 .. 25
    lw = w["layers"][0]
    ql = od.quantize_layer(lw)
    x = od.rmsnorm(emb[rec.reshape(-1)], lw["ln1"], cfg.eps)
    qkv, _, _, _ = oq.w8a8_linear(x, ql["wqkv"][0], ql["wqkv"][1], inv_s=ql["wqkv"][2])
    cos, sin = od.rope_tables(cfg, 26)
    qkv = od.qk_norm_rope(qkv, cfg, lw["q_norm"], lw["k_norm"], cos, sin, (17 + torch.arange(9)).repeat(2))
    D, Hq, Hk = cfg.head_dim, cfg.n_heads, cfg.n_kv_heads
    k = qkv[:, Hq * D:(Hq + Hk) * D].reshape(2, 9, Hk, D).transpose(1, 2).contiguous()
    kq, ks = oq.quantize_rows(k)
    assert torch.equal(kv1[0][0][0][:, :, 17:], kq)
    # and they differ from keys rotated as if the record started at position 0
    qkv0 = od.qk_norm_rope(oq.w8a8_linear(x, ql["wqkv"][0], ql["wqkv"][1], inv_s=ql["wqkv"][2])[0], cfg,
                           lw["q_norm"], lw["k_norm"], cos, sin, torch.arange(9).repeat(2))
    k0 = qkv0[:, Hq * D:(Hq + Hk) * D].reshape(2, 9, Hk, D).transpose(1, 2).contiguous()
    assert not torch.equal(oq.quantize_rows(k0)[0], kq)


# ---- the correctly rounded RMSNorm factor and SiLU that the row kernels reproduce bit for bit

def _nearest_f32(d):
    """The fp32 value nearest to the Decimal d (ties to even), by comparing the neighbours of a float64 guess."""
    import decimal
    import numpy as np
    f = np.float32(float(d))
    best = None
    for c in (np.nextafter(f, np.float32(-np.inf)), f, np.nextafter(f, np.float32(np.inf))):
        err = abs(decimal.Decimal(float(c)) - d)
        key = (err, int(np.array(c).view(np.int32)) & 1)
        if best is None or key < best[0]:
            best = (key, c)
    return float(best[1])


def test_rms_factor_is_the_correctly_rounded_value():
    """rms_factor = RN32(1 / sqrt(sum(x^2) / K + eps32)), checked against 60-digit decimal arithmetic on rows that
    span many binades, and within 2 fp32 ulps of the reference's fp32 expression torch.rsqrt(x.pow(2).mean() + eps)."""
    import decimal
    decimal.getcontext().prec = 60
    g = torch.Generator().manual_seed(21)
    x = (torch.randn(24, 300, generator=g) * torch.exp2(torch.randint(-12, 12, (24, 300), generator=g).float()))
    x = x.to(torch.bfloat16)
    x[3] = 0
    r = od.rms_factor(x, 1e-6)
    eps = decimal.Decimal(float(torch.tensor(1e-6, dtype=torch.float32)))
    for i in range(x.shape[0]):
        ss = sum(decimal.Decimal(float(v)) ** 2 for v in x[i].float().tolist())
        exact = 1 / (ss / x.shape[1] + eps).sqrt()
        assert r[i, 0].item() == _nearest_f32(exact), i
    ref32 = torch.rsqrt(x.float().pow(2).mean(-1, keepdim=True) + 1e-6)
    ulp = (r.view(torch.int32) - ref32.view(torch.int32)).abs()
    assert ulp.max().item() <= 2


def test_silu_bf16_is_the_correctly_rounded_value_on_all_bf16_inputs():
    """silu_bf16(g) = bf16(RN32(g / (1 + exp(-g)))) on all 65536 bf16 inputs: checked against 40-digit decimal
    arithmetic on a spread sample of the finite nonzero inputs with |g| <= 200 (beyond that the result is g or a tiny
    negative, checked directly), and equal bit for bit to torch's own bf16 F.silu (the reference's arithmetic) on every
    input except g < -88, where torch's fp32 exp(-g) overflows and it returns -0 instead of the tiny exact value."""
    import decimal
    decimal.getcontext().prec = 40
    g = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    s = od.silu_bf16(g)
    gf = g.float()
    fin = torch.isfinite(gf) & (gf != 0) & (gf.abs() <= 200)
    idx = fin.nonzero().squeeze(1).tolist()
    for i in idx[::7] + idx[1::97]:  # a seventh of the inputs plus a spread sample (the full set takes ~10 s more)
        d = decimal.Decimal(float(gf[i]))
        exact = d / (1 + (-d).exp())
        want = torch.tensor(_nearest_f32(exact), dtype=torch.float32).to(torch.bfloat16)
        assert s[i].view(torch.int16) == want.view(torch.int16), (gf[i].item(), s[i].item(), want.item())
    big = (gf.abs() > 200) & torch.isfinite(gf)
    assert torch.equal(s[big & (gf > 0)], g[big & (gf > 0)])
    assert (s[big & (gf < 0)].float().abs() <= 2.0 ** -120).all()
    assert s[gf == 0].float().eq(0).all() and torch.isnan(s[torch.isnan(gf)]).all()
    assert s[gf == float("inf")].float().eq(float("inf")).all() and torch.isnan(s[gf == float("-inf")]).all()
    ref = torch.nn.functional.silu(g)
    ok = torch.isfinite(ref) & ~(gf < -88)  # below -88 torch's fp32 exp(-g) overflows and it returns -0
    assert torch.equal(s[ok].view(torch.int16), ref[ok].view(torch.int16))


def test_sigmoid_bf16_is_torch_bf16_sigmoid():
    """sigmoid_bf16 (the output gate's bf16(sigmoid(g)), correctly rounded in fp32 first) equals torch's bf16 sigmoid
    bit for bit on every bf16 input except g < -88 (where torch's fp32 exp(-g) overflows and it returns 0), and the
    60-digit decimal value on a sample."""
    import decimal
    decimal.getcontext().prec = 40
    g = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    s = od.sigmoid_bf16(g)
    gf = g.float()
    ref = torch.sigmoid(g)
    ok = torch.isfinite(ref) & ~(gf < -88)
    assert torch.equal(s[ok].view(torch.int16), ref[ok].view(torch.int16))
    fin = (torch.isfinite(gf) & (gf.abs() <= 80)).nonzero().squeeze(1).tolist()
    for i in fin[::53]:
        d = decimal.Decimal(float(gf[i]))
        want = torch.tensor(_nearest_f32(1 / (1 + (-d).exp())), dtype=torch.float32).to(torch.bfloat16)
        assert s[i].view(torch.int16) == want.view(torch.int16), gf[i].item()


# ---- the end-to-end bar of the GPU tests: what it can see at the harness's decision temperature

E2E_SCORING = (dict(n_layers=2, vocab=1000), 2, 32, 16, 256)   # tests/test_gpu_decoder.py CASES["9b_dims_2_layers"]
T_E2E = 24.0


def test_end_to_end_bar_separates_kernel_mistakes_from_the_oracles_own_noise():
    """At the GPU end-to-end test's configuration and temperature: the oracle with float64 attention accumulation
    moves the option probabilities by well under 1e-4 (its own rounding floor, 1.4e-5), while planted mistakes of the
    kind a kernel can make move them past the 1e-4 bar: a wrong GQA head mapping (2.6e-4), the keys of another state
    (1.9e-4), the SmoothQuant scale dropped before the O projection (1.6e-4). Smaller planted mistakes (one position
    off in RoPE, a non-causal own block, the V scale of the neighbouring token) land below 1e-4 (0.6-0.8e-4); the
    stage-by-stage GPU test, bit-exact outside the attention, is what pins those."""
    from helpers import decoder_case
    from oracle import attention as oa
    cfg_kw, B, n_opt, t, T = E2E_SCORING
    cfg, w, emb, states, ids = decoder_case(cfg_kw, B, n_opt, t, T, T_E2E)
    ref = od.decision_forward(ids, w, emb, cfg, states, T)

    def dp(x):
        return (x.exp() - ref.exp()).abs().max().item()

    floor = dp(od.decision_forward(ids, w, emb, cfg, states, T, attn_dtype=torch.float64))
    orig = oa.branched_attention_int8
    Hq, Hkv = cfg.n_heads, cfg.n_kv_heads
    src = (torch.arange(Hq) % Hkv) * (Hq // Hkv) + torch.arange(Hq) // Hkv
    inv = torch.argsort(src)

    def gqa(q, *a, **k):  # query head h reads KV head h % Hkv instead of h // (Hq / Hkv)
        o, lse = orig(q[:, src], *a, **k)
        return o[:, inv], lse[:, inv]

    oa.branched_attention_int8 = gqa
    try:
        wrong_gqa = dp(od.decision_forward(ids, w, emb, cfg, states, T))
    finally:
        oa.branched_attention_int8 = orig
    other = [((kq.flip(0), ks.flip(0)), v) for (kq, ks), v in states]
    wrong_state = dp(od.decision_forward(ids, w, emb, cfg, other, T))
    orig_q = od.quantize_layer

    def no_smooth_o(lw):
        d = orig_q(lw)
        d["wo"] = (d["wo"][0], d["wo"][1], None)
        return d

    od.quantize_layer = no_smooth_o
    try:
        dropped = dp(od.decision_forward(ids, w, emb, cfg, states, T))
    finally:
        od.quantize_layer = orig_q
    print(f"floor {floor:.2e}; GQA {wrong_gqa:.2e}, other state {wrong_state:.2e}, no 1/s {dropped:.2e}")
    assert floor <= 2e-5
    assert min(wrong_gqa, wrong_state, dropped) >= 1.3e-4


def test_question_cache_equals_rows_that_carry_the_question():
    """The question cache's claim (v3.py:447-450: same features as repeating the question in each row): with float64
    attention, a question pass + option rows over [state ; question K/V] give the same log-probabilities as rows that
    carry [question ; option] tokens over the state alone, pooled over the option tokens only (one question per
    state, no pads): every bf16 attention output agrees, so everything downstream is identical."""
    from helpers import decoder_case
    cfg, w, emb, states, _ = decoder_case(dict(hidden=256, ffn=512, n_heads=4, n_kv_heads=2, head_dim=64,
                                               n_layers=2, vocab=500), 2, 1, 1, 70, 24.0)
    g = torch.Generator().manual_seed(12)
    Lq, n_opt, t = 9, 4, 5
    ids_q = torch.randint(0, 500, (2, Lq), generator=g)
    ids_o = torch.randint(0, 500, (2, n_opt, t), generator=g)
    q_kv = od.question_forward(ids_q, w, emb, cfg, states, 70, [0, 1], attn_dtype=torch.float64)
    lp_qc = od.qcache_decision_forward(ids_o, w, emb, cfg, states, 70, q_kv, [Lq, Lq], [0, 1],
                                       attn_dtype=torch.float64)
    rows = torch.cat([ids_q[:, None, :].expand(2, n_opt, Lq), ids_o], 2)  # (2, n_opt, Lq + t)
    lp_rows = od.decision_forward(rows, w, emb, cfg, states, 70, attn_dtype=torch.float64, pool_last=t)
    assert (lp_qc - lp_rows).abs().max().item() <= 1e-6


def _layer0_attention_inputs():
    """Layer 0's attention inputs at the GPU end-to-end test's 9B scoring configuration, computed by the oracle's
    stage functions exactly as tests/test_gpu_decoder.py's stage-by-stage test does: (qkv before RoPE, cfg, layer
    weights, positions, rope tables, the (R, t) layout, the int8 state, row states)."""
    from helpers import decoder_case
    from oracle import quant as oq
    cfg_kw, B, n_opt, t, T = E2E_SCORING
    cfg, w, emb, states, ids = decoder_case(cfg_kw, B, n_opt, t, T, T_E2E)
    R = B * n_opt
    lw, ql = w["layers"][0], od.quantize_layer(w["layers"][0])
    h = emb[ids.reshape(-1)]
    xq, sx = oq.act_quant(od.rmsnorm(h, lw["ln1"], cfg.eps), ql["wqkv"][2])
    qkv_lin, _ = od.split_qkv(oq.w8a8_epilogue(oq.int_gemm(xq, ql["wqkv"][0]), sx, ql["wqkv"][1]), cfg)
    pos = (T + torch.arange(t)).repeat(R)
    cos, sin = od.rope_tables(cfg, T + t)
    return qkv_lin, cfg, lw, pos, cos, sin, R, t, states[0], torch.arange(B).repeat_interleave(n_opt)


def _heads(qkv, cfg, R, t):
    D, Hq, Hk = cfg.head_dim, cfg.n_heads, cfg.n_kv_heads
    qh = qkv[:, :Hq * D].reshape(R, t, Hq, D).transpose(1, 2)
    kh = qkv[:, Hq * D:(Hq + Hk) * D].reshape(R, t, Hk, D).transpose(1, 2)
    vh = qkv[:, (Hq + Hk) * D:(Hq + 2 * Hk) * D].reshape(R, t, Hk, D).transpose(1, 2)
    return qh, kh, vh


def test_stage_checks_catch_the_mistakes_the_end_to_end_bar_cannot_see():
    """Three kernel mistakes that move the end-to-end probabilities by less than the bar (0.7-1.1e-4 at T = 24, and
    at T = 1 less than the reference's own GPU-vs-CPU spread): RoPE one position off, a non-causal own block, each
    key's V dequantized with the neighbouring token's scale. The GPU stage-by-stage test compares each stage with the
    oracle fed the GPU's input to that stage; here each mistake is planted in a copy of the oracle's stage and the
    same comparison (bit-exact for q/k norm + RoPE, the 2e-3 bar of tests/helpers.py for the attention) rejects it,
    while the unplanted stage passes it."""
    from helpers import assert_close_rel
    from oracle import attention as oa
    qkv_lin, cfg, lw, pos, cos, sin, R, t, ((kq, ks), (vq, vs)), row_state = _layer0_attention_inputs()
    D, Hq = cfg.head_dim, cfg.n_heads
    M = R * t
    # RoPE: the GPU test asserts torch.equal on the bits of the fused QKV + q/k norm + RoPE output
    qkv = od.qk_norm_rope(qkv_lin, cfg, lw["q_norm"], lw["k_norm"], cos, sin, pos)
    qkv_again = od.qk_norm_rope(qkv_lin, cfg, lw["q_norm"], lw["k_norm"], cos, sin, pos)
    qkv_off = od.qk_norm_rope(qkv_lin, cfg, lw["q_norm"], lw["k_norm"], cos, sin, pos - 1)
    assert torch.equal(qkv_again.view(torch.int16), qkv.view(torch.int16))
    assert not torch.equal(qkv_off.view(torch.int16), qkv.view(torch.int16))
    # attention: the GPU test asserts assert_close_rel(GPU output, oracle on the GPU's q/k/v)
    qh, kh, vh = _heads(qkv, cfg, R, t)

    def run(vs_=vs):
        o, _ = oa.branched_attention_int8(qh, kh, vh, kq, ks, vq, vs_, D ** -0.5, None, row_state, dequant="bf16")
        return o.to(torch.bfloat16).float().transpose(1, 2).reshape(M, Hq * D)

    ref = run()
    assert_close_rel(ref, ref, what="the unplanted stage")
    orig = oa.attention
    oa.attention = lambda q, k, v, scale, kvalid=None, causal=True, **kw: orig(q, k, v, scale, kvalid, False, **kw)
    try:
        noncausal = run()
    finally:
        oa.attention = orig
    neighbour = run(vs.roll(-1, dims=2))
    for what, got in (("non-causal own block", noncausal), ("neighbouring V scale", neighbour)):
        with pytest.raises(AssertionError):
            assert_close_rel(got, ref, what=what)
