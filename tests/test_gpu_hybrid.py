"""GPU parity of the hybrid decision forward (Qwen3.5's stack: Gated DeltaNet layers with a full-attention layer
every `full_attention_interval`) against the oracle (oracle/decoder.py + oracle/gdn.py).

Every layer stage by stage, each stage fed the GPU's own input (the attention layers as in the dense stack's
tests). GDN layers: the RMSNorm quantizer, the in_proj GEMM, the conv + SiLU / l2norm / gates, the gated norm +
out_proj quantizer, out_proj + residual and the MLP are bit-exact; the recurrence (fp32 state, hardware reduction
order) is within one bf16 step of the float64 recurrence. Option rows
read their request's conv window and recurrent state in place (seq_state), never a per-row copy. End to end: the
path's bar at the harness's decision temperature T_E2E (probabilities 1e-4, log-probabilities 2e-3), option-order
invariance <= 1e-6, a prefilled and record-appended state, and the captured scoring pass equal to eager. The T = 1
figures are printed, not held to the all-attention stacks' T = 1 bar: the reference runs the Gated DeltaNet layers
through the fla Triton kernels (a dependency absent here, its bf16 chunked arithmetic not restated by the oracle), so
the spread between the reference's own GPU and CPU arithmetic is known for the attention layers only."""
import pytest
import torch

from oracle import attention as oa
from oracle import decoder as od
from oracle import gdn as og
from oracle import quant as oq

from helpers import hybrid_states
from test_gpu_decoder import _assert_e2e, attention_layer_stages

pytestmark = pytest.mark.gpu
DEV = "cuda"
T_E2E = 24.0

TINY = dict(hidden=256, ffn=512, n_heads=4, n_kv_heads=2, head_dim=64, n_layers=4, vocab=500,
            full_attention_interval=2, lin_k_heads=2, lin_v_heads=4, gated=True)
NINE_B = dict(n_layers=4, vocab=1000, full_attention_interval=4, gated=True)   # 3 GDN layers + 1 attention layer
# Qwen3.5's own attention geometry (transformers' Qwen3_5TextConfig): 16 / 4 heads of 256, rotary on the first 64
# dims, zero-centred RMSNorms
QWEN35 = dict(NINE_B, n_heads=16, n_kv_heads=4, head_dim=256, rot_dim=64, norm_offset=True)
TINY_QWEN35 = dict(TINY, rot_dim=16, norm_offset=True)
CASES = [("tiny_hybrid", TINY, 2, 5, 4, 40), ("9b_dims_hybrid_4_layers", NINE_B, 2, 32, 16, 256),
         ("tiny_hybrid_qwen35_geometry", TINY_QWEN35, 2, 5, 4, 40),
         ("qwen35_hybrid_4_layers", QWEN35, 2, 32, 16, 256)]


def _exact(a, b, what):
    a, b = a.cpu(), b.cpu()
    assert a.shape == b.shape, (what, a.shape, b.shape)
    if a.dtype == torch.bfloat16:
        a, b = a.view(torch.int16), b.view(torch.int16)
    elif a.dtype == torch.float32:
        a, b = a.view(torch.int32), b.view(torch.int32)
    bad = a != b
    assert not bad.any(), f"{what}: {int(bad.sum())} of {bad.numel()} differ"


def _random_states(cfg, B, T, seed=4):
    return hybrid_states(cfg, B, T, seed)


def _load_states(dec, cfg, states, B, T, cap):
    st = dec.new_state_caches(B, cap)
    for li, s in enumerate(states):
        if cfg.is_gdn(li):
            st[li].conv.copy_(s[0].to(DEV))
            st[li].rec.copy_(s[1].to(DEV))
            st[li].length = T
        else:
            for c, (q, sc) in zip(st[li], s):
                c.q[:, :, :T].copy_(q.to(DEV))
                c.scale[:, :, :T].copy_(sc.to(DEV))
                c.length = T
                c.touch()
    return st


def _setup(cfg_kw, B, n_opt, t, T):
    from opendecider_amd.decoder import DecoderConfig, DenseDecoder
    cfg = od.DecoderConfig(**cfg_kw)
    w = od.make_weights(cfg, seed=3)
    w["temperature"] = T_E2E
    emb = od.make_embedding(cfg, seed=3)
    states = _random_states(cfg, B, T)
    ids = torch.randint(0, cfg.vocab, (B, n_opt, t), generator=torch.Generator().manual_seed(5))
    dec = DenseDecoder(DecoderConfig(**cfg_kw), w, emb, DEV, max_pos=T + t + 8)
    assert dec.hybrid
    return cfg, w, emb, states, ids, dec, _load_states(dec, cfg, states, B, T, T + 16)


@pytest.mark.parametrize("name,cfg_kw,B,n_opt,t,T", CASES)
def test_hybrid_layers_stage_by_stage(gpu_lib, name, cfg_kw, B, n_opt, t, T):
    from opendecider_amd import kernels
    cfg, w, emb, states, ids, dec, gs = _setup(cfg_kw, B, n_opt, t, T)
    gc = cfg.gdn
    R, M = B * n_opt, B * n_opt * t
    C, V, P = gc.conv_dim, gc.value_dim, gc.proj_out
    kd, nv, rep = gc.key_dim, gc.n_v_heads, gc.n_v_heads // gc.n_k_heads
    pos = (T + torch.arange(t)).repeat(R)
    cos, sin = od.rope_tables(cfg, T + t + 8)
    row_state = torch.arange(B).repeat_interleave(n_opt)
    rs_dev = dec.row_states(B, n_opt)
    rs, mr = kernels.row_start_of([n_opt] * B, DEV)
    ws = dec.workspace(M)
    h, mid = ws["h"]
    h.copy_(emb[ids.reshape(-1)].to(DEV))
    for li in range(cfg.n_layers):
        lw, ql, L = w["layers"][li], od.quantize_layer(w["layers"][li]), dec.layers[li]
        h_in_g = h.clone()
        h_in = h_in_g.cpu()
        print(f"{name}: layer {li} ({'GDN' if cfg.is_gdn(li) else 'attention'})", flush=True)
        if not cfg.is_gdn(li):
            attention_layer_stages(dec, cfg, w, li, ws, gs[li], states[li], R, t, pos, cos, sin, row_state, rs, mr)
            continue
        conv_s, rec_s = states[li]
        dec.gdn_layer(li, h, mid, ws, gs[li], R, t, rs_dev)
        proj_g, qk_g, v_g, g_g, b_g, o_g = (ws[k].cpu() for k in ("proj", "gqk", "gv", "gg", "gbeta", "go"))
        mid_g, hm_g, out_g = mid.cpu(), ws["hmlp"].cpu(), h.cpu()
        # ln1 + quantize, in_proj GEMM (the padding rows stay zero)
        xq, sx = kernels.rmsnorm_quant(h_in_g, L["ln1"], cfg.eps, L["win"].inv_s, offset=cfg.norm_offset)
        rq, rsx = oq.act_quant(od.rmsnorm(h_in, lw["ln1"], cfg.eps, cfg.norm_offset), ql["win"][2])
        _exact(xq, rq, f"layer {li}: ln1 bytes")
        _exact(sx, rsx.reshape(sx.shape), f"layer {li}: ln1 scales")
        proj = oq.w8a8_epilogue(oq.int_gemm(xq.cpu(), ql["win"][0]), sx.cpu(), ql["win"][1])
        _exact(proj_g[:, :P], proj, f"layer {li}: in_proj GEMM")
        assert (proj_g[:, P:] == 0).all()
        # conv + SiLU from each row's state window, l2norm, gates
        qkv, z, b, a = og.split_proj(proj_g[:, :P], gc)
        y, _ = og.conv_silu(qkv.reshape(R, t, C), lw["conv_w"], conv_s[row_state])
        y = y.reshape(M, C)
        q = og.l2norm_bf16(y[:, :kd].reshape(M, gc.n_k_heads, gc.dk)).reshape(M, kd)
        k = og.l2norm_bf16(y[:, kd:2 * kd].reshape(M, gc.n_k_heads, gc.dk)).reshape(M, kd)
        _exact(qk_g, torch.cat([q, k], 1), f"layer {li}: conv + l2norm (q, k)")
        _exact(v_g, y[:, 2 * kd:], f"layer {li}: conv (v)")
        gg, beta = og.gates(a, b, lw["A_log"], lw["dt_bias"])
        _exact(g_g, gg, f"layer {li}: g")
        _exact(b_g, beta, f"layer {li}: beta")
        # the recurrence from each row's shared state, from the GPU's inputs, against float64
        sh = lambda x, d: x.reshape(M, -1, d).repeat_interleave(rep, 1).reshape(R, t, nv, d)
        o, _ = og.recurrence(sh(qk_g[:, :kd], gc.dk), sh(qk_g[:, kd:], gc.dk), v_g.reshape(R, t, nv, gc.dv),
                             g_g.reshape(R, t, nv), b_g.reshape(R, t, nv), rec_s[row_state], torch.float64)
        o = o.reshape(M, V).float()
        d = (o_g.float() - o).abs()
        assert (d <= o.abs() * 2.0 ** -7 + 1e-6).all() and (d.norm() / o.norm()).item() <= 2e-3, \
            f"layer {li}: recurrence {d.max().item()}"
        # gated norm + out_proj quantizer (re-run on the GPU's o: the kernel is deterministic), out_proj + residual
        xq, sx = kernels.gdn_norm_quant(ws["go"], ws["proj"][:, C:C + V], L["gnorm"], cfg.eps, nv, gc.dv,
                                        L["wout"].inv_s)
        yn = og.gated_norm(o_g.reshape(M, nv, gc.dv), z.reshape(M, nv, gc.dv), lw["gnorm"], cfg.eps)
        rq, rsx = oq.act_quant(yn.reshape(M, V), ql["wout"][2])
        _exact(xq, rq, f"layer {li}: gated norm bytes")
        _exact(sx, rsx.reshape(sx.shape), f"layer {li}: gated norm scales")
        h_mid = oq.w8a8_epilogue(oq.int_gemm(rq, ql["wout"][0]), rsx, ql["wout"][1], residual=h_in)
        _exact(mid_g, h_mid, f"layer {li}: out_proj + residual")
        # the MLP
        xq, sx = kernels.rmsnorm_quant(mid.clone(), L["ln2"], cfg.eps, L["gu"].inv_s, offset=cfg.norm_offset)
        rq, rsx = oq.act_quant(od.rmsnorm(mid_g, lw["ln2"], cfg.eps, cfg.norm_offset), ql["wgu"][2])
        _exact(xq, rq, f"layer {li}: ln2")
        gu = oq.w8a8_epilogue(oq.int_gemm(rq, ql["wgu"][0]), rsx, ql["wgu"][1])
        _exact(hm_g, od.swiglu(gu, cfg.ffn), f"layer {li}: gate+up + SwiGLU")
        rq, rsx = oq.act_quant(hm_g, ql["wdown"][2])
        _exact(out_g, oq.w8a8_epilogue(oq.int_gemm(rq, ql["wdown"][0]), rsx, ql["wdown"][1], residual=mid_g),
               f"layer {li}: down + residual")
    lp = dec.readout(h, B, n_opt, t)
    ref = od.readout(h.cpu(), w["final_norm"], w["head"], w["none_logit"], cfg, B, n_opt, t, T_E2E)
    assert (lp.cpu() - ref).abs().max().item() <= 1e-6, "readout"
    # the states were only read
    for li in range(cfg.n_layers):
        if cfg.is_gdn(li):
            _exact(gs[li].conv, states[li][0], f"layer {li}: conv state untouched")
            _exact(gs[li].rec, states[li][1], f"layer {li}: recurrent state untouched")




@pytest.mark.parametrize("name,cfg_kw,B,n_opt,t,T", CASES)
def test_hybrid_decision_forward_end_to_end(gpu_lib, name, cfg_kw, B, n_opt, t, T):
    cfg, w, emb, states, ids, dec, gs = _setup(cfg_kw, B, n_opt, t, T)
    print(f"{name}: e2e B={B} options={n_opt} t={t} T={T}", flush=True)
    ref = od.decision_forward(ids, w, emb, cfg, states, T)
    # the reference's own GPU arithmetic: the blocked flash attention and the recurrence in fp32 (the oracle's
    # reference value uses float64)
    with oa.reference_gpu_arithmetic():
        ref_gpu = od.decision_forward(ids, w, emb, cfg, states, T, gdn_dtype=torch.float32)
    lp = dec.score(ids.to(DEV), gs)
    _assert_e2e(lp, ref, name, ref_gpu, t1_bar=False)
    perm = torch.randperm(n_opt, generator=torch.Generator().manual_seed(6))
    lp_p = dec.score(ids[:, perm].to(DEV), gs)
    assert (lp_p[:, :n_opt].exp() - lp[:, perm.to(DEV)].exp()).abs().max().item() <= 1e-6


@pytest.mark.parametrize("name,cfg_kw,B,n_opt,t,S,records", [("tiny_hybrid", TINY, 2, 5, 4, 37, [24, 2]),
                                                             ("9b_dims_hybrid_4_layers", NINE_B, 2, 32, 16, 256,
                                                              [64]),
                                                             ("tiny_hybrid_qwen35_geometry", TINY_QWEN35, 2, 5, 4, 37,
                                                              [24, 2]),
                                                             ("qwen35_hybrid_4_layers", QWEN35, 2, 32, 16, 256, [64])])
def test_hybrid_prefill_and_score_end_to_end(gpu_lib, name, cfg_kw, B, n_opt, t, S, records):
    """States prefilled from token ids (GDN layers: conv windows and recurrent states written back; attention layers:
    int8 K/V), records appended (GDN layers continue their states), then the option rows scored. Layer 0 (a GDN
    layer, fed the embeddings) leaves a bit-exact conv window and a recurrent state within 1e-5 of the float64 one;
    the probabilities meet the end-to-end bar."""
    from opendecider_amd.decoder import DecoderConfig, DenseDecoder
    cfg = od.DecoderConfig(**cfg_kw)
    w = od.make_weights(cfg, seed=7)
    w["temperature"] = T_E2E
    emb = od.make_embedding(cfg, seed=7)
    cap = S + sum(records)
    dec = DenseDecoder(DecoderConfig(**cfg_kw), w, emb, DEV, max_pos=cap + 64)
    g = torch.Generator().manual_seed(8)
    ids_state = torch.randint(0, cfg.vocab, (B, S), generator=g)
    recs = [torch.randint(0, cfg.vocab, (B, n), generator=g) for n in records]
    ids = torch.randint(0, cfg.vocab, (B, n_opt, t), generator=g)
    print(f"{name}: prefill B={B} S={S} records={records}", flush=True)
    st = dec.new_state_caches(B, cap)
    dec.prefill(ids_state.to(DEV), st)
    torch.cuda.synchronize()
    _, ref_st = od.prefill_forward(ids_state, w, emb, cfg)
    with oa.reference_gpu_arithmetic():
        _, gpu_st = od.prefill_forward(ids_state, w, emb, cfg, gdn_dtype=torch.float32)
    assert cfg.is_gdn(0)
    _exact(st[0].conv, ref_st[0][0], "layer 0 conv window")
    r0 = ref_st[0][1]
    assert torch.allclose(st[0].rec.cpu(), r0, rtol=1e-5, atol=1e-5 * r0.abs().max().item()), "layer 0 state"
    n0 = S
    for r in recs:
        dec.prefill(r.to(DEV), st)
        _, ref_st = od.prefill_forward(r, w, emb, cfg, state_kv=ref_st, n0=n0)
        with oa.reference_gpu_arithmetic():
            _, gpu_st = od.prefill_forward(r, w, emb, cfg, state_kv=gpu_st, n0=n0, gdn_dtype=torch.float32)
        n0 += r.shape[1]
    assert st.length == n0
    torch.cuda.synchronize()
    _exact(st[0].conv, ref_st[0][0], "layer 0 conv window after the records")
    lp = dec.score(ids.to(DEV), st)
    ref = od.decision_forward(ids, w, emb, cfg, ref_st, n0)
    with oa.reference_gpu_arithmetic():
        ref_gpu = od.decision_forward(ids, w, emb, cfg, gpu_st, n0, gdn_dtype=torch.float32)
    _assert_e2e(lp, ref, f"{name} (prefilled)", ref_gpu, t1_bar=False)


@pytest.mark.parametrize("name,cfg_kw,B,n_opt,t,T", CASES)
def test_hybrid_scoring_graph_replays_equal_eager(gpu_lib, name, cfg_kw, B, n_opt, t, T):
    """The hybrid scoring pass captured in one HIP graph: three replays with eager passes on other ids between them
    each equal the eager pass bit for bit; the states are unchanged by any of it."""
    cfg, w, emb, states, ids, dec, gs = _setup(cfg_kw, B, n_opt, t, T)
    run = dec.capture_scoring(gs, B, n_opt, t)
    other = torch.randint(0, cfg.vocab, (B, n_opt, t), generator=torch.Generator().manual_seed(9))
    want = dec.score(ids.to(DEV), gs).clone()
    for i in range(3):
        got = run(ids.to(DEV)).clone()
        dec.score(other.to(DEV), gs)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"replay {i}"
    assert torch.equal(run(other.to(DEV)), dec.score(other.to(DEV), gs))
    for li in range(cfg.n_layers):
        if cfg.is_gdn(li):
            _exact(gs[li].rec, states[li][1], f"layer {li}: recurrent state untouched")


QCACHE_CASES = [("tiny_hybrid_qwen35_geometry", TINY_QWEN35, 2, 40, [0, 0, 1], 12, [12, 7, 3], 4, 5),
                ("qwen35_hybrid_4_layers", QWEN35, 2, 256, [0, 1], 48, [48, 29], 32, 8)]


@pytest.mark.parametrize("name,cfg_kw,B,T,gs,Lq,qlen,n_opt,t", QCACHE_CASES)
def test_hybrid_question_cache_end_to_end(gpu_lib, name, cfg_kw, B, T, gs, Lq, qlen, n_opt, t):
    """The question cache on the hybrid stack (v3.py:446-534 with the batched, right-padded question pass of
    Backbone.padded_continuation): each question continues its state's GDN layers over its real tokens into a
    per-question state and keeps its K/V for the attention layers; the option rows continue that state and attend
    [state ; question]. Against the oracle's question_forward + qcache_decision_forward at the end-to-end bar; the
    request states are left as they were."""
    cfg, w, emb, states, _, dec, gstates = _setup(cfg_kw, B, 1, Lq + t, T)  # rotary tables past T + Lq + t
    g = torch.Generator().manual_seed(11)
    ids_q = torch.randint(0, cfg.vocab, (len(gs), Lq), generator=g)
    ids_o = torch.randint(0, cfg.vocab, (len(gs), n_opt, t), generator=g)
    print(f"{name}: hybrid question cache questions={len(gs)} Lq={Lq} qlen={qlen} options={n_opt} t={t}", flush=True)
    qc = dec.question_pass(ids_q.to(DEV), qlen, gstates, gs)
    lp = dec.score_qcache(ids_o.to(DEV), qc, gstates)
    q_kv = od.question_forward(ids_q, w, emb, cfg, states, T, gs, qlen=qlen)
    ref = od.qcache_decision_forward(ids_o, w, emb, cfg, states, T, q_kv, qlen, gs)
    with oa.reference_gpu_arithmetic():
        q_kv_gpu = od.question_forward(ids_q, w, emb, cfg, states, T, gs, qlen=qlen, gdn_dtype=torch.float32)
        ref_gpu = od.qcache_decision_forward(ids_o, w, emb, cfg, states, T, q_kv_gpu, qlen, gs,
                                             gdn_dtype=torch.float32)
    _assert_e2e(lp, ref, f"{name} (hybrid question cache)", ref_gpu, t1_bar=False)
    for li in range(cfg.n_layers):
        if cfg.is_gdn(li):
            _exact(gstates[li].rec, states[li][1], f"layer {li}: request state untouched")
            _exact(gstates[li].conv, states[li][0], f"layer {li}: request conv window untouched")
    # layer 0 is fed the embeddings on both sides: the questions' conv windows (gathered at each real end) are exact
    assert cfg.is_gdn(0)
    _exact(qc.gdn[0].conv, q_kv[0][0], "layer 0: question conv windows")


def test_hybrid_rejects_what_it_does_not_define(gpu_lib):
    """Key masks (every token enters a recurrent state) and a prefill batch that is not the states' are refused
    before any launch."""
    from opendecider_amd.decoder import DecoderConfig, DenseDecoder
    cfg = od.DecoderConfig(**TINY)
    w = od.make_weights(cfg, seed=3)
    dec = DenseDecoder(DecoderConfig(**TINY), w, od.make_embedding(cfg, seed=3), DEV, max_pos=128)
    st = dec.new_state_caches(2, 64)
    ids = torch.randint(0, cfg.vocab, (2, 8), device=DEV)
    with pytest.raises(ValueError):
        dec.prefill(ids, st, kvalid=torch.ones(2, 8, dtype=torch.uint8, device=DEV))
    with pytest.raises(ValueError):
        dec.prefill(ids[:1], st)
    assert st.length == 0
