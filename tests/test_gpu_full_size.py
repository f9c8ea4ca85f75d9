"""The decision workloads at their full sizes (the shapes the benches run), where the oracle cannot run every layer:
the attention kernels against the oracle on those shapes (every output, or sampled rows where the oracle would take
minutes), and the 36-layer passes through properties that do not depend on size.

* The decision from ids (4 requests, 4096-token states prefilled from ids, 64 options x 24 tokens, 36 layers of 9B
  dims):
  - the causal state attention (od_wide_attn, B 4 x 32 heads x 4096 x 4096) against the blocked oracle on the first
    and the last 128 query positions of every (request, head);
  - the option-row attention over the 4096-token int8 states, every output against the oracle;
  - the pass: a state prefilled as 2048 tokens and then eight appended 256-token records holds, in every one of
    the 36 layers, the same int8 K/V bytes and scales for its first 2048 tokens as the state prefilled at once
    (those tokens see the same keys, and every kernel of the pass is row-independent), and the same layer-0 bytes
    for all 4096 tokens (layer 0's K/V depend on no attention); two scoring passes give the same bits; options
    permuted give the permuted probabilities (<= 1e-6); the probabilities over options and 'none' sum to 1.
* The wide-choice state (one 32768-token shared state grown by 256-token records, 2 x 255 options x 12 tokens):
  - the option-row attention over 33280 int8 keys, sampled rows against the oracle;
  - the pass: two 128-token records appended one at a time give the same layer-0 cache bytes as the two appended
    as one 256-token record; scoring is deterministic and option-order invariant (<= 1e-6).
"""
import pytest
import torch

from helpers import assert_close_rel
from oracle import attention as oa
from test_gpu_attention import make_case, run_gpu, run_oracle
from test_gpu_wide_attention import check_vs_blocked

pytestmark = pytest.mark.gpu
DEV = "cuda"


def test_config3_state_attention_full_shape(gpu_lib):
    from opendecider_amd import wide_attention
    B, H, G, S, D = 4, 32, 8, 4096, 128
    g = torch.Generator().manual_seed(31)
    q = torch.randn(B, H, S, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, G, S, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, G, S, D, generator=g).to(torch.bfloat16)
    print(f"wide_attention causal B={B} H={H} G={G} S={S} D={D}", flush=True)
    out, lse = wide_attention(q.to(DEV), k.to(DEV), v.to(DEV), D ** -0.5, None, causal=True, return_lse=True)
    out, lse = out.float().cpu(), lse.cpu()
    n = 128
    # first n positions: they see keys 0 .. n-1 only; last n positions: all keys (causal offset S - n)
    for what, qs, ks, vs, rows in (("first", q[:, :, :n], k[:, :, :n], v[:, :, :n], slice(0, n)),
                                   ("last", q[:, :, -n:], k, v, slice(S - n, S))):
        ob, _, bound = oa.wide_attention_blocked(qs, ks, vs, D ** -0.5, None, causal=True, with_bound=True)
        _, le = oa.attention(qs, ks, vs, D ** -0.5, None, causal=True)
        assert (lse[:, :, rows] - le).abs().max().item() < 1e-4, what
        check_vs_blocked(out[:, :, rows].reshape(B * H, n, D), ob.reshape(B * H, n, D), bound.reshape(B * H, n, D),
                         f"4 x 4096-token state attention, {what} {n} positions")


def test_config3_row_attention_full_shape(gpu_lib):
    c = make_case(seed=32, Ns=4, row_counts=[64] * 4, Hq=32, Hkv=8, t=24, D=128, T=4096)
    print("branched attention: 4 states x 4096 keys, 4 x 64 rows x 24 tokens", flush=True)
    out, lse = run_gpu(c)
    ref, ref_lse = run_oracle(c)
    st = assert_close_rel(out.float().cpu(), ref, what="4096-token-state row attention")
    print(st)
    assert (lse.cpu() - ref_lse).abs().max().item() <= 1e-4


def test_config4_row_attention_full_shape_sampled_rows(gpu_lib):
    T, R = 32768 + 2 * 256, 510
    c = make_case(seed=33, Ns=1, row_counts=[R], Hq=32, Hkv=8, t=12, D=128, T=T)
    print(f"branched attention: 1 state x {T} keys, {R} rows x 12 tokens", flush=True)
    out, lse = run_gpu(c)
    rows = torch.tensor([0, 1, 2, 63, 64, 127, 254, 255, 256, 300, 381, 447, 508, 509])
    sub = dict(c, q=c["q"][rows], k=c["k"][rows], v=c["v"][rows], row_counts=[len(rows)],
               row_state=torch.zeros(len(rows), dtype=torch.long))
    ref, ref_lse = run_oracle(sub)
    st = assert_close_rel(out.float().cpu()[rows], ref, what="32768-token-state row attention (sampled rows)")
    print(st)
    assert (lse.cpu()[rows] - ref_lse).abs().max().item() <= 1e-4


def test_config3_decision_full_size_properties(gpu_lib):
    from opendecider_amd import decoder as dmod
    cfg = dmod.DecoderConfig()  # 36 layers, 9B dims
    B, S, n_opt, t = 4, 4096, 64, 24
    dec = dmod.random_decoder(cfg, seed=0, device=DEV, max_pos=S + t + 16)
    dec.temperature = 24.0
    g = torch.Generator(device=DEV).manual_seed(3)
    ids_state = torch.randint(0, cfg.vocab, (B, S), generator=g, device=DEV)
    ids = torch.randint(0, cfg.vocab, (B, n_opt, t), generator=g, device=DEV)
    print(f"decision full size: {cfg.n_layers} layers, {B} x {S} prefill, {n_opt} x {t} options", flush=True)
    one = dec.new_state_caches(B, S)
    dec.prefill(ids_state, one)
    two = dec.new_state_caches(B, S)
    dec.prefill(ids_state[:, : S // 2].contiguous(), two)
    for j in range(S // 2, S, 256):  # appended records hold at most 256 tokens
        dec.prefill(ids_state[:, j: j + 256].contiguous(), two)
    torch.cuda.synchronize()
    h = S // 2
    assert torch.equal(one.q[..., :h, :], two.q[..., :h, :]) and torch.equal(one.scale[..., :h], two.scale[..., :h]), \
        "first-chunk K/V of some layer differ between one prefill and a prefill + records"
    assert torch.equal(one.q[:2], two.q[:2]) and torch.equal(one.scale[:2], two.scale[:2]), "layer-0 K/V differ"
    lp = dec.score(ids, one)
    lp2 = dec.score(ids, one)
    assert torch.isfinite(lp).all()
    assert torch.equal(lp, lp2), "two scoring passes differ"
    assert (lp.double().exp().sum(-1) - 1).abs().max().item() <= 1e-5
    perm = torch.randperm(n_opt, generator=torch.Generator().manual_seed(6)).to(DEV)
    lp_p = dec.score(ids[:, perm], one)
    d = (lp_p[:, :n_opt].exp() - lp[:, perm].exp()).abs().max().item()
    print(f"option permutation: max |dp| {d:.2e}")
    assert d <= 1e-6


def test_config4_wide_choice_full_size_properties(gpu_lib):
    from opendecider_amd import decoder as dmod
    cfg = dmod.DecoderConfig()
    S0, rec, n_opt, t = 32768, 128, 510, 12
    cap = S0 + 2 * rec
    dec = dmod.random_decoder(cfg, seed=1, device=DEV, max_pos=cap + t + 16)
    dec.temperature = 24.0
    g = torch.Generator(device=DEV).manual_seed(4)
    a = dec.new_state_caches(1, cap)
    for kc, vc in a:
        for c in (kc, vc):
            c.append(torch.randn(1, cfg.n_kv_heads, S0, cfg.head_dim, generator=g, device=DEV).to(torch.bfloat16))
    b = dec.new_state_caches(1, cap)
    b.q.copy_(a.q)
    b.scale.copy_(a.scale)
    b.set_length(S0)
    r1 = torch.randint(0, cfg.vocab, (1, rec), generator=g, device=DEV)
    r2 = torch.randint(0, cfg.vocab, (1, rec), generator=g, device=DEV)
    ids = torch.randint(0, cfg.vocab, (1, n_opt, t), generator=g, device=DEV)
    print(f"wide-choice full size: {S0}-token state + 2 x {rec}-token records (and as one), {n_opt} x {t} options",
          flush=True)
    dec.prefill(r1, a)
    dec.prefill(r2, a)
    dec.prefill(torch.cat([r1, r2], 1), b)
    torch.cuda.synchronize()
    assert a.length == b.length == cap
    assert torch.equal(a.q[:2], b.q[:2]) and torch.equal(a.scale[:2], b.scale[:2]), "layer-0 K/V differ"
    lp = dec.score(ids, a)
    assert torch.isfinite(lp).all()
    assert torch.equal(lp, dec.score(ids, a)), "two scoring passes differ"
    perm = torch.randperm(n_opt, generator=torch.Generator().manual_seed(7)).to(DEV)
    lp_p = dec.score(ids[:, perm], a)
    d = (lp_p[:, :n_opt].exp() - lp[:, perm].exp()).abs().max().item()
    print(f"option permutation: max |dp| {d:.2e}")
    assert d <= 1e-6
