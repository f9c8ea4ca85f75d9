"""GPU parity of the branched option-row attention (od_branched_attn) against the oracle.

Bar: outputs within 2e-3 relative of the oracle's fp32 result (the three forms in tests/helpers.py), natural-log LSE
within 1e-4 absolute, and option-row order invariance (outputs of permuted rows are the permuted outputs; required
<= 1e-6, checked bitwise). The staged path (od_attn_stage + od_branched_attn_staged, the default) and the direct path
(od_branched_attn, converting in every workgroup) must agree bit for bit. The default dequantization is the
reference's materialize (K/V = q.to(bf16) * s.to(bf16), quant.py:45, prefix_attn.py:145-149) and the oracle runs the
same; the exact fp32 dequantization (OD_DEQUANT_FP32) is held to the oracle's fp32 mode at the same bar.
"""
import pytest
import torch

from helpers import assert_close_rel
from oracle import attention as oa
from oracle import quant as oq

pytestmark = pytest.mark.gpu
DEV = "cuda"


def make_case(seed, Ns, row_counts, Hq, Hkv, t, D, T, cap=None, holes=False, vspread=False):
    g = torch.Generator().manual_seed(seed)
    R = sum(row_counts)
    cap = T if cap is None else cap
    kv_src = torch.randn(2, Ns, Hkv, T, D, generator=g)
    if vspread:  # the values of every 64-token block of the state times 2^u, u uniform in -10..6: the blocks' V frames
        # (the kernel's unit) spread over 17 binades, so consecutive blocks often differ by more than 3 binades
        u = torch.randint(-10, 7, (Ns, Hkv, -(-T // 64), 1, 1), generator=g).float()
        kv_src[1] *= torch.exp2(u).expand(-1, -1, -1, 64, 1).reshape(Ns, Hkv, -1, 1)[:, :, :T]
    kv_src = kv_src.to(torch.bfloat16)
    kq, ks = oq.quantize_rows(kv_src[0])
    vq, vs = oq.quantize_rows(kv_src[1])
    ks, vs = ks[..., 0], vs[..., 0]
    if cap > T:  # capacity beyond the filled length: garbage that must not be read
        pad = lambda x, v: torch.cat([x, torch.full((*x.shape[:2], cap - T, *x.shape[3:]), v, dtype=x.dtype)], 2)
        kq, vq, ks, vs = pad(kq, 99), pad(vq, -99), pad(ks, 1e3), pad(vs, 1e3)
    q = torch.randn(R, Hq, t, D, generator=g).to(torch.bfloat16)
    k = torch.randn(R, Hkv, t, D, generator=g).to(torch.bfloat16)
    v = torch.randn(R, Hkv, t, D, generator=g).to(torch.bfloat16)
    kvalid = None
    if holes:
        kvalid = torch.ones(Ns, T, dtype=torch.bool)
        kvalid[-1, : T // 3] = False
        kvalid[0, T // 2: T // 2 + 5] = False
    row_state = torch.repeat_interleave(torch.arange(Ns), torch.tensor(row_counts))
    return dict(q=q, k=k, v=v, kq=kq, ks=ks, vq=vq, vs=vs, kvalid=kvalid, row_counts=row_counts,
                row_state=row_state, T=T, scale=D ** -0.5)


def run_gpu(c, return_lse=True, q=None, n_split=None, staged=True, dequant="bf16"):
    from opendecider_amd import kernels
    Ns = c["kq"].shape[0]
    return kernels.branched_attn(
        c["q"].to(DEV) if q is None else q, c["k"].to(DEV), c["v"].to(DEV), c["kq"].to(DEV), c["ks"].to(DEV),
        c["vq"].to(DEV), c["vs"].to(DEV), c["scale"],
        kvalid=None if c["kvalid"] is None else c["kvalid"].to(DEV),
        row_counts=c["row_counts"] if Ns > 1 else None, length=c["T"], return_lse=return_lse, n_split=n_split,
        staged=staged, dequant=dequant)


def run_oracle(c, dequant="bf16"):
    T = c["T"]
    return oa.branched_attention_int8(c["q"], c["k"], c["v"], c["kq"][:, :, :T], c["ks"][:, :, :T],
                                      c["vq"][:, :, :T], c["vs"][:, :, :T], c["scale"], c["kvalid"], c["row_state"],
                                      dequant=dequant)


CASES = {
    "two_states_holes": dict(seed=1, Ns=2, row_counts=[3, 2], Hq=8, Hkv=2, t=5, D=128, T=100, holes=True),
    "own_two_chunks_d64": dict(seed=2, Ns=1, row_counts=[3], Hq=4, Hkv=4, t=40, D=64, T=64),
    "own_only_T0": dict(seed=3, Ns=1, row_counts=[2], Hq=4, Hkv=2, t=7, D=128, T=0),
    "gqa8_T130_cap200": dict(seed=4, Ns=1, row_counts=[5], Hq=32, Hkv=4, t=3, D=128, T=130, cap=200),
    "empty_state_group": dict(seed=5, Ns=3, row_counts=[2, 0, 3], Hq=8, Hkv=2, t=9, D=128, T=70),
    "t1_single_token_rows": dict(seed=6, Ns=2, row_counts=[4, 3], Hq=8, Hkv=8, t=1, D=64, T=257),
    "config4_like_t12": dict(seed=7, Ns=1, row_counts=[11], Hq=32, Hkv=8, t=12, D=128, T=300),
    # V scales over 17 binades: the accumulator's power-of-two frame moves up and down across the state blocks and
    # many blocks enter with their probabilities scaled by 2^-1..2^-3
    "v_frames_spread": dict(seed=8, Ns=2, row_counts=[3, 4], Hq=8, Hkv=2, t=6, D=128, T=700, vspread=True),
    # head_dim 256, Qwen3.5's full-attention heads (16 query / 4 KV heads), with key holes; and 8 / 2 heads with
    # rows longer than one 32-key own block
    "qwen35_d256_holes": dict(seed=13, Ns=2, row_counts=[3, 4], Hq=16, Hkv=4, t=6, D=256, T=300, holes=True),
    "d256_gqa4_own_two_chunks": dict(seed=14, Ns=1, row_counts=[5], Hq=8, Hkv=2, t=40, D=256, T=129),
    # rows of 300 tokens (10 own blocks, one slot tile spans a fraction of a row)
    "long_rows_t300": dict(seed=15, Ns=2, row_counts=[2, 1], Hq=8, Hkv=2, t=300, D=128, T=100),
}


@pytest.mark.parametrize("dequant", ["bf16", "fp32"])
@pytest.mark.parametrize("name", list(CASES))
def test_branched_attention_matches_oracle(gpu_lib, name, dequant):
    c = make_case(**CASES[name])
    out, lse = run_gpu(c, dequant=dequant)
    ref, ref_lse = run_oracle(c, dequant=dequant)
    st = assert_close_rel(out.float().cpu(), ref, what=f"{name} ({dequant})")
    dl = (lse.cpu() - ref_lse).abs().max().item()
    print(f"{name} ({dequant}): {st} lse max abs err {dl:.2e}")
    assert dl <= 1e-4


def test_all_prefix_keys_masked_gives_own_part(gpu_lib):
    """A state whose keys are all masked: the rows see only their own keys (wide_attention.py:62 rule)."""
    c = make_case(seed=8, Ns=1, row_counts=[3], Hq=4, Hkv=2, t=6, D=128, T=80)
    c["kvalid"] = torch.zeros(1, 80, dtype=torch.bool)
    out, _ = run_gpu(c)
    own, _ = oa.attention(c["q"], c["k"], c["v"], c["scale"], None, causal=True)
    assert_close_rel(out.float().cpu(), own, what="masked prefix")


def test_strided_query_view(gpu_lib):
    """q as the (R, t, Hq, D) projection viewed (R, Hq, t, D), the layout a fused QKV GEMM produces."""
    c = make_case(seed=9, Ns=1, row_counts=[4], Hq=8, Hkv=2, t=6, D=128, T=90)
    qv = c["q"].transpose(1, 2).contiguous().to(DEV).transpose(1, 2)
    assert not qv.is_contiguous()
    out_s, _ = run_gpu(c, q=qv)
    out_c, _ = run_gpu(c)
    assert torch.equal(out_s, out_c)


@pytest.mark.parametrize("vspread", [False, True])
def test_option_order_invariance_bitwise(gpu_lib, vspread):
    """Shuffling the option rows of each request permutes the outputs and changes nothing else (bitwise), also when
    the state's V frames spread over many binades (the accumulator's frame then moves between blocks)."""
    c = make_case(seed=10, Ns=4, row_counts=[8, 8, 8, 8], Hq=32, Hkv=8, t=16, D=128, T=256, vspread=vspread)
    if vspread:  # own values over a few binades too, so that the rows' own blocks take different frames
        g0 = torch.Generator().manual_seed(12)
        c["v"] = (c["v"].float() * torch.exp2(torch.randint(-6, 7, (32, 1, 1, 1), generator=g0).float())).bfloat16()
    g = torch.Generator().manual_seed(11)
    perm = torch.cat([torch.randperm(8, generator=g) + 8 * i for i in range(4)])
    for staged in (True, False):
        out, lse = run_gpu(c, staged=staged)
        cp = dict(c, q=c["q"][perm], k=c["k"][perm], v=c["v"][perm])
        out_p, lse_p = run_gpu(cp, staged=staged)
        assert torch.equal(out_p, out[perm.to(DEV)]), staged
        assert torch.equal(lse_p, lse[perm.to(DEV)]), staged


def test_config1_branched_attention_full_shape(gpu_lib):
    """8 requests; state S=2048 int8 K/V with per-token-per-head fp32 scales (source bf16 N(0,1)); 32 option rows of
    16 tokens per request; GQA 32 query / 8 KV heads; head_dim 128; no prefix mask; own tokens causal; LSE merge.
    Against the reference's arithmetic (the state materialized as q.to(bf16) * s.to(bf16), quant.py:45, then fp32
    attention, prefix_attn.py:58-76) at the 2e-3 bar in all three forms, and the fp32-dequant mode against the
    oracle's fp32 mode. Also reports the fraction of outputs whose bf16 value differs from the oracle's."""
    c = make_case(seed=1, Ns=8, row_counts=[32] * 8, Hq=32, Hkv=8, t=16, D=128, T=2048)
    for dequant in ("bf16", "fp32"):
        out, lse = run_gpu(c, dequant=dequant)
        ref, ref_lse = run_oracle(c, dequant=dequant)
        st = assert_close_rel(out.float().cpu(), ref, what=f"config1 ({dequant})")
        dl = (lse.cpu() - ref_lse).abs().max().item()
        flips = (out.cpu() != ref.to(torch.bfloat16)).float().mean().item()
        print(f"config1 ({dequant}): {st}, lse max abs err {dl:.2e}, bf16 outputs differing {flips:.4f}")
        assert dl <= 1e-4


# ---- key-range splits (od_branched_attn_split): the same result, merged by LSE

SPLIT_CASES = [("two_states_holes", 2), ("two_states_holes", 7), ("own_two_chunks_d64", 3), ("own_only_T0", 4),
               ("empty_state_group", 3), ("t1_single_token_rows", 5), ("config4_like_t12", 64),
               ("v_frames_spread", 5), ("qwen35_d256_holes", 4), ("long_rows_t300", 2)]


@pytest.mark.parametrize("name,n_split", SPLIT_CASES)
def test_split_matches_oracle(gpu_lib, name, n_split):
    """The state's 64-key blocks dealt to n_split workgroups (more splits than blocks leaves some empty; the own
    keys go to the last split), each split's normalized fp32 partial merged by LSE: the same bar as one pass."""
    c = make_case(**CASES[name])
    print(f"split {name} n_split={n_split}", flush=True)
    out, lse = run_gpu(c, n_split=n_split)
    ref, ref_lse = run_oracle(c)
    assert_close_rel(out.float().cpu(), ref, what=f"{name} split {n_split}")
    assert (lse.cpu() - ref_lse).abs().max().item() <= 1e-4


def test_split_long_state_auto(gpu_lib):
    """Few rows over a long state: the wrapper splits the keys by itself; result within the bar and order
    invariant (bitwise) under a shuffle of the rows."""
    from opendecider_amd import kernels
    c = make_case(seed=12, Ns=2, row_counts=[2, 2], Hq=32, Hkv=8, t=16, D=128, T=4096)
    tiles = -(-(2 * 16 * 4) // 128) * 8 * 2
    assert kernels.split_count(tiles, 4096) > 1
    out, lse = run_gpu(c)
    ref, ref_lse = run_oracle(c)
    assert_close_rel(out.float().cpu(), ref, what="long state auto split")
    assert (lse.cpu() - ref_lse).abs().max().item() <= 1e-4
    perm = torch.tensor([1, 0, 3, 2])
    cp = dict(c, q=c["q"][perm], k=c["k"][perm], v=c["v"][perm])
    out_p, lse_p = run_gpu(cp)
    assert torch.equal(out_p, out[perm.to(DEV)]) and torch.equal(lse_p, lse[perm.to(DEV)])


# ---- staged block images (od_attn_stage + od_branched_attn_staged) against the direct path: the same bits

@pytest.mark.parametrize("name", list(CASES))
def test_staged_equals_direct_bitwise(gpu_lib, name):
    """Both paths build the same block images (one in memory, one in each workgroup's LDS), so outputs and LSE
    agree bit for bit, with and without a key-range split."""
    c = make_case(**CASES[name])
    print(f"staged vs direct {name}", flush=True)
    for n_split, dequant in ((1, "bf16"), (3, "bf16"), (1, "fp32"), (3, "fp32")):
        out_s, lse_s = run_gpu(c, n_split=n_split, staged=True, dequant=dequant)
        out_d, lse_d = run_gpu(c, n_split=n_split, staged=False, dequant=dequant)
        assert torch.equal(out_s.view(torch.int16), out_d.view(torch.int16)), (name, n_split, dequant)
        assert torch.equal(lse_s, lse_d), (name, n_split, dequant)


def test_stage_size_and_errors(gpu_lib):
    """od_attn_stage_size follows Ns * Hkv * ceil(T / 64) * (4 * 64 * D + 528); a too-small image is refused."""
    import ctypes
    from opendecider_amd._lib import lib, check
    n = ctypes.c_int64(0)
    assert lib().od_attn_stage_size(3, 2, 130, 128, ctypes.byref(n)) == 0
    assert n.value == 3 * 2 * 3 * (4 * 64 * 128 + 528)
    assert lib().od_attn_stage_size(1, 1, 64, 64, ctypes.byref(n)) == 0 and n.value == 4 * 64 * 64 + 528
    assert lib().od_attn_stage_size(1, 1, 64, 96, ctypes.byref(n)) != 0
    kq = torch.zeros(1, 1, 64, 128, dtype=torch.int8, device=DEV)
    ks = torch.ones(1, 1, 64, device=DEV)
    img = torch.empty(100, dtype=torch.uint8, device=DEV)
    rc = lib().od_attn_stage(kq.data_ptr(), ks.data_ptr(), kq.data_ptr(), ks.data_ptr(), None, 1, 1, 64, 64, 128,
                             0.125, 0, img.data_ptr(), img.numel(), torch.cuda.current_stream().cuda_stream)
    with pytest.raises(RuntimeError):
        check(rc, "od_attn_stage")
    big = torch.empty(4 * 64 * 128 + 528, dtype=torch.uint8, device=DEV)
    rc = lib().od_attn_stage(kq.data_ptr(), ks.data_ptr(), kq.data_ptr(), ks.data_ptr(), None, 1, 1, 64, 64, 128,
                             0.125, 7, big.data_ptr(), big.numel(), torch.cuda.current_stream().cuda_stream)
    assert rc == -4  # an unknown dequantization is refused


# ---- the reference caller's own arguments: dense bf16 Kp/Vp (prefix_attn.py:127, fed from :145-149)

@pytest.mark.parametrize("n,Hq,Hkv,t,D,T,mask", [(5, 8, 2, 6, 128, 300, True), (3, 4, 4, 17, 64, 129, False),
                                                 (32, 32, 8, 16, 128, 2048, False), (6, 16, 4, 9, 256, 300, True),
                                                 (4, 8, 2, 33, 256, 140, True)])
def test_split_attention_dense_prefix(gpu_lib, n, Hq, Hkv, t, D, T, mask):
    """_split_attention called exactly as the reference's _forward calls it: the state K/V materialized to dense bf16
    (q.to(bf16) * s.to(bf16)), a key mask pm (T,), own k/v, the softmax scale; against the oracle's
    split_attention at the 2e-3 bar. The Int8Tensor call of the same state gives the same result to the bar."""
    from opendecider_amd.prefix_attn import _split_attention
    from opendecider_amd.quant import Int8Tensor
    c = make_case(seed=40 + n, Ns=1, row_counts=[n], Hq=Hq, Hkv=Hkv, t=t, D=D, T=T, holes=mask)
    Kp = oq.dequantize(c["kq"][0], c["ks"][0][..., None], torch.bfloat16)
    Vp = oq.dequantize(c["vq"][0], c["vs"][0][..., None], torch.bfloat16)
    pm = None if c["kvalid"] is None else c["kvalid"][0]
    print(f"dense _split_attention n={n} Hq={Hq} Hkv={Hkv} t={t} D={D} T={T}", flush=True)
    out = _split_attention(c["q"].to(DEV), c["k"].to(DEV), c["v"].to(DEV), Kp.to(DEV), Vp.to(DEV),
                           None if pm is None else pm.to(DEV), c["scale"])
    assert out.dtype == torch.bfloat16 and out.shape == (n, Hq, t, D)
    ref, _ = oa.split_attention(c["q"], c["k"], c["v"], Kp.float(), Vp.float(), pm, c["scale"])
    assert_close_rel(out.float().cpu(), ref, what="dense prefix")
    Ki = Int8Tensor(c["kq"][0].to(DEV), c["ks"][0][..., None].to(DEV), torch.bfloat16)
    Vi = Int8Tensor(c["vq"][0].to(DEV), c["vs"][0][..., None].to(DEV), torch.bfloat16)
    out_i = _split_attention(c["q"].to(DEV), c["k"].to(DEV), c["v"].to(DEV), Ki, Vi,
                             None if pm is None else pm.to(DEV), c["scale"])
    assert_close_rel(out_i.float().cpu(), ref, what="int8 prefix")


# ---- two-level prefix (the question cache): state blocks, then the question's own K/V, then the row's tokens

TWO_LEVEL = [
    dict(seed=61, Ns=2, counts=[2, 0, 3], Hq=8, Hkv=2, t=5, D=128, T=200, T2=70),
    dict(seed=62, Ns=1, counts=[4, 3], Hq=32, Hkv=8, t=16, D=128, T=2048, T2=130),
    dict(seed=63, Ns=3, counts=[1, 2, 1, 3], Hq=4, Hkv=4, t=9, D=64, T=0, T2=40),
    dict(seed=64, Ns=2, counts=[3, 5], Hq=16, Hkv=4, t=12, D=128, T=300, T2=256),
    dict(seed=65, Ns=2, counts=[3, 2], Hq=16, Hkv=4, t=7, D=256, T=200, T2=90),
]


def _two_level_case(seed, Ns, counts, Hq, Hkv, t, D, T, T2):
    g = torch.Generator().manual_seed(seed)
    G, R = len(counts), sum(counts)
    c = make_case(seed=seed, Ns=Ns, row_counts=[R] + [0] * (Ns - 1), Hq=Hq, Hkv=Hkv, t=t, D=D, T=T)
    kq2 = torch.randn(G, Hkv, T2, D, generator=g).to(torch.bfloat16)
    vq2 = torch.randn(G, Hkv, T2, D, generator=g).to(torch.bfloat16)
    lens = torch.randint(1, T2 + 1, (G,), generator=g) if T2 > 0 else torch.zeros(G, dtype=torch.long)
    qmask = torch.arange(T2)[None, :] < lens[:, None]  # each question's K/V right-padded to T2
    group_state = torch.randint(0, Ns, (G,), generator=g, dtype=torch.int32)
    row_group = torch.repeat_interleave(torch.arange(G), torch.tensor(counts))
    return c, kq2, vq2, qmask, group_state, row_group


def _run_two_level(c, kq2, vq2, qmask, group_state, counts, T, T2, n_split=None, q=None):
    from opendecider_amd import kernels
    img = kernels.stage_state(c["kq"].to(DEV), c["ks"].to(DEV), c["vq"].to(DEV), c["vs"].to(DEV), T, c["scale"]) \
        if T > 0 else None
    img2 = kernels.stage_state_bf16(kq2.to(DEV), vq2.to(DEV), T2, c["scale"], qmask.to(torch.uint8).to(DEV)) \
        if T2 > 0 else None
    rs, mr = kernels.row_start_of(counts, DEV)
    return kernels.branched_attn_two_level(c["q"].to(DEV) if q is None else q, c["k"].to(DEV), c["v"].to(DEV), img,
                                           c["kq"].shape[0], T, img2, T2, c["scale"],
                                           group_state=group_state.to(DEV), row_start=rs, max_rows=mr,
                                           return_lse=True, n_split=n_split)


@pytest.mark.parametrize("case", TWO_LEVEL, ids=lambda c: f"Ns{c['Ns']}-G{len(c['counts'])}-T{c['T']}-T2{c['T2']}")
def test_two_level_prefix_matches_oracle(gpu_lib, case):
    """Rows of question g attend [state group_state[g] (int8, bf16-materialized) ; question g's dense K/V (right
    pads masked)] and their own tokens causally (prefix_attn.py:94-99 + _split_attention): against the oracle at the
    2e-3 bar, one pass and split; option order inside a group is bitwise invariant."""
    c, kq2, vq2, qmask, gs, rg = _two_level_case(**case)
    T, T2, counts = case["T"], case["T2"], case["counts"]
    print(f"two-level {case}", flush=True)
    ref, ref_lse = oa.two_level_attention(c["q"], c["k"], c["v"], c["kq"], c["ks"], c["vq"], c["vs"], kq2, vq2,
                                          qmask, c["scale"], rg, gs)
    for n_split in (1, 3):
        out, lse = _run_two_level(c, kq2, vq2, qmask, gs, counts, T, T2, n_split=n_split)
        assert_close_rel(out.float().cpu(), ref, what=f"two-level split {n_split}")
        assert (lse.cpu() - ref_lse).abs().max().item() <= 1e-4
    # shuffle the rows inside every group: outputs permute bitwise
    g = torch.Generator().manual_seed(case["seed"] + 1)
    starts = [0]
    for n in counts:
        starts.append(starts[-1] + n)
    perm = torch.cat([torch.randperm(n, generator=g) + s for n, s in zip(counts, starts)])
    cp = dict(c, q=c["q"][perm], k=c["k"][perm], v=c["v"][perm])
    out_p, _ = _run_two_level(cp, kq2, vq2, qmask, gs, counts, T, T2, n_split=1)
    out1, _ = _run_two_level(c, kq2, vq2, qmask, gs, counts, T, T2, n_split=1)
    assert torch.equal(out_p, out1[perm.to(DEV)])


def test_two_level_without_questions_equals_one_level(gpu_lib):
    """T2 = 0 and group g reading state g: the same bits as od_branched_attn_staged over the same images."""
    from opendecider_amd import kernels
    c = make_case(seed=66, Ns=2, row_counts=[3, 4], Hq=8, Hkv=2, t=6, D=128, T=260)
    ref, ref_lse = run_gpu(c, staged=True, n_split=1)
    out, lse = _run_two_level(c, None, None, None, torch.arange(2, dtype=torch.int32), [3, 4], 260, 0, n_split=1)
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16)) and torch.equal(lse, ref_lse)
