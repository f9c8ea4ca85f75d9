"""GPU parity of the KV-streaming branched attention (od_branched_attn_stream: at most 32 query slots per (state,
KV head), the int8 state streamed from memory into registers) against the oracle.

Bar, as for the block-image paths: outputs within 2e-3 relative of the oracle (the three forms in tests/helpers.py)
in both dequantization modes (the reference's bf16 materialize, quant.py:45 / prefix_attn.py:145-149, and the exact
fp32 q * s), natural-log LSE within 1e-4 absolute, option-row order invariance bitwise. Cases cover lengths that are
not a multiple of the 32-key tile, capacity past the length (garbage that must not be read), masked keys, states
without rows, a state of length 0 (own keys only), GQA 1..8, V scales over 17 binades, key-range splits from 1 to
more splits than tiles, and the few-slot probe shape at its full 32768-key length.
"""
import pytest
import torch

from helpers import assert_close_rel
from test_gpu_attention import make_case, run_oracle

pytestmark = pytest.mark.gpu
DEV = "cuda"

CASES = {
    # yes/no: 2 options x 2 tokens, 4 query heads per KV head: 16 slots per (state, head)
    "yes_no_T5000": dict(seed=21, Ns=4, row_counts=[2, 2, 2, 2], Hq=32, Hkv=8, t=2, D=128, T=5000),
    "one_row_8tok_holes": dict(seed=22, Ns=2, row_counts=[1, 1], Hq=32, Hkv=8, t=8, D=128, T=3000, holes=True),
    "ragged_rows_cap": dict(seed=23, Ns=3, row_counts=[3, 0, 1], Hq=8, Hkv=2, t=2, D=128, T=777, cap=900),
    "gqa1_t6": dict(seed=24, Ns=1, row_counts=[5], Hq=4, Hkv=4, t=6, D=128, T=100),
    "own_only_T0": dict(seed=25, Ns=1, row_counts=[2], Hq=8, Hkv=2, t=3, D=128, T=0),
    "v_frames_spread": dict(seed=26, Ns=2, row_counts=[2, 1], Hq=8, Hkv=2, t=4, D=128, T=1500, vspread=True),
    "t1_single_token": dict(seed=27, Ns=2, row_counts=[4, 3], Hq=8, Hkv=8, t=1, D=128, T=257),
    "short_state_T31": dict(seed=28, Ns=1, row_counts=[2], Hq=32, Hkv=8, t=4, D=128, T=31),
}


def run_stream(c, n_split=None, dequant="bf16", q=None, perm=None):
    from opendecider_amd import kernels
    Ns = c["kq"].shape[0]
    take = (lambda x: x) if perm is None else (lambda x: x[perm])
    return kernels.branched_attn(
        take(c["q"]).to(DEV) if q is None else q, take(c["k"]).to(DEV), take(c["v"]).to(DEV), c["kq"].to(DEV),
        c["ks"].to(DEV), c["vq"].to(DEV), c["vs"].to(DEV), c["scale"],
        kvalid=None if c["kvalid"] is None else c["kvalid"].to(DEV),
        row_counts=c["row_counts"] if Ns > 1 else None, length=c["T"], return_lse=True, n_split=n_split,
        stream=True, dequant=dequant)


@pytest.mark.parametrize("dequant", ["bf16", "fp32"])
@pytest.mark.parametrize("n_split", [1, 3, None])
@pytest.mark.parametrize("name", list(CASES))
def test_stream_matches_oracle(gpu_lib, name, n_split, dequant):
    c = make_case(**CASES[name])
    print(f"stream {name} n_split={n_split} {dequant}", flush=True)
    out, lse = run_stream(c, n_split=n_split, dequant=dequant)
    ref, ref_lse = run_oracle(c, dequant=dequant)
    assert_close_rel(out.float().cpu(), ref, what=f"stream {name} split {n_split} {dequant}")
    assert (lse.cpu() - ref_lse).abs().max().item() <= 1e-4


def test_stream_more_splits_than_tiles(gpu_lib):
    """Splits past the last tile get no keys (an empty partial, LSE -inf) and the merge ignores them."""
    c = make_case(**CASES["gqa1_t6"])
    out, lse = run_stream(c, n_split=9)  # 4 tiles of 32 keys
    ref, ref_lse = run_oracle(c)
    assert_close_rel(out.float().cpu(), ref, what="stream 9 splits over 4 tiles")
    assert (lse.cpu() - ref_lse).abs().max().item() <= 1e-4


def test_stream_option_order_invariance_bitwise(gpu_lib):
    """Shuffling the option rows of each state permutes the outputs and LSEs and changes nothing else, bit for bit."""
    c = make_case(seed=29, Ns=3, row_counts=[4, 2, 3], Hq=32, Hkv=8, t=2, D=128, T=2100, holes=True)
    perm = torch.tensor([2, 0, 3, 1, 5, 4, 8, 6, 7])
    for n_split in (1, 5):
        out, lse = run_stream(c, n_split=n_split)
        out_p, lse_p = run_stream(c, n_split=n_split, perm=perm)
        assert torch.equal(out_p.view(torch.int16), out[perm.to(DEV)].view(torch.int16)), n_split
        assert torch.equal(lse_p, lse[perm.to(DEV)]), n_split


def test_stream_is_the_default_for_few_slots(gpu_lib):
    """With no path chosen, a few-slot shape takes the streaming kernel: the default call equals stream=True bit for
    bit (and differs in path from the direct kernel, which is held to the same bar)."""
    from opendecider_amd import kernels
    c = make_case(**CASES["yes_no_T5000"])
    args = (c["q"].to(DEV), c["k"].to(DEV), c["v"].to(DEV), c["kq"].to(DEV), c["ks"].to(DEV), c["vq"].to(DEV),
            c["vs"].to(DEV), c["scale"])
    kw = dict(row_counts=c["row_counts"], length=c["T"], return_lse=True)
    out_a, lse_a = kernels.branched_attn(*args, **kw)
    out_s, lse_s = kernels.branched_attn(*args, stream=True, **kw)
    out_d, _ = kernels.branched_attn(*args, staged=False, **kw)
    assert torch.equal(out_a.view(torch.int16), out_s.view(torch.int16)) and torch.equal(lse_a, lse_s)
    ref, _ = run_oracle(c)
    assert_close_rel(out_d.float().cpu(), ref, what="direct path, same shape")


def test_stream_probe_full_length(gpu_lib):
    """The few-slot probe at full length: 32768-key int8 states, 2 options x 2 tokens, 32/8 heads (2 of the 8
    probe states, so that the oracle stays quick)."""
    c = make_case(seed=30, Ns=2, row_counts=[2, 2], Hq=32, Hkv=8, t=2, D=128, T=32768)
    out, lse = run_stream(c)
    ref, ref_lse = run_oracle(c)
    st = assert_close_rel(out.float().cpu(), ref, what="stream probe 32768")
    print(f"stream probe: {st}", flush=True)
    assert (lse.cpu() - ref_lse).abs().max().item() <= 1e-4


def test_stream_refuses_what_it_cannot_run(gpu_lib):
    """More than 32 slots per (state, head), or head_dim 64: refused before any launch."""
    from opendecider_amd import kernels
    c = make_case(seed=31, Ns=1, row_counts=[3], Hq=32, Hkv=8, t=4, D=128, T=64)  # 48 slots
    with pytest.raises(ValueError):
        run_stream(c)
    c = make_case(seed=32, Ns=1, row_counts=[1], Hq=8, Hkv=8, t=2, D=64, T=64)
    with pytest.raises(ValueError):
        run_stream(c)
    # 64 (state, head) pairs of 32768 keys on 256 CUs: 4 splits fill the CUs once; 48 pairs: 5 splits (240
    # workgroups), not 6 (288, a second round on 32 CUs); a short state keeps 16 tiles per split
    assert kernels.stream_split_count(8, 8, 32768) == 4
    assert kernels.stream_split_count(6, 8, 32768) == 5
    assert kernels.stream_split_count(1, 1, 1024) == 2


def test_split_attention_int8_few_rows_streams(gpu_lib):
    """The drop-in `_split_attention` with the reference caller's arguments (prefix_attn.py:127: q (n, Hq, t, D), own
    k/v (n, Hkv, t, D), the state Kp/Vp (Hkv, T, D) as Int8Tensor, a key mask pm (T,)) on a yes/no shape takes the
    streaming kernel and meets the bar against the oracle on the same int8 state."""
    from opendecider_amd.prefix_attn import _split_attention
    from opendecider_amd.quant import Int8Tensor
    g = torch.Generator().manual_seed(33)
    n, Hq, Hkv, t, D, T = 2, 32, 8, 2, 128, 4000
    src = torch.randn(2, Hkv, T, D, generator=g).to(torch.bfloat16)
    Kp, Vp = Int8Tensor.quantize(src[0].to(DEV)), Int8Tensor.quantize(src[1].to(DEV))
    pm = torch.ones(T, dtype=torch.bool)
    pm[:37] = False  # leading pads
    q = torch.randn(n, Hq, t, D, generator=g).to(torch.bfloat16)
    k = torch.randn(n, Hkv, t, D, generator=g).to(torch.bfloat16)
    v = torch.randn(n, Hkv, t, D, generator=g).to(torch.bfloat16)
    out = _split_attention(q.to(DEV), k.to(DEV), v.to(DEV), Kp, Vp, pm.to(DEV), D ** -0.5)
    c = dict(q=q, k=k, v=v, kq=Kp.q.cpu()[None], ks=Kp.scale.float().cpu().reshape(1, Hkv, T),
             vq=Vp.q.cpu()[None], vs=Vp.scale.float().cpu().reshape(1, Hkv, T), kvalid=pm[None],
             row_state=torch.zeros(n, dtype=torch.long), T=T, scale=D ** -0.5)
    ref, _ = run_oracle(c)
    assert_close_rel(out.float().cpu(), ref, what="_split_attention few rows (stream)")


def test_stream_fused_merge_repeats_and_replays(gpu_lib):
    """The split merge runs inside the kernel (the last split of a (state, head) to finish merges, then resets its
    counter): ten calls in a row on one workspace give the same bits (the counters return to zero every call), the
    workspace's counters are zero afterwards, a HIP graph of the call replays bit for bit with eager calls on other
    queries between the replays, and the result equals the oracle at the bar."""
    from opendecider_amd import kernels
    c = make_case(seed=33, Ns=4, row_counts=[2, 1, 2, 2], Hq=32, Hkv=8, t=2, D=128, T=4000, holes=True)
    ref, ref_lse = run_oracle(c)
    first, first_lse = run_stream(c, n_split=7)
    assert_close_rel(first.float().cpu(), ref, what="fused merge, 7 splits")
    assert (first_lse.cpu() - ref_lse).abs().max().item() <= 1e-4
    for _ in range(10):
        o, l = run_stream(c, n_split=7)
        assert torch.equal(o.view(torch.int16), first.view(torch.int16)) and torch.equal(l, first_lse)
    torch.cuda.synchronize()
    ws = kernels.stream_workspace(7, 7, 32, 2, 128, 4, 8, DEV)
    assert torch.count_nonzero(ws[-4 * 8:]).item() == 0
    # graph capture: the call recorded once, replayed with eager calls on other queries in between
    q = c["q"].to(DEV)
    args = (c["k"].to(DEV), c["v"].to(DEV), c["kq"].to(DEV), c["ks"].to(DEV), c["vq"].to(DEV), c["vs"].to(DEV),
            c["scale"])
    rs, mr = kernels.row_start_of(c["row_counts"], DEV)
    kw = dict(kvalid=c["kvalid"].to(DEV), row_start=rs, max_rows=mr, length=c["T"], n_split=7, stream=True)
    out = torch.empty_like(q)
    s_ = torch.cuda.Stream()
    with torch.cuda.stream(s_):
        kernels.branched_attn(q, *args, out=out, **kw)  # warm-up: the stream's workspace exists before the capture
        s_.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s_):
            kernels.branched_attn(q, *args, out=out, **kw)
    q2 = torch.randn(q.shape, device=DEV).to(torch.bfloat16)
    other = kernels.branched_attn(q2, *args, **kw)
    for i in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), first.view(torch.int16)), f"replay {i}"
        again = kernels.branched_attn(q2, *args, **kw)
        torch.cuda.synchronize()
        assert torch.equal(again.view(torch.int16), other.view(torch.int16)), f"eager call after replay {i}"
