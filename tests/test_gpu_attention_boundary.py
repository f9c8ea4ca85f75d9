"""GPU tests of the attention drop-in boundary as the reference calls it.

* `_split_attention` called exactly as `_forward` calls it (src/opendecider/prefix_attn.py:127): one state's prefix
  Kp/Vp (Hkv, T, D), a pad mask pm (T,), own k/v, the softmax scale, at head_dim 256 (Qwen3.5's full-attention
  heads; the reference dispatches D in {64, 128, 256}, prefix_attn.py:50), 16/4 and 8/2 heads, with the state as
  Int8Tensor and as dense bf16 (what shared_prefix_attention materializes, :145-149). Against the oracle's
  split_attention at the 2e-3 bar; the LSE of the same call through branched_attn within 1e-4.
* `split_attention_int8` with rows in any state order (the reference's `rows`, prefix_attn.py:103-117,152-154):
  interleaved row_state against the oracle (which takes row_state as it is), and equal bit for bit to the same rows
  grouped by state; with max_rows given (no host read) the same bits.
* od_branched_attn_stream with an understated max_rows: the state's outputs are NaN, not stale memory.
"""
import pytest
import torch

from helpers import assert_close_rel
from oracle import attention as oa
from oracle import quant as oq
from test_gpu_attention import make_case, run_oracle

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _int8_state(c):
    from opendecider_amd.quant import Int8Tensor
    Ki = Int8Tensor(c["kq"][0].to(DEV), c["ks"][0][..., None].to(DEV), torch.bfloat16)
    Vi = Int8Tensor(c["vq"][0].to(DEV), c["vs"][0][..., None].to(DEV), torch.bfloat16)
    return Ki, Vi


@pytest.mark.parametrize("n,Hq,Hkv,t,T", [(6, 16, 4, 8, 500), (5, 8, 2, 12, 257), (40, 16, 4, 16, 1024)])
def test_split_attention_d256_as_forward_calls_it(gpu_lib, n, Hq, Hkv, t, T):
    from opendecider_amd import kernels
    from opendecider_amd.prefix_attn import _split_attention
    D = 256
    c = make_case(seed=300 + n, Ns=1, row_counts=[n], Hq=Hq, Hkv=Hkv, t=t, D=D, T=T, holes=True)
    pm = c["kvalid"][0]
    Kp = oq.dequantize(c["kq"][0], c["ks"][0][..., None], torch.bfloat16)
    Vp = oq.dequantize(c["vq"][0], c["vs"][0][..., None], torch.bfloat16)
    ref, ref_lse = oa.split_attention(c["q"], c["k"], c["v"], Kp.float(), Vp.float(), pm, c["scale"])
    print(f"_split_attention D=256 n={n} Hq={Hq} Hkv={Hkv} t={t} T={T}", flush=True)
    q, k, v = c["q"].to(DEV), c["k"].to(DEV), c["v"].to(DEV)
    # dense bf16 prefix, as the reference's caller passes it
    out_d = _split_attention(q, k, v, Kp.to(DEV), Vp.to(DEV), pm.to(DEV), c["scale"])
    assert out_d.dtype == torch.bfloat16 and out_d.shape == (n, Hq, t, D)
    assert_close_rel(out_d.float().cpu(), ref, what="D=256 dense prefix")
    # the int8 state as Int8Tensor (read directly, bf16-materialized in the kernel)
    Ki, Vi = _int8_state(c)
    out_i = _split_attention(q, k, v, Ki, Vi, pm.to(DEV), c["scale"])
    assert_close_rel(out_i.float().cpu(), ref, what="D=256 Int8Tensor prefix")
    # the LSE of the merged softmax (the quantity the reference merges by, prefix_attn.py:74-76)
    _, lse = kernels.branched_attn(q, k, v, c["kq"].to(DEV), c["ks"].to(DEV), c["vq"].to(DEV), c["vs"].to(DEV),
                                   c["scale"], kvalid=pm[None].to(DEV), return_lse=True)
    _, lse_ref = run_oracle(c)
    assert (lse.cpu() - lse_ref).abs().max().item() <= 1e-4


@pytest.mark.parametrize("D,Hq,Hkv", [(128, 32, 8), (256, 16, 4)])
def test_split_attention_int8_rows_in_any_state_order(gpu_lib, D, Hq, Hkv):
    from opendecider_amd.prefix_attn import split_attention_int8
    Ns, counts, t, T = 3, [4, 2, 5], 6, 333
    c = make_case(seed=310 + D, Ns=Ns, row_counts=counts, Hq=Hq, Hkv=Hkv, t=t, D=D, T=T, holes=True)
    R = sum(counts)
    # an interleaving of the grouped rows: row j of the call is grouped row perm[j]
    perm = torch.randperm(R, generator=torch.Generator().manual_seed(D))
    row_state = c["row_state"][perm]
    assert not torch.equal(row_state, row_state.sort().values)
    q, k, v = c["q"][perm], c["k"][perm], c["v"][perm]
    ref, ref_lse = oa.branched_attention_int8(q, k, v, c["kq"], c["ks"], c["vq"], c["vs"], c["scale"], c["kvalid"],
                                              row_state, dequant="bf16")
    args = (c["kq"].to(DEV), c["ks"].to(DEV), c["vq"].to(DEV), c["vs"].to(DEV), c["kvalid"].to(DEV), c["scale"])
    print(f"split_attention_int8 row_state D={D} R={R} states={Ns}", flush=True)
    out, lse = split_attention_int8(q.to(DEV), k.to(DEV), v.to(DEV), *args, row_state=row_state.to(DEV),
                                    return_lse=True)
    assert_close_rel(out.float().cpu(), ref, what=f"row_state D={D}")
    assert (lse.cpu() - ref_lse).abs().max().item() <= 1e-4
    # the same rows grouped by state (row_counts) give the same bits, permuted
    out_g, lse_g = split_attention_int8(c["q"].to(DEV), c["k"].to(DEV), c["v"].to(DEV), *args, row_counts=counts,
                                        return_lse=True)
    assert torch.equal(out.view(torch.int16), out_g[perm.to(DEV)].view(torch.int16))
    assert torch.equal(lse, lse_g[perm.to(DEV)])
    # max_rows given: no host read, same bits
    out_m = split_attention_int8(q.to(DEV), k.to(DEV), v.to(DEV), *args, row_state=row_state.to(DEV),
                                 max_rows=max(counts))
    assert torch.equal(out_m.view(torch.int16), out.view(torch.int16))


def test_stream_understated_max_rows_gives_nan(gpu_lib):
    """od_branched_attn_stream sizes its waves from max_rows; a state with more rows than that (more than 32 slots
    per (state, head)) gets NaN outputs and LSEs, with and without key-range splits, while the other states'
    results stay correct. The kernel's own guard handles it in bounds (it writes only the rows row_start names)."""
    from opendecider_amd import kernels
    c = make_case(seed=320, Ns=2, row_counts=[2, 5], Hq=8, Hkv=2, t=2, D=128, T=900)
    rs, _ = kernels.row_start_of([2, 5], DEV)   # state 1 has 5 rows x 2 tokens x 4 heads = 40 slots
    ref, _ = run_oracle(c)
    for n_split in (1, 3):
        out, lse = kernels.branched_attn(c["q"].to(DEV), c["k"].to(DEV), c["v"].to(DEV), c["kq"].to(DEV),
                                         c["ks"].to(DEV), c["vq"].to(DEV), c["vs"].to(DEV), c["scale"],
                                         row_start=rs, max_rows=4, return_lse=True, n_split=n_split, stream=True)
        out, lse = out.float().cpu(), lse.cpu()
        assert torch.isnan(out[2:]).all() and torch.isnan(lse[2:]).all(), n_split
        assert_close_rel(out[:2], ref[:2], what=f"state 0 beside the understated state, split {n_split}")
