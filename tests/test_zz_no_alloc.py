"""The allocation-free split attention (od_branched_attn_split_noalloc, through the C ABI) against the split with a
caller-owned workspace (od_branched_attn_split): the same bits on two calls in a row, the second smaller than the
first (the static scratch keeps the first call's partials, which the second must not read), and a request beyond the
scratch refused before any launch."""
import pytest
import torch

from test_gpu_attention import DEV, make_case

pytestmark = pytest.mark.gpu


def _both(c, n_split, dequant="bf16"):
    from opendecider_amd import kernels
    Ns = c["kq"].shape[0]
    args = (c["q"].to(DEV), c["k"].to(DEV), c["v"].to(DEV), c["kq"].to(DEV), c["ks"].to(DEV), c["vq"].to(DEV),
            c["vs"].to(DEV), c["scale"])
    kw = dict(kvalid=None if c["kvalid"] is None else c["kvalid"].to(DEV),
              row_counts=c["row_counts"] if Ns > 1 else None, length=c["T"], return_lse=True, n_split=n_split,
              dequant=dequant)
    ref = kernels.branched_attn(*args, staged=False, **kw)
    got = kernels.branched_attn(*args, static_workspace=True, **kw)
    return ref, got


def test_split_noalloc_equals_split_twice(gpu_lib):
    big = make_case(seed=91, Ns=2, row_counts=[3, 4], Hq=32, Hkv=8, t=16, D=128, T=3000, holes=True)
    small = make_case(seed=92, Ns=1, row_counts=[2], Hq=8, Hkv=2, t=5, D=64, T=500)
    for name, c, n_split, dq in (("big", big, 8, "bf16"), ("small", small, 3, "fp32")):
        print(f"noalloc {name} n_split={n_split}", flush=True)
        (o_ref, l_ref), (o, l) = _both(c, n_split, dq)
        torch.cuda.synchronize()
        assert torch.equal(o.view(torch.int16), o_ref.view(torch.int16)), name
        assert torch.equal(l, l_ref), name


def test_split_noalloc_refuses_more_than_its_scratch(gpu_lib):
    from opendecider_amd import _lib, kernels
    c = make_case(seed=93, Ns=1, row_counts=[64], Hq=32, Hkv=8, t=16, D=128, T=64)
    need = 256 * 64 * 32 * 16 * 129
    assert need > _lib.SPLIT_SCRATCH_FLOATS
    with pytest.raises(RuntimeError, match="static scratch"):
        kernels.branched_attn(c["q"].to(DEV), c["k"].to(DEV), c["v"].to(DEV), c["kq"].to(DEV), c["ks"].to(DEV),
                              c["vq"].to(DEV), c["vs"].to(DEV), c["scale"], length=64, n_split=256,
                              static_workspace=True)
