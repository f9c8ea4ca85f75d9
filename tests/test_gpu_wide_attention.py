"""GPU parity of wide_attention (od_wide_attn, flash attention over bf16 K/V) against the oracle.

Two oracles: oracle.attention.wide_attention_blocked restates the reference kernel's arithmetic step by step
(wide_attention.py:38-67: 64-key blocks, the running max, p rounded to bf16 before the P.V product), and
oracle.attention.attention is exact softmax attention. Against the blocked oracle the kernel is held to the path's
bar of 2e-3 relative (norm-wise over the tensor and over every (batch, head) slice) and, elementwise, to one bf16
step of the output plus the oracle's flip bound: p is rounded to bf16 inside the algorithm, and where the hardware
exp2 and the oracle's differ in the last bit that rounding can land on the neighbouring bf16 value, which moves an
output by at most 2^-7 sum_j p_j |v_j| / l. Its natural-log LSE to 1e-4 absolute against the exact one
(the LSE sums unrounded p), and to the reference test's own bar (max |out - exact| < 2e-2,
tests/test_wide_attention.py:38,62) against the exact one. Shapes: the reference test's four (Dk 448/200) with and
without padding (:19-20), its non-causal LSE case (:47-62), plus the decoder's head width 128 (causal prefill, a
causal offset S - T, GQA 4), 64, and Qwen3.5's 256 (Dk = Dv = 256, which runs as two 128-column halves, as the
reference's Dv = 256 shapes do).
"""
import pytest
import torch

from helpers import BF16_STEP, assert_close_rel
from oracle import attention as oa

pytestmark = pytest.mark.gpu
DEV = "cuda"

SHAPES = [(1, 16, 4, 100, 100, 448, 256), (2, 16, 4, 37, 300, 448, 256), (1, 16, 4, 1, 77, 448, 256),
          (2, 8, 2, 129, 129, 200, 128), (2, 32, 8, 256, 256, 128, 128), (1, 32, 8, 70, 1000, 128, 128),
          (2, 8, 8, 33, 70, 64, 64), (1, 8, 2, 130, 130, 128, 64), (1, 4, 4, 20, 90, 64, 256),
          # Qwen3.5's full-attention heads (16 / 4 x 256): a causal prefill and queries at the end of the keys
          (2, 16, 4, 300, 300, 256, 256), (1, 16, 4, 64, 500, 256, 256)]


def make(seed, B, H, G, T, S, DK, DV, padded):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, T, DK, generator=g).to(torch.bfloat16)
    k = torch.randn(B, G, S, DK, generator=g).to(torch.bfloat16)
    v = torch.randn(B, G, S, DV, generator=g).to(torch.bfloat16)
    kv = None
    if padded:
        kv = torch.ones(B, S, dtype=torch.bool)
        kv[-1, : S // 3] = False
    return q, k, v, kv


def check_vs_blocked(out, ob, bound, what):
    """Norm-relative 2e-3 (whole tensor, every slice along dim 0) and |out - ref| <= 2^-8 |ref| + bound."""
    B = out.shape[0]
    st = assert_close_rel(out, ob, what=what, elem_steps=10 ** 6)  # norm forms only; elementwise below
    bad = (out - ob).abs() > BF16_STEP * ob.abs() + bound + 1e-6
    assert not bad.any(), f"{what}: {int(bad.sum())} elements beyond one bf16 step + flip bound ({st})"


def run(q, k, v, kv, causal, return_lse=True):
    from opendecider_amd import wide_attention
    print(f"wide_attention q{tuple(q.shape)} k{tuple(k.shape)} v{tuple(v.shape)} causal={causal} "
          f"padded={kv is not None}", flush=True)
    r = wide_attention(q.to(DEV), k.to(DEV), v.to(DEV), q.shape[-1] ** -0.5, None if kv is None else kv.to(DEV),
                       causal=causal, return_lse=return_lse)
    torch.cuda.synchronize()
    return r


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("padded", [False, True])
def test_matches_oracle(shape, padded):
    B, H, G, T, S, DK, DV = shape
    q, k, v, kv = make(0, *shape, padded)
    out, lse = run(q, k, v, kv, causal=True)
    scale = DK ** -0.5
    ob, _, bound = oa.wide_attention_blocked(q, k, v, scale, kv, causal=True, with_bound=True)
    oe, le = oa.attention(q, k, v, scale, kv, causal=True)
    out, lse = out.float().cpu(), lse.cpu()
    vis = torch.isfinite(le)
    assert torch.equal(torch.isfinite(lse), vis)
    assert (lse[vis] - le[vis]).abs().max().item() < 1e-4
    assert (out - oe).abs().max().item() < 2e-2
    check_vs_blocked(out.reshape(B * H, T, DV), ob.reshape(B * H, T, DV), bound.reshape(B * H, T, DV),
                     "out vs blocked oracle")


def test_noncausal_lse():
    B, H, G, T, S, DK = 2, 16, 4, 50, 333, 448
    q, k, v, _ = make(1, B, H, G, T, S, DK, 256, False)
    kv = torch.ones(B, S, dtype=torch.bool)
    kv[0, :100] = False
    out, lse = run(q, k, v, kv, causal=False)
    oe, le = oa.attention(q, k, v, DK ** -0.5, kv, causal=False)
    ob, _, bound = oa.wide_attention_blocked(q, k, v, DK ** -0.5, kv, causal=False, with_bound=True)
    assert (out.float().cpu() - oe).abs().max().item() < 2e-2
    assert (lse.cpu() - le).abs().max().item() < 1e-4
    check_vs_blocked(out.float().cpu(), ob, bound, "non-causal out vs blocked oracle")


def test_empty_rows_and_no_lse():
    # every key of batch 1 masked: its queries return 0 and LSE -inf; return_lse=False returns the tensor alone
    q, k, v, _ = make(2, 2, 8, 2, 40, 90, 128, 128, False)
    kv = torch.ones(2, 90, dtype=torch.bool)
    kv[1] = False
    out, lse = run(q, k, v, kv, causal=True)
    assert torch.count_nonzero(out[1]).item() == 0
    assert torch.isinf(lse[1]).all() and (lse[1] < 0).all()
    out2 = run(q, k, v, kv, causal=True, return_lse=False)
    assert torch.equal(out2, out)


def test_head_order_and_batch_independence():
    # batch element b's result does not depend on the other batch elements (same inputs in both slots)
    q, k, v, _ = make(3, 1, 16, 4, 65, 200, 128, 128, False)
    q2, k2, v2 = (torch.cat([x, x]) for x in (q, k, v))
    out1, lse1 = run(q, k, v, None, causal=True)
    out2, lse2 = run(q2, k2, v2, None, causal=True)
    assert torch.equal(out2[0], out1[0]) and torch.equal(out2[1], out1[0])
    assert torch.equal(lse2[1], lse1[0])


def test_strided_inputs():
    # q/k/v as views of a packed (B, T, heads, D) projection output (non-contiguous head/token strides)
    g = torch.Generator().manual_seed(4)
    B, T, H, G, D = 2, 48, 8, 2, 128
    qkv = torch.randn(B, T, H + 2 * G, D, generator=g).to(torch.bfloat16).to(DEV)
    q = qkv[:, :, :H].transpose(1, 2)
    k = qkv[:, :, H:H + G].transpose(1, 2)
    v = qkv[:, :, H + G:].transpose(1, 2)
    from opendecider_amd import wide_attention
    out = wide_attention(q, k, v, D ** -0.5)
    ref = wide_attention(q.contiguous(), k.contiguous(), v.contiguous(), D ** -0.5)
    assert torch.equal(out, ref)


@pytest.mark.parametrize("B,H,G,T,S,D,DV,causal,padded", [
    (2, 16, 4, 200, 333, 128, 128, True, True), (1, 32, 8, 64, 700, 128, 128, False, False),
    (1, 8, 2, 130, 130, 128, 128, True, False), (2, 8, 2, 150, 300, 64, 128, True, True),
    (1, 16, 4, 100, 260, 256, 256, True, True), (1, 8, 2, 40, 200, 256, 128, False, False)])
def test_dma_path_matches_staged_path(B, H, G, T, S, D, DV, causal, padded):
    """Head widths 64, 128 and 256 with 128 value columns per pass (Dv = 256 in two halves) run on the LDS-DMA path
    (rows copied straight into LDS, V^T gathered with transposing LDS reads); head width D - 8 on the
    register-staged path, which pads it to D with zeros. With the last 8 dims of q and k zero both see the same
    scores and must agree bit for bit: the two paths share the arithmetic."""
    from opendecider_amd import wide_attention
    q, k, v, kv = make(11, B, H, G, T, S, D, DV, padded)
    q[..., D - 8:] = 0
    k[..., D - 8:] = 0
    q, k, v = q.to(DEV), k.to(DEV), v.to(DEV)
    kv = None if kv is None else kv.to(DEV)
    print(f"wide_attention DMA vs staged B={B} H={H} G={G} T={T} S={S} D={D} DV={DV} causal={causal} "
          f"padded={padded}", flush=True)
    out_dma, lse_dma = wide_attention(q, k, v, 0.125, kv, causal=causal, return_lse=True)
    out_st, lse_st = wide_attention(q[..., :D - 8].contiguous(), k[..., :D - 8].contiguous(), v, 0.125, kv,
                                    causal=causal, return_lse=True)
    assert torch.equal(out_dma.view(torch.int16), out_st.view(torch.int16))
    assert torch.equal(lse_dma, lse_st)


def test_scale_must_be_positive():
    q, k, v, _ = make(12, 1, 4, 2, 8, 8, 64, 64, False)
    from opendecider_amd import wide_attention
    for bad in (0.0, -0.125):
        with pytest.raises(ValueError):
            wide_attention(q.to(DEV), k.to(DEV), v.to(DEV), bad)
