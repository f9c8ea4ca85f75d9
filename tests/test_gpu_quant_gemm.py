"""GPU parity of the quantizers and the W8A8 GEMM against the oracle (bit-exact bytes, scales and int32 accumulators;
bit-exact bf16 epilogue, which runs the oracle's fp32 operations in the same order)."""
import pytest
import torch

from oracle import decoder as od
from oracle import quant as oq

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _x(g, M, K, outliers=0.01, scale=1.0):
    x = torch.randn(M, K, generator=g) * scale
    n_out = max(1, int(round(outliers * K))) if outliers else 0
    if n_out:
        x[:, torch.randperm(K, generator=g)[:n_out]] *= 20
    return x.to(torch.bfloat16)


@pytest.mark.parametrize("M,K", [(1, 8), (5, 64), (33, 128), (17, 200), (7, 37), (64, 4096), (3, 12288), (300, 520)])
@pytest.mark.parametrize("smooth", [False, True])
def test_act_quant_bit_exact(gpu_lib, M, K, smooth):
    from opendecider_amd import kernels
    g = torch.Generator().manual_seed(M * 1000 + K)
    x = _x(g, M, K)
    if M > 2:
        x[1] = 0                                          # all-zero row: clamp_min(1e-8)
    inv = (1.0 / (torch.rand(K, generator=g) * 1.5 + 0.5)).to(torch.bfloat16) if smooth else None
    xq, sx = kernels.act_quant(x.to(DEV), None if inv is None else inv.to(DEV))
    rq, rs = oq.act_quant(x, inv)
    assert torch.equal(xq.cpu(), rq)
    assert torch.equal(sx.cpu(), rs)


def test_act_quant_strided_rows_and_padding(gpu_lib):
    from opendecider_amd import kernels
    g = torch.Generator().manual_seed(1)
    big = _x(g, 40, 96)
    x = big[:, 16:80]                                     # row stride 96, K = 64
    xd = big.to(DEV)[:, 16:80]
    assert xd.stride(0) == 96
    xq, sx = kernels.act_quant(xd, None, ld=80)
    rq, rs = oq.act_quant(x)
    assert torch.equal(xq[:, :64].cpu(), rq) and torch.equal(sx.cpu(), rs)
    assert (xq[:, 64:] == 0).all()


@pytest.mark.parametrize("B,H,n,D,n0,cap", [(1, 8, 256, 128, 0, 256), (2, 8, 37, 128, 100, 200), (3, 2, 5, 64, 7, 12),
                                            (1, 4, 9, 256, 0, 9), (2, 3, 4, 40, 1, 6)])
def test_kv_quant_append_bytes(gpu_lib, B, H, n, D, n0, cap):
    from opendecider_amd import kernels
    g = torch.Generator().manual_seed(B + H + n + D)
    x = torch.randn(B, H, n, D, generator=g).to(torch.bfloat16)
    qc = torch.zeros(B, H, cap, D, dtype=torch.int8, device=DEV)
    sc = torch.zeros(B, H, cap, dtype=torch.float32, device=DEV)
    kernels.kv_quant_append(x.to(DEV), qc, sc, n0)
    rq, rs = oq.quantize_rows(x)
    assert torch.equal(qc[:, :, n0:n0 + n].cpu(), rq)
    assert torch.equal(sc[:, :, n0:n0 + n].cpu(), rs[..., 0])
    assert (qc[:, :, :n0] == 0).all() and (qc[:, :, n0 + n:] == 0).all() and (sc[:, :, n0 + n:] == 0).all()


def test_kv_append_strided_input_equals_whole(gpu_lib):
    """(B, T, H, D) projections viewed as (B, H, T, D): two appends == quantizing the whole tensor."""
    from opendecider_amd import kernels
    g = torch.Generator().manual_seed(2)
    x = torch.randn(2, 50, 4, 128, generator=g).to(torch.bfloat16)      # (B, T, H, D)
    xv = x.to(DEV).transpose(1, 2)                                       # (B, H, T, D) view
    qc = torch.zeros(2, 4, 64, 128, dtype=torch.int8, device=DEV)
    sc = torch.zeros(2, 4, 64, dtype=torch.float32, device=DEV)
    kernels.kv_quant_append(xv[:, :, :30], qc, sc, 0)
    kernels.kv_quant_append(xv[:, :, 30:], qc, sc, 30)
    rq, rs = oq.quantize_rows(x.transpose(1, 2))
    assert torch.equal(qc[:, :, :50].cpu(), rq) and torch.equal(sc[:, :, :50].cpu(), rs[..., 0])


def _gemm_case(g, M, N, K):
    a = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8)
    w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    sa = torch.rand(M, generator=g) * 0.05 + 1e-3
    sw = torch.rand(N, generator=g) * 1.5e-3 + 0.5e-3
    return a, w, sa, sw


@pytest.mark.parametrize("M,N,K", [(1, 16, 16), (7, 33, 48), (256, 256, 128), (300, 200, 208), (64, 6144, 512),
                                   (513, 4097, 1040), (256, 4096, 4096)])
def test_gemm_int32_accumulators_bit_exact(gpu_lib, M, N, K):
    from opendecider_amd import kernels
    g = torch.Generator().manual_seed(M + N + K)
    a, w, sa, sw = _gemm_case(g, M, N, K)
    out, acc = kernels.w8a8_gemm(a.to(DEV), sa.to(DEV), w.to(DEV), sw.to(DEV), want_acc=True)
    ref_acc = oq.int_gemm(a, w)
    assert torch.equal(acc.cpu(), ref_acc)
    ref_out = oq.w8a8_epilogue(ref_acc, sa, sw)
    assert torch.equal(out.cpu(), ref_out)
    # without the accumulator output small M (<= 512 rows) takes the small-M kernel: the same bits
    assert torch.equal(kernels.w8a8_gemm(a.to(DEV), sa.to(DEV), w.to(DEV), sw.to(DEV)).cpu(), ref_out)


def test_gemm_extreme_accumulators(gpu_lib):
    """+-127 everywhere at K = 12288: the largest |acc| the 9B shapes reach (1.98e8) stays exact."""
    from opendecider_amd import kernels
    M, N, K = 64, 64, 12288
    a = torch.full((M, K), 127, dtype=torch.int8)
    a[1::2] = -127
    w = torch.full((N, K), 127, dtype=torch.int8)
    _, acc = kernels.w8a8_gemm(a.to(DEV), torch.ones(M, device=DEV), w.to(DEV), torch.ones(N, device=DEV),
                               want_acc=True)
    assert torch.equal(acc.cpu(), oq.int_gemm(a, w))
    assert acc[0, 0].item() == 127 * 127 * K and acc[1, 0].item() == -127 * 127 * K


def test_gemm_bias_residual_epilogue(gpu_lib):
    from opendecider_amd import kernels
    g = torch.Generator().manual_seed(3)
    M, N, K = 130, 96, 256
    a, w, sa, sw = _gemm_case(g, M, N, K)
    bias = torch.randn(N, generator=g).to(torch.bfloat16)
    res = torch.randn(M, N, generator=g).to(torch.bfloat16)
    out = kernels.w8a8_gemm(a.to(DEV), sa.to(DEV), w.to(DEV), sw.to(DEV), bias.to(DEV), res.to(DEV))
    assert torch.equal(out.cpu(), oq.w8a8_epilogue(oq.int_gemm(a, w), sa, sw, bias, res))


@pytest.mark.parametrize("M,N,K,with_bias", [(1100, 16384, 128, False), (300, 712, 128, True)])
def test_gemm_wide_epilogue_equals_narrow_epilogue(gpu_lib, M, N, K, with_bias):
    """The wide epilogue (N % 8 == 0, 16-byte aligned scale vectors and rows: the tile's scales staged in LDS, stores
    through a buffer descriptor whose range drops rows past M) against the same GEMM with scale vectors 4 bytes off
    16-byte alignment, which takes the 4-column epilogue: the same bytes, and the oracle's on a sample of rows.
    M = 1100 and N = 16384 make 320 tiles, so some workgroups run two (the scale slots alternate), and the last tile
    row is ragged (76 of 256 rows); N = 712 leaves the last tile column ragged (200 of 256 columns), with a bias."""
    from opendecider_amd import kernels
    g = torch.Generator().manual_seed(11 + M)
    a, w, sa, sw = _gemm_case(g, M, N, K)
    res = torch.randn(M, N, generator=g).to(torch.bfloat16)
    bias = torch.randn(N, generator=g).to(torch.bfloat16) if with_bias else None
    A, W, R = a.to(DEV), w.to(DEV), res.to(DEV)
    Bd = None if bias is None else bias.to(DEV)
    out_w = kernels.w8a8_gemm(A, sa.to(DEV), W, sw.to(DEV), bias=Bd, residual=R)
    sab = torch.zeros(M + 1, device=DEV)
    swb = torch.zeros(N + 1, device=DEV)
    sab[1:] = sa.to(DEV)
    swb[1:] = sw.to(DEV)
    assert sab[1:].data_ptr() % 16 != 0 and swb[1:].data_ptr() % 16 != 0
    out_n = kernels.w8a8_gemm(A, sab[1:], W, swb[1:], bias=Bd, residual=R)
    assert torch.equal(out_w, out_n)
    rows = torch.tensor(sorted({0, 1, 255, 256, 511, 1023, 1024, M - 1} & set(range(M))))
    ref = oq.w8a8_epilogue(oq.int_gemm(a[rows], w), sa[rows], sw, bias, res[rows])
    assert torch.equal(out_w.cpu()[rows], ref)


@pytest.mark.parametrize("M,N,K,epi", [(2048, 2048, 3072, "res"), (2000, 2040, 4096, "bias_res"),
                                       (1024, 4096, 4096, "swiglu"), (512, 6144, 2048, "res"),
                                       (1024, 2048, 128, "bias_res"), (1536, 4096, 1024, "res"),
                                       (1536, 4096, 2048, "swiglu")])
def test_gemm_128x128_tiles_equal_larger_tiles(gpu_lib, M, N, K, epi):
    """Mid-size M x N with a bf16 output through the wide epilogue take 128 x 128 tiles (up to two per CU). Up to one
    tile per CU and K >= 3072 they run on the 4-stage ring (one workgroup per CU): 2048 x 2048; 2000 x 2040 with the
    last tile row (80 of 128 rows) and column (120 of 128 columns) ragged; SwiGLU at F = 2048. Otherwise on 2
    stages: one tile per CU at K = 2048 and 128; 384 tiles, two workgroups on most CUs, at 1536 x 4096 and SwiGLU at
    1536 x 2048. The same GEMM with scale vectors 4 bytes off 16-byte alignment takes the 4-column epilogue on the
    larger tiles: the same bytes, and the oracle's on a sample of rows."""
    from opendecider_amd import kernels
    g = torch.Generator().manual_seed(M + N + K)
    a, w, sa, sw = _gemm_case(g, M, N, K)
    bias = torch.randn(N, generator=g).to(torch.bfloat16) if "bias" in epi else None
    res = torch.randn(M, N, generator=g).to(torch.bfloat16) if "res" in epi else None
    A, W = a.to(DEV), w.to(DEV)
    Bd = None if bias is None else bias.to(DEV)
    R = None if res is None else res.to(DEV)
    sab = torch.zeros(M + 1, device=DEV)
    swb = torch.zeros(N + 1, device=DEV)
    sab[1:] = sa.to(DEV)
    swb[1:] = sw.to(DEV)
    assert sab[1:].data_ptr() % 16 != 0 and swb[1:].data_ptr() % 16 != 0
    print(f"128x128 tiles M={M} N={N} K={K} {epi}", flush=True)
    if epi == "swiglu":
        assert kernels.splitk_workspace(M, N, K, DEV) is None
        out_w = kernels.w8a8_gemm_swiglu(A, sa.to(DEV), W, sw.to(DEV))
        out_n = kernels.w8a8_gemm_swiglu(A, sab[1:], W, swb[1:])
        assert torch.equal(out_w.view(torch.int16), out_n.view(torch.int16))
        gu = oq.w8a8_epilogue(oq.int_gemm(a[:64], w), sa[:64], sw)
        ref = od.swiglu(gu[:, torch.cat([torch.arange(0, N, 2), torch.arange(1, N, 2)])], N // 2).float()
        d = (out_w[:64].cpu().float() - ref).abs()
        assert (d <= ref.abs() * 2.0 ** -6 + 2.0 ** -120).all() and (d > 0).float().mean().item() <= 5e-3
        return
    out_w = kernels.w8a8_gemm(A, sa.to(DEV), W, sw.to(DEV), bias=Bd, residual=R)
    out_n = kernels.w8a8_gemm(A, sab[1:], W, swb[1:], bias=Bd, residual=R)
    assert torch.equal(out_w.view(torch.int16), out_n.view(torch.int16))
    rows = torch.tensor(sorted({0, 1, 127, 128, 1023, 1024, 1920, M - 1} & set(range(M))))
    ref = oq.w8a8_epilogue(oq.int_gemm(a[rows], w), sa[rows], sw, bias, None if res is None else res[rows])
    assert torch.equal(out_w.cpu()[rows], ref)


def test_config0_single_w8a8_linear(gpu_lib):
    """X bf16 [256,4096] N(0,1) with 1% outlier channels x20, per-token int8; W int8 [4096,4096] uniform in
    [-127,127]; per-channel fp32 scales U(0.5e-3, 2e-3); int32 accumulators compared exactly."""
    from opendecider_amd import kernels
    g = torch.Generator().manual_seed(0)
    x = _x(g, 256, 4096)
    w = torch.randint(-127, 128, (4096, 4096), generator=g, dtype=torch.int8)
    sw = torch.rand(4096, generator=g) * 1.5e-3 + 0.5e-3
    xq, sx = kernels.act_quant(x.to(DEV))
    out, acc = kernels.w8a8_gemm(xq, sx, w.to(DEV), sw.to(DEV), want_acc=True)
    rout, racc, rxq, rsx = oq.w8a8_linear(x, w, sw)
    assert torch.equal(xq.cpu(), rxq) and torch.equal(sx.cpu(), rsx)
    assert torch.equal(acc.cpu(), racc)
    assert torch.equal(out.cpu(), rout)
    # the path the linear takes (no accumulator output: the small-M kernel at M = 256)
    assert torch.equal(kernels.w8a8_gemm(xq, sx, w.to(DEV), sw.to(DEV)).cpu(), rout)


def test_w8a8_linear_module_smoothquant(gpu_lib):
    """W8A8Linear.from_linear with a SmoothQuant fold == the oracle's W8A8 linear on the same weights."""
    from opendecider_amd.quant import SmoothedLinear, W8A8Linear, smooth_a8w8_
    g = torch.Generator().manual_seed(4)
    K, N = 512, 384
    lin = torch.nn.Linear(K, N, bias=True).to(torch.bfloat16)
    with torch.no_grad():
        lin.weight.copy_((torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16))
    s = torch.rand(K, generator=g) * 1.5 + 0.5
    x = _x(g, 3 * 41, K).view(3, 41, K)
    net = torch.nn.Sequential(lin).to(DEV)
    smooth_a8w8_(net, {"0": s})
    assert isinstance(net[0], SmoothedLinear) and isinstance(net[0].inner, W8A8Linear)
    y = net(x.to(DEV))
    wq, sw = oq.quantize_weight(oq.smooth_fold(lin.weight.data.cpu(), s))
    inv = net[0].inner.inv_s.cpu()
    # bf16(1/s): the GPU reciprocal may differ from the CPU one by one bf16 step on rare ties
    assert ((inv.float() - oq.smooth_inv(s).float()).abs() <= inv.float().abs() * 2.0 ** -7).all()
    ref, _, _, _ = oq.w8a8_linear(x.reshape(-1, K), wq, sw, lin.bias.data.cpu(), inv)
    assert torch.equal(net[0].inner.qweight.cpu(), wq)
    assert torch.equal(net[0].inner.w_scale.cpu(), sw)
    assert torch.equal(y.reshape(-1, N).cpu(), ref)


def test_fused_kernels_keep_module_objects_and_hooks(gpu_lib):
    """Restates the reference's test_fused_kernels_keep_module_objects_and_hooks (test_int8_gemm.py:52-67) and
    test_dense_path_reads_the_packed_weights_exactly (:33-49) for the W8A8 slot."""
    from opendecider_amd.quant import Int8Linear, fast_int8_kernels_
    torch.manual_seed(0)
    lin = Int8Linear(torch.nn.Linear(256, 128, bias=False).to(DEV).to(torch.bfloat16))
    w_ref = lin.weight.clone()

    class BB:
        device = torch.device(DEV)
        lm = torch.nn.Module()
    BB.lm.layers = torch.nn.Sequential(lin)
    lin.register_forward_hook(lambda mod, args, out: out + 100.0)
    x = torch.randn(8, 256, device=DEV, dtype=torch.bfloat16)
    y0 = BB.lm.layers(x).float()
    assert fast_int8_kernels_(BB) == 1
    assert BB.lm.layers[0] is lin and lin.qweight.numel() == 0
    assert torch.equal(lin.weight, w_ref)
    y1 = BB.lm.layers(x).float()
    assert (y1 - 100.0).abs().mean() < 50 and ((y1 - y0).norm() / y0.norm()).item() < 1e-2


def test_int8_tensor_quantize_matches_reference_formula(gpu_lib):
    from opendecider_amd.quant import Int8Tensor
    g = torch.Generator().manual_seed(5)
    x = torch.randn(3, 5, 64, generator=g).to(torch.bfloat16)
    t = Int8Tensor.quantize(x.to(DEV))
    rq, rs = oq.quantize_rows(x)
    assert torch.equal(t.q.cpu(), rq)
    assert t.scale.dtype == torch.bfloat16 and torch.equal(t.scale.cpu(), rs.to(torch.bfloat16))
    t32 = Int8Tensor.quantize(x.to(DEV), scale_dtype=torch.float32)
    assert torch.equal(t32.scale.cpu(), rs)
    err = (t.dequantize().float().cpu() - x.float()).abs().max()
    assert err <= x.float().abs().amax() / 127 + 1e-2


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.float64])
@pytest.mark.parametrize("K", [4096, 200, 1])
def test_int8_tensor_quantize_float_inputs(gpu_lib, dtype, K):
    """Int8Tensor.quantize of float32 / float16 / float64 input (the reference quantizes x.float() for any dtype,
    quant.py:36-41; od_act_quant_f32): bytes and scales equal the oracle's, the scale stored in x.dtype (fp32 for
    fp32); rows whose values sit on and next to half-integer quotients (fp32 neighbours of (n + 1/2) * scale, which
    the fast reciprocal path alone would round wrongly on some), and NaN / inf rows as torch's rule."""
    import numpy as np
    from opendecider_amd.quant import Int8Tensor
    g = torch.Generator().manual_seed(K + 17)
    x = (torch.randn(9, K, generator=g, dtype=torch.float64) * 3).to(dtype)
    if K >= 200:
        amax = np.float32(x[0].float().abs().max().item())
        scale = np.float32(amax / np.float32(127))
        n = np.arange(-60, 60, dtype=np.float32)
        ties = ((n + np.float32(0.5)) * scale).astype(np.float32)
        near = np.concatenate([ties, np.nextafter(ties, np.float32(np.inf)), np.nextafter(ties, np.float32(-np.inf))])
        near = near[: K - 1]
        if dtype != torch.float16:
            x[0, 1:1 + near.size] = torch.from_numpy(near).to(dtype)
        x[2, 7] = float("nan")
        x[3, K - 1] = float("inf")
        x[4, 0] = float("-inf")
    print(f"Int8Tensor.quantize {dtype} rows of K={K}", flush=True)
    t = Int8Tensor.quantize(x.to(DEV))
    rq, rs = oq.quantize_rows(x)
    assert torch.equal(t.q.cpu(), rq)
    assert t.scale.dtype == dtype and t.scale.shape == (9, 1)
    fin = torch.isfinite(rs[:, 0])
    assert torch.equal(t.scale.cpu()[fin], rs[fin].to(dtype))
    if K >= 200:
        assert torch.isnan(t.scale.cpu()[2]).all() and torch.isinf(t.scale.cpu()[[3, 4]]).all()
    t32 = Int8Tensor.quantize(x.to(DEV), scale_dtype=torch.float32)
    assert torch.equal(t32.scale.cpu()[fin].view(torch.int32), rs[fin].view(torch.int32))
    empty = Int8Tensor.quantize(torch.zeros(0, K, dtype=dtype, device=DEV))
    assert empty.q.shape == (0, K) and empty.scale.shape == (0, 1)
    with pytest.raises(TypeError):
        Int8Tensor.quantize(torch.zeros(2, K, dtype=torch.int32, device=DEV))


@pytest.mark.parametrize("M,K,F", [(4096, 4096, 12288), (300, 272, 520), (77, 4096, 98), (333, 512, 1024)])
def test_w8a8_gemm_swiglu_equals_gemm_then_swiglu(gpu_lib, M, K, F):
    """The SwiGLU epilogue gives the bytes of the plain GEMM followed by the SwiGLU kernel (shared device silu):
    quantizing its h equals od_silu_mul_quant on the plain GEMM's [gate | up] output, bit for bit; and h differs
    from the oracle's SwiGLU of the oracle's (bit-exact) GEMM output on <= 0.5% of elements, by at most two bf16
    steps (the device and host exp may round silu(g) to neighbouring bf16 values, which the product with u keeps).
    Odd shapes take the GENERAL variant (K tail, ragged tiles)."""
    from opendecider_amd import kernels
    g = torch.Generator().manual_seed(M + K + F)
    a = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8)
    w = torch.randint(-127, 128, (2 * F, K), generator=g, dtype=torch.int8)
    sa = torch.rand(M, generator=g) * 1e-2
    sw = torch.rand(2 * F, generator=g) * 1e-3
    print(f"w8a8_gemm_swiglu M={M} K={K} F={F}", flush=True)
    h = kernels.w8a8_gemm_swiglu(a.to(DEV), sa.to(DEV), kernels.interleave_gate_up(w).to(DEV),
                                 kernels.interleave_gate_up(sw).to(DEV))
    gu = kernels.w8a8_gemm(a.to(DEV), sa.to(DEV), w.to(DEV), sw.to(DEV))
    inv = (1 / (torch.rand(F, generator=g) + 0.5)).to(torch.bfloat16).to(DEV)
    xq1, sx1 = kernels.act_quant(h, inv)
    xq2, sx2 = kernels.silu_mul_quant(gu, F, inv)
    assert torch.equal(xq1, xq2) and torch.equal(sx1, sx2)
    ref_gu = oq.w8a8_epilogue(oq.int_gemm(a, w), sa, sw)
    assert torch.equal(gu.cpu(), ref_gu)
    ref = od.swiglu(ref_gu, F).float()
    d = (h.cpu().float() - ref).abs()
    assert (d <= ref.abs() * 2.0 ** -6 + 2.0 ** -120).all() and (d > 0).float().mean().item() <= 5e-3


def test_quantizer_near_half_integer_quotients(gpu_lib):
    """The device quantizer multiplies by 1 / scale and redoes the IEEE division only for quotients within 2^-15
    of a half-integer. Rows are built so that many of their values land there (found by searching all bf16 values
    below each row's absmax): act_quant's bytes and scales must equal the oracle's, with and without the smoothing
    scale (here 1, so the values are unchanged)."""
    import numpy as np
    rng = np.random.default_rng(9)
    allv = torch.arange(1, 0x7F80, dtype=torch.int32).to(torch.int16).view(torch.bfloat16).float().numpy()
    K, rows, n_near = 1024, [], 0
    while len(rows) < 192:
        amax = np.float32(torch.tensor(float(np.exp(rng.uniform(-7, 5)))).bfloat16().float().item())
        scale = np.float32(max(amax, np.float32(1e-8)) / np.float32(127))
        v = allv[allv <= amax]
        q = (v / scale).astype(np.float32)
        near = v[np.abs(np.abs(q - np.rint(q)) - 0.5) <= 2.0 ** -15]
        if near.size == 0:
            continue
        row = rng.choice(v, K).astype(np.float32) * rng.choice([-1.0, 1.0], K).astype(np.float32)
        row[0] = amax
        k = min(near.size, K // 4)
        row[1:1 + 2 * k:2], row[2:2 + 2 * k:2] = near[:k], -near[:k]
        rows.append(row)
        n_near += 2 * k
    from opendecider_amd import kernels
    x = torch.from_numpy(np.stack(rows)).to(torch.bfloat16)
    rq, rs = oq.quantize_rows(x)
    # the multiplication alone (no fallback), restated on the CPU, gets some of these bytes wrong
    xf, sf = x.float().numpy(), rs.numpy().astype(np.float32)
    fast = np.clip(np.rint((xf * (np.float32(1) / sf)).astype(np.float32)), -127, 127).astype(np.int8)
    assert n_near >= 192 and (fast != rq.numpy()).any()
    xq, sx = kernels.act_quant(x.to(DEV))
    assert torch.equal(xq.cpu()[:, :K], rq) and torch.equal(sx.cpu(), rs[:, 0])
    ones = torch.ones(K, dtype=torch.bfloat16, device=DEV)
    xq1, sx1 = kernels.act_quant(x.to(DEV), ones)
    assert torch.equal(xq1.cpu()[:, :K], rq) and torch.equal(sx1.cpu(), rs[:, 0])


@pytest.mark.parametrize("K", [4096, 200, 128])
def test_quantizers_nan_and_inf_rows(gpu_lib, K):
    """torch's rule for non-finite rows (quant.py:38-40 on CPU): a row holding a NaN gets a NaN scale (amax and
    clamp_min propagate it) and zero bytes; a row holding an infinity gets an infinite scale and zero bytes (x / inf
    = 0, inf / inf = NaN -> 0). Both quantizers (per-token activations, per-(token, head) K/V append) follow it, on
    the vector and the scalar paths."""
    from opendecider_amd import kernels
    g = torch.Generator().manual_seed(K)
    x = torch.randn(6, K, generator=g).to(torch.bfloat16)
    x[1, 7] = float("nan")
    x[3, K - 1] = float("inf")
    x[4, 0] = float("-inf")
    x[5, 2] = float("nan")
    x[5, 3] = float("inf")
    rq, rs = oq.quantize_rows(x)
    xq, sx = kernels.act_quant(x.to(DEV))
    assert torch.equal(xq.cpu(), rq)
    assert torch.equal(sx.cpu().view(torch.int32)[[0, 2]], rs[[0, 2], 0].view(torch.int32))
    assert torch.isnan(sx.cpu()[[1, 5]]).all() and torch.isinf(sx.cpu()[[3, 4]]).all()
    if K % 16 == 0 and K <= 256:
        q = torch.full((1, 6, 4, K), 55, dtype=torch.int8, device=DEV)
        s = torch.full((1, 6, 4), -1.0, device=DEV)
        kernels.kv_quant_append(x.view(1, 6, 1, K).to(DEV), q, s, 1)
        assert torch.equal(q[0, :, 1].cpu(), rq) and (q[0, :, 0] == 55).all() and (q[0, :, 2:] == 55).all()
        assert torch.isnan(s[0, [1, 5], 1].cpu()).all() and torch.isinf(s[0, [3, 4], 1].cpu()).all()


@pytest.mark.parametrize("M,K,smooth", [(5, 4096, True), (33, 4096, False), (7, 200, True), (64, 128, True)])
def test_gate_act_quant_bit_exact(gpu_lib, M, K, smooth):
    """od_gate_act_quant = the oracle's act_quant of bf16(x * bf16(sigmoid(g))) (prefix_attn.py:130 then o_proj's
    input quantization), bytes and scales, on the vector and scalar paths and with a gate that is a strided view."""
    from opendecider_amd import kernels
    g = torch.Generator().manual_seed(M + K)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    big = (torch.randn(M, 2 * K, generator=g) * 6).to(torch.bfloat16)
    gate = big[:, K:]
    inv = (1 / (torch.rand(K, generator=g) * 1.5 + 0.5)).to(torch.bfloat16) if smooth else None
    xq, sx = kernels.gate_act_quant(x.to(DEV), big.to(DEV)[:, K:], None if inv is None else inv.to(DEV))
    rq, rs = oq.act_quant(od.output_gate(x, gate), inv)
    assert torch.equal(xq.cpu(), rq) and torch.equal(sx.cpu().view(torch.int32), rs.view(torch.int32))


@pytest.mark.parametrize("K", [1, 8])
def test_gate_sigmoid_on_all_bf16_inputs(gpu_lib, K):
    """bf16(sigmoid(g)) inside od_gate_act_quant on every bf16 bit pattern of g: row r holds x = (1, 0, ...) and the
    gate g_r, so its scale max(bf16(sigmoid(g_r)), 1e-8) / 127 carries the gate value (bit-exact against the
    oracle's correctly rounded table wherever sigmoid(g) >= 1e-8); K = 1 runs the scalar path, K = 8 the vector one."""
    from opendecider_amd import kernels
    gv = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    keep = ((gv.view(torch.int16).int() >> 7) & 0xFF) != 0  # normal numbers, infinities and NaNs
    gv = gv[keep]
    M = gv.numel()
    x = torch.zeros(M, K, dtype=torch.bfloat16)
    x[:, 0] = 1.0
    gate = torch.zeros(M, K, dtype=torch.bfloat16)
    gate[:, 0] = gv
    _, sx = kernels.gate_act_quant(x.to(DEV), gate.to(DEV))
    ref = od.sigmoid_bf16(gv).float().clamp_min(1e-8) / 127.0
    got = sx.cpu()
    nan = torch.isnan(ref)
    assert torch.equal(torch.isnan(got), nan)
    assert torch.equal(got[~nan].view(torch.int32), ref[~nan].view(torch.int32))


def _one_pass(a, sa, w, sw, bias, res, swiglu):
    """The GEMM without split-K, by the 256-row tile kernel: od_w8a8_gemm / od_w8a8_gemm_swiglu called directly (a
    plain GEMM also asks for the int32 accumulators, which only that kernel writes, so small M takes it too)."""
    from opendecider_amd import _lib
    from opendecider_amd._lib import ptr, stream_of
    M, K = a.shape
    N = w.shape[0]
    out = torch.empty(M, N // 2 if swiglu else N, dtype=torch.bfloat16, device=DEV)
    L = _lib.lib()
    if swiglu:
        rc = L.od_w8a8_gemm_swiglu(ptr(a), K, ptr(sa), ptr(w), K, ptr(sw), ptr(out), out.stride(0), M, N, K,
                                   stream_of(a))
    else:
        acc = torch.empty(M, N, dtype=torch.int32, device=DEV)
        rc = L.od_w8a8_gemm(ptr(a), K, ptr(sa), ptr(w), K, ptr(sw), ptr(bias), ptr(res), N if res is not None else 0,
                            ptr(out), N, ptr(acc), N, M, N, K, stream_of(a))
    assert rc == 0
    return out


@pytest.mark.parametrize("M,N,K,epi", [(64, 6144, 2048, "plain"), (1, 2048, 6144, "bias_res"), (7, 3000, 4000, "res"),
                                       (64, 2048, 2048, "bias"), (33, 20, 2064, "bias_res"), (64, 4096, 12288, "res"),
                                       (200, 2048, 6144, "plain"), (256, 4096, 4096, "bias_res"),
                                       (512, 2048, 6144, "res"), (129, 4104, 1040, "bias")])
def test_small_m_kernel_bit_identical_to_256_row_kernel(gpu_lib, M, N, K, epi):
    """Up to 512 rows the GEMM takes the small-M kernel (64-row tiles, K split over the workgroup's waves, the
    partial tiles summed exactly through LDS): the same bits as one pass of the 256-row kernel, and on the smaller
    cases as the oracle's. K tails (K % 128 != 0) and ragged N included."""
    from opendecider_amd import kernels
    g = torch.Generator().manual_seed(M + N + K)
    a, w, sa, sw = _gemm_case(g, M, N, K)
    bias = torch.randn(N, generator=g).to(torch.bfloat16).to(DEV) if "bias" in epi else None
    res = torch.randn(M, N, generator=g).to(torch.bfloat16).to(DEV) if "res" in epi else None
    ad, wd, sad, swd = a.to(DEV), w.to(DEV), sa.to(DEV), sw.to(DEV)
    print(f"small-M M={M} N={N} K={K} {epi}", flush=True)
    assert kernels.splitk_workspace(M, N, K, DEV) is None
    got = kernels.w8a8_gemm(ad, sad, wd, swd, bias, res)
    ref = _one_pass(ad, sad, wd, swd, bias, res, False)
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
    if M * N * K <= 64 * 6144 * 2048:
        refo = oq.w8a8_epilogue(oq.int_gemm(a, w), sa, sw, None if bias is None else bias.cpu(),
                                None if res is None else res.cpu())
        assert torch.equal(got.cpu(), refo)


@pytest.mark.parametrize("M,N,K,epi", [(1024, 2048, 6144, "plain"), (600, 1030, 6144, "swiglu"),
                                       (1024, 4096, 12288, "res"), (700, 2048, 6144, "bias_res"),
                                       (1000, 20, 2064, "bias_res")])
def test_splitk_bit_identical_to_one_pass(gpu_lib, M, N, K, epi):
    """Mid-size M with few tiles takes split-K (int32 partial planes in a workspace, summed exactly, then the same
    epilogue): the output equals the one-pass GEMM's bit for bit, also when the workspace is one element short (the
    call then runs one pass), and on the small cases the oracle's."""
    from opendecider_amd import _lib, kernels
    from opendecider_amd._lib import ptr, stream_of
    g = torch.Generator().manual_seed(M + N + K)
    a, w, sa, sw = _gemm_case(g, M, N, K)
    bias = torch.randn(N, generator=g).to(torch.bfloat16).to(DEV) if "bias" in epi else None
    res = torch.randn(M, N, generator=g).to(torch.bfloat16).to(DEV) if "res" in epi else None
    ad, wd, sad, swd = a.to(DEV), w.to(DEV), sa.to(DEV), sw.to(DEV)
    swiglu = epi == "swiglu"
    print(f"splitk M={M} N={N} K={K} {epi}", flush=True)
    ws = kernels.splitk_workspace(M, N, K, DEV)
    assert ws is not None, "the plan should split this shape"
    if swiglu:
        got = kernels.w8a8_gemm_swiglu(ad, sad, wd, swd)
    else:
        got = kernels.w8a8_gemm(ad, sad, wd, swd, bias, res)
    ref = _one_pass(ad, sad, wd, swd, bias, res, swiglu)
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
    if ws is not None:
        short = torch.empty(ws.numel() - 1, dtype=torch.int32, device=DEV)
        out = torch.empty_like(ref)
        rc = _lib.lib().od_w8a8_gemm_ws(ptr(ad), K, ptr(sad), ptr(wd), K, ptr(swd), ptr(bias), ptr(res),
                                        N if res is not None else 0, ptr(out), out.stride(0), M, N, K, int(swiglu),
                                        ptr(short), short.numel(), stream_of(ad))
        assert rc == 0
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    if M * N * K <= 64 * 6144 * 2048 and not swiglu:
        refo = oq.w8a8_epilogue(oq.int_gemm(a, w), sa, sw, None if bias is None else bias.cpu(),
                                None if res is None else res.cpu())
        assert torch.equal(got.cpu(), refo)
