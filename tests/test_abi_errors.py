"""The C ABI's argument checks, driven on the CPU: every call below is refused by the host-side validation with its
OD_ERR_* code before any HIP call (no GPU work is launched; a call whose arguments pass validation is never made
here). Also the reference's own CPU test of the fused-kernel installer (tests/test_int8_gemm.py:8-16) restated."""
import ctypes
import os

import pytest
import torch

OK, NULL, SHAPE, ALIGN, UNSUP = 0, -1, -2, -3, -4
P = 0x10000  # a 16-byte aligned non-null pointer value; never dereferenced (every call fails validation first)


@pytest.fixture(scope="module")
def L():
    from opendecider_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        from opendecider_amd.build import build
        build()
    return _lib.lib()


def test_act_quant_and_kv_append_checks(L):
    assert L.od_act_quant(P, 16, None, P, 16, P, 4, 0, None) == SHAPE       # K = 0
    assert L.od_act_quant(P, 8, None, P, 16, P, 4, 16, None) == SHAPE       # ldx < K
    assert L.od_act_quant(None, 16, None, P, 16, P, 4, 16, None) == NULL
    assert L.od_act_quant(None, 16, None, None, 16, None, 0, 16, None) == OK  # M = 0: nothing to do, no launch
    assert L.od_act_quant_f32(P, 16, P, 16, P, 4, 0, None) == SHAPE             # K = 0
    assert L.od_act_quant_f32(P, 16, P, 8, P, 4, 16, None) == SHAPE             # ldq < K
    assert L.od_act_quant_f32(P, 16, P, 16, P, -1, 16, None) == SHAPE           # M < 0
    assert L.od_act_quant_f32(P, 16, P, 16, None, 4, 16, None) == NULL
    assert L.od_act_quant_f32(None, 16, None, 16, None, 0, 16, None) == OK
    # n0 + n_new past the capacity
    assert L.od_kv_quant_append(P, 1, 2, 5, 128, 1280, 640, 128, P, P, 8, 4, None) == SHAPE
    assert L.od_kv_quant_append(P, 1, 2, 5, 128, -1, 640, 128, P, P, 16, 4, None) == SHAPE  # negative stride


def test_gemm_checks(L):
    assert L.od_w8a8_gemm(P, 64, P, P, 64, P, None, None, 0, P, 64, None, 0, 4, 64, 0, None) == SHAPE  # K = 0
    assert L.od_w8a8_gemm(None, 64, P, P, 64, P, None, None, 0, P, 64, None, 0, 4, 64, 64, None) == NULL
    assert L.od_w8a8_gemm(P, 64, None, P, 64, P, None, None, 0, P, 64, None, 0, 4, 64, 64, None) == NULL  # no sa
    assert L.od_w8a8_gemm(P, 32, P, P, 64, P, None, None, 0, P, 64, None, 0, 4, 64, 64, None) == SHAPE  # lda < K
    rc = L.od_w8a8_gemm(P, 72, P, P, 72, P, None, None, 0, P, 64, None, 0, 4, 64, 72, None)  # K % 16 != 0
    assert rc in (ALIGN, UNSUP, SHAPE) and rc != OK
    assert L.od_w8a8_gemm_swiglu(P, 64, P, P, 64, P, P, 32, 4, 63, 64, None) != OK  # N odd


def test_attention_checks(L):
    s = (1024, 128, 128) * 3  # strides of q, k_own, v_own
    def branched(D=128, Hq=8, Hkv=2, t=4, dq=0, q=P):
        return L.od_branched_attn(q, *s[:3], P, *s[3:6], P, *s[6:], P, P, P, P, None, None, 2, P, 1024, 128, 128,
                                  None, 2, Hq, Hkv, t, D, 1, 64, 64, 0.1, dq, None)
    assert branched(D=96) == UNSUP
    assert branched(D=512) == UNSUP  # D in {64, 128, 256}, the reference's dispatch set
    assert branched(Hq=6, Hkv=4) == UNSUP
    assert branched(t=0) == SHAPE
    assert branched(dq=5) == UNSUP
    assert branched(q=None) == NULL
    rc = L.od_branched_attn_split(P, *s[:3], P, *s[3:6], P, *s[6:], P, P, P, P, None, None, 2, P, 1024, 128, 128,
                                  None, 2, 8, 2, 4, 128, 1, 64, 64, 0.1, 0, 0, None, 0, None)
    assert rc == SHAPE  # nsplit = 0
    rc = L.od_branched_attn_split(P, *s[:3], P, *s[3:6], P, *s[6:], P, P, P, P, None, None, 2, P, 1024, 128, 128,
                                  None, 2, 8, 2, 4, 128, 1, 64, 64, 0.1, 0, 4, P, 10, None)
    assert rc == SHAPE  # workspace too small for 4 splits
    rc = L.od_branched_attn(P, 1028, 128, 128, P, *s[3:6], P, *s[6:], P, P, P, P, None, None, 2, P, 1024, 128, 128,
                            None, 2, 8, 2, 4, 128, 1, 64, 64, 0.1, 0, None)
    assert rc == ALIGN  # a query stride that breaks the 16-byte loads
    assert L.od_attn_stage(P, P, P, P, None, 1, 1, 64, 32, 128, 0.1, 0, P, 1 << 20, None) == SHAPE  # cap < T
    assert L.od_attn_stage(P, P, P, P, None, 1, 1, 64, 64, 128, 0.1, 3, P, 1 << 20, None) == UNSUP  # dequant
    assert L.od_attn_stage(P, P, P, P, None, 1, 1, 64, 64, 128, 0.1, 0, P, 100, None) == SHAPE  # image too small
    assert L.od_attn_stage(P, P, P, P, None, 1, 1, 64, 64, 256, 0.1, 0, P, 66063, None) == SHAPE  # D = 256 image
    n = ctypes.c_int64(0)
    for D in (64, 128, 256):  # a 64-key image holds 4 * 64 * D bytes of K and V plus 528 of per-key data
        assert L.od_attn_stage_size(2, 3, 65, D, ctypes.byref(n)) == OK and n.value == 2 * 3 * 2 * (256 * D + 528)
    assert L.od_attn_stage_size(1, 1, 64, 96, ctypes.byref(n)) == UNSUP
    w = (1024, 128, 128)
    assert L.od_wide_attn(P, *w, P, *w, P, *w, None, 0, P, *w, None, 1, 2, 2, 4, 4, 128, 96, 1, 0.1, None) == UNSUP
    assert L.od_wide_attn(P, *w, P, *w, P, *w, None, 0, P, *w, None, 1, 3, 2, 4, 4, 128, 128, 1, 0.1, None) == SHAPE
    for bad_scale in (0.0, -0.1, float("inf"), float("nan")):  # the block max is taken on unscaled scores
        assert L.od_wide_attn(P, *w, P, *w, P, *w, None, 0, P, *w, None, 1, 2, 2, 4, 4, 128, 128, 1, bad_scale,
                              None) == UNSUP
    bf = (1024, 128, 128)
    assert L.od_attn_stage_bf16(P, *bf, P, *bf, None, 1, 1, 64, 96, 0.1, P, 1 << 20, None) == UNSUP  # D = 96
    assert L.od_attn_stage_bf16(P, 1028, 128, 128, P, *bf, None, 1, 1, 64, 128, 0.1, P, 1 << 20, None) == ALIGN
    assert L.od_attn_stage_bf16(P, *bf, P, *bf, None, 1, 1, 64, 128, 0.1, P, 100, None) == SHAPE  # image too small


def test_stream_attention_checks(L):
    """od_branched_attn_stream: head_dim 128 only, at most 32 query slots per (state, KV head), the split workspace
    and alignment rules of od_branched_attn_split."""
    s = (1024, 128, 128) * 3
    def stream(D=128, Hq=8, Hkv=2, t=4, max_rows=2, dq=0, nsplit=1, ws=None, ws_floats=0, ks=P, kq=P):
        return L.od_branched_attn_stream(P, *s[:3], P, *s[3:6], P, *s[6:], kq, ks, P, P, None, None, max_rows, P,
                                         1024, 128, 128, None, 2, Hq, Hkv, t, D, 1, 64, 64, 0.1, dq, nsplit, ws,
                                         ws_floats, None)
    assert stream(D=64) == UNSUP
    assert stream(t=5, max_rows=2) == UNSUP       # 2 rows x 5 tokens x 4 heads = 40 slots
    assert stream(Hq=6, Hkv=4) == UNSUP
    assert stream(dq=2) == UNSUP
    assert stream(nsplit=0) == SHAPE
    assert stream(nsplit=3, ws=P, ws_floats=100) == SHAPE   # workspace too small
    # R = 2 rows, Hq = 8, t = 4, D = 128: 3 splits take 3 x 2 x 8 x 4 x 129 floats, plus Ns x Hkv = 2 merge counters
    assert stream(nsplit=3, ws=P, ws_floats=3 * 2 * 8 * 4 * 129 + 1) == SHAPE
    assert stream(nsplit=3) == NULL                          # no workspace
    assert stream(ks=P + 2) == ALIGN                         # scales must be 4-byte aligned
    assert stream(kq=P + 8) == ALIGN                         # int8 K must be 16-byte aligned


def test_row_kernel_checks(L):
    assert L.od_rmsnorm_quant(P, 8, P, None, 1e-6, P, 16, P, 4, 16, None) == SHAPE  # ldx < K
    assert L.od_silu_mul_quant(P, 16, 16, None, P, 16, P, 4, None) == SHAPE  # ldg < 2F
    assert L.od_qk_norm_rope(P, 1024, 4, 4, 2, 96, P, P, P, P, 16, P, 1e-6, None) == UNSUP  # D = 96
    assert L.od_qk_norm_rope_kv_append(P, 2048, 1, 8, 8, 2, 128, P, P, P, P, 64, P, 1e-6, P, P, P, P, 10, 4,
                                       None) == SHAPE  # n0 + S > cap


def test_lm_head_checks(L):
    assert L.od_lm_head_logprob(P, 64, P, 64, 0, P, 32, P, P, 4, 100, 64, P, P, 1 << 20, None) == SHAPE  # ldw < K
    assert L.od_lm_head_logprob(None, 64, P, 64, 0, P, 64, P, P, 4, 100, 64, P, P, 1 << 20, None) == NULL


def test_fast_kernels_noop_on_cpu(monkeypatch):
    """tests/test_int8_gemm.py:8-16: on a CPU backbone, and with OPENDECIDER_INT8_GEMM=dequant, the installer leaves
    the dequantize path untouched and returns 0."""
    import torch.nn as nn
    from opendecider_amd.quant import Int8Linear, fast_int8_kernels_

    class BB:
        device = torch.device("cpu")
        lm = nn.Module()
    BB.lm.layers = nn.Sequential(Int8Linear(nn.Linear(16, 8)))
    assert fast_int8_kernels_(BB) == 0 and isinstance(BB.lm.layers[0], Int8Linear)
    assert "_fused" not in BB.lm.layers[0].__dict__
    monkeypatch.setenv("OPENDECIDER_INT8_GEMM", "dequant")
    assert fast_int8_kernels_(BB) == 0


def test_wrappers_refuse_cpu_tensors():
    """No CPU fallback: the torch wrappers raise before any launch when given host tensors."""
    from opendecider_amd import kernels
    x = torch.zeros(4, 16, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="no CPU path"):
        kernels.act_quant(x)
    with pytest.raises(RuntimeError, match="no CPU path"):
        kernels.w8a8_gemm(torch.zeros(4, 16, dtype=torch.int8), torch.ones(4), torch.zeros(8, 16, dtype=torch.int8),
                          torch.ones(8))
