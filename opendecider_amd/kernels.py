"""Thin torch wrappers of the C ABI (include/od_mi355x.h): shape checks, output allocation on the current device,
and the current HIP stream. Every function requires CUDA (ROCm) tensors and raises otherwise."""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from ._lib import check, lib, ptr, require_gpu, stream_of


def _quant_outputs(M, K, ld, device, xq, sx):
    if xq is None:
        ld = K if ld is None else ld
        xq = (torch.zeros if ld > K else torch.empty)(M, ld, dtype=torch.int8, device=device)
    elif xq.dtype != torch.int8 or xq.shape[0] != M or xq.shape[1] < K or xq.stride(1) != 1:
        raise ValueError("quantized output must be int8 (M, >= K) with contiguous rows")
    if sx is None:
        sx = torch.empty(M, dtype=torch.float32, device=device)
    elif sx.dtype != torch.float32 or sx.numel() != M or not sx.is_contiguous():
        raise ValueError("scale output must be fp32 (M,) contiguous")
    return xq, sx


def _check_out(out, shape, device, name):
    """A caller-given bf16 output must have the exact shape and contiguous rows (the kernels write shape-many
    elements through its strides); None allocates one."""
    if out is None:
        return torch.empty(*shape, dtype=torch.bfloat16, device=device)
    if out.dtype != torch.bfloat16 or tuple(out.shape) != tuple(shape) or out.stride(-1) != 1:
        raise ValueError(f"{name}: out must be bf16 {tuple(shape)} with a contiguous last dim, got "
                         f"{out.dtype} {tuple(out.shape)} strides {out.stride()}")
    if not out.is_cuda:
        raise RuntimeError(f"{name}: out must be on the GPU")
    return out


def _scales(t, n, name):
    """fp32 per-row / per-channel scales, contiguous (the kernels read n floats)."""
    if t.dtype != torch.float32:
        raise TypeError(f"{name} must be float32, got {t.dtype}")
    if t.numel() != n:
        raise ValueError(f"{name} has {t.numel()} elements, expected {n}")
    return t.contiguous()


def _vec(v, n, name):
    if v is None:
        return None
    _lib.bf16_bits(v)
    v = v.contiguous()
    if v.numel() != n:
        raise ValueError(f"{name} has {v.numel()} elements, expected {n}")
    return v


def act_quant(x: torch.Tensor, inv_s: torch.Tensor | None = None, ld: int | None = None, xq=None, sx=None):
    """Per-row int8 quantization of x (..., K) bf16 (Int8Tensor.quantize, quant.py:36-41), with the optional
    SmoothQuant input scale inv_s (K,) bf16 applied first (quant.py:329). Returns (xq int8 (rows, ld), sx fp32
    (rows,)) with rows = x.numel() // K; columns K..ld-1 of a freshly allocated xq are zero (ld >= K pads rows for
    the GEMM). xq / sx may be given (preallocated; xq may be a column slice of a wider buffer)."""
    require_gpu(x, inv_s, xq, sx, name="act_quant")
    _lib.bf16_bits(x)
    K = x.shape[-1]
    x2 = x.reshape(-1, K)
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    M = x2.shape[0]
    xq, sx = _quant_outputs(M, K, ld, x.device, xq, sx)
    inv_s = _vec(inv_s, K, "inv_s")
    check(lib().od_act_quant(ptr(x2), x2.stride(0) if M > 1 else K, ptr(inv_s), ptr(xq), xq.stride(0), ptr(sx), M, K,
                             stream_of(x)), "od_act_quant")
    return xq, sx


def act_quant_float(x: torch.Tensor):
    """Per-row int8 quantization of a float32 / float16 / float64 x (..., K): the formula of act_quant over
    x.float(), as the reference quantizes any dtype (quant.py:38; the conversion is exact for float16, and for
    float64 it is the reference's own first step). Returns (xq int8 (rows, K), sx fp32 (rows,))."""
    require_gpu(x, name="act_quant_float")
    if x.dtype not in (torch.float32, torch.float16, torch.float64):
        raise TypeError(f"act_quant_float: expected float32, float16 or float64, got {x.dtype}")
    K = x.shape[-1]
    x2 = x.reshape(-1, K).float()
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    M = x2.shape[0]
    xq, sx = _quant_outputs(M, K, None, x.device, None, None)
    check(lib().od_act_quant_f32(ptr(x2), x2.stride(0) if M > 1 else K, ptr(xq), xq.stride(0), ptr(sx), M, K,
                                 stream_of(x)), "od_act_quant_f32")
    return xq, sx


def gate_act_quant(x: torch.Tensor, gate: torch.Tensor, inv_s: torch.Tensor | None = None, xq=None, sx=None):
    """Per-row int8 quantization of bf16(x * bf16(sigmoid(gate))) (the attention output times the output gate,
    prefix_attn.py:130), with the optional SmoothQuant input scale inv_s applied after the gate. x, gate (M, K) bf16
    with contiguous rows (any row strides). Returns (xq int8 (M, K), sx fp32 (M,))."""
    require_gpu(x, gate, inv_s, xq, sx, name="gate_act_quant")
    _lib.bf16_bits(x)
    _lib.bf16_bits(gate)
    M, K = x.shape
    if gate.shape != (M, K):
        raise ValueError("gate_act_quant: gate must have x's shape")
    if x.stride(1) != 1:
        x = x.contiguous()
    if gate.stride(1) != 1:
        gate = gate.contiguous()
    xq, sx = _quant_outputs(M, K, None, x.device, xq, sx)
    inv_s = _vec(inv_s, K, "inv_s")
    check(lib().od_gate_act_quant(ptr(x), x.stride(0) if M > 1 else K, ptr(gate), gate.stride(0) if M > 1 else K,
                                  ptr(inv_s), ptr(xq), xq.stride(0), ptr(sx), M, K, stream_of(x)),
          "od_gate_act_quant")
    return xq, sx


def rmsnorm_quant(x: torch.Tensor, w: torch.Tensor, eps: float, inv_s=None, xq=None, sx=None, offset: bool = False):
    """RMSNorm (bf16(w * bf16(x * rsqrt(mean x^2 + eps))), or with offset Qwen3.5's zero-centred
    bf16((x * r) * (1 + w))) -> optional SmoothQuant scale -> per-row int8. x (M, K) bf16 with contiguous rows.
    Returns (xq, sx)."""
    require_gpu(x, w, inv_s, xq, sx, name="rmsnorm_quant")
    _lib.bf16_bits(x)
    M, K = x.shape
    if x.stride(1) != 1:
        x = x.contiguous()
    xq, sx = _quant_outputs(M, K, None, x.device, xq, sx)
    w, inv_s = _vec(w, K, "w"), _vec(inv_s, K, "inv_s")
    check(lib().od_rmsnorm_quant_ex(ptr(x), x.stride(0), ptr(w), ptr(inv_s), float(eps), int(bool(offset)), ptr(xq),
                                    xq.stride(0), ptr(sx), M, K, stream_of(x)), "od_rmsnorm_quant_ex")
    return xq, sx


def silu_mul_quant(gu: torch.Tensor, F: int, inv_s=None, xq=None, sx=None):
    """bf16(bf16(silu(g)) * u) of the fused gate+up output gu (M, >= 2F) -> optional SmoothQuant scale -> per-row
    int8. Returns (xq (M, F), sx)."""
    require_gpu(gu, inv_s, xq, sx, name="silu_mul_quant")
    _lib.bf16_bits(gu)
    M = gu.shape[0]
    if gu.stride(1) != 1 or gu.shape[1] < 2 * F:
        raise ValueError("silu_mul_quant: gu must be (M, >= 2F) with contiguous rows")
    xq, sx = _quant_outputs(M, F, None, gu.device, xq, sx)
    inv_s = _vec(inv_s, F, "inv_s")
    check(lib().od_silu_mul_quant(ptr(gu), gu.stride(0), F, ptr(inv_s), ptr(xq), xq.stride(0), ptr(sx), M,
                                  stream_of(gu)), "od_silu_mul_quant")
    return xq, sx


def _rope_tables_ok(cos_t, sin_t, D: int, rot_dim: int, name: str) -> None:
    if rot_dim not in (D, D // 4):
        raise ValueError(f"{name}: rot_dim must be the head dim ({D}) or a quarter of it, got {rot_dim}")
    if cos_t.shape != sin_t.shape or cos_t.shape[1] != rot_dim // 2 or not (cos_t.is_contiguous() and
                                                                            sin_t.is_contiguous()):
        raise ValueError(f"{name}: cos/sin tables must be contiguous [positions, rot_dim/2]")


def qk_norm_rope(qkv: torch.Tensor, n_heads_q: int, n_heads_k: int, D: int, q_w, k_w, cos_t, sin_t, pos,
                 eps: float, rot_dim: int | None = None, offset: bool = False) -> None:
    """In place on qkv (M, >= (Hq + Hk) D): per-head RMSNorm of the q and k heads (offset: Qwen3.5's zero-centred
    weights), then rotary embedding on the first rot_dim dims (default D; D / 4 is Qwen3.5's partial rotary) with
    the bf16 cos/sin tables [positions, rot_dim/2] at positions pos (M,) int32."""
    require_gpu(qkv, q_w, k_w, cos_t, sin_t, pos, name="qk_norm_rope")
    _lib.bf16_bits(qkv)
    M = qkv.shape[0]
    rot_dim = D if rot_dim is None else rot_dim
    if qkv.stride(1) != 1:
        raise ValueError("qk_norm_rope: qkv must have contiguous rows")
    q_w, k_w = _vec(q_w, D, "q_w"), _vec(k_w, D, "k_w")
    _rope_tables_ok(cos_t, sin_t, D, rot_dim, "qk_norm_rope")
    if pos.dtype != torch.int32 or pos.numel() != M:
        raise ValueError("qk_norm_rope: pos must be int32 (M,)")
    pos = pos.contiguous()  # held across the call
    check(lib().od_qk_norm_rope_ex(ptr(qkv), qkv.stride(0), M, n_heads_q, n_heads_k, D, rot_dim, int(bool(offset)),
                                   ptr(q_w), ptr(k_w), ptr(cos_t), ptr(sin_t), cos_t.shape[0], ptr(pos), float(eps),
                                   stream_of(qkv)),
          "od_qk_norm_rope_ex")


def qk_norm_rope_kv_append(qkv: torch.Tensor, B: int, S: int, n_heads_q: int, n_heads_k: int, D: int, q_w, k_w,
                           cos_t, sin_t, pos, eps: float, k_cache, v_cache, rot_dim: int | None = None,
                           offset: bool = False) -> None:
    """qk_norm_rope on qkv (B S, >= (Hq + 2 Hk) D), then the new tokens' key heads (after RoPE) and value heads
    quantized per (token, head) and written at positions length .. length + S - 1 of the Int8KVCache pair, in one
    pass (the bytes kv_quant_append writes for the same bf16 K/V). The caches' lengths are advanced."""
    require_gpu(qkv, q_w, k_w, cos_t, sin_t, pos, k_cache.q, v_cache.q, name="qk_norm_rope_kv_append")
    _lib.bf16_bits(qkv)
    if qkv.stride(1) != 1 or qkv.shape[0] != B * S:
        raise ValueError("qk_norm_rope_kv_append: qkv must be (B S, ...) with contiguous rows")
    q_w, k_w = _vec(q_w, D, "q_w"), _vec(k_w, D, "k_w")
    rot_dim = D if rot_dim is None else rot_dim
    _rope_tables_ok(cos_t, sin_t, D, rot_dim, "qk_norm_rope_kv_append")
    if pos.dtype != torch.int32 or pos.numel() != B * S:
        raise ValueError("qk_norm_rope_kv_append: pos must be int32 (B S,)")
    pos = pos.contiguous()  # held across the call
    n0 = k_cache.length
    if v_cache.length != n0 or k_cache.q.shape != (B, n_heads_k, k_cache.capacity, D) or \
            v_cache.q.shape != k_cache.q.shape:
        raise ValueError("qk_norm_rope_kv_append: K/V caches must match (B, Hkv, cap, D) at the same length")
    if n0 + S > k_cache.capacity:
        raise ValueError(f"qk_norm_rope_kv_append: {n0} + {S} tokens exceed the capacity {k_cache.capacity}")
    check(lib().od_qk_norm_rope_kv_append_ex(ptr(qkv), qkv.stride(0), B, S, n_heads_q, n_heads_k, D, rot_dim,
                                             int(bool(offset)), ptr(q_w), ptr(k_w), ptr(cos_t), ptr(sin_t),
                                             cos_t.shape[0], ptr(pos), float(eps), ptr(k_cache.q), ptr(k_cache.scale),
                                             ptr(v_cache.q), ptr(v_cache.scale), k_cache.capacity, n0, stream_of(qkv)),
          "od_qk_norm_rope_kv_append_ex")
    k_cache.length += S
    v_cache.length += S
    for c in (k_cache, v_cache):
        if hasattr(c, "touch"):
            c.touch()


_SPLITK_WS: dict = {}


def splitk_workspace(M: int, N: int, Kp: int, device) -> torch.Tensor | None:
    """The int32 workspace od_w8a8_gemm_ws splits K with for this shape on `device` (None when its plan does not
    split: enough 256-row tiles to fill the chip). The plan depends only on the shape and the device's CU count, so
    the size is cached."""
    device = torch.device(device)
    key = (device.index, M, N, Kp)
    n = _SPLITK_WS.get(key)
    if n is None:
        v = ctypes.c_int64(0)
        with torch.cuda.device(device):
            check(lib().od_w8a8_gemm_ws_size(M, N, Kp, ctypes.byref(v)), "od_w8a8_gemm_ws_size")
        n = _SPLITK_WS[key] = v.value
    return torch.empty(n, dtype=torch.int32, device=device) if n else None


def w8a8_gemm(a: torch.Tensor, sa: torch.Tensor, w: torch.Tensor, sw: torch.Tensor, bias=None, residual=None,
              out: torch.Tensor | None = None, want_out: bool = True, want_acc: bool = False):
    """int8 a (M, Kp) x int8 w (N, Kp)^T -> bf16 (M, N) = bf16(float(acc) sa[m] sw[n] + bias + residual); Kp is
    the padded row length (multiple of 16; padding columns are zero in both operands). Returns out, or (out, acc int32 (M, N)) with want_acc."""
    require_gpu(a, sa, w, sw, bias, residual, out, name="w8a8_gemm")
    if a.dtype != torch.int8 or w.dtype != torch.int8:
        raise TypeError("w8a8_gemm: a and w must be int8")
    M, Kp = a.shape
    N = w.shape[0]
    if w.shape[1] != Kp:
        raise ValueError(f"w8a8_gemm: a has {Kp} columns, w has {w.shape[1]}")
    sa, sw = _scales(sa, M, "w8a8_gemm: sa"), _scales(sw, N, "w8a8_gemm: sw")  # kept alive across the launch
    if want_out:
        out = _check_out(out, (M, N), a.device, "w8a8_gemm")
    acc = torch.empty(M, N, dtype=torch.int32, device=a.device) if want_acc else None
    if residual is not None:
        _lib.bf16_bits(residual)
        if residual.shape != (M, N) or residual.stride(-1) != 1:
            raise ValueError("w8a8_gemm: residual must be (M, N) with contiguous rows")
    if bias is not None:
        _lib.bf16_bits(bias)
        bias = bias.contiguous()
    o = out if want_out else None
    ws = splitk_workspace(M, N, Kp, a.device) if want_out and not want_acc else None
    if ws is not None:
        # small M: split-K through the workspace (bit-identical to the one-pass GEMM)
        check(lib().od_w8a8_gemm_ws(ptr(a), a.stride(0), ptr(sa), ptr(w), w.stride(0), ptr(sw), ptr(bias),
                                    ptr(residual), residual.stride(0) if residual is not None else 0, ptr(o),
                                    o.stride(0), M, N, Kp, 0, ptr(ws), ws.numel(), stream_of(a)), "od_w8a8_gemm_ws")
        return o
    check(lib().od_w8a8_gemm(ptr(a), a.stride(0), ptr(sa), ptr(w), w.stride(0), ptr(sw),
                             ptr(bias), ptr(residual), residual.stride(0) if residual is not None else 0, ptr(o),
                             o.stride(0) if o is not None else 0, ptr(acc), N if acc is not None else 0, M, N, Kp,
                             stream_of(a)), "od_w8a8_gemm")
    if want_acc:
        return o, acc
    return o


def interleave_gate_up(w: torch.Tensor) -> torch.Tensor:
    """Rows [gate (F); up (F)] -> [gate 0, up 0, gate 1, up 1, ...], the layout w8a8_gemm_swiglu takes (works on
    weights or per-row scales)."""
    F = w.shape[0] // 2
    return torch.stack([w[:F], w[F:]], 1).reshape(w.shape)


def w8a8_gemm_swiglu(a: torch.Tensor, sa: torch.Tensor, w: torch.Tensor, sw: torch.Tensor,
                     out: torch.Tensor | None = None) -> torch.Tensor:
    """int8 a (M, Kp) x interleaved gate/up int8 w (2F, Kp)^T -> bf16 (M, F) = bf16(bf16(silu(g)) * u) with g, u
    the bf16 gate and up outputs of w8a8_gemm (rows 2f and 2f + 1 of w)."""
    require_gpu(a, sa, w, sw, out, name="w8a8_gemm_swiglu")
    if a.dtype != torch.int8 or w.dtype != torch.int8:
        raise TypeError("w8a8_gemm_swiglu: a and w must be int8")
    M, Kp = a.shape
    N = w.shape[0]
    if w.shape[1] != Kp or N % 2:
        raise ValueError("w8a8_gemm_swiglu: w must be (2F, Kp) with a's Kp")
    sa, sw = _scales(sa, M, "w8a8_gemm_swiglu: sa"), _scales(sw, N, "w8a8_gemm_swiglu: sw")
    out = _check_out(out, (M, N // 2), a.device, "w8a8_gemm_swiglu")
    ws = splitk_workspace(M, N, Kp, a.device)
    if ws is not None:
        check(lib().od_w8a8_gemm_ws(ptr(a), a.stride(0), ptr(sa), ptr(w), w.stride(0), ptr(sw), None, None, 0,
                                    ptr(out), out.stride(0), M, N, Kp, 1, ptr(ws), ws.numel(), stream_of(a)),
              "od_w8a8_gemm_ws")
        return out
    check(lib().od_w8a8_gemm_swiglu(ptr(a), a.stride(0), ptr(sa), ptr(w), w.stride(0),
                                    ptr(sw), ptr(out), out.stride(0), M, N, Kp, stream_of(a)),
          "od_w8a8_gemm_swiglu")
    return out


def kv_quant_append(x: torch.Tensor, q_cache: torch.Tensor, s_cache: torch.Tensor, n0: int) -> None:
    """Quantize x (B, H, n, D) bf16 per (token, head) and write it at positions n0..n0+n-1 of the int8 cache
    q_cache (B, H, cap, D) and its fp32 scales s_cache (B, H, cap) (Int8Tensor.quantize on the new tokens only,
    state_cache.py:79)."""
    require_gpu(x, q_cache, s_cache, name="kv_quant_append")
    _lib.bf16_bits(x)
    B, H, n, D = x.shape
    if q_cache.dtype != torch.int8 or s_cache.dtype != torch.float32:
        raise TypeError("kv_quant_append: cache must be int8 with fp32 scales")
    if q_cache.shape[:2] != (B, H) or q_cache.shape[3] != D or s_cache.shape != q_cache.shape[:3]:
        raise ValueError("kv_quant_append: cache shape does not match the new rows")
    if not (q_cache.is_contiguous() and s_cache.is_contiguous()):
        raise ValueError("kv_quant_append: cache buffers must be contiguous")
    if x.stride(-1) != 1:
        x = x.contiguous()
    cap = q_cache.shape[2]
    check(lib().od_kv_quant_append(ptr(x), B, H, n, D, x.stride(0), x.stride(1), x.stride(2), ptr(q_cache),
                                   ptr(s_cache), cap, n0, stream_of(x)), "od_kv_quant_append")


def kv_copy_rows(src_q: torch.Tensor, src_s: torch.Tensor, dst_q: torch.Tensor, dst_s: torch.Tensor, segs) -> None:
    """Copy runs of int8 cache rows and their fp32 scales, bytes unchanged, in one launch (per 32 runs).
    src_q (n_mats, H, src_cap, D) int8 and src_s (n_mats, H, src_cap) fp32, each matrix [H, cap, D] contiguous (any
    stride between matrices); dst_q / dst_s likewise with their own capacity. segs: (src_row, dst_row, n_rows) runs,
    each copied for every matrix and head."""
    require_gpu(src_q, src_s, dst_q, dst_s, name="kv_copy_rows")
    n_mats, H, src_cap, D = src_q.shape
    dst_cap = dst_q.shape[2]
    if src_q.dtype != torch.int8 or dst_q.dtype != torch.int8 or src_s.dtype != torch.float32 or \
            dst_s.dtype != torch.float32:
        raise TypeError("kv_copy_rows: int8 rows with fp32 scales")
    if dst_q.shape != (n_mats, H, dst_cap, D) or src_s.shape != (n_mats, H, src_cap) or \
            dst_s.shape != (n_mats, H, dst_cap):
        raise ValueError("kv_copy_rows: source and destination shapes do not match")
    for q, s in ((src_q, src_s), (dst_q, dst_s)):
        cap = q.shape[2]
        if q.stride()[1:] != (cap * D, D, 1) or s.stride()[1:] != (cap, 1):
            raise ValueError("kv_copy_rows: every matrix must be a contiguous [H, cap, D] block")
    flat = [int(v) for seg in segs for v in seg]
    if len(flat) % 3:
        raise ValueError("kv_copy_rows: segments are (src_row, dst_row, n_rows) triples")
    arr = (ctypes.c_int64 * max(len(flat), 1))(*flat)
    check(lib().od_kv_copy_rows(ptr(src_q), ptr(src_s), src_q.stride(0), src_s.stride(0), src_cap, ptr(dst_q),
                                ptr(dst_s), dst_q.stride(0), dst_s.stride(0), dst_cap, n_mats, H, D,
                                ctypes.cast(arr, ctypes.c_void_p), len(flat) // 3, stream_of(src_q)),
          "od_kv_copy_rows")


def _rows_aligned(t: torch.Tensor) -> torch.Tensor:
    """Last dim contiguous, 16-byte aligned base and strides that are multiples of 8 elements (16-byte loads)."""
    if t.stride(-1) != 1 or t.data_ptr() % 16 or any(s % 8 for s in t.stride()[:-1]):
        t = t.contiguous()
    return t


def row_start_of(row_counts, device) -> tuple[torch.Tensor, int]:
    """Device int32 offsets (Ns + 1,) of option rows grouped by state, and the largest group, from host counts.
    Validated here on the host, so the kernel never reads an offset past the rows it was given."""
    counts = [int(c) for c in row_counts]
    if not counts or min(counts) < 0:
        raise ValueError("row_counts must be a non-empty list of non-negative ints")
    starts = [0]
    for c in counts:
        starts.append(starts[-1] + c)
    return torch.tensor(starts, dtype=torch.int32).to(device, non_blocking=True), max(counts)


def split_count(slot_tiles: int, T: int, n_cu: int = 256, wg_per_cu: int = 2, min_blocks: int = 4) -> int:
    """Key-range splits for the block-image paths (od_branched_attn_split / _staged / _staged2): with few slot tiles
    over a long state, n splits of `slot_tiles` workgroups cost ceil(slot_tiles n / (n_cu wg_per_cu)) rounds of
    ceil(blocks / n) 64-key blocks plus a workgroup's fixed work (about two blocks: the queries, the own keys, the
    partial); the n of least cost (the smallest on ties), keeping at least `min_blocks` blocks per split. Filling
    the CUs once with longer key ranges measured faster than two rounds of shorter ones (the 128-slot probe over
    32768-key states: 8 splits 266 us, 16 splits 280 us)."""
    blocks = (T + 63) // 64
    cap = max(n_cu * wg_per_cu, 1)
    n_max = max(1, min(blocks // min_blocks, 256))
    best, best_cost = 1, None
    for n in range(1, n_max + 1):
        cost = -(-slot_tiles * n // cap) * (-(-blocks // n) + 2)
        if best_cost is None or cost < best_cost:
            best, best_cost = n, cost
    return best


# The KV-streaming kernel (od_branched_attn_stream): one wave holds every query slot of a (state, head).
STREAM_D = 128
STREAM_MAX_SLOTS = 32


# Workspaces of the streaming kernel's key-range splits, per (device, stream, size): the split partials and LSEs, then
# one merge counter per (state, KV head) that must be zero when a call starts; the kernel sets every counter back to
# zero, so a workspace zeroed once serves every later call made on its stream.
_STREAM_WS: dict = {}


def stream_workspace(nsplit: int, R: int, Hq: int, t: int, D: int, Ns: int, Hkv: int, device) -> torch.Tensor:
    n = nsplit * R * Hq * t * (D + 1) + Ns * Hkv
    device = torch.device(device)
    key = (device.index, torch.cuda.current_stream(device).cuda_stream, n)
    ws = _STREAM_WS.get(key)
    if ws is None:
        ws = _STREAM_WS[key] = torch.zeros(n, dtype=torch.float32, device=device)
    return ws


def stream_split_count(Ns: int, Hkv: int, T: int, n_cu: int = 256, min_tiles: int = 16) -> int:
    """Key-range splits for od_branched_attn_stream. Its 8-wave workgroups take half of every SIMD's registers, so a
    CU runs one at a time, and n splits of Ns x Hkv (state, head) pairs take ceil(pairs n / n_cu) rounds of
    ceil(tiles / n) 32-key tiles plus a workgroup's fixed work (about two tiles per wave: the queries, the wave
    merge, the partials): the n of least cost (the smallest on ties), keeping at least `min_tiles` tiles per split.
    With fewer, larger splits the state is read by fewer concurrent streams, which measured faster than filling the
    CUs twice over."""
    pairs = max(Ns * Hkv, 1)
    tiles = (T + 31) // 32
    n_max = max(1, min(tiles // min_tiles, 256))
    best, best_cost = 1, None
    for n in range(1, n_max + 1):
        cost = -(-pairs * n // n_cu) * (-(-tiles // n) + 16)
        if best_cost is None or cost < best_cost:
            best, best_cost = n, cost
    return best


_CU_COUNT: dict = {}


def cu_count(device) -> int:
    """Compute units of a GPU (cached per device index)."""
    device = torch.device(device)
    idx = device.index if device.index is not None else torch.cuda.current_device()
    n = _CU_COUNT.get(idx)
    if n is None:
        n = _CU_COUNT[idx] = torch.cuda.get_device_properties(idx).multi_processor_count
    return n


# The staged path writes each state block's image (twice the int8 bytes) once and lets every slot tile copy it
# instead of converting it; it pays off when several tiles read each (state, head).
STAGE_MIN_TILES = 4


def stage_size(Ns: int, Hkv: int, length: int, D: int) -> int:
    """Bytes of the block images of Ns x Hkv heads of `length` keys (od_attn_stage_size)."""
    nbytes = ctypes.c_int64(0)
    check(lib().od_attn_stage_size(int(Ns), int(Hkv), int(length), int(D), ctypes.byref(nbytes)),
          "od_attn_stage_size")
    return nbytes.value


def stage_state(kq, ks, vq, vs, length: int, scale: float, kvalid=None, out=None, dequant: str = "bf16"):
    """Block images of an int8 state for od_branched_attn_staged (od_attn_stage): kq/vq (Ns, Hkv, cap, D) int8,
    ks/vs (Ns, Hkv, cap) fp32, the first `length` tokens, the softmax scale of the attention that reads them,
    kvalid (Ns, length) uint8 or None, dequant "bf16" (the reference's materialize) or "fp32" (exact q * s).
    Returns a uint8 device buffer of od_attn_stage_size bytes (`out` is reused when it is large enough)."""
    require_gpu(kq, ks, vq, vs, kvalid, out, name="stage_state")
    Ns, Hkv, cap, D = kq.shape
    nbytes = stage_size(Ns, Hkv, length, D)
    if out is None or out.numel() < nbytes:
        out = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=kq.device)
    elif out.dtype != torch.uint8 or not out.is_contiguous():
        raise ValueError("stage_state: out must be a contiguous uint8 buffer")
    check(lib().od_attn_stage(ptr(kq), ptr(ks), ptr(vq), ptr(vs), ptr(kvalid), Ns, Hkv, int(length), cap, D,
                              float(scale), _lib.dequant_code(dequant), ptr(out), out.numel(), stream_of(kq)),
          "od_attn_stage")
    return out


def stage_state_bf16(k, v, length: int, scale: float, kvalid=None, out=None):
    """Block images of a DENSE bf16 state (od_attn_stage_bf16): k/v (Ns, Hkv, >= length, D) bf16 (any strides that
    are multiples of 8 elements, last dim contiguous), the first `length` tokens, kvalid (Ns, length) uint8 or None.
    Returns a uint8 device buffer for branched_attn_images."""
    require_gpu(k, v, kvalid, out, name="stage_state_bf16")
    _lib.bf16_bits(k)
    _lib.bf16_bits(v)
    Ns, Hkv, _, D = k.shape
    if v.shape[:2] != (Ns, Hkv) or v.shape[3] != D or min(k.shape[2], v.shape[2]) < length:
        raise ValueError("stage_state_bf16: k and v must be (Ns, Hkv, >= length, D)")
    k, v = _rows_aligned(k), _rows_aligned(v)
    nbytes = stage_size(Ns, Hkv, length, D)
    if out is None or out.numel() < nbytes:
        out = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=k.device)
    check(lib().od_attn_stage_bf16(ptr(k), *k.stride()[:3], ptr(v), *v.stride()[:3], ptr(kvalid), Ns, Hkv,
                                   int(length), D, float(scale), ptr(out), out.numel(), stream_of(k)),
          "od_attn_stage_bf16")
    return out


def branched_attn_images(q, k_own, v_own, img, Ns: int, T: int, scale: float, row_start=None, max_rows=None,
                         out=None, return_lse: bool = False, n_split=None):
    """The branched attention over block images already built (stage_state / stage_state_bf16) for Ns states of T
    keys: od_branched_attn_staged. q (R, Hq, t, D), k_own/v_own (R, Hkv, t, D) bf16; rows grouped by state through
    row_start/max_rows (None: one state). Returns out [, lse] as branched_attn."""
    require_gpu(q, k_own, v_own, img, row_start, out, name="branched_attn_images")
    for x in (q, k_own, v_own):
        _lib.bf16_bits(x)
    R, Hq, t, D = q.shape
    Hkv = k_own.shape[1]
    if k_own.shape != (R, Hkv, t, D) or v_own.shape != (R, Hkv, t, D):
        raise ValueError("branched_attn_images: own k/v must be (R, Hkv, t, D)")
    if T > 0 and (img.dtype != torch.uint8 or img.numel() < stage_size(Ns, Hkv, T, D)):
        raise ValueError("branched_attn_images: the block images are smaller than the state needs")
    if row_start is None:
        if Ns != 1:
            raise ValueError("branched_attn_images: row_start is required with several states")
        max_rows = R
    elif row_start.dtype != torch.int32 or row_start.numel() != Ns + 1 or max_rows is None:
        raise ValueError("branched_attn_images: row_start must be int32 (Ns + 1,) with max_rows")
    q, k_own, v_own = _rows_aligned(q), _rows_aligned(k_own), _rows_aligned(v_own)
    out = _check_out(out, (R, Hq, t, D), q.device, "branched_attn_images")
    lse = torch.empty(R, Hq, t, dtype=torch.float32, device=q.device) if return_lse else None
    tiles = -(-(int(max_rows) * t * (Hq // Hkv)) // 128)
    if n_split is None:
        n_split = split_count(tiles * Hkv * Ns, T, cu_count(q.device), 1 if D == 256 else 2)
    ws = torch.empty(n_split * R * Hq * t * (D + 1), dtype=torch.float32, device=q.device) if n_split > 1 else None
    check(lib().od_branched_attn_staged(ptr(q), *q.stride()[:3], ptr(k_own), *k_own.stride()[:3], ptr(v_own),
                                        *v_own.stride()[:3], ptr(img), img.numel(), ptr(row_start), int(max_rows),
                                        ptr(out), *out.stride()[:3], ptr(lse), R, Hq, Hkv, t, D, Ns, T, float(scale),
                                        int(n_split), ptr(ws), 0 if ws is None else ws.numel(), stream_of(q)),
          "od_branched_attn_staged")
    return (out, lse) if return_lse else out


def branched_attn_two_level(q, k_own, v_own, img, n_states: int, T: int, img2, T2: int, scale: float,
                            group_state=None, row_start=None, max_rows=None, out=None, return_lse: bool = False,
                            n_split=None):
    """The branched attention over a two-level prefix (od_branched_attn_staged2): the rows of group g attend the
    block images of state group_state[g] (img: stage_state of n_states states of T keys), then group g's own
    second-level images (img2: stage_state_bf16 of the groups' dense K/V, T2 keys), then their own tokens causally.
    q (R, Hq, t, D), k_own/v_own (R, Hkv, t, D) bf16; rows grouped by group through row_start (int32 (G + 1,)) and
    max_rows; group_state int32 (G,) device tensor or None (group g reads state g). Returns out [, lse]."""
    require_gpu(q, k_own, v_own, img, img2, group_state, row_start, out, name="branched_attn_two_level")
    for x in (q, k_own, v_own):
        _lib.bf16_bits(x)
    R, Hq, t, D = q.shape
    Hkv = k_own.shape[1]
    if k_own.shape != (R, Hkv, t, D) or v_own.shape != (R, Hkv, t, D):
        raise ValueError("branched_attn_two_level: own k/v must be (R, Hkv, t, D)")
    if row_start is None:
        G, max_rows = 1, R
    else:
        if row_start.dtype != torch.int32 or max_rows is None:
            raise ValueError("branched_attn_two_level: row_start must be int32 (G + 1,) with max_rows")
        G = row_start.numel() - 1
    if group_state is not None and (group_state.dtype != torch.int32 or group_state.numel() != G):
        raise ValueError("branched_attn_two_level: group_state must be int32 (G,)")
    if T > 0 and (img is None or img.numel() < stage_size(n_states, Hkv, T, D)):
        raise ValueError("branched_attn_two_level: the level-1 images are smaller than the states need")
    if T2 > 0 and (img2 is None or img2.numel() < stage_size(G, Hkv, T2, D)):
        raise ValueError("branched_attn_two_level: the level-2 images are smaller than the groups need")
    q, k_own, v_own = _rows_aligned(q), _rows_aligned(k_own), _rows_aligned(v_own)
    out = _check_out(out, (R, Hq, t, D), q.device, "branched_attn_two_level")
    lse = torch.empty(R, Hq, t, dtype=torch.float32, device=q.device) if return_lse else None
    tiles = -(-(int(max_rows) * t * (Hq // Hkv)) // 128)
    if n_split is None:
        n_split = split_count(tiles * Hkv * G, T + T2, cu_count(q.device), 1 if D == 256 else 2)
    ws = torch.empty(n_split * R * Hq * t * (D + 1), dtype=torch.float32, device=q.device) if n_split > 1 else None
    check(lib().od_branched_attn_staged2(ptr(q), *q.stride()[:3], ptr(k_own), *k_own.stride()[:3], ptr(v_own),
                                         *v_own.stride()[:3], ptr(img), 0 if img is None else img.numel(),
                                         ptr(group_state), int(n_states), int(T), ptr(img2),
                                         0 if img2 is None else img2.numel(), int(T2), ptr(row_start), int(max_rows),
                                         ptr(out), *out.stride()[:3], ptr(lse), R, Hq, Hkv, t, D, G, float(scale),
                                         int(n_split), ptr(ws), 0 if ws is None else ws.numel(), stream_of(q)),
          "od_branched_attn_staged2")
    return (out, lse) if return_lse else out


def uses_staging(max_rows: int, t: int, n_heads_q: int, n_heads_k: int) -> bool:
    """Whether branched_attn takes the staged path by itself for this row layout (at least STAGE_MIN_TILES slot
    tiles of 128 per (state, head))."""
    return -(-(int(max_rows) * t * (n_heads_q // n_heads_k)) // 128) >= STAGE_MIN_TILES


def branched_attn(q, k_own, v_own, kq, ks, vq, vs, scale: float, kvalid=None, row_counts=None, length=None,
                  out=None, return_lse: bool = False, row_start=None, max_rows=None, n_split=None, staged=None,
                  stage_buf=None, dequant: str = "bf16", images=None, static_workspace: bool = False,
                  stream=None):
    """Branched option-row attention over int8 states. q (R, Hq, t, D) bf16; k_own/v_own (R, Hkv, t, D) bf16;
    kq/vq (Ns, Hkv, cap, D) int8 of which the first T tokens are used (T = `length`, else kvalid.shape[1], else
    cap); ks/vs (Ns, Hkv, cap) fp32; kvalid (Ns, T) bool/uint8 or None.
    Rows are grouped by state: row_counts (host ints, one per state) or a prebuilt (row_start, max_rows) pair from
    row_start_of(); neither means Ns == 1. n_split: key-range splits; None picks them from the grid size
    (split_count). staged: convert the state once into block images (od_attn_stage, into `stage_buf` when given and
    large enough) and run od_branched_attn_staged over them; False runs od_branched_attn / od_branched_attn_split,
    which convert in every workgroup (same results, bit for bit); None stages when at least STAGE_MIN_TILES slot
    tiles read each (state, head), so that the conversion is shared. images: block images already built by
    stage_state for this state, length, scale, mask and dequant (the staged path then skips od_attn_stage; the
    caller keeps them valid). dequant: "bf16", the reference's materialize bf16(q * bf16(s)) (quant.py:45,
    prefix_attn.py:145-149), or "fp32", the exact q * s. static_workspace: the direct path's split partials go to
    the library's static scratch (od_branched_attn_split_noalloc: nothing is allocated for them; calls on one GPU
    must not overlap). stream: the KV-streaming kernel for at most 32 query slots per (state, head)
    (od_branched_attn_stream, head_dim 128); None takes it when the caller chose no other path (staged, images and
    static_workspace left at their defaults) and the shape allows it. Returns out (R, Hq, t, D) bf16
    [, lse (R, Hq, t) fp32]."""
    require_gpu(q, k_own, v_own, kq, ks, vq, vs, kvalid, row_start, out, name="branched_attn")
    for x in (q, k_own, v_own):
        _lib.bf16_bits(x)
    R, Hq, t, D = q.shape
    Hkv = k_own.shape[1]
    Ns, _, cap, _ = kq.shape
    if kq.dtype != torch.int8 or vq.dtype != torch.int8 or ks.dtype != torch.float32 or vs.dtype != torch.float32:
        raise TypeError("branched_attn: state must be int8 with fp32 scales")
    if k_own.shape != (R, Hkv, t, D) or v_own.shape != (R, Hkv, t, D):
        raise ValueError("branched_attn: own k/v must be (R, Hkv, t, D)")
    if kq.shape != (Ns, Hkv, cap, D) or vq.shape != kq.shape or ks.shape != (Ns, Hkv, cap) or vs.shape != ks.shape:
        raise ValueError("branched_attn: state K/V must be (Ns, Hkv, cap, D) with scales (Ns, Hkv, cap)")
    if not (kq.is_contiguous() and vq.is_contiguous() and ks.is_contiguous() and vs.is_contiguous()):
        raise ValueError("branched_attn: state buffers must be contiguous")
    T = int(length) if length is not None else (cap if kvalid is None else kvalid.shape[1])
    if T < 0 or T > cap:
        raise ValueError(f"branched_attn: length {T} outside [0, {cap}]")
    if kvalid is not None:
        if kvalid.shape != (Ns, T) or T > cap:
            raise ValueError("branched_attn: kvalid must be (Ns, T) with T <= cap")
        kvalid = kvalid.to(torch.uint8).contiguous()
    if row_counts is not None:
        if len(row_counts) != Ns or sum(int(c) for c in row_counts) != R:
            raise ValueError("branched_attn: row_counts must have one entry per state and sum to R")
        row_start, max_rows = row_start_of(row_counts, q.device)
    if row_start is None:
        if Ns != 1:
            raise ValueError("branched_attn: row_start is required with several states")
        max_rows = R
    else:
        if row_start.dtype != torch.int32 or row_start.numel() != Ns + 1:
            raise ValueError("branched_attn: row_start must be int32 (Ns + 1,)")
        if max_rows is None:
            raise ValueError("branched_attn: max_rows is required with row_start")
    dq = _lib.dequant_code(dequant)
    q, k_own, v_own = _rows_aligned(q), _rows_aligned(k_own), _rows_aligned(v_own)
    out = _check_out(out, (R, Hq, t, D), q.device, "branched_attn")
    lse = torch.empty(R, Hq, t, dtype=torch.float32, device=q.device) if return_lse else None
    slots = int(max_rows) * t * (Hq // Hkv)  # query slots per (state, head)
    if stream is None:
        stream = (staged is None and images is None and not static_workspace and D == STREAM_D
                  and slots <= STREAM_MAX_SLOTS and T > 0)
    if stream:
        if D != STREAM_D or slots > STREAM_MAX_SLOTS:
            raise ValueError(f"branched_attn: the streaming kernel takes head_dim {STREAM_D} and at most "
                             f"{STREAM_MAX_SLOTS} slots per (state, head), not D={D} with {slots}")
        nsp = stream_split_count(Ns, Hkv, T, cu_count(q.device)) if n_split is None else int(n_split)
        ws = stream_workspace(nsp, R, Hq, t, D, Ns, Hkv, q.device) if nsp > 1 else None
        check(lib().od_branched_attn_stream(ptr(q), *q.stride()[:3], ptr(k_own), *k_own.stride()[:3], ptr(v_own),
                                            *v_own.stride()[:3], ptr(kq), ptr(ks), ptr(vq), ptr(vs), ptr(kvalid),
                                            ptr(row_start), int(max_rows), ptr(out), *out.stride()[:3], ptr(lse), R,
                                            Hq, Hkv, t, D, Ns, T, cap, float(scale), dq, nsp, ptr(ws),
                                            0 if ws is None else ws.numel(), stream_of(q)), "od_branched_attn_stream")
        return (out, lse) if return_lse else out
    tiles = -(-slots // 128)  # slot tiles per (state, head)
    if n_split is None:
        n_split = split_count(tiles * Hkv * Ns, T, cu_count(q.device), 1 if D == 256 else 2)
    if staged is None:
        staged = images is not None or tiles >= STAGE_MIN_TILES
    if static_workspace:
        staged = False
    ws = None
    if n_split > 1 and not static_workspace:
        ws = torch.empty(n_split * R * Hq * t * (D + 1), dtype=torch.float32, device=q.device)
    if staged and T > 0:
        img = images if images is not None else stage_state(kq, ks, vq, vs, T, scale, kvalid, out=stage_buf,
                                                            dequant=dequant)
        if img.numel() < stage_size(Ns, Hkv, T, D):
            raise ValueError("branched_attn: the block images are smaller than the state needs")
        check(lib().od_branched_attn_staged(ptr(q), *q.stride()[:3], ptr(k_own), *k_own.stride()[:3], ptr(v_own),
                                            *v_own.stride()[:3], ptr(img), img.numel(), ptr(row_start),
                                            int(max_rows), ptr(out), *out.stride()[:3], ptr(lse), R, Hq, Hkv, t, D,
                                            Ns, T, float(scale), int(n_split), ptr(ws),
                                            0 if ws is None else ws.numel(), stream_of(q)),
              "od_branched_attn_staged")
    elif static_workspace:
        check(lib().od_branched_attn_split_noalloc(ptr(q), *q.stride()[:3], ptr(k_own), *k_own.stride()[:3],
                                                   ptr(v_own), *v_own.stride()[:3], ptr(kq), ptr(ks), ptr(vq),
                                                   ptr(vs), ptr(kvalid), ptr(row_start), int(max_rows), ptr(out),
                                                   *out.stride()[:3], ptr(lse), R, Hq, Hkv, t, D, Ns, T, cap,
                                                   float(scale), dq, int(n_split), stream_of(q)),
              "od_branched_attn_split_noalloc")
    elif n_split > 1:
        check(lib().od_branched_attn_split(ptr(q), *q.stride()[:3], ptr(k_own), *k_own.stride()[:3], ptr(v_own),
                                           *v_own.stride()[:3], ptr(kq), ptr(ks), ptr(vq), ptr(vs), ptr(kvalid),
                                           ptr(row_start), int(max_rows), ptr(out), *out.stride()[:3], ptr(lse), R,
                                           Hq, Hkv, t, D, Ns, T, cap, float(scale), dq, int(n_split), ptr(ws),
                                           ws.numel(), stream_of(q)), "od_branched_attn_split")
    else:
        check(lib().od_branched_attn(ptr(q), *q.stride()[:3], ptr(k_own), *k_own.stride()[:3], ptr(v_own),
                                     *v_own.stride()[:3], ptr(kq), ptr(ks), ptr(vq), ptr(vs), ptr(kvalid),
                                     ptr(row_start), int(max_rows), ptr(out), *out.stride()[:3], ptr(lse), R, Hq, Hkv,
                                     t, D, Ns, T, cap, float(scale), dq, stream_of(q)), "od_branched_attn")
    return (out, lse) if return_lse else out


def wide_attn(q, k, v, scale: float, kvalid=None, causal: bool = True, return_lse: bool = False, out=None):
    """Flash attention over bf16 K/V (od_wide_attn). q (B, H, T, DK), k (B, G, S, DK), v (B, G, S, DV) bf16 with
    DK % 8 == 0 and DK <= 512, DV in {64, 128, 256}; kvalid (B, S) bool/uint8 or None; scale > 0 and finite.
    Queries are the last T of the S positions. Returns out (B, H, T, DV) bf16 [, lse (B, H, T) fp32]."""
    require_gpu(q, k, v, kvalid, out, name="wide_attn")
    for x in (q, k, v):
        _lib.bf16_bits(x)
    B, H, T, DK = q.shape
    G, S, DV = k.shape[1], k.shape[2], v.shape[-1]
    if k.shape != (B, G, S, DK) or v.shape[:3] != (B, G, S):
        raise ValueError("wide_attn: k must be (B, G, S, DK) and v (B, G, S, DV)")
    if kvalid is not None:
        if kvalid.shape != (B, S):
            raise ValueError("wide_attn: kvalid must be (B, S)")
        kvalid = kvalid.to(torch.uint8).contiguous()
    q, k, v = _rows_aligned(q), _rows_aligned(k), _rows_aligned(v)
    out = _check_out(out, (B, H, T, DV), q.device, "wide_attn")
    lse = torch.empty(B, H, T, dtype=torch.float32, device=q.device) if return_lse else None
    check(lib().od_wide_attn(ptr(q), *q.stride()[:3], ptr(k), *k.stride()[:3], ptr(v), *v.stride()[:3], ptr(kvalid),
                             kvalid.stride(0) if kvalid is not None else 0, ptr(out), *out.stride()[:3], ptr(lse), B, H,
                             G, T, S, DK, DV, 1 if causal else 0, float(scale), stream_of(q)), "od_wide_attn")
    return (out, lse) if return_lse else out


def _lm_h_operands(h: torch.Tensor, K: int):
    """(hb bf16 rows for the matmul, hn rows for the target term, hn_fp32 flag, M, leading shape)."""
    if h.shape[-1] != K:
        raise ValueError(f"h has {h.shape[-1]} features, the table {K}")
    lead = h.shape[:-1]
    h2 = h.reshape(-1, K)
    if h2.dtype == torch.bfloat16:
        hb = _rows_aligned(h2)
        return hb, hb, 0, h2.shape[0], lead
    if h2.dtype == torch.float32:
        ok = h2.stride(-1) == 1 and h2.stride(0) % 4 == 0 and h2.data_ptr() % 16 == 0
        hb = h2.to(torch.bfloat16).contiguous()  # the matmul operand, bf16(h) as the reference's h.to(bfloat16)
        return hb, (h2 if ok else h2.contiguous()), 1, h2.shape[0], lead
    raise TypeError(f"h must be bfloat16 or float32, got {h2.dtype}")


def _lm_common(h, tok, out, M, lead, V):
    if tok.shape != lead:
        raise ValueError(f"tok shape {tuple(tok.shape)} != h's leading shape {tuple(lead)}")
    t32 = tok.reshape(-1).to(torch.int32).contiguous()
    if out is None:
        out = torch.empty(M, dtype=torch.float32, device=h.device)
    elif out.dtype != torch.float32 or out.numel() != M or not out.is_contiguous():
        raise ValueError("out must be fp32 contiguous with one element per row")
    n = ctypes.c_int64()
    check(lib().od_lm_head_logprob_ws(M, V, ctypes.byref(n)), "od_lm_head_logprob_ws")
    ws = torch.empty(max(n.value, 1), dtype=torch.float32, device=h.device)
    return t32, out, ws


def _table_rows(t: torch.Tensor) -> torch.Tensor:
    return t if t.stride(-1) == 1 and t.stride(0) % 16 == 0 and t.data_ptr() % 16 == 0 else t.contiguous()


def lm_head_logprob(h: torch.Tensor, qweight: torch.Tensor, scale: torch.Tensor, tok: torch.Tensor,
                    out: torch.Tensor | None = None) -> torch.Tensor:
    """log softmax(h @ W^T)[tok] for the int8 table W = qweight (V, K) with per-row scales `scale` (V,) or (V, 1)
    bf16 (Backbone.token_logprob, backbone.py:164-178, over Int8Embedding / Int8Linear rows): the normaliser from the
    bf16 logits of bf16(h) against the bf16-dequantized rows, the target term in fp32. h (..., K) bf16 or fp32,
    tok (...) integer. Returns fp32 (...). One pass over the table; no (rows, V) logits are allocated."""
    require_gpu(h, qweight, scale, tok, out, name="lm_head_logprob")
    if qweight.dtype != torch.int8 or qweight.dim() != 2:
        raise TypeError("qweight must be an int8 (V, K) table")
    V, K = qweight.shape
    sc = _lib.bf16_bits(scale).reshape(-1).contiguous()
    if sc.numel() != V:
        raise ValueError(f"scale has {sc.numel()} elements, expected {V}")
    hb, hn, hn_fp32, M, lead = _lm_h_operands(h, K)
    t32, out, ws = _lm_common(h, tok, out, M, lead, V)
    w = _table_rows(qweight)
    check(lib().od_lm_head_logprob(ptr(hb), hb.stride(0), ptr(hn), hn.stride(0), hn_fp32, ptr(w), w.stride(0),
                                   ptr(sc), ptr(t32), M, V, K, ptr(out), ptr(ws), ws.numel(), stream_of(h)),
          "od_lm_head_logprob")
    return out.view(lead)


def lm_head_logprob_q4(h: torch.Tensor, qs: torch.Tensor, d: torch.Tensor, tok: torch.Tensor,
                       out: torch.Tensor | None = None) -> torch.Tensor:
    """lm_head_logprob over a Q4_0 table (Q4Table, quant.py:206-246): qs uint8 (V, K / 2) packed nibbles, d fp16
    (V, K / 32) block scales."""
    require_gpu(h, qs, d, tok, out, name="lm_head_logprob_q4")
    if qs.dtype != torch.uint8 or qs.dim() != 2 or d.dtype != torch.float16 or d.dim() != 2:
        raise TypeError("a Q4 table is qs uint8 (V, K/2) and d float16 (V, K/32)")
    V, K = qs.shape[0], qs.shape[1] * 2
    if d.shape != (V, K // 32):
        raise ValueError(f"d has shape {tuple(d.shape)}, expected {(V, K // 32)}")
    hb, hn, hn_fp32, M, lead = _lm_h_operands(h, K)
    t32, out, ws = _lm_common(h, tok, out, M, lead, V)
    q = _table_rows(qs)
    dd = d if d.stride(-1) == 1 else d.contiguous()
    check(lib().od_lm_head_logprob_q4(ptr(hb), hb.stride(0), ptr(hn), hn.stride(0), hn_fp32, ptr(q), q.stride(0),
                                      ptr(dd), dd.stride(0), ptr(t32), M, V, K, ptr(out), ptr(ws), ws.numel(),
                                      stream_of(h)),
          "od_lm_head_logprob_q4")
    return out.view(lead)


# ------------------------------------------------------------------------------------------- Gated DeltaNet layers
def gdn_prep(proj: torch.Tensor, conv_w: torch.Tensor, A_log: torch.Tensor, dt_bias: torch.Tensor, S: int, L: int,
             n_k: int, n_v: int, dk: int, dv: int, conv_in=None, seq_state=None, conv_out: bool | torch.Tensor = False,
             out=None, seq_len=None):
    """od_gdn_prep: the conv + SiLU, l2norm and gates of a GDN layer. proj (S L, >= proj_out) bf16 with contiguous
    rows ([qkv | z | b | a]); conv_w (C, 4) bf16; A_log, dt_bias (n_v,) bf16; conv_in (n_states, 3, C) bf16 or
    None; seq_state int32 (S,) or None. conv_out: True for a new (S, 3, C) tensor of the new conv states, or a
    contiguous tensor of that shape to write them into (not conv_in's memory: other tokens still read it). out:
    preallocated (qk, v, g, beta). Returns (qk (S L, 2 n_k dk), v (S L, n_v dv), g, beta (S L, n_v) fp32, the new
    conv states or None). seq_len: int32 (S,) real tokens of right-padded sequences (the reference's padded
    continuation: pads leave the recurrent state unchanged and the new conv state ends at the last real token)."""
    require_gpu(proj, conv_w, A_log, dt_bias, conv_in, seq_state, seq_len, name="gdn_prep")
    for t in (proj, conv_w, A_log, dt_bias):
        _lib.bf16_bits(t)
    C = 2 * n_k * dk + n_v * dv
    M = S * L
    if proj.shape[0] != M or proj.shape[1] < C + n_v * dv + 2 * n_v or proj.stride(1) != 1:
        raise ValueError("gdn_prep: proj must be (S L, >= 2 n_k dk + 2 n_v dv + 2 n_v) with contiguous rows")
    conv_w = conv_w.contiguous()
    if conv_w.shape != (C, 4):
        raise ValueError(f"gdn_prep: conv_w must be ({C}, 4)")
    A_log, dt_bias = A_log.contiguous(), dt_bias.contiguous()
    n_states = 0
    if conv_in is not None:
        _lib.bf16_bits(conv_in)
        conv_in = conv_in.contiguous()
        if conv_in.dim() != 3 or conv_in.shape[1:] != (3, C):
            raise ValueError("gdn_prep: conv_in must be (n_states, 3, C)")
        n_states = conv_in.shape[0]
    if seq_state is not None:
        if seq_state.dtype != torch.int32 or seq_state.numel() != S:
            raise ValueError("gdn_prep: seq_state must be int32 (S,)")
        seq_state = seq_state.contiguous()
    if seq_len is not None:
        if seq_len.dtype != torch.int32 or seq_len.numel() != S:
            raise ValueError("gdn_prep: seq_len must be int32 (S,)")
        seq_len = seq_len.contiguous()
    dev = proj.device
    if out is None:
        qk = torch.empty(M, 2 * n_k * dk, dtype=torch.bfloat16, device=dev)
        v = torch.empty(M, n_v * dv, dtype=torch.bfloat16, device=dev)
        g = torch.empty(M, n_v, dtype=torch.float32, device=dev)
        beta = torch.empty(M, n_v, dtype=torch.float32, device=dev)
    else:
        qk, v, g, beta = out
        require_gpu(qk, v, g, beta, name="gdn_prep")
        for t, shape, dt in ((qk, (M, 2 * n_k * dk), torch.bfloat16), (v, (M, n_v * dv), torch.bfloat16),
                             (g, (M, n_v), torch.float32), (beta, (M, n_v), torch.float32)):
            if t.shape != shape or t.dtype != dt or not t.is_contiguous():
                raise ValueError(f"gdn_prep: out tensors must be contiguous {shape} {dt}")
    co = None
    if isinstance(conv_out, torch.Tensor):
        co = conv_out
        require_gpu(co, name="gdn_prep")
        if co.shape != (S, 3, C) or co.dtype != torch.bfloat16 or not co.is_contiguous():
            raise ValueError(f"gdn_prep: conv_out must be contiguous bf16 ({S}, 3, {C})")
        if conv_in is not None and co.data_ptr() < conv_in.data_ptr() + conv_in.numel() * 2 and \
                conv_in.data_ptr() < co.data_ptr() + co.numel() * 2:
            raise ValueError("gdn_prep: conv_out overlaps conv_in")
    elif conv_out:
        co = torch.empty(S, 3, C, dtype=torch.bfloat16, device=dev)
    check(lib().od_gdn_prep_ex(ptr(proj), proj.stride(0) if M > 1 else proj.shape[1], ptr(conv_w), ptr(conv_in),
                               ptr(seq_state), n_states, ptr(seq_len), ptr(A_log), ptr(dt_bias), S, L, n_k, n_v, dk,
                               dv, ptr(qk), ptr(v), ptr(g), ptr(beta), ptr(co), stream_of(proj)), "od_gdn_prep_ex")
    return qk, v, g, beta, co


_GDN_WS: dict = {}


def gdn_chunk_workspace_floats(S: int, L: int, n_v: int) -> int:
    key = (S, L, n_v)
    n = _GDN_WS.get(key)
    if n is None:
        v = ctypes.c_int64(0)
        check(lib().od_gdn_chunk_ws_size(S, L, n_v, ctypes.byref(v)), "od_gdn_chunk_ws_size")
        n = _GDN_WS[key] = v.value
    return n


def gdn_recurrence(qk: torch.Tensor, v: torch.Tensor, g: torch.Tensor, beta: torch.Tensor, S: int, L: int, n_k: int,
                   n_v: int, dk: int, dv: int, init=None, seq_state=None, final: bool | torch.Tensor = False,
                   out=None, chunked: bool = True):
    """The gated delta rule over S sequences of L tokens (inputs as gdn_prep returns them), starting from init
    (n_states, n_v, dk, dv) fp32 through seq_state, or zeros. final: True for a new fp32 state tensor (S, n_v, dk,
    dv), or a tensor to write it into (may be init when seq_state is None). chunked: od_gdn_recurrence_chunked (the
    chunked form on bf16 MFMA, dv a multiple of 64, with a workspace from the caching allocator) where it applies,
    else od_gdn_recurrence (token by token on the vector ALUs). Returns (o (S L, n_v dv) bf16, the final states or
    None)."""
    require_gpu(qk, v, g, beta, init, seq_state, out, name="gdn_recurrence")
    M = S * L
    if qk.shape != (M, 2 * n_k * dk) or v.shape != (M, n_v * dv) or g.shape != (M, n_v) or beta.shape != (M, n_v):
        raise ValueError("gdn_recurrence: inputs do not match S, L and the head dims")
    if g.dtype != torch.float32 or beta.dtype != torch.float32:
        raise TypeError("gdn_recurrence: g and beta must be fp32")
    qk, v, g, beta = qk.contiguous(), v.contiguous(), g.contiguous(), beta.contiguous()
    n_states = 0
    if init is not None:
        if init.dtype != torch.float32 or init.dim() != 4 or init.shape[1:] != (n_v, dk, dv) or not init.is_contiguous():
            raise ValueError("gdn_recurrence: init must be contiguous fp32 (n_states, n_v, dk, dv)")
        n_states = init.shape[0]
    if seq_state is not None:
        if seq_state.dtype != torch.int32 or seq_state.numel() != S:
            raise ValueError("gdn_recurrence: seq_state must be int32 (S,)")
        seq_state = seq_state.contiguous()
    fs = None
    if final is True:
        fs = torch.empty(S, n_v, dk, dv, dtype=torch.float32, device=qk.device)
    elif isinstance(final, torch.Tensor):
        fs = final
        if fs.dtype != torch.float32 or fs.shape != (S, n_v, dk, dv) or not fs.is_contiguous():
            raise ValueError("gdn_recurrence: final must be contiguous fp32 (S, n_v, dk, dv)")
        if init is not None and fs.data_ptr() == init.data_ptr() and seq_state is not None:
            raise ValueError("gdn_recurrence: an in-place state update needs seq_state None")
    o = _check_out(out, (M, n_v * dv), qk.device, "gdn_recurrence")
    if chunked and dk == 128 and dv % 64 == 0 and M > 0:
        ws = torch.empty(gdn_chunk_workspace_floats(S, L, n_v), dtype=torch.float32, device=qk.device)
        check(lib().od_gdn_recurrence_chunked(ptr(qk), ptr(v), ptr(g), ptr(beta), ptr(init), ptr(seq_state), n_states,
                                              S, L, n_k, n_v, dk, dv, ptr(o), ptr(fs), ptr(ws), ws.numel(),
                                              stream_of(qk)), "od_gdn_recurrence_chunked")
        return o, fs
    check(lib().od_gdn_recurrence(ptr(qk), ptr(v), ptr(g), ptr(beta), ptr(init), ptr(seq_state), n_states, S, L, n_k,
                                  n_v, dk, dv, ptr(o), ptr(fs), stream_of(qk)), "od_gdn_recurrence")
    return o, fs


def gdn_norm_quant(o: torch.Tensor, z: torch.Tensor, w: torch.Tensor, eps: float, n_v: int, dv: int, inv_s=None,
                   xq=None, sx=None):
    """od_gdn_norm_quant: the gated RMSNorm of o (M, n_v dv) bf16 with gate z (M, n_v dv) bf16 (a column slice of the
    projection is fine) and weight w (dv,) bf16, then the out_proj input quantizer (inv_s (n_v dv,) bf16 or None).
    Returns (xq int8 (M, n_v dv), sx fp32 (M,))."""
    require_gpu(o, z, w, inv_s, xq, sx, name="gdn_norm_quant")
    for t in (o, z, w):
        _lib.bf16_bits(t)
    M, V = o.shape
    if V != n_v * dv or z.shape != (M, V):
        raise ValueError("gdn_norm_quant: o and z must be (M, n_v dv)")
    if o.stride(1) != 1:
        o = o.contiguous()
    if z.stride(1) != 1:
        z = z.contiguous()
    w = w.contiguous()
    xq, sx = _quant_outputs(M, V, None, o.device, xq, sx)
    inv_s = _vec(inv_s, V, "inv_s")
    check(lib().od_gdn_norm_quant(ptr(o), o.stride(0) if M > 1 else V, ptr(z), z.stride(0) if M > 1 else V, ptr(w),
                                  ptr(inv_s), eps, M, n_v, dv, ptr(xq), xq.stride(0), ptr(sx), stream_of(o)),
          "od_gdn_norm_quant")
    return xq, sx
