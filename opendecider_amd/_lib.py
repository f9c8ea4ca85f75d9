"""ctypes binding of libod_mi355x.so (include/od_mi355x.h) and the torch-side plumbing around it.

The library must have been built in-tree (python -m opendecider_amd.build). There is no fallback: every op of this
package fails loudly when the library is missing or a tensor is not on the GPU.
"""
from __future__ import annotations

import ctypes
import os

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libod_mi355x.so")
ABI_VERSION = 2

_c_ptr = ctypes.c_void_p
_i64 = ctypes.c_int64

# name -> argtypes, matching include/od_mi355x.h
SIGNATURES = {
    "od_strerror": [ctypes.c_int],
    "od_abi_version": [],
    "od_act_quant": [_c_ptr, _i64, _c_ptr, _c_ptr, _i64, _c_ptr, _i64, _i64, _c_ptr],
    "od_gate_act_quant": [_c_ptr, _i64, _c_ptr, _i64, _c_ptr, _c_ptr, _i64, _c_ptr, _i64, _i64, _c_ptr],
    "od_act_quant_f32": [_c_ptr, _i64, _c_ptr, _i64, _c_ptr, _i64, _i64, _c_ptr],
    "od_w8a8_gemm": [_c_ptr, _i64, _c_ptr, _c_ptr, _i64, _c_ptr, _c_ptr, _c_ptr, _i64, _c_ptr, _i64, _c_ptr, _i64,
                     _i64, _i64, _i64, _c_ptr],
    "od_kv_quant_append": [_c_ptr, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _c_ptr, _c_ptr, _i64, _i64, _c_ptr],
    "od_branched_attn": [_c_ptr, _i64, _i64, _i64, _c_ptr, _i64, _i64, _i64, _c_ptr, _i64, _i64, _i64,
                         _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _i64, _c_ptr, _i64, _i64, _i64, _c_ptr,
                         _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, ctypes.c_float, ctypes.c_int, _c_ptr],
    "od_branched_attn_split": [_c_ptr, _i64, _i64, _i64, _c_ptr, _i64, _i64, _i64, _c_ptr, _i64, _i64, _i64,
                               _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _i64, _c_ptr, _i64, _i64, _i64,
                               _c_ptr, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, ctypes.c_float, ctypes.c_int, _i64,
                               _c_ptr, _i64, _c_ptr],
    "od_branched_attn_stream": [_c_ptr, _i64, _i64, _i64, _c_ptr, _i64, _i64, _i64, _c_ptr, _i64, _i64, _i64,
                                _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _i64, _c_ptr, _i64, _i64, _i64,
                                _c_ptr, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, ctypes.c_float, ctypes.c_int,
                                _i64, _c_ptr, _i64, _c_ptr],
    "od_branched_attn_split_noalloc": [_c_ptr, _i64, _i64, _i64, _c_ptr, _i64, _i64, _i64, _c_ptr, _i64, _i64, _i64,
                                       _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _i64, _c_ptr, _i64, _i64,
                                       _i64, _c_ptr, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                       ctypes.c_float, ctypes.c_int, _i64, _c_ptr],
    "od_attn_stage_size": [_i64, _i64, _i64, _i64, _c_ptr],
    "od_attn_stage": [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _i64, _i64, _i64, _i64, _i64, ctypes.c_float,
                      ctypes.c_int, _c_ptr, _i64, _c_ptr],
    "od_branched_attn_staged": [_c_ptr, _i64, _i64, _i64, _c_ptr, _i64, _i64, _i64, _c_ptr, _i64, _i64, _i64,
                                _c_ptr, _i64, _c_ptr, _i64, _c_ptr, _i64, _i64, _i64, _c_ptr, _i64, _i64, _i64, _i64,
                                _i64, _i64, _i64, ctypes.c_float, _i64, _c_ptr, _i64, _c_ptr],
    "od_branched_attn_staged2": [_c_ptr, _i64, _i64, _i64, _c_ptr, _i64, _i64, _i64, _c_ptr, _i64, _i64, _i64,
                                 _c_ptr, _i64, _c_ptr, _i64, _i64, _c_ptr, _i64, _i64, _c_ptr, _i64, _c_ptr, _i64,
                                 _i64, _i64, _c_ptr, _i64, _i64, _i64, _i64, _i64, _i64, ctypes.c_float, _i64,
                                 _c_ptr, _i64, _c_ptr],
    "od_wide_attn": [_c_ptr, _i64, _i64, _i64, _c_ptr, _i64, _i64, _i64, _c_ptr, _i64, _i64, _i64, _c_ptr, _i64,
                     _c_ptr, _i64, _i64, _i64, _c_ptr, _i64, _i64, _i64, _i64, _i64, _i64, _i64, ctypes.c_int,
                     ctypes.c_float, _c_ptr],
    "od_rmsnorm_quant": [_c_ptr, _i64, _c_ptr, _c_ptr, ctypes.c_float, _c_ptr, _i64, _c_ptr, _i64, _i64, _c_ptr],
    "od_rmsnorm_quant_ex": [_c_ptr, _i64, _c_ptr, _c_ptr, ctypes.c_float, ctypes.c_int, _c_ptr, _i64, _c_ptr, _i64,
                            _i64, _c_ptr],
    "od_silu_mul_quant": [_c_ptr, _i64, _i64, _c_ptr, _c_ptr, _i64, _c_ptr, _i64, _c_ptr],
    "od_qk_norm_rope": [_c_ptr, _i64, _i64, _i64, _i64, _i64, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _i64, _c_ptr,
                        ctypes.c_float, _c_ptr],
    "od_qk_norm_rope_ex": [_c_ptr, _i64, _i64, _i64, _i64, _i64, _i64, ctypes.c_int, _c_ptr, _c_ptr, _c_ptr, _c_ptr,
                           _i64, _c_ptr, ctypes.c_float, _c_ptr],
    "od_w8a8_gemm_swiglu": [_c_ptr, _i64, _c_ptr, _c_ptr, _i64, _c_ptr, _c_ptr, _i64, _i64, _i64, _i64, _c_ptr],
    "od_w8a8_gemm_ws_size": [_i64, _i64, _i64, _c_ptr],
    "od_w8a8_gemm_ws": [_c_ptr, _i64, _c_ptr, _c_ptr, _i64, _c_ptr, _c_ptr, _c_ptr, _i64, _c_ptr, _i64, _i64, _i64,
                        _i64, ctypes.c_int, _c_ptr, _i64, _c_ptr],
    "od_kv_copy_rows": [_c_ptr, _c_ptr, _i64, _i64, _i64, _c_ptr, _c_ptr, _i64, _i64, _i64, _i64, _i64, _i64, _c_ptr,
                        _i64, _c_ptr],
    "od_qk_norm_rope_kv_append": [_c_ptr, _i64, _i64, _i64, _i64, _i64, _i64, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _i64,
                                  _c_ptr, ctypes.c_float, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _i64, _i64, _c_ptr],
    "od_qk_norm_rope_kv_append_ex": [_c_ptr, _i64, _i64, _i64, _i64, _i64, _i64, _i64, ctypes.c_int, _c_ptr, _c_ptr,
                                     _c_ptr, _c_ptr, _i64, _c_ptr, ctypes.c_float, _c_ptr, _c_ptr, _c_ptr, _c_ptr,
                                     _i64, _i64, _c_ptr],
    "od_attn_stage_bf16": [_c_ptr, _i64, _i64, _i64, _c_ptr, _i64, _i64, _i64, _c_ptr, _i64, _i64, _i64, _i64,
                           ctypes.c_float, _c_ptr, _i64, _c_ptr],
    "od_gdn_prep": [_c_ptr, _i64, _c_ptr, _c_ptr, _c_ptr, _i64, _c_ptr, _c_ptr, _i64, _i64, _i64, _i64, _i64, _i64,
                    _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr],
    "od_gdn_prep_ex": [_c_ptr, _i64, _c_ptr, _c_ptr, _c_ptr, _i64, _c_ptr, _c_ptr, _c_ptr, _i64, _i64, _i64, _i64, _i64,
                       _i64, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr],
    "od_gdn_recurrence": [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                          _c_ptr, _c_ptr, _c_ptr],
    "od_gdn_norm_quant": [_c_ptr, _i64, _c_ptr, _i64, _c_ptr, _c_ptr, ctypes.c_float, _i64, _i64, _i64, _c_ptr, _i64,
                          _c_ptr, _c_ptr],
    "od_gdn_chunk_ws_size": [_i64, _i64, _i64, _c_ptr],
    "od_gdn_recurrence_chunked": [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _i64, _i64, _i64, _i64, _i64, _i64,
                                  _i64, _c_ptr, _c_ptr, _c_ptr, _i64, _c_ptr],
    "od_lm_head_logprob_ws": [_i64, _i64, _c_ptr],
    "od_lm_head_logprob": [_c_ptr, _i64, _c_ptr, _i64, ctypes.c_int, _c_ptr, _i64, _c_ptr, _c_ptr, _i64, _i64, _i64,
                           _c_ptr, _c_ptr, _i64, _c_ptr],
    "od_lm_head_logprob_q4": [_c_ptr, _i64, _c_ptr, _i64, ctypes.c_int, _c_ptr, _i64, _c_ptr, _i64, _c_ptr, _i64,
                              _i64, _i64, _c_ptr, _c_ptr, _i64, _c_ptr],
}

_LIB = None


def lib() -> ctypes.CDLL:
    """The loaded library (loaded once). Raises RuntimeError if it has not been built."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m opendecider_amd.build` "
                               "(there is no CPU fallback for these kernels)")
        L = ctypes.CDLL(LIB_PATH)
        for name, argtypes in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = argtypes
            fn.restype = ctypes.c_char_p if name == "od_strerror" else ctypes.c_int
        if L.od_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH}: ABI version {L.od_abi_version()} != {ABI_VERSION}; rebuild it")
        _LIB = L
    return _LIB


# the static scratch of od_branched_attn_split_noalloc (include/od_mi355x.h), in floats
SPLIT_SCRATCH_FLOATS = 16 * 1024 * 1024

# od_branched_attn / od_attn_stage dequantization of the int8 state (include/od_mi355x.h)
DEQUANT = {"bf16": 0, "fp32": 1}


def dequant_code(mode: str) -> int:
    if mode not in DEQUANT:
        raise ValueError(f"dequant must be one of {sorted(DEQUANT)}, got {mode!r}")
    return DEQUANT[mode]


def check(rc: int, name: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{name} failed: {lib().od_strerror(rc).decode()} (code {rc})")


def ptr(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_of(t: torch.Tensor):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def require_gpu(*tensors, name: str) -> None:
    """The ops run only on the GPU through the HIP library; anything else is an error, never a fallback."""
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError(f"{name}: tensors must be on the MI355X (got device {t.device}); "
                               "opendecider_amd has no CPU path")


def bf16_bits(t: torch.Tensor) -> torch.Tensor:
    if t.dtype != torch.bfloat16:
        raise TypeError(f"expected bfloat16, got {t.dtype}")
    return t
