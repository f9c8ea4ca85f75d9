"""MI355X-native (gfx950, HIP) quantized scoring path of OpenDecider: W8A8 int8 linears, the int8 KV-cache
quantize/append and branched option-row attention over an int8 state, behind the reference's Python module API
(Int8Tensor, Int8Linear, gemlite_a8w8_/smooth_a8w8_/fast_int8_kernels_, _split_attention, wide_attention), and the
LM head's token log-prob over a frozen int8 or Q4_0 table (Int8Table, Q4Table, token_logprob).

The kernels live in libod_mi355x.so (C ABI: include/od_mi355x.h), built by `python -m opendecider_amd.build`.
"""
from .quant import (Int8Linear, Int8Tensor, SmoothedLinear, W8A8Linear, fast_int8_kernels_, gemlite_a8w8_,
                    int8_to_w8a8_, kv_mode, materialize, maybe_quantize, quantize_int8_, smooth_a8w8_, smooth_scales,
                    w8a8_)
from .prefix_attn import _split_attention, split_attention, split_attention_int8
from .kv_cache import Int8KVCache
from .wide_attention import wide_attention
from .lm_head import Int8Table, Q4Table, token_logprob

__all__ = ["Int8Linear", "Int8Tensor", "SmoothedLinear", "W8A8Linear", "fast_int8_kernels_", "gemlite_a8w8_",
           "int8_to_w8a8_", "kv_mode", "materialize", "maybe_quantize", "quantize_int8_", "smooth_a8w8_",
           "smooth_scales", "w8a8_", "_split_attention", "split_attention", "split_attention_int8", "Int8KVCache", "wide_attention",
           "Int8Table", "Q4Table", "token_logprob"]
