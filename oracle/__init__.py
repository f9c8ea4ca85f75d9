"""CPU oracle for OpenDecider's quantized scoring path. TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU and in plain torch/numpy arithmetic, the reference algorithms that the HIP
kernels of `opendecider_amd` replace. It is the checker, never the thing measured or shipped: only `tests/`,
`__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` may import it. Product code must not import it
and has no CPU fallback that routes here.

Modules
  quant      Int8Tensor.quantize / dequantize, Int8Linear weight quantization, W8A8 linear (per-token int8
             activations x per-channel int8 weights, int32 accumulate, bf16 epilogue), SmoothQuant fold.
             Reference: src/opendecider/quant.py.
  attention  wide_attention semantics (causal offset S-T, key-valid mask, empty rows -> 0 / -inf LSE) and the
             Hydragen split attention with its log-sum-exp merge, over an int8 KV state.
             Reference: src/opendecider/wide_attention.py, src/opendecider/prefix_attn.py.
  decoder    A dense 9B-class decoder layer stack used as the decision-forward harness around the path, and the
             option pooling + 'none' logit + log-softmax readout.
  gdn        The Gated DeltaNet (linear-attention) layer of the Qwen3.5 hybrid backbone: conv + SiLU, l2norm,
             gates, the gated delta rule, the gated RMSNorm. Reference: transformers' Qwen3.5 modules, which the
             reference runs (src/opendecider/backbone.py:256-289, skipkv.py:208-231).

Pinning (how each function is checked, in tests/test_oracle_*.py)
  quant.quantize_rows      brute-force per-element IEEE float32 arithmetic with numpy and round-half-even, hand
                           known answers (ties, zero rows, absmax -> +-127), error bound |q*s - x| <= s/2,
                           slice invariance (quantizing new rows only == quantizing the whole tensor).
  quant.int_gemm           exact int64 matmul and pure-Python loops on tiny shapes; ones-vector closed forms.
  quant.w8a8_epilogue      float64 product within one bf16 rounding; fixed fp32 operation order.
  quant.smooth_*           the reference test test_int8_gemm.py:70-88 restated (float64 exactness, formula).
  attention.*              float64 brute-force softmax loops on tiny shapes; merge == one softmax over the
                           concatenated keys; permutation equivariance; empty key set; torch.logsumexp.
  gdn.*                    transformers' own functions (causal_conv1d_fn / _update, l2norm, the recurrent and
                           chunked gated delta rule, Qwen3_5RMSNormGated), a pure-decay closed form, continuation ==
                           whole sequence, decimal rsqrt.
  decoder.*                the layer is the build's own harness (not a reference function): each sub-step is
                           pinned separately (RMSNorm closed form, RoPE rotation norm preservation and the
                           position-difference invariance of q.k, SwiGLU) and the whole forward is checked for
                           option-order invariance.
"""
