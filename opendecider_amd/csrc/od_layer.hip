// Row kernels of the dense decoder layer around the W8A8 GEMMs and the branched attention (gfx950):
//   od_rmsnorm_quant   RMSNorm -> (SmoothQuant input scale) -> per-token int8, one pass over HBM
//   od_qk_norm_rope    per-head RMSNorm of q and k + rotary embedding, in place on the QKV GEMM output
//   od_silu_mul_quant  SwiGLU (silu(gate) * up) -> (SmoothQuant input scale) -> per-token int8
// All are HBM-bound (a few bytes per element); each fuses what would otherwise be separate bf16 round trips.
// Rounding follows the bf16 module arithmetic of the decoder they serve (every elementwise product of two bf16
// tensors is rounded to bf16 once), so the CPU oracle reproduces them up to the fp32 reduction order and the
// rsqrt / exp of the device.
#include "od_common.h"

namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ float bfr(float v) { return od_bf16_to_f32(od_f32_to_bf16(v)); }

__device__ __forceinline__ float block_sum(float v, float* red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, OD_WAVE);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < kThreads / OD_WAVE; ++i) s += red[i];
  return s;
}

__device__ __forceinline__ float block_max(float v, float* red) {
  v = od_wave_max(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < kThreads / OD_WAVE; ++i) s = fmaxf(s, red[i]);
  return s;
}

__device__ __forceinline__ int8_t q8(float v, float scale) {
  float qf = rintf(v / scale);
  qf = fminf(fmaxf(qf, -127.0f), 127.0f);
  return (int8_t)(int)qf;
}

// ---------------------------------------------------------------------------- RMSNorm + quantize
// y_k = bf16(w_k * bf16(x_k * r)), r = 1 / sqrt(mean(x^2) + eps); then optionally y_k = bf16(y_k * inv_s_k);
// then the per-row int8 quantizer. One workgroup per row; the row is read three times (L1/L2 after the first).
__device__ __forceinline__ float rms_val(const uint16_t* xr, const uint16_t* w, const uint16_t* inv_s, int k, float r) {
  float y = bfr(od_bf16_to_f32(w[k]) * bfr(od_bf16_to_f32(xr[k]) * r));
  if (inv_s) y = bfr(y * od_bf16_to_f32(inv_s[k]));
  return y;
}

__global__ __launch_bounds__(kThreads) void rmsnorm_quant_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                                 const uint16_t* __restrict__ w,
                                                                 const uint16_t* __restrict__ inv_s, float eps,
                                                                 int8_t* __restrict__ xq, int64_t ldq,
                                                                 float* __restrict__ sx, int K) {
  __shared__ float red[kThreads / OD_WAVE];
  const int64_t row = blockIdx.x;
  const uint16_t* xr = x + row * ldx;
  float ss = 0.0f;
  for (int k = threadIdx.x; k < K; k += kThreads) {
    const float v = od_bf16_to_f32(xr[k]);
    ss = fmaf(v, v, ss);
  }
  ss = block_sum(ss, red);
  const float r = 1.0f / sqrtf(ss / (float)K + eps);
  float amax = 0.0f;
  for (int k = threadIdx.x; k < K; k += kThreads) amax = fmaxf(amax, fabsf(rms_val(xr, w, inv_s, k, r)));
  amax = block_max(amax, red);
  const float scale = fmaxf(amax, 1e-8f) / 127.0f;
  int8_t* qr = xq + row * ldq;
  for (int k = threadIdx.x; k < K; k += kThreads) qr[k] = q8(rms_val(xr, w, inv_s, k, r), scale);
  if (threadIdx.x == 0) sx[row] = scale;
}

// ---------------------------------------------------------------------------- SwiGLU + quantize
// y_k = bf16(bf16(silu(g_k)) * u_k), silu(g) = g / (1 + exp(-g)) in fp32, g = gu[row, k], u = gu[row, F + k].
__device__ __forceinline__ float swiglu_val(const uint16_t* gr, int64_t F, const uint16_t* inv_s, int64_t k) {
  const float g = od_bf16_to_f32(gr[k]);
  const float u = od_bf16_to_f32(gr[F + k]);
  float y = bfr(bfr(g / (1.0f + expf(-g))) * u);
  if (inv_s) y = bfr(y * od_bf16_to_f32(inv_s[k]));
  return y;
}

__global__ __launch_bounds__(kThreads) void silu_mul_quant_kernel(const uint16_t* __restrict__ gu, int64_t ldg,
                                                                  int64_t F, const uint16_t* __restrict__ inv_s,
                                                                  int8_t* __restrict__ aq, int64_t ldq,
                                                                  float* __restrict__ sa) {
  __shared__ float red[kThreads / OD_WAVE];
  const int64_t row = blockIdx.x;
  const uint16_t* gr = gu + row * ldg;
  float amax = 0.0f;
  for (int64_t k = threadIdx.x; k < F; k += kThreads) amax = fmaxf(amax, fabsf(swiglu_val(gr, F, inv_s, k)));
  amax = block_max(amax, red);
  const float scale = fmaxf(amax, 1e-8f) / 127.0f;
  int8_t* qr = aq + row * ldq;
  for (int64_t k = threadIdx.x; k < F; k += kThreads) qr[k] = q8(swiglu_val(gr, F, inv_s, k), scale);
  if (threadIdx.x == 0) sa[row] = scale;
}

// ---------------------------------------------------------------------------- q/k RMSNorm + RoPE
// For every token row and every q head then k head (D values at qkv[row, head * D ...]):
//   n_d = bf16(w_d * bf16(x_d * r)),  r = 1 / sqrt(mean(x^2) + eps)
//   out_d = bf16(bf16(n_d * cos_d) + bf16(rot_d * sin_d)),  rot = (-n[D/2:], n[:D/2]) (rotate_half)
// cos/sin: bf16 tables [n_pos, D/2] (the two halves of a head share them), row index = pos[token].
// A group of D/2 lanes owns one head; lane i holds the pair (i, i + D/2).
template <int D>
__global__ __launch_bounds__(kThreads) void qk_norm_rope_kernel(uint16_t* __restrict__ qkv, int64_t ld, int64_t M,
                                                                int n_heads_q, int n_heads_k,
                                                                const uint16_t* __restrict__ qw,
                                                                const uint16_t* __restrict__ kw,
                                                                const uint16_t* __restrict__ cos_t,
                                                                const uint16_t* __restrict__ sin_t, int64_t n_pos,
                                                                const int32_t* __restrict__ pos, float eps) {
  constexpr int L = D / 2;
  constexpr int kHeadsPerBlock = kThreads / L;
  const int heads = n_heads_q + n_heads_k;
  const int64_t gh = (int64_t)blockIdx.x * kHeadsPerBlock + threadIdx.x / L;
  if (gh >= M * heads) return;  // whole lane groups exit together; the reductions below stay within a group
  const int64_t row = gh / heads;
  const int head = (int)(gh % heads);
  const int i = threadIdx.x % L;
  uint16_t* hp = qkv + row * ld + (int64_t)head * D;
  const uint16_t* w = head < n_heads_q ? qw : kw;
  const float a = od_bf16_to_f32(hp[i]), b = od_bf16_to_f32(hp[i + L]);
  float ss = fmaf(a, a, b * b);
#pragma unroll
  for (int o = L / 2; o > 0; o >>= 1) ss += __shfl_xor(ss, o, OD_WAVE);
  const float r = 1.0f / sqrtf(ss / (float)D + eps);
  const float na = bfr(od_bf16_to_f32(w[i]) * bfr(a * r));
  const float nb = bfr(od_bf16_to_f32(w[i + L]) * bfr(b * r));
  const int64_t p = pos[row];
  const bool in_table = p >= 0 && p < n_pos;  // a position past the tables yields NaN, never an out-of-bounds read
  const float c = in_table ? od_bf16_to_f32(cos_t[p * L + i]) : __builtin_nanf("");
  const float s = in_table ? od_bf16_to_f32(sin_t[p * L + i]) : __builtin_nanf("");
  hp[i] = od_f32_to_bf16(bfr(na * c) + bfr(-nb * s));
  hp[i + L] = od_f32_to_bf16(bfr(nb * c) + bfr(na * s));
}

}  // namespace

extern "C" int od_rmsnorm_quant(const uint16_t* x, int64_t ldx, const uint16_t* w, const uint16_t* inv_s, float eps,
                                int8_t* xq, int64_t ldq, float* sx, int64_t M, int64_t K, od_stream_t stream) {
  if (M < 0 || K < 1 || K > (1 << 30) || ldx < K || ldq < K) return OD_ERR_SHAPE;
  if (M == 0) return OD_OK;
  if (!x || !w || !xq || !sx) return OD_ERR_NULL;
  if (M > 0x7fffffff) return OD_ERR_SHAPE;
  rmsnorm_quant_kernel<<<dim3((unsigned)M), dim3(kThreads), 0, (hipStream_t)stream>>>(x, ldx, w, inv_s, eps, xq, ldq,
                                                                                      sx, (int)K);
  return od_launch_status();
}

extern "C" int od_silu_mul_quant(const uint16_t* gu, int64_t ldg, int64_t F, const uint16_t* inv_s, int8_t* aq,
                                 int64_t ldq, float* sa, int64_t M, od_stream_t stream) {
  if (M < 0 || F < 1 || ldg < 2 * F || ldq < F) return OD_ERR_SHAPE;
  if (M == 0) return OD_OK;
  if (!gu || !aq || !sa) return OD_ERR_NULL;
  if (M > 0x7fffffff) return OD_ERR_SHAPE;
  silu_mul_quant_kernel<<<dim3((unsigned)M), dim3(kThreads), 0, (hipStream_t)stream>>>(gu, ldg, F, inv_s, aq, ldq,
                                                                                       sa);
  return od_launch_status();
}

extern "C" int od_qk_norm_rope(uint16_t* qkv, int64_t ld, int64_t M, int64_t n_heads_q, int64_t n_heads_k,
                               int64_t D, const uint16_t* q_w, const uint16_t* k_w, const uint16_t* cos_t,
                               const uint16_t* sin_t, int64_t n_pos, const int32_t* pos, float eps,
                               od_stream_t stream) {
  if (M < 0 || n_heads_q < 0 || n_heads_k < 0 || ld < (n_heads_q + n_heads_k) * D) return OD_ERR_SHAPE;
  if (D != 64 && D != 128) return OD_ERR_UNSUPPORTED;
  const int64_t heads = n_heads_q + n_heads_k;
  if (M == 0 || heads == 0) return OD_OK;
  if (!qkv || !q_w || !k_w || !cos_t || !sin_t || !pos) return OD_ERR_NULL;
  const int64_t per_block = kThreads / (D / 2);
  const int64_t blocks = (M * heads + per_block - 1) / per_block;
  if (blocks > 0x7fffffff || heads > 0x7fffffff) return OD_ERR_SHAPE;
  hipStream_t st = (hipStream_t)stream;
  if (D == 128) {
    qk_norm_rope_kernel<128><<<dim3((unsigned)blocks), dim3(kThreads), 0, st>>>(
        qkv, ld, M, (int)n_heads_q, (int)n_heads_k, q_w, k_w, cos_t, sin_t, n_pos, pos, eps);
  } else {
    qk_norm_rope_kernel<64><<<dim3((unsigned)blocks), dim3(kThreads), 0, st>>>(
        qkv, ld, M, (int)n_heads_q, (int)n_heads_k, q_w, k_w, cos_t, sin_t, n_pos, pos, eps);
  }
  return od_launch_status();
}
