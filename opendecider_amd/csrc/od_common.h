// Shared device helpers for the gfx950 kernels: bf16 bit conversions, wave reductions, error plumbing.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/od_mi355x.h"

#define OD_WAVE 64

// bf16 bits -> fp32 (exact).
__device__ __forceinline__ float od_bf16_to_f32(uint16_t b) { return __uint_as_float(((uint32_t)b) << 16); }

// fp32 -> bf16 bits, round to nearest even; NaN stays a quiet NaN. gfx950 does this in hardware
// (v_cvt_pk_bf16_f32, two values per instruction); it equals the integer formulation
// u += 0x7fff + ((u >> 16) & 1), NaN -> (u >> 16) | 0x40, on all 2^32 inputs (checked exhaustively on the GPU).
__device__ __forceinline__ uint16_t od_f32_to_bf16(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

typedef float od_f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 od_bf16x2 __attribute__((ext_vector_type(2)));

typedef unsigned short od_u16x2 __attribute__((ext_vector_type(2)));

// Rounds two fp32 values to bf16 (nearest even) and back to fp32 with one v_cvt_pk_bf16_f32; returns the packed
// bf16 pair (a in the low half).
__device__ __forceinline__ uint32_t od_bfr2(float& a, float& b) {
  const uint32_t p = __builtin_bit_cast(uint32_t, __builtin_convertvector((od_f32x2){a, b}, od_bf16x2));
  a = __uint_as_float(p << 16);
  b = __uint_as_float(p & 0xffff0000u);
  return p;
}

// Rounds two fp32 values to bf16 (nearest even) and packs them, a in the low half: one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t od_pack_bf16x2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((od_f32x2){a, b}, od_bf16x2));
}

// Running max of |bf16| over packed pairs, on the bit patterns (monotonic in the magnitude; a NaN dominates, as
// in a float amax that propagates NaN): one v_pk_max_u16 per pair.
__device__ __forceinline__ uint32_t od_absmax_bf16x2(uint32_t acc, uint32_t p) {
  const od_u16x2 r = __builtin_elementwise_max(__builtin_bit_cast(od_u16x2, acc),
                                               __builtin_bit_cast(od_u16x2, p & 0x7fff7fffu));
  return __builtin_bit_cast(uint32_t, r);
}
// The fp32 value of the larger half of a packed absmax.
__device__ __forceinline__ float od_absmax_bf16x2_value(uint32_t acc) {
  const uint32_t lo = acc & 0xffffu, hi = acc >> 16;
  return __uint_as_float((lo > hi ? lo : hi) << 16);
}

// bf16(RN32(silu(g))), silu(g) = g / (1 + exp(-g)): the fp32 value of silu correctly rounded, then rounded to
// bf16 (the SwiGLU of a bf16 module computes silu in fp32 and rounds to bf16). Fast step for |g| < 16:
// exp(-g) = v_exp_f32(RN(-g L)) with L = log2(e) in fp32; the argument (|arg| < 23.1) is off by at most 2^-20 from
// the product's rounding plus 16 |L - log2(e)| < 3.1e-7 from the constant, i.e. 1.3e-6, which costs 7.5 fp32 ulps
// in exp; v_exp_f32 adds one more, and the sum, the reciprocal and the product keep the fast value within 11 ulps of
// silu(g). Its bf16 rounding is then the bf16 rounding of the correctly rounded value unless
// its low 16 bits lie within 16 ulps of the bf16 midpoint 0x8000. Those values (about 1 in 2000), and |g| >= 16, are
// recomputed in float64 and rounded once to fp32. Every SwiGLU kernel uses this one function, so fused and unfused
// paths agree bit for bit, and g has 65536 values, so it is checked against the oracle exhaustively.
// The three steps are also callable one by one (a kernel can check several fast values before one branch).
__device__ __forceinline__ float od_silu_fast32(float g) {
  return g * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(g * -1.44269504088896341f));
}
__device__ __forceinline__ bool od_silu_needs_slow(float g, float s) {
  const uint32_t lo = __float_as_uint(s) & 0xffffu;
  return (lo - 0x7ff0u) <= 0x20u || !(fabsf(g) < 16.0f);
}
__device__ __forceinline__ float od_silu_slow32(float g) {
  const double gd = (double)g;
  return (float)(gd / (1.0 + exp(-gd)));
}
__device__ __forceinline__ float od_silu_bf16(float g) {
  float s = od_silu_fast32(g);
  if (__builtin_expect(od_silu_needs_slow(g, s), 0)) s = od_silu_slow32(g);
  return od_bf16_to_f32(od_f32_to_bf16(s));
}

// bf16(RN32(sigmoid(g))), sigmoid(g) = 1 / (1 + exp(-g)), for the output gate (torch.sigmoid on a bf16 tensor
// computes in fp32 and rounds to bf16): the same exp(-g) as od_silu_bf16, then the sum and a reciprocal, within
// 10 fp32 ulps; values within 16 ulps of a bf16 midpoint, and |g| >= 16, are recomputed in float64.
__device__ __forceinline__ float od_sigmoid_bf16(float g) {
  float s = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(g * -1.44269504088896341f));
  const uint32_t lo = __float_as_uint(s) & 0xffffu;
  if (__builtin_expect((lo - 0x7ff0u) <= 0x20u || !(fabsf(g) < 16.0f), 0)) {
    const double gd = (double)g;
    s = (float)(1.0 / (1.0 + exp(-gd)));
  }
  return od_bf16_to_f32(od_f32_to_bf16(s));
}

// The RMSNorm factor r = RN32(1 / sqrt(ss / K + eps)) from a float64 sum of squares ss: every square of a bf16 value
// is exact in float64 and so is their sum unless the row spans more than ~25 binades, so r does not depend on the
// order of the sum; division and square root are the IEEE float64 operations, rounded once to fp32 at the end.
__device__ __forceinline__ float od_rms_factor(double ss, int64_t K, float eps) {
  return (float)(1.0 / sqrt(ss / (double)K + (double)eps));
}

// Sum of a double over aligned groups of G lanes (G a power of two <= 64), every lane of the group gets it.
template <int G>
__device__ __forceinline__ double od_group_sum_f64(double v) {
#pragma unroll
  for (int o = G / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, OD_WAVE);
  return v;
}

// Max over the 64 lanes of a wave (every lane gets the result).
__device__ __forceinline__ float od_wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, OD_WAVE));
  return v;
}

// Max over aligned groups of G lanes (G a power of two <= 64).
template <int G>
__device__ __forceinline__ float od_group_max(float v) {
#pragma unroll
  for (int o = G / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, OD_WAVE));
  return v;
}

static inline int od_launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? OD_OK : OD_ERR_LAUNCH;
}

static inline bool od_aligned16(const void* p) { return (((uintptr_t)p) & 15u) == 0; }

// One DPP step of a max reduction: x = max(x, x moved by CTRL); lanes of rows outside ROW_MASK compare with
// themselves (update_dpp keeps `old` there).
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float od_dpp_max_step(float x) {
  const int y = __builtin_amdgcn_update_dpp(__float_as_int(x), __float_as_int(x), CTRL, ROW_MASK, 0xf, false);
  return fmaxf(x, __int_as_float(y));
}

// Max over the 64 lanes of a wave with DPP row operations (no LDS round trips), returned wave-uniform.
__device__ __forceinline__ float od_wave_max_dpp(float v) {
  v = od_dpp_max_step<0xB1, 0xf>(v);   // quad_perm [1,0,3,2]
  v = od_dpp_max_step<0x4E, 0xf>(v);   // quad_perm [2,3,0,1]
  v = od_dpp_max_step<0x124, 0xf>(v);  // row_ror:4
  v = od_dpp_max_step<0x128, 0xf>(v);  // row_ror:8   -> every lane holds its row's max
  v = od_dpp_max_step<0x142, 0xa>(v);  // row_bcast:15 into rows 1 and 3
  v = od_dpp_max_step<0x143, 0xc>(v);  // row_bcast:31 into rows 2 and 3 -> lane 63 holds the wave max
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Sum over the 64 lanes of a wave with DPP row operations, returned wave-uniform. The additions run in a fixed
// order (pairs, quads, rows of 16, then the four row sums), so the result is deterministic.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float od_dpp_sum_step(float x) {
  // lanes of rows outside ROW_MASK receive `old` = 0 and keep x
  const int y = __builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, ROW_MASK, 0xf, false);
  return x + __int_as_float(y);
}
__device__ __forceinline__ float od_wave_sum_dpp(float v) {
  v = od_dpp_sum_step<0xB1, 0xf>(v);   // quad_perm [1,0,3,2]
  v = od_dpp_sum_step<0x4E, 0xf>(v);   // quad_perm [2,3,0,1]
  v = od_dpp_sum_step<0x124, 0xf>(v);  // row_ror:4
  v = od_dpp_sum_step<0x128, 0xf>(v);  // row_ror:8   -> every lane holds its row's sum
  v = od_dpp_sum_step<0x142, 0xa>(v);  // row_bcast:15: rows 1 and 3 add rows 0 and 2
  v = od_dpp_sum_step<0x143, 0xc>(v);  // row_bcast:31: rows 2 and 3 add rows 0 + 1 -> lane 63 holds the sum
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Max of unsigned values over the 64 lanes of a wave (DPP), returned wave-uniform.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint32_t od_dpp_umax_step(uint32_t x) {
  const uint32_t y = (uint32_t)__builtin_amdgcn_update_dpp((int)x, (int)x, CTRL, ROW_MASK, 0xf, false);
  return x > y ? x : y;
}
__device__ __forceinline__ uint32_t od_wave_umax_dpp(uint32_t v) {
  v = od_dpp_umax_step<0xB1, 0xf>(v);
  v = od_dpp_umax_step<0x4E, 0xf>(v);
  v = od_dpp_umax_step<0x124, 0xf>(v);
  v = od_dpp_umax_step<0x128, 0xf>(v);
  v = od_dpp_umax_step<0x142, 0xa>(v);
  v = od_dpp_umax_step<0x143, 0xc>(v);
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// Lane l and lane l ^ 32 exchange through v_permlane32_swap: swap(u, u) returns {u[l mod 32], u[32 + l mod 32]}
// in every lane, so the low-half value comes first in both lanes of a pair.
__device__ __forceinline__ void od_xor32_pair(float v, float& lo, float& hi) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  lo = __uint_as_float(r[0]);
  hi = __uint_as_float(r[1]);
}
__device__ __forceinline__ float od_xor32_max(float v) {
  float lo, hi;
  od_xor32_pair(v, lo, hi);
  return fmaxf(lo, hi);
}
__device__ __forceinline__ float od_xor32_sum(float v) {
  float lo, hi;
  od_xor32_pair(v, lo, hi);
  return lo + hi;
}

// ---------------------------------------------------------------------------- per-row int8 quantizer
// q = clamp(rint(v / scale), -127, 127), rint rounding half to even and v / scale the IEEE fp32 quotient, without a
// division per element. With inv = RN(1 / scale), q' = RN(v * inv) is within 1.5 * 2^-23 |q| of the quotient
// RN(v / scale), and |q| <= 127.0001 because scale = max|v| / 127; so rint(q') equals rint(RN(v / scale)) unless q'
// lies within 2^-15 of a half-integer. Such lanes are flagged and redone with the division (a few in 10^5 values).
// Values carry 1.5 * 2^23 + rint(q): adding that constant rounds to an integer in fp32, and the low byte of the bit
// pattern is then the int8 value in two's complement. NaN inputs give 0.
constexpr float kOdRoundMagic = 12582912.0f;  // 1.5 * 2^23

// scale = max(amax, 1e-8) / 127 with torch's NaN rule (amax and clamp_min propagate NaN): a row holding a NaN gets a
// NaN scale, and its bytes then come out 0 (1 / NaN is NaN, and the quantizer's NaN values carry a zero low byte).
// A row holding an infinity gets an infinite scale and zero bytes, as in torch (x / inf = 0, inf / inf = NaN -> 0).
__device__ __forceinline__ float od_q8_scale(float amax) {
  return (amax != amax ? amax : fmaxf(amax, 1e-8f)) / 127.0f;
}

// Returns 1.5 * 2^23 + rint(v * inv); dmax collects |v * inv - rint(v * inv)| (<= 0.5), and a lane needs the
// division when it reaches 0.5 - 2^-15.
constexpr float kOdTieEdge = 0.5f - 0x1p-15f;

__device__ __forceinline__ float od_q8_fast(float v, float inv, float& dmax) {
  const float q = v * inv;
  const float t = q + kOdRoundMagic;
  const float d = q - (t - kOdRoundMagic);  // exact: q minus its nearest integer
  dmax = fmaxf(dmax, fabsf(d));
  return t;
}

__device__ __forceinline__ float od_q8_exact(float v, float scale) {
  float q = rintf(v / scale);
  q = q < -127.0f ? -127.0f : q;  // comparisons keep NaN, which then gives 0 like the fast step
  q = q > 127.0f ? 127.0f : q;
  return q + kOdRoundMagic;
}

// Low bytes of four magic-carrying values -> one word, t0 in the lowest byte.
__device__ __forceinline__ uint32_t od_q8_pack4(float t0, float t1, float t2, float t3) {
  const uint32_t lo = __builtin_amdgcn_perm(__float_as_uint(t1), __float_as_uint(t0), 0x0c0c0400u);
  const uint32_t hi = __builtin_amdgcn_perm(__float_as_uint(t3), __float_as_uint(t2), 0x0c0c0400u);
  return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
}

// N values (N % 4 == 0) -> N / 4 packed words. The exact division runs only when a lane of the wave is flagged.
template <int N>
__device__ __forceinline__ void od_q8_words(const float (&y)[N], float scale, float inv, uint32_t (&w)[N / 4]) {
  float t[N];
  float dmax = 0.0f;
#pragma unroll
  for (int i = 0; i < N; ++i) t[i] = od_q8_fast(y[i], inv, dmax);
  if (__builtin_expect(__any(dmax >= kOdTieEdge), 0)) {
    asm volatile("");  // keeps this rare block a branch: without it the divisions are if-converted and always run
#pragma unroll
    for (int i = 0; i < N; ++i) {
      float di = 0.0f;
      (void)od_q8_fast(y[i], inv, di);
      if (di >= kOdTieEdge) t[i] = od_q8_exact(y[i], scale);
    }
  }
#pragma unroll
  for (int i = 0; i < N / 4; ++i) w[i] = od_q8_pack4(t[4 * i], t[4 * i + 1], t[4 * i + 2], t[4 * i + 3]);
}

// One value, for scalar tails.
__device__ __forceinline__ int8_t od_q8_one(float v, float scale, float inv) {
  float d = 0.0f;
  float t = od_q8_fast(v, inv, d);
  if (d >= kOdTieEdge) t = od_q8_exact(v, scale);
  return (int8_t)(__float_as_uint(t) & 0xffu);
}
