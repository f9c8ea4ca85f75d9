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
