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
