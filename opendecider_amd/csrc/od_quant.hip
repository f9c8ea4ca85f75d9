// Per-row dynamic int8 quantization (activations, weights, KV-cache rows) for gfx950.
//
// One formula everywhere (src/opendecider/quant.py:38-40):
//   scale = max(max_k |v_k|, 1e-8) / 127          (IEEE fp32 division)
//   q_k   = clamp(rint(v_k / scale), -127, 127)     (IEEE fp32 division, round half to even)
// where v_k = float(x_k), or float(bf16(float(x_k) * float(inv_s_k))) with a SmoothQuant input scale
// (quant.py:329: the product is rounded to bf16 before it is quantized).
//
// HBM-bound: every element is read from HBM once (the second pass over a row hits L1/L2: a row is at most a few
// tens of KB and is owned by one workgroup) and written once as int8. A group of LANES threads owns a row; rows
// of 64..512 elements (KV heads, small linears) use 8..64 lanes so that a wave covers several rows, wider rows
// use a whole 256-thread workgroup. Loads are 16 B (8 bf16) per lane when the row layout allows it.
#include "od_common.h"

namespace {

constexpr int kThreads = 256;

enum Mode { kAct = 0, kKv = 1 };

struct RowMap {
  // kAct: row r of x (stride ldx) -> row r of q (stride ldq), scale s[r].
  // kKv : row r = ((b * H + h) * n_new + i) of x (strides sxb, sxh, sxt) -> cache row (b * H + h) * cap + n0 + i.
  const uint16_t* x;
  int8_t* q;
  float* s;
  int64_t ldx, ldq;
  int64_t H, n_new, sxb, sxh, sxt, cap, n0;
};

template <int MODE>
__device__ __forceinline__ void map_row(const RowMap& m, int64_t r, const uint16_t*& xin, int8_t*& qout,
                                        float*& sout) {
  if (MODE == kAct) {
    xin = m.x + r * m.ldx;
    qout = m.q + r * m.ldq;
    sout = m.s + r;
  } else {
    const int64_t i = r % m.n_new;
    const int64_t bh = r / m.n_new;
    const int64_t b = bh / m.H, h = bh % m.H;
    xin = m.x + b * m.sxb + h * m.sxh + i * m.sxt;
    const int64_t orow = bh * m.cap + m.n0 + i;
    qout = m.q + orow * m.ldq;
    sout = m.s + orow;
  }
}

template <bool HAS_INV>
__device__ __forceinline__ float load_val(const uint16_t* xin, const uint16_t* inv_s, int64_t k) {
  float v = od_bf16_to_f32(xin[k]);
  if (HAS_INV) v = od_bf16_to_f32(od_f32_to_bf16(v * od_bf16_to_f32(inv_s[k])));
  return v;
}

template <bool HAS_INV>
__device__ __forceinline__ void load8(const uint16_t* xin, const uint16_t* inv_s, int64_t k, float (&v)[8]) {
  const uint4 raw = *reinterpret_cast<const uint4*>(xin + k);
  const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    v[2 * j] = __uint_as_float(w[j] << 16);
    v[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
  }
  if (HAS_INV) {
    const uint4 rs = *reinterpret_cast<const uint4*>(inv_s + k);
    const uint32_t ws[4] = {rs.x, rs.y, rs.z, rs.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[2 * j] = od_bf16_to_f32(od_f32_to_bf16(v[2 * j] * __uint_as_float(ws[j] << 16)));
      v[2 * j + 1] = od_bf16_to_f32(od_f32_to_bf16(v[2 * j + 1] * __uint_as_float(ws[j] & 0xffff0000u)));
    }
  }
}

__device__ __forceinline__ int8_t quant1(float v, float scale) {
  float qf = rintf(v / scale);
  qf = fminf(fmaxf(qf, -127.0f), 127.0f);
  return (int8_t)(int)qf;
}

// LANES threads per row; VEC = 8 (16-byte loads) or 1.
template <int LANES, int VEC, int MODE, bool HAS_INV>
__global__ __launch_bounds__(kThreads) void quant_rows_kernel(RowMap m, const uint16_t* __restrict__ inv_s,
                                                              int64_t n_rows, int64_t K) {
  constexpr int kRowsPerBlock = kThreads / LANES;
  const int lane = threadIdx.x % LANES;
  const int64_t r = (int64_t)blockIdx.x * kRowsPerBlock + threadIdx.x / LANES;
  const bool live = r < n_rows;  // no early return: the 256-lane variant has a barrier below
  const uint16_t* xin = nullptr;
  int8_t* qout = nullptr;
  float* sout = nullptr;
  if (live) map_row<MODE>(m, r, xin, qout, sout);

  float amax = 0.0f;
  if (live) {
    if constexpr (VEC == 8) {
      for (int64_t k = (int64_t)lane * 8; k < K; k += LANES * 8) {
        float v[8];
        load8<HAS_INV>(xin, inv_s, k, v);
#pragma unroll
        for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(v[j]));
      }
    } else {
      for (int64_t k = lane; k < K; k += LANES) amax = fmaxf(amax, fabsf(load_val<HAS_INV>(xin, inv_s, k)));
    }
  }
  if constexpr (LANES <= OD_WAVE) {
    amax = od_group_max<LANES <= OD_WAVE ? LANES : OD_WAVE>(amax);
  } else {
    __shared__ float red[kThreads / OD_WAVE];
    amax = od_wave_max(amax);
    if (threadIdx.x % OD_WAVE == 0) red[threadIdx.x / OD_WAVE] = amax;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kThreads / OD_WAVE; ++i) amax = fmaxf(amax, red[i]);
  }
  if (!live) return;
  const float scale = fmaxf(amax, 1e-8f) / 127.0f;

  if constexpr (VEC == 8) {
    for (int64_t k = (int64_t)lane * 8; k < K; k += LANES * 8) {
      float v[8];
      load8<HAS_INV>(xin, inv_s, k, v);
      uint32_t lo = 0, hi = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) lo |= ((uint32_t)(uint8_t)quant1(v[j], scale)) << (8 * j);
#pragma unroll
      for (int j = 0; j < 4; ++j) hi |= ((uint32_t)(uint8_t)quant1(v[4 + j], scale)) << (8 * j);
      *reinterpret_cast<uint2*>(qout + k) = make_uint2(lo, hi);
    }
  } else {
    for (int64_t k = lane; k < K; k += LANES) qout[k] = quant1(load_val<HAS_INV>(xin, inv_s, k), scale);
  }
  if (lane == 0) *sout = scale;
}

template <int MODE, bool HAS_INV, int VEC>
int launch_lanes(const RowMap& m, const uint16_t* inv_s, int64_t n_rows, int64_t K, hipStream_t st) {
  const int64_t per_lane = (K + VEC - 1) / VEC;
  int lanes = per_lane <= 8 ? 8 : per_lane <= 16 ? 16 : per_lane <= 32 ? 32 : per_lane <= 64 ? 64 : 256;
  const int64_t rows_per_block = kThreads / lanes;
  const int64_t blocks = (n_rows + rows_per_block - 1) / rows_per_block;
  if (blocks > 0x7fffffff) return OD_ERR_SHAPE;
  dim3 grid((unsigned)blocks), block(kThreads);
  switch (lanes) {
    case 8: quant_rows_kernel<8, VEC, MODE, HAS_INV><<<grid, block, 0, st>>>(m, inv_s, n_rows, K); break;
    case 16: quant_rows_kernel<16, VEC, MODE, HAS_INV><<<grid, block, 0, st>>>(m, inv_s, n_rows, K); break;
    case 32: quant_rows_kernel<32, VEC, MODE, HAS_INV><<<grid, block, 0, st>>>(m, inv_s, n_rows, K); break;
    case 64: quant_rows_kernel<64, VEC, MODE, HAS_INV><<<grid, block, 0, st>>>(m, inv_s, n_rows, K); break;
    default: quant_rows_kernel<256, VEC, MODE, HAS_INV><<<grid, block, 0, st>>>(m, inv_s, n_rows, K); break;
  }
  return od_launch_status();
}

template <int MODE>
int launch_quant(const RowMap& m, const uint16_t* inv_s, int64_t n_rows, int64_t K, bool vec_ok, hipStream_t st) {
  if (n_rows == 0) return OD_OK;
  if (inv_s) {
    return vec_ok ? launch_lanes<MODE, true, 8>(m, inv_s, n_rows, K, st)
                  : launch_lanes<MODE, true, 1>(m, inv_s, n_rows, K, st);
  }
  return vec_ok ? launch_lanes<MODE, false, 8>(m, inv_s, n_rows, K, st)
                : launch_lanes<MODE, false, 1>(m, inv_s, n_rows, K, st);
}

}  // namespace

extern "C" int od_act_quant(const uint16_t* x, int64_t ldx, const uint16_t* inv_s, int8_t* xq, int64_t ldq,
                            float* sx, int64_t M, int64_t K, od_stream_t stream) {
  if (M < 0 || K < 1 || ldx < K || ldq < K) return OD_ERR_SHAPE;
  if (M == 0) return OD_OK;
  if (!x || !xq || !sx) return OD_ERR_NULL;
  RowMap m{};
  m.x = x;
  m.q = xq;
  m.s = sx;
  m.ldx = ldx;
  m.ldq = ldq;
  const bool vec_ok = (K % 8 == 0) && (ldx % 8 == 0) && (ldq % 8 == 0) && od_aligned16(x) &&
                      ((((uintptr_t)xq) & 7u) == 0) && (!inv_s || od_aligned16(inv_s));
  return launch_quant<kAct>(m, inv_s, M, K, vec_ok, (hipStream_t)stream);
}

extern "C" int od_kv_quant_append(const uint16_t* x, int64_t B, int64_t H, int64_t n_new, int64_t D, int64_t sxb,
                                  int64_t sxh, int64_t sxt, int8_t* q, float* s, int64_t cap, int64_t n0,
                                  od_stream_t stream) {
  if (B < 0 || H < 0 || n_new < 0 || D < 1 || n0 < 0 || cap < 0 || n0 + n_new > cap) return OD_ERR_SHAPE;
  if (sxb < 0 || sxh < 0 || sxt < 0) return OD_ERR_SHAPE;
  const int64_t n_rows = B * H * n_new;
  if (n_rows == 0) return OD_OK;
  if (!x || !q || !s) return OD_ERR_NULL;
  RowMap m{};
  m.x = x;
  m.q = q;
  m.s = s;
  m.ldq = D;
  m.H = H;
  m.n_new = n_new;
  m.sxb = sxb;
  m.sxh = sxh;
  m.sxt = sxt;
  m.cap = cap;
  m.n0 = n0;
  const bool vec_ok = (D % 8 == 0) && (sxb % 8 == 0) && (sxh % 8 == 0) && (sxt % 8 == 0) && od_aligned16(x) &&
                      ((((uintptr_t)q) & 7u) == 0);
  return launch_quant<kKv>(m, nullptr, n_rows, D, vec_ok, (hipStream_t)stream);
}

extern "C" const char* od_strerror(int code) {
  switch (code) {
    case OD_OK: return "ok";
    case OD_ERR_NULL: return "a required pointer is NULL";
    case OD_ERR_SHAPE: return "a size or stride is out of range or inconsistent";
    case OD_ERR_ALIGN: return "a pointer or leading dimension breaks the 16-byte alignment the kernel needs";
    case OD_ERR_UNSUPPORTED: return "head dim / GQA ratio / row length outside what the kernels are built for";
    case OD_ERR_LAUNCH: return "kernel launch failed";
    default: return "unknown error";
  }
}

extern "C" int od_abi_version(void) { return 1; }
