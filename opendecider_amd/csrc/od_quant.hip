// Per-row dynamic int8 quantization (activations, weights, KV-cache rows) for gfx950.
//
// One formula everywhere (src/opendecider/quant.py:38-40):
//   scale = max(max_k |v_k|, 1e-8) / 127          (IEEE fp32 division)
//   q_k   = clamp(rint(v_k / scale), -127, 127)     (IEEE fp32 division, round half to even)
// where v_k = float(x_k), or float(bf16(float(x_k) * float(inv_s_k))) with a SmoothQuant input scale
// (quant.py:329: the product is rounded to bf16 before it is quantized). The gated mode (od_gate_act_quant) first
// forms x_k = bf16(x_k * bf16(sigmoid(g_k))), the attention output times the output gate (prefix_attn.py:130).
//
// The division by scale is a multiplication by 1 / scale with an exact fallback (od_q8_words), which gives the
// quotient's result bit for bit. The row max runs on bf16 bit patterns, so a NaN in a row makes its scale NaN and
// its bytes 0, as torch's amax (which propagates NaN) and float -> int8 conversion on x86 do.
//
// Every element is read from HBM once and written once as int8: rows up to 6 * 256 * 8 elements stay in registers
// between the max and the quantization; longer rows are read twice (the second pass hits L1/L2). A group of LANES
// threads owns a row; rows of 64..512 elements (KV heads, small linears) use 8..64 lanes so that a wave covers
// several rows, wider rows use a whole 256-thread workgroup. Loads are 16 B (8 bf16) per lane when the row layout
// allows it.
#include "od_common.h"

namespace {

constexpr int kThreads = 256;

enum Mode { kAct = 0, kKv = 1, kGate = 2 };

struct RowMap {
  // kAct: row r of x (stride ldx) -> row r of q (stride ldq), scale s[r].
  // kKv : row r = ((b * H + h) * n_new + i) of x (strides sxb, sxh, sxt) -> cache row (b * H + h) * cap + n0 + i.
  // kGate: as kAct, with the gate row r of `gate` (stride ldg) beside x.
  const uint16_t* x;
  int8_t* q;
  float* s;
  int64_t ldx, ldq;
  int64_t H, n_new, sxb, sxh, sxt, cap, n0;
  const uint16_t* gate;
  int64_t ldg;
};

template <int MODE>
__device__ __forceinline__ void map_row(const RowMap& m, int64_t r, const uint16_t*& xin, int8_t*& qout,
                                        float*& sout, const uint16_t*& gin) {
  gin = MODE == kGate ? m.gate + r * m.ldg : nullptr;
  if (MODE != kKv) {
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

template <bool HAS_INV, bool GATE>
__device__ __forceinline__ float load_val(const uint16_t* xin, const uint16_t* gin, const uint16_t* inv_s, int64_t k) {
  float v = od_bf16_to_f32(xin[k]);
  if (GATE) v = od_bf16_to_f32(od_f32_to_bf16(v * od_sigmoid_bf16(od_bf16_to_f32(gin[k]))));
  if (HAS_INV) v = od_bf16_to_f32(od_f32_to_bf16(v * od_bf16_to_f32(inv_s[k])));
  return v;
}

// 8 consecutive values of a row from one 16-byte load, times the smoothing scale and rounded to bf16 when there is
// one; returns the packed |bf16| max of the 8 (see od_absmax_bf16x2).
template <bool HAS_INV, bool GATE>
__device__ __forceinline__ uint32_t load8(const uint16_t* xin, const uint16_t* gin, const uint16_t* inv_s, int64_t k,
                                          float (&v)[8]) {
  const uint4 raw = *reinterpret_cast<const uint4*>(xin + k);
  const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
  uint4 rs{}, rg{};
  if (HAS_INV) rs = *reinterpret_cast<const uint4*>(inv_s + k);
  if (GATE) rg = *reinterpret_cast<const uint4*>(gin + k);
  const uint32_t ws[4] = {rs.x, rs.y, rs.z, rs.w};
  const uint32_t wg[4] = {rg.x, rg.y, rg.z, rg.w};
  uint32_t am = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float a = __uint_as_float(w[j] << 16), b = __uint_as_float(w[j] & 0xffff0000u);
    uint32_t p = w[j];
    if (GATE) {
      a *= od_sigmoid_bf16(__uint_as_float(wg[j] << 16));
      b *= od_sigmoid_bf16(__uint_as_float(wg[j] & 0xffff0000u));
      p = od_bfr2(a, b);
    }
    if (HAS_INV) {
      a *= __uint_as_float(ws[j] << 16);
      b *= __uint_as_float(ws[j] & 0xffff0000u);
      p = od_bfr2(a, b);
    }
    v[2 * j] = a;
    v[2 * j + 1] = b;
    am = od_absmax_bf16x2(am, p);
  }
  return am;
}

__device__ __forceinline__ uint32_t umax(uint32_t a, uint32_t b) { return a > b ? a : b; }

// Max of the row's bit patterns over the LANES threads that own it (LANES = 256: the whole workgroup).
template <int LANES>
__device__ __forceinline__ uint32_t row_umax(uint32_t v) {
  if constexpr (LANES == OD_WAVE) {
    return od_wave_umax_dpp(v);
  } else if constexpr (LANES < OD_WAVE) {
#pragma unroll
    for (int o = LANES / 2; o > 0; o >>= 1) v = umax(v, (uint32_t)__shfl_xor((int)v, o, OD_WAVE));
    return v;
  } else {
    __shared__ uint32_t red[kThreads / OD_WAVE];
    v = od_wave_umax_dpp(v);
    if (threadIdx.x % OD_WAVE == 0) red[threadIdx.x / OD_WAVE] = v;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kThreads / OD_WAVE; ++i) v = umax(v, red[i]);
    return v;
  }
}

// LANES threads per row; VEC = 8 (16-byte loads) or 1. With VEC = 8 and NIT > 0 a lane holds its NIT groups of 8
// values in registers (K <= NIT * LANES * 8), so the row is read once; NIT = 0 reads it twice (the second pass
// hits L1/L2).
template <int LANES, int VEC, int MODE, bool HAS_INV, int NIT>
__global__ __launch_bounds__(kThreads) void quant_rows_kernel(RowMap m, const uint16_t* __restrict__ inv_s,
                                                              int64_t n_rows, int64_t K) {
  constexpr int kRowsPerBlock = kThreads / LANES;
  const int lane = threadIdx.x % LANES;
  const int64_t r = (int64_t)blockIdx.x * kRowsPerBlock + threadIdx.x / LANES;
  const bool live = r < n_rows;  // no early return: the 256-lane variant has a barrier below
  constexpr bool GATE = MODE == kGate;
  const uint16_t* xin = nullptr;
  const uint16_t* gin = nullptr;
  int8_t* qout = nullptr;
  float* sout = nullptr;
  if (live) map_row<MODE>(m, r, xin, qout, sout, gin);

  if constexpr (VEC == 8 && NIT > 0) {
    float v[NIT][8];
    uint32_t am = 0;
#pragma unroll
    for (int i = 0; i < NIT; ++i) {
      const int64_t k = ((int64_t)i * LANES + lane) * 8;
      if (live && k < K) am = od_absmax_bf16x2(am, load8<HAS_INV, GATE>(xin, gin, inv_s, k, v[i]));
    }
    const float amax = __uint_as_float(row_umax<LANES>(__float_as_uint(od_absmax_bf16x2_value(am))));
    if (!live) return;
    const float scale = od_q8_scale(amax), inv = 1.0f / scale;
#pragma unroll
    for (int i = 0; i < NIT; ++i) {
      const int64_t k = ((int64_t)i * LANES + lane) * 8;
      if (k < K) {
        uint32_t w[2];
        od_q8_words<8>(v[i], scale, inv, w);
        *reinterpret_cast<uint2*>(qout + k) = make_uint2(w[0], w[1]);
      }
    }
    if (lane == 0) *sout = scale;
  } else if constexpr (VEC == 8) {
    uint32_t am = 0;
    if (live) {
      for (int64_t k = (int64_t)lane * 8; k < K; k += LANES * 8) {
        float v[8];
        am = od_absmax_bf16x2(am, load8<HAS_INV, GATE>(xin, gin, inv_s, k, v));
      }
    }
    const float amax = __uint_as_float(row_umax<LANES>(__float_as_uint(od_absmax_bf16x2_value(am))));
    if (!live) return;
    const float scale = od_q8_scale(amax), inv = 1.0f / scale;
    for (int64_t k = (int64_t)lane * 8; k < K; k += LANES * 8) {
      float v[8];
      (void)load8<HAS_INV, GATE>(xin, gin, inv_s, k, v);
      uint32_t w[2];
      od_q8_words<8>(v, scale, inv, w);
      *reinterpret_cast<uint2*>(qout + k) = make_uint2(w[0], w[1]);
    }
    if (lane == 0) *sout = scale;
  } else {
    uint32_t am = 0;
    if (live) {
      for (int64_t k = lane; k < K; k += LANES)
        am = umax(am, __float_as_uint(fabsf(load_val<HAS_INV, GATE>(xin, gin, inv_s, k))));
    }
    const float amax = __uint_as_float(row_umax<LANES>(am));
    if (!live) return;
    const float scale = od_q8_scale(amax), inv = 1.0f / scale;
    for (int64_t k = lane; k < K; k += LANES)
      qout[k] = od_q8_one(load_val<HAS_INV, GATE>(xin, gin, inv_s, k), scale, inv);
    if (lane == 0) *sout = scale;
  }
}

template <int LANES, int VEC, int MODE, bool HAS_INV>
void launch_nit(dim3 grid, hipStream_t st, const RowMap& m, const uint16_t* inv_s, int64_t n_rows, int64_t K) {
  const int64_t groups = (K + VEC * LANES - 1) / (VEC * LANES);  // groups of VEC values per lane
  if (VEC == 8 && groups <= 1) {
    quant_rows_kernel<LANES, VEC, MODE, HAS_INV, 1><<<grid, dim3(kThreads), 0, st>>>(m, inv_s, n_rows, K);
  } else if (VEC == 8 && groups <= 2) {
    quant_rows_kernel<LANES, VEC, MODE, HAS_INV, 2><<<grid, dim3(kThreads), 0, st>>>(m, inv_s, n_rows, K);
  } else if (VEC == 8 && groups <= 4) {
    quant_rows_kernel<LANES, VEC, MODE, HAS_INV, 4><<<grid, dim3(kThreads), 0, st>>>(m, inv_s, n_rows, K);
  } else if (VEC == 8 && LANES == 256 && groups <= 6) {
    quant_rows_kernel<LANES, VEC, MODE, HAS_INV, 6><<<grid, dim3(kThreads), 0, st>>>(m, inv_s, n_rows, K);
  } else {
    quant_rows_kernel<LANES, VEC, MODE, HAS_INV, 0><<<grid, dim3(kThreads), 0, st>>>(m, inv_s, n_rows, K);
  }
}

template <int MODE, bool HAS_INV, int VEC>
int launch_lanes(const RowMap& m, const uint16_t* inv_s, int64_t n_rows, int64_t K, hipStream_t st) {
  const int64_t per_lane = (K + VEC - 1) / VEC;
  int lanes = per_lane <= 8 ? 8 : per_lane <= 16 ? 16 : per_lane <= 32 ? 32 : per_lane <= 64 ? 64 : 256;
  const int64_t rows_per_block = kThreads / lanes;
  const int64_t blocks = (n_rows + rows_per_block - 1) / rows_per_block;
  if (blocks > 0x7fffffff) return OD_ERR_SHAPE;
  dim3 grid((unsigned)blocks);
  switch (lanes) {
    case 8: launch_nit<8, VEC, MODE, HAS_INV>(grid, st, m, inv_s, n_rows, K); break;
    case 16: launch_nit<16, VEC, MODE, HAS_INV>(grid, st, m, inv_s, n_rows, K); break;
    case 32: launch_nit<32, VEC, MODE, HAS_INV>(grid, st, m, inv_s, n_rows, K); break;
    case 64: launch_nit<64, VEC, MODE, HAS_INV>(grid, st, m, inv_s, n_rows, K); break;
    default: launch_nit<256, VEC, MODE, HAS_INV>(grid, st, m, inv_s, n_rows, K); break;
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

extern "C" int od_gate_act_quant(const uint16_t* x, int64_t ldx, const uint16_t* gate, int64_t ldg,
                                 const uint16_t* inv_s, int8_t* xq, int64_t ldq, float* sx, int64_t M, int64_t K,
                                 od_stream_t stream) {
  if (M < 0 || K < 1 || ldx < K || ldq < K || ldg < K) return OD_ERR_SHAPE;
  if (M == 0) return OD_OK;
  if (!x || !gate || !xq || !sx) return OD_ERR_NULL;
  RowMap m{};
  m.x = x;
  m.q = xq;
  m.s = sx;
  m.ldx = ldx;
  m.ldq = ldq;
  m.gate = gate;
  m.ldg = ldg;
  const bool vec_ok = (K % 8 == 0) && (ldx % 8 == 0) && (ldq % 8 == 0) && (ldg % 8 == 0) && od_aligned16(x) &&
                      od_aligned16(gate) && ((((uintptr_t)xq) & 7u) == 0) && (!inv_s || od_aligned16(inv_s));
  return launch_quant<kGate>(m, inv_s, M, K, vec_ok, (hipStream_t)stream);
}

namespace {

// fp32 rows: Int8Tensor.quantize of float32 input, and of float16 / float64 input through x.float() (the reference
// quantizes xf = x.float() whatever the dtype, quant.py:38). One wave per row, 4 rows per workgroup; the max runs on
// |x| bit patterns (a NaN has the largest pattern, so it reaches the scale as in the bf16 rows); the same per-element
// quantizer as the bf16 rows. Not a hot path: the decoder's activations and caches are bf16.
__global__ __launch_bounds__(kThreads) void quant_rows_f32_kernel(const float* __restrict__ x, int64_t ldx,
                                                                  int8_t* __restrict__ q, int64_t ldq,
                                                                  float* __restrict__ s, int64_t n_rows, int64_t K) {
  const int lane = threadIdx.x % OD_WAVE;
  const int64_t r = (int64_t)blockIdx.x * (kThreads / OD_WAVE) + threadIdx.x / OD_WAVE;
  if (r >= n_rows) return;  // a whole wave leaves; no barrier in this kernel
  const float* xin = x + r * ldx;
  uint32_t am = 0;
  for (int64_t k = lane; k < K; k += OD_WAVE) am = umax(am, __float_as_uint(fabsf(xin[k])));
  const float amax = __uint_as_float(od_wave_umax_dpp(am));
  const float scale = od_q8_scale(amax), inv = 1.0f / scale;
  int8_t* qout = q + r * ldq;
  for (int64_t k = lane; k < K; k += OD_WAVE) qout[k] = od_q8_one(xin[k], scale, inv);
  if (lane == 0) s[r] = scale;
}

}  // namespace

extern "C" int od_act_quant_f32(const float* x, int64_t ldx, int8_t* xq, int64_t ldq, float* sx, int64_t M,
                                int64_t K, od_stream_t stream) {
  if (M < 0 || K < 1 || ldx < K || ldq < K) return OD_ERR_SHAPE;
  if (M == 0) return OD_OK;
  if (!x || !xq || !sx) return OD_ERR_NULL;
  constexpr int64_t kRows = kThreads / OD_WAVE;
  const int64_t blocks = (M + kRows - 1) / kRows;
  if (blocks > 0x7fffffff) return OD_ERR_SHAPE;
  quant_rows_f32_kernel<<<dim3((unsigned)blocks), dim3(kThreads), 0, (hipStream_t)stream>>>(x, ldx, xq, ldq, sx, M, K);
  return od_launch_status();
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

namespace {

// ---------------------------------------------------------------------------- int8 K/V row copies
// Copies runs of cache rows (int8 [rows, D] + fp32 scale per row) between two buffers laid out as
// [n_mats][H][cap][D] (a matrix is one layer's K or V of one state). A launch takes up to kMaxSegs runs by value; a
// workgroup copies one 64-row chunk of one run for one (matrix, head): 16-byte loads and stores, HBM-bound.
constexpr int kMaxSegs = 32;
constexpr int kCopyRows = 64;

struct CopySegs {
  int64_t src_row[kMaxSegs], dst_row[kMaxSegs], n_rows[kMaxSegs];
  int first_chunk[kMaxSegs + 1];
  int n_seg;
};

struct CopyArgs {
  const int8_t* src_q;
  const float* src_s;
  int8_t* dst_q;
  float* dst_s;
  int64_t src_mat_q, src_mat_s, src_cap, dst_mat_q, dst_mat_s, dst_cap;
  int H, D;
};

__global__ __launch_bounds__(kThreads) void kv_copy_rows_kernel(CopyArgs a, CopySegs sg) {
  const int chunk = blockIdx.x;
  int s = 0;
  while (s + 1 < sg.n_seg && sg.first_chunk[s + 1] <= chunk) ++s;  // wave-uniform
  const int64_t r0 = (int64_t)(chunk - sg.first_chunk[s]) * kCopyRows;
  const int64_t n = min((int64_t)kCopyRows, sg.n_rows[s] - r0);
  const int mat = blockIdx.y / a.H, h = blockIdx.y % a.H;
  const int64_t src_row = (int64_t)h * a.src_cap + sg.src_row[s] + r0;
  const int64_t dst_row = (int64_t)h * a.dst_cap + sg.dst_row[s] + r0;
  const int8_t* sq = a.src_q + mat * a.src_mat_q + src_row * a.D;
  int8_t* dq = a.dst_q + mat * a.dst_mat_q + dst_row * a.D;
  const int64_t vecs = n * a.D / 16;  // D % 16 == 0
  for (int64_t i = threadIdx.x; i < vecs; i += kThreads)
    reinterpret_cast<uint4*>(dq)[i] = reinterpret_cast<const uint4*>(sq)[i];
  if (threadIdx.x < n) a.dst_s[mat * a.dst_mat_s + dst_row + threadIdx.x] = a.src_s[mat * a.src_mat_s + src_row + threadIdx.x];
}

}  // namespace

extern "C" int od_kv_copy_rows(const int8_t* src_q, const float* src_s, int64_t src_mat_q, int64_t src_mat_s,
                               int64_t src_cap, int8_t* dst_q, float* dst_s, int64_t dst_mat_q, int64_t dst_mat_s,
                               int64_t dst_cap, int64_t n_mats, int64_t H, int64_t D, const int64_t* seg,
                               int64_t n_seg, od_stream_t stream) {
  if (n_mats < 0 || H < 0 || D < 16 || D % 16 || n_seg < 0 || src_cap < 0 || dst_cap < 0) return OD_ERR_SHAPE;
  if (n_mats == 0 || H == 0 || n_seg == 0) return OD_OK;
  if (!src_q || !src_s || !dst_q || !dst_s || !seg) return OD_ERR_NULL;
  if (n_mats * H > 65535) return OD_ERR_SHAPE;
  if (src_mat_q < H * src_cap * D || dst_mat_q < H * dst_cap * D || src_mat_s < H * src_cap || dst_mat_s < H * dst_cap)
    return OD_ERR_SHAPE;
  if (!od_aligned16(src_q) || !od_aligned16(dst_q) || (src_mat_q % 16) || (dst_mat_q % 16)) return OD_ERR_ALIGN;
  for (int64_t i = 0; i < n_seg; ++i) {  // every run inside both buffers (the kernel trusts the table)
    const int64_t s0 = seg[3 * i], d0 = seg[3 * i + 1], n = seg[3 * i + 2];
    if (n < 0 || s0 < 0 || d0 < 0 || s0 + n > src_cap || d0 + n > dst_cap) return OD_ERR_SHAPE;
  }
  CopyArgs a{src_q, src_s, dst_q, dst_s, src_mat_q, src_mat_s, src_cap, dst_mat_q, dst_mat_s, dst_cap, (int)H, (int)D};
  for (int64_t base = 0; base < n_seg; base += kMaxSegs) {
    CopySegs sg{};
    int chunks = 0;
    for (int64_t i = base; i < n_seg && sg.n_seg < kMaxSegs; ++i) {
      const int64_t n = seg[3 * i + 2];
      if (n == 0) continue;
      const int k = sg.n_seg++;
      sg.src_row[k] = seg[3 * i];
      sg.dst_row[k] = seg[3 * i + 1];
      sg.n_rows[k] = n;
      sg.first_chunk[k] = chunks;
      const int64_t c = (n + kCopyRows - 1) / kCopyRows;
      if (chunks + c > 0x7fffffff) return OD_ERR_SHAPE;
      chunks += (int)c;
    }
    if (sg.n_seg == 0) continue;
    sg.first_chunk[sg.n_seg] = chunks;
    kv_copy_rows_kernel<<<dim3((unsigned)chunks, (unsigned)(n_mats * H)), dim3(kThreads), 0, (hipStream_t)stream>>>(a, sg);
    const int rc = od_launch_status();
    if (rc != OD_OK) return rc;
  }
  return OD_OK;
}

extern "C" const char* od_strerror(int code) {
  switch (code) {
    case OD_OK: return "ok";
    case OD_ERR_NULL: return "a required pointer is NULL";
    case OD_ERR_SHAPE: return "a size or stride is out of range or inconsistent";
    case OD_ERR_ALIGN: return "a pointer or leading dimension breaks the 16-byte alignment the kernel needs";
    case OD_ERR_UNSUPPORTED: return "head dim / GQA ratio / row length outside what the kernels are built for";
    case OD_ERR_LAUNCH: return "kernel launch failed";
    case OD_ERR_SCRATCH: return "the work needs more than the library's static scratch (od_*_noalloc)";
    default: return "unknown error";
  }
}

extern "C" int od_abi_version(void) { return 2; }
