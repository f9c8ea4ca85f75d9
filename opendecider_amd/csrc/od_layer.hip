// Row kernels of the dense decoder layer around the W8A8 GEMMs and the branched attention (gfx950):
//   od_rmsnorm_quant   RMSNorm -> (SmoothQuant input scale) -> per-token int8, one pass over HBM
//   od_qk_norm_rope    per-head RMSNorm of q and k + rotary embedding, in place on the QKV GEMM output
//   od_silu_mul_quant  SwiGLU (silu(gate) * up) -> (SmoothQuant input scale) -> per-token int8
// All are HBM-bound (a few bytes per element); each fuses what would otherwise be separate bf16 round trips.
// Rounding follows the bf16 module arithmetic of the decoder they serve (every elementwise product of two bf16
// tensors is rounded to bf16 once). The two values that a plain fp32 evaluation would leave dependent on the device
// (the order of a sum, the last bit of exp / rsqrt) are correctly rounded instead: the RMSNorm factor comes from a
// float64 sum of squares (od_rms_factor) and silu from od_silu_bf16, so the outputs equal the oracle's bit for bit.
#include <type_traits>

#include "od_common.h"

namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ float bfr(float v) { return od_bf16_to_f32(od_f32_to_bf16(v)); }

// Workgroup sum of doubles (wave shuffles, then the per-wave sums in a fixed order).
__device__ __forceinline__ double block_sum_f64(double v, double* red) {
  v = od_group_sum_f64<OD_WAVE>(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  double s = 0.0;
#pragma unroll
  for (int i = 0; i < kThreads / OD_WAVE; ++i) s += red[i];
  return s;
}

// Max over the workgroup of non-negative fp32 values compared as bit patterns (a NaN dominates).
__device__ __forceinline__ float block_max_bits(float f, float* red) {
  const uint32_t v = od_wave_umax_dpp(__float_as_uint(f));
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = __uint_as_float(v);
  __syncthreads();
  uint32_t s = 0;
#pragma unroll
  for (int i = 0; i < kThreads / OD_WAVE; ++i) s = max(s, __float_as_uint(red[i]));
  return __uint_as_float(s);
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

// ---------------------------------------------------------------------------- RMSNorm + quantize
// y_k = bf16(w_k * bf16(x_k * r)), r = 1 / sqrt(mean(x^2) + eps) (od_rms_factor), or with zc (Qwen3.5's norm, one
// rounding) y_k = bf16((x_k * r) * (1 + w_k)) in fp32; then optionally y_k = bf16(y_k * inv_s_k);
// then the per-row int8 quantizer. One workgroup per row; the row is read three times (L1/L2 after the first).
__device__ __forceinline__ float rms_val(const uint16_t* xr, const uint16_t* w, const uint16_t* inv_s, int k, float r,
                                         bool zc) {
  const float x = od_bf16_to_f32(xr[k]), wk = od_bf16_to_f32(w[k]);
  float y = zc ? bfr((x * r) * (1.0f + wk)) : bfr(wk * bfr(x * r));
  if (inv_s) y = bfr(y * od_bf16_to_f32(inv_s[k]));
  return y;
}

__global__ __launch_bounds__(kThreads) void rmsnorm_quant_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                                 const uint16_t* __restrict__ w,
                                                                 const uint16_t* __restrict__ inv_s, float eps,
                                                                 int8_t* __restrict__ xq, int64_t ldq,
                                                                 float* __restrict__ sx, int K, int zc) {
  __shared__ float red[kThreads / OD_WAVE];
  __shared__ double red64[kThreads / OD_WAVE];
  const int64_t row = blockIdx.x;
  const uint16_t* xr = x + row * ldx;
  double ss = 0.0;
  for (int k = threadIdx.x; k < K; k += kThreads) {
    const double v = (double)od_bf16_to_f32(xr[k]);
    ss = fma(v, v, ss);
  }
  ss = block_sum_f64(ss, red64);
  const float r = od_rms_factor(ss, K, eps);
  float amax = 0.0f;
  for (int k = threadIdx.x; k < K; k += kThreads) amax = fmaxf(amax, fabsf(rms_val(xr, w, inv_s, k, r, zc)));
  amax = block_max(amax, red);
  const float scale = od_q8_scale(amax), inv = 1.0f / scale;
  int8_t* qr = xq + row * ldq;
  for (int k = threadIdx.x; k < K; k += kThreads) qr[k] = od_q8_one(rms_val(xr, w, inv_s, k, r, zc), scale, inv);
  if (threadIdx.x == 0) sx[row] = scale;
}

// ---------------------------------------------------------------------------- SwiGLU + quantize
// y_k = bf16(bf16(silu(g_k)) * u_k) with bf16(silu(g)) from od_silu_bf16, g = gu[row, k], u = gu[row, F + k].
__device__ __forceinline__ float swiglu_val(const uint16_t* gr, int64_t F, const uint16_t* inv_s, int64_t k) {
  const float g = od_bf16_to_f32(gr[k]);
  const float u = od_bf16_to_f32(gr[F + k]);
  float y = bfr(od_silu_bf16(g) * u);
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
  const float scale = od_q8_scale(amax), inv = 1.0f / scale;
  int8_t* qr = aq + row * ldq;
  for (int64_t k = threadIdx.x; k < F; k += kThreads) qr[k] = od_q8_one(swiglu_val(gr, F, inv_s, k), scale, inv);
  if (threadIdx.x == 0) sa[row] = scale;
}

// ---------------------------------------------------------------------------- q/k RMSNorm + RoPE
// For every token row and every q head then k head (D values at qkv[row, head * D ...]):
//   n_d = bf16(w_d * bf16(x_d * r)),  r = 1 / sqrt(mean(x^2) + eps) (od_rms_factor)
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
  const double ss = od_group_sum_f64<L>(fma((double)a, (double)a, (double)b * (double)b));
  const float r = od_rms_factor(ss, D, eps);
  const float na = bfr(od_bf16_to_f32(w[i]) * bfr(a * r));
  const float nb = bfr(od_bf16_to_f32(w[i + L]) * bfr(b * r));
  const int64_t p = pos[row];
  const bool in_table = p >= 0 && p < n_pos;  // a position past the tables yields NaN, never an out-of-bounds read
  const float c = in_table ? od_bf16_to_f32(cos_t[p * L + i]) : __builtin_nanf("");
  const float s = in_table ? od_bf16_to_f32(sin_t[p * L + i]) : __builtin_nanf("");
  hp[i] = od_f32_to_bf16(bfr(na * c) + bfr(-nb * s));
  hp[i + L] = od_f32_to_bf16(bfr(nb * c) + bfr(na * s));
}

// ---------------------------------------------------------------------------- register-resident fast paths
// A row of 256 * 8 * NV elements is held in registers (NV 16-byte vectors of 8 bf16 per thread, vector v of thread
// t covering elements (v * 256 + t) * 8 .. +7), so the row is read from HBM once and written once. Every load of a
// row (x, the norm weight, the smoothing scale) is issued before the first reduction. These kernels are bound by
// VALU issue rather than HBM at 4096 x 4096: the bf16 round trips go two values per v_cvt_pk_bf16_f32 and the
// quantizer multiplies by 1 / scale (exact, see od_q8_words).
__device__ __forceinline__ void unpack2(uint32_t w, float& lo, float& hi) {
  lo = __uint_as_float(w << 16);
  hi = __uint_as_float(w & 0xffff0000u);
}

__device__ __forceinline__ uint32_t word(const uint4& u, int j) { return j == 0 ? u.x : j == 1 ? u.y : j == 2 ? u.z : u.w; }

__device__ __forceinline__ void store_q8(int8_t* dst, const float (&y)[8], float scale, float inv) {
  uint32_t w[2];
  od_q8_words<8>(y, scale, inv, w);
  *reinterpret_cast<uint2*>(dst) = make_uint2(w[0], w[1]);
}

template <int NV, bool INV, bool ZC>
__global__ __launch_bounds__(kThreads) void rmsnorm_quant_vec_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                                     const uint16_t* __restrict__ w,
                                                                     const uint16_t* __restrict__ inv_s, float eps,
                                                                     int8_t* __restrict__ xq, int64_t ldq,
                                                                     float* __restrict__ sx) {
  constexpr int K = kThreads * 8 * NV;
  __shared__ float red[kThreads / OD_WAVE];
  const int64_t row = blockIdx.x;
  const uint16_t* xr = x + row * ldx;
  uint4 xv[NV], wv[NV], iv[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int k = (v * kThreads + threadIdx.x) * 8;
    xv[v] = *reinterpret_cast<const uint4*>(xr + k);
    wv[v] = *reinterpret_cast<const uint4*>(w + k);
    if (INV) iv[v] = *reinterpret_cast<const uint4*>(inv_s + k);
  }
  __shared__ double red64[kThreads / OD_WAVE];
  float y[NV][8];
  double ss = 0.0;
#pragma unroll
  for (int v = 0; v < NV; ++v) {
#pragma unroll
    for (int j = 0; j < 4; ++j) unpack2(word(xv[v], j), y[v][2 * j], y[v][2 * j + 1]);
#pragma unroll
    for (int e = 0; e < 8; ++e) ss = fma((double)y[v][e], (double)y[v][e], ss);
  }
  ss = block_sum_f64(ss, red64);
  const float r = od_rms_factor(ss, K, eps);
  uint32_t am = 0;
#pragma unroll
  for (int v = 0; v < NV; ++v) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float a = y[v][2 * j] * r, b = y[v][2 * j + 1] * r, wa, wb;
      if (!ZC) od_bfr2(a, b);
      unpack2(word(wv[v], j), wa, wb);
      if (ZC) {
        a *= 1.0f + wa;
        b *= 1.0f + wb;
      } else {
        a *= wa;
        b *= wb;
      }
      uint32_t p = od_bfr2(a, b);
      if (INV) {
        float ia, ib;
        unpack2(word(iv[v], j), ia, ib);
        a *= ia;
        b *= ib;
        p = od_bfr2(a, b);
      }
      y[v][2 * j] = a;
      y[v][2 * j + 1] = b;
      am = od_absmax_bf16x2(am, p);
    }
  }
  const float amax = block_max_bits(od_absmax_bf16x2_value(am), red);
  const float scale = od_q8_scale(amax), inv = 1.0f / scale;
  int8_t* qr = xq + row * ldq;
#pragma unroll
  for (int v = 0; v < NV; ++v) store_q8(qr + (v * kThreads + threadIdx.x) * 8, y[v], scale, inv);
  if (threadIdx.x == 0) sx[row] = scale;
}


template <int NV, bool INV>
__global__ __launch_bounds__(kThreads) void silu_mul_quant_vec_kernel(const uint16_t* __restrict__ gu, int64_t ldg,
                                                                      const uint16_t* __restrict__ inv_s,
                                                                      int8_t* __restrict__ aq, int64_t ldq,
                                                                      float* __restrict__ sa) {
  constexpr int F = kThreads * 8 * NV;
  __shared__ float red[kThreads / OD_WAVE];
  const int64_t row = blockIdx.x;
  const uint16_t* gr = gu + row * ldg;
  float y[NV][8];
  uint32_t am = 0;
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int k = (v * kThreads + threadIdx.x) * 8;
    const uint4 g8 = *reinterpret_cast<const uint4*>(gr + k);
    const uint4 u8 = *reinterpret_cast<const uint4*>(gr + F + k);
    uint4 i8;
    if (INV) i8 = *reinterpret_cast<const uint4*>(inv_s + k);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float ga, gb, ua, ub;
      unpack2(word(g8, j), ga, gb);
      unpack2(word(u8, j), ua, ub);
      float a = od_silu_bf16(ga), b = od_silu_bf16(gb);
      a *= ua;
      b *= ub;
      uint32_t p = od_bfr2(a, b);
      if (INV) {
        float ia, ib;
        unpack2(word(i8, j), ia, ib);
        a *= ia;
        b *= ib;
        p = od_bfr2(a, b);
      }
      y[v][2 * j] = a;
      y[v][2 * j + 1] = b;
      am = od_absmax_bf16x2(am, p);
    }
  }
  const float amax = block_max_bits(od_absmax_bf16x2_value(am), red);
  const float scale = od_q8_scale(amax), inv = 1.0f / scale;
  int8_t* qr = aq + row * ldq;
#pragma unroll
  for (int v = 0; v < NV; ++v) store_q8(qr + (v * kThreads + threadIdx.x) * 8, y[v], scale, inv);
  if (threadIdx.x == 0) sa[row] = scale;
}

// q/k RMSNorm + RoPE with G = D / 8 lanes per head (lane j holds d = 4j..4j+3 and the rotary partners
// D/2 + 4j..D/2 + 4j + 3: 8-byte loads and stores) or, for 16-byte aligned rows, G = D / 16 (8 + 8 values per lane,
// 16-byte accesses); no lane exchange is needed for the rotation.
// APPEND: the launch also covers the n_heads_k value heads of every row, and the key heads (after RoPE) and value
// heads are quantized per (token, head) into int8 caches, with the bytes od_kv_quant_append writes for the same
// bf16 values (row m = b * S + i of qkv goes to cache row (b * n_heads_k + h) * cap + n0 + i).
struct KvAppend {
  int8_t* kq;
  float* ks;
  int8_t* vq;
  float* vs;
  int64_t S, cap, n0;
};

// H = 4 bf16 values (8 bytes) or H = 8 (16 bytes) of one vector load
template <int H>
using VecH = std::conditional_t<H == 4, uint2, uint4>;

template <int H>
__device__ __forceinline__ void unpackh(const VecH<H>& u, float (&f)[H]) {
  const uint32_t* w = reinterpret_cast<const uint32_t*>(&u);
#pragma unroll
  for (int k = 0; k < H / 2; ++k) {
    f[2 * k] = __uint_as_float(w[k] << 16);
    f[2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
  }
}

template <int H>
__device__ __forceinline__ VecH<H> packh(const uint16_t (&h)[H]) {
  VecH<H> v;
  uint32_t* w = reinterpret_cast<uint32_t*>(&v);
#pragma unroll
  for (int k = 0; k < H / 2; ++k) w[k] = (uint32_t)h[2 * k] | ((uint32_t)h[2 * k + 1] << 16);
  return v;
}

// Quantizes a head's D bf16 values held 2H per lane (oa: d = da .. da + H - 1, ob: d = db .. db + H - 1) over the G
// lanes of its group and writes the int8 row and its scale.
template <int D, int H>
__device__ __forceinline__ void quant_head(const uint16_t (&oa)[H], const uint16_t (&ob)[H], int j, int da, int db,
                                           int8_t* qrow, float* srow) {
  constexpr int G = D / (2 * H);
  float y[2 * H];
  uint32_t bits = 0;
#pragma unroll
  for (int e = 0; e < H; ++e) {
    y[e] = od_bf16_to_f32(oa[e]);
    y[H + e] = od_bf16_to_f32(ob[e]);
    bits = max(bits, (uint32_t)(oa[e] & 0x7fffu));
    bits = max(bits, (uint32_t)(ob[e] & 0x7fffu));
  }
#pragma unroll
  for (int o = G / 2; o > 0; o >>= 1) bits = max(bits, (uint32_t)__shfl_xor((int)bits, o, OD_WAVE));
  const float scale = od_q8_scale(__uint_as_float(bits << 16)), inv = 1.0f / scale;
  uint32_t w[2 * H / 4];
  od_q8_words<2 * H>(y, scale, inv, w);
  if constexpr (H == 4) {
    *reinterpret_cast<uint32_t*>(qrow + da) = w[0];
    *reinterpret_cast<uint32_t*>(qrow + db) = w[1];
  } else {
    *reinterpret_cast<uint2*>(qrow + da) = make_uint2(w[0], w[1]);
    *reinterpret_cast<uint2*>(qrow + db) = make_uint2(w[2], w[3]);
  }
  if (j == 0) *srow = scale;
}

// Partial rotary (RD < D, Qwen3.5's 64 of 256): rotate_half acts on the first RD dims only (pairs d, d + RD/2) and the
// other D - RD pass through the norm unrotated. A group of G = D / (2H) lanes owns a head: lane j < RD / (2H) holds
// the pairs Hj .. Hj + H - 1 and RD/2 + Hj .., a lane j >= RD / (2H) the 2H dims RD + 2H (j - RD / (2H)) .. +2H - 1, so
// no lane exchange is needed for the rotation. H = 4: 8-byte loads and stores; H = 8: 16-byte ones (rows and tables
// 16-byte aligned), half the lanes per head. The tables are [n_pos, RD/2]. ZC: the Qwen3.5 norm, one rounding:
// n_d = bf16((x_d * r) * (1 + w_d)) (fp32 products), instead of bf16(w_d * bf16(x_d * r)).
template <int D, int RD, bool ZC, bool APPEND, int H>
__global__ __launch_bounds__(kThreads) void qk_rope_vec_kernel(uint16_t* __restrict__ qkv, int64_t ld, int64_t M,
                                                               int n_heads_q, int n_heads_k,
                                                               const uint16_t* __restrict__ qw,
                                                               const uint16_t* __restrict__ kw,
                                                               const uint16_t* __restrict__ cos_t,
                                                               const uint16_t* __restrict__ sin_t, int64_t n_pos,
                                                               const int32_t* __restrict__ pos, float eps,
                                                               KvAppend kv) {
  constexpr int G = D / (2 * H), RL = RD / (2 * H), RH = RD / 2;
  static_assert(RD % (2 * H) == 0 && RD <= D, "rotary dims");
  using V = VecH<H>;
  const int heads = n_heads_q + n_heads_k * (APPEND ? 2 : 1);
  const int64_t gh = (int64_t)blockIdx.x * (kThreads / G) + threadIdx.x / G;
  if (gh >= M * heads) return;  // whole G-lane groups exit together
  const int64_t row = gh / heads;
  const int head = (int)(gh % heads);
  const int j = threadIdx.x % G;
  const bool rot = j < RL;  // this lane holds rotary pairs
  const int da = rot ? H * j : RD + 2 * H * (j - RL), db = rot ? RH + H * j : da + H;
  uint16_t* hp = qkv + row * ld + (int64_t)head * D;
  const V ra = *reinterpret_cast<const V*>(hp + da), rb = *reinterpret_cast<const V*>(hp + db);
  int64_t crow = 0;
  if (APPEND) {
    const int64_t b = row / kv.S, i = row % kv.S;
    crow = (b * n_heads_k + (head - n_heads_q) % n_heads_k) * kv.cap + kv.n0 + i;
  }
  if (APPEND && head >= n_heads_q + n_heads_k) {  // a value head: quantize only
    const uint32_t* wa = reinterpret_cast<const uint32_t*>(&ra);
    const uint32_t* wb = reinterpret_cast<const uint32_t*>(&rb);
    uint16_t va[H], vb[H];
#pragma unroll
    for (int k = 0; k < H / 2; ++k) {
      va[2 * k] = (uint16_t)wa[k];
      va[2 * k + 1] = (uint16_t)(wa[k] >> 16);
      vb[2 * k] = (uint16_t)wb[k];
      vb[2 * k + 1] = (uint16_t)(wb[k] >> 16);
    }
    quant_head<D, H>(va, vb, j, da, db, kv.vq + crow * D, kv.vs + crow);
    return;
  }
  const uint16_t* w = head < n_heads_q ? qw : kw;
  float a[H], b[H], fa[H], fb[H];
  unpackh<H>(ra, a);
  unpackh<H>(rb, b);
  unpackh<H>(*reinterpret_cast<const V*>(w + da), fa);
  unpackh<H>(*reinterpret_cast<const V*>(w + db), fb);
  double ss = 0.0;
#pragma unroll
  for (int e = 0; e < H; ++e) ss = fma((double)b[e], (double)b[e], fma((double)a[e], (double)a[e], ss));
  ss = od_group_sum_f64<G>(ss);
  const float r = od_rms_factor(ss, D, eps);
  float na[H], nb[H];
#pragma unroll
  for (int e = 0; e < H; ++e) {
    if constexpr (ZC) {
      na[e] = bfr((a[e] * r) * (1.0f + fa[e]));
      nb[e] = bfr((b[e] * r) * (1.0f + fb[e]));
    } else {
      na[e] = bfr(fa[e] * bfr(a[e] * r));
      nb[e] = bfr(fb[e] * bfr(b[e] * r));
    }
  }
  uint16_t oa[H], ob[H];
  if (rot) {
    const int64_t p = pos[row];
    const bool in_table = p >= 0 && p < n_pos;  // a position past the tables yields NaN, never an out-of-bounds read
    float c[H], sn[H];
    if (in_table) {
      unpackh<H>(*reinterpret_cast<const V*>(cos_t + p * RH + H * j), c);
      unpackh<H>(*reinterpret_cast<const V*>(sin_t + p * RH + H * j), sn);
    } else {
#pragma unroll
      for (int e = 0; e < H; ++e) c[e] = sn[e] = __builtin_nanf("");
    }
#pragma unroll
    for (int e = 0; e < H; ++e) {
      oa[e] = od_f32_to_bf16(bfr(na[e] * c[e]) + bfr(-nb[e] * sn[e]));
      ob[e] = od_f32_to_bf16(bfr(nb[e] * c[e]) + bfr(na[e] * sn[e]));
    }
  } else {
#pragma unroll
    for (int e = 0; e < H; ++e) {
      oa[e] = od_f32_to_bf16(na[e]);
      ob[e] = od_f32_to_bf16(nb[e]);
    }
  }
  *reinterpret_cast<V*>(hp + da) = packh<H>(oa);
  *reinterpret_cast<V*>(hp + db) = packh<H>(ob);
  if (APPEND && head >= n_heads_q) quant_head<D, H>(oa, ob, j, da, db, kv.kq + crow * D, kv.ks + crow);
}

template <int NV>
void launch_rmsnorm_vec(dim3 grid, hipStream_t st, const uint16_t* x, int64_t ldx, const uint16_t* w,
                        const uint16_t* inv_s, float eps, int8_t* xq, int64_t ldq, float* sx, bool zc) {
  if (zc) {
    if (inv_s) rmsnorm_quant_vec_kernel<NV, true, true><<<grid, dim3(kThreads), 0, st>>>(x, ldx, w, inv_s, eps, xq, ldq, sx);
    else rmsnorm_quant_vec_kernel<NV, false, true><<<grid, dim3(kThreads), 0, st>>>(x, ldx, w, inv_s, eps, xq, ldq, sx);
  } else {
    if (inv_s) rmsnorm_quant_vec_kernel<NV, true, false><<<grid, dim3(kThreads), 0, st>>>(x, ldx, w, inv_s, eps, xq, ldq, sx);
    else rmsnorm_quant_vec_kernel<NV, false, false><<<grid, dim3(kThreads), 0, st>>>(x, ldx, w, inv_s, eps, xq, ldq, sx);
  }
}

template <int NV>
void launch_silu_vec(dim3 grid, hipStream_t st, const uint16_t* gu, int64_t ldg, const uint16_t* inv_s, int8_t* aq,
                     int64_t ldq, float* sa) {
  if (inv_s) {
    silu_mul_quant_vec_kernel<NV, true><<<grid, dim3(kThreads), 0, st>>>(gu, ldg, inv_s, aq, ldq, sa);
  } else {
    silu_mul_quant_vec_kernel<NV, false><<<grid, dim3(kThreads), 0, st>>>(gu, ldg, inv_s, aq, ldq, sa);
  }
}

}  // namespace

extern "C" int od_rmsnorm_quant_ex(const uint16_t* x, int64_t ldx, const uint16_t* w, const uint16_t* inv_s,
                                   float eps, int weight_offset, int8_t* xq, int64_t ldq, float* sx, int64_t M,
                                   int64_t K, od_stream_t stream) {
  if (M < 0 || K < 1 || K > (1 << 30) || ldx < K || ldq < K) return OD_ERR_SHAPE;
  if (weight_offset != 0 && weight_offset != 1) return OD_ERR_UNSUPPORTED;
  if (M == 0) return OD_OK;
  if (!x || !w || !xq || !sx) return OD_ERR_NULL;
  if (M > 0x7fffffff) return OD_ERR_SHAPE;
  hipStream_t st = (hipStream_t)stream;
  const bool zc = weight_offset != 0;
  const bool vec = (ldx % 8 == 0) && (ldq % 8 == 0) && od_aligned16(x) && od_aligned16(w) &&
                   (!inv_s || od_aligned16(inv_s)) && ((((uintptr_t)xq) & 7u) == 0);
  const dim3 grid((unsigned)M), block(kThreads);
  if (vec && K == 2048) {
    launch_rmsnorm_vec<1>(grid, st, x, ldx, w, inv_s, eps, xq, ldq, sx, zc);
  } else if (vec && K == 4096) {
    launch_rmsnorm_vec<2>(grid, st, x, ldx, w, inv_s, eps, xq, ldq, sx, zc);
  } else if (vec && K == 8192) {
    launch_rmsnorm_vec<4>(grid, st, x, ldx, w, inv_s, eps, xq, ldq, sx, zc);
  } else {
    rmsnorm_quant_kernel<<<grid, block, 0, st>>>(x, ldx, w, inv_s, eps, xq, ldq, sx, (int)K, zc ? 1 : 0);
  }
  return od_launch_status();
}

extern "C" int od_rmsnorm_quant(const uint16_t* x, int64_t ldx, const uint16_t* w, const uint16_t* inv_s, float eps,
                                int8_t* xq, int64_t ldq, float* sx, int64_t M, int64_t K, od_stream_t stream) {
  return od_rmsnorm_quant_ex(x, ldx, w, inv_s, eps, 0, xq, ldq, sx, M, K, stream);
}

extern "C" int od_silu_mul_quant(const uint16_t* gu, int64_t ldg, int64_t F, const uint16_t* inv_s, int8_t* aq,
                                 int64_t ldq, float* sa, int64_t M, od_stream_t stream) {
  if (M < 0 || F < 1 || ldg < 2 * F || ldq < F) return OD_ERR_SHAPE;
  if (M == 0) return OD_OK;
  if (!gu || !aq || !sa) return OD_ERR_NULL;
  if (M > 0x7fffffff) return OD_ERR_SHAPE;
  hipStream_t st = (hipStream_t)stream;
  const bool vec = (ldg % 8 == 0) && (F % 8 == 0) && (ldq % 8 == 0) && od_aligned16(gu) &&
                   (!inv_s || od_aligned16(inv_s)) && ((((uintptr_t)aq) & 7u) == 0);
  const dim3 grid((unsigned)M), block(kThreads);
  if (vec && F == 2048 * 6) {
    launch_silu_vec<6>(grid, st, gu, ldg, inv_s, aq, ldq, sa);
  } else if (vec && F == 2048 * 4) {
    launch_silu_vec<4>(grid, st, gu, ldg, inv_s, aq, ldq, sa);
  } else if (vec && F == 2048 * 3) {
    launch_silu_vec<3>(grid, st, gu, ldg, inv_s, aq, ldq, sa);
  } else {
    silu_mul_quant_kernel<<<grid, block, 0, st>>>(gu, ldg, F, inv_s, aq, ldq, sa);
  }
  return od_launch_status();
}

namespace {

bool aligned8(const void* p) { return (((uintptr_t)p) & 7u) == 0; }

template <int D, int RD, bool ZC, bool APPEND>
void launch_rope_vec_t(bool wide, int64_t items, hipStream_t st, uint16_t* qkv, int64_t ld, int64_t M,
                       int64_t n_heads_q, int64_t n_heads_k, const uint16_t* q_w, const uint16_t* k_w,
                       const uint16_t* cos_t, const uint16_t* sin_t, int64_t n_pos, const int32_t* pos, float eps,
                       const KvAppend& kv) {
  // items: (row, head) pairs; a workgroup takes kThreads / G of them, G = D / 16 lanes (wide) or D / 8
  if (wide) {
    const dim3 grid((unsigned)((items + kThreads / (D / 16) - 1) / (kThreads / (D / 16))));
    qk_rope_vec_kernel<D, RD, ZC, APPEND, 8><<<grid, dim3(kThreads), 0, st>>>(
        qkv, ld, M, (int)n_heads_q, (int)n_heads_k, q_w, k_w, cos_t, sin_t, n_pos, pos, eps, kv);
  } else {
    const dim3 grid((unsigned)((items + kThreads / (D / 8) - 1) / (kThreads / (D / 8))));
    qk_rope_vec_kernel<D, RD, ZC, APPEND, 4><<<grid, dim3(kThreads), 0, st>>>(
        qkv, ld, M, (int)n_heads_q, (int)n_heads_k, q_w, k_w, cos_t, sin_t, n_pos, pos, eps, kv);
  }
}

// The (D, rotary dims) pairs the vector kernel is built for: full rotary at D = 64, 128, 256 and a quarter of the
// head (Qwen3.5's partial_rotary_factor 0.25).
bool rope_shape_ok(int64_t D, int64_t rot_dim) {
  return (D == 64 || D == 128 || D == 256) && (rot_dim == D || rot_dim == D / 4);
}

template <bool APPEND>
int launch_rope_vec(uint16_t* qkv, int64_t ld, int64_t M, int64_t n_heads_q, int64_t n_heads_k, int64_t D,
                    int64_t rot_dim, bool zc, const uint16_t* q_w, const uint16_t* k_w, const uint16_t* cos_t,
                    const uint16_t* sin_t, int64_t n_pos, const int32_t* pos, float eps, const KvAppend& kv,
                    hipStream_t st) {
  const int64_t heads = n_heads_q + n_heads_k * (APPEND ? 2 : 1);
  const int64_t per_block = kThreads / (D / 8);
  const int64_t blocks = (M * heads + per_block - 1) / per_block;
  if (blocks > 0x7fffffff || heads > 0x7fffffff) return OD_ERR_SHAPE;
  if (!rope_shape_ok(D, rot_dim)) return OD_ERR_UNSUPPORTED;
  // 16-byte rows, weights and tables (and 8-byte cache rows): 16 values per lane, 16-byte loads and stores
  auto al16 = [](const void* q) { return (((uintptr_t)q) & 15u) == 0; };
  const bool wide = ld % 8 == 0 && al16(qkv) && al16(q_w) && al16(k_w) && al16(cos_t) && al16(sin_t) &&
                    (!APPEND || (aligned8(kv.kq) && aligned8(kv.vq)));
  const int64_t items = M * heads;
  auto go = [&](auto DC) {
    constexpr int DD = decltype(DC)::value;
    const bool full = rot_dim == DD;
    if (zc) {
      if (full) launch_rope_vec_t<DD, DD, true, APPEND>(wide, items, st, qkv, ld, M, n_heads_q, n_heads_k, q_w, k_w, cos_t, sin_t, n_pos, pos, eps, kv);
      else launch_rope_vec_t<DD, DD / 4, true, APPEND>(wide, items, st, qkv, ld, M, n_heads_q, n_heads_k, q_w, k_w, cos_t, sin_t, n_pos, pos, eps, kv);
    } else {
      if (full) launch_rope_vec_t<DD, DD, false, APPEND>(wide, items, st, qkv, ld, M, n_heads_q, n_heads_k, q_w, k_w, cos_t, sin_t, n_pos, pos, eps, kv);
      else launch_rope_vec_t<DD, DD / 4, false, APPEND>(wide, items, st, qkv, ld, M, n_heads_q, n_heads_k, q_w, k_w, cos_t, sin_t, n_pos, pos, eps, kv);
    }
  };
  if (D == 256) go(std::integral_constant<int, 256>{});
  else if (D == 128) go(std::integral_constant<int, 128>{});
  else go(std::integral_constant<int, 64>{});
  return od_launch_status();
}

}  // namespace

extern "C" int od_qk_norm_rope_ex(uint16_t* qkv, int64_t ld, int64_t M, int64_t n_heads_q, int64_t n_heads_k,
                                  int64_t D, int64_t rot_dim, int weight_offset, const uint16_t* q_w,
                                  const uint16_t* k_w, const uint16_t* cos_t, const uint16_t* sin_t, int64_t n_pos,
                                  const int32_t* pos, float eps, od_stream_t stream) {
  if (M < 0 || n_heads_q < 0 || n_heads_k < 0 || ld < (n_heads_q + n_heads_k) * D) return OD_ERR_SHAPE;
  if (weight_offset != 0 && weight_offset != 1) return OD_ERR_UNSUPPORTED;
  if (!rope_shape_ok(D, rot_dim)) return OD_ERR_UNSUPPORTED;
  const int64_t heads = n_heads_q + n_heads_k;
  if (M == 0 || heads == 0) return OD_OK;
  if (!qkv || !q_w || !k_w || !cos_t || !sin_t || !pos) return OD_ERR_NULL;
  const bool vec = (ld % 4 == 0) && aligned8(qkv) && aligned8(q_w) && aligned8(k_w) && aligned8(cos_t) &&
                   aligned8(sin_t);
  hipStream_t st = (hipStream_t)stream;
  if (vec)
    return launch_rope_vec<false>(qkv, ld, M, n_heads_q, n_heads_k, D, rot_dim, weight_offset != 0, q_w, k_w, cos_t,
                                  sin_t, n_pos, pos, eps, KvAppend{}, st);
  // unaligned rows: the scalar kernel, for the full-rotary Llama-style norm at D = 64 or 128 only
  if (rot_dim != D || weight_offset != 0 || D == 256) return OD_ERR_ALIGN;
  const int64_t per_block = kThreads / (D / 2);
  const int64_t blocks = (M * heads + per_block - 1) / per_block;
  if (blocks > 0x7fffffff || heads > 0x7fffffff) return OD_ERR_SHAPE;
  if (D == 128)
    qk_norm_rope_kernel<128><<<dim3((unsigned)blocks), dim3(kThreads), 0, st>>>(
        qkv, ld, M, (int)n_heads_q, (int)n_heads_k, q_w, k_w, cos_t, sin_t, n_pos, pos, eps);
  else
    qk_norm_rope_kernel<64><<<dim3((unsigned)blocks), dim3(kThreads), 0, st>>>(
        qkv, ld, M, (int)n_heads_q, (int)n_heads_k, q_w, k_w, cos_t, sin_t, n_pos, pos, eps);
  return od_launch_status();
}

extern "C" int od_qk_norm_rope(uint16_t* qkv, int64_t ld, int64_t M, int64_t n_heads_q, int64_t n_heads_k,
                               int64_t D, const uint16_t* q_w, const uint16_t* k_w, const uint16_t* cos_t,
                               const uint16_t* sin_t, int64_t n_pos, const int32_t* pos, float eps,
                               od_stream_t stream) {
  if (D != 64 && D != 128) return OD_ERR_UNSUPPORTED;
  return od_qk_norm_rope_ex(qkv, ld, M, n_heads_q, n_heads_k, D, D, 0, q_w, k_w, cos_t, sin_t, n_pos, pos, eps,
                            stream);
}

extern "C" int od_qk_norm_rope_kv_append_ex(uint16_t* qkv, int64_t ld, int64_t B, int64_t S, int64_t n_heads_q,
                                            int64_t n_heads_k, int64_t D, int64_t rot_dim, int weight_offset,
                                            const uint16_t* q_w, const uint16_t* k_w, const uint16_t* cos_t,
                                            const uint16_t* sin_t, int64_t n_pos, const int32_t* pos, float eps,
                                            int8_t* kq, float* ks, int8_t* vq, float* vs, int64_t cap, int64_t n0,
                                            od_stream_t stream) {
  if (B < 0 || S < 0 || n_heads_q < 0 || n_heads_k < 0 || ld < (n_heads_q + 2 * n_heads_k) * D) return OD_ERR_SHAPE;
  if (n0 < 0 || cap < 0 || n0 + S > cap) return OD_ERR_SHAPE;
  if (weight_offset != 0 && weight_offset != 1) return OD_ERR_UNSUPPORTED;
  if (!rope_shape_ok(D, rot_dim)) return OD_ERR_UNSUPPORTED;
  const int64_t M = B * S;
  if (M == 0 || n_heads_q + n_heads_k == 0) return OD_OK;
  if (!qkv || !q_w || !k_w || !cos_t || !sin_t || !pos) return OD_ERR_NULL;
  if (n_heads_k > 0 && (!kq || !ks || !vq || !vs)) return OD_ERR_NULL;
  if (B * n_heads_k * cap > (int64_t)1 << 40) return OD_ERR_SHAPE;
  if ((ld % 4) || !aligned8(qkv) || !aligned8(q_w) || !aligned8(k_w) || !aligned8(cos_t) || !aligned8(sin_t) ||
      (((uintptr_t)kq) & 3u) || (((uintptr_t)vq) & 3u))
    return OD_ERR_ALIGN;
  KvAppend kv{kq, ks, vq, vs, S, cap, n0};
  return launch_rope_vec<true>(qkv, ld, M, n_heads_q, n_heads_k, D, rot_dim, weight_offset != 0, q_w, k_w, cos_t,
                               sin_t, n_pos, pos, eps, kv, (hipStream_t)stream);
}

extern "C" int od_qk_norm_rope_kv_append(uint16_t* qkv, int64_t ld, int64_t B, int64_t S, int64_t n_heads_q,
                                         int64_t n_heads_k, int64_t D, const uint16_t* q_w, const uint16_t* k_w,
                                         const uint16_t* cos_t, const uint16_t* sin_t, int64_t n_pos,
                                         const int32_t* pos, float eps, int8_t* kq, float* ks, int8_t* vq, float* vs,
                                         int64_t cap, int64_t n0, od_stream_t stream) {
  if (D != 64 && D != 128) return OD_ERR_UNSUPPORTED;
  return od_qk_norm_rope_kv_append_ex(qkv, ld, B, S, n_heads_q, n_heads_k, D, D, 0, q_w, k_w, cos_t, sin_t, n_pos,
                                      pos, eps, kq, ks, vq, vs, cap, n0, stream);
}
