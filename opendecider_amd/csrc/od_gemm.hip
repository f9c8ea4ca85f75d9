// W8A8 GEMM for gfx950: int8 A [M,K] x int8 W [N,K]^T -> exact int32 accumulators on the CDNA4 int8 matrix
// cores (V_MFMA_I32_32X32X32_I8), then the dequant epilogue out = bf16(float(acc) * sa[m] * sw[n] (+ bias)
// (+ residual)).
//
// Tiling (MFMA-bound at the 9B shapes; one workgroup of 8 waves per CU, two per SIMD so that one wave's MFMAs
// cover the other's LDS latency and barrier waits):
//   * workgroup tile BM x BN = 256 x 256, 256 x 192 or 128 x 256 (chosen per shape: 128-row tiles when M is too
//     small to fill the chip with 256-row ones), or 128 x 128 for mid-size M x N with a bf16 output through the
//     wide epilogue (two workgroups per CU, or one on a 4-stage LDS ring when every tile has a CU and K >= 3072);
//     K advances 128 bytes per stage, so every row segment a stage loads is one whole 128-byte line (64-byte
//     segments measured at about 60% of the L2 -> CU rate).
//   * persistent workgroups, one per CU: workgroup b computes tiles b, b + G, b + 2G, ... (G = grid size), as one
//     pipeline over its (tile, k-tile) stages, so the next tile's first stage loads during the last stage of the
//     current one (launched one tile per workgroup, every CU stalled on its epilogue at the same time: about
//     10-15 us per wave of tiles).
//   * global -> LDS by LDS DMA (buffer_load_dwordx4 ... lds): no register staging and no LDS write instructions;
//     the LDS holds two stages (2 x (256 + BN) x 128 B <= 128 KB) and the loads of the next stage are issued at
//     the start of the current one. Rows past M/N and bytes past K read as zeros (buffer range check).
//   * BM/64 x 8/(BM/64) waves (4 x 2 or 2 x 4), each owning a 64 x BN/(8/(BM/64)) sub-tile = 2 x TN MFMA tiles of
//     32 x 32 (up to 128 int32 accumulators per lane). Per 32 k a wave reads 2 + TN fragments (ds_read_b128) for
//     2 x TN MFMAs.
//   * software pipeline: fragments are double-buffered in registers across k-steps and across stages; the DMA
//     loads of the next stage are spread between the MFMAs of one k-step; one barrier per stage.
//   * LDS rows are 128 B (8 chunks of 16 B); chunk c of row r is stored at c ^ ((r >> 1) & 7). gfx950 serves 16
//     lanes of a ds_read_b128 per cycle from 64 banks (256-byte period): a fragment read (16 consecutive rows,
//     one chunk) then hits 16 distinct 16-byte bank quads.
//   * blockIdx -> tile is XCD-aware: workgroups are dealt round-robin over the 8 XCDs, so each XCD gets a contiguous
//     range of tiles in a grouped (kGroupM tile-rows) order, and the tiles one XCD runs together share A/W panels
//     in its L2 (G is a multiple of 8, so a workgroup's later tiles stay on its XCD's range).
//   * epilogue: each wave stages its accumulators 16 rows at a time through a private LDS band and writes 4
//     columns per lane, a wave covering whole row segments; scales, bias and residual are applied in fp32 in the
//     oracle's order and rounded once to bf16.
// Measured ceiling on MI355X: int8 MFMAs on changing operands, fed by LDS fragment reads and no global traffic,
// sustain about 3.0-3.1 of the 5.0 POP/s peak (the clock drops to about 1.9-2.1 GHz under that load; with constant
// operands the same loop reaches 4.9 POP/s at 2.38 GHz).
// int32 accumulation is exact for K < 133,144 (|acc| <= 127^2 K < 2^31), so any correct GEMM is bit-exact.
#include <atomic>
#include <type_traits>

#include "od_common.h"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kThreads = 512;  // 8 waves
// wave grid of a workgroup with BM rows: BM / 64 x 8 / (BM / 64) waves, each owning 64 rows
template <int BM>
struct WaveGrid {
  static constexpr int kWM = BM / 64, kWN = 8 / kWM;
};
constexpr int kMaxBM = 256;
constexpr int BK = 128;      // bytes of K per stage
constexpr int kCpr = BK / 16;  // 16-byte chunks per row per stage
constexpr int kGroupM = 4;
constexpr int kScaleRows = 256;  // the WIDE variant's LDS scale slot: kScaleRows row scales, then 256 column scales
constexpr int kOOB = 0x7ffffff0;  // a buffer offset past any range: the load returns zeros
// The SwiGLU epilogue's LDS table of bf16(silu(g)) (od_silu_bf16) for 2^-8 <= |g| < 16: bf16 patterns
// kSiluLo .. kSiluHi - 1 of each sign, positive ones first (2 x 1536 entries, 6 KB)
constexpr uint32_t kSiluLo = 0x3b80u, kSiluHi = 0x4180u, kSiluHalf = kSiluHi - kSiluLo;

struct GemmArgs {
  const int8_t* a;
  const float* sa;
  const int8_t* w;
  const float* sw;
  const uint16_t* bias;
  const uint16_t* residual;
  uint16_t* out;
  int32_t* acc;
  int64_t lda, ldw, ldr, ldo, ldacc;
  int64_t M, N, K;
  int tiles_m, tiles_n;
  int kt_per;            // k-tiles per split (blockIdx.y = split); nk without split-K
  int64_t split_stride;  // int32 elements between the partial-sum planes of two splits (ACC_ONLY)
};

__device__ __forceinline__ float bfr(float v) { return od_bf16_to_f32(od_f32_to_bf16(v)); }

// byte offset of logical chunk c (0..7) of row r inside a slab
__device__ __forceinline__ int swz(int row, int chunk) { return row * BK + ((chunk ^ ((row >> 1) & 7)) << 4); }

__device__ __forceinline__ void tile_of(int bid, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int ntiles = tiles_m * tiles_n;
  const int xcd = bid & 7, local = bid >> 3;
  const int per = ntiles >> 3, rem = ntiles & 7;
  const int id = xcd < rem ? xcd * (per + 1) + local : rem * (per + 1) + (xcd - rem) * per + local;
  const int group = id / (kGroupM * tiles_n);
  const int first_m = group * kGroupM;
  const int gsz = min(tiles_m - first_m, kGroupM);
  const int in_group = id - group * kGroupM * tiles_n;
  tm = first_m + in_group % gsz;
  tn = in_group / gsz;
}

// Epilogue of one tile, per wave, in passes of 16 rows of the wave's kRowsW x kCols sub-tile (two per 32-row
// MFMA band):
//  1. In the MFMA result layout (lane l holds column l % 32 of each 32x32 tile and rows 8*(r/4) + 4*(l/32) + r%4),
//     t = (float(acc) * sa[m]) * sw[n] (the raw int32 with ACC_ONLY) goes to a private LDS band (16 x kCols 4-byte
//     words; the eight bands fill at most one stage buffer). A lane needs one sw per column tile and 16 sa per
//     32-row band, loaded up front.
//  2. Row-major: lane l takes the 4 columns 4 (l % kC4) .. +3 of rows l / kC4 + kRowsPass * it, so its bias
//     values are fixed for the tile; y = bf16((t + bias) + residual), the same fp32 operation order as the
//     unfused product, with one rounding. Rows go in groups of 4 whose residual loads issue together. The wide
//     variant (epilogue8: N % 8 == 0, 16-byte aligned rows) takes 8 columns per lane: 16-byte band reads, residual
//     loads and stores, 5% less time on the QKV and O shapes at M = 4096 (the stores dominate the epilogue).
// Only the GENERAL variant carries the scalar paths for unaligned rows and a ragged last column group.
template <int BM, int BN, bool ACC_ONLY, bool GENERAL, bool SWIGLU, int TM, int TN>
__device__ __forceinline__ void epilogue(const GemmArgs& p, const v16i (&acc)[TM][TN], int8_t* stage_buf, int tm,
                                         int tn, int wm, int wn, int wave, int lane) {
  constexpr int kWM = WaveGrid<BM>::kWM, kWN = WaveGrid<BM>::kWN;
  constexpr int kRowsW = BM / kWM;
  constexpr int kCols = BN / kWN;             // columns of the wave's sub-tile
  constexpr int kC4 = kCols / 4;              // 4-column chunks per row
  constexpr int kRowsPass = 64 / kC4;         // rows one pass of the wave covers
  constexpr int kHalf = 16;                   // rows per band
  constexpr int kPasses = (kHalf + kRowsPass - 1) / kRowsPass;
  static_assert(kPasses % 4 == 0, "row groups of 4");
  constexpr int kBand = kHalf * kCols * 4;    // bytes of one band
  static_assert(kWM * kWN * kBand <= (BM + BN) * BK, "epilogue bands do not fit in a stage buffer");
  uint32_t* band = reinterpret_cast<uint32_t*>(stage_buf + wave * kBand);
  const int64_t m_w = (int64_t)tm * BM + wm * kRowsW;
  const int64_t n_w = (int64_t)tn * BN + wn * kCols;
  const int col = lane & 31, h = lane >> 5;
  float swv[TN];
#pragma unroll
  for (int j = 0; j < TN; ++j) swv[j] = ACC_ONLY ? 0.0f : p.sw[min(n_w + j * 32 + col, p.N - 1)];
  // row pass: this lane's 4 columns and their bias
  const int c4 = lane % kC4, rr = lane / kC4;
  const int64_t n = n_w + 4 * c4;
  const bool lane_on = rr < kRowsPass && n < p.N;
  float bias4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (!ACC_ONLY && p.bias) {
    if constexpr (GENERAL) {
#pragma unroll
      for (int e = 0; e < 4; ++e) bias4[e] = od_bf16_to_f32(p.bias[min(n + e, p.N - 1)]);
    } else if (lane_on) {
      const uint2 b = *reinterpret_cast<const uint2*>(p.bias + n);
      bias4[0] = __uint_as_float(b.x << 16);
      bias4[1] = __uint_as_float(b.x & 0xffff0000u);
      bias4[2] = __uint_as_float(b.y << 16);
      bias4[3] = __uint_as_float(b.y & 0xffff0000u);
    }
  }
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int64_t m_band = m_w + i * 32;
    float sav[16];
#pragma unroll
    for (int r = 0; r < 16; ++r)
      sav[r] = ACC_ONLY ? 0.0f : p.sa[min(m_band + 8 * (r >> 2) + 4 * h + (r & 3), p.M - 1)];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      __builtin_amdgcn_sched_barrier(0);  // one band at a time (hoisting the next band's loads spills)
      // rows 16 q .. 16 q + 15 of the 32-row band: r = 8 q .. 8 q + 7
#pragma unroll
      for (int j = 0; j < TN; ++j) {
#pragma unroll
        for (int r = 8 * q; r < 8 * q + 8; ++r) {
          const int row = 8 * ((r >> 2) & 1) + 4 * h + (r & 3);
          uint32_t word;
          if constexpr (ACC_ONLY) {
            word = (uint32_t)acc[i][j][r];
          } else {
            float t = (float)acc[i][j][r] * sav[r];
            t = t * swv[j];
            word = __float_as_uint(t);
          }
          band[row * kCols + j * 32 + col] = word;
        }
      }
      if (!lane_on) continue;
      const int64_t m_half = m_band + 16 * q;
#pragma unroll 1
      for (int it0 = 0; it0 < kPasses; it0 += 4) {
        uint2 res[4];
        if (!ACC_ONLY && p.residual) {
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const uint16_t* rp = p.residual + min(m_half + kRowsPass * (it0 + u) + rr, p.M - 1) * p.ldr;
            if constexpr (GENERAL) {
              uint32_t e4[4];
#pragma unroll
              for (int e = 0; e < 4; ++e) e4[e] = rp[min(n + e, p.N - 1)];
              res[u] = make_uint2(e4[0] | (e4[1] << 16), e4[2] | (e4[3] << 16));
            } else {
              res[u] = *reinterpret_cast<const uint2*>(rp + n);
            }
          }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int row = kRowsPass * (it0 + u) + rr;
          const int64_t m = m_half + row;
          if (row >= kHalf || m >= p.M) continue;
          const uint4 v = *reinterpret_cast<const uint4*>(band + row * kCols + 4 * c4);
          if constexpr (ACC_ONLY) {
            int32_t* dst = p.acc + m * p.ldacc + n;
            if constexpr (GENERAL) {
              const uint32_t vv[4] = {v.x, v.y, v.z, v.w};
              for (int e = 0; e < 4 && n + e < p.N; ++e) dst[e] = (int32_t)vv[e];
            } else {
              *reinterpret_cast<uint4*>(dst) = v;
            }
          } else if constexpr (SWIGLU) {
            // columns n .. n+3 are (gate f, up f, gate f+1, up f+1) with f = n / 2: out[m, f] =
            // bf16(bf16(silu(g)) * u), g and u being the bf16 gate and up outputs (no bias, no residual)
            const float g0 = bfr(__uint_as_float(v.x)), u0 = bfr(__uint_as_float(v.y));
            const float g1 = bfr(__uint_as_float(v.z)), u1 = bfr(__uint_as_float(v.w));
            const uint32_t h0 = od_f32_to_bf16(od_silu_bf16(g0) * u0), h1 = od_f32_to_bf16(od_silu_bf16(g1) * u1);
            uint16_t* dst = p.out + m * p.ldo + n / 2;
            if constexpr (GENERAL) {
              if (n < p.N) dst[0] = (uint16_t)h0;
              if (n + 2 < p.N) dst[1] = (uint16_t)h1;
            } else {
              *reinterpret_cast<uint32_t*>(dst) = h0 | (h1 << 16);
            }
          } else {
            const uint32_t vv[4] = {v.x, v.y, v.z, v.w};
            const uint32_t rw[4] = {res[u].x << 16, res[u].x & 0xffff0000u, res[u].y << 16, res[u].y & 0xffff0000u};
            uint32_t o[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              float y = __uint_as_float(vv[e]);
              if (p.bias) y = y + bias4[e];
              if (p.residual) y = y + __uint_as_float(rw[e]);
              o[e] = od_f32_to_bf16(y);
            }
            uint16_t* dst = p.out + m * p.ldo + n;
            if constexpr (GENERAL) {
              for (int e = 0; e < 4 && n + e < p.N; ++e) dst[e] = (uint16_t)o[e];
            } else {
              *reinterpret_cast<uint2*>(dst) = make_uint2(o[0] | (o[1] << 16), o[2] | (o[3] << 16));
            }
          }
        }
      }
    }
  }
}

// The epilogue of the WIDE variant: N % 8 == 0, 16-byte aligned out / bias / residual rows (8-byte out rows for
// SwiGLU), 16-byte aligned scale vectors, row strides below 2^22 elements. Same arithmetic as `epilogue`, with fewer
// instructions and waits:
//  * the tile's row and column scales come from LDS (`sc`: kScaleRows row scales, then the column scales), where the
//    stage that loaded the tile's first operands put them, instead of global loads between the epilogue's stores;
//  * the row pass takes 8 columns per lane (16-byte band reads, residual loads and stores; 8-byte stores for
//    SwiGLU);
//  * output and residual go through buffer descriptors over the tile's valid rows with 32-bit offsets: rows past M
//    are dropped by the range check (stores) or read as zeros (loads), so there is no per-row bounds arithmetic;
//  * the residual of the next 16-row band-half is loaded before the current band-half's stores are issued, so that
//    waiting for it does not wait for them (vector-memory operations complete in issue order);
//  * SwiGLU: g and u are rounded to bf16 by one conversion, the fast SiLU values of a lane's four outputs are
//    checked together for the rare float64 recomputation, and each pair of products is rounded and packed by one
//    conversion.
template <int BM, int BN, bool SWIGLU, int TM, int TN>
__device__ __forceinline__ void epilogue8(const GemmArgs& p, const v16i (&acc)[TM][TN], int8_t* stage_buf,
                                          const float* sc, const uint16_t* stab, int tm, int tn, int wm, int wn,
                                          int wave, int lane) {
  constexpr int kWM = WaveGrid<BM>::kWM, kWN = WaveGrid<BM>::kWN;
  constexpr int kRowsW = BM / kWM;
  constexpr int kCols = BN / kWN;
  constexpr int kC8 = kCols / 8;
  constexpr int kRowsPass = 64 / kC8;
  constexpr int kHalf = 16;
  constexpr int kPasses = (kHalf + kRowsPass - 1) / kRowsPass;
  static_assert(kPasses <= 4, "one group of residual loads per band");
  constexpr int kBand = kHalf * kCols * 4;
  uint32_t* band = reinterpret_cast<uint32_t*>(stage_buf + wave * kBand);
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  const int rows_valid = (int)min((int64_t)BM, p.M - m0);
  const int col = lane & 31, h = lane >> 5;
  const float* ssa = sc + wm * kRowsW;
  const float* ssw = sc + kScaleRows + wn * kCols;
  float swv[TN];
#pragma unroll
  for (int j = 0; j < TN; ++j) swv[j] = ssw[j * 32 + col];
  const int c8 = lane % kC8, rr = lane / kC8;
  const int nl = wn * kCols + 8 * c8;  // the lane's first column inside the tile
  const bool lane_on = rr < kRowsPass && n0 + nl < p.N;
  const int ldo = (int)p.ldo, ldr = (int)p.ldr;
  const __amdgpu_buffer_rsrc_t rout = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.out + m0 * p.ldo + (SWIGLU ? n0 / 2 : n0)), (short)0, rows_valid * ldo * 2, 0x00020000);
  const int row0 = wm * kRowsW + rr;  // the lane's row in band-half 0, pass 0
  const int ovo = (row0 * ldo + (SWIGLU ? nl / 2 : nl)) * 2;
  float bias8[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  if (!SWIGLU && p.bias && lane_on) {
    const uint4 b = *reinterpret_cast<const uint4*>(p.bias + n0 + nl);
    const uint32_t bw[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      bias8[2 * e] = __uint_as_float(bw[e] << 16);
      bias8[2 * e + 1] = __uint_as_float(bw[e] & 0xffff0000u);
    }
  }
  const bool has_res = !SWIGLU && p.residual && lane_on;
  const __amdgpu_buffer_rsrc_t rres = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(has_res ? p.residual + m0 * p.ldr + n0 : p.residual), (short)0, has_res ? rows_valid * ldr * 2 : 0,
      0x00020000);
  const int rvo = (row0 * ldr + nl) * 2;
  // residual rows of band-half bq (rows 16 bq .. 16 bq + 15 of the wave's sub-tile)
  auto load_res = [&](int bq, uint4 (&r)[kPasses]) {
#pragma unroll
    for (int u = 0; u < kPasses; ++u)
      r[u] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                           rres, rvo, (16 * bq + kRowsPass * u) * ldr * 2, 0));
  };
  uint4 res[kPasses], resn[kPasses];
  if (has_res) load_res(0, res);
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    float sav[16];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float4 s4 = *reinterpret_cast<const float4*>(ssa + i * 32 + 8 * k + 4 * h);
      sav[4 * k] = s4.x;
      sav[4 * k + 1] = s4.y;
      sav[4 * k + 2] = s4.z;
      sav[4 * k + 3] = s4.w;
    }
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 0; j < TN; ++j) {
#pragma unroll
        for (int r = 8 * q; r < 8 * q + 8; ++r) {
          const int row = 8 * ((r >> 2) & 1) + 4 * h + (r & 3);
          float t = (float)acc[i][j][r] * sav[r];
          t = t * swv[j];
          band[row * kCols + j * 32 + col] = __float_as_uint(t);
        }
      }
      if (!lane_on) continue;
      const int bq = 2 * i + q;
      if (has_res && bq + 1 < 2 * TM) load_res(bq + 1, resn);
#pragma unroll
      for (int u = 0; u < kPasses; ++u) {
        const int row = kRowsPass * u + rr;
        if (kRowsPass * kPasses > kHalf && row >= kHalf) continue;
        const int soff = (16 * bq + kRowsPass * u) * ldo * 2;
        const uint4 va = *reinterpret_cast<const uint4*>(band + row * kCols + 8 * c8);
        const uint4 vb = *reinterpret_cast<const uint4*>(band + row * kCols + 8 * c8 + 4);
        const uint32_t vv[8] = {va.x, va.y, va.z, va.w, vb.x, vb.y, vb.z, vb.w};
        if constexpr (SWIGLU) {
          // columns 2e, 2e + 1 of the group are (gate, up) of output column nl / 2 + e
          // bf16(silu(g)) = od_silu_bf16(g) of the bf16 gate g: for 2^-125 <= |g| < 2^-8 it is bf16(g / 2) (checked
          // on every bf16 g), the bf16 pattern with the exponent one lower; for 2^-8 <= |g| < 16 the LDS table;
          // the function itself for the rest (zero, tiny and |g| >= 16 or NaN: rare)
          float g[4], uu[4], s[4];
          bool rare = false;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            g[e] = __uint_as_float(vv[2 * e]);
            uu[e] = __uint_as_float(vv[2 * e + 1]);
            od_bfr2(g[e], uu[e]);
            const uint32_t gb = __float_as_uint(g[e]) >> 16, a = gb & 0x7fffu;
            const uint32_t idx = min(max(a, kSiluLo), kSiluHi - 1u) - kSiluLo + (gb >> 15) * kSiluHalf;
            const uint32_t tv = stab[idx];
            s[e] = __uint_as_float((a < kSiluLo ? gb - 0x80u : tv) << 16);
            rare |= a >= kSiluHi || a < 0x0100u;
          }
          if (__builtin_expect(rare, 0)) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const uint32_t a = (__float_as_uint(g[e]) >> 16) & 0x7fffu;
              if (a >= kSiluHi || a < 0x0100u) s[e] = od_silu_bf16(g[e]);
            }
          }
          typedef unsigned v2u __attribute__((ext_vector_type(2)));
          const v2u w = {od_pack_bf16x2(s[0] * uu[0], s[1] * uu[1]), od_pack_bf16x2(s[2] * uu[2], s[3] * uu[3])};
          __builtin_amdgcn_raw_buffer_store_b64(w, rout, ovo, soff, 0);
        } else {
          const uint32_t rw4[4] = {res[u].x, res[u].y, res[u].z, res[u].w};
          float y[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            y[e] = __uint_as_float(vv[e]);
            if (p.bias) y[e] = y[e] + bias8[e];
            if (has_res) y[e] = y[e] + __uint_as_float(e & 1 ? (rw4[e >> 1] & 0xffff0000u) : (rw4[e >> 1] << 16));
          }
          typedef unsigned v4u __attribute__((ext_vector_type(4)));
          const v4u w = {od_pack_bf16x2(y[0], y[1]), od_pack_bf16x2(y[2], y[3]), od_pack_bf16x2(y[4], y[5]),
                         od_pack_bf16x2(y[6], y[7])};
          __builtin_amdgcn_raw_buffer_store_b128(w, rout, ovo, soff, 0);
        }
      }
      if (has_res) {
#pragma unroll
        for (int u = 0; u < kPasses; ++u) res[u] = resn[u];
      }
    }
  }
}

// One LDS-DMA load (buffer_load_dwordx4 ... lds): lane l copies the 16 bytes at byte vo + soff of buffer r to LDS
// byte lds_base + 16 l (lds_base is wave-uniform, passed in M0); bytes past the buffer's range arrive as zeros.
// Inline asm, so that the compiler does not track it: the kernel waits for it (vmcnt) and orders it with barriers
// itself, where the compiler would wait for it before every LDS read it cannot prove disjoint from the copy (every
// read of the other stage buffer). M0 is declared clobbered.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, int vo, int soff, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %3\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds" ::"v"(vo), "s"(r), "s"(soff),
               "s"(lds_base)
               : "memory", "m0");
}

// buffer descriptors of one tile's A panel (BM rows) and W panel (BN rows); a zero range reads zeros
struct Panels {
  __amdgpu_buffer_rsrc_t a, w;
};

template <int BM, int BN>
__device__ __forceinline__ Panels panels_of(const GemmArgs& p, int v, int ntiles) {
  if (v >= ntiles) {
    return {__builtin_amdgcn_make_buffer_rsrc((void*)p.a, (short)0, 0, 0x00020000),
            __builtin_amdgcn_make_buffer_rsrc((void*)p.w, (short)0, 0, 0x00020000)};
  }
  int tm, tn;
  tile_of(v, p.tiles_m, p.tiles_n, tm, tn);
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  const int64_t rows_a = min((int64_t)BM, p.M - m0), rows_w = min((int64_t)BN, p.N - n0);
  return {__builtin_amdgcn_make_buffer_rsrc((void*)(p.a + m0 * p.lda), (short)0,
                                            (int)((rows_a - 1) * p.lda + p.K), 0x00020000),
          __builtin_amdgcn_make_buffer_rsrc((void*)(p.w + n0 * p.ldw), (short)0,
                                            (int)((rows_w - 1) * p.ldw + p.K), 0x00020000)};
}

// NS: LDS stage buffers. 2: the pipeline below. 4 (128 x 128 tiles, one workgroup per CU): a ring with three
// stages of loads in flight, for tiles whose main loop would otherwise wait on a single stage's loads.
template <int BM, int BN, bool ACC_ONLY, bool GENERAL, bool SWIGLU, bool WIDE, int NS = 2>
__global__ __launch_bounds__(kThreads, BM == 128 && BN == 128 && NS == 2 ? 4 : 1) void w8a8_gemm_kernel(GemmArgs p) {
  constexpr int kWM = WaveGrid<BM>::kWM, kWN = WaveGrid<BM>::kWN;
  constexpr int kRowsW = BM / kWM, kColsW = BN / kWN;  // a wave's sub-tile: 64 x BN/kWN
  constexpr int TM = kRowsW / 32;    // 2
  constexpr int TN = kColsW / 32;    // 4 or 3 (BM = 256), 2 (BM = 128)
  static_assert(kColsW % 32 == 0, "a wave's columns are whole 32-column MFMA tiles");
  constexpr int kSlabA = BM * BK, kSlabB = BN * BK, kStage = kSlabA + kSlabB;
  constexpr int kOpsA = BM / 64, kOpsB = BN / 64;  // DMA loads per wave per stage (8 waves x 8 rows each)
  static_assert(NS == 2 || (NS == 4 && BM == 128 && BN == 128 && WIDE && !ACC_ONLY && !GENERAL), "stage ring");
  __shared__ __attribute__((aligned(16))) int8_t smem[NS * kStage];
  // WIDE: the row and column scales of a tile, NS slots by the tile's index among the workgroup's tiles (mod NS), each
  // loaded by the stage that loads the tile's first operands (one 1 KB LDS-DMA load each; rows / columns past M / N
  // read as zeros)
  constexpr int kSlot = 2 * kScaleRows;
  __shared__ __attribute__((aligned(16))) float sscale[WIDE ? NS * kSlot : 4];
  // the wide SwiGLU epilogue's silu table, filled here (its first stage's barrier orders the fill before any read)
  __shared__ uint16_t stab[SWIGLU && WIDE ? 2 * kSiluHalf : 2];
  if constexpr (SWIGLU && WIDE) {
    for (int i = threadIdx.x; i < (int)(2 * kSiluHalf); i += kThreads) {
      const uint32_t h = (uint32_t)i >= kSiluHalf;
      const uint32_t bits = (h << 15) | (kSiluLo + (uint32_t)i - h * kSiluHalf);
      stab[i] = od_f32_to_bf16(od_silu_bf16(__uint_as_float(bits << 16)));
    }
  }

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / kWN, wn = wave % kWN;
  const int K = (int)p.K;
  const int nk = (K + BK - 1) / BK;
  const int ntiles = p.tiles_m * p.tiles_n;
  // split-K: this workgroup sums k-tiles kb .. ke-1 (all of them without split) and, with ACC_ONLY, writes its
  // partial sums to plane blockIdx.y of p.acc
  const int kb = blockIdx.y * p.kt_per, ke = min(nk, kb + p.kt_per);
  if constexpr (ACC_ONLY) p.acc += blockIdx.y * p.split_stride;
  const int lda_step = (int)(p.lda * 64), ldw_step = (int)(p.ldw * 64);
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) int8_t*)(smem);
  auto dma_scales = [&](int v, int slot) {
    if constexpr (WIDE) {
      if (v >= ntiles || wave > 1) return;
      int tm, tn;
      tile_of(v, p.tiles_m, p.tiles_n, tm, tn);
      const uint32_t lds_sc = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) float*)(sscale + slot * kSlot);
      if (wave == 0) {
        const int64_t m0 = (int64_t)tm * BM;
        dma16(__builtin_amdgcn_make_buffer_rsrc((void*)(p.sa + m0), (short)0, (int)(min((int64_t)BM, p.M - m0) * 4),
                                                0x00020000),
              lane * 16, 0, lds_sc);
      } else {
        const int64_t n0 = (int64_t)tn * BN;
        dma16(__builtin_amdgcn_make_buffer_rsrc((void*)(p.sw + n0), (short)0, (int)(min((int64_t)BN, p.N - n0) * 4),
                                                0x00020000),
              lane * 16, 0, lds_sc + kScaleRows * 4);
      }
    }
  };

  // DMA load o of a stage: wave w moves slab rows 8 (w + 8 o') .. +7 (o' = o, or o - kOpsA for the W slab); lane
  // l takes row l / 8 of those and physical chunk l % 8 of the row, which holds logical chunk (l % 8) ^ ((row >> 1)
  // & 7): the LDS row is then already in the swizzled layout frags() reads. (row >> 1) & 7 depends only on the
  // wave's parity and l / 16, so each lane's vector offset is the same for every load; the load's rows and the
  // k-tile go in the scalar offset. In the GENERAL variant a chunk past K gets the vector offset kOOB - soffset:
  // the sum is kOOB, past the range (zeros).
  const int dc = (lane & 7) ^ ((4 * (wave & 1) + (lane >> 4)) & 7);
  const int dvo_a = (int)((8 * wave + (lane >> 3)) * p.lda) + dc * 16;
  const int dvo_w = (int)((8 * wave + (lane >> 3)) * p.ldw) + dc * 16;
  auto dma = [&](int buf, const Panels& pn, int kt, int o) {
    if (o < kOpsA) {
      const int soff = kt * BK + o * lda_step;
      int vo = dvo_a;
      if (GENERAL && kt * BK + dc * 16 >= K) vo = kOOB - soff;
      dma16(pn.a, vo, soff, lds0 + buf * kStage + wave * 1024 + o * 8192);
    } else {
      const int soff = kt * BK + (o - kOpsA) * ldw_step;
      int vo = dvo_w;
      if (GENERAL && kt * BK + dc * 16 >= K) vo = kOOB - soff;
      dma16(pn.w, vo, soff, lds0 + buf * kStage + kSlabA + wave * 1024 + (o - kOpsA) * 8192);
    }
  };
  // operand fragments of k-step s (32 of the stage's 128 k) of stage buffer buf
  auto frags = [&](int buf, int s, v4i (&fa)[TM], v4i (&fb)[TN]) {
    const int chunk = s * 2 + (lane >> 5);
    const int8_t* la = smem + buf * kStage;
    const int8_t* lb = la + kSlabA;
#pragma unroll
    for (int i = 0; i < TM; ++i) fa[i] = *reinterpret_cast<const v4i*>(la + swz(wm * kRowsW + i * 32 + (lane & 31), chunk));
#pragma unroll
    for (int j = 0; j < TN; ++j) fb[j] = *reinterpret_cast<const v4i*>(lb + swz(wn * kColsW + j * 32 + (lane & 31), chunk));
  };

  v16i acc[TM][TN];
  auto zero_acc = [&]() {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = v16i{0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
  };

  // The MFMAs of one k-step; `fill` issues the o-th of this k-step's kOps memory operations after MFMA
  // o * kMf / kOps (spreading them so that no wave stalls on a full queue while its MFMA pipe idles).
  constexpr int kMf = TM * TN;
  auto mma = [&](const v4i (&fa)[TM], const v4i (&fb)[TN], auto fill, auto OPS) {
    constexpr int kOps = decltype(OPS)::value;
#pragma unroll
    for (int x = 0; x < kMf; ++x) {
      acc[x / TN][x % TN] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[x / TN], fb[x % TN], acc[x / TN][x % TN], 0, 0, 0);
#pragma unroll
      for (int o = 0; o < kOps; ++o)
        if (o * kMf / (kOps > 0 ? kOps : 1) == x) fill(o);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  auto nofill = [](int) {};
  using Zero = std::integral_constant<int, 0>;

  // Pipeline over the sequence of (tile, k-tile) stages of this workgroup: tiles v = blockIdx.x + i * gridDim.x
  // (gridDim.x is a multiple of 8 or covers every tile, so all of a workgroup's tiles come from its XCD's range).
  // LDS buffer CUR holds the stage being computed; stage s:
  //   k-step 0: read k-step 1's fragments; MFMAs of k-step 0 interleaved with the DMA loads of the next stage of
  //             the sequence (k-tile kt + 1 of this tile, or k-tile 0 of the next tile) into buffer NXT, free since
  //             the barrier that ended the previous stage
  //   k-steps 1, 2: read the next k-step's fragments, MFMAs
  //   k-step 3: vmcnt + lgkmcnt wait and barrier (the next stage is in LDS for every wave, every wave is done
  //             reading CUR), read k-step 0 of the next stage, MFMAs of k-step 3
  // After a tile's last stage its accumulators go out through the epilogue, which stages them in buffer CUR of
  // that stage (read by no one any more) while NXT already holds the next tile's first stage. (The next tile's first
  // stage waits for the epilogue's stores: the compiler counts the epilogue's conditional loads as outstanding there
  // and waits for every memory operation.)
  if constexpr (NS > 2) {
    // The ring: stage j of the workgroup's sequence of (tile, k-tile) stages computes from buffer j % NS, and its
    // loads go out during stage j - (NS - 1), into the buffer stage j - NS read (free since the barrier that ended
    // that stage). A stage ends by waiting for the next stage's loads, leaving the NS - 2 later stages' loads in flight
    // (vector memory operations complete in issue order; a scale load or an epilogue's loads and stores issued after
    // them only make the wait stricter).
    v4i f0a[TM], f0b[TN], f1a[TM], f1b[TN];
    constexpr int kOps0 = kOpsA + kOpsB;
    static_assert(2 * kOps0 == 8, "the ring's wait count: two stages of loads in flight");
    int v = blockIdx.x;
    const int G = (int)gridDim.x;
    const int nks = ke - kb;  // stages per tile
    Panels cur = panels_of<BM, BN>(p, v, ntiles);
    Panels nxt = panels_of<BM, BN>(p, v + G, ntiles);
    // the panels of the tile d tiles after the current one
    auto src_of = [&](int d) { return d == 0 ? cur : d == 1 ? nxt : panels_of<BM, BN>(p, v + d * G, ntiles); };
    // stages 0 .. NS - 2 (stage j in buffer j), then wait for stage 0 only
    for (int q = 0; q < NS - 1; ++q) {
      const int d = q / nks, ktt = kb + q - d * nks;
      const Panels src = src_of(d);
#pragma unroll
      for (int o = 0; o < kOps0; ++o) dma(q, src, ktt, o);
      if (ktt == kb) dma_scales(v + d * G, d % NS);
    }
    asm volatile("s_waitcnt vmcnt(8)\n\ts_barrier" ::: "memory");
    frags(0, 0, f0a, f0b);
    zero_acc();
    int cb = 0;  // the current stage's buffer
    for (int i = 0; v < ntiles; v += G, ++i) {
      for (int kr = 0; kr < nks; ++kr) {
        const int tgt = kr + NS - 1;  // the stage whose loads go out now, counted from this tile's first
        const int d = tgt < nks ? 0 : tgt / nks;
        const int ktt = kb + tgt - d * nks;
        const int nb = cb == NS - 1 ? 0 : cb + 1, lb = cb == 0 ? NS - 1 : cb - 1;
        const Panels src = src_of(d);
        frags(cb, 1, f1a, f1b);
        __builtin_amdgcn_sched_barrier(0);
        auto fill0 = [&](int o) { dma(lb, src, ktt, o); };
        mma(f0a, f0b, fill0, std::integral_constant<int, kOps0>{});
        if (d > 0 && ktt == kb) dma_scales(v + d * G, (i + d) % NS);
        frags(cb, 2, f0a, f0b);
        __builtin_amdgcn_sched_barrier(0);
        mma(f1a, f1b, nofill, Zero{});
        frags(cb, 3, f1a, f1b);
        __builtin_amdgcn_sched_barrier(0);
        mma(f0a, f0b, nofill, Zero{});
        asm volatile("s_waitcnt vmcnt(8) lgkmcnt(0)\n\ts_barrier" ::: "memory");
        frags(nb, 0, f0a, f0b);
        __builtin_amdgcn_sched_barrier(0);
        mma(f1a, f1b, nofill, Zero{});
        cb = nb;
      }
      int tm, tn;
      tile_of(v, p.tiles_m, p.tiles_n, tm, tn);
      epilogue8<BM, BN, SWIGLU, TM, TN>(p, acc, smem + (cb == 0 ? NS - 1 : cb - 1) * kStage,
                                        sscale + (i % NS) * kSlot, stab, tm, tn, wm, wn, wave, lane);
      // A wait the compiler sees. It cannot relate the epilogue's loads' conditions to those of their uses and
      // would otherwise count them outstanding into the next tile's stages, waiting for every memory operation (the
      // ring's loads included) at the top of each stage. Here it costs one drain per tile.
      __builtin_amdgcn_s_waitcnt(0);
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      zero_acc();
      cur = nxt;
      nxt = panels_of<BM, BN>(p, v + 2 * G, ntiles);
    }
    // the loads of the stages past the last tile (zeros from empty ranges) land before the workgroup's LDS is freed
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    return;
  }
  v4i f0a[TM], f0b[TN], f1a[TM], f1b[TN];
  constexpr int kOps0 = kOpsA + kOpsB;
  int v = blockIdx.x;
  Panels cur = panels_of<BM, BN>(p, v, ntiles);
#pragma unroll
  for (int o = 0; o < kOps0; ++o) dma(0, cur, kb, o);
  dma_scales(v, 0);
  asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
  frags(0, 0, f0a, f0b);
  zero_acc();

  auto stage = [&](int CUR, const Panels& src, int kt_src, int scale_tile, int slot) {
    const int NXT = 1 - CUR;
    frags(CUR, 1, f1a, f1b);
    __builtin_amdgcn_sched_barrier(0);
    auto fill0 = [&](int o) { dma(NXT, src, kt_src, o); };
    mma(f0a, f0b, fill0, std::integral_constant<int, kOps0>{});
    if (scale_tile >= 0) dma_scales(scale_tile, slot);
    frags(CUR, 2, f0a, f0b);
    __builtin_amdgcn_sched_barrier(0);
    mma(f1a, f1b, nofill, Zero{});
    frags(CUR, 3, f1a, f1b);
    __builtin_amdgcn_sched_barrier(0);
    mma(f0a, f0b, nofill, Zero{});
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    frags(NXT, 0, f0a, f0b);
    __builtin_amdgcn_sched_barrier(0);
    mma(f1a, f1b, nofill, Zero{});
  };

  int buf = 0, parity = 0;
  // (the stage buffer is a run-time value: unrolling two stages with compile-time buffer indices lengthens the
  // live ranges)
  for (; v < ntiles; v += gridDim.x) {
    const Panels nxt = panels_of<BM, BN>(p, v + (int)gridDim.x, ntiles);
    for (int kt = kb; kt + 1 < ke; ++kt) {
      stage(buf, cur, kt + 1, -1, 0);
      buf ^= 1;
    }
    stage(buf, nxt, kb, v + (int)gridDim.x, parity ^ 1);
    buf ^= 1;
    int tm, tn;
    tile_of(v, p.tiles_m, p.tiles_n, tm, tn);
    if constexpr (WIDE)
      epilogue8<BM, BN, SWIGLU, TM, TN>(p, acc, smem + (buf ^ 1) * kStage, sscale + parity * kSlot, stab, tm, tn,
                                        wm, wn, wave, lane);
    else
      epilogue<BM, BN, ACC_ONLY, GENERAL, SWIGLU, TM, TN>(p, acc, smem + (buf ^ 1) * kStage, tm, tn, wm, wn, wave,
                                                          lane);
    // every wave is done with its band (in the buffer the next stage's DMA loads overwrite) before that stage
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    zero_acc();
    cur = nxt;
    parity ^= 1;
  }
}

// ------------------------------------------------------------------------------------------------ small M
// The small-M kernel (M up to a few hundred rows and few tiles: a single 256-row linear, the question and record
// passes): the 256-row tiles above leave most CUs idle there, and splitting K across workgroups costs int32 partial
// planes in memory (2 x splits x M x N x 4 bytes) and a second launch. Here one workgroup of 4 waves owns a
// 64 x BN tile and splits K inside itself: wave w sums the 128-byte k-chunks w, w + 4, w + 8, ... of the tile. Each
// wave has two LDS buffers of its own (a chunk's 64 A rows and BN W rows, 128 bytes each, in the swizzled layout of
// the 256-row kernel) and moves its next chunk in by LDS DMA (8 lanes per 128-byte line; rows past M / N and bytes
// past K read as zeros) while it computes the current one, so the waves never wait for each other until the end.
// The four partial tiles are then added through LDS (integer sums: exact, in any order) and the epilogue runs on
// the sum. (Tried: operands loaded straight into the MFMA registers, 32 rows per load instruction, 1.8x slower;
// three chunks in flight per wave staged through registers and copied to LDS, 1.3x slower.)
constexpr int kSmWaves = 4;
constexpr int kSmBM = 64;

template <int BN>
__device__ __forceinline__ void small_tile_of(int bid, int tiles_m, int tiles_n, int& tm, int& tn) {
  // XCD-aware: workgroup b runs on XCD b % 8; each XCD takes a contiguous range of tiles, M fastest, so the tiles
  // that read one W panel share an XCD's L2
  const int ntiles = tiles_m * tiles_n;
  const int xcd = bid & 7, local = bid >> 3;
  const int per = ntiles >> 3, rem = ntiles & 7;
  const int id = xcd < rem ? xcd * (per + 1) + local : rem * (per + 1) + (xcd - rem) * per + local;
  tm = id % tiles_m;
  tn = id / tiles_m;
}

template <int BN, bool SWIGLU>
__global__ __launch_bounds__(kSmWaves * 64, 1) void w8a8_gemm_small_kernel(GemmArgs p) {
  constexpr int TM = kSmBM / 32, TN = BN / 32;
  constexpr int kRows = kSmBM + BN;        // rows of one chunk: A rows, then W rows
  constexpr int kChunk = kRows * BK;       // bytes of one chunk buffer
  constexpr int kLoads = kRows / 8;        // LDS DMA loads of a chunk (8 rows of 128 bytes each)
  constexpr int kLoadsA = kSmBM / 8;
  static_assert(kLoads <= 63, "the vmcnt wait counts one chunk's loads");
  // [wave][buffer][chunk bytes]; after the main loop the first 64 x BN x 4 x 4 bytes hold the partial tiles
  __shared__ __attribute__((aligned(16))) int8_t smem[kSmWaves * 2 * kChunk];
  static_assert(kSmWaves * TM * TN * 4 * 64 * 16 <= kSmWaves * 2 * kChunk, "partial tiles fit the chunk buffers");
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int h = lane >> 5, c = lane & 31;
  int tm, tn;
  small_tile_of<BN>(blockIdx.x, p.tiles_m, p.tiles_n, tm, tn);
  const int64_t m0 = (int64_t)tm * kSmBM, n0 = (int64_t)tn * BN;
  const int rows_a = (int)min((int64_t)kSmBM, p.M - m0), rows_w = (int)min((int64_t)BN, p.N - n0);
  const int K = (int)p.K;
  const auto ra = __builtin_amdgcn_make_buffer_rsrc((void*)(p.a + m0 * p.lda), (short)0,
                                                    (int)((rows_a - 1) * p.lda + K), 0x00020000);
  const auto rw = __builtin_amdgcn_make_buffer_rsrc((void*)(p.w + n0 * p.ldw), (short)0,
                                                    (int)((rows_w - 1) * p.ldw + K), 0x00020000);
  // DMA load o moves chunk rows 8 o .. 8 o + 7: lane l takes row 8 o + l / 8 and physical 16-byte chunk l % 8 of it,
  // which holds logical chunk (l % 8) ^ ((row >> 1) & 7) = (l % 8) ^ ((4 (o & 1) + l / 16) & 7)
  const int dc0 = (lane & 7) ^ ((lane >> 4) & 7), dc1 = (lane & 7) ^ ((4 + (lane >> 4)) & 7);
  const int va0 = (int)((lane >> 3) * p.lda) + dc0 * 16, va1 = (int)((lane >> 3) * p.lda) + dc1 * 16;
  const int vw0 = (int)((lane >> 3) * p.ldw) + dc0 * 16, vw1 = (int)((lane >> 3) * p.ldw) + dc1 * 16;
  const uint32_t lds_w = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) int8_t*)(smem) + wave * 2 * kChunk;
  auto dma_chunk = [&](int b, int kc) {
    const int kb = __builtin_amdgcn_readfirstlane(kc * BK);  // wave-uniform (the scalar offset of the loads)
    b = __builtin_amdgcn_readfirstlane(b);
#pragma unroll
    for (int o = 0; o < kLoads; ++o) {
      const bool is_a = o < kLoadsA;
      const int oo = is_a ? o : o - kLoadsA;
      const int dc = (o & 1) ? dc1 : dc0;
      const int soff = kb + oo * 8 * (int)(is_a ? p.lda : p.ldw);
      int vo = is_a ? ((o & 1) ? va1 : va0) : ((o & 1) ? vw1 : vw0);
      if (kb + dc * 16 >= K) vo = kOOB - soff;  // a K tail, or a chunk past the last: zeros
      dma16(is_a ? ra : rw, vo, soff, lds_w + b * kChunk + o * 1024);
    }
  };
  v16i acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = v16i{0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
  const int nk = (K + BK - 1) / BK;
  int kc = wave, b = 0;
  dma_chunk(0, kc);
  while (kc < nk) {
    dma_chunk(b ^ 1, kc + kSmWaves);  // always issued (past the last chunk it reads zeros), so the count is fixed
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kLoads) : "memory");  // this chunk's loads are in LDS
    const int8_t* lb = smem + (wave * 2 + b) * kChunk;
#pragma unroll
    for (int s = 0; s < BK / 32; ++s) {
      const int chunk = s * 2 + h;
      v4i fa[TM], fb[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) fa[i] = *reinterpret_cast<const v4i*>(lb + swz(32 * i + c, chunk));
#pragma unroll
      for (int j = 0; j < TN; ++j) fb[j] = *reinterpret_cast<const v4i*>(lb + swz(kSmBM + 32 * j + c, chunk));
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
    }
    // every fragment read of this buffer is done before the next iteration's DMA overwrites it
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    b ^= 1;
    kc += kSmWaves;
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the last (unused) chunk's loads, before the LDS is reused
  __syncthreads();
  // the partial tiles in the MFMA result layout: [wave][tile][quad of registers][lane] as int4
  v4i* part = reinterpret_cast<v4i*>(smem);
  auto pidx = [](int w, int x, int r4, int l) { return ((w * TM * TN + x) * 4 + r4) * 64 + l; };
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4)
        part[pidx(wave, i * TN + j, r4, lane)] = v4i{acc[i][j][4 * r4], acc[i][j][4 * r4 + 1], acc[i][j][4 * r4 + 2],
                                                     acc[i][j][4 * r4 + 3]};
  __syncthreads();
  // thread (r4 = wave, lane) of tile x holds rows 32 i + 8 r4 + 4 h + 0..3 of column 32 j + c; the epilogue is the
  // fp32 arithmetic of the 256-row kernel in its order: t = (float(acc) sa[m]) sw[n], then + bias, + residual, one
  // bf16 rounding; SwiGLU pairs columns (gate 2f, up 2f + 1) across neighbouring lanes
#pragma unroll
  for (int x = 0; x < TM * TN; ++x) {
    const int i = x / TN, j = x % TN;
    v4i s4 = part[pidx(0, x, wave, lane)];
#pragma unroll
    for (int w = 1; w < kSmWaves; ++w) s4 = s4 + part[pidx(w, x, wave, lane)];
    const int64_t n = n0 + 32 * j + c;
    const bool n_ok = n < p.N;
    const float swn = n_ok ? p.sw[n] : 0.0f;
    const float bn = (!SWIGLU && n_ok && p.bias) ? od_bf16_to_f32(p.bias[n]) : 0.0f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int64_t m = m0 + 32 * i + 8 * wave + 4 * h + e;
      const bool m_ok = m < p.M;
      const float sam = m_ok ? p.sa[m] : 0.0f;
      const float t = ((float)s4[e] * sam) * swn;
      if constexpr (SWIGLU) {
        const float u = __shfl_xor(t, 1, 64);  // the up value of the pair, from lane c ^ 1
        if (m_ok && n_ok && (c & 1) == 0)
          p.out[m * p.ldo + n / 2] = (uint16_t)od_f32_to_bf16(od_silu_bf16(bfr(t)) * bfr(u));
      } else {
        if (m_ok && n_ok) {
          float y = t;
          if (p.bias) y = y + bn;
          if (p.residual) y = y + od_bf16_to_f32(p.residual[m * p.ldr + n]);
          p.out[m * p.ldo + n] = (uint16_t)od_f32_to_bf16(y);
        }
      }
    }
  }
}

}  // namespace

namespace {

// compute units of the current device, rounded down to a multiple of 8 (whole XCDs), cached per device
int cu_count() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 8) n = 256;
    n -= n % 8;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

struct Tiling {
  int bm, bn;
  int64_t tiles_m, tiles_n;
  double rel;  // time of one tile relative to a 256 x 256 one
};

// Tile shape: 256 x 256, 256 x 192 or 128 x 256, whichever takes the least time by the number of tiles each
// persistent workgroup runs times the time of one tile. Measured per-tile times relative to 256 x 256 (K = 4096 and
// 12288, N = 4096 to 24576, M = 512 to 16384): 0.79-0.88 for 256 x 192, 0.61-0.69 for 128 x 256 (a smaller tile
// reads more LDS fragments per MFMA); 0.84 and 0.68 pick the fastest of the three at every measured shape.
// With `small` (a bf16 output through the wide epilogue, no accumulator output) 128 x 128 is a fourth candidate,
// for mid-size M x N that leave most CUs without a larger tile. Its workgroup needs 68 KB of LDS and at most 128
// VGPRs per lane, so two run on a CU (the persistent grid is twice the CUs): measured on the sweep's and the 9B
// shapes at M = 512 to 2048, one such tile per CU takes 0.53 of a 256 x 256 tile's time (its main loop waits on
// its one stage of loads in flight) and two together 0.60. It is a candidate only up to two tiles per CU: with more,
// each pair of tiles measured 0.71-0.73 (M = 6144: O and down projections 2-8% slower than on 256 x 256 tiles).
constexpr double kRel128x128 = 0.53, kRel128x128Pair = 0.60;
Tiling tiling_of(int64_t M, int64_t N, bool small) {
  const struct { int bm, bn; double cost; } cand[4] = {
      {256, 256, 1.0}, {256, 192, 0.84}, {128, 256, 0.68}, {128, 128, kRel128x128}};
  const int64_t cus = cu_count();
  Tiling best{256, 256, 0, 0, 1.0};
  double best_cost = 0.0;
  for (const auto& c : cand) {
    const bool t128 = c.bn == 128;
    if (t128 && !small) continue;
    const int64_t tm = (M + c.bm - 1) / c.bm, tn = (N + c.bn - 1) / c.bn;
    if (t128 && tm * tn > 2 * cus) continue;
    const double cost = t128 ? (tm * tn <= cus ? kRel128x128 : kRel128x128Pair)
                             : (double)((tm * tn + cus - 1) / cus) * c.cost;
    if (best.tiles_m == 0 || cost < best_cost) {
      best = {c.bm, c.bn, tm, tn, c.cost};
      best_cost = cost;
    }
  }
  return best;
}

// Split-K for shapes with too few tiles to fill the chip (small M): `splits` workgroups per tile each sum
// kt_per k-tiles into their own int32 plane of a workspace [splits][M][ldws], and splitk_finalize_kernel adds the
// planes (integer sums: exact) and applies the same epilogue. Chosen when a simple cost model (about 1.2 us per
// k-tile stage of a 256 x 256 tile, scaled by the tile's relative time; the partial planes written and read once
// at ~3 TB/s; ~2.5 us for the extra launch) predicts at least 15% less time than one pass.
struct SplitPlan {
  int splits, kt_per;
  int64_t ldws, ws_ints;
};

// Shapes for the small-M kernel (w8a8_gemm_small_kernel): up to 512 rows and at most two of its 64 x 64 tiles per
// CU (it runs one workgroup per CU and pays each tile's first-chunk latency in full; M = 512 x N = 6144 is faster on
// the 128 x 256 tiles with split-K). Its tile width: 64 columns when that gives every CU a tile, else 32 (twice the
// tiles, each reading A again).
constexpr int64_t kSmallMaxM = 512;
bool small_m(int64_t M, int64_t N) {
  return M <= kSmallMaxM && ((M + kSmBM - 1) / kSmBM) * ((N + 63) / 64) <= 2 * (int64_t)cu_count();
}
int small_bn(int64_t M, int64_t N) {
  const int64_t tiles64 = ((M + kSmBM - 1) / kSmBM) * ((N + 63) / 64);
  return tiles64 >= cu_count() ? 64 : 32;
}

SplitPlan split_plan(int64_t M, int64_t N, int64_t K) {
  const int nk = (int)((K + BK - 1) / BK);
  const SplitPlan none{1, nk, 0, 0};
  if (small_m(M, N)) return none;  // the small-M kernel splits K inside its workgroups
  const Tiling t = tiling_of(M, N, false);
  const int64_t ntiles = t.tiles_m * t.tiles_n, cus = cu_count();
  if (ntiles * 2 > cus || nk < 4) return none;
  const double t_stage = 1.2 * t.rel;  // us per k-tile stage of one tile
  const double base = nk * t_stage;
  double best = 0.85 * base;
  SplitPlan bp = none;
  for (int s = 2; s <= 16 && ntiles * s <= cus; ++s) {
    const int per = (nk + s - 1) / s;
    const int used = (nk + per - 1) / per;  // splits that get k-tiles
    if (used != s) continue;
    const double est = per * t_stage + 2.0 * s * (double)M * (double)N * 4.0 / 3.0e6 + 2.5;
    if (est < best) {
      best = est;
      const int64_t ldws = (N + 3) / 4 * 4;
      bp = {s, per, ldws, (int64_t)s * M * ldws};
    }
  }
  return bp;
}

// out from the split-K partial planes: one thread per 4 columns of a row; the sum of the planes is the exact int32
// accumulator, then the epilogue's fp32 operations in its order (SwiGLU pairs columns as the GEMM's epilogue does).
template <bool SWIGLU>
__global__ __launch_bounds__(256) void splitk_finalize_kernel(GemmArgs p, const int32_t* ws, int splits,
                                                              int64_t stride) {
  const int64_t n4 = (p.N + 3) / 4;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= p.M * n4) return;
  const int64_t m = idx / n4, n = (idx - m * n4) * 4;
  const int32_t* src = ws + m * p.ldacc + n;
  int32_t a4[4] = {0, 0, 0, 0};
  if (n + 4 <= p.N) {
    for (int sp = 0; sp < splits; ++sp) {
      const int4 v = *reinterpret_cast<const int4*>(src + sp * stride);
      a4[0] += v.x;
      a4[1] += v.y;
      a4[2] += v.z;
      a4[3] += v.w;
    }
  } else {
    for (int sp = 0; sp < splits; ++sp)
      for (int e = 0; n + e < p.N; ++e) a4[e] += src[sp * stride + e];
  }
  const float sam = p.sa[m];
  float t[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float x = (float)a4[e] * sam;
    t[e] = x * p.sw[min(n + e, p.N - 1)];
  }
  if constexpr (SWIGLU) {
    // columns n .. n+3 are (gate f, up f, gate f+1, up f+1) with f = n / 2 (N even)
    uint16_t* dst = p.out + m * p.ldo + n / 2;
    dst[0] = (uint16_t)od_f32_to_bf16(od_silu_bf16(bfr(t[0])) * bfr(t[1]));
    if (n + 2 < p.N) dst[1] = (uint16_t)od_f32_to_bf16(od_silu_bf16(bfr(t[2])) * bfr(t[3]));
  } else {
    for (int e = 0; e < 4 && n + e < p.N; ++e) {
      float y = t[e];
      if (p.bias) y = y + od_bf16_to_f32(p.bias[n + e]);
      if (p.residual) y = y + od_bf16_to_f32(p.residual[m * p.ldr + n + e]);
      p.out[m * p.ldo + n + e] = (uint16_t)od_f32_to_bf16(y);
    }
  }
}

int gemm_launch(const GemmArgs& p0, bool swiglu, hipStream_t st, const SplitPlan* sp = nullptr,
                int32_t* ws = nullptr) {
  GemmArgs p = p0;
  const int64_t M = p.M, N = p.N, K = p.K;
  if (!p.acc && small_m(M, N)) {
    const int bn = small_bn(M, N);
    const int64_t tiles_m = (M + kSmBM - 1) / kSmBM, tiles_n = (N + bn - 1) / bn;
    if (tiles_m * tiles_n > 0x7fffffff) return OD_ERR_SHAPE;
    p.tiles_m = (int)tiles_m;
    p.tiles_n = (int)tiles_n;
    const dim3 grid((unsigned)(tiles_m * tiles_n)), block(kSmWaves * 64);
    if (bn == 64) {
      swiglu ? w8a8_gemm_small_kernel<64, true><<<grid, block, 0, st>>>(p)
             : w8a8_gemm_small_kernel<64, false><<<grid, block, 0, st>>>(p);
    } else {
      swiglu ? w8a8_gemm_small_kernel<32, true><<<grid, block, 0, st>>>(p)
             : w8a8_gemm_small_kernel<32, false><<<grid, block, 0, st>>>(p);
    }
    return od_launch_status();
  }
  // The fast variant needs whole k-tiles and 4-column output groups that are 8-byte (bf16) / 16-byte (int32)
  // aligned (with SwiGLU, 2-column output groups 4-byte aligned); anything else takes the GENERAL variant. The wide
  // variant (the epilogue's row pass on 8-column groups: 16-byte loads and stores) needs N % 8 == 0 and 16-byte
  // aligned bf16 rows (8-byte with SwiGLU).
  auto al = [](const void* q, unsigned a) { return (((uintptr_t)q) & (a - 1)) == 0; };
  const bool fast_k = K % BK == 0 && N % 4 == 0;
  const bool fast_out = fast_k && (swiglu ? (p.ldo % 2 == 0 && al(p.out, 4))
                                          : (p.ldo % 4 == 0 && al(p.out, 8) && al(p.bias, 8) && p.ldr % 4 == 0 &&
                                             al(p.residual, 8)));
  const bool wide_out = fast_out && N % 8 == 0 && al(p.sa, 16) && al(p.sw, 16) && p.ldo < (1 << 22) &&
                        (swiglu ? (p.ldo % 4 == 0 && al(p.out, 8))
                                : (p.ldo % 8 == 0 && al(p.out, 16) && al(p.bias, 16) && p.ldr % 8 == 0 &&
                                   p.ldr < (1 << 22) && al(p.residual, 16)));
  const bool split = sp && sp->splits > 1;
  // 128 x 128 tiles only for a bf16 output through the wide epilogue (one launch, no accumulator output)
  const Tiling t = tiling_of(M, N, wide_out && !split && !p.acc);
  const int64_t tiles_m = t.tiles_m, tiles_n = t.tiles_n;
  if (tiles_m * tiles_n > 0x7fffffff) return OD_ERR_SHAPE;
  p.tiles_m = (int)tiles_m;
  p.tiles_n = (int)tiles_n;
  p.kt_per = (int)((K + BK - 1) / BK);
  p.split_stride = 0;
  // persistent workgroups: one per CU (the kernel's LDS admits one; two of the 128 x 128 tile's), each looping over
  // tiles bid + i * grid
  const int64_t ntiles = tiles_m * tiles_n;
  const int64_t gmax = (t.bm == 128 && t.bn == 128 ? 2 : 1) * cu_count();
  dim3 grid((unsigned)(ntiles <= gmax ? ntiles : gmax)), block(kThreads);
  enum { kFast, kGeneral, kWide };
  auto launch = [&](auto BMc, auto BNc, auto ACCc, auto GENc, auto SWc, auto WIc) {
    w8a8_gemm_kernel<decltype(BMc)::value, decltype(BNc)::value, decltype(ACCc)::value, decltype(GENc)::value,
                     decltype(SWc)::value, decltype(WIc)::value><<<grid, block, 0, st>>>(p);
  };
  auto launch1 = [&](auto BMc, auto BNc, auto ACCc, auto SWc, int variant) {
    using F = std::false_type;
    using T = std::true_type;
    if (variant == kGeneral) {
      launch(BMc, BNc, ACCc, T{}, SWc, F{});
    } else if constexpr (!decltype(ACCc)::value) {
      if (variant == kWide) launch(BMc, BNc, ACCc, F{}, SWc, T{});
      else launch(BMc, BNc, ACCc, F{}, SWc, F{});
    } else {
      launch(BMc, BNc, ACCc, F{}, SWc, F{});
    }
  };
  auto launch2 = [&](auto ACCc, auto SWc, int variant) {
    using I = std::integral_constant<int, 256>;
    using H = std::integral_constant<int, 128>;
    if (t.bm == 128 && t.bn == 128) {
      // chosen only for the wide variant without accumulators (the 4-column epilogue needs 64-column sub-tiles);
      // at most one tile per CU and K >= 3072: one workgroup per CU on the 4-stage ring (M = N = 2048, K = 6144: 41.7
      // -> 33.3 us; at K = 2048 it measured 3% slower, its three stages of prologue loads a larger share of the tile),
      // else two workgroups per CU on 2 stages each
      if constexpr (!decltype(ACCc)::value) {
        if (variant == kWide) {
          if (ntiles <= cu_count() && p.kt_per >= 24)
            w8a8_gemm_kernel<128, 128, false, false, decltype(SWc)::value, true, 4><<<grid, block, 0, st>>>(p);
          else
            launch(H{}, H{}, ACCc, std::false_type{}, SWc, std::true_type{});
        }
      }
    } else if (t.bm == 128) {
      launch1(H{}, I{}, ACCc, SWc, variant);
    } else if (t.bn == 192) {
      launch1(I{}, std::integral_constant<int, 192>{}, ACCc, SWc, variant);
    } else {
      launch1(I{}, I{}, ACCc, SWc, variant);
    }
  };
  if (split) {
    // partial planes into the workspace, then the finalize pass writes out
    GemmArgs q = p;
    p.out = nullptr;
    p.acc = ws;
    p.ldacc = sp->ldws;
    p.kt_per = sp->kt_per;
    p.split_stride = M * sp->ldws;
    grid.y = (unsigned)sp->splits;
    launch2(std::true_type{}, std::false_type{}, fast_k && al(ws, 16) ? kFast : kGeneral);
    const int rc = od_launch_status();
    if (rc != OD_OK) return rc;
    q.ldacc = sp->ldws;
    const int64_t threads = M * ((N + 3) / 4);
    const dim3 fgrid((unsigned)((threads + 255) / 256));
    if (swiglu) {
      splitk_finalize_kernel<true><<<fgrid, 256, 0, st>>>(q, ws, sp->splits, M * sp->ldws);
    } else {
      splitk_finalize_kernel<false><<<fgrid, 256, 0, st>>>(q, ws, sp->splits, M * sp->ldws);
    }
    return od_launch_status();
  }
  const int out_variant = wide_out ? kWide : (fast_out ? kFast : kGeneral);
  const bool fast_acc = fast_k && p.ldacc % 4 == 0 && al(p.acc, 16);
  if (p.acc) {
    launch2(std::true_type{}, std::false_type{}, fast_acc ? kFast : kGeneral);
    const int rc = od_launch_status();
    if (rc != OD_OK) return rc;
  }
  if (p.out) {
    if (swiglu) {
      launch2(std::false_type{}, std::true_type{}, out_variant);
    } else {
      launch2(std::false_type{}, std::false_type{}, out_variant);
    }
  }
  return od_launch_status();
}

int gemm_check(const int8_t* a, int64_t lda, const int8_t* w, int64_t ldw, int64_t K) {
  if (K % 16 || lda % 16 || ldw % 16 || !od_aligned16(a) || !od_aligned16(w)) return OD_ERR_ALIGN;
  if (K >= 133144) return OD_ERR_UNSUPPORTED;  // int32 accumulators could overflow
  // buffer offsets are 32-bit: one tile's A panel (256 rows) and W panel must stay below 2 GiB
  if ((int64_t)kMaxBM * lda >= (1ll << 31) || (int64_t)256 * ldw >= (1ll << 31)) return OD_ERR_UNSUPPORTED;
  return OD_OK;
}

}  // namespace

extern "C" int od_w8a8_gemm(const int8_t* a, int64_t lda, const float* sa, const int8_t* w, int64_t ldw,
                            const float* sw, const uint16_t* bias, const uint16_t* residual, int64_t ldr,
                            uint16_t* out, int64_t ldo, int32_t* acc, int64_t ldacc, int64_t M, int64_t N, int64_t K,
                            od_stream_t stream) {
  if (M < 0 || N < 0 || K < 1) return OD_ERR_SHAPE;
  if (M == 0 || N == 0) return OD_OK;
  if (!a || !w || (!out && !acc)) return OD_ERR_NULL;
  if (out && (!sa || !sw)) return OD_ERR_NULL;
  if (lda < K || ldw < K || (out && ldo < N) || (acc && ldacc < N) || (residual && ldr < N)) return OD_ERR_SHAPE;
  const int rc = gemm_check(a, lda, w, ldw, K);
  if (rc != OD_OK) return rc;
  GemmArgs p{a, sa, w, sw, bias, residual, out, acc, lda, ldw, ldr, ldo, ldacc, M, N, K, 0, 0, 0, 0};
  return gemm_launch(p, false, (hipStream_t)stream);
}

extern "C" int od_w8a8_gemm_swiglu(const int8_t* a, int64_t lda, const float* sa, const int8_t* w, int64_t ldw,
                                   const float* sw, uint16_t* out, int64_t ldo, int64_t M, int64_t N, int64_t K,
                                   od_stream_t stream) {
  if (M < 0 || N < 0 || K < 1 || N % 2) return OD_ERR_SHAPE;
  if (M == 0 || N == 0) return OD_OK;
  if (!a || !w || !out || !sa || !sw) return OD_ERR_NULL;
  if (lda < K || ldw < K || ldo < N / 2) return OD_ERR_SHAPE;
  const int rc = gemm_check(a, lda, w, ldw, K);
  if (rc != OD_OK) return rc;
  GemmArgs p{a, sa, w, sw, nullptr, nullptr, out, nullptr, lda, ldw, 0, ldo, 0, M, N, K, 0, 0, 0, 0};
  return gemm_launch(p, true, (hipStream_t)stream);
}

extern "C" int od_w8a8_gemm_ws_size(int64_t M, int64_t N, int64_t K, int64_t* ws_ints) {
  if (!ws_ints) return OD_ERR_NULL;
  if (M < 0 || N < 0 || K < 1) return OD_ERR_SHAPE;
  *ws_ints = (M == 0 || N == 0) ? 0 : split_plan(M, N, K).ws_ints;
  return OD_OK;
}

extern "C" int od_w8a8_gemm_ws(const int8_t* a, int64_t lda, const float* sa, const int8_t* w, int64_t ldw,
                               const float* sw, const uint16_t* bias, const uint16_t* residual, int64_t ldr,
                               uint16_t* out, int64_t ldo, int64_t M, int64_t N, int64_t K, int swiglu, int32_t* ws,
                               int64_t ws_ints, od_stream_t stream) {
  if (M < 0 || N < 0 || K < 1 || ws_ints < 0 || (swiglu && N % 2)) return OD_ERR_SHAPE;
  if (M == 0 || N == 0) return OD_OK;
  if (!a || !w || !out || !sa || !sw) return OD_ERR_NULL;
  if (swiglu && (bias || residual)) return OD_ERR_UNSUPPORTED;
  if (lda < K || ldw < K || ldo < (swiglu ? N / 2 : N) || (residual && ldr < N)) return OD_ERR_SHAPE;
  const int rc = gemm_check(a, lda, w, ldw, K);
  if (rc != OD_OK) return rc;
  GemmArgs p{a, sa, w, sw, bias, residual, out, nullptr, lda, ldw, ldr, ldo, 0, M, N, K, 0, 0, 0, 0};
  const SplitPlan sp = split_plan(M, N, K);
  const bool split = sp.splits > 1 && ws && ws_ints >= sp.ws_ints && od_aligned16(ws);
  return gemm_launch(p, swiglu != 0, (hipStream_t)stream, split ? &sp : nullptr, split ? ws : nullptr);
}
