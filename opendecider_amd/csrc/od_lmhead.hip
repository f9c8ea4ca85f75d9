// LM-head token log-prob over an int8 vocabulary table, for gfx950 (src/opendecider/backbone.py:164-178 over the
// Int8Embedding / Int8Linear rows of src/opendecider/quant.py:122-132,183-203):
//
//   out[m] = sum_k float(h[m,k]) * float(q[t,k] * s[t])  -  log sum_v exp( bf16( bf16(h[m]) . bf16(q[v] * s[v]) ) )
//
// with t = tok[m], the table rows dequantized in bf16 (dequant_rows: the product q * s rounded to bf16), the logits
// the bf16 output of a bf16 matmul (fp32 accumulation, one rounding), the target term in fp32. Two kernels:
//   * lm_logits_kernel: a 256 (rows) x 256 (vocabulary) tile of the logits on V_MFMA_F32_32X32X16_BF16. The table's
//     int8 rows are dequantized on their way from registers into LDS (xor 0x80, v_cvt_f32_ubyte, one fma that gives
//     q * s exactly, v_cvt_pk_bf16_f32), so the MFMAs see exactly the reference's bf16 rows. The logits are rounded
//     to bf16 and reduced per row to (max, sum exp(l - max)) over each wave's 128 columns; nothing of the
//     rows x vocabulary matrix is stored.
//   * lm_combine_kernel: one wave per row merges the partials into the log-sum-exp and computes the target term.
// Tiling and pipeline are those of the W8A8 GEMM (od_gemm.hip): 8 waves (4 x 2, 64 x 128 each, two per SIMD), a
// stage of 128 bytes of every bf16 row (64 k) double-buffered in LDS (2 x 64 KB) with the next stage in registers,
// 16-byte chunks swizzled by (row >> 1) & 7, and an XCD-aware tile order in which the row tiles of one vocabulary
// tile run together on one XCD (they share its table panel in L2).
#include <type_traits>

#include "od_common.h"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kWM = 4, kWN = 2;
constexpr int kThreads = 64 * kWM * kWN;  // 512
constexpr int BM = 256, BN = 256;
constexpr int kRowBytes = 128;            // bytes of a bf16 row per stage (64 k)
constexpr int BK = kRowBytes / 2;         // k per stage
constexpr int kCpr = kRowBytes / 16;      // 16-byte chunks per LDS row
constexpr int kSlab = BM * kRowBytes;     // 32 KB (BM == BN)
constexpr int kStage = 2 * kSlab;
constexpr int kRowsW = BM / kWM, kColsW = BN / kWN;  // 64 x 128
constexpr int TM = kRowsW / 32, TN = kColsW / 32;    // 2 x 4 MFMA tiles
constexpr int kLoadsA = BM * kCpr / kThreads;        // 4 16-byte loads of the h slab per thread
constexpr int kLoadsB = BN * (kRowBytes / 2) / 16 / kThreads;  // 2 16-byte loads of int8 table rows per thread
constexpr float kLog2e = 1.4426950408889634f;

struct LmArgs {
  const uint16_t* h;      // bf16 [M, ldh]
  const int8_t* w;        // int8 [V, ldw] (Q4: the packed nibbles, uint8 [V, ldw >= K / 2])
  const uint16_t* scale;  // bf16 [V] (Q4: fp16 block scales [V, ldd >= K / 32])
  float* part;            // [M, n_parts, 2]: (max, sum exp(l - max)) of each wave's 128 columns
  int64_t ldh, ldw, ldd, M, V, K;
  int tiles_m, tiles_n, n_parts;
};
constexpr int kLoadsBQ4 = 1;  // Q4: one 16-byte load (a 32-value block) of table rows per thread

__device__ __forceinline__ int swz(int row, int chunk) { return row * kRowBytes + ((chunk ^ ((row >> 1) & 7)) << 4); }

__device__ __forceinline__ void barrier_lds() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// 16 int8 table values of one row -> 16 bf16 bf16(q * s), as two 16-byte chunks. With u = q + 128 (xor 0x80 on the
// byte) converted exactly by v_cvt_f32_ubyte, fma(u, s, -128 s) is q * s exactly (at most 15 significant bits),
// then rounded to nearest even by v_cvt_pk_bf16_f32: the reference's bf16 product.
__device__ __forceinline__ void dequant16(v4i raw, float s, v4i& lo, v4i& hi) {
  const float nb = -128.0f * s;
  uint32_t out[8];
#pragma unroll
  for (int wd = 0; wd < 4; ++wd) {
    const uint32_t u = (uint32_t)raw[wd] ^ 0x80808080u;
    float v0 = fmaf((float)(u & 0xffu), s, nb), v1 = fmaf((float)((u >> 8) & 0xffu), s, nb);
    float v2 = fmaf((float)((u >> 16) & 0xffu), s, nb), v3 = fmaf((float)(u >> 24), s, nb);
    out[2 * wd] = od_bfr2(v0, v1);
    out[2 * wd + 1] = od_bfr2(v2, v3);
  }
  lo = v4i{(int)out[0], (int)out[1], (int)out[2], (int)out[3]};
  hi = v4i{(int)out[4], (int)out[5], (int)out[6], (int)out[7]};
}

__device__ __forceinline__ float fp16_bits_to_f32(uint16_t b) { return (float)__builtin_bit_cast(_Float16, b); }

// One Q4_0 block (16 bytes: positions 0-15 in the low nibbles, 16-31 in the high ones) -> 32 bf16
// bf16((n - 8) * d), d the block scale already rounded to bf16 (the reference's d.to(bfloat16)): fma(n, d, -8 d) is
// (n - 8) d exactly (at most 12 significant bits), then one rounding to nearest even. Four 16-byte chunks: positions
// 0-7, 8-15, 16-23, 24-31.
__device__ __forceinline__ void dequant_q4(v4i raw, float d, v4i (&c)[4]) {
  const float nb = -8.0f * d;
  uint32_t out[16];
#pragma unroll
  for (int wd = 0; wd < 4; ++wd) {
    const uint32_t u = (uint32_t)raw[wd];
#pragma unroll
    for (int hi = 0; hi < 2; ++hi) {
      const uint32_t n4 = (hi ? u >> 4 : u) & 0x0f0f0f0fu;
      float v0 = fmaf((float)(n4 & 0xffu), d, nb), v1 = fmaf((float)((n4 >> 8) & 0xffu), d, nb);
      float v2 = fmaf((float)((n4 >> 16) & 0xffu), d, nb), v3 = fmaf((float)(n4 >> 24), d, nb);
      // positions 16 hi + 4 wd .. +3 -> words (16 hi + 4 wd) / 2 .. +1 of the 16-word block
      out[8 * hi + 2 * wd] = od_bfr2(v0, v1);
      out[8 * hi + 2 * wd + 1] = od_bfr2(v2, v3);
    }
  }
#pragma unroll
  for (int q = 0; q < 4; ++q)
    c[q] = v4i{(int)out[4 * q], (int)out[4 * q + 1], (int)out[4 * q + 2], (int)out[4 * q + 3]};
}

template <bool Q4>
__global__ __launch_bounds__(kThreads, 1) void lm_logits_kernel(LmArgs p) {
  __shared__ __attribute__((aligned(16))) int8_t smem[2 * kStage];
  // tile order: flat ids are dealt round-robin over the 8 XCDs; id = the XCD's contiguous range; row tiles fastest
  const int ntiles = p.tiles_m * p.tiles_n;
  const int f = blockIdx.x, xcd = f & 7, local = f >> 3, per = ntiles >> 3, rem = ntiles & 7;
  const int id = xcd < rem ? xcd * (per + 1) + local : rem * (per + 1) + (xcd - rem) * per + local;
  const int tm = id % p.tiles_m, tn = id / p.tiles_m;
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / kWN, wn = wave % kWN;

  // buffer descriptors over the tile's panels: rows past M / V read as zeros
  const int64_t rows_a = min((int64_t)BM, p.M - m0), rows_b = min((int64_t)BN, p.V - n0);
  const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.h + m0 * p.ldh), (short)0, (int)(((rows_a - 1) * p.ldh + p.K) * 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.w + n0 * p.ldw), (short)0, (int)((rows_b - 1) * p.ldw + (Q4 ? p.K / 2 : p.K)), 0x00020000);
  // h slab: load i covers row i * 64 + tid / 8, chunk tid % 8 (8 lanes read one 128-byte row segment)
  const int a_row = tid / kCpr, a_chunk = tid % kCpr;
  const int a_vo = (int)(a_row * p.ldh * 2) + a_chunk * 16, a_lo = swz(a_row, a_chunk);
  const int a_step = (int)(p.ldh * 2 * (kThreads / kCpr));
  // int8 table slab: load i covers row i * 128 + tid / 4, bytes 16 (tid % 4) .. +15 of the row's 64-byte segment,
  // which become bf16 chunks 2 (tid % 4) and 2 (tid % 4) + 1 of the LDS row. Q4: thread t covers row t / 2, block
  // t % 2 of the stage's two 32-value blocks (16 bytes of nibbles), which become chunks 4 (t % 2) .. +3.
  constexpr int LB = Q4 ? kLoadsBQ4 : kLoadsB;
  const int b_row = Q4 ? tid / 2 : tid / 4, b_c = Q4 ? tid % 2 : tid % 4;
  const int b_vo = (int)(b_row * p.ldw) + b_c * 16;
  const int b_step = (int)(p.ldw * (kThreads / 4));
  constexpr int kStageBytesB = Q4 ? BK / 2 : BK;  // table bytes of a row per stage
  float b_s[LB];
  if constexpr (!Q4) {
#pragma unroll
    for (int i = 0; i < LB; ++i) b_s[i] = od_bf16_to_f32(p.scale[min(n0 + i * (kThreads / 4) + b_row, p.V - 1)]);
  }
  const uint16_t* d_row = p.scale + min(n0 + b_row, p.V - 1) * p.ldd + b_c;  // Q4: this thread's block scales
  const int nk = (int)(p.K / BK);

  v4i ga[kLoadsA], gb[LB];
  uint16_t gd = 0;  // Q4: the block scale of the staged block (fp16 bits)
  // a k-tile past the end reads through zero-length descriptors and gets zeros (no branch)
  const __amdgpu_buffer_rsrc_t ra0 = __builtin_amdgcn_make_buffer_rsrc((void*)p.h, (short)0, 0, 0x00020000);
  const __amdgpu_buffer_rsrc_t rb0 = __builtin_amdgcn_make_buffer_rsrc((void*)p.w, (short)0, 0, 0x00020000);
  auto gload_a = [&](int kt, int i) {
    ga[i] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(kt < nk ? ra : ra0, a_vo,
                                                                         kt * kRowBytes + i * a_step, 0));
  };
  auto gload_b = [&](int kt, int i) {
    gb[i] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(kt < nk ? rb : rb0, b_vo,
                                                                         kt * kStageBytesB + i * b_step, 0));
    if constexpr (Q4) gd = d_row[2 * min(kt, nk - 1)];
  };
  auto swrite_a = [&](int buf, int i) {
    *reinterpret_cast<v4i*>(smem + buf * kStage + a_lo + i * (kThreads / kCpr) * kRowBytes) = ga[i];
  };
  auto swrite_b = [&](int buf, int i) {
    int8_t* lb = smem + buf * kStage + kSlab;
    if constexpr (Q4) {
      float d = fp16_bits_to_f32(gd), unused = 0.0f;
      od_bfr2(d, unused);  // the block scale in bf16, as d.to(bfloat16)
      v4i c[4];
      dequant_q4(gb[i], d, c);
#pragma unroll
      for (int q = 0; q < 4; ++q) *reinterpret_cast<v4i*>(lb + swz(b_row, 4 * b_c + q)) = c[q];
    } else {
      v4i lo, hi;
      dequant16(gb[i], b_s[i], lo, hi);
      const int row = i * (kThreads / 4) + b_row;
      *reinterpret_cast<v4i*>(lb + swz(row, 2 * b_c)) = lo;
      *reinterpret_cast<v4i*>(lb + swz(row, 2 * b_c + 1)) = hi;
    }
  };
  auto frags = [&](int buf, int s, v4i (&fa)[TM], v4i (&fb)[TN]) {
    const int chunk = s * 2 + (lane >> 5);
    const int8_t* la = smem + buf * kStage;
    const int8_t* lb = la + kSlab;
#pragma unroll
    for (int i = 0; i < TM; ++i) fa[i] = *reinterpret_cast<const v4i*>(la + swz(wm * kRowsW + i * 32 + (lane & 31), chunk));
#pragma unroll
    for (int j = 0; j < TN; ++j) fb[j] = *reinterpret_cast<const v4i*>(lb + swz(wn * kColsW + j * 32 + (lane & 31), chunk));
  };

  v16f acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = v16f{0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};

  constexpr int kMf = TM * TN;
  auto mma = [&](const v4i (&fa)[TM], const v4i (&fb)[TN], auto fill, auto OPS) {
    constexpr int kOps = decltype(OPS)::value;
#pragma unroll
    for (int x = 0; x < kMf; ++x) {
      acc[x / TN][x % TN] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, fa[x / TN]),
                                                                   __builtin_bit_cast(bf16x8, fb[x % TN]),
                                                                   acc[x / TN][x % TN], 0, 0, 0);
#pragma unroll
      for (int o = 0; o < kOps; ++o)
        if (o * kMf / (kOps > 0 ? kOps : 1) == x) fill(o);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  auto nofill = [](int) {};
  using Zero = std::integral_constant<int, 0>;

  // pipeline (as in the W8A8 GEMM): LDS buffer kt % 2 holds k-tile kt while it is computed, the registers hold
  // k-tile kt + 1 until k-step 0 of stage kt writes it (table rows dequantized) into the other buffer and loads
  // k-tile kt + 2; one barrier per stage
  v4i f0a[TM], f0b[TN], f1a[TM], f1b[TN];
  constexpr int kOps0 = 2 * (kLoadsA + LB);
#pragma unroll
  for (int i = 0; i < kLoadsA; ++i) gload_a(0, i);
#pragma unroll
  for (int i = 0; i < LB; ++i) gload_b(0, i);
#pragma unroll
  for (int i = 0; i < kLoadsA; ++i) swrite_a(0, i);
#pragma unroll
  for (int i = 0; i < LB; ++i) swrite_b(0, i);
#pragma unroll
  for (int i = 0; i < kLoadsA; ++i) gload_a(1, i);
#pragma unroll
  for (int i = 0; i < LB; ++i) gload_b(1, i);
  barrier_lds();
  frags(0, 0, f0a, f0b);

  auto stage = [&](int CUR, int kt) {
    const int NXT = 1 - CUR;
    frags(CUR, 1, f1a, f1b);
    __builtin_amdgcn_sched_barrier(0);
    auto fill0 = [&](int o) {
      if (o < kLoadsA) swrite_a(NXT, o);
      else if (o < kLoadsA + LB) swrite_b(NXT, o - kLoadsA);
      else if (o < 2 * kLoadsA + LB) gload_a(kt + 2, o - kLoadsA - LB);
      else gload_b(kt + 2, o - 2 * kLoadsA - LB);
    };
    mma(f0a, f0b, fill0, std::integral_constant<int, kOps0>{});
    frags(CUR, 2, f0a, f0b);
    __builtin_amdgcn_sched_barrier(0);
    mma(f1a, f1b, nofill, Zero{});
    frags(CUR, 3, f1a, f1b);
    __builtin_amdgcn_sched_barrier(0);
    mma(f0a, f0b, nofill, Zero{});
    barrier_lds();
    frags(NXT, 0, f0a, f0b);
    __builtin_amdgcn_sched_barrier(0);
    mma(f1a, f1b, nofill, Zero{});
  };
  for (int kt = 0; kt < nk; ++kt) stage(kt & 1, kt);

  // Epilogue: lane l holds column n0 + wn * 128 + j * 32 + l % 32 of tile (i, j) and rows
  // 8 (r / 4) + 4 (l / 32) + r % 4 of the tile's 32. Per row: the bf16 logits of the wave's 128 columns (columns
  // past V are -inf), their max and sum exp(l - max) over the 32 lanes of the half, written by lane 0 of the half.
  const int col = lane & 31, h = lane >> 5;
  bool col_ok[TN];
#pragma unroll
  for (int j = 0; j < TN; ++j) col_ok[j] = n0 + wn * kColsW + j * 32 + col < p.V;
  const int part = tn * kWN + wn;
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float l[TN];
      float mx = -INFINITY;
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        float a = acc[i][j][r], b = 0.0f;
        od_bfr2(a, b);
        l[j] = col_ok[j] ? a : -INFINITY;
        mx = fmaxf(mx, l[j]);
      }
#pragma unroll
      for (int o = 16; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, OD_WAVE));
      float sm = 0.0f;
      if (mx != -INFINITY) {
#pragma unroll
        for (int j = 0; j < TN; ++j) sm += __builtin_amdgcn_exp2f((l[j] - mx) * kLog2e);
      }
#pragma unroll
      for (int o = 16; o > 0; o >>= 1) sm += __shfl_xor(sm, o, OD_WAVE);
      const int64_t m = m0 + wm * kRowsW + i * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
      if (col == 0 && m < p.M) {
        float* dst = p.part + (m * p.n_parts + part) * 2;
        *reinterpret_cast<float2*>(dst) = make_float2(mx, sm);
      }
    }
  }
}

// One wave per row: lse = M + log sum_p s_p exp(m_p - M) over the partials (M = max_p m_p), and the target term
// sum_k float(h[m,k]) * (q[t,k] * s[t]) (each product rounded to fp32, then summed, as the reference's
// (h.float() * row).sum(-1); here each lane sums 8 consecutive k at a time, then the wave); out = target - lse, NaN
// for a token id outside [0, V). Loads are 8 int8 / 8 bf16 / 2 x 4 fp32 per lane (K % 8 == 0, aligned rows).
// Q4: the target row is ((n - 8) * d) with the block scale d in fp32 (the reference's dequant_rows(tok, float32)).
template <bool HF32, bool Q4>
__global__ __launch_bounds__(256) void lm_combine_kernel(const float* __restrict__ part, int n_parts,
                                                         const void* __restrict__ hn, int64_t ldhn,
                                                         const int8_t* __restrict__ w, int64_t ldw,
                                                         const uint16_t* __restrict__ scale, int64_t ldd,
                                                         const int32_t* __restrict__ tok, int64_t M, int64_t V,
                                                         int64_t K, float* __restrict__ out) {
  const int64_t m = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (m >= M) return;  // wave-uniform
  const float2* pr = reinterpret_cast<const float2*>(part + m * n_parts * 2);
  float mx = -INFINITY;
#pragma unroll 4
  for (int q = lane; q < n_parts; q += 64) mx = fmaxf(mx, pr[q].x);
  mx = od_wave_max_dpp(mx);
  float sm = 0.0f;
#pragma unroll 4
  for (int q = lane; q < n_parts; q += 64) {
    const float2 v = pr[q];
    if (v.x != -INFINITY) sm += v.y * __builtin_amdgcn_exp2f((v.x - mx) * kLog2e);
  }
  sm = od_wave_sum_dpp(sm);
  const float lse = mx + __logf(sm);
  const int32_t t = tok[m];
  float dot = 0.0f;
  const bool valid = t >= 0 && t < V;
  if (valid) {
    const int8_t* row = w + (int64_t)t * ldw;
    const float s = Q4 ? 0.0f : od_bf16_to_f32(scale[t]);
#pragma unroll 2
    for (int64_t k = (int64_t)lane * 8; k < K; k += 64 * 8) {
      float wv[8];
      if constexpr (Q4) {
        // k .. k+7 lie in block k / 32 at positions p0 .. p0+7, p0 = k % 32: bytes p0 % 16 .. +7 of the block's
        // 16, low nibbles for p0 < 16, high ones otherwise
        const int64_t blk = k >> 5;
        const int p0 = (int)(k & 31);
        const uint2 b8 = *reinterpret_cast<const uint2*>(row + blk * 16 + (p0 & 15));
        const float d = fp16_bits_to_f32(scale[(int64_t)t * ldd + blk]);
        const uint32_t bb[2] = {b8.x, b8.y};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint32_t byte = (bb[e >> 2] >> (8 * (e & 3))) & 0xffu;
          const uint32_t nib = p0 < 16 ? (byte & 15u) : (byte >> 4);
          wv[e] = ((float)nib - 8.0f) * d;
        }
      } else {
        const uint2 qw = *reinterpret_cast<const uint2*>(row + k);
        const uint32_t qq[2] = {qw.x, qw.y};
#pragma unroll
        for (int e = 0; e < 8; ++e) wv[e] = (float)(int8_t)((qq[e >> 2] >> (8 * (e & 3))) & 0xffu) * s;
      }
      float hv[8];
      if constexpr (HF32) {
        const float4* hp = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(hn) + m * ldhn + k);
        const float4 a = hp[0], b = hp[1];
        hv[0] = a.x; hv[1] = a.y; hv[2] = a.z; hv[3] = a.w; hv[4] = b.x; hv[5] = b.y; hv[6] = b.z; hv[7] = b.w;
      } else {
        const uint4 hb = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(hn) + m * ldhn + k);
        const uint32_t hw[4] = {hb.x, hb.y, hb.z, hb.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          hv[2 * e] = __uint_as_float(hw[e] << 16);
          hv[2 * e + 1] = __uint_as_float(hw[e] & 0xffff0000u);
        }
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) dot += hv[e] * wv[e];
    }
  }
  dot = od_wave_sum_dpp(dot);
  if (lane == 0) out[m] = valid ? dot - lse : __builtin_nanf("");
}

}  // namespace

extern "C" int od_lm_head_logprob_ws(int64_t M, int64_t V, int64_t* ws_floats) {
  if (!ws_floats) return OD_ERR_NULL;
  if (M < 0 || V < 1) return OD_ERR_SHAPE;
  *ws_floats = M * ((V + BN - 1) / BN) * kWN * 2;
  return OD_OK;
}

namespace {

// the checks shared by both table formats; fills the tile counts of p
int lm_prepare(LmArgs& p, const void* hn, int64_t ldhn, int hn_fp32, int64_t ws_floats) {
  if (p.ldh < p.K || ldhn < p.K) return OD_ERR_SHAPE;
  // whole 64-k stages and 16-byte rows; buffer offsets are 32-bit: a tile's panels stay below 2 GiB
  if (p.K % BK || p.ldh % 8 || p.ldw % 16 || !od_aligned16(p.h) || !od_aligned16(p.w)) return OD_ERR_ALIGN;
  if (!od_aligned16(hn) || ldhn % (hn_fp32 ? 4 : 8)) return OD_ERR_ALIGN;
  if ((int64_t)BM * p.ldh * 2 >= (1ll << 31) || (int64_t)BN * p.ldw >= (1ll << 31)) return OD_ERR_UNSUPPORTED;
  int64_t need = 0;
  od_lm_head_logprob_ws(p.M, p.V, &need);
  if (ws_floats < need) return OD_ERR_SHAPE;
  const int64_t tiles_m = (p.M + BM - 1) / BM, tiles_n = (p.V + BN - 1) / BN;
  if (tiles_m * tiles_n > 0x7fffffff || tiles_n * kWN > 0x7fffffff) return OD_ERR_SHAPE;
  p.tiles_m = (int)tiles_m;
  p.tiles_n = (int)tiles_n;
  p.n_parts = (int)(tiles_n * kWN);
  return OD_OK;
}

template <bool Q4>
int lm_launch(const LmArgs& p, const void* hn, int64_t ldhn, int hn_fp32, const int32_t* tok, float* out,
              hipStream_t st) {
  lm_logits_kernel<Q4><<<dim3((unsigned)(p.tiles_m * p.tiles_n)), dim3(kThreads), 0, st>>>(p);
  const int rc = od_launch_status();
  if (rc != OD_OK) return rc;
  const dim3 grid((unsigned)((p.M + 3) / 4));
  if (hn_fp32) {
    lm_combine_kernel<true, Q4><<<grid, dim3(256), 0, st>>>(p.part, p.n_parts, hn, ldhn, p.w, p.ldw, p.scale, p.ldd,
                                                            tok, p.M, p.V, p.K, out);
  } else {
    lm_combine_kernel<false, Q4><<<grid, dim3(256), 0, st>>>(p.part, p.n_parts, hn, ldhn, p.w, p.ldw, p.scale,
                                                             p.ldd, tok, p.M, p.V, p.K, out);
  }
  return od_launch_status();
}

}  // namespace

extern "C" int od_lm_head_logprob(const uint16_t* hb, int64_t ldh, const void* hn, int64_t ldhn, int hn_fp32,
                                  const int8_t* w, int64_t ldw, const uint16_t* scale, const int32_t* tok, int64_t M,
                                  int64_t V, int64_t K, float* out, float* ws, int64_t ws_floats,
                                  od_stream_t stream) {
  if (M < 0 || V < 1 || K < 1) return OD_ERR_SHAPE;
  if (M == 0) return OD_OK;
  if (!hb || !hn || !w || !scale || !tok || !out || !ws) return OD_ERR_NULL;
  if (ldw < K) return OD_ERR_SHAPE;
  LmArgs p{hb, w, scale, ws, ldh, ldw, 0, M, V, K, 0, 0, 0};
  const int rc = lm_prepare(p, hn, ldhn, hn_fp32, ws_floats);
  if (rc != OD_OK) return rc;
  return lm_launch<false>(p, hn, ldhn, hn_fp32, tok, out, (hipStream_t)stream);
}

extern "C" int od_lm_head_logprob_q4(const uint16_t* hb, int64_t ldh, const void* hn, int64_t ldhn, int hn_fp32,
                                     const uint8_t* qs, int64_t ldq, const uint16_t* d, int64_t ldd,
                                     const int32_t* tok, int64_t M, int64_t V, int64_t K, float* out, float* ws,
                                     int64_t ws_floats, od_stream_t stream) {
  if (M < 0 || V < 1 || K < 1) return OD_ERR_SHAPE;
  if (M == 0) return OD_OK;
  if (!hb || !hn || !qs || !d || !tok || !out || !ws) return OD_ERR_NULL;
  if (ldq < K / 2 || ldd < K / 32) return OD_ERR_SHAPE;
  if ((((uintptr_t)d) & 1u) != 0) return OD_ERR_ALIGN;
  LmArgs p{hb, reinterpret_cast<const int8_t*>(qs), d, ws, ldh, ldq, ldd, M, V, K, 0, 0, 0};
  const int rc = lm_prepare(p, hn, ldhn, hn_fp32, ws_floats);
  if (rc != OD_OK) return rc;
  return lm_launch<true>(p, hn, ldhn, hn_fp32, tok, out, (hipStream_t)stream);
}
