// Chunked gated delta rule on bf16 MFMA (gfx950), the fast form of od_gdn_recurrence's arithmetic.
//
// The recurrence of a value head (state S in R^{dk x dv}, token i: S_i = e^{g_i} S_{i-1} + k_i delta_i^T,
// delta_i = beta_i (v_i - (e^{g_i} S_{i-1})^T k_i), o_i = S_i^T q~_i with q~ = q / sqrt(dk); transformers'
// torch_recurrent_gated_delta_rule, which the reference runs for Qwen3.5's linear-attention layers) is unrolled over
// chunks of C = 32 tokens. With gamma_i = g_1 + ... + g_i inside the chunk and S_0 the state at its start:
//   A_ij = beta_i e^{gamma_i - gamma_j} (k_i . k_j)  (j < i),   T = (I + A)^{-1} diag(beta)
//   delta = T V - T diag(e^gamma) K S_0
//   O     = diag(e^gamma) Q~ S_0 + (Q~ K^T o D) delta,            D_ij = e^{gamma_i - gamma_j} (j <= i), else 0
//   S_C   = e^{gamma_C} S_0 + K^T diag(e^{gamma_C - gamma}) delta
// (the WY form of the chunked delta rule, as transformers' torch_chunk_gated_delta_rule evaluates it). Every
// exponent is of a non-positive number, so nothing overflows whatever the decay.
//
// Two kernels. gdn_chunk_t, per (sequence, chunk, key head): K K^T on MFMA and T by forward substitution in fp32 for
// each value head of that key head, written as bf16 hi / lo in the layout the second kernel copies straight into
// LDS, with the vectors gamma, e^gamma, e^{gamma_C - gamma} and e^{gamma_C}. gdn_chunk_state, per (sequence, value
// head, 64 state columns), four waves of 16 columns each, chunk after chunk (the only sequential part): P from
// K Q~^T on MFMA, then the products above. The state lives in the MFMA accumulators
// (V_MFMA_F32_16X16X32_BF16, lane l: column l % 16, rows 4 (l / 16) + i of each 16 x 16 tile) and feeds the next
// products straight from there: an accumulator tile's rows become a B operand's k-values in the order
// (4h .. 4h+3, 16+4h .. 16+4h+3) for lane group h, and the A operand reads its k-index in the same order, so no
// transpose goes through LDS; T diag(e^gamma) X is taken as T (diag(e^gamma) X), the scaling on X's rows. Products
// whose operands are both exact in bf16 (K K^T, K Q^T) take one MFMA; an fp32 operand is split into bf16 hi + lo
// (16 significant bits; residual 2^-17 relative) and a product of two fp32 operands takes hi.hi + hi.lo + lo.hi, so
// every product carries ~16 bits against fp32's 24, accumulated in fp32.
#include "od_common.h"

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kC = 32;                // tokens per chunk
constexpr int kDk = 128;
constexpr int kCols = 64;             // state columns per workgroup of gdn_chunk_state (16 per wave)
// workspace per (sequence, chunk, value head): T as two bf16 [32][32] matrices (hi, lo), then 112 floats: gamma [32],
// e^gamma [32], e^{gamma_C - gamma} [32], e^{gamma_C}, padding
constexpr int kMat = kC * kC;                      // bf16 per matrix
constexpr int kVecOff = 2 * kMat / 2;              // float offset of the vectors
constexpr int kVecN = 112;
constexpr int kTWs = kVecOff + kVecN;              // floats per block (4544 bytes, a multiple of 16)

__device__ __forceinline__ v4f mfma16(bf16x8 a, bf16x8 b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ __bf16 bfr(float x) { return __builtin_bit_cast(__bf16, od_f32_to_bf16(x)); }
__device__ __forceinline__ float bff(__bf16 x) { return __uint_as_float((uint32_t)__builtin_bit_cast(uint16_t, x) << 16); }
// x = hi + lo + O(2^-17 |x|), hi and lo bf16
__device__ __forceinline__ void split(float x, __bf16& hi, __bf16& lo) {
  hi = bfr(x);
  lo = bfr(x - bff(hi));
}
// 8 bf16 of an LDS row in the permuted k-order of an accumulator used as a B operand: elements
// base + 4h .. base + 4h + 3, then base + 16 + 4h .. base + 16 + 4h + 3
__device__ __forceinline__ bf16x8 lds_perm(const uint16_t* row, int base, int h) {
  const uint2 a = *reinterpret_cast<const uint2*>(row + base + 4 * h);
  const uint2 b = *reinterpret_cast<const uint2*>(row + base + 16 + 4 * h);
  const uint4 w = make_uint4(a.x, a.y, b.x, b.y);
  return __builtin_bit_cast(bf16x8, w);
}
__device__ __forceinline__ bf16x8 lds8(const uint16_t* p) {
  return __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(p));
}
// two fp32 values -> their bf16 hi and lo parts, each pair packed in one word (a in the low half)
__device__ __forceinline__ void split2(float a, float b, uint32_t& hi, uint32_t& lo) {
  hi = __builtin_bit_cast(uint32_t, __builtin_convertvector((od_f32x2){a, b}, od_bf16x2));
  const float ra = a - __uint_as_float(hi << 16), rb = b - __uint_as_float(hi & 0xffff0000u);
  lo = __builtin_bit_cast(uint32_t, __builtin_convertvector((od_f32x2){ra, rb}, od_bf16x2));
}
// the B operand, split, of accumulator tiles a (rows 0..15) and b (rows 16..31): values 4h .. 4h + 3 of a, then of b
__device__ __forceinline__ void acc_to_b(const v4f& a, const v4f& b, bf16x8& hi, bf16x8& lo) {
  uint32_t h[4], l[4];
  split2(a[0], a[1], h[0], l[0]);
  split2(a[2], a[3], h[1], l[1]);
  split2(b[0], b[1], h[2], l[2]);
  split2(b[2], b[3], h[3], l[3]);
  hi = __builtin_bit_cast(bf16x8, make_uint4(h[0], h[1], h[2], h[3]));
  lo = __builtin_bit_cast(bf16x8, make_uint4(l[0], l[1], l[2], l[3]));
}
// 8 bf16 in natural order from an 8-byte aligned row
__device__ __forceinline__ bf16x8 lds_nat(const uint16_t* p) {
  const uint2 a = *reinterpret_cast<const uint2*>(p);
  const uint2 b = *reinterpret_cast<const uint2*>(p + 4);
  return __builtin_bit_cast(bf16x8, make_uint4(a.x, a.y, b.x, b.y));
}
__device__ __forceinline__ uint16_t bf_bits(float x) { return od_f32_to_bf16(x); }

// ------------------------------------------------------------------------------------------------ gdn_chunk_t
struct TArgs {
  const uint16_t* qk;
  const float* g;
  const float* beta;
  float* ws;
  int64_t L, nchunk;
  int n_k, n_v;
};

// One wave per (sequence, chunk, key head); lanes 0..31 and 32..63 take two of the key head's value heads at once,
// lane j of a half owning column j of T during the solve and row j of the outputs after it.
__global__ __launch_bounds__(64) void gdn_chunk_t_kernel(TArgs p) {
  __shared__ float kk[kC][kC + 1];
  __shared__ __attribute__((aligned(16))) float A[2][kC][kC];
  __shared__ float gam[2][kC], bet[2][kC];
  const int64_t bid = blockIdx.x;
  const int hk = (int)(bid % p.n_k);
  const int64_t c = (bid / p.n_k) % p.nchunk;
  const int64_t s = bid / ((int64_t)p.n_k * p.nchunk);
  const int l = threadIdx.x, h4 = l >> 4, lc = l & 15;
  const int64_t t0 = c * kC, m0 = s * p.L;
  const int64_t kd = (int64_t)p.n_k * kDk;
  const int rep = p.n_v / p.n_k;

  // K K^T, tiles (0,0), (1,0), (1,1): both operands are rows (token 16 t + lc, dk 32 m + 8 h4 .. + 7)
  bf16x8 kf[2][4];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int64_t tok = t0 + 16 * t + lc;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      uint4 wk = make_uint4(0, 0, 0, 0);
      if (tok < p.L) wk = *reinterpret_cast<const uint4*>(p.qk + (m0 + tok) * 2 * kd + kd + (int64_t)hk * kDk + 32 * m +
                                                          8 * h4);
      kf[t][m] = __builtin_bit_cast(bf16x8, wk);
    }
  }
  v4f a00 = {0, 0, 0, 0}, a10 = a00, a11 = a00;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    a00 = mfma16(kf[0][m], kf[0][m], a00);
    a10 = mfma16(kf[1][m], kf[0][m], a10);
    a11 = mfma16(kf[1][m], kf[1][m], a11);
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    kk[4 * h4 + r][lc] = a00[r];
    kk[16 + 4 * h4 + r][lc] = a10[r];
    kk[16 + 4 * h4 + r][16 + lc] = a11[r];
  }

  const int half = l >> 5, j = l & 31;
  for (int pp = 0; pp < rep; pp += 2) {
    const bool valid = pp + half < rep;
    const int hv = hk * rep + pp + half;
    const int64_t tok = t0 + j;
    float gj = 0.0f, bj = 0.0f;
    if (valid && tok < p.L) {
      gj = p.g[(m0 + tok) * p.n_v + hv];
      bj = p.beta[(m0 + tok) * p.n_v + hv];
    }
    gam[half][j] = gj;
    __syncthreads();
    float cum = 0.0f;
    for (int u = 0; u <= j; ++u) cum += gam[half][u];
    __syncthreads();
    gam[half][j] = cum;
    bet[half][j] = bj;
    __syncthreads();
    // column j of A: beta_i e^{gamma_i - gamma_j} kk_ij below the diagonal
    for (int i = 0; i < kC; ++i)
      A[half][i][j] = i > j ? bet[half][i] * __expf(gam[half][i] - cum) * kk[i][j] : 0.0f;
    __syncthreads();
    // column j of (I + A)^{-1} by forward substitution; T = (I + A)^{-1} diag(beta)
    float x[kC];
#pragma unroll
    for (int i = 0; i < kC; ++i) {
      float acc = i == j ? 1.0f : 0.0f;
      const float4* row = reinterpret_cast<const float4*>(&A[half][i][0]);
#pragma unroll
      for (int m4 = 0; m4 < i / 4 + (i % 4 ? 1 : 0); ++m4) {
        const float4 a = row[m4];
        const float av[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (4 * m4 + e < i) acc = fmaf(-av[e], x[4 * m4 + e], acc);
      }
      x[i] = acc;
    }
    __syncthreads();  // every lane is done reading A: column j of T goes where column j of A was
#pragma unroll
    for (int i = 0; i < kC; ++i) A[half][i][j] = x[i] * bj;
    gam[half][j] = cum;
    bet[half][j] = __expf(cum);  // e^{gamma_j} from here on
    __syncthreads();
    // lane (half, i) writes row i of T of its value head, split into bf16 hi / lo, in 16-byte stores
    const int i = j;
    uint4* blk = reinterpret_cast<uint4*>(p.ws + ((s * p.nchunk + c) * p.n_v + hv) * (int64_t)kTWs);
#pragma unroll
    for (int j8 = 0; j8 < kC; j8 += 8) {
      uint32_t th[4], tl[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) split2(A[half][i][j8 + 2 * e], A[half][i][j8 + 2 * e + 1], th[e], tl[e]);
      if (valid) {
        const int q = (i * kC + j8) / 8;  // 16-byte unit of row i, columns j8 .. j8 + 7
        blk[q] = make_uint4(th[0], th[1], th[2], th[3]);
        blk[kMat / 8 + q] = make_uint4(tl[0], tl[1], tl[2], tl[3]);
      }
    }
    if (valid) {
      const float glast = gam[half][kC - 1];
      float* vec = reinterpret_cast<float*>(blk) + kVecOff;
      vec[j] = cum;
      vec[kC + j] = bet[half][j];
      vec[2 * kC + j] = __expf(glast - cum);
      if (j == 0) vec[3 * kC] = __expf(glast);
    }
    __syncthreads();
  }
}

// ------------------------------------------------------------------------------------------------ gdn_chunk_state
struct CArgs {
  const uint16_t* qk;
  const uint16_t* v;
  const float* init;
  const int32_t* seq_state;
  const float* ws;
  uint16_t* o;
  float* final_state;
  int64_t L, nchunk, n_states;
  int n_k, n_v, dv;
};

constexpr int kRowK = kDk + 8;    // K, Q rows (272 bytes: conflict-free 8-byte reads per half-wave)
constexpr int kRowT = kC + 4;     // K^T, V^T rows (72 bytes: conflict-free paired-token 4-byte writes)
constexpr int kRowM = kC + 8;     // the six matrices (80 bytes, 16-byte aligned rows)

struct CStage {
  uint16_t k[kC][kRowK];          // K (tokens x dk)
  uint16_t q[kC][kRowK];          // Q (tokens x dk)
  uint16_t kt[kDk][kRowT];        // K^T (dk x tokens)
  uint16_t vt[kCols][kRowT];      // V^T of the workgroup's 64 columns (columns x tokens)
  uint16_t m4[4][kC][kRowM];      // T hi, lo; P hi, lo
  float vec[kVecN];               // gamma [32], e^gamma [32], e^{gamma_C - gamma} [32], e^{gamma_C}
};

__device__ __forceinline__ uint32_t lo_pair(uint32_t a, uint32_t b) { return (a & 0xffffu) | (b << 16); }
__device__ __forceinline__ uint32_t hi_pair(uint32_t a, uint32_t b) { return (a >> 16) | (b & 0xffff0000u); }

__global__ __launch_bounds__(256) void gdn_chunk_state_kernel(CArgs p) {
  __shared__ __attribute__((aligned(16))) CStage st;
  __shared__ __attribute__((aligned(16))) uint16_t ob[kC][kCols + 8];
  const int nblk = p.dv / kCols;
  const int64_t bid = blockIdx.x;
  const int cb = (int)(bid % nblk);
  const int h = (int)((bid / nblk) % p.n_v);
  const int64_t s = bid / ((int64_t)nblk * p.n_v);
  const int hk = h / (p.n_v / p.n_k);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, h4 = lane >> 4, lc = lane & 15;
  const int64_t kd = (int64_t)p.n_k * kDk, ldv = (int64_t)p.n_v * p.dv;
  const int64_t m0 = s * p.L;
  const int col = cb * kCols + 16 * w + lc;  // this lane's state column
  const float qscale = (float)0.08838834764831845;  // fp32(1 / sqrt(128)), the reference's query scale

  // the state: tile r holds dk rows 16 r + 4 h4 + i of column `col`
  v4f S[8];
  const int64_t sidx = p.seq_state ? (int64_t)p.seq_state[s] : s;
  const bool has_init = p.init && sidx >= 0 && sidx < p.n_states;
#pragma unroll
  for (int r = 0; r < 8; ++r)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      S[r][i] = has_init ? p.init[((sidx * p.n_v + h) * kDk + 16 * r + 4 * h4 + i) * p.dv + col] : 0.0f;

  // chunk inputs, prefetched into registers one chunk ahead. K and V: thread (tp, part) takes tokens 2 tp and
  // 2 tp + 1 of one 8-wide part, so that the transposed copies are written as token pairs
  const int tp = tid & 15, kp = tid >> 4, vp = (tid >> 4) & 7;
  struct Pre {
    uint4 k0, k1, q0, q1, v0, v1, w0, vec;
  };
  auto gload = [&](int64_t c) -> Pre {
    const int64_t t0 = c * kC;
    const uint4 z = make_uint4(0, 0, 0, 0);
    Pre r;
    {
      const int64_t ta = t0 + 2 * tp, tb = ta + 1;
      const uint16_t* src = p.qk + kd + (int64_t)hk * kDk + 8 * kp;
      r.k0 = ta < p.L ? *reinterpret_cast<const uint4*>(src + (m0 + ta) * 2 * kd) : z;
      r.k1 = tb < p.L ? *reinterpret_cast<const uint4*>(src + (m0 + tb) * 2 * kd) : z;
    }
    {
      const int64_t ta = t0 + (tid >> 4), tb = ta + 16;
      const uint16_t* src = p.qk + (int64_t)hk * kDk + 8 * (tid & 15);
      r.q0 = ta < p.L ? *reinterpret_cast<const uint4*>(src + (m0 + ta) * 2 * kd) : z;
      r.q1 = tb < p.L ? *reinterpret_cast<const uint4*>(src + (m0 + tb) * 2 * kd) : z;
    }
    {
      const int64_t ta = t0 + 2 * tp, tb = ta + 1;
      const uint16_t* src = p.v + (int64_t)h * p.dv + cb * kCols + 8 * vp;
      r.v0 = tid < 128 && ta < p.L ? *reinterpret_cast<const uint4*>(src + (m0 + ta) * ldv) : z;
      r.v1 = tid < 128 && tb < p.L ? *reinterpret_cast<const uint4*>(src + (m0 + tb) * ldv) : z;
    }
    const uint4* blk = reinterpret_cast<const uint4*>(p.ws + ((s * p.nchunk + c) * p.n_v + h) * (int64_t)kTWs);
    r.w0 = blk[tid];                                              // T hi, lo: 256 pieces
    r.vec = tid < kVecN / 4 ? blk[2 * kMat / 8 + tid] : z;        // the vectors: 28 pieces
    return r;
  };
  auto swrite = [&](const Pre& r) {
    *reinterpret_cast<uint4*>(&st.k[2 * tp][8 * kp]) = r.k0;
    *reinterpret_cast<uint4*>(&st.k[2 * tp + 1][8 * kp]) = r.k1;
    {
      const uint32_t a[4] = {r.k0.x, r.k0.y, r.k0.z, r.k0.w}, b[4] = {r.k1.x, r.k1.y, r.k1.z, r.k1.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        *reinterpret_cast<uint32_t*>(&st.kt[8 * kp + 2 * e][2 * tp]) = lo_pair(a[e], b[e]);
        *reinterpret_cast<uint32_t*>(&st.kt[8 * kp + 2 * e + 1][2 * tp]) = hi_pair(a[e], b[e]);
      }
    }
    *reinterpret_cast<uint4*>(&st.q[tid >> 4][8 * (tid & 15)]) = r.q0;
    *reinterpret_cast<uint4*>(&st.q[16 + (tid >> 4)][8 * (tid & 15)]) = r.q1;
    if (tid < 128) {
      const uint32_t a[4] = {r.v0.x, r.v0.y, r.v0.z, r.v0.w}, b[4] = {r.v1.x, r.v1.y, r.v1.z, r.v1.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        *reinterpret_cast<uint32_t*>(&st.vt[8 * vp + 2 * e][2 * tp]) = lo_pair(a[e], b[e]);
        *reinterpret_cast<uint32_t*>(&st.vt[8 * vp + 2 * e + 1][2 * tp]) = hi_pair(a[e], b[e]);
      }
    }
    *reinterpret_cast<uint4*>(&st.m4[tid >> 7][(tid & 127) >> 2][8 * (tid & 3)]) = r.w0;
    if (tid < kVecN / 4) *reinterpret_cast<uint4*>(&st.vec[4 * tid]) = r.vec;
  };

  // one chunk on the staged inputs: the outputs go to `ob`, the state advances
  const float* gam = st.vec;
  const float* eg = st.vec + kC;
  const float* ec = st.vec + 2 * kC;
  auto compute = [&]() {
    // P^T = K Q~^T o D^T on MFMA, tiles (key tile, query tile) = (0,0), (0,1), (1,1) on waves 0..2; lane: query i,
    // keys 4 h4 .. 4 h4 + 3 of the tile, written as P[i][j] hi / lo 8 bytes at a time. Wave 3 clears the upper tile.
    if (w < 3) {
      const int tj = w == 2 ? 1 : 0, ti = w == 0 ? 0 : 1;
      v4f a = {0, 0, 0, 0};
#pragma unroll
      for (int m = 0; m < 4; ++m)
        a = mfma16(lds8(&st.k[16 * tj + lc][32 * m + 8 * h4]), lds8(&st.q[16 * ti + lc][32 * m + 8 * h4]), a);
      const int i = 16 * ti + lc, j0 = 16 * tj + 4 * h4;
      float pv[4];
#pragma unroll
      for (int r = 0; r < 4; ++r)
        pv[r] = j0 + r <= i ? a[r] * qscale * __expf(gam[i] - gam[j0 + r]) : 0.0f;
      uint32_t h0, l0, h1, l1;
      split2(pv[0], pv[1], h0, l0);
      split2(pv[2], pv[3], h1, l1);
      *reinterpret_cast<uint2*>(&st.m4[2][i][j0]) = make_uint2(h0, h1);
      *reinterpret_cast<uint2*>(&st.m4[3][i][j0]) = make_uint2(l0, l1);
    } else {
      *reinterpret_cast<uint2*>(&st.m4[2][lc][16 + 4 * h4]) = make_uint2(0, 0);
      *reinterpret_cast<uint2*>(&st.m4[3][lc][16 + 4 * h4]) = make_uint2(0, 0);
    }
    __syncthreads();
    // X = K S_0 and Y = Q S_0 (tokens x this wave's 16 columns), S_0 split from the accumulators
    bf16x8 sh[4], sl[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) acc_to_b(S[2 * m], S[2 * m + 1], sh[m], sl[m]);
    v4f X[2], Y[2], U[2], D[2], O[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      X[t] = v4f{0, 0, 0, 0};
      Y[t] = v4f{0, 0, 0, 0};
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const bf16x8 ak = lds_perm(&st.k[16 * t + lc][0], 32 * m, h4);
        const bf16x8 aq = lds_perm(&st.q[16 * t + lc][0], 32 * m, h4);
        X[t] = mfma16(ak, sh[m], X[t]);
        Y[t] = mfma16(aq, sh[m], Y[t]);
        X[t] = mfma16(ak, sl[m], X[t]);
        Y[t] = mfma16(aq, sl[m], Y[t]);
      }
    }
    // U = T V (natural token order)
    const bf16x8 bv = lds_nat(&st.vt[16 * w + lc][8 * h4]);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      U[t] = mfma16(lds8(&st.m4[0][16 * t + lc][8 * h4]), bv, v4f{0, 0, 0, 0});
      U[t] = mfma16(lds8(&st.m4[1][16 * t + lc][8 * h4]), bv, U[t]);
    }
    // delta = U - T (diag(e^gamma) X)
    v4f x0, x1;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x0[e] = -eg[4 * h4 + e] * X[0][e];
      x1[e] = -eg[16 + 4 * h4 + e] * X[1][e];
    }
    bf16x8 xh, xl;
    acc_to_b(x0, x1, xh, xl);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const bf16x8 ath = lds_perm(&st.m4[0][16 * t + lc][0], 0, h4), atl = lds_perm(&st.m4[1][16 * t + lc][0], 0, h4);
      D[t] = mfma16(ath, xh, U[t]);
      D[t] = mfma16(ath, xl, D[t]);
      D[t] = mfma16(atl, xh, D[t]);
    }
    // O = diag(e^gamma / sqrt(dk)) Y + P delta
    bf16x8 dh, dl;
    acc_to_b(D[0], D[1], dh, dl);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int r = 0; r < 4; ++r) O[t][r] = eg[16 * t + 4 * h4 + r] * qscale * Y[t][r];
      const bf16x8 aph = lds_perm(&st.m4[2][16 * t + lc][0], 0, h4), apl = lds_perm(&st.m4[3][16 * t + lc][0], 0, h4);
      O[t] = mfma16(aph, dh, O[t]);
      O[t] = mfma16(aph, dl, O[t]);
      O[t] = mfma16(apl, dh, O[t]);
#pragma unroll
      for (int r = 0; r < 4; ++r) ob[16 * t + 4 * h4 + r][16 * w + lc] = bf_bits(O[t][r]);
    }
    // S = e^{gamma_C} S_0 + K^T diag(e^{gamma_C - gamma}) delta
    v4f d0, d1;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      d0[e] = ec[4 * h4 + e] * D[0][e];
      d1[e] = ec[16 + 4 * h4 + e] * D[1][e];
    }
    bf16x8 eh, el;
    acc_to_b(d0, d1, eh, el);
    const float elast = st.vec[3 * kC];
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      S[r] *= elast;
      const bf16x8 akt = lds_perm(&st.kt[16 * r + lc][0], 0, h4);
      S[r] = mfma16(akt, eh, S[r]);
      S[r] = mfma16(akt, el, S[r]);
    }
  };
  auto finish = [&](int64_t c) {
    __syncthreads();  // every wave is done with the stage and has written its outputs
    const int64_t tt = c * kC + (tid >> 3);
    if (tt < p.L)
      *reinterpret_cast<uint4*>(p.o + (m0 + tt) * ldv + (int64_t)h * p.dv + cb * kCols + 8 * (tid & 7)) =
          *reinterpret_cast<const uint4*>(&ob[tid >> 3][8 * (tid & 7)]);
  };

  // chunk inputs are loaded two chunks ahead (two register sets, alternating)
  Pre pa = gload(0);
  swrite(pa);
  __syncthreads();
  Pre pb = pa;
  if (p.nchunk > 1) pb = gload(1);
  for (int64_t c = 0; c < p.nchunk; c += 2) {
    if (c + 2 < p.nchunk) pa = gload(c + 2);
    compute();
    finish(c);
    if (c + 1 >= p.nchunk) break;
    swrite(pb);
    __syncthreads();
    if (c + 3 < p.nchunk) pb = gload(c + 3);
    compute();
    finish(c + 1);
    if (c + 2 < p.nchunk) swrite(pa);
    __syncthreads();
  }
  if (p.final_state) {
#pragma unroll
    for (int r = 0; r < 8; ++r)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        p.final_state[((s * p.n_v + h) * kDk + 16 * r + 4 * h4 + i) * p.dv + col] = S[r][i];
  }
}

}  // namespace

extern "C" int od_gdn_chunk_ws_size(int64_t S, int64_t L, int64_t n_v, int64_t* ws_floats) {
  if (!ws_floats) return OD_ERR_NULL;
  if (S < 0 || L < 0 || n_v < 1) return OD_ERR_SHAPE;
  *ws_floats = S * ((L + kC - 1) / kC) * n_v * kTWs;
  return OD_OK;
}

extern "C" int od_gdn_recurrence_chunked(const uint16_t* qk, const uint16_t* v, const float* g, const float* beta,
                                         const float* init, const int32_t* seq_state, int64_t n_states, int64_t S,
                                         int64_t L, int64_t n_k, int64_t n_v, int64_t dk, int64_t dv, uint16_t* o,
                                         float* final_state, float* ws, int64_t ws_floats, od_stream_t stream) {
  if (S < 0 || L < 0 || n_k < 1 || n_v < 1 || n_states < 0) return OD_ERR_SHAPE;
  if (S == 0 || L == 0) return (S > 0 && final_state) ? OD_ERR_SHAPE : OD_OK;
  if (!qk || !v || !g || !beta || !o || !ws) return OD_ERR_NULL;
  if (dk != kDk || dv % kCols || n_v % n_k) return OD_ERR_UNSUPPORTED;
  if (!od_aligned16(qk) || !od_aligned16(v) || !od_aligned16(o) || !od_aligned16(ws)) return OD_ERR_ALIGN;
  const int64_t nchunk = (L + kC - 1) / kC;
  if (ws_floats < S * nchunk * n_v * kTWs) return OD_ERR_SHAPE;
  const int64_t tblocks = S * nchunk * n_k, cblocks = S * n_v * (dv / kCols);
  if (tblocks > 0x7fffffffll || cblocks > 0x7fffffffll || S * L > 0x7fffffffll) return OD_ERR_SHAPE;
  TArgs tp{qk, g, beta, ws, L, nchunk, (int)n_k, (int)n_v};
  gdn_chunk_t_kernel<<<dim3((unsigned)tblocks), dim3(64), 0, (hipStream_t)stream>>>(tp);
  CArgs cp{qk, v, init, seq_state, ws, o, final_state, L, nchunk, n_states, (int)n_k, (int)n_v, (int)dv};
  gdn_chunk_state_kernel<<<dim3((unsigned)cblocks), dim3(256), 0, (hipStream_t)stream>>>(cp);
  return od_launch_status();
}
