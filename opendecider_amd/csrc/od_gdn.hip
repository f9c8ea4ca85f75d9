// Gated DeltaNet (linear-attention) layer of the Qwen3.5 hybrid backbone, for gfx950: the three passes between the
// layer's two W8A8 linears (in_proj, out_proj).
//
// Math (transformers' Qwen3_5GatedDeltaNet, which the reference runs: src/opendecider/backbone.py:256-289,
// src/opendecider/skipkv.py:208-231; branch rows reading the shared prefix state instead of copying it,
// docs/branched_shared_prefix_math.md:16-37). Per token of a sequence and per value head, state S in R^{dk x dv}:
//   od_gdn_prep        y = bf16(silu(bf16(sum_j w[c, j] x[t - 3 + j, c]))) over [previous 3 inputs ; the sequence]
//                      (depthwise causal conv, kernel 4); q, k = l2norm(y) per head in bf16 arithmetic; v = y;
//                      beta = bf16(sigmoid(b)), g = -exp(A_log) softplus(a + dt_bias) in fp32; the sequence's last
//                      3 inputs become its new conv state
//   od_gdn_recurrence  S <- S e^g ; kv = S^T k ; delta = (v - kv) beta ; S <- S + k delta^T ; o = S^T (q / sqrt(dk))
//                      (fp32), S starting from the state the sequence continues (none: zeros)
//   od_gdn_norm_quant  bf16(bf16(w * bf16(o * rms(o))) * silu(z)) per value head (the gated RMSNorm), then the
//                      out_proj input quantizer (optional SmoothQuant factors), per token
// Every sum whose order torch leaves open (the conv taps, the squares of the l2norm and of the RMSNorm) is taken
// exactly in float64 and rounded once, the transcendental functions of the gates are evaluated in float64, and the
// SiLUs are fp32 fast steps that fall back to float64 wherever their rounding could differ, so od_gdn_prep and
// od_gdn_norm_quant give the oracle's bytes; the recurrence keeps fp32 with reductions in hardware
// order.
//
// Layouts: proj bf16 [M, ldp] = [qkv (C = 2 n_k dk + n_v dv) | z (n_v dv) | b (n_v) | a (n_v)] with M = S L tokens,
// sequence s holding tokens s L .. s L + L - 1; conv states bf16 [., 3, C]; q|k bf16 [M, 2 n_k dk]; v bf16
// [M, n_v dv]; g, beta fp32 [M, n_v]; recurrent states fp32 [., n_v, dk, dv]; o bf16 [M, n_v dv].
#include "od_common.h"

namespace {

constexpr int kConvTaps = 4;
constexpr int kChan = 16;  // channels per thread in the row passes

// ------------------------------------------------------------------------------------------------ od_gdn_prep
struct PrepArgs {
  const uint16_t* proj;
  const uint16_t* conv_w;
  const uint16_t* conv_in;
  const int32_t* seq_state;
  const uint16_t* A_log;
  const uint16_t* dt_bias;
  uint16_t* qk;
  uint16_t* v;
  float* g;
  float* beta;
  uint16_t* conv_out;
  const int32_t* seq_len;  // real tokens of each sequence (NULL: L); the rest are right pads
  int64_t ldp, S, L, n_states;
  int n_k, n_v, dk, dv, C;
};

__device__ __forceinline__ void load16(const uint16_t* p, float (&f)[kChan]) {
  const uint4 a = *reinterpret_cast<const uint4*>(p);
  const uint4 b = *reinterpret_cast<const uint4*>(p + 8);
  const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    f[2 * i] = __uint_as_float(w[i] << 16);
    f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}

__device__ __forceinline__ void store16(uint16_t* p, const float (&f)[kChan]) {
  uint32_t w[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) w[i] = (uint32_t)od_f32_to_bf16(f[2 * i]) | ((uint32_t)od_f32_to_bf16(f[2 * i + 1]) << 16);
  *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
  *reinterpret_cast<uint4*>(p + 8) = make_uint4(w[4], w[5], w[6], w[7]);
}

__device__ __forceinline__ float bf(float x) { return od_bf16_to_f32(od_f32_to_bf16(x)); }

// od_silu_bf16 with its float64 step out of line: the prep kernel calls it for 16 channels per token, and 16
// inlined copies of the rare float64 path cost registers the common path needs
__device__ __noinline__ float silu_bf16_slow(float g) {
  const double gd = (double)g;
  return od_bf16_to_f32(od_f32_to_bf16((float)(gd / (1.0 + exp(-gd)))));
}
// bf16(RN32(hw * RN32(silu(z)))), the gated norm's product (hw times silu of the fp32 gate, both fp32, then bf16).
// Fast step for |z| < 16: the fp32 silu of od_silu_bf16 (within 11 ulps of silu(z)) times hw lands within 26 ulps of
// RN32(hw * RN32(silu(z))), so its bf16 rounding is that of the reference value unless its low 16 bits lie within 48
// ulps of the bf16 midpoint 0x8000; those (about 1 in 700), and |z| >= 16, take the float64 silu.
__device__ __noinline__ float silu_mul_slow(float hw, float z) {
  const double zd = (double)z;
  const float sl = (float)(zd / (1.0 + exp(-zd)));
  return od_bf16_to_f32(od_f32_to_bf16(hw * sl));
}
__device__ __forceinline__ float silu_mul_bf16(float hw, float z) {
  const float sl = z * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(z * -1.44269504088896341f));
  const float pr = hw * sl;
  const uint32_t lo = __float_as_uint(pr) & 0xffffu;
  if (__builtin_expect((lo - 0x7fd0u) <= 0x60u || !(fabsf(z) < 16.0f), 0)) return silu_mul_slow(hw, z);
  return od_bf16_to_f32(od_f32_to_bf16(pr));
}
__device__ __forceinline__ float silu_bf16(float g) {
  const float s = g * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(g * -1.44269504088896341f));
  const uint32_t lo = __float_as_uint(s) & 0xffffu;
  if (__builtin_expect((lo - 0x7ff0u) <= 0x20u || !(fabsf(g) < 16.0f), 0)) return silu_bf16_slow(g);
  return od_bf16_to_f32(od_f32_to_bf16(s));
}

// One workgroup per (tile of kTok consecutive tokens of one sequence, block of 8192 channels); thread i handles
// channels 16 i .. 16 i + 15 of the block (a q / k head is dk / 16 consecutive threads, all in one wave) and slides
// the conv window (the previous 3 inputs of its channels) along the tile in registers, so each input row is read
// once per tile instead of four times.
constexpr int kTok = 8;
constexpr int kPrepThreads = 512;

__global__ __launch_bounds__(kPrepThreads, 4) void gdn_prep_kernel(PrepArgs p) {
  const int64_t ntile = (p.L + kTok - 1) / kTok;
  const int64_t s = blockIdx.x / ntile, t0 = (blockIdx.x % ntile) * kTok;
  const int64_t m_s = s * p.L;  // first token of the sequence
  const int tid = threadIdx.x;
  const int c0 = ((int)blockIdx.y * kPrepThreads + tid) * kChan;
  const bool on = c0 < p.C;
  const int64_t st = p.seq_state ? (int64_t)p.seq_state[s] : s;
  const bool st_ok = p.conv_in != nullptr && st >= 0 && st < p.n_states;
  const int kd = p.n_k * p.dk;
  const int G = p.dk / kChan;  // lanes per head (a power of two <= 64)
  const int tn = (int)min((int64_t)kTok, p.L - t0);
  // real tokens of the sequence (clamped into [0, L]); tokens at or past it are right pads
  const int64_t len = p.seq_len ? min(max((int64_t)p.seq_len[s], (int64_t)0), p.L) : p.L;

  // row r of full = [state (3 rows) ; the sequence's tokens]: full[r] = state row r (r < 3) or token r - 3, as 8
  // words of bf16 pairs (the window and the next row stay in this raw form: half the registers of fp32)
  auto load_full = [&](int64_t r, uint32_t (&x)[kChan / 2]) {
    const uint16_t* src = nullptr;
    if (r >= kConvTaps - 1) src = p.proj + (m_s + r - (kConvTaps - 1)) * p.ldp + c0;
    else if (st_ok) src = p.conv_in + (st * (kConvTaps - 1) + r) * p.C + c0;
    if (src) {
      const uint4 lo = *reinterpret_cast<const uint4*>(src), hi = *reinterpret_cast<const uint4*>(src + 8);
      x[0] = lo.x; x[1] = lo.y; x[2] = lo.z; x[3] = lo.w; x[4] = hi.x; x[5] = hi.y; x[6] = hi.z; x[7] = hi.w;
    } else {
#pragma unroll
      for (int i = 0; i < kChan / 2; ++i) x[i] = 0u;
    }
  };
  auto store_raw = [&](uint16_t* dst, const uint32_t (&x)[kChan / 2]) {
    *reinterpret_cast<uint4*>(dst) = make_uint4(x[0], x[1], x[2], x[3]);
    *reinterpret_cast<uint4*>(dst + 8) = make_uint4(x[4], x[5], x[6], x[7]);
  };
  // channel i of a raw row, as fp32
  auto chan = [](const uint32_t (&x)[kChan / 2], int i) {
    return __uint_as_float((i & 1) ? (x[i >> 1] & 0xffff0000u) : (x[i >> 1] << 16));
  };
  uint32_t wr[kChan * kConvTaps / 2];  // the conv taps of this thread's channels, bf16 pairs (channel i: 2 words)
  uint32_t win[kConvTaps - 1][kChan / 2];  // full rows t0 .. t0 + 2 (the inputs before token t0)
  if (on) {
#pragma unroll
    for (int i = 0; i < kChan * kConvTaps / 8; ++i)
      *reinterpret_cast<uint4*>(&wr[4 * i]) = *reinterpret_cast<const uint4*>(p.conv_w + (int64_t)c0 * kConvTaps + 8 * i);
#pragma unroll
    for (int j = 0; j < kConvTaps - 1; ++j) load_full(t0 + j, win[j]);
  }
  // the new conv state is the 3 rows of [state ; tokens] that end at the last real token (rows len .. len + 2):
  // the window after that token, or, for a sequence with no real token, the state's own window
  if (p.conv_out && on && len == 0 && t0 == 0) {
#pragma unroll
    for (int j = 0; j < kConvTaps - 1; ++j) store_raw(p.conv_out + (s * (kConvTaps - 1) + j) * p.C + c0, win[j]);
  }

  // the next token's input row is loaded one token ahead, so its latency overlaps this token's work
  uint32_t xn[kChan / 2];
  if (on && tn > 0) load_full(t0 + kConvTaps - 1, xn);
  for (int tt = 0; tt < tn; ++tt) {
    const int64_t t = t0 + tt, m = m_s + t;
    float y[kChan];
    if (on) {
      uint32_t x[kChan / 2];
#pragma unroll
      for (int i = 0; i < kChan / 2; ++i) x[i] = xn[i];
      if (tt + 1 < tn) load_full(t + kConvTaps, xn);
#pragma unroll
      for (int i = 0; i < kChan; ++i) {
        uint32_t w01 = wr[2 * i], w23 = wr[2 * i + 1];
        // keeps the float64 taps out of the registers between tokens (hoisted, 64 doubles would take 128 VGPRs)
        asm volatile("" : "+v"(w01), "+v"(w23));
        double acc = (double)__uint_as_float(w01 << 16) * (double)chan(win[0], i);
        acc += (double)__uint_as_float(w01 & 0xffff0000u) * (double)chan(win[1], i);
        acc += (double)__uint_as_float(w23 << 16) * (double)chan(win[2], i);
        acc += (double)__uint_as_float(w23 & 0xffff0000u) * (double)chan(x, i);
        y[i] = silu_bf16(bf((float)acc));
      }
#pragma unroll
      for (int i = 0; i < kChan / 2; ++i) {
        win[0][i] = win[1][i];
        win[1][i] = win[2][i];
        win[2][i] = x[i];
      }
      if (p.conv_out && t == len - 1) {
#pragma unroll
        for (int j = 0; j < kConvTaps - 1; ++j) store_raw(p.conv_out + (s * (kConvTaps - 1) + j) * p.C + c0, win[j]);
      }
    } else {
#pragma unroll
      for (int i = 0; i < kChan; ++i) y[i] = 0.0f;
    }
    // l2norm of the q and k heads: squares rounded to bf16, their exact sum rounded to bf16, + eps, rsqrt and the
    // product each rounded to bf16 (torch's bf16 arithmetic, with a correctly rounded rsqrt)
    const bool qk_chan = on && c0 < 2 * kd;
    double ss = 0.0;
    if (qk_chan) {
#pragma unroll
      for (int i = 0; i < kChan; ++i) ss += (double)bf(y[i] * y[i]);
    }
    for (int o = G / 2; o > 0; o >>= 1) ss += __shfl_xor(ss, o, OD_WAVE);
    if (qk_chan) {
      const float sb = bf((float)ss);
      const float den = bf(sb + 1e-6f);
      const float inv = bf((float)(1.0 / sqrt((double)den)));
#pragma unroll
      for (int i = 0; i < kChan; ++i) y[i] = bf(y[i] * inv);
      store16(p.qk + m * (int64_t)(2 * kd) + c0, y);
    } else if (on) {
      store16(p.v + m * (int64_t)(p.n_v * p.dv) + (c0 - 2 * kd), y);
    }
  }

  // gates of the tile's tokens (first channel block): thread i takes (token i / n_v, value head i % n_v). A right pad
  // gets beta = 0 and g = -0, what b = a = -inf give (sigmoid(-inf) = 0, softplus(-inf) = 0): the state passes
  // through it unchanged (e^g = 1, no write)
  for (int i = blockIdx.y == 0 ? tid : tn * p.n_v; i < tn * p.n_v; i += blockDim.x) {
    const int64_t m = m_s + t0 + i / p.n_v;
    const int hh = i % p.n_v;
    if (t0 + i / p.n_v >= len) {
      p.beta[m * p.n_v + hh] = 0.0f;
      p.g[m * p.n_v + hh] = -0.0f;
      continue;
    }
    const uint16_t* row = p.proj + m * p.ldp + p.C + (int64_t)p.n_v * p.dv;
    const float b = od_bf16_to_f32(row[hh]), a = od_bf16_to_f32(row[p.n_v + hh]);
    p.beta[m * p.n_v + hh] = od_sigmoid_bf16(b);
    const float e = (float)exp((double)od_bf16_to_f32(p.A_log[hh]));
    const float x = (float)((double)a + (double)od_bf16_to_f32(p.dt_bias[hh]));
    const float sp = x > 20.0f ? x : (float)log1p(exp((double)x));
    p.g[m * p.n_v + hh] = (float)(-((double)e * (double)sp));
  }

}

// ------------------------------------------------------------------------------------------------ recurrence
// One workgroup of 4 waves per (sequence, value head, 32 columns of the state); wave w owns columns 8 w .. 8 w + 7
// of those, lane l column l / 8 and rows 16 (l % 8) .. + 15 (dk = 128), 16 fp32 state values in registers. The
// columns of S evolve independently (column j only needs k, q, v_j, g, beta), so the waves never exchange anything;
// the 8 lanes of a column reduce their partial dot products with DPP.
//
// Per token the decay multiplies the whole state by one scalar, so the state is held as S = c S' with a scalar c per
// workgroup, and one pass over S' gives both dot products (e = e^g; c' = c e; kq = k . q~ with q~ = q / sqrt(dk)):
//   A = S'^T k, B = S'^T q~ ; kv = c' A ; delta = (v - kv) beta ; o = c' B + kq delta ; S' += k (delta / c') ; c = c'
// which is the reference's S <- S e^g ; kv = S^T k ; delta = (v - kv) beta ; S <- S + k delta^T ; o = S^T q~ with the
// decay folded into c (o = (e S + k delta^T)^T q~ = e S^T q~ + (k . q~) delta): three fmas per state value and token
// instead of a multiply and four fmas. When c' leaves [2^-64, 2^64] the state is renormalized (S' <- c' S', c' = 1),
// so delta / c' stays finite (a zero decay factor empties the state, as e^g = 0 does). The token inputs go through LDS in
// chunks of 16 tokens as fp32 (q pre-scaled, e^g and k . q~ computed once per token), the next chunk loaded into
// registers while the current one is computed; the outputs of a chunk leave through LDS in 16-byte stores.
constexpr int kRecThreads = 256;
constexpr int kRecCols = 32;   // state columns per workgroup
constexpr int kChunk = 16;     // tokens per staged chunk
constexpr int kDk = 128;
constexpr int kRowPad = 160;   // fp32 per staged k / q row: rows 16 g .. 16 g + 15 at 20 g (conflict-free b128 reads)

struct RecArgs {
  const uint16_t* qk;
  const uint16_t* v;
  const float* g;
  const float* beta;
  const float* init;
  const int32_t* seq_state;
  uint16_t* o;
  float* final_state;
  int64_t S, L, n_states;
  int n_k, n_v, dv;
};

struct RecStage {
  float q[kChunk][kRowPad];
  float k[kChunk][kRowPad];
  float v[kChunk][kRecCols];
  float4 tok[kChunk];  // (e^g, beta, k . q~, unused)
};

template <int CTRL>
__device__ __forceinline__ float dpp_add(float x) {
  return x + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}
// sum over the 8 lanes of an aligned group: quads, then the two quads of a half-row (row_half_mirror)
__device__ __forceinline__ float sum8(float x) {
  x = dpp_add<0xB1>(x);   // quad_perm [1,0,3,2]
  x = dpp_add<0x4E>(x);   // quad_perm [2,3,0,1]
  return dpp_add<0x141>(x);  // row_half_mirror: lane i of 8 adds lane 7 - i (the other quad's sum)
}
// sum over the 16 lanes of a DPP row
__device__ __forceinline__ float sum16(float x) {
  x = sum8(x);
  return dpp_add<0x140>(x);  // row_mirror: lane i of 16 adds lane 15 - i (the other half-row's sum)
}

__device__ __forceinline__ int rec_pos(int r) { return 20 * (r >> 4) + (r & 15); }

__global__ __launch_bounds__(kRecThreads) void gdn_recurrence_kernel(RecArgs p) {
  __shared__ __attribute__((aligned(16))) RecStage sm[2];
  __shared__ __attribute__((aligned(16))) uint16_t ob[kChunk][kRecCols];
  const int nblk = p.dv / kRecCols;
  const int64_t bid = blockIdx.x;
  const int cb = (int)(bid % nblk);
  const int h = (int)((bid / nblk) % p.n_v);
  const int64_t s = bid / ((int64_t)nblk * p.n_v);
  const int hk = h / (p.n_v / p.n_k);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int rg = lane & 7;                        // rows 16 rg .. 16 rg + 15
  const int cl = wave * 8 + (lane >> 3);          // column within the workgroup's 32
  const int col = cb * kRecCols + cl;             // column of the head's state
  const int64_t kd = (int64_t)p.n_k * kDk;
  const int64_t m0 = s * p.L;
  const int64_t ldv = (int64_t)p.n_v * p.dv;

  float S[16];
  float c = 1.0f;
  const int64_t st = p.seq_state ? (int64_t)p.seq_state[s] : s;
  if (p.init && st >= 0 && st < p.n_states) {
    const float* src = p.init + ((st * p.n_v + h) * kDk + 16 * rg) * p.dv + col;
#pragma unroll
    for (int r = 0; r < 16; ++r) S[r] = src[(int64_t)r * p.dv];
  } else {
#pragma unroll
    for (int r = 0; r < 16; ++r) S[r] = 0.0f;
  }
  const float qscale = (float)0.08838834764831845;  // fp32(1 / sqrt(128)), as the reference scales the fp32 query

  // chunk loads: thread i takes the 8-row pieces (token i / 16, part i % 16) of q and of k; threads 0..63 the 16-byte
  // pieces of the chunk's v block (16 tokens x 64 B), threads 64..79 g and 80..95 beta
  uint4 rq, rk, rv;
  float rgb = 0.0f;
  const int ptok = tid >> 4, part = tid & 15;
  auto gload = [&](int64_t t0) {
    const int64_t tt = t0 + ptok;
    const bool in = tt < p.L;
    const uint16_t* src = p.qk + (m0 + tt) * 2 * kd + (int64_t)hk * kDk + part * 8;
    rq = in ? *reinterpret_cast<const uint4*>(src) : make_uint4(0, 0, 0, 0);
    rk = in ? *reinterpret_cast<const uint4*>(src + kd) : make_uint4(0, 0, 0, 0);
    if (tid < 64) {
      const int64_t tv = t0 + (tid >> 2);
      rv = tv < p.L ? *reinterpret_cast<const uint4*>(p.v + (m0 + tv) * ldv + (int64_t)h * p.dv + cb * kRecCols +
                                                      (tid & 3) * 8)
                    : make_uint4(0, 0, 0, 0);
    } else if (tid < 96) {
      const int64_t tg = t0 + (tid & 15);
      rgb = tg < p.L ? (tid < 80 ? p.g : p.beta)[(m0 + tg) * p.n_v + h] : 0.0f;
    }
  };
  auto swrite = [&](int buf) {
    const uint32_t wq[4] = {rq.x, rq.y, rq.z, rq.w}, wk[4] = {rk.x, rk.y, rk.z, rk.w};
    float qf[8], kf[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      qf[2 * i] = __uint_as_float(wq[i] << 16) * qscale;
      qf[2 * i + 1] = __uint_as_float(wq[i] & 0xffff0000u) * qscale;
      kf[2 * i] = __uint_as_float(wk[i] << 16);
      kf[2 * i + 1] = __uint_as_float(wk[i] & 0xffff0000u);
    }
    float kq = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) kq = fmaf(kf[i], qf[i], kq);
    kq = sum16(kq);  // the 16 parts of a token are the 16 lanes of one DPP row
    const int pos = rec_pos(part * 8);
    float4* dq = reinterpret_cast<float4*>(&sm[buf].q[ptok][pos]);
    float4* dk = reinterpret_cast<float4*>(&sm[buf].k[ptok][pos]);
    dq[0] = make_float4(qf[0], qf[1], qf[2], qf[3]);
    dq[1] = make_float4(qf[4], qf[5], qf[6], qf[7]);
    dk[0] = make_float4(kf[0], kf[1], kf[2], kf[3]);
    dk[1] = make_float4(kf[4], kf[5], kf[6], kf[7]);
    if (part == 0) sm[buf].tok[ptok].z = kq;   // every lane of the row holds the full sum
    if (tid < 64) {
      const uint32_t wv[4] = {rv.x, rv.y, rv.z, rv.w};
      float4* dv = reinterpret_cast<float4*>(&sm[buf].v[tid >> 2][(tid & 3) * 8]);
      dv[0] = make_float4(__uint_as_float(wv[0] << 16), __uint_as_float(wv[0] & 0xffff0000u),
                          __uint_as_float(wv[1] << 16), __uint_as_float(wv[1] & 0xffff0000u));
      dv[1] = make_float4(__uint_as_float(wv[2] << 16), __uint_as_float(wv[2] & 0xffff0000u),
                          __uint_as_float(wv[3] << 16), __uint_as_float(wv[3] & 0xffff0000u));
    } else if (tid < 80) {
      sm[buf].tok[tid & 15].x = expf(rgb);
    } else if (tid < 96) {
      sm[buf].tok[tid & 15].y = rgb;
    }
  };
  auto ostore = [&](int64_t t0) {
    if (tid < 64) {
      const int64_t tt = t0 + (tid >> 2);
      if (tt < p.L)
        *reinterpret_cast<uint4*>(p.o + (m0 + tt) * ldv + (int64_t)h * p.dv + cb * kRecCols + (tid & 3) * 8) =
            *reinterpret_cast<const uint4*>(&ob[tid >> 2][(tid & 3) * 8]);
    }
  };

  const int64_t nchunk = (p.L + kChunk - 1) / kChunk;
  gload(0);
  swrite(0);
  __syncthreads();
  for (int64_t ch = 0; ch < nchunk; ++ch) {
    const int buf = (int)(ch & 1);
    const int64_t t0 = ch * kChunk;
    if (ch + 1 < nchunk) gload(t0 + kChunk);
    const int ntok = (int)min((int64_t)kChunk, p.L - t0);
    const RecStage& b = sm[buf];
    // token tt's inputs are read from LDS during token tt - 1 (software pipelined)
    float kf[16], qf[16], vv;
    float4 ti;
    auto lds_token = [&](int tt, float (&kd)[16], float (&qd)[16], float& vd, float4& td) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float4 a = *reinterpret_cast<const float4*>(&b.k[tt][20 * rg + 4 * i]);
        const float4 e = *reinterpret_cast<const float4*>(&b.q[tt][20 * rg + 4 * i]);
        kd[4 * i] = a.x, kd[4 * i + 1] = a.y, kd[4 * i + 2] = a.z, kd[4 * i + 3] = a.w;
        qd[4 * i] = e.x, qd[4 * i + 1] = e.y, qd[4 * i + 2] = e.z, qd[4 * i + 3] = e.w;
      }
      vd = b.v[tt][cl];
      td = b.tok[tt];
    };
    auto step = [&](int tt, const float (&kd)[16], const float (&qd)[16], float vd, float4 td) {
      float cn = c * td.x;
      if (cn < 0x1p-64f || cn > 0x1p64f) {  // renormalize (c is the same in every lane: a uniform branch)
#pragma unroll
        for (int r = 0; r < 16; ++r) S[r] *= cn;
        cn = 1.0f;
      }
      float a0 = 0.0f, a1 = 0.0f, b0 = 0.0f, b1 = 0.0f;
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        a0 = fmaf(S[r], kd[r], a0);
        b0 = fmaf(S[r], qd[r], b0);
        a1 = fmaf(S[r + 1], kd[r + 1], a1);
        b1 = fmaf(S[r + 1], qd[r + 1], b1);
      }
      const float A = sum8(a0 + a1), B = sum8(b0 + b1);
      const float delta = (vd - cn * A) * td.y;
      const float os = fmaf(cn, B, td.z * delta);
      const float dd = delta * __builtin_amdgcn_rcpf(cn);
#pragma unroll
      for (int r = 0; r < 16; ++r) S[r] = fmaf(kd[r], dd, S[r]);
      c = cn;
      if (rg == 0) ob[tt][cl] = od_f32_to_bf16(os);
    };
    // two register sets, alternating, so that no copy is needed between tokens
    float kn[16], qn[16], vn = 0.0f;
    float4 tn = make_float4(1.0f, 0.0f, 0.0f, 0.0f);
    if (ntok > 0) lds_token(0, kf, qf, vv, ti);
    for (int tt = 0; tt < ntok; tt += 2) {
      if (tt + 1 < ntok) lds_token(tt + 1, kn, qn, vn, tn);
      step(tt, kf, qf, vv, ti);
      if (tt + 1 < ntok) {
        if (tt + 2 < ntok) lds_token(tt + 2, kf, qf, vv, ti);
        step(tt + 1, kn, qn, vn, tn);
      }
    }
    __syncthreads();  // every wave is done with buffer buf ^ 1 (read in chunk ch - 1) and has written its outputs
    ostore(t0);
    if (ch + 1 < nchunk) swrite(buf ^ 1);
    __syncthreads();
  }
  if (p.final_state) {
    float* dst = p.final_state + ((s * p.n_v + h) * kDk + 16 * rg) * p.dv + col;
#pragma unroll
    for (int r = 0; r < 16; ++r) dst[(int64_t)r * p.dv] = c * S[r];
  }
}

// ------------------------------------------------------------------------------------------------ norm + quant
struct NormArgs {
  const uint16_t* o;
  const uint16_t* z;
  const uint16_t* w;
  const uint16_t* inv_s;
  int8_t* xq;
  float* sx;
  int64_t ldo, ldz, ldq;
  int n_v, dv;
  float eps;
  int vec_w;  // w and inv_s 16-byte aligned: a thread's 16 weights and scales come in two 16-byte loads each
};

// One workgroup per token; thread i handles values 16 i .. 16 i + 15 of the n_v dv outputs (a head is dv / 16
// consecutive threads in one wave).
__global__ __launch_bounds__(1024) void gdn_norm_quant_kernel(NormArgs p) {
  __shared__ uint32_t red[16];
  const int64_t m = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int V = p.n_v * p.dv;
  const int c0 = tid * kChan;
  const bool on = c0 < V;
  float o[kChan], z[kChan], wv[kChan], sv[kChan];
  if (on) {
    load16(p.o + m * p.ldo + c0, o);
    load16(p.z + m * p.ldz + c0, z);
    // the thread's 16 channels lie in one head (dv % 16 == 0): weights c0 % dv .. +15, scales c0 .. c0 + 15
    if (p.vec_w) {
      load16(p.w + c0 % p.dv, wv);
      if (p.inv_s) load16(p.inv_s + c0, sv);
    } else {
#pragma unroll
      for (int i = 0; i < kChan; ++i) {
        wv[i] = od_bf16_to_f32(p.w[(c0 + i) % p.dv]);
        if (p.inv_s) sv[i] = od_bf16_to_f32(p.inv_s[c0 + i]);
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < kChan; ++i) o[i] = z[i] = wv[i] = sv[i] = 0.0f;
  }
  double ss = 0.0;
#pragma unroll
  for (int i = 0; i < kChan; ++i) ss += (double)o[i] * (double)o[i];
  const int G = p.dv / kChan;
  for (int d = G / 2; d > 0; d >>= 1) ss += __shfl_xor(ss, d, OD_WAVE);
  const float r = od_rms_factor(ss, p.dv, p.eps);
  float y[kChan];
  uint32_t amax = 0;
#pragma unroll
  for (int i = 0; i < kChan; ++i) {
    const float hn = bf(o[i] * r);
    const float hw = bf(wv[i] * hn);
    float v = silu_mul_bf16(hw, z[i]);
    if (p.inv_s) v = bf(v * sv[i]);
    y[i] = on ? v : 0.0f;
    const uint32_t a = (__float_as_uint(y[i]) >> 16) & 0x7fffu;  // |bf16| bits: NaN patterns exceed every number
    amax = a > amax ? a : amax;
  }
  amax = od_wave_umax_dpp(amax);
  if (lane == 0) red[wave] = amax;
  __syncthreads();
  if (tid == 0) {
    uint32_t mx = 0;
    for (int w = 0; w < (int)(blockDim.x >> 6); ++w) mx = red[w] > mx ? red[w] : mx;
    red[0] = mx;
  }
  __syncthreads();
  const float scale = od_q8_scale(__uint_as_float(red[0] << 16));
  const float inv = 1.0f / scale;
  uint32_t wq[kChan / 4];
  od_q8_words<kChan>(y, scale, inv, wq);
  if (on) *reinterpret_cast<uint4*>(p.xq + m * p.ldq + c0) = make_uint4(wq[0], wq[1], wq[2], wq[3]);
  if (tid == 0) p.sx[m] = scale;
}

int threads_for(int64_t channels) {
  const int64_t t = (channels / kChan + 63) / 64 * 64;
  return (int)t;
}

bool pow2(int64_t x) { return x > 0 && (x & (x - 1)) == 0; }

}  // namespace

extern "C" int od_gdn_prep_ex(const uint16_t* proj, int64_t ldp, const uint16_t* conv_w, const uint16_t* conv_in,
                              const int32_t* seq_state, int64_t n_states, const int32_t* seq_len,
                              const uint16_t* A_log, const uint16_t* dt_bias, int64_t S, int64_t L, int64_t n_k,
                              int64_t n_v, int64_t dk, int64_t dv, uint16_t* qk, uint16_t* v, float* g, float* beta,
                              uint16_t* conv_out, od_stream_t stream) {
  if (S < 0 || L < 0 || n_k < 1 || n_v < 1 || dk < 1 || dv < 1 || n_states < 0) return OD_ERR_SHAPE;
  if (S == 0 || L == 0) return OD_OK;
  if (!proj || !conv_w || !A_log || !dt_bias || !qk || !v || !g || !beta) return OD_ERR_NULL;
  const int64_t C = 2 * n_k * dk + n_v * dv;
  if (n_v % n_k || dk % kChan || dv % kChan || !pow2(dk / kChan) || dk / kChan > 64 || C / kChan > 1024 ||
      n_v > C / kChan)
    return OD_ERR_UNSUPPORTED;
  if (ldp < C + n_v * dv + 2 * n_v) return OD_ERR_SHAPE;
  if (ldp % 8 || !od_aligned16(proj) || !od_aligned16(conv_w) || (conv_in && !od_aligned16(conv_in)) ||
      !od_aligned16(qk) || !od_aligned16(v) || (conv_out && !od_aligned16(conv_out)))
    return OD_ERR_ALIGN;
  if (S * L > 0x7fffffffll) return OD_ERR_SHAPE;
  PrepArgs p{proj, conv_w, conv_in, seq_state, A_log, dt_bias, qk, v, g, beta, conv_out, seq_len, ldp, S, L,
             n_states, (int)n_k, (int)n_v, (int)dk, (int)dv, (int)C};
  const int64_t tiles = S * ((L + kTok - 1) / kTok);
  const int64_t cblocks = (C / kChan + kPrepThreads - 1) / kPrepThreads;
  gdn_prep_kernel<<<dim3((unsigned)tiles, (unsigned)cblocks), dim3(min(threads_for(C), kPrepThreads)), 0,
                    (hipStream_t)stream>>>(p);
  return od_launch_status();
}

extern "C" int od_gdn_prep(const uint16_t* proj, int64_t ldp, const uint16_t* conv_w, const uint16_t* conv_in,
                           const int32_t* seq_state, int64_t n_states, const uint16_t* A_log, const uint16_t* dt_bias,
                           int64_t S, int64_t L, int64_t n_k, int64_t n_v, int64_t dk, int64_t dv, uint16_t* qk,
                           uint16_t* v, float* g, float* beta, uint16_t* conv_out, od_stream_t stream) {
  return od_gdn_prep_ex(proj, ldp, conv_w, conv_in, seq_state, n_states, nullptr, A_log, dt_bias, S, L, n_k, n_v, dk,
                        dv, qk, v, g, beta, conv_out, stream);
}

extern "C" int od_gdn_recurrence(const uint16_t* qk, const uint16_t* v, const float* g, const float* beta,
                                 const float* init, const int32_t* seq_state, int64_t n_states, int64_t S, int64_t L,
                                 int64_t n_k, int64_t n_v, int64_t dk, int64_t dv, uint16_t* o, float* final_state,
                                 od_stream_t stream) {
  if (S < 0 || L < 0 || n_k < 1 || n_v < 1 || n_states < 0) return OD_ERR_SHAPE;
  if (S == 0 || L == 0) {
    if (S > 0 && final_state) {
      // an empty continuation: the final state is the initial one (zeros without init) -- not supported here
      return OD_ERR_SHAPE;
    }
    return OD_OK;
  }
  if (!qk || !v || !g || !beta || !o) return OD_ERR_NULL;
  if (dk != kDk || dv % kRecCols || n_v % n_k) return OD_ERR_UNSUPPORTED;
  if (!od_aligned16(qk) || !od_aligned16(v) || !od_aligned16(o)) return OD_ERR_ALIGN;
  const int64_t blocks = S * n_v * (dv / kRecCols);
  if (blocks > 0x7fffffffll) return OD_ERR_SHAPE;
  RecArgs p{qk, v, g, beta, init, seq_state, o, final_state, S, L, n_states, (int)n_k, (int)n_v, (int)dv};
  gdn_recurrence_kernel<<<dim3((unsigned)blocks), dim3(kRecThreads), 0, (hipStream_t)stream>>>(p);
  return od_launch_status();
}

extern "C" int od_gdn_norm_quant(const uint16_t* o, int64_t ldo, const uint16_t* z, int64_t ldz, const uint16_t* w,
                                 const uint16_t* inv_s, float eps, int64_t M, int64_t n_v, int64_t dv, int8_t* xq,
                                 int64_t ldq, float* sx, od_stream_t stream) {
  if (M < 0 || n_v < 1 || dv < 1) return OD_ERR_SHAPE;
  if (M == 0) return OD_OK;
  if (!o || !z || !w || !xq || !sx) return OD_ERR_NULL;
  const int64_t V = n_v * dv;
  if (dv % kChan || !pow2(dv / kChan) || dv / kChan > 64 || V / kChan > 1024) return OD_ERR_UNSUPPORTED;
  if (ldo < V || ldz < V || ldq < V) return OD_ERR_SHAPE;
  if (ldo % 8 || ldz % 8 || ldq % 16 || !od_aligned16(o) || !od_aligned16(z) || !od_aligned16(xq)) return OD_ERR_ALIGN;
  if (M > 0x7fffffffll) return OD_ERR_SHAPE;
  NormArgs p{o, z, w, inv_s, xq, sx, ldo, ldz, ldq, (int)n_v, (int)dv, eps,
             od_aligned16(w) && (!inv_s || od_aligned16(inv_s)) ? 1 : 0};
  gdn_norm_quant_kernel<<<dim3((unsigned)M), dim3(threads_for(V)), 0, (hipStream_t)stream>>>(p);
  return od_launch_status();
}
