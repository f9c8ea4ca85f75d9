// Branched (Hydragen) option-row attention over an int8 shared state, for gfx950.
//
// Math (src/opendecider/prefix_attn.py:43-76, src/opendecider/wide_attention.py:13-67): every query of every
// option row attends (a) all valid keys of its state's prefix and (b) its own row's keys 0..i (causal); the two
// softmax parts are merged by log-sum-exp. Here both parts run through ONE online softmax (FlashAttention-2
// style): the prefix key blocks first, then the row's own keys as extra masked blocks. Merging partials by LSE and
// continuing the online softmax over the own keys are the same computation.
//
// Work decomposition. A "slot" is one query (option row, token, GQA head of the KV group). Grid =
// (slot tiles, Hkv, states); a workgroup of 4 waves owns 128 consecutive slots of one (state, KV head) and streams
// that state's int8 K/V once for all of them; a wave owns 32 slots.
//
// Layout trick. Scores are computed transposed, S^T = K Q^T, on V_MFMA_F32_32X32X16_F16 with the 32 keys of a key
// tile as rows and the wave's 32 slots as columns. In the MFMA result layout lane l holds slot l % 32, so the
// running max / sum / rescale of the online softmax are lane-local (plus one exchange with lane l ^ 32), and the
// probabilities already sit where the second MFMA, O^T += V^T P^T, wants its B operand: k-step m of the P.V
// product takes registers 8 (m % 2) .. +7 of key tile m / 2. The V tile is written to LDS transposed (V^T, d-major)
// with the key order inside every 16-key group permuted to match (bits 2 and 3 of the key index swapped).
//
// Numerics (all exact except the fp32 accumulation and the two fp16 roundings noted):
//  * int8 K/V values are converted to fp16 exactly (|q| <= 127) with the 0x6400 magic-number trick;
//  * the per-(token, head) fp32 K scale is folded into the scores: s = raw * ks[j] (+ -inf for masked keys);
//  * queries are bf16; each slot's query is multiplied by a power of two 2^e (exact) so that its absmax lies in
//    [2^14, 2^15) and converted to fp16 (exact: fp16 has more mantissa bits than bf16); the factor 2^-e is folded
//    with the softmax scale and log2(e) into one per-slot multiplier;
//  * the row's own bf16 K/V get one power-of-two factor per 32-key block in the same way;
//  * the per-key V scale is folded into the probabilities, P' = p * vs[j] / 2^E_b, rounded to fp16 (relative
//    error 2^-11), with E_b the exponent of the block's largest V scale so that P' lies in [0, 1]; the power of two
//    is carried in the rescale of the accumulator. P and V are therefore never rounded to bf16.
// Masked keys get a -inf score; a block with no visible key is an exact no-op for a slot; every row's arithmetic is
// independent of its position among the rows (fixed key order, no cross-slot reduction), so option order cannot
// change a result.
#include "od_common.h"

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;
constexpr int kWaves = 4;
constexpr int kSlotsPerTile = kWaves * 32;
constexpr int kBlockKeys = 64;  // prefix keys per block (2 key tiles of 32)
constexpr int kOwnKeys = 32;    // own keys per block (1 key tile)
constexpr float kLn2 = 0.693147180559945309f;
// Lazy rescaling. The running max of a slot only moves when a block raises its scaled scores by more than kSlack
// (log2 units), so p = exp2(s - m) <= 2^kSlack; the power-of-two frame E of the V scales (fv = vs / 2^E) only
// moves when a block's largest V scale leaves [2^(E - kFrame), 2^(E + kFrame)), so fv < 2^kFrame and
// P' = p fv < 2^15 stays inside fp16. The accumulator is rescaled only when either moves.
constexpr float kSlack = 8.0f;
constexpr int kFrame = 7;
constexpr int kNoFrame = -1000000;

struct AttnArgs {
  const uint16_t* q;
  const uint16_t* k_own;
  const uint16_t* v_own;
  const int8_t* kq;
  const float* ks;
  const int8_t* vq;
  const float* vs;
  const uint8_t* kvalid;
  const int32_t* row_start;
  uint16_t* out;
  float* lse;
  int64_t sqr, sqh, sqt, skr, skh, skt, svr, svh, svt, sor, soh, sot;
  int R, Hq, Hkv, t, Ns, T, cap, rep;
  float scale_log2;
  int nsplit;   // key-range splits (1: one pass writes out/lse)
  float* part;  // nsplit > 1: fp32 partials, o [nsplit][R][Hq][t][D] then lse [nsplit][R][Hq][t]
};

// Every array is 16-byte aligned so that fragment and scale accesses compile to single ds_read_b128 /
// ds_write_b128 instructions (without the alignment the compiler splits them into 4-byte pairs).
template <int D>
struct alignas(16) Smem {
  alignas(16) _Float16 k[2][kBlockKeys * D];   // [key][d], 16-byte chunks swizzled (k_off)
  alignas(16) _Float16 vt[2][D * kBlockKeys];  // [d][permuted key], 16-byte chunks swizzled (vt_off)
  alignas(16) float gk[2][kBlockKeys];         // score multiplier of key j (its K scale)
  alignas(16) float kb[2][kBlockKeys];         // 0, or -inf for a masked key
  alignas(16) float fv[2][kBlockKeys];         // V scale of key j divided by 2^E_b
  int eb[2];                                   // E_b
  int ef;                                      // the frame prefix_store gives the next block (kNoFrame: none yet)
  float red[2][kWaves];
};

// LDS swizzles. gfx950 LDS: reads see 64 4-byte banks (a 256-byte period) and serve 16 lanes of a ds_read_b128
// per cycle; writes go 128 bytes per cycle with a 128-byte bank period (8 lanes of a ds_write_b128, 16 lanes of a
// ds_write_b64). A fragment read has lanes 16g .. 16g+15 take 16 consecutive rows (keys of K, d of V^T) at one
// logical 16-byte chunk, so the chunk is XORed with a function of the row that gives those 16 rows 16 distinct
// bank quads:
//  * K, rows of 2D bytes (D/8 chunks): 128/D rows share a 256-byte period, XOR with (key / (128/D)) mod D/8;
//  * V^T, rows of 128 bytes (8 chunks), two rows per period: XOR with ((d >> 1) ^ (d >> 3)) & 7, which is a
//    bijection on any 8 consecutive even (or odd) d and also on {8 dg + e : dg = 8 consecutive values} for a
//    fixed e, which the transposing store needs (see vmap).
template <int D>
__device__ __forceinline__ int k_off(int key, int chunk) {
  return key * D + ((chunk ^ ((key / (128 / D)) & (D / 8 - 1))) << 3);
}
__device__ __forceinline__ int vt_off(int d, int chunk) {
  return d * kBlockKeys + ((chunk ^ (((d >> 1) ^ (d >> 3)) & 7)) << 3);
}

// Thread -> (d group dg of 8 d, key group kg of 4 keys) of the transposing V store. A thread writes 8 bytes (its
// 4 keys) into each of the V^T rows 8 dg .. 8 dg + 7. Lanes 16i .. 16i+15 form one ds_write_b64 bank cycle: bits
// 0..2 of the lane pick 8 consecutive dg (8 distinct chunks after the V^T swizzle) and bit 3 flips bit 1 of kg,
// which is the half of the 16-byte chunk the 4 keys occupy, so the 16 lanes write 16 distinct 8-byte slots.
// D = 128: 16 dg x 16 kg = 256 threads; D = 64: 8 dg x 16 kg = threads 0..127. kg < 8 <=> thread < D.
template <int D>
__device__ __forceinline__ void vmap(int tid, int& dg, int& kg) {
  const int lo = tid & 7, t3 = (tid >> 3) & 1, hi = tid >> 4;
  if constexpr (D == 128) {
    dg = lo | ((hi & 1) << 3);
    kg = (t3 << 1) | ((hi >> 1) & 1) | ((hi >> 2) << 2);
  } else {
    dg = lo;
    kg = (t3 << 1) | (hi & 1) | ((hi >> 1) << 2);
  }
}
// position of key j (0..63) inside its V^T row: bits 2 and 3 swapped
__device__ __forceinline__ int jj_of(int j) { return (j & ~12) | ((j & 4) << 1) | ((j & 8) >> 1); }

__device__ __forceinline__ half2v h2_bits(uint32_t u) { return __builtin_bit_cast(half2v, u); }
__device__ __forceinline__ uint32_t bits_h2(half2v h) { return __builtin_bit_cast(uint32_t, h); }

// 4 int8 (one dword) -> 4 exact fp16 (two dwords): byte u = q + 128 goes into the low mantissa of 1024 + u
// (fp16 0x6400 | u), then 1152 is subtracted (exact).
__device__ __forceinline__ void i8x4_to_h(uint32_t w, uint32_t& lo, uint32_t& hi) {
  const uint32_t u = w ^ 0x80808080u;
  const half2v bias = {(_Float16)1152.0f, (_Float16)1152.0f};
  lo = bits_h2(h2_bits(__builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) - bias);
  hi = bits_h2(h2_bits(__builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)) - bias);
}

__device__ __forceinline__ uint32_t pack_h2(float a, float b) {
  half2v h = {(_Float16)a, (_Float16)b};
  return bits_h2(h);
}

// exponent e with |x| < 2^e (x != 0); 0 for x == 0
__device__ __forceinline__ int exp_above(float amax) {
  int e = 0;
  if (amax > 0.0f) frexpf(amax, &e);
  return e;
}

// ---------------------------------------------------------------------------------------------- block loaders
// Prefix block (int8 state, keys j0 .. j0+63): registers first (issued before the previous block's compute), then
// converted into LDS buffer `buf`.
template <int D>
struct PrefixRegs {
  uint4 k[(kBlockKeys * D / 16 + kThreads - 1) / kThreads];
  uint2 v[4];
  float sc;   // thread < 64: K scale of key tid; 64 <= thread < 128: V scale of key tid - 64
  int ok;     // key valid (thread < 64)
};

template <int D>
__device__ __forceinline__ void prefix_load(const AttnArgs& p, int s, int g, int j0, PrefixRegs<D>& r) {
  const int tid = threadIdx.x;
  const int64_t head_base = ((int64_t)s * p.Hkv + g) * p.cap;
  constexpr int kChunks = kBlockKeys * D / 16;  // 16-byte int8 chunks per K block
  constexpr int kCpk = D / 16;                  // chunks per key
#pragma unroll
  for (int i = 0; i < (kChunks + kThreads - 1) / kThreads; ++i) {
    const int cid = i * kThreads + tid;
    const int key = cid / kCpk, c = cid % kCpk;
    r.k[i] = make_uint4(0, 0, 0, 0);
    if (cid < kChunks && j0 + key < p.T)
      r.k[i] = *reinterpret_cast<const uint4*>(p.kq + (head_base + j0 + key) * D + c * 16);
  }
  int dg, kg;
  vmap<D>(tid, dg, kg);
#pragma unroll
  for (int a = 0; a < 4; ++a) {
    const int key = 4 * kg + a;
    r.v[a] = make_uint2(0, 0);
    if (tid < 2 * D && j0 + key < p.T)
      r.v[a] = *reinterpret_cast<const uint2*>(p.vq + (head_base + j0 + key) * D + 8 * dg);
  }
  r.sc = 0.0f;
  r.ok = 0;
  // wave 0 reads the K scales and the key mask, wave 1 the V scales (the choice is wave-uniform, so the base
  // pointers stay scalar)
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  if (wv < 2) {
    const int j = j0 + (tid & 63);
    const float* sc = (wv == 0 ? p.ks : p.vs) + head_base;
    if (j < p.T) {
      r.sc = sc[j];
      r.ok = (wv == 0 && p.kvalid) ? (p.kvalid[(int64_t)s * p.T + j] != 0) : 1;
    }
  }
}

template <int D>
__device__ __forceinline__ void prefix_store(Smem<D>& sm, int buf, const PrefixRegs<D>& r) {
  const int tid = threadIdx.x;
  constexpr int kChunks = kBlockKeys * D / 16;
  constexpr int kCpk = D / 16;
#pragma unroll
  for (int i = 0; i < (kChunks + kThreads - 1) / kThreads; ++i) {
    const int cid = i * kThreads + tid;
    if (cid < kChunks) {
      const int key = cid / kCpk, c = cid % kCpk;
      // the 16 int8 values become two fp16 chunks, 2c and 2c + 1; lanes with bit 2 set store 2c + 1 first, so
      // that the 8 lanes of a ds_write_b128 bank cycle hit 8 distinct chunks of the 128-byte period
      const int flip = (tid >> 2) & 1;
      const uint32_t a0 = flip ? r.k[i].z : r.k[i].x, a1 = flip ? r.k[i].w : r.k[i].y;
      const uint32_t b0 = flip ? r.k[i].x : r.k[i].z, b1 = flip ? r.k[i].y : r.k[i].w;
      uint4 h0, h1;
      i8x4_to_h(a0, h0.x, h0.y);
      i8x4_to_h(a1, h0.z, h0.w);
      i8x4_to_h(b0, h1.x, h1.y);
      i8x4_to_h(b1, h1.z, h1.w);
      *reinterpret_cast<uint4*>(&sm.k[buf][k_off<D>(key, 2 * c + flip)]) = h0;
      *reinterpret_cast<uint4*>(&sm.k[buf][k_off<D>(key, 2 * c + 1 - flip)]) = h1;
    }
  }
  int dg, kg;
  vmap<D>(tid, dg, kg);
  if (tid < 2 * D) {
    // 4 keys x 8 bytes -> for each of the 8 d: the 4 keys' bytes (a 4x4 byte transpose per dword half)
    uint32_t cols[8];
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const uint32_t L0 = half ? r.v[0].y : r.v[0].x, L1 = half ? r.v[1].y : r.v[1].x;
      const uint32_t L2 = half ? r.v[2].y : r.v[2].x, L3 = half ? r.v[3].y : r.v[3].x;
      const uint32_t t0 = __builtin_amdgcn_perm(L1, L0, 0x05010400u);  // L0b0 L1b0 L0b1 L1b1
      const uint32_t t1 = __builtin_amdgcn_perm(L3, L2, 0x05010400u);  // L2b0 L3b0 L2b1 L3b1
      const uint32_t t2 = __builtin_amdgcn_perm(L1, L0, 0x07030602u);  // L0b2 L1b2 L0b3 L1b3
      const uint32_t t3 = __builtin_amdgcn_perm(L3, L2, 0x07030602u);
      cols[half * 4 + 0] = __builtin_amdgcn_perm(t1, t0, 0x05040100u);
      cols[half * 4 + 1] = __builtin_amdgcn_perm(t1, t0, 0x07060302u);
      cols[half * 4 + 2] = __builtin_amdgcn_perm(t3, t2, 0x05040100u);
      cols[half * 4 + 3] = __builtin_amdgcn_perm(t3, t2, 0x07060302u);
    }
    const int jj0 = jj_of(4 * kg);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int d = 8 * dg + e;
      uint2 hv;
      i8x4_to_h(cols[e], hv.x, hv.y);
      *reinterpret_cast<uint2*>(&sm.vt[buf][vt_off(d, jj0 >> 3) + (jj0 & 7)]) = hv;
    }
  }
  // scales: wave 0 -> K scales and masks, wave 1 -> V scales with the block's power-of-two normalisation
  if (tid < kBlockKeys) {
    sm.gk[buf][tid] = r.ok ? r.sc : 0.0f;
    sm.kb[buf][tid] = r.ok ? 0.0f : -INFINITY;
  } else if (tid < 2 * kBlockKeys) {
    // the block's V scales in the current power-of-two frame (kept in LDS; only wave 1 reads and writes it, and
    // the workgroup barrier between two blocks orders its accesses)
    // common case, two ballots: every scale below 2^(frame + kFrame) and one at least 2^(frame - kFrame - 1);
    // otherwise (rare, and the first block) the frame moves to the exponent of the block's largest scale
    int e_frame = sm.ef;
    const bool keep = e_frame != kNoFrame &&
                      __builtin_amdgcn_ballot_w64(r.sc >= ldexpf(1.0f, e_frame + kFrame)) == 0 &&
                      __builtin_amdgcn_ballot_w64(r.sc >= ldexpf(1.0f, e_frame - kFrame - 1)) != 0;
    if (!keep) e_frame = exp_above(od_wave_max(r.sc));
    sm.fv[buf][tid - kBlockKeys] = ldexpf(r.sc, -e_frame);
    if (tid == kBlockKeys) {
      sm.eb[buf] = e_frame;
      sm.ef = e_frame;
    }
  }
}

// ------------------------------------------------------------------------------------------------- compute
template <int D, int KT, bool OWN>
__device__ __forceinline__ void attend_block(const Smem<D>& sm, int buf, const half8 (&qf)[D / 16], float c_i,
                                             float& m_run, float& l_run, int& e_run, v16f (&o)[D / 32], int own_row,
                                             int own_j0, int slot_row, int slot_tok) {
  const int lane = threadIdx.x & 63;
  const int h = lane >> 5, col = lane & 31;
  v16f s[KT];
#pragma unroll
  for (int kt = 0; kt < KT; ++kt) {
    s[kt] = v16f{0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
      const half8 a = *reinterpret_cast<const half8*>(&sm.k[buf][k_off<D>(kt * 32 + col, ks * 2 + h)]);
      s[kt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qf[ks], s[kt], 0, 0, 0);
    }
  }
  // scores of this lane's slot: key = kt*32 + 8*(r/4) + 4*h + r%4
  float mloc = -INFINITY;
#pragma unroll
  for (int kt = 0; kt < KT; ++kt) {
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      const int key0 = kt * 32 + 8 * r4 + 4 * h;
      const float4 g4 = *reinterpret_cast<const float4*>(&sm.gk[buf][key0]);
      const float4 b4 = *reinterpret_cast<const float4*>(&sm.kb[buf][key0]);
      const float gg[4] = {g4.x, g4.y, g4.z, g4.w}, bb[4] = {b4.x, b4.y, b4.z, b4.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float y = fmaf(s[kt][4 * r4 + e], gg[e], bb[e]);
        if (OWN && !(slot_row == own_row && own_j0 + key0 + e <= slot_tok)) y = -INFINITY;
        s[kt][4 * r4 + e] = y;
        mloc = fmaxf(mloc, y);
      }
    }
  }
  mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
  const float mc = mloc * c_i;
  const int eb = sm.eb[buf];
  // rescale (wave-uniform branch) only if some slot's max grows by more than kSlack or the V frame moved. Each slot
  // moves its own max only on its own condition (the others get alpha = exp2(0) = 1), so a slot's arithmetic does
  // not depend on which slots share its wave and option order cannot change a result.
  const bool grow = mc > m_run + kSlack;
  if (__builtin_amdgcn_ballot_w64(grow) != 0 || eb != e_run) {
    const float m_new = grow ? mc : m_run;
    const float alpha = __builtin_amdgcn_exp2f(m_run - (m_new == -INFINITY ? 0.0f : m_new));
    const float rs = ldexpf(alpha, e_run - eb);
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[dt][r] *= rs;
    l_run *= alpha;
    m_run = m_new;
    e_run = eb;
  }
  const float m_safe = m_run == -INFINITY ? 0.0f : m_run;
  float psum = 0.0f;
  half8 pb[2 * KT];
#pragma unroll
  for (int kt = 0; kt < KT; ++kt) {
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      const int key0 = kt * 32 + 8 * r4 + 4 * h;
      const float4 f4 = *reinterpret_cast<const float4*>(&sm.fv[buf][key0]);
      const float ff[4] = {f4.x, f4.y, f4.z, f4.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = 4 * r4 + e;
        const float pr = __builtin_amdgcn_exp2f(fmaf(s[kt][r], c_i, -m_safe));
        psum += pr;
        pb[kt * 2 + (r >> 3)][r & 7] = (_Float16)(pr * ff[e]);
      }
    }
  }
  psum += __shfl_xor(psum, 32, 64);
  l_run += psum;
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt) {
#pragma unroll
    for (int m = 0; m < 2 * KT; ++m) {
      const half8 a = *reinterpret_cast<const half8*>(&sm.vt[buf][vt_off(dt * 32 + col, 2 * m + h)]);
      o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pb[m], o[dt], 0, 0, 0);
    }
  }
}

// Workgroup max of two values (every thread gets both).
__device__ __forceinline__ void wg_max2(float (&red)[2][kWaves], float& a, float& b) {
  a = od_wave_max(a);
  b = od_wave_max(b);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    red[0][w] = a;
    red[1][w] = b;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kWaves; ++i) {
    a = fmaxf(a, red[0][i]);
    b = fmaxf(b, red[1][i]);
  }
}

// Own keys j0 .. j0+31 of option row `row` (bf16) into LDS buffer 0, scaled by powers of two into fp16.
template <int D>
__device__ __forceinline__ void own_stage(const AttnArgs& p, Smem<D>& sm, int row, int g, int j0) {
  const int tid = threadIdx.x;
  const int n_keys = min(kOwnKeys, p.t - j0);
  const uint16_t* kb = p.k_own + (int64_t)row * p.skr + (int64_t)g * p.skh;
  const uint16_t* vb = p.v_own + (int64_t)row * p.svr + (int64_t)g * p.svh;
  constexpr int kCpk = D / 8;                 // 8-value chunks per key
  constexpr int kChunks = kOwnKeys * kCpk;    // K chunks of the block
  constexpr int kKIt = (kChunks + kThreads - 1) / kThreads;
  uint4 kr[kKIt];
  float ka = 0.0f, va = 0.0f;
#pragma unroll
  for (int i = 0; i < kKIt; ++i) {
    const int cid = i * kThreads + tid;
    const int key = cid / kCpk, c = cid % kCpk;
    kr[i] = make_uint4(0, 0, 0, 0);
    if (cid < kChunks && key < n_keys) kr[i] = *reinterpret_cast<const uint4*>(kb + (int64_t)(j0 + key) * p.skt + 8 * c);
    const uint32_t w4[4] = {kr[i].x, kr[i].y, kr[i].z, kr[i].w};
#pragma unroll
    for (int e = 0; e < 4; ++e)
      ka = fmaxf(ka, fmaxf(fabsf(__uint_as_float(w4[e] << 16)), fabsf(__uint_as_float(w4[e] & 0xffff0000u))));
  }
  // V: a thread takes 4 keys x 8 d (kOwnKeys / 4 key groups x D / 8 d groups, threads 0 .. D - 1)
  int dg, kg;
  vmap<D>(tid, dg, kg);
  const bool vact = tid < D;
  uint4 vr[4];
#pragma unroll
  for (int a = 0; a < 4; ++a) {
    const int key = 4 * kg + a;
    vr[a] = make_uint4(0, 0, 0, 0);
    if (vact && key < n_keys) vr[a] = *reinterpret_cast<const uint4*>(vb + (int64_t)(j0 + key) * p.svt + 8 * dg);
    const uint32_t w4[4] = {vr[a].x, vr[a].y, vr[a].z, vr[a].w};
#pragma unroll
    for (int e = 0; e < 4; ++e)
      va = fmaxf(va, fmaxf(fabsf(__uint_as_float(w4[e] << 16)), fabsf(__uint_as_float(w4[e] & 0xffff0000u))));
  }
  wg_max2(sm.red, ka, va);
  const int ek = 15 - exp_above(ka), ev = 15 - exp_above(va);  // |x| 2^e < 2^15
#pragma unroll
  for (int i = 0; i < kKIt; ++i) {
    const int cid = i * kThreads + tid;
    if (cid < kChunks) {
      const int key = cid / kCpk, c = cid % kCpk;
      const uint32_t w4[4] = {kr[i].x, kr[i].y, kr[i].z, kr[i].w};
      uint4 hk;
      uint32_t* ho = &hk.x;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        ho[e] = pack_h2(ldexpf(__uint_as_float(w4[e] << 16), ek), ldexpf(__uint_as_float(w4[e] & 0xffff0000u), ek));
      *reinterpret_cast<uint4*>(&sm.k[0][k_off<D>(key, c)]) = hk;
    }
  }
  if (vact) {
    const int jj0 = jj_of(4 * kg);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float vals[4];
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const uint32_t w4[4] = {vr[a].x, vr[a].y, vr[a].z, vr[a].w};
        const uint32_t wd = w4[e >> 1];
        vals[a] = ldexpf(__uint_as_float((e & 1) ? (wd & 0xffff0000u) : (wd << 16)), ev);
      }
      uint2 hv = make_uint2(pack_h2(vals[0], vals[1]), pack_h2(vals[2], vals[3]));
      *reinterpret_cast<uint2*>(&sm.vt[0][vt_off(8 * dg + e, jj0 >> 3) + (jj0 & 7)]) = hv;
    }
  }
  if (tid < kOwnKeys) {
    const bool ok = tid < n_keys;
    sm.gk[0][tid] = ok ? ldexpf(1.0f, -ek) : 0.0f;
    sm.kb[0][tid] = ok ? 0.0f : -INFINITY;
    // V' = V 2^ev, so the block's frame is -ev with fv = 1. (Not the running frame: which frame the accumulator
    // is in when a row's own block comes depends on the rows before it in the tile, and a P' that is an fp16
    // subnormal in one frame and normal in another would round differently, breaking option-order invariance.)
    sm.fv[0][tid] = 1.0f;
    if (tid == 0) sm.eb[0] = -ev;
  }
}

template <int D>
__global__ __launch_bounds__(kThreads, 2) void branched_attn_kernel(AttnArgs p) {
  __shared__ Smem<D> sm;
  const int s = blockIdx.z / p.nsplit, sp = blockIdx.z % p.nsplit, g = blockIdx.y;
  const int row0 = p.row_start ? p.row_start[s] : 0;
  const int nrows = p.row_start ? p.row_start[s + 1] - row0 : p.R;
  const int per_row = p.t * p.rep;
  const int nslots = nrows * per_row;
  const int slot_base = blockIdx.x * kSlotsPerTile;
  if (slot_base >= nslots) return;  // uniform over the workgroup

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int h = lane >> 5, col = lane & 31;
  const int z = slot_base + wave * 32 + col;
  const bool slot_ok = z < nslots;
  int slot_row = -1, slot_tok = 0, slot_head = 0;
  if (slot_ok) {
    const int rl = z / per_row, rem = z - rl * per_row;
    slot_row = row0 + rl;
    slot_tok = rem / p.rep;
    slot_head = g * p.rep + rem % p.rep;
  }

  // query fragments: lane holds Q[slot][ks*16 + 8h .. +8] for ks = 0 .. D/16-1, scaled by 2^eq into fp16
  half8 qf[D / 16];
  float c_i;  // per-slot multiplier: softmax scale * log2(e) * 2^-eq
  {
    uint4 raw[D / 16];
    float qa = 0.0f;
    const uint16_t* qp = p.q + (int64_t)slot_row * p.sqr + (int64_t)slot_head * p.sqh + (int64_t)slot_tok * p.sqt;
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
      raw[ks] = slot_ok ? *reinterpret_cast<const uint4*>(qp + ks * 16 + 8 * h) : make_uint4(0, 0, 0, 0);
      const uint32_t w4[4] = {raw[ks].x, raw[ks].y, raw[ks].z, raw[ks].w};
#pragma unroll
      for (int e = 0; e < 4; ++e)
        qa = fmaxf(qa, fmaxf(fabsf(__uint_as_float(w4[e] << 16)), fabsf(__uint_as_float(w4[e] & 0xffff0000u))));
    }
    qa = fmaxf(qa, __shfl_xor(qa, 32, 64));
    const int eq = 15 - exp_above(qa);
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
      const uint32_t w4[4] = {raw[ks].x, raw[ks].y, raw[ks].z, raw[ks].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        qf[ks][2 * e] = (_Float16)ldexpf(__uint_as_float(w4[e] << 16), eq);
        qf[ks][2 * e + 1] = (_Float16)ldexpf(__uint_as_float(w4[e] & 0xffff0000u), eq);
      }
    }
    c_i = ldexpf(p.scale_log2, -eq);
  }

  float m_run = -INFINITY, l_run = 0.0f;
  int e_run = 0;  // the V-scale frame the accumulator is in (follows the blocks' frames)
  if (threadIdx.x == kBlockKeys) sm.ef = kNoFrame;  // read and written by this wave only (prefix_store)
  v16f o[D / 32];
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt) o[dt] = v16f{0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};

  // ---- prefix: the state's int8 K/V, 64 keys per block, double buffered; split sp of nsplit takes the blocks
  // [sp * bps, (sp + 1) * bps)
  const int nb_all = (p.T + kBlockKeys - 1) / kBlockKeys;
  const int bps = (nb_all + p.nsplit - 1) / p.nsplit;
  const int b_lo = min(nb_all, sp * bps), b_hi = min(nb_all, b_lo + bps);
  if (b_hi > b_lo) {
    PrefixRegs<D> pr;
    prefix_load<D>(p, s, g, b_lo * kBlockKeys, pr);
    prefix_store<D>(sm, 0, pr);
    __syncthreads();
    for (int b = b_lo; b < b_hi; ++b) {
      const int cur = (b - b_lo) & 1;
      if (b + 1 < b_hi) prefix_load<D>(p, s, g, (b + 1) * kBlockKeys, pr);
      attend_block<D, 2, false>(sm, cur, qf, c_i, m_run, l_run, e_run, o, 0, 0, slot_row, slot_tok);
      if (b + 1 < b_hi) prefix_store<D>(sm, cur ^ 1, pr);
      __syncthreads();
    }
  }

  // ---- own keys (the last split): every option row that has a slot in this tile, 32 keys per block
  const int last = min(slot_base + kSlotsPerTile, nslots) - 1;
  const int r_lo = row0 + slot_base / per_row, r_hi = sp == p.nsplit - 1 ? row0 + last / per_row : r_lo - 1;
  for (int row = r_lo; row <= r_hi; ++row) {
    for (int j0 = 0; j0 < p.t; j0 += kOwnKeys) {
      __syncthreads();  // LDS buffer 0 free
      own_stage<D>(p, sm, row, g, j0);
      __syncthreads();
      attend_block<D, 1, true>(sm, 0, qf, c_i, m_run, l_run, e_run, o, row, j0, slot_row, slot_tok);
    }
  }

  if (!slot_ok) return;
  // ---- epilogue: out = O 2^E / l (bf16), lse = (m + log2 l) ln 2
  const float inv = l_run > 0.0f ? ldexpf(1.0f / l_run, e_run) : 0.0f;
  const float lse_v = l_run > 0.0f ? (m_run + __log2f(l_run)) * kLn2 : -INFINITY;
  const int64_t slot_idx = ((int64_t)slot_row * p.Hq + slot_head) * p.t + slot_tok;
  if (p.nsplit > 1) {
    // this split's normalized fp32 partial and its LSE, merged by od_attn_combine
    const int64_t nsl = (int64_t)p.R * p.Hq * p.t;
    float* po = p.part + ((int64_t)sp * nsl + slot_idx) * D;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4)
        *reinterpret_cast<float4*>(po + dt * 32 + 8 * r4 + 4 * h) =
            make_float4(o[dt][4 * r4] * inv, o[dt][4 * r4 + 1] * inv, o[dt][4 * r4 + 2] * inv,
                        o[dt][4 * r4 + 3] * inv);
    if (h == 0) p.part[(int64_t)p.nsplit * nsl * D + (int64_t)sp * nsl + slot_idx] = lse_v;
    return;
  }
  uint16_t* op = p.out + (int64_t)slot_row * p.sor + (int64_t)slot_head * p.soh + (int64_t)slot_tok * p.sot;
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt) {
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      const int d0 = dt * 32 + 8 * r4 + 4 * h;
      const uint32_t lo = (uint32_t)od_f32_to_bf16(o[dt][4 * r4] * inv) |
                          ((uint32_t)od_f32_to_bf16(o[dt][4 * r4 + 1] * inv) << 16);
      const uint32_t hi = (uint32_t)od_f32_to_bf16(o[dt][4 * r4 + 2] * inv) |
                          ((uint32_t)od_f32_to_bf16(o[dt][4 * r4 + 3] * inv) << 16);
      *reinterpret_cast<uint2*>(op + d0) = make_uint2(lo, hi);
    }
  }
  if (p.lse && h == 0) p.lse[slot_idx] = lse_v;
}

// LSE merge of the key-range splits (prefix_attn.py:74-76 generalised to n parts): M = max_s lse_s,
// w_s = exp(lse_s - M), out = sum_s w_s o_s / sum_s w_s (bf16), lse = M + log(sum_s w_s); no visible key in any
// split -> 0 and -inf. One thread per (slot, 8 values of d).
template <int D>
__global__ __launch_bounds__(256) void combine_kernel(AttnArgs p) {
  const int64_t nsl = (int64_t)p.R * p.Hq * p.t;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t slot = gid / (D / 8);
  const int d0 = (int)(gid % (D / 8)) * 8;
  if (slot >= nsl) return;
  const float* lse_p = p.part + (int64_t)p.nsplit * nsl * D;
  float M = -INFINITY;
  for (int sp = 0; sp < p.nsplit; ++sp) M = fmaxf(M, lse_p[sp * nsl + slot]);
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  float wsum = 0.0f;
  if (M != -INFINITY) {
    for (int sp = 0; sp < p.nsplit; ++sp) {
      const float l = lse_p[sp * nsl + slot];
      if (l == -INFINITY) continue;
      const float w = __expf(l - M);
      wsum += w;
      const float4* po = reinterpret_cast<const float4*>(p.part + (sp * nsl + slot) * D + d0);
      const float4 a = po[0], b = po[1];
      acc[0] += w * a.x; acc[1] += w * a.y; acc[2] += w * a.z; acc[3] += w * a.w;
      acc[4] += w * b.x; acc[5] += w * b.y; acc[6] += w * b.z; acc[7] += w * b.w;
    }
  }
  const int row = (int)(slot / ((int64_t)p.Hq * p.t)), rem = (int)(slot % ((int64_t)p.Hq * p.t));
  const int head = rem / p.t, tok = rem % p.t;
  const float inv = wsum > 0.0f ? 1.0f / wsum : 0.0f;
  uint32_t w4[4];
#pragma unroll
  for (int e = 0; e < 4; ++e)
    w4[e] = (uint32_t)od_f32_to_bf16(acc[2 * e] * inv) | ((uint32_t)od_f32_to_bf16(acc[2 * e + 1] * inv) << 16);
  uint16_t* op = p.out + (int64_t)row * p.sor + (int64_t)head * p.soh + (int64_t)tok * p.sot + d0;
  *reinterpret_cast<uint2*>(op) = make_uint2(w4[0], w4[1]);
  *reinterpret_cast<uint2*>(op + 4) = make_uint2(w4[2], w4[3]);
  if (p.lse && d0 == 0) p.lse[slot] = wsum > 0.0f ? M + __logf(wsum) : -INFINITY;
}

}  // namespace

namespace {

int branched_launch(const uint16_t* q, int64_t sqr, int64_t sqh, int64_t sqt, const uint16_t* k_own, int64_t skr,
                    int64_t skh, int64_t skt, const uint16_t* v_own, int64_t svr, int64_t svh, int64_t svt,
                    const int8_t* kq, const float* ks, const int8_t* vq, const float* vs, const uint8_t* kvalid,
                    const int32_t* row_start, int64_t max_rows, uint16_t* out, int64_t sor, int64_t soh, int64_t sot,
                    float* lse, int64_t R, int64_t Hq, int64_t Hkv, int64_t t, int64_t D, int64_t Ns, int64_t T,
                    int64_t cap, float scale, int64_t nsplit, float* ws, int64_t ws_floats, od_stream_t stream) {
  if (R < 0 || Hq < 1 || Hkv < 1 || t < 1 || Ns < 1 || T < 0 || cap < T || max_rows < 0) return OD_ERR_SHAPE;
  if (Hq % Hkv) return OD_ERR_UNSUPPORTED;
  if (D != 64 && D != 128) return OD_ERR_UNSUPPORTED;
  if (t > 256) return OD_ERR_UNSUPPORTED;
  if (!row_start && Ns != 1) return OD_ERR_SHAPE;
  if (nsplit < 1 || nsplit > 256) return OD_ERR_SHAPE;
  if (!row_start) max_rows = R;
  if (R == 0 || max_rows == 0) return OD_OK;
  if (!q || !k_own || !v_own || !out || (T > 0 && (!kq || !ks || !vq || !vs))) return OD_ERR_NULL;
  if (nsplit > 1) {
    if (!ws) return OD_ERR_NULL;
    if (ws_floats < nsplit * R * Hq * t * (D + 1)) return OD_ERR_SHAPE;
    if (!od_aligned16(ws)) return OD_ERR_ALIGN;
  }
  const int64_t strides[] = {sqr, sqh, sqt, skr, skh, skt, svr, svh, svt};
  for (int64_t st : strides)
    if (st < 0 || st % 8) return OD_ERR_ALIGN;
  if (sor < 0 || soh < 0 || sot < 0 || sor % 4 || soh % 4 || sot % 4) return OD_ERR_ALIGN;
  if (!od_aligned16(q) || !od_aligned16(k_own) || !od_aligned16(v_own) || (((uintptr_t)out) & 7u)) return OD_ERR_ALIGN;
  if (T > 0 && (!od_aligned16(kq) || !od_aligned16(vq))) return OD_ERR_ALIGN;
  const int64_t rep = Hq / Hkv;
  const int64_t tiles = (max_rows * t * rep + kSlotsPerTile - 1) / kSlotsPerTile;
  if (tiles > 0x7fffffff || Hkv > 65535 || Ns * nsplit > 65535 || R * t * rep > 0x7fffffff ||
      cap * Hkv * Ns * D > (1ll << 40) || nsplit * R * Hq * t * (D + 1) > (1ll << 40))
    return OD_ERR_SHAPE;
  AttnArgs a{q, k_own, v_own, kq, ks, vq, vs, kvalid, row_start, out, lse, sqr, sqh, sqt, skr, skh, skt, svr, svh,
             svt, sor, soh, sot, (int)R, (int)Hq, (int)Hkv, (int)t, (int)Ns, (int)T, (int)cap, (int)rep,
             scale * 1.4426950408889634f, (int)nsplit, nsplit > 1 ? ws : nullptr};
  dim3 grid((unsigned)tiles, (unsigned)Hkv, (unsigned)(Ns * nsplit)), block(kThreads);
  hipStream_t st = (hipStream_t)stream;
  if (D == 128) {
    branched_attn_kernel<128><<<grid, block, 0, st>>>(a);
  } else {
    branched_attn_kernel<64><<<grid, block, 0, st>>>(a);
  }
  if (nsplit > 1) {
    const int rc = od_launch_status();
    if (rc != OD_OK) return rc;
    const int64_t threads = R * Hq * t * (D / 8);
    const unsigned blocks = (unsigned)((threads + 255) / 256);
    if (D == 128) {
      combine_kernel<128><<<blocks, 256, 0, st>>>(a);
    } else {
      combine_kernel<64><<<blocks, 256, 0, st>>>(a);
    }
  }
  return od_launch_status();
}

}  // namespace

extern "C" int od_branched_attn(const uint16_t* q, int64_t sqr, int64_t sqh, int64_t sqt, const uint16_t* k_own,
                                int64_t skr, int64_t skh, int64_t skt, const uint16_t* v_own, int64_t svr,
                                int64_t svh, int64_t svt, const int8_t* kq, const float* ks, const int8_t* vq,
                                const float* vs, const uint8_t* kvalid, const int32_t* row_start, int64_t max_rows,
                                uint16_t* out, int64_t sor, int64_t soh, int64_t sot, float* lse, int64_t R,
                                int64_t Hq, int64_t Hkv, int64_t t, int64_t D, int64_t Ns, int64_t T, int64_t cap,
                                float scale, od_stream_t stream) {
  return branched_launch(q, sqr, sqh, sqt, k_own, skr, skh, skt, v_own, svr, svh, svt, kq, ks, vq, vs, kvalid,
                         row_start, max_rows, out, sor, soh, sot, lse, R, Hq, Hkv, t, D, Ns, T, cap, scale, 1, nullptr,
                         0, stream);
}

extern "C" int od_branched_attn_split(const uint16_t* q, int64_t sqr, int64_t sqh, int64_t sqt, const uint16_t* k_own,
                                      int64_t skr, int64_t skh, int64_t skt, const uint16_t* v_own, int64_t svr,
                                      int64_t svh, int64_t svt, const int8_t* kq, const float* ks, const int8_t* vq,
                                      const float* vs, const uint8_t* kvalid, const int32_t* row_start,
                                      int64_t max_rows, uint16_t* out, int64_t sor, int64_t soh, int64_t sot,
                                      float* lse, int64_t R, int64_t Hq, int64_t Hkv, int64_t t, int64_t D, int64_t Ns,
                                      int64_t T, int64_t cap, float scale, int64_t nsplit, float* ws,
                                      int64_t ws_floats, od_stream_t stream) {
  return branched_launch(q, sqr, sqh, sqt, k_own, skr, skh, skt, v_own, svr, svh, svt, kq, ks, vq, vs, kvalid,
                         row_start, max_rows, out, sor, soh, sot, lse, R, Hq, Hkv, t, D, Ns, T, cap, scale, nsplit, ws,
                         ws_floats, stream);
}
