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
// that state's K/V once for all of them; a wave owns 32 slots.
//
// State blocks. The state's keys go in blocks of 64. A block is consumed from LDS as a "block image": its keys as
// exact bf16 integers with their score multipliers beside them, its values in fp16 with the per-key scales folded in,
// both in the swizzled layout the fragment reads want, a -inf bias row for masked keys and the block constants (V
// exponent, has-a-masked-key). Two paths build it: od_attn_stage writes every block's image to memory once per
// state (then each workgroup copies images straight into LDS with global_load_lds and converts nothing), and
// od_branched_attn converts the int8 blocks itself in every workgroup. Both produce the same bytes, so both give
// bit-identical results; the host takes the staged path when a (state, KV head) has enough slot tiles to share the
// images.
//
// Layout trick. Scores are computed transposed, S^T = K Q^T, on V_MFMA_F32_32X32X16_BF16 with the 32 keys of a key
// tile as rows and the wave's 32 slots as columns. In the MFMA result layout lane l holds slot l % 32, so the
// running max / sum / rescale of the online softmax are lane-local (plus one exchange with lane l ^ 32), and the
// probabilities already sit where the second MFMA, O^T += V^T P^T on V_MFMA_F32_32X32X16_F16, wants its B operand:
// k-step m of the P.V product takes registers 8 (m % 2) .. +7 of key tile m / 2. The V tile is stored transposed
// (V^T, d-major) with the key order inside every 16-key group permuted to match (bits 2 and 3 of the key index
// swapped).
//
// Numerics (fp32 accumulation; the roundings noted are the only others):
//  * the state's int8 K/V are dequantized in one of two ways (the `dq` argument):
//    - OD_DEQUANT_BF16, the reference's materialize (quant.py:45, prefix_attn.py:145-149): K' = bf16(q bf16(ks_j))
//      and V' = bf16(q bf16(vs_j)), each product rounded once to bf16. K' goes to the score MFMAs as it is (the
//      bf16 products with the queries are exact) and the score of key j is raw_j * scale log2(e); V' (8 significant
//      bits) is stored as fp16 V' 2^-eb, exact;
//    - OD_DEQUANT_FP32, the exact q * s: a state key's int8 values are exact bf16 integers and the score of key j
//      is raw_j * gk_j with gk_j = ks_j scale log2(e) (one rounding in gk_j, one in the product); a state value
//      becomes fp16(q vs_j 2^-eb), one rounding;
//    eb is the block's V exponent; the accumulator carries one power-of-two frame, moved lazily (a state block in
//    a frame up to kFrameSlack below it enters with its probabilities times 2^(eb - frame), exact while those stay
//    normal fp16);
//  * queries are used as they are (bf16), and so are the row's own bf16 keys, with the multiplier scale log2(e);
//  * the row's own bf16 values get one power-of-two factor per 32-key block and are converted to fp16;
//  * probabilities p = exp2(y) <= 2^8 are rounded to fp16 for the P.V product; their sum is taken unrounded.
// Masked keys get a -inf score; a block with no visible key is an exact no-op for a slot; every row's arithmetic is
// independent of its position among the rows (fixed key order, no cross-slot reduction), so option order cannot
// change a result.
#include <mutex>

#include "od_common.h"

// The split workspace of od_branched_attn_split_noalloc: a static device array (one copy per GPU, alive until the
// process ends). Host code never passes this name to a kernel or a copy (on the host it is a stand-in, not a device
// address): scratch_ptr() resolves each device's copy with hipGetSymbolAddress once and the kernels take that
// pointer.
static __device__ __align__(256) float scratch[OD_SPLIT_SCRATCH_FLOATS];

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef unsigned int v4u __attribute__((ext_vector_type(4)));
typedef float v4f_t __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kWaves = 4;
constexpr int kSlotsPerTile = kWaves * 32;
constexpr int kBlockKeys = 64;  // prefix keys per block (2 key tiles of 32)
constexpr int kOwnKeys = 32;    // own keys per block (1 key tile)
constexpr float kLn2 = 0.693147180559945309f;
// Lazy rescaling: the running max of a slot only moves when a block raises its scaled scores by more than kSlack
// (log2 units), so p = exp2(s - m) <= 2^kSlack; the accumulator is rescaled only when the max or its frame moves.
constexpr float kSlack = 8.0f;
constexpr int kNoFrame = -1000000;  // a block without a visible key leaves the accumulator's frame alone
// The accumulator's power-of-two frame moves down to a block's V frame only when that lies more than kFrameSlack
// below it; such a block's probabilities carry 2^(eb - frame) >= 2^-kFrameSlack instead.
constexpr int kFrameSlack = 3;

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
  int dq;       // OD_DEQUANT_BF16 or OD_DEQUANT_FP32 (the int8 path; staged images carry their own)
  int nsplit;   // key-range splits (1: one pass writes out/lse)
  float* part;  // nsplit > 1: fp32 partials, o [nsplit][R][Hq][t][D] then lse [nsplit][R][Hq][t]
  const uint8_t* img;  // staged block images [Ns][Hkv][nb] (null: convert the int8 state in the kernel)
  // Two-level prefix (staged only): row group s reads the first level of state group_state[s] (its `img` images)
  // and then its own second-level images img2 [groups][Hkv][nb2] of T2 keys (a question's K/V).
  const uint8_t* img2;
  const int32_t* group_state;
  int T2, n_states;
  int* ctr;  // od_branched_attn_stream with splits: one merge counter per (state, KV head), zero between calls
};

// One block of 64 state keys as the attention reads it from LDS (and as od_attn_stage stores it, byte for byte).
// Every array is 16-byte aligned so that fragment accesses compile to single ds_read_b128 / ds_write_b128
// instructions (without the alignment the compiler splits them into 4-byte pairs).
template <int D>
struct alignas(16) BlockImg {
  alignas(16) uint16_t k[kBlockKeys * D];   // [key][d] bf16 keys (K', or the int8 values), chunks swizzled (k_off)
  alignas(16) _Float16 vt[D * kBlockKeys];  // [d][permuted key] V', swizzled (vt_off)
  alignas(16) float gk[kBlockKeys];         // score multiplier of key j: scale log2(e) [* ks_j] (1 if masked)
  alignas(16) float kb[kBlockKeys];         // 0, or -inf for a masked key
  alignas(16) int info[4];                  // the block constants: 0, eb, masked, 0
};
static_assert(sizeof(BlockImg<256>) == 4 * kBlockKeys * 256 + 8 * kBlockKeys + 16, "block image layout");
static_assert(sizeof(BlockImg<128>) == 4 * kBlockKeys * 128 + 8 * kBlockKeys + 16, "block image layout");
static_assert(sizeof(BlockImg<64>) == 4 * kBlockKeys * 64 + 8 * kBlockKeys + 16, "block image layout");

// Head dims of the block-image kernels. D = 256 (Qwen3.5's full-attention heads) holds twice the accumulators and
// query fragments of D = 128 and two 66 KB images: one workgroup per CU, one wave per SIMD with its 512 registers.
constexpr bool block_d_ok(int64_t D) { return D == 64 || D == 128 || D == 256; }
template <int D>
constexpr int kWgPerCu = D == 256 ? 1 : 2;

template <int D>
struct alignas(16) Smem {  // double-buffered block images
  BlockImg<D> b[2];
  float red[2][kWaves];
};

// The block constants (wave-uniform).
struct BlockInfo {
  int ek;      // the block's scores carry 2^-ek (own blocks; 0 for state blocks)
  int eb;      // the block's values carry 2^-eb (kNoFrame: no visible key)
  int masked;  // some key of the block is masked (its kb row must be added)
};

// LDS swizzles. gfx950 LDS: reads see 64 4-byte banks (a 256-byte period) and serve 16 lanes of a ds_read_b128
// per cycle; writes go 128 bytes per cycle with a 128-byte bank period (8 lanes of a ds_write_b128, 16 lanes of a
// ds_write_b64). A fragment read has lanes 16g .. 16g+15 take 16 consecutive rows (keys of K, d of V^T) at one
// logical 16-byte chunk, so the chunk is XORed with a function of the row that gives those 16 rows 16 distinct
// bank quads:
//  * K, rows of 2D bytes (D/8 chunks): D = 64, two rows share a 256-byte period, XOR with (key / 2) mod 8; D >= 128,
//    a row spans whole periods, XOR with key mod 16;
//  * V^T, rows of 128 bytes (8 chunks), two rows per period: XOR with ((d >> 1) ^ (d >> 3)) & 7, which is a
//    bijection on any 8 consecutive even (or odd) d and also on {8 dg + e : dg = 8 consecutive values} for a
//    fixed e, which the transposing store needs (see vmap).
template <int D>
__device__ __forceinline__ int k_off(int key, int chunk) {
  constexpr int kRowsPerPeriod = D >= 128 ? 1 : 128 / D;
  constexpr int kMask = D >= 128 ? 15 : D / 8 - 1;
  return key * D + ((chunk ^ ((key / kRowsPerPeriod) & kMask)) << 3);
}
__device__ __forceinline__ int vt_off(int d, int chunk) {
  return d * kBlockKeys + ((chunk ^ (((d >> 1) ^ (d >> 3)) & 7)) << 3);
}

// Thread -> (d group dg of 8 d, key group kg of 4 keys) of the transposing V store. A thread writes 8 bytes (its
// 4 keys) into each of the V^T rows 8 dg .. 8 dg + 7. Lanes 16i .. 16i+15 form one ds_write_b64 bank cycle: bits
// 0..2 of the lane pick 8 consecutive dg (8 distinct chunks after the V^T swizzle) and bit 3 flips bit 1 of kg,
// which is the half of the 16-byte chunk the 4 keys occupy, so the 16 lanes write 16 distinct 8-byte slots.
// D = 128: 16 dg x 16 kg = 256 threads; D = 64: 8 dg x 16 kg = threads 0..127. kg < 8 <=> thread < D.
// D = 256: 32 dg x 8 kg = 256 threads, and a 64-key block takes two passes (pass 1: kg + 8).
template <int D>
constexpr int kVPasses = D == 256 ? 2 : 1;
template <int D>
__device__ __forceinline__ void vmap(int tid, int pass, int& dg, int& kg) {
  const int lo = tid & 7, t3 = (tid >> 3) & 1, hi = tid >> 4;
  if constexpr (D == 256) {
    dg = lo | ((hi & 3) << 3);
    kg = (t3 << 1) | ((hi >> 2) & 1) | ((hi >> 3) << 2) | (pass << 3);
  } else if constexpr (D == 128) {
    dg = lo | ((hi & 1) << 3);
    kg = (t3 << 1) | ((hi >> 1) & 1) | ((hi >> 2) << 2);
  } else {
    dg = lo;
    kg = (t3 << 1) | (hi & 1) | ((hi >> 1) << 2);
  }
}
// whether thread tid takes part in a 64-key block's transposing V store (16 kg x D / 8 dg per pass)
template <int D>
__device__ __forceinline__ bool v_active(int tid) { return D == 256 || tid < 2 * D; }
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
// 4 int8 (one dword) -> 4 exact bf16 (two dwords): |q| <= 127 has at most 7 significant bits, so the fp32 value's
// top half is the exact bf16
__device__ __forceinline__ void i8x4_to_bf16(uint32_t w, uint32_t& lo, uint32_t& hi) {
  const uint32_t f0 = __float_as_uint((float)(int8_t)(w & 0xffu)), f1 = __float_as_uint((float)(int8_t)((w >> 8) & 0xffu));
  const uint32_t f2 = __float_as_uint((float)(int8_t)((w >> 16) & 0xffu)), f3 = __float_as_uint((float)(int8_t)(w >> 24));
  lo = __builtin_amdgcn_perm(f1, f0, 0x07060302u);
  hi = __builtin_amdgcn_perm(f3, f2, 0x07060302u);
}

// an exact fp16 pair times two fp32 factors, each product rounded once to fp16 (v_fma_mixlo/mixhi_f16)
__device__ __forceinline__ uint32_t h2_times(uint32_t h, float f0, float f1) {
  const half2v a = h2_bits(h);
  const half2v r = {(_Float16)__builtin_fmaf((float)a.x, f0, 0.0f), (_Float16)__builtin_fmaf((float)a.y, f1, 0.0f)};
  return bits_h2(r);
}

// bf16 materialize of 4 int8 key values (one dword) with the key's bf16 scale sb: bf16(q * sb) per value (the
// fp32 product of a 7-bit integer and an 8-bit significand is exact; one rounding to bf16)
__device__ __forceinline__ void i8x4_times_bf16(uint32_t w, float sb, uint32_t& lo, uint32_t& hi) {
  const float f0 = (float)(int8_t)(w & 0xffu) * sb, f1 = (float)(int8_t)((w >> 8) & 0xffu) * sb;
  const float f2 = (float)(int8_t)((w >> 16) & 0xffu) * sb, f3 = (float)(int8_t)(w >> 24) * sb;
  lo = __builtin_bit_cast(uint32_t, __builtin_convertvector((od_f32x2){f0, f1}, od_bf16x2));
  hi = __builtin_bit_cast(uint32_t, __builtin_convertvector((od_f32x2){f2, f3}, od_bf16x2));
}

// an exact fp16 pair of int8 values times two fp32 factors f = bf16(vs) 2^-eb (exact), each product rounded once to
// bf16 precision (the reference's bf16 product; the power of two does not change the rounding) and stored as fp16,
// which holds the 8 significant bits exactly (v_cvt_pkrtz_f16_f32 on an exactly representable value is exact)
__device__ __forceinline__ uint32_t h2_times_bf16(uint32_t h, float f0, float f1) {
  const half2v a = h2_bits(h);
  const uint32_t p = __builtin_bit_cast(uint32_t, __builtin_convertvector(
                                                      (od_f32x2){(float)a.x * f0, (float)a.y * f1}, od_bf16x2));
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(__uint_as_float(p << 16), __uint_as_float(p & 0xffff0000u)));
}

// bf16 rounding of an fp32 scale, as an fp32 value
__device__ __forceinline__ float bf16_round(float f) { return od_bf16_to_f32(od_f32_to_bf16(f)); }

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

// ----------------------------------------------------------------------------------------- state block images
// Loads of one int8 state block (keys j0 .. j0+63 of one (state, KV head)) go through buffer descriptors over the
// head's slab: the range check returns zeros for keys at or past the state's length, so no load is predicated, and
// every per-thread offset is a 32-bit constant (the block's position is the scalar offset).
struct PrefixSrc {
  __amdgpu_buffer_rsrc_t k, v, ks, vs, valid;
  bool has_valid;
};

template <int D>
__device__ __forceinline__ PrefixSrc prefix_src(const int8_t* kq, const float* ks, const int8_t* vq, const float* vs,
                                                const uint8_t* kvalid, int Hkv, int T, int cap, int s, int g) {
  const int64_t head_base = ((int64_t)s * Hkv + g) * cap;
  PrefixSrc src;
  src.k = __builtin_amdgcn_make_buffer_rsrc((void*)(kq + head_base * D), (short)0, T * D, 0x00020000);
  src.v = __builtin_amdgcn_make_buffer_rsrc((void*)(vq + head_base * D), (short)0, T * D, 0x00020000);
  src.ks = __builtin_amdgcn_make_buffer_rsrc((void*)(ks + head_base), (short)0, T * 4, 0x00020000);
  src.vs = __builtin_amdgcn_make_buffer_rsrc((void*)(vs + head_base), (short)0, T * 4, 0x00020000);
  src.has_valid = kvalid != nullptr;
  src.valid = __builtin_amdgcn_make_buffer_rsrc((void*)(kvalid ? kvalid + (int64_t)s * T : nullptr), (short)0,
                                                kvalid ? T : 0, 0x00020000);
  return src;
}

template <int D>
struct PrefixRegs {
  uint4 k[(kBlockKeys * D / 16 + kThreads - 1) / kThreads];
  uint2 v[4 * kVPasses<D>];  // pass p: v[4 p + a]
  float ks, vs;  // lane l of every wave: the K and V scale of key j0 + l (0 past the state's length)
  int in_range;  // lane l: key j0 + l exists
  int valid;     // lane l: its kvalid byte (1 without a mask); only read when converting, so the load is not waited
};

template <int D>
__device__ __forceinline__ void prefix_load(const PrefixSrc& src, int T, int j0, PrefixRegs<D>& r) {
  const int tid = threadIdx.x;
  constexpr int kChunks = kBlockKeys * D / 16;  // 16-byte int8 chunks per K block; chunk cid = bytes 16 cid ..
#pragma unroll
  for (int i = 0; i < (kChunks + kThreads - 1) / kThreads; ++i) {
    const int cid = i * kThreads + tid;
    r.k[i] = make_uint4(0, 0, 0, 0);
    if (cid < kChunks)
      r.k[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(src.k, cid * 16, j0 * D, 0));
  }
#pragma unroll
  for (int ps = 0; ps < kVPasses<D>; ++ps) {
    int dg, kg;
    vmap<D>(tid, ps, dg, kg);
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      r.v[4 * ps + a] = make_uint2(0, 0);
      if (v_active<D>(tid))
        r.v[4 * ps + a] = __builtin_bit_cast(
            uint2, __builtin_amdgcn_raw_buffer_load_b64(src.v, (4 * kg + a) * D + 8 * dg, j0 * D, 0));
    }
  }
  const int l = tid & 63;
  r.ks = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(src.ks, l * 4, j0 * 4, 0));
  r.vs = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(src.vs, l * 4, j0 * 4, 0));
  r.in_range = j0 + l < T;
  r.valid = src.has_valid ? (int)__builtin_amdgcn_raw_buffer_load_b8(src.valid, l, j0, 0) : 1;
}

// Converts a loaded int8 block into its image `dst` (LDS, or memory for od_attn_stage) and returns the block
// constants.
//  * dq = OD_DEQUANT_BF16: K' = bf16(q bf16(ks_j)) beside the multiplier scale_log2 (the softmax scale in log2
//    units); V' = bf16(q bf16(vs_j)) 2^-eb in fp16 (exact: 8 significant bits, |V'| < 128).
//  * dq = OD_DEQUANT_FP32: the int8 values as exact bf16 beside the multipliers gk_j = ks_j scale_log2 (one fp32
//    rounding); V' = fp16(q fv_j), one rounding (v_fma_mix), with the fp32 factor fv_j = vs_j 2^-eb (exact).
//    (Rounding fv_j to fp16 first would shift all of key j's values the same way, which under cancellation is
//    visible in the output.)
// 2^eb lies above the block's largest V scale. A masked key gets a zero V factor (P V' must stay finite), a -inf
// bias (added to its raw score) and the multiplier 1 (so the score stays -inf). Every wave derives the constants
// from the same 64 scales, so the waves agree without exchanging them.
template <int D>
__device__ __forceinline__ BlockInfo convert_block(const PrefixRegs<D>& r, BlockImg<D>& dst, float scale_log2,
                                                   int dq) {
  const bool mat = dq == OD_DEQUANT_BF16;
  const int tid = threadIdx.x;
  const bool ok = r.in_range && r.valid != 0;
  const float vs_ok = ok ? r.vs : 0.0f;
  BlockInfo bi;
  bi.masked = __builtin_amdgcn_ballot_w64(!ok) != 0;
  bi.ek = 0;
  const float vmax = od_wave_max_dpp(vs_ok);
  bi.eb = __builtin_amdgcn_ballot_w64(ok) != 0 ? exp_above(vmax) : kNoFrame;
  const float fv = ok ? ldexpf(mat ? bf16_round(vs_ok) : vs_ok, -bi.eb) : 0.0f;  // lane l: key l's V factor
  const float ksb = bf16_round(r.ks);  // lane l: key l's bf16 K scale (materialize)

  constexpr int kChunks = kBlockKeys * D / 16;
  constexpr int kCpk = D / 16;
#pragma unroll
  for (int i = 0; i < (kChunks + kThreads - 1) / kThreads; ++i) {
    const int cid = i * kThreads + tid;
    if (cid < kChunks) {
      const int key = cid / kCpk, c = cid % kCpk;
      // the 16 int8 values become two bf16 chunks, 2c and 2c + 1; lanes with bit 2 set store 2c + 1 first, so
      // that the 8 lanes of a ds_write_b128 bank cycle hit 8 distinct chunks of the 128-byte period
      const int flip = (tid >> 2) & 1;
      const uint32_t a0 = flip ? r.k[i].z : r.k[i].x, a1 = flip ? r.k[i].w : r.k[i].y;
      const uint32_t b0 = flip ? r.k[i].x : r.k[i].z, b1 = flip ? r.k[i].y : r.k[i].w;
      uint4 h0, h1;
      if (mat) {
        const float sb = __shfl(ksb, key, 64);
        i8x4_times_bf16(a0, sb, h0.x, h0.y);
        i8x4_times_bf16(a1, sb, h0.z, h0.w);
        i8x4_times_bf16(b0, sb, h1.x, h1.y);
        i8x4_times_bf16(b1, sb, h1.z, h1.w);
      } else {
        i8x4_to_bf16(a0, h0.x, h0.y);
        i8x4_to_bf16(a1, h0.z, h0.w);
        i8x4_to_bf16(b0, h1.x, h1.y);
        i8x4_to_bf16(b1, h1.z, h1.w);
      }
      *reinterpret_cast<uint4*>(&dst.k[k_off<D>(key, 2 * c + flip)]) = h0;
      *reinterpret_cast<uint4*>(&dst.k[k_off<D>(key, 2 * c + 1 - flip)]) = h1;
    }
  }
#pragma unroll
  for (int ps = 0; ps < kVPasses<D>; ++ps) {
  int dg, kg;
  vmap<D>(tid, ps, dg, kg);
  if (v_active<D>(tid)) {
    // 4 keys x 8 bytes -> for each of the 8 d: the 4 keys' bytes (a 4x4 byte transpose per dword half)
    const uint2* rv = &r.v[4 * ps];
    uint32_t cols[8];
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const uint32_t L0 = half ? rv[0].y : rv[0].x, L1 = half ? rv[1].y : rv[1].x;
      const uint32_t L2 = half ? rv[2].y : rv[2].x, L3 = half ? rv[3].y : rv[3].x;
      const uint32_t t0 = __builtin_amdgcn_perm(L1, L0, 0x05010400u);  // L0b0 L1b0 L0b1 L1b1
      const uint32_t t1 = __builtin_amdgcn_perm(L3, L2, 0x05010400u);  // L2b0 L3b0 L2b1 L3b1
      const uint32_t t2 = __builtin_amdgcn_perm(L1, L0, 0x07030602u);  // L0b2 L1b2 L0b3 L1b3
      const uint32_t t3 = __builtin_amdgcn_perm(L3, L2, 0x07030602u);
      cols[half * 4 + 0] = __builtin_amdgcn_perm(t1, t0, 0x05040100u);
      cols[half * 4 + 1] = __builtin_amdgcn_perm(t1, t0, 0x07060302u);
      cols[half * 4 + 2] = __builtin_amdgcn_perm(t3, t2, 0x05040100u);
      cols[half * 4 + 3] = __builtin_amdgcn_perm(t3, t2, 0x07060302u);
    }
    // the factors of the thread's 4 keys (a V^T dword holds keys 0,1 or keys 2,3 of the group)
    const float f0 = __shfl(fv, 4 * kg, 64), f1 = __shfl(fv, 4 * kg + 1, 64);
    const float f2 = __shfl(fv, 4 * kg + 2, 64), f3 = __shfl(fv, 4 * kg + 3, 64);
    const int jj0 = jj_of(4 * kg);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int d = 8 * dg + e;
      uint2 hv;
      i8x4_to_h(cols[e], hv.x, hv.y);
      if (mat) {
        hv.x = h2_times_bf16(hv.x, f0, f1);
        hv.y = h2_times_bf16(hv.y, f2, f3);
      } else {
        hv.x = h2_times(hv.x, f0, f1);
        hv.y = h2_times(hv.y, f2, f3);
      }
      *reinterpret_cast<uint2*>(&dst.vt[vt_off(d, jj0 >> 3) + (jj0 & 7)]) = hv;
    }
  }
  }
  if (tid < kBlockKeys) {
    dst.gk[tid] = ok ? (mat ? scale_log2 : r.ks * scale_log2) : 1.0f;
    dst.kb[tid] = ok ? 0.0f : -INFINITY;
  }
  if (tid == 0) *reinterpret_cast<int4*>(dst.info) = make_int4(bi.ek, bi.eb, bi.masked, 0);
  return bi;
}

// The block constants of an image in LDS, as wave-uniform values.
__device__ __forceinline__ BlockInfo read_info(const int* info) {
  const int4 v = *reinterpret_cast<const int4*>(info);
  BlockInfo bi;
  bi.ek = __builtin_amdgcn_readfirstlane(v.x);
  bi.eb = __builtin_amdgcn_readfirstlane(v.y);
  bi.masked = __builtin_amdgcn_readfirstlane(v.z);
  return bi;
}

// One global_load_lds_dwordx4: lane l copies 16 bytes from its `src` to LDS byte lds_base + 16 l (lds_base is
// wave-uniform, passed in M0). Written as inline asm so that the compiler does not track it: the caller waits for it
// (vmcnt) and orders it with barriers, whereas the compiler would wait for it before every LDS read that it cannot
// prove disjoint from the copy, which is every read of the other image buffer. The compiler keeps nothing in M0 in
// these kernels (no LDS DMA, movrel or sendmsg of its own), so setting it here disturbs no live value.
__device__ __forceinline__ void dma16(const void* src, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds_base), "v"(src)
               : "memory", "m0");
}

template <typename T>
__device__ __forceinline__ uint32_t lds_addr(T* p) {
  return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)(p);
}

// Copies NBYTES (a multiple of 16) of a staged image into LDS, 16 bytes per lane and no registers: round i moves
// bytes [4096 i, 4096 (i + 1)), wave w the 1 KiB at 1024 w of it; the tail round has every wave copy the last
// 1 KiB (bytes already copied are written again with the same values), so that no round branches on the lane or
// the wave and a caller's code around the copies stays one basic block (one scheduling region).
// Completion is a vmcnt wait by every thread that issued a part, then a barrier.
template <int NBYTES>
struct CopyShape {
  static constexpr int kRound = kThreads * 16;
  static constexpr int kFull = NBYTES / kRound;
  static constexpr int kTailLanes = (NBYTES - kFull * kRound) / 16;
  static constexpr int kRounds = kFull + (kTailLanes > 0 ? 1 : 0);
  static_assert(NBYTES % 16 == 0 && NBYTES >= 1024 && kTailLanes <= 64, "copy shape");
};

// Round i of such a copy (so that a caller can spread the rounds over its work).
template <int NBYTES>
__device__ __forceinline__ void copy_round(const void* src, void* dst, int i) {
  using C = CopyShape<NBYTES>;
  const int tid = threadIdx.x;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const char* s = reinterpret_cast<const char*>(src);
  const uint32_t d = __builtin_amdgcn_readfirstlane(lds_addr(dst));
  const int lane = tid & 63;
  if (i < C::kFull)
    dma16(s + i * C::kRound + tid * 16, d + i * C::kRound + wave * 1024);
  else
    dma16(s + NBYTES - 1024 + lane * 16, d + NBYTES - 1024);
}

template <int NBYTES>
__device__ __forceinline__ void copy_bytes(const void* src, void* dst) {
#pragma unroll
  for (int i = 0; i < CopyShape<NBYTES>::kRounds; ++i) copy_round<NBYTES>(src, dst, i);
}

// ------------------------------------------------------------------------------------------------- compute
// One block of the online softmax for the wave's 32 slots, in three pieces:
//  * qk_scores: S^T = K Q^T on V_MFMA_F32_32X32X16_BF16 (exact products; fragment reads KA k-steps ahead);
//  * softmax_block: y = S gk + kb - m (log2 units; gk the per-key K scale times the softmax scale, kb the mask; own
//    blocks: y = S c - m with the causal mask), the block max, the running max m moved only when the block raises it
//    by more than kSlack, p = exp2(y), P to fp16, l = l alpha + sum p; it returns whether some slot's max moved
//    (the accumulator is rescaled then, or when its frame moves);
//  * pv_block: O^T += V'^T P^T (fragment reads VA steps ahead).
// Each slot moves its own max only on its own condition (the others get alpha = exp2(0) = 1), so a slot's arithmetic
// does not depend on which slots share its wave and option order cannot change a result.
// The schedule of qk_scores' reads and MFMAs: the reads KA k-steps ahead of the MFMAs (left alone, the scheduler sinks
// each read to its MFMA). With NV > 0, NV VALU instructions go after each k-step's MFMAs, so that they issue while
// the MFMAs run: these are taken from the code between the qk_scores call (with SCHED false) and this call, which
// must be independent of the scores.
template <int D, int KT, int KA, int NV>
__device__ __forceinline__ void qk_sched() {
  constexpr int KS = D / 16;
  __builtin_amdgcn_sched_group_barrier(0x100, KA * KT, 0);
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    if (ks + KA < KS) __builtin_amdgcn_sched_group_barrier(0x100, KT, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, KT, 0);
    if (NV > 0) __builtin_amdgcn_sched_group_barrier(0x002, NV, 0);
  }
}

template <int D, int KT, int KA, bool SCHED = true>
__device__ __forceinline__ void qk_scores(const uint16_t* kimg, const bf16x8 (&qf)[D / 16], v16f (&s)[KT]) {
  const int lane = threadIdx.x & 63;
  const int h = lane >> 5, col = lane & 31;
  constexpr int KS = D / 16;
#pragma unroll
  for (int kt = 0; kt < KT; ++kt) s[kt] = v16f{0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
  bf16x8 kf[KA + 1][KT];
  auto kread = [&](int ks) {
#pragma unroll
    for (int kt = 0; kt < KT; ++kt)
      kf[ks % (KA + 1)][kt] = *reinterpret_cast<const bf16x8*>(&kimg[k_off<D>(kt * 32 + col, ks * 2 + h)]);
  };
#pragma unroll
  for (int ks = 0; ks < KA; ++ks) kread(ks);
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    if (ks + KA < KS) kread(ks + KA);
#pragma unroll
    for (int kt = 0; kt < KT; ++kt)
      s[kt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[ks % (KA + 1)][kt], qf[ks], s[kt], 0, 0, 0);
  }
  if (SCHED) qk_sched<D, KT, KA, 0>();
}

// Adds a state block's bias row (0, or -inf for a masked key) to the raw scores: a masked key's score is then -inf
// whatever its multiplier (which is 1 for a masked key, so the product stays -inf).
template <int KT>
__device__ __forceinline__ void apply_mask(const float* kb, v16f (&s)[KT]) {
  const int h = (threadIdx.x & 63) >> 5;
#pragma unroll
  for (int kt = 0; kt < KT; ++kt)
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      const float4 b4 = *reinterpret_cast<const float4*>(&kb[kt * 32 + 8 * r4 + 4 * h]);
      s[kt][4 * r4] += b4.x;
      s[kt][4 * r4 + 1] += b4.y;
      s[kt][4 * r4 + 2] += b4.z;
      s[kt][4 * r4 + 3] += b4.w;
    }
}

// c: own blocks' score multiplier.
// dlt = eb - e_new <= 0: the block's values are in frame eb and the accumulator in frame e_new, so the block's
// probabilities enter the P.V product as p 2^dlt (folded into the exponent, exact while p 2^dlt is a normal fp16).
// A state block with masked keys has had its bias row added to the raw scores (apply_mask). sched() runs at the end
// of the common path, which is straight-line code (the caller's scheduling directives for that region).
template <int D, int KT, bool OWN, typename Sched>
__device__ __forceinline__ bool softmax_block(const float* gk, v16f (&s)[KT], float c, int dlt,
                                              float& m_run, float& l_run, float& alpha, half8 (&pb)[2 * KT],
                                              int own_row, int own_j0, int slot_row, int slot_tok, Sched&& sched) {
  const int lane = threadIdx.x & 63;
  const int h = lane >> 5;
  const float m_safe = m_run == -INFINITY ? 0.0f : m_run;
  const float fdlt = (float)dlt;
  const float bias = fdlt - m_safe;
  // this lane's slot sees keys kt*32 + 8*(r/4) + 4*h + r%4
  if constexpr (OWN) {
#pragma unroll
    for (int kt = 0; kt < KT; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = own_j0 + kt * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
        s[kt][r] = (slot_row == own_row && key <= slot_tok) ? fmaf(s[kt][r], c, bias) : -INFINITY;
      }
  } else {
#pragma unroll
    for (int kt = 0; kt < KT; ++kt)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const float4 g4 = *reinterpret_cast<const float4*>(&gk[kt * 32 + 8 * r4 + 4 * h]);
        s[kt][4 * r4] = fmaf(s[kt][4 * r4], g4.x, bias);
        s[kt][4 * r4 + 1] = fmaf(s[kt][4 * r4 + 1], g4.y, bias);
        s[kt][4 * r4 + 2] = fmaf(s[kt][4 * r4 + 2], g4.z, bias);
        s[kt][4 * r4 + 3] = fmaf(s[kt][4 * r4 + 3], g4.w, bias);
      }
  }
  float amax = -INFINITY;
#pragma unroll
  for (int kt = 0; kt < KT; ++kt)
#pragma unroll
    for (int r = 0; r < 16; ++r) amax = fmaxf(amax, s[kt][r]);
  amax = od_xor32_max(amax) - fdlt;  // the block max relative to the running max
  // a slot whose block max exceeds its running max by more than kSlack (or that sees its first key) moves its max
  // to the block max and shifts its y (wave-uniform branch, rare)
  const bool grow = m_run == -INFINITY ? amax > -INFINITY : amax > kSlack;
  alpha = 1.0f;
  float psum = 0.0f;
  // p = exp2(y - shift) into fp16 P, psum = sum p
  auto probs = [&](float shift) {
    psum = 0.0f;
#pragma unroll
    for (int kt = 0; kt < KT; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float pr = __builtin_amdgcn_exp2f(s[kt][r] - shift);
        psum += pr;
        pb[kt * 2 + (r >> 3)][r & 7] = (_Float16)pr;
      }
  };
  // The common case (no slot grows, shift 0) runs straight through, so that the whole softmax is one scheduling
  // region that a caller can interleave with MFMAs; a block where some slot grows redoes the probabilities.
  const bool any_grow = __builtin_amdgcn_ballot_w64(grow) != 0;
  probs(0.0f);
  sched();
  // pins the common path's results here: without it the compiler sinks them into the no-growth side of the branch
  if constexpr (KT == 2)
    asm volatile("" : "+v"(pb[0]), "+v"(pb[1]), "+v"(pb[2]), "+v"(pb[3]), "+v"(psum));
  else
    asm volatile("" : "+v"(pb[0]), "+v"(pb[1]), "+v"(psum));
  if (any_grow) {
    const float shift = grow ? amax : 0.0f;
    const float m_new = m_safe + shift;
    alpha = __builtin_amdgcn_exp2f(m_run - m_new);  // 0 for a slot's first visible block, 1 if it did not grow
    if (grow) m_run = m_new;
    probs(shift);
  }
  l_run = fmaf(l_run, alpha, ldexpf(od_xor32_sum(psum), -dlt));
  return any_grow;
}

// The accumulator into frame e_new (and each slot's new max): O *= alpha 2^(e_run - e_new).
template <int D>
__device__ __forceinline__ void rescale(v16f (&o)[D / 32], float alpha, int e_new, int& e_run) {
  const float rs = ldexpf(alpha, e_run - e_new);
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[dt][r] *= rs;
  e_run = e_new;
}

template <int D, int KT, int VA>
__device__ __forceinline__ void pv_block(const _Float16* vtimg, const half8 (&pb)[2 * KT], v16f (&o)[D / 32]) {
  const int lane = threadIdx.x & 63;
  const int h = lane >> 5, col = lane & 31;
  constexpr int kVA = VA < 2 * KT ? VA : 2 * KT - 1;
  half8 vf[kVA + 1][D / 32];
  auto vread = [&](int m) {
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
      vf[m % (kVA + 1)][dt] = *reinterpret_cast<const half8*>(&vtimg[vt_off(dt * 32 + col, 2 * m + h)]);
  };
#pragma unroll
  for (int m = 0; m < kVA; ++m) vread(m);
#pragma unroll
  for (int m = 0; m < 2 * KT; ++m) {
    if (m + kVA < 2 * KT) vread(m + kVA);
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
      o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf[m % (kVA + 1)][dt], pb[m], o[dt], 0, 0, 0);
  }
  __builtin_amdgcn_sched_group_barrier(0x100, kVA * (D / 32), 0);
#pragma unroll
  for (int m = 0; m < 2 * KT; ++m) {
    if (m + kVA < 2 * KT) __builtin_amdgcn_sched_group_barrier(0x100, D / 32, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, D / 32, 0);
  }
}

// The frame the accumulator takes for a block whose values are in frame eb. Over the state blocks it follows the
// blocks' V exponents lazily: it moves up to a block's frame (P 2^dlt must not exceed the fp16 range) and down only
// by more than kFrameSlack (to keep small P 2^dlt normal); in between the block's probabilities carry
// 2^dlt = 2^(eb - frame). Every slot sees the same state blocks in the same order, so the frames do not depend on
// the option rows. An own block always takes its own frame: the frame the accumulator is in when it comes depends
// on the rows before it in the tile, and P 2^dlt can round differently (subnormal fp16) from P. Wave-uniform, like
// the frames.
template <bool OWN>
__device__ __forceinline__ int frame_for(int e_blk, int e_run) {
  return (OWN || e_run == kNoFrame || e_blk > e_run || e_blk < e_run - kFrameSlack) ? e_blk : e_run;
}

// The three pieces in sequence. `mid` runs between the softmax and the P V product (the int8 path issues the next
// block's global loads there, so that their registers are not held through the score and softmax phases).
template <int D, int DV, int KT, bool OWN, typename Mid>
__device__ __forceinline__ void attend_block(const uint16_t* kimg, const _Float16* vtimg, const float* gk,
                                             const float* kb, const bf16x8 (&qf)[D / 16], float c, int eb,
                                             bool masked, float& m_run, float& l_run, int& e_run, v16f (&o)[DV / 32],
                                             int own_row, int own_j0, int slot_row, int slot_tok, Mid&& mid) {
  constexpr int KA = 2;
  v16f s[KT];
  __builtin_amdgcn_s_setprio(1);  // a wave issuing MFMAs goes first, the other wave's softmax fills the gaps
  qk_scores<D, KT, KA>(kimg, qf, s);
  __builtin_amdgcn_s_setprio(0);
  const int e_blk = eb == kNoFrame ? e_run : eb;
  const int e_new = frame_for<OWN>(e_blk, e_run);
  float alpha;
  half8 pb[2 * KT];
  if (!OWN && masked) apply_mask<KT>(kb, s);
  const bool grow = softmax_block<D, KT, OWN>(gk, s, c, e_blk - e_new, m_run, l_run, alpha, pb, own_row, own_j0,
                                              slot_row, slot_tok, [] {});
  mid();
  if (grow || e_new != e_run) rescale<DV>(o, alpha, e_new, e_run);
  __builtin_amdgcn_s_setprio(1);
  pv_block<DV, KT, 1>(vtimg, pb, o);
  __builtin_amdgcn_s_setprio(0);
}

// One state block of the staged path, software-pipelined over the blocks: the NEXT block's scores (keys at knext)
// are computed while this block's softmax runs, then this block's P.V product. s holds this block's scores on entry;
// sn receives the next block's. The score MFMAs go one k-step at a time, each followed by a share of the softmax's
// common path (a group of 4 scores: multiplier, max, exp2, sum, fp16) that the scheduler may not move across the
// k-steps, so the wave issues VALU work while its MFMAs run; dma(ks) issues the k-step's share of the copies of
// later blocks. The arithmetic per block is that of attend_block (the same operations on the same values in the
// same order), so both paths give the same bits.
template <int D, int DV, typename Dma>
__device__ __forceinline__ void staged_step(const BlockImg<D>& cur, const uint16_t* knext, const bf16x8 (&qf)[D / 16],
                                            v16f (&s)[2], v16f (&sn)[2], float& m_run, float& l_run, int& e_run,
                                            v16f (&o)[DV / 32], int vh, Dma&& dma) {
  constexpr int KT = 2, KA = 1, KS = D / 16;
  constexpr int kGroups = KT * 4;  // groups of 4 scores: (key tile kt, register quad r4)
  // D = 128: one group per k-step; D = 64: two; D = 256: one on every second k-step
  constexpr int kPerStep = kGroups >= KS ? kGroups / KS : 1;
  constexpr int kStride = KS > kGroups ? KS / kGroups : 1;
  static_assert(kPerStep * KS == kGroups * kStride, "score groups per k-step");
  const int lane = threadIdx.x & 63;
  const int h = lane >> 5, col = lane & 31;
  const BlockInfo ci = read_info(cur.info);
  const int e_blk = ci.eb == kNoFrame ? e_run : ci.eb;
  const int e_new = frame_for<false>(e_blk, e_run);
  const int dlt = e_blk - e_new;
  if (ci.masked) apply_mask<KT>(cur.kb, s);  // rare: a state's last block, or a key mask
  const float m_safe = m_run == -INFINITY ? 0.0f : m_run;
  const float fdlt = (float)dlt;
  const float bias = fdlt - m_safe;
  float amax = -INFINITY, psum = 0.0f;
  half8 pb[2 * KT];

#pragma unroll
  for (int kt = 0; kt < KT; ++kt) sn[kt] = v16f{0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
  bf16x8 kf[KA + 1][KT];
  auto kread = [&](int ks) {
#pragma unroll
    for (int kt = 0; kt < KT; ++kt)
      kf[ks % (KA + 1)][kt] = *reinterpret_cast<const bf16x8*>(&knext[k_off<D>(kt * 32 + col, ks * 2 + h)]);
  };
#pragma unroll
  for (int ks = 0; ks < KA; ++ks) kread(ks);
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    // this k-step's key multipliers are read ahead of the next k-step's K fragments, so that waiting for them
    // leaves those fragments in flight
    const bool gstep = ks % kStride == kStride - 1;  // this k-step carries score groups (a constant once unrolled)
    const int g0 = (ks / kStride) * kPerStep;
    float4 g4s[kPerStep];
    if (gstep) {
#pragma unroll
      for (int c = 0; c < kPerStep; ++c) {
        const int grp = g0 + c, kt = grp / 4, r4 = grp % 4;
        g4s[c] = *reinterpret_cast<const float4*>(&cur.gk[kt * 32 + 8 * r4 + 4 * h]);
      }
    }
    if (ks + KA < KS) kread(ks + KA);
#pragma unroll
    for (int kt = 0; kt < KT; ++kt)
      sn[kt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[ks % (KA + 1)][kt], qf[ks], sn[kt], 0, 0, 0);
    dma(ks);
#pragma unroll
    for (int c = 0; c < (gstep ? kPerStep : 0); ++c) {
      const int grp = g0 + c, kt = grp / 4, r4 = grp % 4;
      const float4 g4 = g4s[c];
      const float gg[4] = {g4.x, g4.y, g4.z, g4.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = 4 * r4 + e;
        s[kt][r] = fmaf(s[kt][r], gg[e], bias);
        amax = fmaxf(amax, s[kt][r]);
        const float pr = __builtin_amdgcn_exp2f(s[kt][r]);
        psum += pr;
        pb[kt * 2 + (r >> 3)][r & 7] = (_Float16)pr;
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  // pins the common path's results here: without it the compiler sinks them into the no-growth side of the branch
  asm volatile("" : "+v"(pb[0]), "+v"(pb[1]), "+v"(pb[2]), "+v"(pb[3]), "+v"(psum));
  // the rest of softmax_block: growth (rare), the running sum, the rescale
  amax = od_xor32_max(amax) - fdlt;
  const bool grow = m_run == -INFINITY ? amax > -INFINITY : amax > kSlack;
  float alpha = 1.0f;
  const bool any_grow = __builtin_amdgcn_ballot_w64(grow) != 0;
  if (any_grow) {
    const float shift = grow ? amax : 0.0f;
    const float m_new = m_safe + shift;
    alpha = __builtin_amdgcn_exp2f(m_run - m_new);
    if (grow) m_run = m_new;
    psum = 0.0f;
#pragma unroll
    for (int kt = 0; kt < KT; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float pr = __builtin_amdgcn_exp2f(s[kt][r] - shift);
        psum += pr;
        pb[kt * 2 + (r >> 3)][r & 7] = (_Float16)pr;
      }
  }
  l_run = fmaf(l_run, alpha, ldexpf(od_xor32_sum(psum), -dlt));
  if (any_grow || e_new != e_run) rescale<DV>(o, alpha, e_new, e_run);
  __builtin_amdgcn_s_setprio(1);
  pv_block<DV, KT, 1>(cur.vt + vh * DV * kBlockKeys, pb, o);
  __builtin_amdgcn_s_setprio(0);
}

// Workgroup max of two values (every thread gets both).
__device__ __forceinline__ void wg_max2(float (&red)[2][kWaves], float& a, float& b) {
  a = od_wave_max_dpp(a);
  b = od_wave_max_dpp(b);
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

// Own keys j0 .. j0+31 of option row `row` into a block image's K and V arrays: the bf16 keys as they are (the
// score MFMAs take bf16), the bf16 values scaled by one power of two into fp16, V' = V 2^ev (exact), whose frame
// bi.eb = -ev is the block's own (not the running frame: which frame the accumulator is in when a row's own block
// comes depends on the rows before it in the tile, and a P V' product that rounds differently in another frame would
// break option-order invariance).
template <int D>
__device__ __forceinline__ void own_stage(const AttnArgs& p, float (&red)[2][kWaves], uint16_t* kdst,
                                          _Float16* vtdst, int row, int g, int j0, BlockInfo& bi) {
  const int tid = threadIdx.x;
  const int n_keys = min(kOwnKeys, p.t - j0);
  const uint16_t* kb = p.k_own + (int64_t)row * p.skr + (int64_t)g * p.skh;
  const uint16_t* vb = p.v_own + (int64_t)row * p.svr + (int64_t)g * p.svh;
  constexpr int kCpk = D / 8;                 // 8-value chunks per key
  constexpr int kChunks = kOwnKeys * kCpk;    // K chunks of the block
  constexpr int kKIt = (kChunks + kThreads - 1) / kThreads;
#pragma unroll
  for (int i = 0; i < kKIt; ++i) {
    const int cid = i * kThreads + tid;
    const int key = cid / kCpk, c = cid % kCpk;
    if (cid < kChunks) {
      uint4 kr = make_uint4(0, 0, 0, 0);
      if (key < n_keys) kr = *reinterpret_cast<const uint4*>(kb + (int64_t)(j0 + key) * p.skt + 8 * c);
      *reinterpret_cast<uint4*>(&kdst[k_off<D>(key, c)]) = kr;
    }
  }
  // V: a thread takes 4 keys x 8 d (kOwnKeys / 4 key groups x D / 8 d groups, threads 0 .. D - 1)
  int dg, kg;
  vmap<D>(tid, 0, dg, kg);
  const bool vact = tid < D;
  uint4 vr[4];
  float va = 0.0f, unused = 0.0f;
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
  wg_max2(red, va, unused);
  const int ev = 15 - exp_above(va);  // |x| 2^ev < 2^15
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
      *reinterpret_cast<uint2*>(&vtdst[vt_off(8 * dg + e, jj0 >> 3) + (jj0 & 7)]) = hv;
    }
  }
  bi.ek = 0;
  bi.eb = -ev;
  bi.masked = 0;  // the causal mask is applied per score
}

// DV: the value columns one workgroup accumulates (D, or D / 2 at D = 256: the two halves of a slot tile are two
// workgroups, each recomputing the same scores and softmax; see branched_launch).
template <int D, int DV, bool STAGED>
__device__ __forceinline__ void branched_attn_body(const AttnArgs& p, Smem<D>& sm) {
  constexpr int kHalves = D / DV;
  static_assert(kHalves == 1 || kHalves == 2, "value halves");
  // XCD-aware work order: workgroups are dealt round-robin over the 8 XCDs, so flat id f runs on XCD f % 8. Work item
  // w = (state split, KV head, slot tile) with the tile fastest is given to XCD (w's range), so that the tiles of
  // one (state, head) share one XCD's L2 for the state blocks they all stream.
  // (the value halves of a slot tile, blockIdx.x = 2 tile + half, are adjacent work items and share the XCD too)
  const int nx = gridDim.x;
  const int n_items = nx * gridDim.y * gridDim.z;
  const int f = blockIdx.x + nx * (blockIdx.y + gridDim.y * blockIdx.z);
  const int xcd = f & 7, local = f >> 3, per = n_items >> 3, rem = n_items & 7;
  const int w = xcd < rem ? xcd * (per + 1) + local : rem * (per + 1) + (xcd - rem) * per + local;
  const int tile = (w % nx) / kHalves, vh = (w % nx) % kHalves, zy = w / nx;
  const int g = zy % gridDim.y, zz = zy / gridDim.y;
  const int s = zz / p.nsplit, sp = zz % p.nsplit;
  const int row0 = p.row_start ? p.row_start[s] : 0;
  const int nrows = p.row_start ? p.row_start[s + 1] - row0 : p.R;
  const int per_row = p.t * p.rep;
  const int nslots = nrows * per_row;
  const int slot_base = tile * kSlotsPerTile;
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

  // ---- prefix: the state's blocks (then, two-level, the group's own second-level blocks); split sp of nsplit takes
  // the blocks [sp * bps, (sp + 1) * bps)
  const int nb1_all = (p.T + kBlockKeys - 1) / kBlockKeys;
  int st = s;  // the state whose (first-level) blocks this row group reads
  if (p.group_state) st = p.group_state[s];
  const bool st_ok = st >= 0 && st < p.n_states;  // a group naming no valid state reads no first-level keys
  if (!st_ok) st = 0;
  const int nb1 = st_ok ? nb1_all : 0;
  const int nb2 = p.img2 ? (p.T2 + kBlockKeys - 1) / kBlockKeys : 0;
  const int nb_all = nb1 + nb2;
  const int bps = (nb_all + p.nsplit - 1) / p.nsplit;
  const int b_lo = min(nb_all, sp * bps), b_hi = min(nb_all, b_lo + bps);
  // the first block's copy (staged path) goes out before the queries are read
  const BlockImg<D>* img1 =
      STAGED ? reinterpret_cast<const BlockImg<D>*>(p.img) + ((int64_t)st * p.Hkv + g) * nb1_all : nullptr;
  const BlockImg<D>* img2 =
      STAGED && p.img2 ? reinterpret_cast<const BlockImg<D>*>(p.img2) + ((int64_t)s * p.Hkv + g) * nb2 : nullptr;
  auto blk = [&](int b) { return b < nb1 ? img1 + b : img2 + (b - nb1); };
  if (STAGED && b_hi > b_lo) copy_bytes<(int)sizeof(BlockImg<D>)>(blk(b_lo), &sm.b[0]);

  // query fragments: lane holds Q[slot][ks*16 + 8h .. +8] for ks = 0 .. D/16-1, bf16 as given
  bf16x8 qf[D / 16];
  {
    const uint16_t* qp = p.q + (int64_t)slot_row * p.sqr + (int64_t)slot_head * p.sqh + (int64_t)slot_tok * p.sqt;
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks)
      qf[ks] = __builtin_bit_cast(bf16x8, slot_ok ? *reinterpret_cast<const uint4*>(qp + ks * 16 + 8 * h)
                                                  : make_uint4(0, 0, 0, 0));
  }

  float m_run = -INFINITY, l_run = 0.0f;
  int e_run = kNoFrame;  // the power-of-two frame the accumulator is in (follows the blocks' V exponents)
  v16f o[DV / 32];
#pragma unroll
  for (int dt = 0; dt < DV / 32; ++dt) o[dt] = v16f{0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
  const int vcol = vh * DV * kBlockKeys;  // this workgroup's value rows in a block image's V^T

  if (b_hi > b_lo) {
    if constexpr (STAGED) {
      // Block images straight from memory into the double-buffered LDS images, the keys one block ahead of the rest:
      // block j lives in buffer (j - b_lo) & 1; during block b's step, whose score MFMAs read block b + 1's keys,
      // block b + 2's keys go into buffer b (its keys were read in the previous step) and block b + 1's values,
      // multipliers and constants into the other buffer (block b - 1's, read in the previous step).
      constexpr int kKeyBytes = (int)offsetof(BlockImg<D>, vt);
      constexpr int kRestBytes = (int)sizeof(BlockImg<D>) - kKeyBytes;
      auto rest = [](const BlockImg<D>* bi) { return reinterpret_cast<const char*>(bi) + kKeyBytes; };
      if (b_lo + 1 < b_hi) copy_bytes<kKeyBytes>(blk(b_lo + 1), sm.b[1].k);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      v16f s0[2], s1[2];
      qk_scores<D, 2, 2>(sm.b[0].k, qf, s0);
      __syncthreads();  // block b_lo's keys are read: block b_lo + 2's may go into buffer 0
      // the copies' rounds (global_load_lds instructions) are spread over the step's k-steps: issued all at once, the
      // eight waves of a CU queue behind each other at the texture unit
      constexpr int kKR = CopyShape<kKeyBytes>::kRounds, kNR = kKR + CopyShape<kRestBytes>::kRounds;
      auto step = [&](int b, v16f (&sc)[2], v16f (&sn)[2]) {
        const int buf = (b - b_lo) & 1;
        BlockImg<D>& cur = sm.b[buf];
        BlockImg<D>& nxt = sm.b[buf ^ 1];
        auto dma = [&](int ks) {
#pragma unroll
          for (int r = ks * kNR / (D / 16); r < (ks + 1) * kNR / (D / 16); ++r) {
            // past the last block the copies repeat the last block into buffers no later step reads, so that
            // the step has no branch: its score MFMAs and softmax groups stay one scheduling region
            if (r < kKR)
              copy_round<kKeyBytes>(blk(min(b + 2, b_hi - 1)), cur.k, r);
            else
              copy_round<kRestBytes>(rest(blk(min(b + 1, b_hi - 1))), reinterpret_cast<char*>(&nxt) + kKeyBytes,
                                     r - kKR);
          }
        };
        // the last block's step scores its own keys again (in place of a next block), and the result is not used
        staged_step<D, DV>(cur, b + 1 < b_hi ? nxt.k : cur.k, qf, sc, sn, m_run, l_run, e_run, o, vh, dma);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
      };
      // two blocks per trip, so that the scores alternate between s0 and s1 without register copies
      for (int b = b_lo; b < b_hi; b += 2) {
        step(b, s0, s1);
        if (b + 1 < b_hi) step(b + 1, s1, s0);
      }
    } else {
      // the int8 state, converted here: registers first (loads issued during the previous block), then LDS
      const PrefixSrc src = prefix_src<D>(p.kq, p.ks, p.vq, p.vs, p.kvalid, p.Hkv, p.T, p.cap, s, g);
      PrefixRegs<D> pr;
      prefix_load<D>(src, p.T, b_lo * kBlockKeys, pr);
      BlockInfo cur = convert_block<D>(pr, sm.b[0], p.scale_log2, p.dq);
      __syncthreads();
      for (int b = b_lo; b < b_hi; ++b) {
        const int buf = (b - b_lo) & 1;
        const BlockImg<D>& bk = sm.b[buf];
        attend_block<D, DV, 2, false>(bk.k, bk.vt + vcol, bk.gk, bk.kb, qf, 0.0f, cur.eb, cur.masked != 0, m_run,
                                      l_run, e_run, o,
                                  0, 0, slot_row, slot_tok, [&] {
                                    if (b + 1 < b_hi) prefix_load<D>(src, p.T, (b + 1) * kBlockKeys, pr);
                                  });
        BlockInfo nxt = cur;
        if (b + 1 < b_hi) nxt = convert_block<D>(pr, sm.b[buf ^ 1], p.scale_log2, p.dq);
        __syncthreads();
        cur = nxt;
      }
    }
  }

  // ---- own keys (the last split): every option row that has a slot in this tile, 32 keys per block
  const int last = min(slot_base + kSlotsPerTile, nslots) - 1;
  const int r_lo = row0 + slot_base / per_row, r_hi = sp == p.nsplit - 1 ? row0 + last / per_row : r_lo - 1;
  for (int row = r_lo; row <= r_hi; ++row) {
    // only the own blocks that some slot of the tile can see: keys up to the largest token of this row in the tile
    const int rl = row - row0;
    const int tok_hi = (min(last, (rl + 1) * per_row - 1) - rl * per_row) / p.rep;
    for (int j0 = 0; j0 <= tok_hi; j0 += kOwnKeys) {
      __syncthreads();  // LDS image 0 free
      BlockInfo bi;
      own_stage<D>(p, sm.red, sm.b[0].k, sm.b[0].vt, row, g, j0, bi);
      __syncthreads();
      // a wave with no slot in this row skips its block (all its scores would be masked)
      if (__builtin_amdgcn_ballot_w64(slot_row == row) != 0)
        attend_block<D, DV, 1, true>(sm.b[0].k, sm.b[0].vt + vcol, nullptr, nullptr, qf, p.scale_log2, bi.eb, false,
                                     m_run, l_run, e_run, o, row, j0, slot_row, slot_tok, [] {});
    }
  }

  if (!slot_ok) return;
  // ---- epilogue: out = O 2^E / l (bf16), lse = (m + log2 l) ln 2
  const float inv = l_run > 0.0f ? ldexpf(1.0f / l_run, e_run) : 0.0f;
  const float lse_v = l_run > 0.0f ? (m_run + __log2f(l_run)) * kLn2 : -INFINITY;
  const int64_t slot_idx = ((int64_t)slot_row * p.Hq + slot_head) * p.t + slot_tok;
  if (p.nsplit > 1) {
    // this split's normalized fp32 partial (this half's columns) and its LSE, merged by combine_kernel
    const int64_t nsl = (int64_t)p.R * p.Hq * p.t;
    float* po = p.part + ((int64_t)sp * nsl + slot_idx) * D + vh * DV;
#pragma unroll
    for (int dt = 0; dt < DV / 32; ++dt)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4)
        *reinterpret_cast<float4*>(po + dt * 32 + 8 * r4 + 4 * h) =
            make_float4(o[dt][4 * r4] * inv, o[dt][4 * r4 + 1] * inv, o[dt][4 * r4 + 2] * inv,
                        o[dt][4 * r4 + 3] * inv);
    if (h == 0 && vh == 0) p.part[(int64_t)p.nsplit * nsl * D + (int64_t)sp * nsl + slot_idx] = lse_v;
    return;
  }
  uint16_t* op = p.out + (int64_t)slot_row * p.sor + (int64_t)slot_head * p.soh + (int64_t)slot_tok * p.sot + vh * DV;
#pragma unroll
  for (int dt = 0; dt < DV / 32; ++dt) {
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
  if (p.lse && h == 0 && vh == 0) p.lse[slot_idx] = lse_v;
}

// The int8 path: two workgroups per CU (two waves per SIMD hide each other's phases; one at D = 256).
template <int D, int DV>
__global__ __launch_bounds__(kThreads, kWgPerCu<D>) void branched_attn_kernel(AttnArgs p) {
  __shared__ Smem<D> sm;
  branched_attn_body<D, DV, false>(p, sm);
}

// The staged path: the same, each workgroup copying block images into LDS.
template <int D, int DV>
__global__ __launch_bounds__(kThreads, kWgPerCu<D>) void branched_staged_kernel(AttnArgs p) {
  __shared__ Smem<D> sm;
  branched_attn_body<D, DV, true>(p, sm);
}

// od_attn_stage: one workgroup per (block, KV head, state) converts an int8 block into its image.
struct StageArgs {
  const int8_t* kq;
  const float* ks;
  const int8_t* vq;
  const float* vs;
  const uint8_t* kvalid;
  uint8_t* img;
  int Hkv, T, cap, nb;
  float scale_log2;
  int dq;
};

template <int D>
__global__ __launch_bounds__(kThreads) void stage_kernel(StageArgs p) {
  const int b = blockIdx.x, g = blockIdx.y, s = blockIdx.z;
  const PrefixSrc src = prefix_src<D>(p.kq, p.ks, p.vq, p.vs, p.kvalid, p.Hkv, p.T, p.cap, s, g);
  PrefixRegs<D> pr;
  prefix_load<D>(src, p.T, b * kBlockKeys, pr);
  const int64_t blk = ((int64_t)s * p.Hkv + g) * p.nb + b;
  convert_block<D>(pr, reinterpret_cast<BlockImg<D>*>(p.img)[blk], p.scale_log2, p.dq);
}

// od_attn_stage_bf16: one workgroup per (block, KV head, state) writes the image of 64 keys of a dense bf16 state
// (the reference's materialized K/V): the keys as they are beside the multiplier scale_log2, the values as
// V' = fp16(v 2^-eb) with 2^eb above the block's largest |v| (exact while |v| >= 2^(eb - 14); smaller values become
// fp16 subnormals, within 2^(eb - 25) of v), a masked key (past T or kvalid 0) with zero K and V, multiplier 1 and a
// -inf bias, as convert_block writes them.
struct StageBf16Args {
  const uint16_t* k;
  const uint16_t* v;
  const uint8_t* kvalid;
  uint8_t* img;
  int64_t skb, skh, skt, svb, svh, svt;
  int Hkv, T, nb;
  float scale_log2;
};

template <int D>
__global__ __launch_bounds__(kThreads) void stage_bf16_kernel(StageBf16Args p) {
  __shared__ float red[kWaves];
  const int b = blockIdx.x, g = blockIdx.y, s = blockIdx.z;
  const int tid = threadIdx.x;
  const int j0 = b * kBlockKeys;
  BlockImg<D>& dst = reinterpret_cast<BlockImg<D>*>(p.img)[((int64_t)s * p.Hkv + g) * p.nb + b];
  const uint16_t* kbase = p.k + (int64_t)s * p.skb + (int64_t)g * p.skh;
  const uint16_t* vbase = p.v + (int64_t)s * p.svb + (int64_t)g * p.svh;
  auto valid = [&](int key) {
    return j0 + key < p.T && (!p.kvalid || p.kvalid[(int64_t)s * p.T + j0 + key] != 0);
  };
  constexpr int kChunks = kBlockKeys * D / 8;  // 16-byte chunks of 8 bf16
  for (int cid = tid; cid < kChunks; cid += kThreads) {
    const int key = cid / (D / 8), c = cid % (D / 8);
    uint4 val = make_uint4(0, 0, 0, 0);
    if (valid(key)) val = *reinterpret_cast<const uint4*>(kbase + (int64_t)(j0 + key) * p.skt + 8 * c);
    *reinterpret_cast<uint4*>(&dst.k[k_off<D>(key, c)]) = val;
  }
  constexpr int kP = kVPasses<D>;
  uint4 vv[4 * kP];  // pass ps: vv[4 ps + a]
  float vmax = 0.0f;
#pragma unroll
  for (int ps = 0; ps < kP; ++ps) {
    int dg, kg;
    vmap<D>(tid, ps, dg, kg);
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      uint4& x = vv[4 * ps + a];
      x = make_uint4(0, 0, 0, 0);
      if (v_active<D>(tid) && valid(4 * kg + a))
        x = *reinterpret_cast<const uint4*>(vbase + (int64_t)(j0 + 4 * kg + a) * p.svt + 8 * dg);
      const uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
      for (int e = 0; e < 4; ++e)
        vmax = fmaxf(vmax, fmaxf(fabsf(__uint_as_float(w[e] << 16)), fabsf(__uint_as_float(w[e] & 0xffff0000u))));
    }
  }
  vmax = od_wave_max_dpp(vmax);
  if ((tid & 63) == 0) red[tid >> 6] = vmax;
  __syncthreads();
  vmax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const bool ok = valid(tid & 63);
  const bool any = __builtin_amdgcn_ballot_w64(ok) != 0;
  const int masked = __builtin_amdgcn_ballot_w64(!ok) != 0;  // taken with the whole wave active
  const int eb = any ? exp_above(vmax) : kNoFrame;
#pragma unroll
  for (int ps = 0; ps < kP; ++ps) {
    int dg, kg;
    vmap<D>(tid, ps, dg, kg);
    if (v_active<D>(tid)) {
      const float f = any ? ldexpf(1.0f, -eb) : 0.0f;
      const int jj0 = jj_of(4 * kg);
#pragma unroll
      for (int e = 0; e < 8; ++e) {  // d = 8 dg + e: the 4 keys' values
        float x[4];
#pragma unroll
        for (int a = 0; a < 4; ++a) {
          const uint4& y = vv[4 * ps + a];
          const uint32_t w = e < 2 ? y.x : e < 4 ? y.y : e < 6 ? y.z : y.w;
          x[a] = __uint_as_float((e & 1) ? (w & 0xffff0000u) : (w << 16)) * f;
        }
        const uint2 hv = make_uint2(pack_h2(x[0], x[1]), pack_h2(x[2], x[3]));
        *reinterpret_cast<uint2*>(&dst.vt[vt_off(8 * dg + e, jj0 >> 3) + (jj0 & 7)]) = hv;
      }
    }
  }
  if (tid < kBlockKeys) {
    dst.gk[tid] = ok ? p.scale_log2 : 1.0f;
    dst.kb[tid] = ok ? 0.0f : -INFINITY;
  }
  if (tid == 0) *reinterpret_cast<int4*>(dst.info) = make_int4(0, eb, masked, 0);
}

// LSE merge of the key-range splits (prefix_attn.py:74-76 generalised to n parts): M = max_s lse_s,
// w_s = exp(lse_s - M), out = sum_s w_s o_s / sum_s w_s (bf16), lse = M + log(sum_s w_s); no visible key in any
// split -> 0 and -inf. One thread per (slot, 8 values of d); M is taken as a running max in the same pass.
template <int D>
__global__ __launch_bounds__(256) void combine_kernel(AttnArgs p) {
  const int64_t nsl = (int64_t)p.R * p.Hq * p.t;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t slot = gid / (D / 8);
  const int d0 = (int)(gid % (D / 8)) * 8;
  if (slot >= nsl) return;
  const float* lse_p = p.part + (int64_t)p.nsplit * nsl * D;
  // one pass with a running max (the sum rescaled when the max moves), so that no load waits for another: the loop
  // is unrolled and every split's LSE and partial are in flight together
  float M = -INFINITY;
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  float wsum = 0.0f;
#pragma unroll 8
  for (int sp = 0; sp < p.nsplit; ++sp) {
    const float l = lse_p[sp * nsl + slot];
    const float4* po = reinterpret_cast<const float4*>(p.part + (sp * nsl + slot) * D + d0);
    const float4 a = po[0], b = po[1];
    if (l == -INFINITY) continue;  // a split with no visible key
    if (l > M) {
      const float r = __expf(M - l);  // M = -inf: 0 (nothing accumulated yet)
      wsum *= r;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] *= r;
      M = l;
    }
    const float w = __expf(l - M);
    wsum += w;
    acc[0] += w * a.x; acc[1] += w * a.y; acc[2] += w * a.z; acc[3] += w * a.w;
    acc[4] += w * b.x; acc[5] += w * b.y; acc[6] += w * b.z; acc[7] += w * b.w;
  }
  const int row = (int)(slot / ((int64_t)p.Hq * p.t)), rem = (int)(slot % ((int64_t)p.Hq * p.t));
  const int head = rem / p.t, tok = rem % p.t;
  // wsum 0: no visible key (0 and -inf); NaN (a NaN partial) propagates to the output and the LSE
  const float inv = wsum > 0.0f ? 1.0f / wsum : wsum == 0.0f ? 0.0f : wsum;
  uint32_t w4[4];
#pragma unroll
  for (int e = 0; e < 4; ++e)
    w4[e] = (uint32_t)od_f32_to_bf16(acc[2 * e] * inv) | ((uint32_t)od_f32_to_bf16(acc[2 * e + 1] * inv) << 16);
  uint16_t* op = p.out + (int64_t)row * p.sor + (int64_t)head * p.soh + (int64_t)tok * p.sot + d0;
  *reinterpret_cast<uint2*>(op) = make_uint2(w4[0], w4[1]);
  *reinterpret_cast<uint2*>(op + 4) = make_uint2(w4[2], w4[3]);
  if (p.lse && d0 == 0) p.lse[slot] = wsum > 0.0f ? M + __logf(wsum) : wsum == 0.0f ? -INFINITY : wsum;
}

}  // namespace

namespace {

int64_t stage_blocks(int64_t Ns, int64_t Hkv, int64_t T) { return Ns * Hkv * ((T + kBlockKeys - 1) / kBlockKeys); }
int64_t stage_block_bytes(int64_t D) {
  return D == 256 ? (int64_t)sizeof(BlockImg<256>) : D == 128 ? (int64_t)sizeof(BlockImg<128>) : (int64_t)sizeof(BlockImg<64>);
}

// The second prefix level of od_branched_attn_staged2 (absent for the other entry points).
struct Level2 {
  const void* img2;
  int64_t img2_bytes;
  const int32_t* group_state;
  int64_t T2, n_states;
};

int branched_launch(const uint16_t* q, int64_t sqr, int64_t sqh, int64_t sqt, const uint16_t* k_own, int64_t skr,
                    int64_t skh, int64_t skt, const uint16_t* v_own, int64_t svr, int64_t svh, int64_t svt,
                    const int8_t* kq, const float* ks, const int8_t* vq, const float* vs, const uint8_t* kvalid,
                    const void* img, const int32_t* row_start, int64_t max_rows, uint16_t* out,
                    int64_t sor, int64_t soh, int64_t sot, float* lse, int64_t R, int64_t Hq, int64_t Hkv, int64_t t,
                    int64_t D, int64_t Ns, int64_t T, int64_t cap, float scale, int dq, int64_t nsplit, float* ws,
                    int64_t ws_floats, od_stream_t stream, const Level2* l2 = nullptr) {
  const bool staged = img != nullptr || l2 != nullptr;
  if (dq != OD_DEQUANT_BF16 && dq != OD_DEQUANT_FP32) return OD_ERR_UNSUPPORTED;
  if (R < 0 || Hq < 1 || Hkv < 1 || t < 1 || Ns < 1 || T < 0 || cap < T || max_rows < 0) return OD_ERR_SHAPE;
  if (Hq % Hkv) return OD_ERR_UNSUPPORTED;
  if (!block_d_ok(D)) return OD_ERR_UNSUPPORTED;
  if (!row_start && Ns != 1) return OD_ERR_SHAPE;
  if (nsplit < 1 || nsplit > 256) return OD_ERR_SHAPE;
  if (!row_start) max_rows = R;
  if (R == 0 || max_rows == 0) return OD_OK;
  if (!q || !k_own || !v_own || !out) return OD_ERR_NULL;
  if (T > 0 && !staged && (!kq || !ks || !vq || !vs)) return OD_ERR_NULL;
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
  if (T > 0 && !staged && (!od_aligned16(kq) || !od_aligned16(vq))) return OD_ERR_ALIGN;
  if (T > 0 && staged && (!img || !od_aligned16(img))) return img ? OD_ERR_ALIGN : OD_ERR_NULL;
  const int64_t rep = Hq / Hkv;
  const int64_t tiles = (max_rows * t * rep + kSlotsPerTile - 1) / kSlotsPerTile;
  if (tiles > 0x7fffffff || Hkv > 65535 || Ns * nsplit > 65535 || R * t * rep > 0x7fffffff ||
      cap * Hkv * Ns * D > (1ll << 40) || nsplit * R * Hq * t * (D + 1) > (1ll << 40) ||
      T * D >= (1ll << 31))  // one (state, head) slab is addressed with 32-bit buffer offsets
    return OD_ERR_SHAPE;
  if (l2) {
    if (l2->T2 < 0 || l2->n_states < 1 || l2->n_states > 65535 || l2->T2 * D >= (1ll << 31)) return OD_ERR_SHAPE;
    if (l2->T2 > 0 && !l2->img2) return OD_ERR_NULL;
    if (l2->T2 > 0 && !od_aligned16(l2->img2)) return OD_ERR_ALIGN;
    if (l2->T2 > 0 && l2->img2_bytes < stage_blocks(Ns, Hkv, l2->T2) * stage_block_bytes(D)) return OD_ERR_SHAPE;
  }
  AttnArgs a{q, k_own, v_own, kq, ks, vq, vs, kvalid, row_start, out, lse, sqr, sqh, sqt, skr, skh, skt, svr, svh,
             svt, sor, soh, sot, (int)R, (int)Hq, (int)Hkv, (int)t, (int)Ns, (int)T, (int)cap, (int)rep,
             scale * 1.4426950408889634f, dq, (int)nsplit, nsplit > 1 ? ws : nullptr,
             static_cast<const uint8_t*>(img),
             l2 && l2->T2 > 0 ? static_cast<const uint8_t*>(l2->img2) : nullptr, l2 ? l2->group_state : nullptr,
             l2 ? (int)l2->T2 : 0, l2 ? (int)l2->n_states : (int)Ns};
  // D = 256 on the staged path runs as two workgroups per slot tile, each accumulating 128 of the value columns
  // (blockIdx.x = 2 tile + half): one pass over all 256 columns holds 256-column accumulators beside 256-dim query
  // fragments, which spilled (136 bytes per lane) and moved accumulators between register files every block; each
  // half recomputes the scores and softmax, so its outputs are those of one pass (bit for bit), and the pass takes
  // 0.63x the time (4 states x 4096 keys, 64 rows x 24 tokens, 16 / 4 heads: 1088 -> 683 us). The int8 path keeps
  // one workgroup per tile: its halves would each convert the whole block, and its few-row shapes measured slower.
  const int64_t halves = D == 256 && staged ? 2 : 1;
  if (tiles * halves > 0x7fffffff) return OD_ERR_SHAPE;
  dim3 grid((unsigned)(tiles * halves), (unsigned)Hkv, (unsigned)(Ns * nsplit)), block(kThreads);
  hipStream_t st = (hipStream_t)stream;
  if (D == 256) {
    staged ? branched_staged_kernel<256, 128><<<grid, block, 0, st>>>(a)
           : branched_attn_kernel<256, 256><<<grid, block, 0, st>>>(a);
  } else if (D == 128) {
    staged ? branched_staged_kernel<128, 128><<<grid, block, 0, st>>>(a)
           : branched_attn_kernel<128, 128><<<grid, block, 0, st>>>(a);
  } else {
    staged ? branched_staged_kernel<64, 64><<<grid, block, 0, st>>>(a)
           : branched_attn_kernel<64, 64><<<grid, block, 0, st>>>(a);
  }
  if (nsplit > 1) {
    const int rc = od_launch_status();
    if (rc != OD_OK) return rc;
    const int64_t threads = R * Hq * t * (D / 8);
    const unsigned blocks = (unsigned)((threads + 255) / 256);
    if (D == 256) {
      combine_kernel<256><<<blocks, 256, 0, st>>>(a);
    } else if (D == 128) {
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
                                float scale, int dequant, od_stream_t stream) {
  return branched_launch(q, sqr, sqh, sqt, k_own, skr, skh, skt, v_own, svr, svh, svt, kq, ks, vq, vs, kvalid,
                         nullptr, row_start, max_rows, out, sor, soh, sot, lse, R, Hq, Hkv, t, D, Ns, T, cap, scale,
                         dequant, 1, nullptr, 0, stream);
}

extern "C" int od_branched_attn_split(const uint16_t* q, int64_t sqr, int64_t sqh, int64_t sqt, const uint16_t* k_own,
                                      int64_t skr, int64_t skh, int64_t skt, const uint16_t* v_own, int64_t svr,
                                      int64_t svh, int64_t svt, const int8_t* kq, const float* ks, const int8_t* vq,
                                      const float* vs, const uint8_t* kvalid, const int32_t* row_start,
                                      int64_t max_rows, uint16_t* out, int64_t sor, int64_t soh, int64_t sot,
                                      float* lse, int64_t R, int64_t Hq, int64_t Hkv, int64_t t, int64_t D, int64_t Ns,
                                      int64_t T, int64_t cap, float scale, int dequant, int64_t nsplit, float* ws,
                                      int64_t ws_floats, od_stream_t stream) {
  return branched_launch(q, sqr, sqh, sqt, k_own, skr, skh, skt, v_own, svr, svh, svt, kq, ks, vq, vs, kvalid,
                         nullptr, row_start, max_rows, out, sor, soh, sot, lse, R, Hq, Hkv, t, D, Ns, T, cap, scale,
                         dequant, nsplit, ws, ws_floats, stream);
}

extern "C" int od_attn_stage_size(int64_t Ns, int64_t Hkv, int64_t T, int64_t D, int64_t* img_bytes) {
  if (Ns < 1 || Hkv < 1 || T < 0) return OD_ERR_SHAPE;
  if (!block_d_ok(D)) return OD_ERR_UNSUPPORTED;
  if (!img_bytes) return OD_ERR_NULL;
  *img_bytes = stage_blocks(Ns, Hkv, T) * stage_block_bytes(D);
  return OD_OK;
}

extern "C" int od_attn_stage(const int8_t* kq, const float* ks, const int8_t* vq, const float* vs,
                             const uint8_t* kvalid, int64_t Ns, int64_t Hkv, int64_t T, int64_t cap, int64_t D,
                             float scale, int dequant, void* img, int64_t img_bytes, od_stream_t stream) {
  if (Ns < 1 || Hkv < 1 || T < 0 || cap < T) return OD_ERR_SHAPE;
  if (dequant != OD_DEQUANT_BF16 && dequant != OD_DEQUANT_FP32) return OD_ERR_UNSUPPORTED;
  if (!block_d_ok(D)) return OD_ERR_UNSUPPORTED;
  if (T == 0) return OD_OK;
  if (!kq || !ks || !vq || !vs || !img) return OD_ERR_NULL;
  if (!od_aligned16(kq) || !od_aligned16(vq) || !od_aligned16(img)) return OD_ERR_ALIGN;
  const int64_t nb = (T + kBlockKeys - 1) / kBlockKeys;
  if (img_bytes < stage_blocks(Ns, Hkv, T) * stage_block_bytes(D)) return OD_ERR_SHAPE;
  if (nb > 0x7fffffff || Hkv > 65535 || Ns > 65535 || T * D >= (1ll << 31) || cap * Hkv * Ns * D > (1ll << 40))
    return OD_ERR_SHAPE;
  StageArgs a{kq, ks, vq, vs, kvalid, static_cast<uint8_t*>(img), (int)Hkv, (int)T, (int)cap, (int)nb,
              scale * 1.4426950408889634f, dequant};
  dim3 grid((unsigned)nb, (unsigned)Hkv, (unsigned)Ns), block(kThreads);
  hipStream_t st = (hipStream_t)stream;
  if (D == 256) {
    stage_kernel<256><<<grid, block, 0, st>>>(a);
  } else if (D == 128) {
    stage_kernel<128><<<grid, block, 0, st>>>(a);
  } else {
    stage_kernel<64><<<grid, block, 0, st>>>(a);
  }
  return od_launch_status();
}

extern "C" int od_branched_attn_staged(const uint16_t* q, int64_t sqr, int64_t sqh, int64_t sqt,
                                       const uint16_t* k_own, int64_t skr, int64_t skh, int64_t skt,
                                       const uint16_t* v_own, int64_t svr, int64_t svh, int64_t svt, const void* img,
                                       int64_t img_bytes, const int32_t* row_start, int64_t max_rows, uint16_t* out,
                                       int64_t sor, int64_t soh, int64_t sot, float* lse, int64_t R, int64_t Hq,
                                       int64_t Hkv, int64_t t, int64_t D, int64_t Ns, int64_t T, float scale,
                                       int64_t nsplit, float* ws, int64_t ws_floats, od_stream_t stream) {
  if (T > 0 && !img) return OD_ERR_NULL;
  if (block_d_ok(D) && Ns >= 1 && Hkv >= 1 && T > 0 && img_bytes < stage_blocks(Ns, Hkv, T) * stage_block_bytes(D))
    return OD_ERR_SHAPE;
  return branched_launch(q, sqr, sqh, sqt, k_own, skr, skh, skt, v_own, svr, svh, svt, nullptr, nullptr, nullptr,
                         nullptr, nullptr, T > 0 ? img : nullptr, row_start, max_rows, out, sor, soh, sot, lse, R, Hq,
                         Hkv, t, D, Ns, T, T, scale, OD_DEQUANT_BF16, nsplit, ws, ws_floats, stream);
}


extern "C" int od_attn_stage_bf16(const uint16_t* k, int64_t skb, int64_t skh, int64_t skt, const uint16_t* v,
                                  int64_t svb, int64_t svh, int64_t svt, const uint8_t* kvalid, int64_t Ns,
                                  int64_t Hkv, int64_t T, int64_t D, float scale, void* img, int64_t img_bytes,
                                  od_stream_t stream) {
  if (Ns < 1 || Hkv < 1 || T < 0) return OD_ERR_SHAPE;
  if (!block_d_ok(D)) return OD_ERR_UNSUPPORTED;
  if (T == 0) return OD_OK;
  if (!k || !v || !img) return OD_ERR_NULL;
  const int64_t strides[] = {skb, skh, skt, svb, svh, svt};
  for (int64_t st : strides)
    if (st < 0 || st % 8) return OD_ERR_ALIGN;
  if (!od_aligned16(k) || !od_aligned16(v) || !od_aligned16(img)) return OD_ERR_ALIGN;
  const int64_t nb = (T + kBlockKeys - 1) / kBlockKeys;
  if (img_bytes < stage_blocks(Ns, Hkv, T) * stage_block_bytes(D)) return OD_ERR_SHAPE;
  if (nb > 0x7fffffff || Hkv > 65535 || Ns > 65535 || T > 0x7fffffff) return OD_ERR_SHAPE;
  StageBf16Args a{k, v, kvalid, static_cast<uint8_t*>(img), skb, skh, skt, svb, svh, svt, (int)Hkv, (int)T, (int)nb,
                  scale * 1.4426950408889634f};
  dim3 grid((unsigned)nb, (unsigned)Hkv, (unsigned)Ns), block(kThreads);
  hipStream_t st = (hipStream_t)stream;
  if (D == 256) {
    stage_bf16_kernel<256><<<grid, block, 0, st>>>(a);
  } else if (D == 128) {
    stage_bf16_kernel<128><<<grid, block, 0, st>>>(a);
  } else {
    stage_bf16_kernel<64><<<grid, block, 0, st>>>(a);
  }
  return od_launch_status();
}

namespace {

std::mutex g_scratch_mu;
constexpr int kMaxDevices = 64;
float* g_scratch[kMaxDevices] = {};

// This device's copy of `scratch` (resolved on the first call made with the device current).
int scratch_ptr(float** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return OD_ERR_LAUNCH;
  if (dev < 0 || dev >= kMaxDevices) return OD_ERR_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return OD_ERR_LAUNCH;
    g_scratch[dev] = static_cast<float*>(p);
  }
  *out = g_scratch[dev];
  return OD_OK;
}

}  // namespace

extern "C" int od_branched_attn_split_noalloc(const uint16_t* q, int64_t sqr, int64_t sqh, int64_t sqt,
                                              const uint16_t* k_own, int64_t skr, int64_t skh, int64_t skt,
                                              const uint16_t* v_own, int64_t svr, int64_t svh, int64_t svt,
                                              const int8_t* kq, const float* ks, const int8_t* vq, const float* vs,
                                              const uint8_t* kvalid, const int32_t* row_start, int64_t max_rows,
                                              uint16_t* out, int64_t sor, int64_t soh, int64_t sot, float* lse,
                                              int64_t R, int64_t Hq, int64_t Hkv, int64_t t, int64_t D, int64_t Ns,
                                              int64_t T, int64_t cap, float scale, int dequant, int64_t nsplit,
                                              od_stream_t stream) {
  if (R < 0 || Hq < 1 || t < 1 || D < 1 || nsplit < 1 || nsplit > 256) return OD_ERR_SHAPE;
  const int64_t need = nsplit > 1 ? nsplit * R * Hq * t * (D + 1) : 0;
  if (need > OD_SPLIT_SCRATCH_FLOATS) return OD_ERR_SCRATCH;
  float* ws = nullptr;
  if (need > 0) {
    const int rc = scratch_ptr(&ws);
    if (rc != OD_OK) return rc;
  }
  return branched_launch(q, sqr, sqh, sqt, k_own, skr, skh, skt, v_own, svr, svh, svt, kq, ks, vq, vs, kvalid,
                         nullptr, row_start, max_rows, out, sor, soh, sot, lse, R, Hq, Hkv, t, D, Ns, T, cap, scale,
                         dequant, nsplit, ws, need, stream);
}

extern "C" int od_branched_attn_staged2(const uint16_t* q, int64_t sqr, int64_t sqh, int64_t sqt,
                                        const uint16_t* k_own, int64_t skr, int64_t skh, int64_t skt,
                                        const uint16_t* v_own, int64_t svr, int64_t svh, int64_t svt,
                                        const void* img, int64_t img_bytes, const int32_t* group_state,
                                        int64_t n_states, int64_t T, const void* img2, int64_t img2_bytes, int64_t T2,
                                        const int32_t* row_start, int64_t max_rows, uint16_t* out, int64_t sor,
                                        int64_t soh, int64_t sot, float* lse, int64_t R, int64_t Hq, int64_t Hkv,
                                        int64_t t, int64_t D, int64_t n_groups, float scale, int64_t nsplit,
                                        float* ws, int64_t ws_floats, od_stream_t stream) {
  if (n_groups < 1 || n_states < 1 || T < 0) return OD_ERR_SHAPE;
  if (T > 0 && !img) return OD_ERR_NULL;
  if (!group_state && n_groups > n_states) return OD_ERR_SHAPE;
  if (block_d_ok(D) && T > 0 && img_bytes < stage_blocks(n_states, Hkv, T) * stage_block_bytes(D))
    return OD_ERR_SHAPE;
  const Level2 l2{img2, img2_bytes, group_state, T2, n_states};
  // with T = 0 the level-1 images may be absent: the staged path then reads only the second level
  return branched_launch(q, sqr, sqh, sqt, k_own, skr, skh, skt, v_own, svr, svh, svt, nullptr, nullptr, nullptr,
                         nullptr, nullptr, T > 0 ? img : nullptr, row_start, max_rows, out, sor, soh, sot, lse, R,
                         Hq, Hkv, t, D, n_groups, T, T, scale, OD_DEQUANT_BF16, nsplit, ws, ws_floats, stream, &l2);
}

// ================================================================================================ KV streaming
// od_branched_attn_stream: the few-slot case. When every (state, KV head) carries at most 32 query slots (a few
// short option rows, e.g. a yes/no decision over a long state), the attention does at most 32 x 4 FLOP per state key
// and dimension against 2 bytes of int8 K/V, so it is bound by reading the state from HBM, and the block-image paths
// (LDS images, 128-slot tiles) leave most of their MFMA columns and conversion work idle. Here one wave takes all
// slots of its (state, head) as NC column tiles of 16 (NC = 1 for up to 16 slots, 2 for up to 32) and streams the
// state's int8 K/V straight from HBM into registers, 32 keys per tile, one tile ahead, converting there; a
// workgroup's 8 waves take interleaved tiles of one key range, the key range of each (state, head) is split over
// workgroups (nsplit, chosen by the caller so that the workgroups fill the CUs once), and the last workgroup of a
// (state, head) merges the splits' partials by log-sum-exp. The K/V loads are non-temporal: each byte is read once,
// and keeping it out of the caches measured 12% faster on 32768-key states.
//
// On V_MFMA_F32_16X16X32_BF16 (lane l: column l % 16; result rows 4 (l / 16) + i), per tile (keys kb .. kb + 31 as
// two 16-key row tiles kr), lane l = (j, g) = (l % 16, l / 16):
//  * scores S^T[kr] = K'[kr] Q^T: k-step ks takes dims 32 g + 8 ks .. +7 of both operands (a permutation of the
//    reduction index, applied to both sides); the lane loads 32 contiguous bytes of each of its keys kb + j and
//    kb + 16 + j and converts them: K' = bf16(q bf16(ks_j)) (OD_DEQUANT_BF16) or the exact integer q
//    (OD_DEQUANT_FP32, the key's fp32 multiplier then goes on the score). The result gives lane (j, g) slot
//    16 nc + j and keys 16 kr + 4 g + i, so a slot's online softmax is lane-local plus two exchanges (l ^ 16, l ^ 32);
//  * values O^T[dt] += V'^T[dt] P^T, output row r of d-tile dt being d = 8 r + dt, with the keys in the order
//    kappa(g, i) = (4 g + i, i < 4; 12 + 4 g + i, i >= 4): the B operand is then exactly the lane's own 8
//    probabilities, and the A operand of lane (r, g) is byte dt of the 8 bytes d = 8 r .. 8 r + 7 it loaded for each
//    of its keys kappa(g, 0..7) (16 lanes read a key's whole 128-byte row). V' = bf16(q bf16(vs_j)) (exact bf16) or,
//    OD_DEQUANT_FP32, the integer q with vs_j folded into the probability;
//  * P goes to the P.V product as two bf16 parts, hi = bf16(p) and lo = bf16(p - hi) (16 significant bits, two
//    MFMAs per d-tile): V' is exactly the reference's bf16 value and P keeps fp16-level precision. The row sum is
//    taken on the unrounded fp32 p.
// Lane (j, g) ends with slot 16 nc + j's dims 32 g .. 32 g + 31. The rows' own keys (at most 32: rows x t <= slots)
// are one extra masked tile of bf16 K/V, taken by wave 0 of the last split. Each slot's arithmetic depends only on
// its own scores, so option order cannot change a result.
namespace {

constexpr int kStrWaves = 8;
constexpr int kStrKeys = 32;
constexpr int kStrD = 128;

// The per-wave LDS of the streaming kernel: a tile's per-key factors, written by lane l for key l % 32 and read
// back in the score layout (keys 16 kr + 4 g + 0..3 as one float4).
struct StrKeyLds {
  float4 f[2][8];  // [0]: V factor (bf16(vs) or vs), [1]: score multiplier (OD_DEQUANT_FP32: ks scale log2(e))
};

// One (state, KV head)'s int8 state as the streaming kernel reads it.
struct StrSrc {
  const int8_t* k;
  const int8_t* v;
  const float* ks;
  const float* vs;
  const uint8_t* valid;  // null: no mask
  int T;
};

__device__ __forceinline__ float f4_at(const float4& v, int j) { return j == 0 ? v.x : j == 1 ? v.y : j == 2 ? v.z : v.w; }

// int8 byte b of w, times an fp32 factor
__device__ __forceinline__ float byte_times(uint32_t w, int b, float f) { return (float)(int8_t)((w >> (8 * b)) & 0xffu) * f; }

__device__ __forceinline__ uint32_t pk_bf16(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((od_f32x2){a, b}, od_bf16x2));
}

// The queries of the workgroup's (at most 32) slots in LDS, read per k-step (lane (j, g) of k-step ks: slot
// 16 nc + j, dims 32 g + 8 ks .. +7); the row stride of 272 bytes puts 16 consecutive slots on 16 distinct bank quads.
constexpr int kStrQRow = kStrD + 8;

__device__ __forceinline__ v4f_t mfma16(bf16x8 a, bf16x8 b, v4f_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ int s16_kappa(int g, int i) { return i < 4 ? 4 * g + i : 12 + 4 * g + i; }

// One tile of the stream in registers.
struct S16Tile {
  uint4 k[4];     // lane (j, g): int8 bytes 32 g .. 32 g + 15 and + 16 .. + 31 of key kb + j (k[0], k[1]), kb + 16 + j
  uint2 v[8];     // lane (r, g): V bytes 8 r .. 8 r + 7 of key kb + kappa(g, i)
  float vs, ks;   // lane l: the V and K scales of key kb + (l & 31)
  int valid;      // lane l: the kvalid byte of key kb + (l & 31) (0 without a mask)
};

// The cache policy of the stream's loads: non-temporal (nt), for data read exactly once.
constexpr int kStreamOnce = 2;

// The tile's loads, all unconditional (a conditional load makes the compiler wait for every load in flight). Each
// load goes through a descriptor made for the tile (base at key kb, length T - kb keys: keys past the length read
// as zeros), so the per-lane offsets are loop-invariant and no address register is rewritten while loads are in
// flight.
__device__ __forceinline__ void s16_load(const StrSrc& src, int kb, int lane, S16Tile& tl) {
  const int n = max(src.T - kb, 0);
  constexpr int kF = 0x00020000;
  const auto rk = __builtin_amdgcn_make_buffer_rsrc((void*)(src.k + (int64_t)kb * kStrD), (short)0, n * kStrD, kF);
  const auto rv = __builtin_amdgcn_make_buffer_rsrc((void*)(src.v + (int64_t)kb * kStrD), (short)0, n * kStrD, kF);
  const auto rks = __builtin_amdgcn_make_buffer_rsrc((void*)(src.ks + kb), (short)0, n * 4, kF);
  const auto rvs = __builtin_amdgcn_make_buffer_rsrc((void*)(src.vs + kb), (short)0, n * 4, kF);
  const auto rva = __builtin_amdgcn_make_buffer_rsrc((void*)(src.valid ? src.valid + kb : nullptr), (short)0,
                                                     src.valid ? n : 0, kF);
  const int j = lane & 15, g = lane >> 4, c = lane & 31;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    tl.k[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                            rk, ((i >> 1) * 16 + j) * kStrD + 32 * g + 16 * (i & 1), 0, kStreamOnce));
#pragma unroll
  for (int i = 0; i < 8; ++i)
    tl.v[i] = __builtin_bit_cast(
        uint2, __builtin_amdgcn_raw_buffer_load_b64(rv, s16_kappa(g, i) * kStrD + 8 * j, 0, kStreamOnce));
  tl.vs = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rvs, c * 4, 0, kStreamOnce));
  tl.ks = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rks, c * 4, 0, kStreamOnce));
  tl.valid = __builtin_amdgcn_raw_buffer_load_b8(rva, c, 0, kStreamOnce);  // 0 past the mask (or without one)
}

// The queries' B operand of k-step ks for column tile nc: slot 16 nc + j, dims 32 g + 8 ks .. +7.
__device__ __forceinline__ bf16x8 s16_q(const uint16_t* qs, int slot, int g, int ks) {
  return __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(qs + slot * kStrQRow + 32 * g + 8 * ks));
}

// One tile's online-softmax update and P.V product on the 16 x 16 layout. y[nc]: the lane's 8 scores of column tile
// nc (log2 units, -inf masked), in the key order kappa; pw: a factor on p for the P.V product only (the fp32 path's
// V scales); vf(dt): the V'^T A operand of d-tile dt (shared by the column tiles). The max over a slot's keys runs
// over the lane's 8 scores and the 4 lane groups g that hold the same column.
template <int NC, bool PW, class VF>
__device__ __forceinline__ void s16_update(float (&y)[NC][8], const float (&pw)[8], float (&m_run)[NC],
                                           float (&l_run)[NC], v4f_t (&o)[NC][8], VF&& vf) {
  bf16x8 bh[NC], bl[NC];
#pragma unroll
  for (int nc = 0; nc < NC; ++nc) {
    float mx = y[nc][0];
#pragma unroll
    for (int i = 1; i < 8; ++i) mx = fmaxf(mx, y[nc][i]);
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const bool move = mx > m_run[nc] + kSlack;  // lazy: p = exp2(y - m) <= 2^kSlack otherwise
    if (__builtin_amdgcn_ballot_w64(move) != 0) {
      const float a = move ? __builtin_amdgcn_exp2f(m_run[nc] - mx) : 1.0f;  // m_run = -inf: 0
#pragma unroll
      for (int dt = 0; dt < 8; ++dt)
#pragma unroll
        for (int i = 0; i < 4; ++i) o[nc][dt][i] *= a;
      l_run[nc] *= a;
      if (move) m_run[nc] = mx;
    }
    const float msub = m_run[nc] == -INFINITY ? 0.0f : m_run[nc];
    float pr[8];
    float ls = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      pr[i] = __builtin_amdgcn_exp2f(y[nc][i] - msub);
      ls += pr[i];
    }
    l_run[nc] += ls;
    uint32_t hw[4], lw[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float a = PW ? pr[2 * e] * pw[2 * e] : pr[2 * e];
      const float b = PW ? pr[2 * e + 1] * pw[2 * e + 1] : pr[2 * e + 1];
      hw[e] = pk_bf16(a, b);
      lw[e] = pk_bf16(a - __uint_as_float(hw[e] << 16), b - __uint_as_float(hw[e] & 0xffff0000u));
    }
    bh[nc] = __builtin_bit_cast(bf16x8, make_uint4(hw[0], hw[1], hw[2], hw[3]));
    bl[nc] = __builtin_bit_cast(bf16x8, make_uint4(lw[0], lw[1], lw[2], lw[3]));
  }
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) {
    const bf16x8 a = vf(dt);
#pragma unroll
    for (int nc = 0; nc < NC; ++nc) {
      o[nc][dt] = mfma16(a, bh[nc], o[nc][dt]);
      o[nc][dt] = mfma16(a, bl[nc], o[nc][dt]);
    }
  }
}

// One state tile (32 keys) of the 16 x 16 stream.
template <int DQ, int NC>
__device__ __forceinline__ void s16_state_tile(const S16Tile& tl, const uint16_t* qs, StrKeyLds& kl, float c2,
                                               int lane, bool key_ok, float (&m_run)[NC], float (&l_run)[NC],
                                               v4f_t (&o)[NC][8]) {
  const int j = lane & 15, g = lane >> 4, c = lane & 31;
  // the tile's per-key factors through LDS into the layouts that read them (in-order LDS access within the wave;
  // lanes c and c + 32 write the same value)
  reinterpret_cast<float*>(kl.f[0])[c] = DQ == OD_DEQUANT_BF16 ? bf16_round(tl.vs) : tl.vs;
  if constexpr (DQ == OD_DEQUANT_FP32) reinterpret_cast<float*>(kl.f[1])[c] = tl.ks * c2;
  float sk[2] = {0.0f, 0.0f};  // the bf16 K scales of the lane's keys kb + j and kb + 16 + j
  if constexpr (DQ == OD_DEQUANT_BF16) {
    sk[0] = bf16_round(__shfl(tl.ks, j, 64));
    sk[1] = bf16_round(__shfl(tl.ks, 16 + j, 64));
  }
  v4f_t s[NC][2];
#pragma unroll
  for (int nc = 0; nc < NC; ++nc) s[nc][0] = s[nc][1] = v4f_t{0, 0, 0, 0};
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
    for (int kr = 0; kr < 2; ++kr) {
      const uint4 w = tl.k[2 * kr + (ks >> 1)];
      const uint32_t w0 = (ks & 1) ? w.z : w.x, w1 = (ks & 1) ? w.w : w.y;
      uint4 a;
      if constexpr (DQ == OD_DEQUANT_BF16) {
        i8x4_times_bf16(w0, sk[kr], a.x, a.y);
        i8x4_times_bf16(w1, sk[kr], a.z, a.w);
      } else {
        i8x4_to_bf16(w0, a.x, a.y);
        i8x4_to_bf16(w1, a.z, a.w);
      }
#pragma unroll
      for (int nc = 0; nc < NC; ++nc)
        s[nc][kr] = mfma16(__builtin_bit_cast(bf16x8, a), s16_q(qs, 16 * nc + j, g, ks), s[nc][kr]);
    }
  }
  // keys 16 kr + 4 g + i: masked keys (past the state's length or by kvalid) from one ballot (bit k: key kb + k)
  const uint32_t vm = (uint32_t)__builtin_amdgcn_ballot_w64(key_ok);
  const float4 fv[2] = {kl.f[0][g], kl.f[0][4 + g]};
  float4 gk[2] = {make_float4(c2, c2, c2, c2), make_float4(c2, c2, c2, c2)};
  if constexpr (DQ == OD_DEQUANT_FP32) {
    gk[0] = kl.f[1][g];
    gk[1] = kl.f[1][4 + g];
  }
  float y[NC][8], f[8];
#pragma unroll
  for (int kr = 0; kr < 2; ++kr)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[4 * kr + i] = f4_at(fv[kr], i);
#pragma unroll
      for (int nc = 0; nc < NC; ++nc) y[nc][4 * kr + i] = s[nc][kr][i] * f4_at(gk[kr], i);
    }
  if (vm != 0xffffffffu) {
#pragma unroll
    for (int kr = 0; kr < 2; ++kr) {
      const uint32_t bits = vm >> (16 * kr + 4 * g);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (!((bits >> i) & 1u))
#pragma unroll
          for (int nc = 0; nc < NC; ++nc) y[nc][4 * kr + i] = -INFINITY;
    }
  }
  auto vf = [&](int dt) {
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i0 = 2 * e, i1 = 2 * e + 1;
      const uint32_t x0 = dt < 4 ? tl.v[i0].x : tl.v[i0].y, x1 = dt < 4 ? tl.v[i1].x : tl.v[i1].y;
      if constexpr (DQ == OD_DEQUANT_BF16)
        w[e] = pk_bf16(byte_times(x0, dt & 3, f[i0]), byte_times(x1, dt & 3, f[i1]));
      else
        w[e] = pk_bf16(byte_times(x0, dt & 3, 1.0f), byte_times(x1, dt & 3, 1.0f));
    }
    return __builtin_bit_cast(bf16x8, make_uint4(w[0], w[1], w[2], w[3]));
  };
  s16_update<NC, DQ == OD_DEQUANT_FP32>(y, f, m_run, l_run, o, vf);
}

// Device-scope coherent store / load of one float (agent-scope relaxed atomics: the access goes to the level all
// XCDs share instead of this XCD's L2), for the split partials the merging workgroup reads. Device-scope fences
// would do the same by writing back and invalidating the whole L2 of every XCD in every workgroup, which measured
// twice as slow on the K/V streams.
__device__ __forceinline__ void str_put(float* a, float v) {
  __hip_atomic_store(a, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float str_get(const float* a) {
  return __hip_atomic_load(const_cast<float*>(a), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// 16 bytes at float offset `off` of the partials, with the device-scope coherence policy (sc1) of the stores and loads
// above; the partials of a call are below 2 GiB (checked by the host), so a 32-bit offset reaches them all
constexpr int kCoherent = 16;  // the sc1 bit of the buffer instructions' cache policy
__device__ __forceinline__ void str_put4(float* part, int off, float4 v) {
  const auto r = __builtin_amdgcn_make_buffer_rsrc(part, (short)0, 0x7fffffff, 0x00020000);
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u, v), r, off * 4, 0, kCoherent);
}
__device__ __forceinline__ float4 str_get4(const float* part, int off) {
  const auto r = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(part), (short)0, 0x7fffffff, 0x00020000);
  return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, off * 4, 0, kCoherent));
}

// The splits of one (state, KV head) after their partials are written: each has stored its partial with the coherent
// policy above, waits until those stores have completed, and counts itself on the (state, head)'s counter
// (device-scope atomic); the workgroup that arrives last reads every split's partial with coherent loads and merges
// them for all slots of the (state, head) with combine_kernel's arithmetic (the same operations in the same order, so
// the result equals the separate merge launch bit for bit), then sets the counter back to zero for the next call.
__device__ __forceinline__ void str_merge_last(const AttnArgs& p, int* counters, int s, int g, int row0, int nslots,
                                               int per_row) {
  __shared__ int last;
  // every thread's coherent partial stores have completed before the workgroup is counted
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  int* ctr = counters + (int64_t)s * p.Hkv + g;
  if (threadIdx.x == 0)
    last = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == p.nsplit - 1;
  __syncthreads();
  if (!last) return;
  constexpr int D = kStrD;
  const int64_t nsl = (int64_t)p.R * p.Hq * p.t;
  const float* lse_p = p.part + (int64_t)p.nsplit * nsl * D;
  // item (slot z, f): the 4 dims 4 f .. 4 f + 3; consecutive threads take consecutive float4 of a slot
  for (int i = threadIdx.x; i < nslots * (D / 4); i += blockDim.x) {
    const int z = i / (D / 4), d0 = (i % (D / 4)) * 4;
    const int zr = z / per_row, zrem = z - zr * per_row;
    const int row = row0 + zr, head = g * p.rep + zrem % p.rep, tok = zrem / p.rep;
    const int64_t slot = ((int64_t)row * p.Hq + head) * p.t + tok;
    float M = -INFINITY;
    float acc[4] = {0, 0, 0, 0};
    float wsum = 0.0f;
    // unrolled, so that every split's LSE and partial are in flight together (one round trip, not one per split)
#pragma unroll 8
    for (int sp = 0; sp < p.nsplit; ++sp) {
      const float l = str_get(lse_p + sp * nsl + slot);
      const float4 a = str_get4(p.part, (int)((sp * nsl + slot) * D + d0));
      if (l == -INFINITY) continue;
      if (l > M) {
        const float r = __expf(M - l);
        wsum *= r;
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[e] *= r;
        M = l;
      }
      const float w = __expf(l - M);
      wsum += w;
      acc[0] += w * a.x; acc[1] += w * a.y; acc[2] += w * a.z; acc[3] += w * a.w;
    }
    const float inv = wsum > 0.0f ? 1.0f / wsum : wsum == 0.0f ? 0.0f : wsum;
    uint16_t* op = p.out + (int64_t)row * p.sor + (int64_t)head * p.soh + (int64_t)tok * p.sot + d0;
    *reinterpret_cast<uint2*>(op) = make_uint2(pk_bf16(acc[0] * inv, acc[1] * inv), pk_bf16(acc[2] * inv, acc[3] * inv));
    if (p.lse && d0 == 0) p.lse[slot] = wsum > 0.0f ? M + __logf(wsum) : wsum == 0.0f ? -INFINITY : wsum;
  }
  if (threadIdx.x == 0) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // for the next call
}

// The stream: workgroup (split sp, KV head hk, state s) with 8 waves; wave w takes tiles t_lo + w, t_lo + w + 8, ...
// of the split's key range, two register sets with loads one tile ahead (a third set measured no faster).
template <int DQ, int NC>
__global__ __launch_bounds__(kStrWaves * 64, NC == 1 ? 2 : 1) void stream_kernel(AttnArgs p) {
  constexpr int D = kStrD;
  constexpr int kSlots = 16 * NC;
  __shared__ __attribute__((aligned(16))) union {
    uint16_t q[32 * kStrQRow];
    float o[kStrWaves][kSlots][D + 4];
  } sm;
  __shared__ float sml[kStrWaves][2][kSlots];
  __shared__ StrKeyLds skl[kStrWaves];
  const int sp = blockIdx.x, hk = blockIdx.y, s = blockIdx.z;
  const int row0 = p.row_start ? p.row_start[s] : 0;
  const int nrows = p.row_start ? p.row_start[s + 1] - row0 : p.R;
  const int per_row = p.t * p.rep;
  const int nslots = nrows * per_row;
  if (nslots <= 0) return;  // uniform over the workgroup
  if (nslots > kSlots) {
    // more slots than the wave's column tiles hold (the caller's max_rows understated this state's rows): NaN
    // outputs, written by split 0 (no split publishes a partial or counts itself)
    if (sp != 0) return;
    for (int i = threadIdx.x; i < nslots * (D / 8); i += blockDim.x) {
      const int z = i / (D / 8), d0 = (i % (D / 8)) * 8;
      const int zr = z / per_row, zrem = z - zr * per_row;
      const int row = row0 + zr, head = hk * p.rep + zrem % p.rep, tk = zrem / p.rep;
      if (row >= p.R) break;
      const int64_t slot_idx = ((int64_t)row * p.Hq + head) * p.t + tk;
      uint16_t* op = p.out + (int64_t)row * p.sor + (int64_t)head * p.soh + (int64_t)tk * p.sot + d0;
      *reinterpret_cast<uint2*>(op) = make_uint2(0x7fc07fc0u, 0x7fc07fc0u);
      *reinterpret_cast<uint2*>(op + 4) = make_uint2(0x7fc07fc0u, 0x7fc07fc0u);
      if (p.lse && d0 == 0) p.lse[slot_idx] = __builtin_nanf("");
    }
    return;
  }
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 15, qd = lane >> 4, c = lane & 31;
  {
    // thread: slot z = tid / 8, dims 16 (tid % 8) .. +15 (rows past the slots are zeros)
    const int z = threadIdx.x >> 3, d0 = (threadIdx.x & 7) * 16;
    if (z < 32) {
      uint4 a = make_uint4(0, 0, 0, 0), b = a;
      if (z < nslots) {
        const int zr = z / per_row, zrem = z - zr * per_row;
        const uint16_t* qp = p.q + (int64_t)(row0 + zr) * p.sqr + (int64_t)(hk * p.rep + zrem % p.rep) * p.sqh +
                             (int64_t)(zrem / p.rep) * p.sqt + d0;
        a = *reinterpret_cast<const uint4*>(qp);
        b = *reinterpret_cast<const uint4*>(qp + 8);
      }
      *reinterpret_cast<uint4*>(sm.q + z * kStrQRow + d0) = a;
      *reinterpret_cast<uint4*>(sm.q + z * kStrQRow + d0 + 8) = b;
    }
  }
  __syncthreads();
  float m_run[NC], l_run[NC];
  v4f_t o[NC][8];
#pragma unroll
  for (int nc = 0; nc < NC; ++nc) {
    m_run[nc] = -INFINITY;
    l_run[nc] = 0.0f;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) o[nc][dt] = v4f_t{0, 0, 0, 0};
  }

  // ---- the state's tiles of this split: [t_lo, t_hi)
  const int n_tiles = (p.T + kStrKeys - 1) / kStrKeys;
  const int tps = (n_tiles + p.nsplit - 1) / p.nsplit;
  const int t_lo = min(n_tiles, sp * tps), t_hi = min(n_tiles, t_lo + tps);
  const int64_t head_base = ((int64_t)s * p.Hkv + hk) * p.cap;
  const StrSrc src{p.kq + head_base * D, p.vq + head_base * D, p.ks + head_base, p.vs + head_base,
                   p.kvalid ? p.kvalid + (int64_t)s * p.T : nullptr, p.T};
  int tt = t_lo + wave;
  if (tt < t_hi) {
    const bool has_valid = p.kvalid != nullptr;
    auto ok = [&](const S16Tile& tl, int t0) { return t0 * kStrKeys + c < p.T && (!has_valid || tl.valid != 0); };
    S16Tile ta, tb;
    s16_load(src, tt * kStrKeys, lane, ta);
    for (;; tt += 2 * kStrWaves) {
      const bool more1 = tt + kStrWaves < t_hi;
      s16_load(src, (more1 ? tt + kStrWaves : tt) * kStrKeys, lane, tb);
      __builtin_amdgcn_sched_barrier(0);
      s16_state_tile<DQ, NC>(ta, sm.q, skl[wave], p.scale_log2, lane, ok(ta, tt), m_run, l_run, o);
      if (!more1) break;
      const bool more2 = tt + 2 * kStrWaves < t_hi;
      s16_load(src, (more2 ? tt + 2 * kStrWaves : tt + kStrWaves) * kStrKeys, lane, ta);
      __builtin_amdgcn_sched_barrier(0);
      s16_state_tile<DQ, NC>(tb, sm.q, skl[wave], p.scale_log2, lane, ok(tb, tt + kStrWaves), m_run, l_run, o);
      if (!more2) break;
    }
  }

  // ---- the rows' own keys: one masked tile of bf16 K/V (key k = row k / t, token k % t), wave 0 of the last split
  if (sp == p.nsplit - 1 && wave == 0) {
    const int n_own = nrows * p.t;
    v4f_t sc[NC][2];
#pragma unroll
    for (int nc = 0; nc < NC; ++nc) sc[nc][0] = sc[nc][1] = v4f_t{0, 0, 0, 0};
#pragma unroll
    for (int kr = 0; kr < 2; ++kr) {
      const int kk = 16 * kr + j;
      const bool kok = kk < n_own;
      const int orow = kok ? kk / p.t : 0, oj = kok ? kk % p.t : 0;
      const uint16_t* kp =
          p.k_own + (int64_t)(row0 + orow) * p.skr + (int64_t)hk * p.skh + (int64_t)oj * p.skt + 32 * qd;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const bf16x8 a =
            __builtin_bit_cast(bf16x8, kok ? *reinterpret_cast<const uint4*>(kp + 8 * ks) : make_uint4(0, 0, 0, 0));
#pragma unroll
        for (int nc = 0; nc < NC; ++nc) sc[nc][kr] = mfma16(a, s16_q(sm.q, 16 * nc + j, qd, ks), sc[nc][kr]);
      }
    }
    float y[NC][8], one[8];
#pragma unroll
    for (int nc = 0; nc < NC; ++nc) {
      const int z = 16 * nc + j;
      const bool zok = z < nslots;
      const int rl = zok ? z / per_row : 0, tok = zok ? (z - rl * per_row) / p.rep : 0;
#pragma unroll
      for (int kr = 0; kr < 2; ++kr)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int kk = 16 * kr + 4 * qd + i;
          const bool vis = zok && kk < n_own && kk >= rl * p.t && kk <= rl * p.t + tok;
          y[nc][4 * kr + i] = vis ? sc[nc][kr][i] * p.scale_log2 : -INFINITY;
        }
    }
    uint4 vo[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      one[i] = 1.0f;
      const int kk = s16_kappa(qd, i);
      vo[i] = make_uint4(0, 0, 0, 0);
      if (kk < n_own) {
        const int orow = kk / p.t, oj = kk % p.t;
        vo[i] = *reinterpret_cast<const uint4*>(p.v_own + (int64_t)(row0 + orow) * p.svr + (int64_t)hk * p.svh +
                                                (int64_t)oj * p.svt + 8 * j);
      }
    }
    auto word = [](const uint4& v, int w) { return w == 0 ? v.x : w == 1 ? v.y : w == 2 ? v.z : v.w; };
    auto vf = [&](int dt) {
      uint32_t w[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t xa = word(vo[2 * e], dt >> 1), xb = word(vo[2 * e + 1], dt >> 1);
        w[e] = (dt & 1) ? ((xa >> 16) | (xb & 0xffff0000u)) : ((xa & 0xffffu) | (xb << 16));
      }
      return __builtin_bit_cast(bf16x8, make_uint4(w[0], w[1], w[2], w[3]));
    };
    s16_update<NC, false>(y, one, m_run, l_run, o, vf);
  }

  // ---- merge the waves (LDS), then this split's normalized partial + LSE, or the output
  float l_tot[NC];
#pragma unroll
  for (int nc = 0; nc < NC; ++nc) {
    l_tot[nc] = l_run[nc] + __shfl_xor(l_run[nc], 16, 64);
    l_tot[nc] += __shfl_xor(l_tot[nc], 32, 64);
  }
  __syncthreads();  // every wave is done with the queries: their LDS now takes the accumulators
  // lane (j, qd) of column tile nc: slot 16 nc + j, dims 32 qd + 8 i + dt in o[nc][dt][i]
#pragma unroll
  for (int nc = 0; nc < NC; ++nc) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float* dst = &sm.o[wave][16 * nc + j][32 * qd + 8 * i];
      *reinterpret_cast<float4*>(dst) = make_float4(o[nc][0][i], o[nc][1][i], o[nc][2][i], o[nc][3][i]);
      *reinterpret_cast<float4*>(dst + 4) = make_float4(o[nc][4][i], o[nc][5][i], o[nc][6][i], o[nc][7][i]);
    }
    if (qd == 0) {
      sml[wave][0][16 * nc + j] = m_run[nc];
      sml[wave][1][16 * nc + j] = l_tot[nc];
    }
  }
  __syncthreads();
  // thread (slot z, j8): the four float4 of dims 4 j8 + 32 e .. +3 (e = 0..3), so that the 8 threads of a slot write
  // whole 128-byte lines of its partial per instruction
  const int z = threadIdx.x >> 3, j8 = threadIdx.x & 7;
  if (z < nslots) {
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kStrWaves; ++w) M = fmaxf(M, sml[w][0][z]);
    float L = 0.0f;
    float4 acc[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[e] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < kStrWaves; ++w) {
        const float mw = sml[w][0][z];
        if (mw == -INFINITY) continue;
        const float a = __builtin_amdgcn_exp2f(mw - M);
        L += a * sml[w][1][z];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float4 v = *reinterpret_cast<const float4*>(&sm.o[w][z][4 * j8 + 32 * e]);
          acc[e].x += a * v.x; acc[e].y += a * v.y; acc[e].z += a * v.z; acc[e].w += a * v.w;
        }
      }
    }
    const int zr = z / per_row, zrem = z - zr * per_row;
    const int64_t slot_idx = ((int64_t)(row0 + zr) * p.Hq + hk * p.rep + zrem % p.rep) * p.t + zrem / p.rep;
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    const float lse_v = L > 0.0f ? (M + __log2f(L)) * kLn2 : -INFINITY;
    if (p.nsplit == 1) {
      uint16_t* op = p.out + (int64_t)(row0 + zr) * p.sor + (int64_t)(hk * p.rep + zrem % p.rep) * p.soh +
                     (int64_t)(zrem / p.rep) * p.sot;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        *reinterpret_cast<uint2*>(op + 4 * j8 + 32 * e) = make_uint2(pk_bf16(acc[e].x * inv, acc[e].y * inv),
                                                                     pk_bf16(acc[e].z * inv, acc[e].w * inv));
      if (p.lse && j8 == 0) p.lse[slot_idx] = lse_v;
    } else {
      const int64_t nsl = (int64_t)p.R * p.Hq * p.t;
      const int base = (int)(((int64_t)sp * nsl + slot_idx) * D);
#pragma unroll
      for (int e = 0; e < 4; ++e)
        str_put4(p.part, base + 4 * j8 + 32 * e,
                 make_float4(acc[e].x * inv, acc[e].y * inv, acc[e].z * inv, acc[e].w * inv));
      if (j8 == 0) str_put(p.part + (int64_t)p.nsplit * nsl * D + (int64_t)sp * nsl + slot_idx, lse_v);
    }
  }
  if (p.nsplit > 1) str_merge_last(p, p.ctr, s, hk, row0, nslots, per_row);
}


}  // namespace

extern "C" int od_branched_attn_stream(const uint16_t* q, int64_t sqr, int64_t sqh, int64_t sqt,
                                       const uint16_t* k_own, int64_t skr, int64_t skh, int64_t skt,
                                       const uint16_t* v_own, int64_t svr, int64_t svh, int64_t svt,
                                       const int8_t* kq, const float* ks, const int8_t* vq, const float* vs,
                                       const uint8_t* kvalid, const int32_t* row_start, int64_t max_rows,
                                       uint16_t* out, int64_t sor, int64_t soh, int64_t sot, float* lse,
                                       int64_t R, int64_t Hq, int64_t Hkv, int64_t t, int64_t D, int64_t Ns,
                                       int64_t T, int64_t cap, float scale, int dequant, int64_t nsplit, float* ws,
                                       int64_t ws_floats, od_stream_t stream) {
  if (dequant != OD_DEQUANT_BF16 && dequant != OD_DEQUANT_FP32) return OD_ERR_UNSUPPORTED;
  if (R < 0 || Hq < 1 || Hkv < 1 || t < 1 || Ns < 1 || T < 0 || cap < T || max_rows < 0) return OD_ERR_SHAPE;
  if (Hq % Hkv || D != kStrD) return OD_ERR_UNSUPPORTED;
  if (!row_start && Ns != 1) return OD_ERR_SHAPE;
  if (nsplit < 1 || nsplit > 256) return OD_ERR_SHAPE;
  if (!row_start) max_rows = R;
  const int64_t rep = Hq / Hkv;
  if (max_rows * t * rep > 32) return OD_ERR_UNSUPPORTED;  // one wave holds all slots of a (state, head)
  if (R == 0 || max_rows == 0) return OD_OK;
  if (!q || !k_own || !v_own || !out) return OD_ERR_NULL;
  if (T > 0 && (!kq || !ks || !vq || !vs)) return OD_ERR_NULL;
  if (nsplit > 1) {
    if (!ws) return OD_ERR_NULL;
    if (ws_floats < nsplit * R * Hq * t * (D + 1) + Ns * Hkv) return OD_ERR_SHAPE;
    if (!od_aligned16(ws)) return OD_ERR_ALIGN;
  }
  const int64_t strides[] = {sqr, sqh, sqt, skr, skh, skt, svr, svh, svt};
  for (int64_t st : strides)
    if (st < 0 || st % 8) return OD_ERR_ALIGN;
  if (sor < 0 || soh < 0 || sot < 0 || sor % 4 || soh % 4 || sot % 4) return OD_ERR_ALIGN;
  if (!od_aligned16(q) || !od_aligned16(k_own) || !od_aligned16(v_own) || (((uintptr_t)out) & 7u)) return OD_ERR_ALIGN;
  if (T > 0 && (!od_aligned16(kq) || !od_aligned16(vq) || (((uintptr_t)ks | (uintptr_t)vs) & 3u))) return OD_ERR_ALIGN;
  if (Hkv > 65535 || Ns > 65535 || R * t * rep > 0x7fffffff || cap * Hkv * Ns * D > (1ll << 40) ||
      nsplit * R * Hq * t * (D + 1) * 4 >= (1ll << 31) || T * D >= (1ll << 31))  // partials: 32-bit byte offsets
    return OD_ERR_SHAPE;
  AttnArgs a{q, k_own, v_own, kq, ks, vq, vs, kvalid, row_start, out, lse, sqr, sqh, sqt, skr, skh, skt, svr, svh,
             svt, sor, soh, sot, (int)R, (int)Hq, (int)Hkv, (int)t, (int)Ns, (int)T, (int)cap, (int)rep,
             scale * 1.4426950408889634f, dequant, (int)nsplit, nsplit > 1 ? ws : nullptr, nullptr, nullptr,
             nullptr, 0, (int)Ns,
             nsplit > 1 ? reinterpret_cast<int*>(ws + nsplit * R * Hq * t * (D + 1)) : nullptr};
  dim3 grid((unsigned)nsplit, (unsigned)Hkv, (unsigned)Ns), block(kStrWaves * 64);
  hipStream_t st = (hipStream_t)stream;
  const bool one_tile = max_rows * t * rep <= 16;  // every (state, head)'s slots fit one 16-column tile
  if (dequant == OD_DEQUANT_BF16) {
    if (one_tile)
      stream_kernel<OD_DEQUANT_BF16, 1><<<grid, block, 0, st>>>(a);
    else
      stream_kernel<OD_DEQUANT_BF16, 2><<<grid, block, 0, st>>>(a);
  } else {
    if (one_tile)
      stream_kernel<OD_DEQUANT_FP32, 1><<<grid, block, 0, st>>>(a);
    else
      stream_kernel<OD_DEQUANT_FP32, 2><<<grid, block, 0, st>>>(a);
  }
  return od_launch_status();
}
