// Flash attention over bf16 K/V (the wide_attention contract), for gfx950.
//
// Math (src/opendecider/wide_attention.py:13-67): queries are the last T of S key positions (query t sits at
// position t + S - T); with causal it sees keys 0 .. t + S - T, kvalid (B, S) masks keys, GQA head h reads KV group
// h / (H / G). Online softmax in the exp2 domain over 64-key blocks, as the reference's kernel: s = (q.k) * scale *
// log2(e), m, l, acc as FlashAttention-2 (the running max exact, moved by every block that raises it); P is rounded to
// bf16 before the P.V product (the reference's p.to(v.dtype)); out = acc / l, 0 for a query with no visible key;
// LSE = (m + log2 l) ln 2, -inf for such a query. p = exp2(s scale log2(e) - m) is formed with one rounding (an fma)
// where the reference rounds the product first: the same p up to its last bit. The scale must be positive (the max
// is taken on the unscaled scores).
//
// Work decomposition. A "slot" is one (token, head of the KV group) pair, slot z -> token z / rep, head
// g * rep + z % rep (the reference's row order). Grid = (slot tiles of 128, B * G); a workgroup of 4 waves owns 128
// consecutive slots of one (batch, KV group) and streams that group's K/V once for all of them; a wave owns 32.
//
// Layout trick (as in the branched kernel): scores are computed transposed, S^T = K Q^T, on
// V_MFMA_F32_32X32X16_BF16 with the 32 keys of a key tile as rows and the wave's 32 slots as columns, so the online
// softmax is lane-local, and the probabilities sit where O^T += V^T P^T wants its B operand; its A operand holds V^T
// with the keys in the score layout's order (bits 2 and 3 of the key index swapped inside each 16-key group). Q is
// held in registers (the reduction dimension DK is padded with zeros to DKP).
//
// Two paths: the LDS-DMA path (DK = 64, 128 or 256 with 128 value columns per pass: the decoder's prefill, 256-wide
// heads in two halves) copies K and V rows straight into LDS and reads V^T out of the row-major block with
// transposing LDS reads; the register-staged path (any other shape) passes each block through registers and stores
// V transposed.
#include "od_common.h"

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;
constexpr int kSlotsPerTile = 128;
constexpr int kBK = 64;  // keys per block (2 key tiles of 32)
constexpr float kLn2 = 0.693147180559945309f;

struct WideArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const uint8_t* kvalid;
  uint16_t* out;
  float* lse;
  int64_t sqb, sqh, sqt, skb, skg, sks, svb, svg, svs, sob, soh, sot, smb;
  int H, G, T, S, DK, rep, causal;
  float scale_log2;
  int dv_half;  // value columns blockIdx.z * dv_half .. +dv_half of a wider head (0: one launch covers DV)
};

template <int DKP, int DV, int NBUF>
struct alignas(16) WSmem {
  alignas(16) uint16_t k[NBUF][kBK * DKP];   // [key][d], 16-byte chunks swizzled (wk_off)
  alignas(16) uint16_t vt[NBUF][DV * kBK];   // [d][permuted key], 16-byte chunks swizzled (wvt_off)
  alignas(16) float kb[NBUF][kBK];           // 0, or -inf for a key out of range or masked by kvalid
  int mk[NBUF];                              // the block has a key out of range or masked (its kb row is needed)
};

// LDS swizzles for gfx950's banking (reads: 64 4-byte banks, 16 lanes of a ds_read_b128 per cycle; writes: a
// 128-byte period, 8 lanes of a ds_write_b128 or 16 of a ds_write_b64 per cycle). A fragment read has lanes
// 16i .. 16i+15 take 16 consecutive rows at one logical chunk:
//  * K rows are 2 DKP bytes (DKP/8 chunks): for DKP >= 128 every row starts a 256-byte period and the chunk is XORed
//    with key & 15; for DKP = 64 two rows share a period and it is XORed with (key >> 1) & 7;
//  * V^T rows are 128 bytes (8 chunks of 8 keys): XOR with ((d >> 1) ^ (d >> 3)) & 7, a bijection on 8
//    consecutive even (or odd) d and on {8 dg + e} for 8 consecutive dg, which the transposing store uses (wvmap).
template <int DKP>
__device__ __forceinline__ int wk_x(int key) {
  return DKP == 64 ? ((key >> 1) & 7) : (key & 15);
}
template <int DKP>
__device__ __forceinline__ int wk_off(int key, int chunk) {
  return key * DKP + ((chunk ^ wk_x<DKP>(key)) << 3);
}
__device__ __forceinline__ int wvt_off(int d, int chunk) {
  return d * kBK + ((chunk ^ (((d >> 1) ^ (d >> 3)) & 7)) << 3);
}
// position of key j (0..63) inside its V^T row: bits 2 and 3 swapped
__device__ __forceinline__ int wjj_of(int j) { return (j & ~12) | ((j & 4) << 1) | ((j & 8) >> 1); }

// Thread -> (d group dg of 8 d, key group kg of 4 keys) for the transposing V store, for 128 d (16 dg x 16 kg over
// 256 threads). Lanes 16i .. 16i+15 form one ds_write_b64 bank cycle: lane bits 0..2 pick 8 consecutive dg (8
// distinct chunks after the V^T swizzle) and bit 3 flips bit 1 of kg, the half of the 16-byte chunk its 4 keys
// occupy, so the 16 lanes write 16 distinct 8-byte slots. DV = 64 uses threads 0..127 (dg < 8), DV = 256 runs the
// map twice with dg + 16 (d + 128 leaves the swizzle's low bits unchanged).
__device__ __forceinline__ void wvmap(int tid, int& dg, int& kg) {
  const int lo = tid & 7, t3 = (tid >> 3) & 1, hi = tid >> 4;
  dg = lo | ((hi & 1) << 3);
  kg = (t3 << 1) | ((hi >> 1) & 1) | ((hi >> 2) << 2);
}

template <int DV>
__device__ __forceinline__ void wvmap_dv(int tid, int& dg, int& kg, bool& on) {
  if constexpr (DV == 64) {
    // 8 dg x 16 kg over threads 0..127 (same lane pattern with bit 3 of dg taken from bit 4 of the thread)
    const int lo = tid & 7, t3 = (tid >> 3) & 1, hi = tid >> 4;
    dg = lo;
    kg = (t3 << 1) | (hi & 1) | ((hi >> 1) << 2);
    on = tid < 128;
  } else {
    wvmap(tid, dg, kg);
    on = true;
  }
}

constexpr int kVPairs(int DV) { return DV == 256 ? 2 : 1; }

template <int DKP, int DV>
struct BlockRegs {
  uint4 k[(kBK * DKP / 8 + kThreads - 1) / kThreads];
  uint4 v[kVPairs(DV)][4];
  int ok;  // thread < 64: key tid valid
};

// One block's K / V rows through buffer descriptors based at the block's first key and bounded by the keys that
// exist (S - j0 rows): rows past S read as zeros without a per-lane check, and the per-lane offsets (key * stride +
// chunk) are the same for every block, so no 64-bit address stays live across the loop.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rows_rsrc(const uint16_t* base, int64_t stride, int64_t rows) {
  const int64_t bytes = rows * stride * 2;
  return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, (int)(bytes < 0x7fffffff ? bytes : 0x7fffffff),
                                           0x00020000);
}

template <int DKP, int DV>
__device__ __forceinline__ void block_load(const WideArgs& p, int b, int g, int j0, BlockRegs<DKP, DV>& r) {
  const int tid = threadIdx.x;
  const uint16_t* kbase = p.k + (int64_t)b * p.skb + (int64_t)g * p.skg + (int64_t)j0 * p.sks;
  const uint16_t* vbase = p.v + (int64_t)b * p.svb + (int64_t)g * p.svg + (int64_t)j0 * p.svs;
  const __amdgpu_buffer_rsrc_t rk = rows_rsrc(kbase, p.sks, p.S - j0), rv = rows_rsrc(vbase, p.svs, p.S - j0);
  constexpr int kCpk = DKP / 8;                 // 16-byte chunks per key
  constexpr int kChunks = kBK * kCpk;
#pragma unroll
  for (int i = 0; i < (kChunks + kThreads - 1) / kThreads; ++i) {
    const int cid = i * kThreads + tid;
    const int key = cid / kCpk, c = cid % kCpk;
    r.k[i] = make_uint4(0, 0, 0, 0);
    if (cid < kChunks && 8 * c < p.DK)
      r.k[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rk, (int)(key * p.sks * 2 + 16 * c), 0, 0));
  }
  int dg, kg;
  bool on;
  wvmap_dv<DV>(tid, dg, kg, on);
#pragma unroll
  for (int hp = 0; hp < kVPairs(DV); ++hp) {
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const int key = 4 * kg + a;
      r.v[hp][a] = make_uint4(0, 0, 0, 0);
      if (on)
        r.v[hp][a] = __builtin_bit_cast(
            uint4, __builtin_amdgcn_raw_buffer_load_b128(rv, (int)(key * p.svs * 2 + 16 * (dg + 16 * hp)), 0, 0));
    }
  }
  r.ok = 0;
  if (tid < kBK) {
    const int j = j0 + tid;
    r.ok = j < p.S && (!p.kvalid || p.kvalid[(int64_t)b * p.smb + j] != 0);
  }
}

template <int DKP, int DV, int NBUF>
__device__ __forceinline__ void block_store(WSmem<DKP, DV, NBUF>& sm, int buf, const BlockRegs<DKP, DV>& r) {
  const int tid = threadIdx.x;
  constexpr int kCpk = DKP / 8;
  constexpr int kChunks = kBK * kCpk;
#pragma unroll
  for (int i = 0; i < (kChunks + kThreads - 1) / kThreads; ++i) {
    const int cid = i * kThreads + tid;
    if (cid < kChunks) *reinterpret_cast<uint4*>(&sm.k[buf][wk_off<DKP>(cid / kCpk, cid % kCpk)]) = r.k[i];
  }
  int dg, kg;
  bool on;
  wvmap_dv<DV>(tid, dg, kg, on);
  if (on) {
    const int jj0 = wjj_of(4 * kg);
#pragma unroll
    for (int hp = 0; hp < kVPairs(DV); ++hp) {
      const uint32_t w[4][4] = {{r.v[hp][0].x, r.v[hp][0].y, r.v[hp][0].z, r.v[hp][0].w},
                                {r.v[hp][1].x, r.v[hp][1].y, r.v[hp][1].z, r.v[hp][1].w},
                                {r.v[hp][2].x, r.v[hp][2].y, r.v[hp][2].z, r.v[hp][2].w},
                                {r.v[hp][3].x, r.v[hp][3].y, r.v[hp][3].z, r.v[hp][3].w}};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        // element e of the 4 keys: bf16 halves of dword e / 2
        const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
        uint2 hv;
        hv.x = __builtin_amdgcn_perm(w[1][e >> 1], w[0][e >> 1], sel);
        hv.y = __builtin_amdgcn_perm(w[3][e >> 1], w[2][e >> 1], sel);
        const int d = 8 * (dg + 16 * hp) + e;
        *reinterpret_cast<uint2*>(&sm.vt[buf][wvt_off(d, jj0 >> 3) + (jj0 & 7)]) = hv;
      }
    }
  }
  if (tid < kBK) {
    sm.kb[buf][tid] = r.ok ? 0.0f : -INFINITY;
    const bool all_ok = __builtin_amdgcn_ballot_w64(r.ok != 0) == ~0ull;  // wave 0 holds the block's 64 keys
    if (tid == 0) sm.mk[buf] = all_ok ? 0 : 1;
  }
}

// The three pieces of one 64-key block for the wave's 32 slots (kBK = 2 key tiles of 32):
//  * wide_qk: S^T = K Q^T from the block's K rows in LDS (wk_off layout);
//  * wide_softmax: the online-softmax update of the block's scores into P (bf16) with the running max, sum and
//    output rescale; kb / masked: the block's key bias row and whether it is needed;
//  * wide_pv: O^T += V^T P^T, the A operand from vfrag(dt, kk): value rows dt * 32 + (lane & 31) and the 16 keys
//    of k-step kk (key 16 kk + 8 (i / 4) + 4 (lane / 32) + i % 4 in element i, the order of the score layout), made
//    of VR LDS reads.
// Fragment reads run RA fragments ahead of the MFMAs that consume them (one fragment = one MFMA operand), through a
// ring of RA + 1 fragments.
constexpr int wide_ra(int DKP, int DV) { return DKP + DV <= 192 ? 2 : 1; }

template <int DKP, int DV>
__device__ __forceinline__ void wide_qk(const uint16_t* kblk, const bf16x8 (&qf)[DKP / 16], v16f (&s)[kBK / 32]) {
  const int lane = threadIdx.x & 63;
  const int h = lane >> 5, col = lane & 31;
  constexpr int KT = kBK / 32;
  constexpr int KS = DKP / 16;
  constexpr int RA = wide_ra(DKP, DV);
#pragma unroll
  for (int kt = 0; kt < KT; ++kt) s[kt] = v16f{0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
  {
    constexpr int NQ = KS * KT;  // MFMA i: k-step i / KT, key tile i % KT
    bf16x8 kf[RA + 1];
    auto kread = [&](int i) {
      kf[i % (RA + 1)] = *reinterpret_cast<const bf16x8*>(&kblk[wk_off<DKP>((i % KT) * 32 + col, (i / KT) * 2 + h)]);
    };
#pragma unroll
    for (int i = 0; i < RA; ++i) kread(i);
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      if (i + RA < NQ) kread(i + RA);
      s[i % KT] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[i % (RA + 1)], qf[i / KT], s[i % KT], 0, 0, 0);
    }
    // keep the reads RA MFMAs ahead (left alone, the scheduler sinks each read to its MFMA)
    __builtin_amdgcn_sched_group_barrier(0x100, RA, 0);
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      if (i + RA < NQ) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    }
  }
}

template <int DV>
__device__ __forceinline__ void wide_softmax(v16f (&s)[kBK / 32], const float* kb, int masked, float scale_log2,
                                             float& m_run, float& l_run, v16f (&o)[DV / 32], bool check_causal,
                                             int j0, int qpos, bf16x8 (&pb)[kBK / 16]) {
  const int h = (threadIdx.x & 63) >> 5;
  constexpr int KT = kBK / 32;
  // Masked keys (raw score + -inf) and keys past a query's causal limit drop out first; then FlashAttention-2's
  // update with the exact running max, as the reference's kernel: m' = max(m, max y) with y = s scale log2(e) (the
  // max is taken on the raw scores: a positive scale preserves order under rounding, so it is bitwise the max of the
  // rounded products), p = exp2(s scale log2(e) - m') in one rounding (fma), rounded to bf16 for P.V,
  // l' = l exp2(m - m') + sum p, O' = O exp2(m - m'). This lane's slot sees keys kt*32 + 8*(r/4) + 4*h + r%4.
  // O is only multiplied when some slot of the wave moved its max (otherwise the factor is exactly 1).
  if (__builtin_amdgcn_readfirstlane(masked)) {
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
  if (check_causal) {
#pragma unroll
    for (int kt = 0; kt < KT; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (j0 + kt * 32 + 8 * (r >> 2) + 4 * h + (r & 3) > qpos) s[kt][r] = -INFINITY;
  }
  float mraw = -INFINITY;
#pragma unroll
  for (int kt = 0; kt < KT; ++kt)
#pragma unroll
    for (int r = 0; r < 16; ++r) mraw = fmaxf(mraw, s[kt][r]);
  const float mloc = od_xor32_max(mraw) * scale_log2;
  const bool moved = mloc > m_run;
  const float m_new = moved ? mloc : m_run;
  const float m_safe = m_new == -INFINITY ? 0.0f : m_new;
  const bool any_moved = __builtin_amdgcn_ballot_w64(moved) != 0;
  const float alpha = moved ? __builtin_amdgcn_exp2f(m_run - m_safe) : 1.0f;
  float psum = 0.0f;
#pragma unroll
  for (int kt = 0; kt < KT; ++kt)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float pr = __builtin_amdgcn_exp2f(fmaf(s[kt][r], scale_log2, -m_safe));
      psum += pr;
      pb[kt * 2 + (r >> 3)][r & 7] = (__bf16)pr;
    }
  l_run = l_run * alpha + od_xor32_sum(psum);
  m_run = m_new;
  if (any_moved) {
#pragma unroll
    for (int dt = 0; dt < DV / 32; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[dt][r] *= alpha;
  }
}

template <int DKP, int DV, int VR, typename VFrag>
__device__ __forceinline__ void wide_pv(VFrag&& vfrag, const bf16x8 (&pb)[kBK / 16], v16f (&o)[DV / 32]) {
  constexpr int KT = kBK / 32;
  constexpr int RA = wide_ra(DKP, DV);
  {
    constexpr int NV = 2 * KT * (DV / 32);  // MFMA i: k-step i / (DV / 32), d tile i % (DV / 32)
    bf16x8 vf[RA + 1];
    auto vread = [&](int i) { vf[i % (RA + 1)] = vfrag(i % (DV / 32), i / (DV / 32)); };
#pragma unroll
    for (int i = 0; i < RA; ++i) vread(i);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      if (i + RA < NV) vread(i + RA);
      o[i % (DV / 32)] =
          __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf[i % (RA + 1)], pb[i / (DV / 32)], o[i % (DV / 32)], 0, 0, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x100, RA * VR, 0);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      if (i + RA < NV) __builtin_amdgcn_sched_group_barrier(0x100, VR, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    }
  }
}

// One whole block: scores, softmax, P.V. `mid` runs between the softmax and the P.V product: the register-staged
// kernel issues the next block's global loads there, so that their registers are not held through the score and
// softmax phases.
template <int DKP, int DV, int VR, typename VFrag, typename Mid>
__device__ __forceinline__ void wide_block(const uint16_t* kblk, const float* kb, int masked, VFrag&& vfrag,
                                           const bf16x8 (&qf)[DKP / 16], float scale_log2, float& m_run,
                                           float& l_run, v16f (&o)[DV / 32], bool check_causal, int j0, int qpos,
                                           Mid&& mid) {
  v16f s[kBK / 32];
  bf16x8 pb[kBK / 16];
  wide_qk<DKP, DV>(kblk, qf, s);
  wide_softmax<DV>(s, kb, masked, scale_log2, m_run, l_run, o, check_causal, j0, qpos, pb);
  mid();
  wide_pv<DKP, DV, VR>(vfrag, pb, o);
}

// A workgroup's place in the grid and what each lane owns before the key loop.
struct WideTile {
  int b, g;           // batch, KV group
  int slot_ok;        // the lane's slot exists
  int tok, head, qpos;
  int nb;             // 64-key blocks the tile sees
  int free_until;     // a block whose last key is at or below this position needs no causal check (for the wave)
};

// Work item of the workgroup: SPT consecutive slots of one (batch, KV group), 32 per wave. Returns false for a
// workgroup past the last slot tile (uniform over the workgroup).
template <int SPT>
__device__ __forceinline__ bool wide_tile(WideArgs& p, WideTile& t) {
  // a head of 2 DV value columns in two halves (blockIdx.z): each half recomputes the same scores and softmax and
  // accumulates its own columns, so both halves' outputs are those of one pass over all columns; half 0 writes LSE
  if (p.dv_half) {
    p.v += blockIdx.z * p.dv_half;
    p.out += blockIdx.z * p.dv_half;
    if (blockIdx.z) p.lse = nullptr;
  }
  // XCD-aware order: workgroups are dealt round-robin over the 8 XCDs (flat id f runs on XCD f % 8); work item
  // w = bg * tiles + tile goes to XCD (w's range), so the slot tiles of one (batch, KV group) share an L2 for the
  // K/V they all stream. A bijection of [0, tiles * B G). Causal with the queries' own triangle at least half of
  // the keys (a prefill): a tile's work grows with its index, so each (batch, group) deals its tiles last first and
  // the light tiles fill the end instead of the heaviest ones (4 x 4096-token causal prefill, 32 / 8 heads of 128: 761 -> 703 us).
  const int tiles = gridDim.x, total = gridDim.x * gridDim.y;
  const int f = blockIdx.x + blockIdx.y * tiles;
  const int per = total >> 3, rem = total & 7, xcd = f & 7, local = f >> 3;
  const int w = xcd < rem ? xcd * (per + 1) + local : rem * (per + 1) + (xcd - rem) * per + local;
  const int bg = w / tiles;
  t.b = bg / p.G;
  t.g = bg % p.G;
  const int nslots = p.T * p.rep;
  const int tile = p.causal && 2 * p.T >= p.S ? tiles - 1 - w % tiles : w % tiles;
  const int slot_base = tile * SPT;
  if (slot_base >= nslots) return false;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int z = slot_base + wave * 32 + (lane & 31);
  t.slot_ok = z < nslots;
  t.tok = t.slot_ok ? z / p.rep : p.T - 1;
  t.head = t.g * p.rep + (t.slot_ok ? z % p.rep : 0);
  const int shift = p.S - p.T;
  t.qpos = t.tok + shift;
  // keys this tile can see: causal stops after the last token's position
  const int last = min(slot_base + SPT, nslots) - 1;
  const int tok_hi = last / p.rep;
  const int kend = p.causal ? min(p.S, tok_hi + shift + 1) : p.S;
  t.nb = (kend + kBK - 1) / kBK;
  t.free_until = (slot_base + wave * 32) / p.rep + shift;
  return true;
}

// query fragments: lane holds Q[slot][ks*16 + 8h .. +8], zero past DK
template <int DKP>
__device__ __forceinline__ void wide_q(const WideArgs& p, const WideTile& t, bf16x8 (&qf)[DKP / 16]) {
  const int h = (threadIdx.x & 63) >> 5;
  const uint16_t* qp = p.q + (int64_t)t.b * p.sqb + (int64_t)t.head * p.sqh + (int64_t)t.tok * p.sqt;
#pragma unroll
  for (int ks = 0; ks < DKP / 16; ++ks) {
    uint4 raw = make_uint4(0, 0, 0, 0);
    if (t.slot_ok && ks * 16 + 8 * h < p.DK) raw = *reinterpret_cast<const uint4*>(qp + ks * 16 + 8 * h);
    qf[ks] = __builtin_bit_cast(bf16x8, raw);
  }
}

// out = acc / l (0 where l = 0), lse = (m + log2 l) ln 2
template <int DV>
__device__ __forceinline__ void wide_epilogue(const WideArgs& p, const WideTile& t, const v16f (&o)[DV / 32],
                                              float m_run, float l_run) {
  if (!t.slot_ok) return;
  const int h = (threadIdx.x & 63) >> 5;
  uint16_t* op = p.out + (int64_t)t.b * p.sob + (int64_t)t.head * p.soh + (int64_t)t.tok * p.sot;
  const float den = l_run == 0.0f ? 1.0f : l_run;
#pragma unroll
  for (int dt = 0; dt < DV / 32; ++dt) {
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      const int d0 = dt * 32 + 8 * r4 + 4 * h;
      const uint32_t lo = (uint32_t)od_f32_to_bf16(o[dt][4 * r4] / den) |
                          ((uint32_t)od_f32_to_bf16(o[dt][4 * r4 + 1] / den) << 16);
      const uint32_t hi = (uint32_t)od_f32_to_bf16(o[dt][4 * r4 + 2] / den) |
                          ((uint32_t)od_f32_to_bf16(o[dt][4 * r4 + 3] / den) << 16);
      *reinterpret_cast<uint2*>(op + d0) = make_uint2(lo, hi);
    }
  }
  if (p.lse && h == 0)
    p.lse[((int64_t)t.b * p.H + t.head) * p.T + t.tok] = (m_run + __log2f(l_run)) * kLn2;
}

// Register-staged path (any DK up to 512, DV 64 / 128 / 256): each block's K / V pass through registers; V is
// transposed on its way into LDS.
template <int DKP, int DV, int NBUF, int OCC>
__global__ __launch_bounds__(kThreads, OCC) void wide_attn_kernel(WideArgs p) {
  __shared__ WSmem<DKP, DV, NBUF> sm;
  WideTile t;
  if (!wide_tile<kSlotsPerTile>(p, t)) return;
  const int lane = threadIdx.x & 63;
  const int h = lane >> 5, col = lane & 31;
  bf16x8 qf[DKP / 16];
  wide_q<DKP>(p, t, qf);
  float m_run = -INFINITY, l_run = 0.0f;
  v16f o[DV / 32];
#pragma unroll
  for (int dt = 0; dt < DV / 32; ++dt) o[dt] = v16f{0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
  const int nb = t.nb;
  if (nb > 0) {
    BlockRegs<DKP, DV> br;
    block_load<DKP, DV>(p, t.b, t.g, 0, br);
    block_store<DKP, DV, NBUF>(sm, 0, br);
    __syncthreads();
    for (int blk = 0; blk < nb; ++blk) {
      const int cur = NBUF == 2 ? (blk & 1) : 0;
      const int j0 = blk * kBK;
      wide_block<DKP, DV, 1>(
          sm.k[cur], sm.kb[cur], sm.mk[cur],
          [&](int dt, int kk) {
            return *reinterpret_cast<const bf16x8*>(&sm.vt[cur][wvt_off(dt * 32 + col, 2 * kk + h)]);
          },
          qf, p.scale_log2, m_run, l_run, o, p.causal && j0 + kBK - 1 > t.free_until, j0, t.qpos, [&] {
            if (blk + 1 < nb) block_load<DKP, DV>(p, t.b, t.g, j0 + kBK, br);
          });
      if (blk + 1 < nb) {
        if constexpr (NBUF == 1) __syncthreads();  // every wave is done with the single buffer
        block_store<DKP, DV, NBUF>(sm, NBUF == 2 ? (cur ^ 1) : 0, br);
      }
      __syncthreads();
    }
  }
  wide_epilogue<DV>(p, t, o, m_run, l_run);
}

// ---- LDS-DMA path: DK = DKP in {64, 128, 256}, 128 value columns per pass (DV = 128, or DV = 256 in two halves) ----
//
// Each block's K and V rows go from HBM straight into LDS (buffer_load ... lds, 16 bytes per lane, rows past S read
// as zeros through the buffer range) with no staging registers. One LDS buffer per workgroup (48 / 32 / 24 KB at
// DKP = 256 / 128 / 64), so two workgroups share a CU and one's copy overlaps the other's compute: at DKP = 256 a
// double-buffered workgroup (96 KB) ran alone on its CU and took 1.72x as long (4 x 16 / 4 heads of 256, 4096 causal
// tokens); at DKP = 128 both forms measured within 3%. V stays row-major
// ([key][d]) in LDS; the A operand of O^T += V^T P^T is gathered with ds_read_b64_tr_b16, which hands lane l of
// each 16-lane group element e of the 4 elements at the address of lane 4 e + l / 4 of the group, column l % 4
// (measured): with lane 4 e + c pointing at V[k + e][d + 4 c], lane l receives V[k .. k + 3][d + l]. Two such reads
// (keys k and k + 8) make one operand. Outputs are bit-identical to the register-staged path (same products, same
// order). No spills (176 VGPRs at DKP = 128, against 256 and 10 spilled for the register-staged kernel).
constexpr int kDvT = 128;

template <int DKP>
struct alignas(16) WDSmem {
  alignas(16) uint16_t k[kBK * DKP];   // [key][d], 16-byte chunks swizzled (wk_off)
  alignas(16) uint16_t v[kBK * kDvT];  // [key][d], 16-byte chunk c of key j at chunk c ^ 4 (j & 3)
  alignas(16) float kb[kBK];
  int mk;
};

// The transposing read's 16 lanes touch 4 consecutive keys (j & 3 = 0..3) x 2 chunks of 8 d: XOR-ing the chunk's
// bits 2-3 with j & 3 spreads them over 8 distinct chunks of a 256-byte bank period (16 for the 32 lanes of the two
// groups that differ in d + 16).
__device__ __forceinline__ int wv_chunk(int key, int chunk) { return chunk ^ ((key & 3) << 2); }

// One LDS-DMA load: lane l copies the 16 bytes at byte vo of buffer r to LDS byte lds_base + 16 l (lds_base is
// wave-uniform, passed in M0); bytes past the buffer's range arrive as zeros. Inline asm, so that the compiler does
// not track it: the kernel waits for it (vmcnt) and orders it with barriers itself. M0 is declared clobbered; the
// compiler keeps nothing in M0 in this kernel.
__device__ __forceinline__ void wdma16(__amdgpu_buffer_rsrc_t r, int vo, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(vo), "s"(r),
               "s"(lds_base)
               : "memory", "m0");
}

template <typename T>
__device__ __forceinline__ uint32_t wlds_addr(T* ptr) {
  return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)(ptr);
}

// The A operand for value rows dt * 32 + (lane & 31), keys 16 kk + 8 (i / 4) + 4 (lane / 32) + i % 4 (i = 0..7):
// two transposing reads at the lane's base vb (wv_chunk layout) and 8 keys further.
__device__ __forceinline__ bf16x8 wv_frag(const uint16_t* vblk, int vb, int kk) {
  typedef short v4s __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) v4s lds_v4s;
  uint16_t* base = const_cast<uint16_t*>(vblk) + vb + kk * 16 * kDvT;
  const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)base);
  const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(base + 8 * kDvT));
  return __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

template <int DKP, int OCC>
__global__ __launch_bounds__(kThreads, OCC) void wide_dma_kernel(WideArgs p) {
  constexpr int DV = kDvT;
  constexpr int KI = kBK * DKP * 2 / 4096;  // DMA rounds per block: a round moves 4 KB (16 bytes x 256 lanes)
  constexpr int VI = kBK * DV * 2 / 4096;
  __shared__ WDSmem<DKP> sm;
  WideTile t;
  if (!wide_tile<kSlotsPerTile>(p, t)) return;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave_u = __builtin_amdgcn_readfirstlane(tid >> 6);
  bf16x8 qf[DKP / 16];
  wide_q<DKP>(p, t, qf);
  float m_run = -INFINITY, l_run = 0.0f;
  v16f o[DV / 32];
#pragma unroll
  for (int dt = 0; dt < DV / 32; ++dt) o[dt] = v16f{0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};

  // DMA source offsets, the same for every block: round i, wave w, lane l fills LDS byte 4096 i + 1024 w + 16 l of
  // the block, i.e. (row, chunk slot) of that position, and loads the logical chunk that the swizzle puts there
  int kvo[KI], vvo[VI];
#pragma unroll
  for (int i = 0; i < KI; ++i) {
    const int pe = (4096 * i + 1024 * wave_u + 16 * lane) / 2;
    const int row = pe / DKP, slot = (pe % DKP) / 8;
    kvo[i] = row * (int)p.sks * 2 + 16 * (slot ^ wk_x<DKP>(row));
  }
#pragma unroll
  for (int i = 0; i < VI; ++i) {
    const int pe = (4096 * i + 1024 * wave_u + 16 * lane) / 2;
    const int row = pe / DV, slot = (pe % DV) / 8;
    vvo[i] = row * (int)p.svs * 2 + 16 * wv_chunk(row, slot);
  }
  // transposing-read bases: group g16 = lane / 16 covers value rows + 16 (g16 & 1) and keys + 4 (g16 >> 1); lane
  // 4 e + c of the group points at key e, value columns 4 c .. 4 c + 3 of its 16
  int vb[DV / 32];
  {
    const int hh = lane >> 5, mh = (lane >> 4) & 1, e = (lane >> 2) & 3, c = lane & 3;
#pragma unroll
    for (int dt = 0; dt < DV / 32; ++dt)
      vb[dt] = (4 * hh + e) * DV + (wv_chunk(e, 4 * dt + 2 * mh + (c >> 1)) << 3) + 4 * (c & 1);
  }

  const uint16_t* kg0 = p.k + (int64_t)t.b * p.skb + (int64_t)t.g * p.skg;
  const uint16_t* vg0 = p.v + (int64_t)t.b * p.svb + (int64_t)t.g * p.svg;
  auto issue = [&](int j0) {
    const __amdgpu_buffer_rsrc_t rk = rows_rsrc(kg0 + (int64_t)j0 * p.sks, p.sks, p.S - j0);
    const __amdgpu_buffer_rsrc_t rv = rows_rsrc(vg0 + (int64_t)j0 * p.svs, p.svs, p.S - j0);
    const uint32_t kl = wlds_addr(&sm.k[0]) + 1024 * wave_u, vl = wlds_addr(&sm.v[0]) + 1024 * wave_u;
#pragma unroll
    for (int i = 0; i < KI; ++i) wdma16(rk, kvo[i], kl + 4096 * i);
#pragma unroll
    for (int i = 0; i < VI; ++i) wdma16(rv, vvo[i], vl + 4096 * i);
  };
  // key bias of a block: thread < 64 owns key j0 + thread
  auto key_ok = [&](int j0) {
    int ok = 0;
    if (tid < kBK) {
      const int j = j0 + tid;
      ok = j < p.S && (!p.kvalid || p.kvalid[(int64_t)t.b * p.smb + j] != 0);
    }
    return ok;
  };
  auto put_bias = [&](int ok) {
    if (tid < kBK) {
      sm.kb[tid] = ok ? 0.0f : -INFINITY;
      const bool all_ok = __builtin_amdgcn_ballot_w64(ok != 0) == ~0ull;  // wave 0 holds the block's 64 keys
      if (tid == 0) sm.mk = all_ok ? 0 : 1;
    }
  };

  const int nb = t.nb;
  if (nb > 0) {
    issue(0);
    put_bias(key_ok(0));
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    for (int blk = 0; blk < nb; ++blk) {
      const int j0 = blk * kBK;
      const bool more = blk + 1 < nb;
      const int ok_next = more ? key_ok(j0 + kBK) : 0;
      const uint16_t* vblk = sm.v;
      wide_block<DKP, DV, 2>(
          sm.k, sm.kb, sm.mk, [&](int dt, int kk) { return wv_frag(vblk, vb[dt], kk); }, qf, p.scale_log2, m_run,
          l_run, o, p.causal && j0 + kBK - 1 > t.free_until, j0, t.qpos, [] {});
      if (more) {
        __syncthreads();  // every wave is done with the buffer
        issue(j0 + kBK);
        put_bias(ok_next);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
      }
    }
  }
  wide_epilogue<DV>(p, t, o, m_run, l_run);
}

// Two workgroups per CU (two waves per SIMD; the accumulators in VGPRs: this file is built with the VGPR-only MFMA
// form, which keeps DKP = 256 at 220 VGPRs with no AGPR copies). DV = 256 runs as two 128-column halves (grid.z = 2),
// as on the register-staged path.
template <int DKP>
void launch_wide_dma(WideArgs a, dim3 grid, bool halves, hipStream_t st) {
  if (halves) {
    a.dv_half = kDvT;
    grid.z = 2;
  }
  wide_dma_kernel<DKP, 2><<<grid, dim3(kThreads), 0, st>>>(a);
}

template <int DKP, int DV>
void launch_wide(const WideArgs& a, dim3 grid, hipStream_t st) {
  // LDS: double-buffered K + V^T up to DKP = 256; DKP = 512 is single-buffered (its K block alone is 64 KB).
  // Two workgroups per CU where the registers allow it (Q and O fragments grow with DKP and DV).
  constexpr int NBUF = DKP <= 256 ? 2 : 1;
  constexpr int OCC = (DKP <= 128 && DV <= 128) ? 2 : 1;
  wide_attn_kernel<DKP, DV, NBUF, OCC><<<grid, dim3(kThreads), 0, st>>>(a);
}

// DV = 256 with DK > 128 runs as two DV = 128 halves (grid.z = 2): the 256-column accumulators next to the
// 256-dim query fragments and the block staging registers spill (121 VGPRs, ~100 scratch accesses per 64-key block,
// 4x slower), the halves do not; each half repeats the score MFMAs, 1.5x the FLOPs of one pass.
template <int DKP>
void launch_wide_halves(WideArgs a, dim3 grid, hipStream_t st) {
  a.dv_half = 128;
  grid.z = 2;
  launch_wide<DKP, 128>(a, grid, st);
}

}  // namespace

extern "C" int od_wide_attn(const uint16_t* q, int64_t sqb, int64_t sqh, int64_t sqt, const uint16_t* k, int64_t skb,
                            int64_t skg, int64_t sks, const uint16_t* v, int64_t svb, int64_t svg, int64_t svs,
                            const uint8_t* kvalid, int64_t smb, uint16_t* out, int64_t sob, int64_t soh, int64_t sot,
                            float* lse, int64_t B, int64_t H, int64_t G, int64_t T, int64_t S, int64_t DK, int64_t DV,
                            int causal, float scale, od_stream_t stream) {
  if (B < 0 || H < 1 || G < 1 || T < 0 || S < 0 || DK < 1) return OD_ERR_SHAPE;
  if (H % G) return OD_ERR_SHAPE;
  if (DV != 64 && DV != 128 && DV != 256) return OD_ERR_UNSUPPORTED;
  if (DK > 512) return OD_ERR_UNSUPPORTED;
  if (!(scale > 0.0f) || !(scale < INFINITY)) return OD_ERR_UNSUPPORTED;  // the max is taken on unscaled scores
  if (B == 0 || T == 0) return OD_OK;
  if (!q || !k || !v || !out) return OD_ERR_NULL;
  if (DK % 8) return OD_ERR_ALIGN;
  const int64_t strides[] = {sqb, sqh, sqt, skb, skg, sks, svb, svg, svs};
  for (int64_t s : strides)
    if (s < 0 || s % 8) return OD_ERR_ALIGN;
  if (sob < 0 || soh < 0 || sot < 0 || sob % 4 || soh % 4 || sot % 4 || smb < 0) return OD_ERR_ALIGN;
  if (!od_aligned16(q) || !od_aligned16(k) || !od_aligned16(v) || (((uintptr_t)out) & 7u)) return OD_ERR_ALIGN;
  const int64_t rep = H / G;
  const int64_t tiles = (T * rep + kSlotsPerTile - 1) / kSlotsPerTile;
  if (tiles > 0x7fffffff || B * G > 65535 || T * rep > 0x7fffffff || S > 0x7fffffff - kBK) return OD_ERR_SHAPE;
  WideArgs a{q, k, v, kvalid, out, lse, sqb, sqh, sqt, skb, skg, sks, svb, svg, svs, sob, soh, sot, smb,
             (int)H, (int)G, (int)T, (int)S, (int)DK, (int)rep, causal ? 1 : 0, scale * 1.4426950408889634f, 0};
  dim3 grid((unsigned)tiles, (unsigned)(B * G));
  hipStream_t st = (hipStream_t)stream;
  const int dkp = DK <= 64 ? 64 : DK <= 128 ? 128 : DK <= 256 ? 256 : 512;
  // LDS-DMA path: K rows of exactly DKP (no zero padding to insert), 128 value columns per pass, rows that do not
  // overlap (the buffer range ends at the last row's end) and 64-row block offsets that fit the 32-bit offsets
  const bool dma = DK == dkp && dkp <= 256 && (DV == 128 || (DV == 256 && dkp == 256)) && sks >= DK && svs >= DV &&
                   sks < (1 << 24) && svs < (1 << 24);
  if (dma) {
    if (dkp == 64) launch_wide_dma<64>(a, grid, false, st);
    else if (dkp == 128) launch_wide_dma<128>(a, grid, false, st);
    else launch_wide_dma<256>(a, grid, DV == 256, st);
    return od_launch_status();
  }
  auto by_dv = [&](auto DKc) {
    constexpr int DKP = decltype(DKc)::value;
    if (DV == 64) launch_wide<DKP, 64>(a, grid, st);
    else if (DV == 128) launch_wide<DKP, 128>(a, grid, st);
    else if (DKP > 128) launch_wide_halves<DKP>(a, grid, st);
    else launch_wide<DKP, 256>(a, grid, st);
  };
  if (dkp == 64) by_dv(std::integral_constant<int, 64>{});
  else if (dkp == 128) by_dv(std::integral_constant<int, 128>{});
  else if (dkp == 256) by_dv(std::integral_constant<int, 256>{});
  else by_dv(std::integral_constant<int, 512>{});
  return od_launch_status();
}
