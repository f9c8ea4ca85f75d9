// W8A8 GEMM for gfx950: int8 A [M,K] x int8 W [N,K]^T -> exact int32 accumulators on the CDNA4 int8 matrix
// cores (V_MFMA_I32_32X32X32_I8), then the dequant epilogue out = bf16(float(acc) * sa[m] * sw[n] (+ bias)
// (+ residual)).
//
// Tiling (MFMA-bound at the 9B shapes; one workgroup of 8 waves per CU):
//   * workgroup tile BM x BN = 256 x {256 | 192}; K streams through LDS in 64-byte slabs, 4 stages deep
//     (4 x (16 KB + BN * 64 B) <= 128 KB of the 160 KB LDS). Global -> LDS uses direct-to-LDS buffer loads (16 B
//     per lane, no staging registers) issued 3 stages ahead; a stage is waited for with a vmcnt that leaves the
//     newer stages in flight, then one barrier. Rows past M/N and bytes past K read as zeros (buffer range check).
//   * every stage (A slab + W slab) is its own __shared__ array: the compiler can then tell that an LDS read of
//     stage s does not alias the DMA filling stage s + 3 and does not serialize them.
//   * 4 x 2 waves (2 per SIMD, so one wave's MFMAs cover the other's LDS latency), each owning a 64 x BN/2
//     sub-tile = 2 x (BN/64) MFMA tiles of 32 x 32 (up to 128 int32 accumulators per lane).
//   * LDS rows are 64 B (4 chunks of 16 B); chunk c of row r is stored at chunk c ^ ((r >> 1) & 3), so the 8 lanes
//     the LDS serves together (rows r..r+7, one logical chunk) hit 8 different bank groups; the swizzle is applied
//     on the global side of the DMA (lane i fetches the chunk that belongs in slot i).
//   * blockIdx -> tile is XCD-aware: workgroups are dealt round-robin over the 8 XCDs, so each XCD gets a contiguous
//     range of tiles in a grouped (kGroupM tile-rows) order, and the tiles one XCD runs together share A/W panels
//     in its L2.
//   * epilogue: each wave stages its accumulators 32 rows at a time through a private LDS band and writes 4
//     columns per lane, a wave covering whole row segments; scales, bias and residual are applied in fp32 in the
//     oracle's order and rounded once to bf16. No workgroup barrier after the one that ends the main loop.
// int32 accumulation is exact for K < 133,144 (|acc| <= 127^2 K < 2^31), so any correct GEMM is bit-exact.
#include <type_traits>

#include "od_common.h"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr int kWM = 4, kWN = 2;            // wave grid of a workgroup
constexpr int kThreads = 64 * kWM * kWN;   // 512
constexpr int BM = 256;
constexpr int BK = 64;       // bytes of K per stage
constexpr int kStages = 4;
constexpr int kGroupM = 4;
constexpr int kOOB = 0x7ffffff0;  // a buffer offset past any range: the load returns zeros

template <int N>
using IC = std::integral_constant<int, N>;

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
};

// Chunk swizzle of the 64-byte LDS rows. An operand read is a ds_read_b128 in which lanes 16g..16g+15 take 16
// consecutive rows at one logical chunk, and gfx950 serves 16 lanes of a ds_read_b128 per cycle from 64 4-byte
// banks (a 256-byte period): rows r and r + 4 share their bank set unless their chunks differ, so the chunk is
// XORed with bits 2..3 of the row, which makes the 16 reads of a group land on 16 distinct 16-byte bank quads.
__device__ __forceinline__ int chunk_xor(int row) { return (row >> 2) & 3; }

// byte offset of logical 16-byte chunk c (0..3) of row r inside a stage buffer
__device__ __forceinline__ int swz(int row, int chunk) { return row * BK + ((chunk ^ chunk_xor(row)) << 4); }

template <int N>
__device__ __forceinline__ void wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Workgroup barrier without a memory fence: the stage waits are explicit vmcnt waits (a fenced __syncthreads would
// wait for every DMA in flight, including the stages being prefetched). The "memory" clobber keeps the compiler
// from moving LDS accesses across it.
__device__ __forceinline__ void barrier() { asm volatile("s_barrier" ::: "memory"); }

// DMA of a ROWS x 64 B slab into LDS. Per wave instruction, lane l writes LDS bytes [base + 16 l, +16): LDS chunk
// index cid = i * 256 + wave * 64 + lane, row = cid / 4, physical chunk = cid % 4, which holds logical chunk
// (cid % 4) ^ chunk_xor(row). The per-lane part of the global offset (row * ld + 16 * logical chunk) is fixed
// for the whole K loop (voff[i]); the k0 of the slab goes in the instruction's scalar offset. With KTAIL (K not a
// multiple of the slab) chunks past K are sent out of the buffer's range and read as zeros.
// A slab of ROWS x 64 B is ROWS / 16 wave-instructions of 64 lanes x 16 B, dealt round-robin to the waves: wave w
// issues instruction i * kWaves + w for i = 0, 1, ... while it is below ROWS / 16.
constexpr int kWaves = kWM * kWN;

template <int ROWS>
__device__ __forceinline__ constexpr int slab_iters() { return (ROWS / 16 + kWaves - 1) / kWaves; }

// DMA instructions wave w issues for one ROWS-row slab
template <int ROWS>
__device__ __forceinline__ int slab_loads(int wave) {
  constexpr int n = ROWS / 16;
  return n / kWaves + (wave < n % kWaves ? 1 : 0);
}

template <int ROWS>
struct SlabOffsets {
  int v[slab_iters<ROWS>()];
  int col[slab_iters<ROWS>()];  // byte column of the chunk inside the slab
  __device__ __forceinline__ void init(int64_t ld) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < slab_iters<ROWS>(); ++i) {
      const int cid = (i * kWaves + wave) * 64 + lane;
      const int row = cid >> 2;
      col[i] = ((cid & 3) ^ chunk_xor(row)) << 4;
      v[i] = (int)(row * ld) + col[i];
    }
  }
};

// One direct-to-LDS 16-byte load per lane: LDS[m0 + 16 lane] = buffer[voff + soff]. Written as inline assembly so
// that the compiler's wait-count pass does not see it: the compiler would otherwise wait for every DMA in flight
// before the next LDS read (it cannot always tell the stage buffers apart), collapsing the pipeline. The waits for
// these loads are the explicit vmcnt waits of the pipeline. m0 is not used by anything else in this kernel.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t rsrc, uint32_t lds_base, int voff, int soff) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :
               : "s"(lds_base), "v"(voff), "s"(rsrc), "s"(soff)
               : "memory", "m0");
}

__device__ __forceinline__ uint32_t lds_addr(const int8_t* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) int8_t*)p;
}

// DMA of a ROWS x 64 B slab into LDS. Lane l of wave-instruction q writes LDS bytes [16 (64 q + l), +16): chunk
// index cid = 64 q + l, row = cid / 4, physical chunk = cid % 4, holding logical chunk (cid % 4) ^ chunk_xor(row).
// The per-lane part of the global offset (row * ld + 16 * logical chunk) is fixed for the whole K loop (so.v); the
// k0 of the slab goes in the instruction's scalar offset. With KTAIL (K not a multiple of the slab) chunks past K
// are sent out of the buffer's range and read as zeros.
template <int ROWS, bool KTAIL>
__device__ __forceinline__ void dma_slab(__amdgpu_buffer_rsrc_t rsrc, const SlabOffsets<ROWS>& so, int k0, int K,
                                         int8_t* lds) {
  const int wave = threadIdx.x >> 6;
#pragma unroll
  for (int i = 0; i < slab_iters<ROWS>(); ++i) {
    const int q = i * kWaves + wave;
    if ((ROWS / 16) % kWaves != 0 && q >= ROWS / 16) break;  // wave-uniform
    int voff = so.v[i];
    if constexpr (KTAIL) voff = (k0 + so.col[i] < K) ? voff : kOOB;
    dma16(rsrc, __builtin_amdgcn_readfirstlane(lds_addr(lds + q * 64 * 16)), voff, k0);
  }
}

// Instruction i (0 .. slab_iters - 1) of this wave's share of dma_slab, if the wave has one (wave-uniform).
template <int ROWS, bool KTAIL>
__device__ __forceinline__ void dma_one(__amdgpu_buffer_rsrc_t rsrc, const SlabOffsets<ROWS>& so, int i, int k0, int K,
                                        int8_t* lds) {
  const int q = i * kWaves + (threadIdx.x >> 6);
  if ((ROWS / 16) % kWaves != 0 && q >= ROWS / 16) return;
  int voff = so.v[i];
  if constexpr (KTAIL) voff = (k0 + so.col[i] < K) ? voff : kOOB;
  dma16(rsrc, __builtin_amdgcn_readfirstlane(lds_addr(lds + q * 64 * 16)), voff, k0);
}

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

template <int BN, bool ACC_ONLY, bool GENERAL>
__global__ __launch_bounds__(kThreads, 1) void w8a8_gemm_kernel(GemmArgs p) {
  constexpr int kRowsW = BM / kWM, kColsW = BN / kWN;  // a wave's sub-tile
  constexpr int TM = kRowsW / 32;    // 32-row MFMA tiles per wave
  constexpr int TN = kColsW / 32;    // 32-col MFMA tiles per wave
  constexpr int kSlabA = BM * BK, kSlabB = BN * BK;
  // DMA instructions this wave issues per stage (the W slab of BN = 192 does not split evenly over the waves)
  constexpr int kLoadsHi = BM / 16 / kWaves + (BN / 16 + kWaves - 1) / kWaves;
  constexpr int kLoadsLo = BM / 16 / kWaves + (BN / 16) / kWaves;
  // stage buffers: A slab at offset 0, W slab at offset kSlabA (four LDS objects: the compiler tracks DMA into each)
  __shared__ __attribute__((aligned(16))) int8_t s0[kSlabA + kSlabB], s1[kSlabA + kSlabB], s2[kSlabA + kSlabB],
      s3[kSlabA + kSlabB];

  int tm, tn;
  tile_of(blockIdx.x, p.tiles_m, p.tiles_n, tm, tn);
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / kWN, wn = wave % kWN;

  const int64_t rows_a = min((int64_t)BM, p.M - m0), rows_b = min((int64_t)BN, p.N - n0);
  const __amdgpu_buffer_rsrc_t ra =
      __builtin_amdgcn_make_buffer_rsrc((void*)(p.a + m0 * p.lda), (short)0, (int)((rows_a - 1) * p.lda + p.K),
                                        0x00020000);
  const __amdgpu_buffer_rsrc_t rb =
      __builtin_amdgcn_make_buffer_rsrc((void*)(p.w + n0 * p.ldw), (short)0, (int)((rows_b - 1) * p.ldw + p.K),
                                        0x00020000);

  auto abuf = [&](auto I) -> int8_t* {
    if constexpr (decltype(I)::value == 0) return s0;
    else if constexpr (decltype(I)::value == 1) return s1;
    else if constexpr (decltype(I)::value == 2) return s2;
    else return s3;
  };
  auto bbuf = [&](auto I) -> int8_t* { return abuf(I) + kSlabA; };
  SlabOffsets<BM> soa;
  SlabOffsets<BN> sob;
  soa.init(p.lda);
  sob.init(p.ldw);
  const int K = (int)p.K;
  auto issue = [&](auto I, int kt) {
    dma_slab<BM, GENERAL>(ra, soa, kt * BK, K, abuf(I));
    dma_slab<BN, GENERAL>(rb, sob, kt * BK, K, bbuf(I));
  };
  // the same DMA one instruction at a time: j < slab_iters<BM> is A instruction j, then the W instructions
  constexpr int kDmaA = slab_iters<BM>(), kDma = kDmaA + slab_iters<BN>();
  auto issue_one = [&](auto I, int kt, int j) {
    if (j < kDmaA) dma_one<BM, GENERAL>(ra, soa, j, kt * BK, K, abuf(I));
    else dma_one<BN, GENERAL>(rb, sob, j - kDmaA, kt * BK, K, bbuf(I));
  };

  v16i acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = v16i{0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};

  const int nk = (int)((p.K + BK - 1) / BK);
  const bool hi = slab_loads<BM>(wave) + slab_loads<BN>(wave) == kLoadsHi;  // wave-uniform
  // wait until at most `newer` stages issued after the awaited one are still in flight (this wave's DMAs)
  auto wait_stage = [&](int newer) {
    if (newer >= 2) {
      if (hi) wait_vm<2 * kLoadsHi>(); else wait_vm<2 * kLoadsLo>();
    } else if (newer == 1) {
      if (hi) wait_vm<kLoadsHi>(); else wait_vm<kLoadsLo>();
    } else {
      wait_vm<0>();
    }
  };
  // operand fragments of k-step s (32 of the stage's 64 k) of one stage buffer
  auto frags = [&](const int8_t* la, const int8_t* lb, int s, v4i (&fa)[TM], v4i (&fb)[TN]) {
    const int chunk = s * 2 + (lane >> 5);
#pragma unroll
    for (int i = 0; i < TM; ++i) fa[i] = *reinterpret_cast<const v4i*>(la + swz(wm * kRowsW + i * 32 + (lane & 31), chunk));
#pragma unroll
    for (int j = 0; j < TN; ++j) fb[j] = *reinterpret_cast<const v4i*>(lb + swz(wn * kColsW + j * 32 + (lane & 31), chunk));
  };
  auto mma = [&](const v4i (&fa)[TM], const v4i (&fb)[TN]) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
  };
  // The MFMAs of one k-step with the refill DMA of stage I (k-tile kt) spread between them, one instruction after
  // every TM*TN/kDma MFMAs: issued as one burst right after the barrier, the DMAs of all 8 waves fill the
  // texture-address queue and the waves stall at issue instead of running their MFMAs.
  auto mma_dma = [&](const v4i (&fa)[TM], const v4i (&fb)[TN], auto I, int kt, bool refill) {
    constexpr int kMf = TM * TN;
#pragma unroll
    for (int x = 0; x < kMf; ++x) {
      acc[x / TN][x % TN] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[x / TN], fb[x % TN], acc[x / TN][x % TN], 0, 0, 0);
#pragma unroll
      for (int j = 0; j < kDma; ++j)
        if (j * kMf / kDma == x && refill) issue_one(I, kt, j);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // Pipeline. Stage buffer I % 4 holds k-tile I; three k-tiles are in flight ahead of the one being computed.
  // Fragments are register double-buffered across k-steps and across stages: step kt loads k-step 1 of its
  // stage, runs k-step 0, then (once stage kt+1 has landed for every wave: own vmcnt wait + barrier) loads k-step 0
  // of stage kt+1 and runs k-step 1 while refilling the buffer of k-tile kt-1 with k-tile kt+3 (every wave is past
  // its last read of kt-1: those reads fed MFMAs issued before the barrier). LDS latency is thus always
  // covered by 8 MFMAs of the same wave.
  v4i f0a[TM], f0b[TN], f1a[TM], f1b[TN];
  issue(IC<0>{}, 0);
  if (nk > 1) issue(IC<1>{}, 1);
  if (nk > 2) issue(IC<2>{}, 2);
  wait_stage(min(2, nk - 1));
  barrier();
  frags(abuf(IC<0>{}), bbuf(IC<0>{}), 0, f0a, f0b);

  auto step = [&](auto I, int kt) {
    if (kt >= nk) return;
    constexpr int kI = decltype(I)::value, kN = (kI + 1) % kStages, kR = (kI + 3) % kStages;
    frags(abuf(I), bbuf(I), 1, f1a, f1b);
    __builtin_amdgcn_sched_barrier(0);  // keep the reads ahead of the MFMAs they overlap
    mma(f0a, f0b);
    // Unconditional also on the last k-tile (then it reads an idle, in-bounds stage buffer whose values are
    // never used): a branch here would merge two paths with different numbers of LDS reads in flight, and the
    // compiler's lgkmcnt wait before k-step 1 would then also wait for the reads of the next stage.
    wait_stage(min(1, nk - 2 - kt));
    barrier();
    frags(abuf(IC<kN>{}), bbuf(IC<kN>{}), 0, f0a, f0b);
    __builtin_amdgcn_sched_barrier(0);
    mma_dma(f1a, f1b, IC<kR>{}, kt + 3, kt + 3 < nk);
  };

  for (int kt = 0; kt < nk; kt += kStages) {
    step(IC<0>{}, kt);
    step(IC<1>{}, kt + 1);
    step(IC<2>{}, kt + 2);
    step(IC<3>{}, kt + 3);
  }
  __syncthreads();  // every wave is done reading the stage buffers; each now reuses one as its private band

  // Epilogue, in two passes per band of 32 rows of the wave's kRowsW x kColsW sub-tile.
  //  1. In the MFMA result layout (lane l holds column l % 32 of each 32x32 tile and rows
  //     8*(r/4) + 4*(l/32) + r%4), t = (float(acc) * sa[m]) * sw[n] (the raw int32 with ACC_ONLY) goes to a private
  //     LDS band (32 x kColsW 4-byte words; wave w uses half w % 2 of stage buffer w / 2). A lane needs one sw per
  //     column tile and 16 sa per band, loaded up front.
  //  2. Row-major: lane l takes the 4 columns 4 (l % kC4) .. +3 of rows l / kC4 + kRowsPass * it, so its bias
  //     values are fixed for the tile; y = bf16((t + bias) + residual), the same fp32 operation order as the
  //     unfused product, with one rounding. Rows go in groups of 4 whose residual loads issue together.
  // The epilogue runs once per tile, so its code is kept small (it is fetched anew for every tile): only the
  // GENERAL variant carries the scalar paths for unaligned rows and a ragged last column group.
  int8_t* stage_of_wave = (wave >> 1) == 0 ? s0 : (wave >> 1) == 1 ? s1 : (wave >> 1) == 2 ? s2 : s3;
  constexpr int kCols = kColsW;               // columns of the wave's sub-tile
  constexpr int kC4 = kCols / 4;              // 4-column chunks per row
  constexpr int kRowsPass = 64 / kC4;         // rows one pass of the wave covers
  constexpr int kPasses = (32 + kRowsPass - 1) / kRowsPass;
  static_assert(kPasses % 4 == 0, "row groups of 4");
  constexpr int kBand = 32 * kCols * 4;       // bytes of one band
  static_assert(2 * kBand <= kSlabA + kSlabB, "epilogue bands do not fit");
  uint32_t* band = reinterpret_cast<uint32_t*>(stage_of_wave + (wave & 1) * kBand);
  const int64_t n_w = n0 + wn * kCols;
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
    const int64_t m_band = m0 + wm * kRowsW + i * 32;
    float sav[16];
#pragma unroll
    for (int r = 0; r < 16; ++r)
      sav[r] = ACC_ONLY ? 0.0f : p.sa[min(m_band + 8 * (r >> 2) + 4 * h + (r & 3), p.M - 1)];
#pragma unroll
    for (int j = 0; j < TN; ++j) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = 8 * (r >> 2) + 4 * h + (r & 3);
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
#pragma unroll 1
    for (int it0 = 0; it0 < kPasses; it0 += 4) {
      uint2 res[4];
      if (!ACC_ONLY && p.residual) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const uint16_t* rp = p.residual + min(m_band + kRowsPass * (it0 + u) + rr, p.M - 1) * p.ldr;
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
        const int64_t m = m_band + row;
        if (row >= 32 || m >= p.M) continue;
        const uint4 v = *reinterpret_cast<const uint4*>(band + row * kCols + 4 * c4);
        if constexpr (ACC_ONLY) {
          int32_t* dst = p.acc + m * p.ldacc + n;
          if constexpr (GENERAL) {
            const uint32_t vv[4] = {v.x, v.y, v.z, v.w};
            for (int e = 0; e < 4 && n + e < p.N; ++e) dst[e] = (int32_t)vv[e];
          } else {
            *reinterpret_cast<uint4*>(dst) = v;
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
  if (K % 16 || lda % 16 || ldw % 16 || !od_aligned16(a) || !od_aligned16(w)) return OD_ERR_ALIGN;
  if (K >= 133144) return OD_ERR_UNSUPPORTED;  // int32 accumulators could overflow
  // buffer offsets are 32-bit: one tile's A panel (256 rows) and W panel must stay below 2 GiB
  if ((int64_t)BM * lda >= (1ll << 31) || (int64_t)256 * ldw >= (1ll << 31)) return OD_ERR_UNSUPPORTED;
  GemmArgs p{a, sa, w, sw, bias, residual, out, acc, lda, ldw, ldr, ldo, ldacc, M, N, K, 0, 0};
  const int64_t tiles_m = (M + BM - 1) / BM;
  // BN: 256, or 192 when that takes fewer tile-widths of work at 256 workgroups per wave (e.g. N = 6144).
  const int64_t t256 = tiles_m * ((N + 255) / 256), t192 = tiles_m * ((N + 191) / 192);
  const int64_t cost256 = ((t256 + 255) / 256) * 256, cost192 = ((t192 + 255) / 256) * 192;
  const bool use192 = cost192 < cost256;
  const int64_t tiles_n = use192 ? (N + 191) / 192 : (N + 255) / 256;
  if (tiles_m * tiles_n > 0x7fffffff) return OD_ERR_SHAPE;
  p.tiles_m = (int)tiles_m;
  p.tiles_n = (int)tiles_n;
  dim3 grid((unsigned)(tiles_m * tiles_n)), block(kThreads);
  hipStream_t st = (hipStream_t)stream;
  // The fast variant needs whole k-tiles and 4-column output groups that are 8-byte (bf16) / 16-byte (int32)
  // aligned; anything else takes the GENERAL variant.
  auto al = [](const void* q, unsigned a) { return (((uintptr_t)q) & (a - 1)) == 0; };
  const bool fast_k = K % BK == 0 && N % 4 == 0;
  const bool fast_out = fast_k && ldo % 4 == 0 && al(out, 8) && al(bias, 8) && ldr % 4 == 0 && al(residual, 8);
  const bool fast_acc = fast_k && ldacc % 4 == 0 && al(acc, 16);
  auto launch = [&](auto BNc, auto ACCc, auto GENc) {
    w8a8_gemm_kernel<decltype(BNc)::value, decltype(ACCc)::value, decltype(GENc)::value><<<grid, block, 0, st>>>(p);
  };
  auto launch2 = [&](auto ACCc, bool general) {
    if (use192) {
      general ? launch(IC<192>{}, ACCc, std::true_type{}) : launch(IC<192>{}, ACCc, std::false_type{});
    } else {
      general ? launch(IC<256>{}, ACCc, std::true_type{}) : launch(IC<256>{}, ACCc, std::false_type{});
    }
  };
  if (acc) {
    launch2(std::true_type{}, !fast_acc);
    const int rc = od_launch_status();
    if (rc != OD_OK) return rc;
  }
  if (out) launch2(std::false_type{}, !fast_out);
  return od_launch_status();
}
