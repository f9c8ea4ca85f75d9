// W8A8 GEMM for gfx950: int8 A [M,K] x int8 W [N,K]^T -> exact int32 accumulators on the CDNA4 int8 matrix
// cores (V_MFMA_I32_32X32X32_I8), then the dequant epilogue out = bf16(float(acc) * sa[m] * sw[n] (+ bias)
// (+ residual)).
//
// Tiling (MFMA-bound at the 9B shapes; one workgroup of 4 waves per CU):
//   * workgroup tile BM x BN = 256 x {256 | 192}; K is staged through LDS in 128-byte slabs, double buffered
//     (2 x (32 KB + BN * 128 B) <= 128 KB of the 160 KB LDS);
//   * global -> LDS with direct-to-LDS buffer loads (16 B per lane, no staging registers); rows past M/N and bytes
//     past K come back as zeros from the buffer range check;
//   * 2 x 2 waves, each owning a 128 x BN/2 sub-tile = 4 x (BN/64) MFMA tiles of 32 x 32 (up to 256 int32
//     accumulators per lane, held in the accumulation registers);
//   * LDS rows are 128 B; the 16-byte chunk c of row r lives at chunk c ^ (r & 7), so the 8 lanes the LDS serves
//     together (rows r..r+7, one logical chunk) hit 8 different bank groups; the swizzle is applied on the global
//     side of the DMA (lane i fetches the chunk that belongs in slot i);
//   * blockIdx -> tile is XCD-aware: the hardware deals workgroups round-robin over the 8 XCDs, so each XCD gets a
//     contiguous range of tiles in a grouped (kGroupM tile-rows) order, and the tiles one XCD runs together share
//     A/W panels in that XCD's L2;
//   * epilogue: fp32 dequantized values staged through the (now idle) LDS in two 128-row halves, then the
//     residual is added, the value rounded once to bf16 and stored 4 columns per lane, a wave per row segment;
//   * the exact int32 accumulators (parity / debug) come from a separate instantiation that only writes them.
// int32 accumulation is exact for K < 133,144 (|acc| <= 127^2 K < 2^31), so any correct GEMM is bit-exact.
#include "od_common.h"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr int kThreads = 256;
constexpr int BM = 256;
constexpr int BK = 128;
constexpr int kGroupM = 4;
constexpr int kOOB = 0x7ffffff0;  // a buffer offset past any range: the load returns zeros

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

__device__ __forceinline__ int swz(int row, int chunk) { return row * BK + ((chunk ^ (row & 7)) << 4); }

// DMA of a ROWS x 128 B slab (rows row0.., bytes k0..k0+127) into LDS. Per wave instruction, lane l writes LDS
// bytes [base + 16 l, base + 16 l + 16): LDS chunk index cid = i * 256 + wave * 64 + lane, row = cid / 8,
// physical chunk = cid % 8, which holds logical chunk (cid % 8) ^ (row & 7).
template <int ROWS>
__device__ __forceinline__ void dma_slab(__amdgpu_buffer_rsrc_t rsrc, int64_t ld, int64_t k0, int64_t K,
                                         int8_t* lds) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
  for (int i = 0; i < ROWS * 8 / kThreads; ++i) {
    const int cid = i * kThreads + wave * 64 + lane;
    const int row = cid >> 3;
    const int lchunk = (cid & 7) ^ (row & 7);
    const int64_t gk = k0 + (lchunk << 4);
    const int off = gk < K ? (int)(row * ld + gk) : kOOB;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void*)(lds + (i * kThreads + wave * 64) * 16), 16, off, 0, 0,
                                             0);
  }
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

template <int BN, bool ACC_ONLY>
__global__ __launch_bounds__(kThreads, 1) void w8a8_gemm_kernel(GemmArgs p) {
  constexpr int TM = 4;              // 32-row MFMA tiles per wave (128 rows)
  constexpr int TN = BN / 64;        // 32-col MFMA tiles per wave (BN / 2 cols)
  constexpr int kSlabA = BM * BK, kSlabB = BN * BK;
  __shared__ __attribute__((aligned(16))) int8_t lds[2 * (kSlabA + kSlabB)];

  int tm, tn;
  tile_of(blockIdx.x, p.tiles_m, p.tiles_n, tm, tn);
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const bool vec8 = (p.ldo % 4 == 0) && ((((uintptr_t)p.out) & 7u) == 0);

  const int64_t rows_a = min((int64_t)BM, p.M - m0), rows_b = min((int64_t)BN, p.N - n0);
  const __amdgpu_buffer_rsrc_t ra =
      __builtin_amdgcn_make_buffer_rsrc((void*)(p.a + m0 * p.lda), (short)0, (int)((rows_a - 1) * p.lda + p.K),
                                        0x00020000);
  const __amdgpu_buffer_rsrc_t rb =
      __builtin_amdgcn_make_buffer_rsrc((void*)(p.w + n0 * p.ldw), (short)0, (int)((rows_b - 1) * p.ldw + p.K),
                                        0x00020000);

  v16i acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = v16i{0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};

  const int nk = (int)((p.K + BK - 1) / BK);
  dma_slab<BM>(ra, p.lda, 0, p.K, lds);
  dma_slab<BN>(rb, p.ldw, 0, p.K, lds + 2 * kSlabA);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) {
      dma_slab<BM>(ra, p.lda, (int64_t)(kt + 1) * BK, p.K, lds + (cur ^ 1) * kSlabA);
      dma_slab<BN>(rb, p.ldw, (int64_t)(kt + 1) * BK, p.K, lds + 2 * kSlabA + (cur ^ 1) * kSlabB);
    }
    const int8_t* la = lds + cur * kSlabA;
    const int8_t* lb = lds + 2 * kSlabA + cur * kSlabB;
#pragma unroll
    for (int s = 0; s < BK / 32; ++s) {
      const int chunk = s * 2 + (lane >> 5);
      v4i fa[TM], fb[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int row = wm * 128 + i * 32 + (lane & 31);
        fa[i] = *reinterpret_cast<const v4i*>(la + swz(row, chunk));
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int row = wn * (BN / 2) + j * 32 + (lane & 31);
        fb[j] = *reinterpret_cast<const v4i*>(lb + swz(row, chunk));
      }
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  }

  // Epilogue. C layout of a 32x32 MFMA tile: lane l holds column l % 32 and rows 8*(r/4) + 4*(l/32) + r%4.
  if constexpr (ACC_ONLY) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int64_t n = n0 + wn * (BN / 2) + j * 32 + (lane & 31);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t m = m0 + wm * 128 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
          if (m < p.M && n < p.N) p.acc[m * p.ldacc + n] = acc[i][j][r];
        }
    }
    return;
  }
  // Scales into LDS (the main loop ended with a barrier, so the LDS is free).
  __shared__ float s_sa[BM], s_sw[BN], s_bias[BN];
  for (int i = threadIdx.x; i < BM; i += kThreads) s_sa[i] = (m0 + i < p.M) ? p.sa[m0 + i] : 0.0f;
  for (int i = threadIdx.x; i < BN; i += kThreads) {
    const bool ok = n0 + i < p.N;
    s_sw[i] = ok ? p.sw[n0 + i] : 0.0f;
    s_bias[i] = (ok && p.bias) ? od_bf16_to_f32(p.bias[n0 + i]) : 0.0f;
  }
  // Two halves of 128 rows: the waves of half h write their fp32 values ((acc * sa) * sw + bias) into an LDS
  // tile [128][BN] (16-byte chunks swizzled by row & 7); then every thread adds the residual, rounds once to
  // bf16 and stores 4 columns (8 B) per step, a wave covering 256 contiguous columns of a row.
  float* ft = reinterpret_cast<float*>(lds);
  constexpr int kC4 = BN / 4;  // 16-byte chunks per fp32 row
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    __syncthreads();
    if (wm == half) {
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int nl = wn * (BN / 2) + j * 32 + (lane & 31);
        const float swn = s_sw[nl], bn = s_bias[nl];
#pragma unroll
        for (int i = 0; i < TM; ++i) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int ml = i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);  // row within the half
            float y = (float)acc[i][j][r] * s_sa[half * 128 + ml];
            y = y * swn;
            y = y + bn;
            ft[ml * BN + (((nl >> 2) ^ (ml & 7)) << 2) + (nl & 3)] = y;
          }
        }
      }
    }
    __syncthreads();
    for (int id = threadIdx.x; id < 128 * kC4; id += kThreads) {
      const int ml = id / kC4, c = id % kC4;
      const int64_t m = m0 + half * 128 + ml, n = n0 + c * 4;
      if (m >= p.M || n >= p.N) continue;
      const float4 v = *reinterpret_cast<const float4*>(ft + ml * BN + ((c ^ (ml & 7)) << 2));
      float y[4] = {v.x, v.y, v.z, v.w};
      if (p.residual) {
        const uint16_t* rr = p.residual + m * p.ldr + n;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (n + e < p.N) y[e] = y[e] + od_bf16_to_f32(rr[e]);
      }
      uint16_t* dst = p.out + m * p.ldo + n;
      if (vec8 && n + 4 <= p.N) {
        const uint32_t lo = (uint32_t)od_f32_to_bf16(y[0]) | ((uint32_t)od_f32_to_bf16(y[1]) << 16);
        const uint32_t hi = (uint32_t)od_f32_to_bf16(y[2]) | ((uint32_t)od_f32_to_bf16(y[3]) << 16);
        *reinterpret_cast<uint2*>(dst) = make_uint2(lo, hi);
      } else {
        for (int e = 0; e < 4 && n + e < p.N; ++e) dst[e] = od_f32_to_bf16(y[e]);
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
  if (acc) {
    if (use192) {
      w8a8_gemm_kernel<192, true><<<grid, block, 0, st>>>(p);
    } else {
      w8a8_gemm_kernel<256, true><<<grid, block, 0, st>>>(p);
    }
    const int rc = od_launch_status();
    if (rc != OD_OK) return rc;
  }
  if (out) {
    if (use192) {
      w8a8_gemm_kernel<192, false><<<grid, block, 0, st>>>(p);
    } else {
      w8a8_gemm_kernel<256, false><<<grid, block, 0, st>>>(p);
    }
  }
  return od_launch_status();
}
