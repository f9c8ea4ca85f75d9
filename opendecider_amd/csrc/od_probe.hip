// Matrix-core and HBM ceiling probes for MI355X (gfx950), used by bench.py to put the GEMM and attention rooflines
// next to what the chip sustains, not only next to the published peaks. Built into their own library
// (libod_probe.so); no part of the scoring path calls them.
//
// One workgroup of 8 waves per CU (two per SIMD, as the W8A8 GEMM runs); each wave issues `iters` rounds of 8
// independent MFMAs into 8 accumulator tiles. Modes:
//   0  int8  V_MFMA_I32_32X32X32_I8, the same register operands every round
//   1  int8, operands changed every round by a few VALU ops (as real data toggles the multipliers)
//   2  int8, operands read from LDS (6 ds_read_b128 per 8 MFMAs, the GEMM's fragment-read ratio at BN = 256)
//   3  bf16  V_MFMA_F32_32X32X16_BF16, operands changed every round
//   4  bf16, operands read from LDS
// Thread 0 of each workgroup samples the core clock counter (s_memtime) and the constant-rate counter
// (s_memrealtime) around the loop, so the mean core clock under the load comes out with the rate.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <vector>

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

constexpr int kThreads = 512;
constexpr int kLds = 65536;

__device__ __forceinline__ void round8(v16i (&acc)[2][4], const v4i (&fa)[2], const v4i (&fb)[4]) {
#pragma unroll
  for (int x = 0; x < 8; ++x) {
    acc[x / 4][x % 4] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[x / 4], fb[x % 4], acc[x / 4][x % 4], 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
  }
}

__device__ __forceinline__ void round8(v16f (&acc)[2][4], const v8bf (&fa)[2], const v8bf (&fb)[4]) {
#pragma unroll
  for (int x = 0; x < 8; ++x) {
    acc[x / 4][x % 4] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[x / 4], fb[x % 4], acc[x / 4][x % 4], 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
  }
}

template <int MODE>
__global__ __launch_bounds__(kThreads, 1) void mfma_probe_kernel(int iters, long long* stamps, int* sink,
                                                                 const int* seed) {
  __shared__ __attribute__((aligned(16))) int8_t lds[kLds];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  // pseudo-random bytes in LDS: thread t writes bytes [128 t, 128 t + 128)
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t o = threadIdx.x * 128 + i * 16;
    const v4i v = {(int)((uint32_t)seed[0] * (o + 1u)), (int)((uint32_t)seed[1] ^ (o * 2654435761u)),
                   (int)(o * 40503u + (uint32_t)seed[2]), (int)((o ^ (uint32_t)seed[3]) * 97u)};
    *reinterpret_cast<v4i*>(lds + o) = v;
  }
  __syncthreads();
  long long t0 = 0, r0 = 0;
  if (threadIdx.x == 0) {
    t0 = __builtin_amdgcn_s_memtime();
    r0 = __builtin_amdgcn_s_memrealtime();
  }
  // fragment f of round it: 16 bytes per lane at ((it * 6 + wave * 8 + f) mod 64) KB-slots, always in bounds
  auto slot = [&](int it, int f) { return (((it * 6 + wave * 8 + f) & 63) << 10) + lane * 16; };
  int s = 0;
  if constexpr (MODE <= 2) {
    v4i fa[2], fb[4], ga[2], gb[4];
#pragma unroll
    for (int i = 0; i < 2; ++i) fa[i] = *reinterpret_cast<const v4i*>(lds + slot(0, i));
#pragma unroll
    for (int j = 0; j < 4; ++j) fb[j] = *reinterpret_cast<const v4i*>(lds + slot(0, 2 + j));
    v16i acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = v16i{};
    for (int it = 0; it < iters; ++it) {
      if constexpr (MODE == 2) {
#pragma unroll
        for (int i = 0; i < 2; ++i) ga[i] = *reinterpret_cast<const v4i*>(lds + slot(it + 1, i));
#pragma unroll
        for (int j = 0; j < 4; ++j) gb[j] = *reinterpret_cast<const v4i*>(lds + slot(it + 1, 2 + j));
      } else if constexpr (MODE == 1) {
        const int u = (int)((uint32_t)it * 0x9e3779b9u);
#pragma unroll
        for (int i = 0; i < 2; ++i) ga[i] = fa[i] ^ (v4i){u, it, it * 7, it * 13};
#pragma unroll
        for (int j = 0; j < 4; ++j) gb[j] = fb[j] + (v4i){u, it * 3, it, it * 5};
      }
      __builtin_amdgcn_sched_barrier(0);
      round8(acc, fa, fb);
      if constexpr (MODE != 0) {
#pragma unroll
        for (int i = 0; i < 2; ++i) fa[i] = ga[i];
#pragma unroll
        for (int j = 0; j < 4; ++j) fb[j] = gb[j];
      }
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) s += acc[i][j][r];
  } else {
    v8bf fa[2], fb[4], ga[2], gb[4];
#pragma unroll
    for (int i = 0; i < 2; ++i) fa[i] = *reinterpret_cast<const v8bf*>(lds + slot(0, i));
#pragma unroll
    for (int j = 0; j < 4; ++j) fb[j] = *reinterpret_cast<const v8bf*>(lds + slot(0, 2 + j));
    v16f acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = v16f{};
    for (int it = 0; it < iters; ++it) {
      if constexpr (MODE == 4) {
#pragma unroll
        for (int i = 0; i < 2; ++i) ga[i] = *reinterpret_cast<const v8bf*>(lds + slot(it + 1, i));
#pragma unroll
        for (int j = 0; j < 4; ++j) gb[j] = *reinterpret_cast<const v8bf*>(lds + slot(it + 1, 2 + j));
      } else {
        // flip low mantissa bits (keeps the values finite)
        const int u = (int)(((uint32_t)it * 0x9e3779b9u) & 0x007f007fu);
#pragma unroll
        for (int i = 0; i < 2; ++i) ga[i] = __builtin_bit_cast(v8bf, __builtin_bit_cast(v4i, fa[i]) ^ (v4i){u, u, u, u});
#pragma unroll
        for (int j = 0; j < 4; ++j) gb[j] = __builtin_bit_cast(v8bf, __builtin_bit_cast(v4i, fb[j]) ^ (v4i){u, u, u, u});
      }
      __builtin_amdgcn_sched_barrier(0);
      round8(acc, fa, fb);
#pragma unroll
      for (int i = 0; i < 2; ++i) fa[i] = ga[i];
#pragma unroll
      for (int j = 0; j < 4; ++j) fb[j] = gb[j];
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) s += (int)acc[i][j][r];
  }
  sink[blockIdx.x * kThreads + threadIdx.x] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    const long long t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
    stamps[4 * blockIdx.x + 0] = t0;
    stamps[4 * blockIdx.x + 1] = t1;
    stamps[4 * blockIdx.x + 2] = r0;
    stamps[4 * blockIdx.x + 3] = r1;
  }
}

// HBM read-bandwidth probe: every thread streams 16-byte pieces of a buffer far larger than the caches (grid-stride,
// 8 loads in flight per thread) and folds them into one word it stores, so that no load can be dropped.
typedef unsigned int v4u __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void hbm_read_kernel(const v4u* __restrict__ src, int64_t n16, int* sink) {
  const int64_t tid = (int64_t)blockIdx.x * 256 + threadIdx.x, stride = (int64_t)gridDim.x * 256;
  uint32_t acc = 0;
  int64_t i = tid;
  for (; i + 7 * stride < n16; i += 8 * stride) {
    v4u v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = __builtin_nontemporal_load(src + i + u * stride);
#pragma unroll
    for (int u = 0; u < 8; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  for (; i < n16; i += stride) {
    const v4u v = src[i];
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  sink[tid] = (int)acc;
}

// The same read as contiguous chunks: workgroup b (8 waves) reads bytes [b chunk, (b + 1) chunk) of the buffer in
// 4 KB pieces, wave w taking pieces w, w + 8, ... with four pieces (16 loads of 16 bytes per lane) in flight, through a
// buffer descriptor bounded to the chunk (the pieces past its end read as zeros, none past the buffer), with the
// non-temporal cache policy; the access pattern of a key-range stream over an int8 state.
__global__ __launch_bounds__(512) void hbm_chunk_kernel(const uint8_t* __restrict__ src, int64_t chunk, int* sink) {
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const auto r = __builtin_amdgcn_make_buffer_rsrc((void*)(src + (int64_t)blockIdx.x * chunk), (short)0, (int)chunk,
                                                   0x00020000);
  const int pieces = (int)(chunk >> 12);
  uint32_t acc = 0;
  for (int pc = wave; pc < pieces; pc += 32) {
    v4u v[16];
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
      for (int u = 0; u < 4; ++u)
        v[4 * k + u] = __builtin_amdgcn_raw_buffer_load_b128(r, ((pc + 8 * k) << 12) + 1024 * u + 16 * lane, 0, 2);
#pragma unroll
    for (int u = 0; u < 16; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  sink[blockIdx.x * 512 + threadIdx.x] = (int)acc;
}

}  // namespace

// Reads a `bytes`-byte device buffer (filled first) with hbm_read_kernel at 4, 8 and 16 workgroups of 4 waves per
// CU and with hbm_chunk_kernel at 1 and 2 workgroups of 8 waves per CU, `reps` timed launches each after a warm-up
// launch, on the current device; synchronous. Writes the best read rate in GB/s (of the bytes each launch reads).
// Returns 0, or -1 (bad argument) / -2 (HIP error).
extern "C" int od_probe_hbm_read(int64_t bytes, int reps, double* gbs) {
  if (bytes < (1 << 24) || bytes % 16 || reps < 1 || !gbs) return -1;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess) return -2;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1) return -2;
  v4u* buf = nullptr;
  int* sink = nullptr;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  int rc = 0;
  double best = 0.0;
  const int64_t n16 = bytes / 16;
  if (hipMalloc(&buf, bytes) != hipSuccess || hipMalloc(&sink, sizeof(int) * 256 * 16 * (size_t)cus) != hipSuccess ||
      hipMemset(buf, 0x5a, bytes) != hipSuccess || hipEventCreate(&e0) != hipSuccess ||
      hipEventCreate(&e1) != hipSuccess) {
    rc = -2;
  }
  // variants 0..2: grid-stride at 4, 8, 16 workgroups per CU; 3, 4: chunks at 1, 2 workgroups per CU
  for (int var = 0; var < 5 && rc == 0; ++var) {
    const int grid = var < 3 ? (4 << var) * cus : (var - 2) * cus;
    const int64_t chunk = (bytes / grid) & ~(int64_t)4095;  // whole 4 KB pieces
    if (var >= 3 && (chunk < 4096 || chunk >= (1ll << 30))) continue;  // 32-bit piece offsets, 24 pieces past the end
    const double read = var < 3 ? (double)bytes : (double)chunk * grid;
    auto launch = [&]() {
      if (var < 3)
        hbm_read_kernel<<<grid, 256>>>(buf, n16, sink);
      else
        hbm_chunk_kernel<<<grid, 512>>>(reinterpret_cast<const uint8_t*>(buf), chunk, sink);
    };
    float ms = 0.0f;
    launch();
    if (hipGetLastError() != hipSuccess || hipDeviceSynchronize() != hipSuccess || hipEventRecord(e0, 0) != hipSuccess) {
      rc = -2;
      break;
    }
    for (int r = 0; r < reps; ++r) launch();
    if (hipGetLastError() != hipSuccess || hipEventRecord(e1, 0) != hipSuccess ||
        hipDeviceSynchronize() != hipSuccess || hipEventElapsedTime(&ms, e0, e1) != hipSuccess || ms <= 0.0f) {
      rc = -2;
      break;
    }
    const double rate = read * reps / (ms * 1e-3) / 1e9;
    if (rate > best) best = rate;
  }
  if (rc == 0) *gbs = best;
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  if (buf) (void)hipFree(buf);
  if (sink) (void)hipFree(sink);
  return rc;
}

// Runs mode `mode` (0..4) with one workgroup per CU for `iters` rounds per wave, after one warm-up launch, on the
// current device; synchronous. Writes the throughput (dense TOPS / TFLOP/s) and the mean core clock in MHz.
// Returns 0, or -1 (bad argument) / -2 (HIP error).
extern "C" int od_probe_mfma(int mode, int iters, double* tops, double* mhz) {
  if (mode < 0 || mode > 4 || iters < 1 || !tops || !mhz) return -1;
  int dev = 0, cus = 0, wall_khz = 0;
  if (hipGetDevice(&dev) != hipSuccess) return -2;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1) return -2;
  if (hipDeviceGetAttribute(&wall_khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess || wall_khz < 1)
    return -2;
  long long* st = nullptr;
  int* sink = nullptr;
  int* seed = nullptr;
  int rc = 0;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  const int hs[4] = {12345, 678910, 111213, 141516};
  std::vector<long long> h(4 * (size_t)cus);
  float ms = 0.0f;
  auto launch = [&]() {
    switch (mode) {
      case 0: mfma_probe_kernel<0><<<cus, kThreads>>>(iters, st, sink, seed); break;
      case 1: mfma_probe_kernel<1><<<cus, kThreads>>>(iters, st, sink, seed); break;
      case 2: mfma_probe_kernel<2><<<cus, kThreads>>>(iters, st, sink, seed); break;
      case 3: mfma_probe_kernel<3><<<cus, kThreads>>>(iters, st, sink, seed); break;
      default: mfma_probe_kernel<4><<<cus, kThreads>>>(iters, st, sink, seed); break;
    }
    return hipGetLastError() == hipSuccess;
  };
  if (hipMalloc(&st, sizeof(long long) * 4 * cus) != hipSuccess ||
      hipMalloc(&sink, sizeof(int) * kThreads * cus) != hipSuccess || hipMalloc(&seed, sizeof(hs)) != hipSuccess ||
      hipMemcpy(seed, hs, sizeof(hs), hipMemcpyHostToDevice) != hipSuccess || hipEventCreate(&e0) != hipSuccess ||
      hipEventCreate(&e1) != hipSuccess || !launch() || hipDeviceSynchronize() != hipSuccess ||
      hipEventRecord(e0, 0) != hipSuccess || !launch() || hipEventRecord(e1, 0) != hipSuccess ||
      hipDeviceSynchronize() != hipSuccess || hipEventElapsedTime(&ms, e0, e1) != hipSuccess ||
      hipMemcpy(h.data(), st, sizeof(long long) * 4 * cus, hipMemcpyDeviceToHost) != hipSuccess) {
    rc = -2;
  }
  if (rc == 0) {
    double clk = 0.0;
    int n = 0;
    for (int b = 0; b < cus; ++b) {
      const double dt = (double)(h[4 * b + 1] - h[4 * b]), dr = (double)(h[4 * b + 3] - h[4 * b + 2]);
      if (dr > 0) {
        clk += dt / dr * (wall_khz / 1000.0);
        ++n;
      }
    }
    const double per = mode <= 2 ? 2.0 * 32 * 32 * 32 : 2.0 * 32 * 32 * 16;  // ops per MFMA
    *tops = per * 8.0 * iters * (kThreads / 64) * (double)cus / (ms * 1e-3) / 1e12;
    *mhz = n ? clk / n : 0.0;
  }
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  if (st) (void)hipFree(st);
  if (sink) (void)hipFree(sink);
  if (seed) (void)hipFree(seed);
  return rc;
}
