// K-loop lab for the S layer shape (8192 x 4096 x 4096 i8, 256 x 256 tiles,
// 256 workgroups x 2 tiles x 64 K steps of 64 bytes): times the large GEMM's
// K loop with parts of it taken away, and the overlap of independent VALU
// work with the i8 MFMAs.  Measurement only: every variant computes
// something, folds it into a sink that is written only when it equals an
// impossible value, and performs the S layer's MFMA count (8.39 M
// v_mfma_i32_16x16x64_i8 = 274.9 G ops) -- except the VALU overlap rows,
// which add VALU instructions to the register-only loop.
//
//   mfma             the 32 MFMAs of a wave's K step on register operands
//   mfma+barrier     + the workgroup barrier of every K step
//   mfma+barrier+lds + the step's 12 fragment reads from LDS (ring stages
//                    rotated, no DMA)
//   mfma32*          the three above with v_mfma_i32_32x32x32_i8 (16 MFMAs
//                    per step, the same wave tile and fragment reads)
//   production/4     gemm_core.h big_kloop, the 4-stage DMA ring of the
//                    product's 256 x 256 GEMM, on random A [8192, 4096] and
//                    B [4096, 4096]
//   production/3     the same with a 3-stage ring
//   wide/lds         4 waves of 128 x 128 (one per SIMD, 256 accumulators):
//                    16 fragment reads per step for 64 MFMAs, 2/3 of the
//                    LDS bytes per MAC of the 8-wave tile
//   wide/lds+pf      the same with the next step's fragments prefetched
//   overlap/V        the register-only loop with V independent FMAs per MFMA
//
// Prints "<variant> <us per layer> <TOPS>" lines (median of `reps` launches
// after 3 warm-up launches).  Usage: kloop_lab [reps]
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "../../rustgears_amd/csrc/gemm_core.h"

namespace rgnpu {
hipEvent_t next_launch_event() { return nullptr; }
}  // namespace rgnpu
using namespace rgnpu;
typedef int v16i __attribute__((ext_vector_type(16)));

#define CK(e)                                                                             \
  do {                                                                                    \
    hipError_t r_ = (e);                                                                  \
    if (r_ != hipSuccess) {                                                               \
      std::printf("HIP error %s at line %d\n", hipGetErrorString(r_), __LINE__);         \
      std::exit(1);                                                                       \
    }                                                                                     \
  } while (0)

constexpr int kTiles = 512, kSteps = 64, kBlocks = 256;

// Register-only variants: MODE 0 mfma, 1 + barrier, 2 + LDS fragment reads;
// VALU > 0 adds VALU independent FMAs per MFMA (on 8 separate chains).
template <int MODE, int VALU>
__global__ __launch_bounds__(512, 1) void reg_loop(const int32_t* __restrict__ seed, int32_t never,
                                                   int32_t* __restrict__ sink) {
  __shared__ __attribute__((aligned(1024))) int8_t smem[4 * 32768];
  const int l = threadIdx.x, lane = l & 63, wave = l >> 6;
  for (int i = l; i < 4 * 32768 / 4; i += 512) reinterpret_cast<int32_t*>(smem)[i] = seed[i & 255] ^ (i * 0x9e3779b9);
  __syncthreads();
  v4i a[8], b[4], acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; i++)
    a[i] = v4i{seed[(l + i) & 255], seed[(l + 3 * i + 1) & 255], seed[(l + 5 * i + 2) & 255], seed[(l + 7 * i + 3) & 255]};
#pragma unroll
  for (int j = 0; j < 4; j++)
    b[j] = v4i{seed[(l + 11 * j) & 255], seed[(l + 13 * j + 5) & 255], seed[(l + 17 * j + 6) & 255],
               seed[(l + 19 * j + 7) & 255]};
#pragma unroll
  for (int i = 0; i < 8; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) acc[i][j] = v4i{0, 0, 0, 0};
  float f[8];
#pragma unroll
  for (int c = 0; c < 8; c++) f[c] = (float)(seed[(l + c) & 255] & 7) * 0.125f;
  const float fa = 0.999f, fb = 1e-3f;
  const int wm = wave / 4, wn = wave % 4;
  const uint32_t rd = (uint32_t)((lane & 15) * 64 + (((lane >> 4) ^ lds_swz(lane & 15)) << 4));
  const uint32_t rda = rd + (uint32_t)(wm * 16 * 8 * 64), rdb = rd + (uint32_t)(16384 + wn * 64 * 64);
  uint32_t st = 0;
  for (int it = 0; it < 2 * kSteps; it++) {  // 2 tiles per workgroup
    if constexpr (MODE >= 1) {
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
    }
    if constexpr (MODE == 2) {
      const int8_t* sa = smem + st;
#pragma unroll
      for (int j = 0; j < 4; j++) b[j] = *reinterpret_cast<const v4i*>(sa + rdb + j * 16 * 64);
#pragma unroll
      for (int i = 0; i < 8; i++) a[i] = *reinterpret_cast<const v4i*>(sa + rda + i * 16 * 64);
      st = st == 3 * 32768 ? 0 : st + 32768;
    }
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
      for (int j = 0; j < 4; j++) {
        acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[i], b[j], acc[i][j], 0, 0, 0);
#pragma unroll
        for (int v = 0; v < VALU; v++) f[(4 * i + j + v) & 7] = __builtin_fmaf(f[(4 * i + j + v) & 7], fa, fb);
      }
  }
  int32_t x = 0;
#pragma unroll
  for (int i = 0; i < 8; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) x ^= acc[i][j][0] ^ acc[i][j][1] ^ acc[i][j][2] ^ acc[i][j][3];
#pragma unroll
  for (int c = 0; c < 8; c++) x ^= __float_as_int(f[c]);
  if (x == never) sink[0] = x;
}

// The register-only variants with v_mfma_i32_32x32x32_i8: the same 128 x 64
// wave tile as 4 x 2 blocks of 32 x 32, each K step of 64 bytes as two
// halves, so 16 MFMAs of twice the work per step (the same 274.9 G ops) and,
// with MODE 2, the same 12 fragment reads of 16 bytes per lane (lane l reads
// row l % 32 of its block, K bytes 32 h + 16 (l / 32) of the half h).
template <int MODE>
__global__ __launch_bounds__(512, 1) void reg_loop32(const int32_t* __restrict__ seed, int32_t never,
                                                     int32_t* __restrict__ sink) {
  __shared__ __attribute__((aligned(1024))) int8_t smem[4 * 32768];
  const int l = threadIdx.x, lane = l & 63, wave = l >> 6;
  for (int i = l; i < 4 * 32768 / 4; i += 512) reinterpret_cast<int32_t*>(smem)[i] = seed[i & 255] ^ (i * 0x9e3779b9);
  __syncthreads();
  v4i a[4][2], b[2][2];
  v16i acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int h = 0; h < 2; h++)
      a[i][h] = v4i{seed[(l + 2 * i + h) & 255], seed[(l + 3 * i + 1) & 255], seed[(l + 5 * i + h + 2) & 255],
                    seed[(l + 7 * i + 3) & 255]};
#pragma unroll
  for (int j = 0; j < 2; j++)
#pragma unroll
    for (int h = 0; h < 2; h++)
      b[j][h] = v4i{seed[(l + 11 * j + h) & 255], seed[(l + 13 * j + 5) & 255], seed[(l + 17 * j + h + 6) & 255],
                    seed[(l + 19 * j + 7) & 255]};
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[i][j][e] = 0;
  const int wm = wave / 4, wn = wave % 4;
  const int row = lane & 31;
  uint32_t rdh[2];
#pragma unroll
  for (int h = 0; h < 2; h++)
    rdh[h] = (uint32_t)(row * 64 + (((2 * h + (lane >> 5)) ^ lds_swz(row & 15)) << 4));
  uint32_t st = 0;
  for (int it = 0; it < 2 * kSteps; it++) {  // 2 tiles per workgroup
    if constexpr (MODE >= 1) {
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
    }
    if constexpr (MODE == 2) {
      const int8_t* sa = smem + st;
#pragma unroll
      for (int h = 0; h < 2; h++) {
#pragma unroll
        for (int j = 0; j < 2; j++)
          b[j][h] = *reinterpret_cast<const v4i*>(sa + 16384 + (wn * 64 + j * 32) * 64 + rdh[h]);
#pragma unroll
        for (int i = 0; i < 4; i++) a[i][h] = *reinterpret_cast<const v4i*>(sa + (wm * 128 + i * 32) * 64 + rdh[h]);
      }
      st = st == 3 * 32768 ? 0 : st + 32768;
    }
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i][h], b[j][h], acc[i][j], 0, 0, 0);
  }
  int32_t x = 0;
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) x ^= acc[i][j][e];
  if (x == never) sink[0] = x;
}

// 4 waves (2 x 2), wave tile 128 x 128 (8 x 8 blocks, 256 accumulators),
// one wave per SIMD: 16 fragment reads per K step from LDS (ring stages
// rotated, no DMA) for 64 MFMAs.  PF: the next step's fragments are read
// while this step's MFMAs run (registers double-buffered).
template <bool PF>
__global__ __launch_bounds__(256, 1) void wide_loop(const int32_t* __restrict__ seed, int32_t never,
                                                    int32_t* __restrict__ sink) {
  __shared__ __attribute__((aligned(1024))) int8_t smem[4 * 32768];
  const int l = threadIdx.x, lane = l & 63, wave = l >> 6;
  for (int i = l; i < 4 * 32768 / 4; i += 256) reinterpret_cast<int32_t*>(smem)[i] = seed[i & 255] ^ (i * 0x9e3779b9);
  __syncthreads();
  v4i acc[8][8];
#pragma unroll
  for (int i = 0; i < 8; i++)
#pragma unroll
    for (int j = 0; j < 8; j++) acc[i][j] = v4i{0, 0, 0, 0};
  const int wm = wave / 2, wn = wave % 2;
  const uint32_t rd = (uint32_t)((lane & 15) * 64 + (((lane >> 4) ^ lds_swz(lane & 15)) << 4));
  const uint32_t rda = rd + (uint32_t)(wm * 128 * 64), rdb = rd + (uint32_t)(16384 + wn * 128 * 64);
  auto read = [&](uint32_t st, v4i (&a_)[8], v4i (&b_)[8]) {
    const int8_t* sa = smem + st;
#pragma unroll
    for (int j = 0; j < 8; j++) b_[j] = *reinterpret_cast<const v4i*>(sa + rdb + j * 16 * 64);
#pragma unroll
    for (int i = 0; i < 8; i++) a_[i] = *reinterpret_cast<const v4i*>(sa + rda + i * 16 * 64);
  };
  auto mf = [&](const v4i (&a_)[8], const v4i (&b_)[8]) {
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
      for (int j = 0; j < 8; j++) acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a_[i], b_[j], acc[i][j], 0, 0, 0);
  };
  uint32_t st = 0;
  auto nst = [](uint32_t s) { return s == 3 * 32768 ? 0u : s + 32768; };
  if constexpr (!PF) {
    v4i af[8], bf[8];
    for (int it = 0; it < 2 * kSteps; it++) {
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      read(st, af, bf);
      st = nst(st);
      mf(af, bf);
    }
  } else {
    v4i af[8], bf[8], na[8], nb[8];
    read(st, af, bf);
    st = nst(st);
    for (int it = 0; it < 2 * kSteps; it += 2) {
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      read(st, na, nb);
      st = nst(st);
      mf(af, bf);
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      read(st, af, bf);
      st = nst(st);
      mf(na, nb);
    }
  }
  int32_t x = 0;
#pragma unroll
  for (int i = 0; i < 8; i++)
#pragma unroll
    for (int j = 0; j < 8; j++) x ^= acc[i][j][0] ^ acc[i][j][1] ^ acc[i][j][2] ^ acc[i][j][3];
  if (x == never) sink[0] = x;
}

// The product's K loop over two tiles per workgroup, tile order as the GEMM.
template <int STAGES>
__global__ __launch_bounds__(512, 1) void ring_loop(const int8_t* __restrict__ A, const int8_t* __restrict__ B,
                                                    int32_t never, int32_t* __restrict__ sink) {
  __shared__ __attribute__((aligned(1024))) int8_t smem[STAGES * 32768 + 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / 4, wn = wave % 4;
  v4i acc[8][4];
  int32_t x = 0;
  for (int t = blockIdx.x; t < kTiles; t += gridDim.x) {
    int tm, tn;
    tile_coords(t, 32, 16, tm, tn);
    big_kloop<256, 256, 2, 4, STAGES, 8, kModeI8>(smem, A, B, 4096, (int64_t)tm * 256, (int64_t)tn * 256, 0, kSteps,
                                                  wave, wm, wn, lane, acc);
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
      for (int j = 0; j < 4; j++) x ^= acc[i][j][0] ^ acc[i][j][1] ^ acc[i][j][2] ^ acc[i][j][3];
  }
  if (x == never) sink[0] = x;
}

template <typename F>
static float median_ms(F launch, int reps) {
  hipEvent_t e0, e1;
  CK(hipEventCreate(&e0));
  CK(hipEventCreate(&e1));
  for (int i = 0; i < 3; i++) launch();
  CK(hipDeviceSynchronize());
  std::vector<float> t;
  for (int r = 0; r < reps; r++) {
    CK(hipEventRecord(e0));
    launch();
    CK(hipEventRecord(e1));
    CK(hipEventSynchronize(e1));
    float ms = 0;
    CK(hipEventElapsedTime(&ms, e0, e1));
    t.push_back(ms);
  }
  CK(hipEventDestroy(e0));
  CK(hipEventDestroy(e1));
  std::sort(t.begin(), t.end());
  return t[t.size() / 2];
}

int main(int argc, char** argv) {
  const int reps = argc > 1 ? std::atoi(argv[1]) : 20;
  const double ops = 2.0 * 8192.0 * 4096.0 * 4096.0;  // one S layer
  // random operand bytes (SplitMix64)
  const size_t abytes = (size_t)8192 * 4096, bbytes = (size_t)4096 * 4096;
  std::vector<int8_t> h(abytes + bbytes);
  uint64_t s = 0x5bd1e995ull;
  for (size_t i = 0; i < h.size(); i += 8) {
    uint64_t z = (s += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    z ^= z >> 31;
    for (int k = 0; k < 8 && i + k < h.size(); k++) h[i + k] = (int8_t)(z >> (8 * k));
  }
  int8_t *A = nullptr, *B = nullptr;
  int32_t *seed = nullptr, *sink = nullptr;
  CK(hipMalloc(&A, abytes));
  CK(hipMalloc(&B, bbytes));
  CK(hipMalloc(&seed, 256 * 4));
  CK(hipMalloc(&sink, 64));
  CK(hipMemcpy(A, h.data(), abytes, hipMemcpyHostToDevice));
  CK(hipMemcpy(B, h.data() + abytes, bbytes, hipMemcpyHostToDevice));
  CK(hipMemcpy(seed, h.data(), 256 * 4, hipMemcpyHostToDevice));
  const int32_t never = 0x7fedcba9;
  auto report = [&](const char* name, float ms) {
    std::printf("%-18s %8.1f %8.1f\n", name, ms * 1e3, ops / (ms * 1e-3) / 1e12);
    std::fflush(stdout);
  };
  report("mfma", median_ms([&] { hipLaunchKernelGGL((reg_loop<0, 0>), dim3(kBlocks), dim3(512), 0, 0, seed, never, sink); }, reps));
  report("mfma+barrier", median_ms([&] { hipLaunchKernelGGL((reg_loop<1, 0>), dim3(kBlocks), dim3(512), 0, 0, seed, never, sink); }, reps));
  report("mfma+barrier+lds", median_ms([&] { hipLaunchKernelGGL((reg_loop<2, 0>), dim3(kBlocks), dim3(512), 0, 0, seed, never, sink); }, reps));
  report("mfma32", median_ms([&] { hipLaunchKernelGGL((reg_loop32<0>), dim3(kBlocks), dim3(512), 0, 0, seed, never, sink); }, reps));
  report("mfma32+barrier", median_ms([&] { hipLaunchKernelGGL((reg_loop32<1>), dim3(kBlocks), dim3(512), 0, 0, seed, never, sink); }, reps));
  report("mfma32+barrier+lds", median_ms([&] { hipLaunchKernelGGL((reg_loop32<2>), dim3(kBlocks), dim3(512), 0, 0, seed, never, sink); }, reps));
  report("production/4", median_ms([&] { hipLaunchKernelGGL((ring_loop<4>), dim3(kBlocks), dim3(512), 0, 0, A, B, never, sink); }, reps));
  report("production/3", median_ms([&] { hipLaunchKernelGGL((ring_loop<3>), dim3(kBlocks), dim3(512), 0, 0, A, B, never, sink); }, reps));
  report("wide/lds", median_ms([&] { hipLaunchKernelGGL((wide_loop<false>), dim3(kBlocks), dim3(256), 0, 0, seed, never, sink); }, reps));
  report("wide/lds+pf", median_ms([&] { hipLaunchKernelGGL((wide_loop<true>), dim3(kBlocks), dim3(256), 0, 0, seed, never, sink); }, reps));
  report("overlap/1", median_ms([&] { hipLaunchKernelGGL((reg_loop<0, 1>), dim3(kBlocks), dim3(512), 0, 0, seed, never, sink); }, reps));
  report("overlap/2", median_ms([&] { hipLaunchKernelGGL((reg_loop<0, 2>), dim3(kBlocks), dim3(512), 0, 0, seed, never, sink); }, reps));
  report("overlap/3", median_ms([&] { hipLaunchKernelGGL((reg_loop<0, 3>), dim3(kBlocks), dim3(512), 0, 0, seed, never, sink); }, reps));
  report("overlap/4", median_ms([&] { hipLaunchKernelGGL((reg_loop<0, 4>), dim3(kBlocks), dim3(512), 0, 0, seed, never, sink); }, reps));
  report("overlap/6", median_ms([&] { hipLaunchKernelGGL((reg_loop<0, 6>), dim3(kBlocks), dim3(512), 0, 0, seed, never, sink); }, reps));
  report("overlap/8", median_ms([&] { hipLaunchKernelGGL((reg_loop<0, 8>), dim3(kBlocks), dim3(512), 0, 0, seed, never, sink); }, reps));
  CK(hipGetLastError());
  CK(hipFree(A));
  CK(hipFree(B));
  CK(hipFree(seed));
  CK(hipFree(sink));
  return 0;
}
