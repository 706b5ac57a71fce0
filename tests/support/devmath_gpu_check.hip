// Exhaustive device check of the branch-free activation math used by the
// GEMM epilogues: for every f32 bit pattern x, compares on the GPU
//   tanhf_fast(x) with tanhf_fdlibm(x)   and   gelu_fast(x) with gelu(x).
// The reference forms use IEEE division and equal glibc on all inputs (host
// check); the fast forms divide with rcp + two FMAs.  Prints
// "<name> <checked> <mismatches> <first_bad_hex>" per function; exit 0.
// Usage: devmath_gpu_check [stride]   (stride 1 = all 2^32 inputs)
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

#include "../../rustgears_amd/csrc/devmath.h"

__global__ __launch_bounds__(256) void check(unsigned long long n, unsigned long long stride, unsigned long long* bad,
                                             unsigned int* first) {
  const unsigned long long per = 64;
  const unsigned long long base = ((unsigned long long)blockIdx.x * blockDim.x + threadIdx.x) * per;
  for (unsigned long long j = 0; j < per; j++) {
    const unsigned long long i = (base + j) * stride;
    if (i >= n) break;
    const float x = rgmath::bitsf((unsigned int)i);
    const float a = rgmath::tanhf_fast(x), b = rgmath::tanhf_fdlibm(x);
    const float c = rgmath::gelu_fast(x), d = rgmath::gelu(x);
    const bool ok_t = rgmath::fbits(a) == rgmath::fbits(b) || (a != a && b != b);
    const bool ok_g = rgmath::fbits(c) == rgmath::fbits(d) || (c != c && d != d);
    if (!ok_t) { atomicAdd(&bad[0], 1ull); atomicMin(&first[0], (unsigned int)i); }
    if (!ok_g) { atomicAdd(&bad[1], 1ull); atomicMin(&first[1], (unsigned int)i); }
  }
}

int main(int argc, char** argv) {
  const unsigned long long stride = argc > 1 ? strtoull(argv[1], 0, 0) : 1;
  const unsigned long long n = 1ull << 32;
  const unsigned long long count = (n + stride - 1) / stride;
  unsigned long long* bad;
  unsigned int* first;
  if (hipMalloc(&bad, 16) != hipSuccess || hipMalloc(&first, 8) != hipSuccess) return 2;
  unsigned long long zero[2] = {0, 0};
  unsigned int ff[2] = {0xffffffffu, 0xffffffffu};
  if (hipMemcpy(bad, zero, 16, hipMemcpyHostToDevice) != hipSuccess) return 2;
  if (hipMemcpy(first, ff, 8, hipMemcpyHostToDevice) != hipSuccess) return 2;
  const unsigned long long threads = (count + 63) / 64;
  const unsigned int blocks = (unsigned int)((threads + 255) / 256);
  hipLaunchKernelGGL(check, dim3(blocks), dim3(256), 0, 0, n, stride, bad, first);
  if (hipDeviceSynchronize() != hipSuccess) return 3;
  unsigned long long hb[2];
  unsigned int hf[2];
  if (hipMemcpy(hb, bad, 16, hipMemcpyDeviceToHost) != hipSuccess) return 2;
  if (hipMemcpy(hf, first, 8, hipMemcpyDeviceToHost) != hipSuccess) return 2;
  printf("tanhf_fast %llu %llu %08x\n", count, hb[0], hf[0]);
  printf("gelu_fast %llu %llu %08x\n", count, hb[1], hf[1]);
  return 0;
}
