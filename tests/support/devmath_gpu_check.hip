// Exhaustive device check of the branch-free activation math used by the
// GEMM epilogues: for every f32 bit pattern x, compares on the GPU
//   tanhf_fast(x) with tanhf_fdlibm(x)   and   gelu_fast(x) with gelu(x).
// The reference forms use IEEE division and equal glibc on all inputs (host
// check); the fast forms divide with rcp + two FMAs.  Prints
// "<name> <checked> <mismatches> <first_bad_hex>" per function; exit 0.
// Third line: the certified GELU bound, for every finite x,
//   |gelu_approx(x) - gelu(x)| <= kGeluApproxRel |x| + kGeluApproxAbs
// (computed in double), as "gelu_approx <checked> <violations>
// <first_bad_hex> <largest |error| / |x| over |x| >= 2^-100, f32 bits>".
// Usage: devmath_gpu_check [stride]   (stride 1 = all 2^32 inputs)
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

#include "../../rustgears_amd/csrc/devmath.h"

__global__ __launch_bounds__(256) void check(unsigned long long n, unsigned long long stride, unsigned long long* bad,
                                             unsigned int* first, unsigned int* worst) {
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
    if (__builtin_isfinite(x)) {
      const float g = rgmath::gelu_approx(x);
      const double err = __builtin_fabs((double)g - (double)d), ax = __builtin_fabs((double)x);
      const bool ok_a = err <= (double)rgmath::kGeluApproxRel * ax + (double)rgmath::kGeluApproxAbs;
      if (!ok_a) { atomicAdd(&bad[2], 1ull); atomicMin(&first[2], (unsigned int)i); }
      if (ax >= 0x1p-100) atomicMax(worst, rgmath::fbits((float)(err / ax)));
      if (ok_a) atomicAdd(&bad[3], 1ull);  // checked (finite) inputs that hold the bound
    }
  }
}

int main(int argc, char** argv) {
  const unsigned long long stride = argc > 1 ? strtoull(argv[1], 0, 0) : 1;
  const unsigned long long n = 1ull << 32;
  const unsigned long long count = (n + stride - 1) / stride;
  unsigned long long* bad;
  unsigned int *first, *worst;
  if (hipMalloc(&bad, 32) != hipSuccess || hipMalloc(&first, 12) != hipSuccess || hipMalloc(&worst, 4) != hipSuccess)
    return 2;
  unsigned long long zero[4] = {0, 0, 0, 0};
  unsigned int ff[3] = {0xffffffffu, 0xffffffffu, 0xffffffffu}, z = 0;
  if (hipMemcpy(bad, zero, 32, hipMemcpyHostToDevice) != hipSuccess) return 2;
  if (hipMemcpy(first, ff, 12, hipMemcpyHostToDevice) != hipSuccess) return 2;
  if (hipMemcpy(worst, &z, 4, hipMemcpyHostToDevice) != hipSuccess) return 2;
  const unsigned long long threads = (count + 63) / 64;
  const unsigned int blocks = (unsigned int)((threads + 255) / 256);
  hipLaunchKernelGGL(check, dim3(blocks), dim3(256), 0, 0, n, stride, bad, first, worst);
  if (hipDeviceSynchronize() != hipSuccess) return 3;
  unsigned long long hb[4];
  unsigned int hf[3], hw;
  if (hipMemcpy(hb, bad, 32, hipMemcpyDeviceToHost) != hipSuccess) return 2;
  if (hipMemcpy(hf, first, 12, hipMemcpyDeviceToHost) != hipSuccess) return 2;
  if (hipMemcpy(&hw, worst, 4, hipMemcpyDeviceToHost) != hipSuccess) return 2;
  printf("tanhf_fast %llu %llu %08x\n", count, hb[0], hf[0]);
  printf("gelu_fast %llu %llu %08x\n", count, hb[1], hf[1]);
  printf("gelu_approx %llu %llu %08x %08x\n", hb[2] + hb[3], hb[2], hf[2], hw);
  return 0;
}
