// Input-quantization lab for the S input (8192 x 4096 f32 = 134 MB): what the
// one-pass form (read everything, one scale, quantize) can reach on this
// GPU.  Measurement only; nothing here is checked against the quantize rule
// (the product's kernel is input_quant_kernel in requant.hip, and these
// variants use a per-workgroup scale and round-to-nearest).
//
//   read/stream     a grid-strided read of the input, 8 16-byte loads in
//                   flight per thread, 1024 x 256 threads: the read ceiling
//   read/hold16     each 512-thread workgroup loads 16 units per thread
//                   before it uses any (1024 workgroups, not all resident)
//   onepass/8w      the one-pass shape of the product's kernel for S: one
//                   512-thread workgroup per CU keeps 64 units per thread
//                   (19 in LDS, 45 in registers; 49 loads in flight, then
//                   15), takes its absmax, then quantizes and stores what it
//                   holds (no grid barrier)
//   onepass/16w     the same with 1024 threads keeping 32 units each
//                   (9 in LDS, 23 in registers)
//   twopass         an absmax pass (read/stream) and a quantize pass that
//                   reads the input again and writes the i8 operand
//   copy            a grid-strided f32 copy of the input (read + write)
//
// The input rotates over three buffers (402 MB, more than the memory-side
// cache), as in a program whose layers displace its input.  Prints
// "<variant> <us> <TB/s of input + operand bytes>" lines (the median of
// `reps` batches of 20 launches, after 5 warm-up launches).
// Usage: input_quant_lab [reps]
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <vector>

typedef float v4f __attribute__((ext_vector_type(4)));

#define CHECK(x)                                                                              \
  do {                                                                                        \
    hipError_t e_ = (x);                                                                      \
    if (e_ != hipSuccess) {                                                                   \
      std::fprintf(stderr, "%s failed: %s (line %d)\n", #x, hipGetErrorString(e_), __LINE__); \
      std::exit(1);                                                                           \
    }                                                                                         \
  } while (0)

namespace {

constexpr uint32_t kDrop = 0x80000000u;  // a buffer offset past every record: the load returns 0

__device__ __forceinline__ float amax4(float m, v4f v) {
  m = __builtin_fmaxf(m, __builtin_fabsf(v[0]));
  m = __builtin_fmaxf(m, __builtin_fabsf(v[1]));
  m = __builtin_fmaxf(m, __builtin_fabsf(v[2]));
  return __builtin_fmaxf(m, __builtin_fabsf(v[3]));
}

__device__ __forceinline__ uint32_t q4(v4f v, float inv) {
  uint32_t r = 0;
#pragma unroll
  for (int e = 0; e < 4; e++) r |= ((uint32_t)(int)__builtin_rintf(v[e] * inv) & 255u) << (8 * e);
  return r;
}

__device__ __forceinline__ v4f load_unit(__amdgpu_buffer_rsrc_t r, uint32_t w, uint32_t W) {
  return __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(r, (int)(w < W ? w * 16u : kDrop), 0, 2));
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ float block_max(float m, float* red, int nw) {
  for (int o = 32; o; o >>= 1) m = __builtin_fmaxf(m, __shfl_xor(m, o));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  float t = red[0];
  for (int w = 1; w < nw; w++) t = __builtin_fmaxf(t, red[w]);
  return t;
}

// grid-strided absmax, D loads in flight per thread; the maximum goes to
// amax[0] through an atomic
template <int D>
__global__ __launch_bounds__(256) void stream_absmax(const float* x, uint32_t W, uint32_t* amax) {
  __shared__ float red[4];
  const __amdgpu_buffer_rsrc_t r = rsrc(x, W * 16u);
  const uint32_t NT = gridDim.x * 256u;
  float m = 0.f;
  for (uint32_t w = blockIdx.x * 256u * D + threadIdx.x; w < W; w += NT * D) {
    v4f v[D];
#pragma unroll
    for (int j = 0; j < D; j++) v[j] = load_unit(r, w + j * 256u, W);
#pragma unroll
    for (int j = 0; j < D; j++) m = amax4(m, v[j]);
  }
  const float t = block_max(m, red, 4);
  if (threadIdx.x == 0) atomicMax(amax, __float_as_uint(t));
}

// grid-strided quantize with the scale from amax[0]
template <int D>
__global__ __launch_bounds__(256) void stream_quant(const float* x, uint32_t W, const uint32_t* amax, uint32_t* q) {
  const __amdgpu_buffer_rsrc_t r = rsrc(x, W * 16u), rq = rsrc(q, W * 4u);
  const float a = __uint_as_float(*amax);
  const float inv = 127.0f / (a > 0.f ? a : 1.f);
  const uint32_t NT = gridDim.x * 256u;
  for (uint32_t w = blockIdx.x * 256u * D + threadIdx.x; w < W; w += NT * D) {
    v4f v[D];
#pragma unroll
    for (int j = 0; j < D; j++) v[j] = load_unit(r, w + j * 256u, W);
#pragma unroll
    for (int j = 0; j < D; j++) __builtin_amdgcn_raw_buffer_store_b32(q4(v[j], inv), rq, (int)((w + j * 256u) * 4u), 0, 0);
  }
}

__global__ __launch_bounds__(256) void stream_copy(const v4f* x, v4f* y, uint32_t W) {
  for (uint32_t w = blockIdx.x * 256u + threadIdx.x; w < W; w += gridDim.x * 256u) y[w] = x[w];
}

// workgroup b, thread t loads units b U T + j T + t (j < U) before it uses any
template <int U, int T>
__global__ __launch_bounds__(T) void hold_absmax(const float* x, uint32_t W, uint32_t* amax) {
  __shared__ float red[T / 64];
  const __amdgpu_buffer_rsrc_t r = rsrc(x, W * 16u);
  const uint32_t w0 = blockIdx.x * U * T + threadIdx.x;
  v4f v[U];
#pragma unroll
  for (int j = 0; j < U; j++) v[j] = load_unit(r, w0 + j * T, W);
  float m = 0.f;
#pragma unroll
  for (int j = 0; j < U; j++) m = amax4(m, v[j]);
  const float t = block_max(m, red, T / 64);
  if (threadIdx.x == 0) atomicMax(amax, __float_as_uint(t));
}

// the one-pass shape: KL units per thread in LDS, KR in registers (KF of
// them loaded with the LDS units), then the quantized units stored
template <int T, int KL, int KR, int KF>
__global__ __launch_bounds__(T) void onepass(const float* x, uint32_t W, uint32_t* q) {
  __shared__ v4f lds[KL * T];
  __shared__ float red[T / 64];
  const __amdgpu_buffer_rsrc_t r = rsrc(x, W * 16u), rq = rsrc(q, W * 4u);
  const int tid = threadIdx.x;
  const uint32_t w0 = blockIdx.x * (KL + KR) * T + tid;
  v4f keep[KR], part[KL];
  float m = 0.f;
#pragma unroll
  for (int j = 0; j < KL; j++) part[j] = load_unit(r, w0 + j * T, W);
#pragma unroll
  for (int j = 0; j < KF; j++) keep[j] = load_unit(r, w0 + (KL + j) * T, W);
#pragma unroll
  for (int j = 0; j < KL; j++) {
    m = amax4(m, part[j]);
    lds[tid * KL + j] = part[j];
  }
#pragma unroll
  for (int j = KF; j < KR; j++) keep[j] = load_unit(r, w0 + (KL + j) * T, W);
#pragma unroll
  for (int j = 0; j < KR; j++) m = amax4(m, keep[j]);
  const float t = block_max(m, red, T / 64);
  const float inv = 127.0f / (t > 0.f ? t : 1.f);
#pragma unroll
  for (int j = 0; j < KL; j++)
    __builtin_amdgcn_raw_buffer_store_b32(q4(lds[tid * KL + j], inv), rq, (int)((w0 + j * T) * 4u), 0, 0);
#pragma unroll
  for (int j = 0; j < KR; j++)
    __builtin_amdgcn_raw_buffer_store_b32(q4(keep[j], inv), rq, (int)((w0 + (KL + j) * T) * 4u), 0, 0);
}

}  // namespace

int main(int argc, char** argv) {
  const int reps = argc > 1 ? std::atoi(argv[1]) : 10;
  const uint32_t M = 8192, K = 4096, W = M * K / 4;  // 16-byte units
  const size_t in_bytes = (size_t)W * 16, q_bytes = (size_t)W * 4;
  constexpr int NB = 3;
  float* x[NB];
  std::vector<float> host(in_bytes / 4);
  uint64_t s = 0x9E3779B97F4A7C15ull;
  for (auto& f : host) {
    s = s * 6364136223846793005ull + 1442695040888963407ull;
    f = (float)((int64_t)(s >> 40) - (1 << 23)) * (1.0f / (1 << 20));
  }
  for (int i = 0; i < NB; i++) {
    CHECK(hipMalloc(&x[i], in_bytes));
    CHECK(hipMemcpy(x[i], host.data(), in_bytes, hipMemcpyHostToDevice));
  }
  uint32_t *q, *amax;
  v4f* y;
  CHECK(hipMalloc(&q, q_bytes));
  CHECK(hipMalloc(&y, in_bytes));
  CHECK(hipMalloc(&amax, 256));
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));

  auto run = [&](const char* name, size_t bytes, auto launch) {
    int it = 0;
    for (int i = 0; i < 5; i++) launch(x[it++ % NB]);
    CHECK(hipDeviceSynchronize());
    std::vector<double> us;
    for (int rep = 0; rep < reps; rep++) {
      CHECK(hipEventRecord(e0));
      for (int i = 0; i < 20; i++) launch(x[it++ % NB]);
      CHECK(hipEventRecord(e1));
      CHECK(hipEventSynchronize(e1));
      float ms;
      CHECK(hipEventElapsedTime(&ms, e0, e1));
      us.push_back(ms * 1000.0 / 20);
    }
    std::sort(us.begin(), us.end());
    const double med = us[us.size() / 2];
    std::printf("%s %.2f %.2f\n", name, med, bytes / med / 1e6);
    std::fflush(stdout);
  };
  run("read/stream", in_bytes, [&](float* p) { stream_absmax<8><<<1024, 256>>>(p, W, amax); });
  run("read/hold16", in_bytes, [&](float* p) { hold_absmax<16, 512><<<W / (16 * 512), 512>>>(p, W, amax); });
  static_assert(19 + 45 == 64 && 9 + 23 == 32, "units per thread");
  run("onepass/8w", in_bytes + q_bytes, [&](float* p) { onepass<512, 19, 45, 30><<<W / (64 * 512), 512>>>(p, W, q); });
  run("onepass/16w", in_bytes + q_bytes, [&](float* p) { onepass<1024, 9, 23, 23><<<W / (32 * 1024), 1024>>>(p, W, q); });
  run("twopass", 2 * in_bytes + q_bytes, [&](float* p) {
    stream_absmax<8><<<1024, 256>>>(p, W, amax);
    stream_quant<8><<<1024, 256>>>(p, W, amax, q);
  });
  run("copy", 2 * in_bytes, [&](float* p) { stream_copy<<<2048, 256>>>(reinterpret_cast<const v4f*>(p), y, W); });
  CHECK(hipGetLastError());
  CHECK(hipDeviceSynchronize());
  return 0;
}
