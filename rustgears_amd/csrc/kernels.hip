// kernels.hip — gfx950 kernels of the MI355X INT8 execution provider.
//
// Hot path (one Linear layer of InferenceSession::run, npu.rs:307-318):
//   absmax (grid reduction) -> quantize rows (round half away, clamp ±127)
//   -> i8 x i8 -> i32 MFMA GEMM with the fused dequant/bias/activation
//   epilogue, which also reduces the absmax of its f32 output for the next
//   layer's quantization.
// Conv2d (npu.rs:319-383) runs as an implicit GEMM whose im2col gather is
// done while filling the LDS tile; MaxPool2d (kernels.rs:165-213) is a
// bandwidth kernel that can emit per-image absmax for the following conv.
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <stdexcept>

#include "devmath.h"
#include "gemm_core.h"
#include "rgnpu_internal.h"

namespace rgnpu {

// Launch-event sink (see set_launch_events): every kernel launched while it
// is set carries the next event as the stop event of its own dispatch.
static thread_local hipEvent_t* t_sink = nullptr;
static thread_local int t_sink_cap = 0, t_sink_used = 0;

void set_launch_events(hipEvent_t* events, int cap) {
  t_sink = events;
  t_sink_cap = cap;
  t_sink_used = 0;
}

int launch_events_used() { return t_sink_used; }

hipEvent_t next_launch_event() {
  if (t_sink && t_sink_used < t_sink_cap) return t_sink[t_sink_used++];
  return nullptr;
}

// ---------------------------------------------------------------------------
// fill
// ---------------------------------------------------------------------------
__global__ void fill_u32_kernel(uint32_t* p, int64_t n, uint32_t v) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

void launch_fill_u32(uint32_t* p, int64_t n, uint32_t v, hipStream_t s) {
  if (n <= 0) return;
  int64_t blocks = (n + 255) / 256;
  RG_LAUNCH(fill_u32_kernel, dim3((unsigned)blocks), dim3(256), 0, s, p, n, v);
}

// The runtime loads a code object on a device at the first launch of one of
// its kernels.  Launching this empty kernel when a program is created moves
// that one-time load (milliseconds) out of the first run and its profile.
__global__ void load_probe_kernel() {}

void load_code_object(hipStream_t s) {
  hipLaunchKernelGGL(load_probe_kernel, dim3(1), dim3(64), 0, s);
  load_requant_code_object(s);
}

// Reads n 16-byte words so that the memory-side cache (256 MB on MI355X)
// holds them instead of whatever a run left there.  The xor of everything
// read lands in sink[0] only if it equals `never`, which the caller picks
// so that the reads cannot be dropped (the buffer is zero, `never` is not).
__global__ __launch_bounds__(256) void evict_kernel(const v4i* __restrict__ p, int64_t n, uint32_t never,
                                                    uint32_t* __restrict__ sink) {
  uint32_t x = 0;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const v4i v = p[i];  // plain loads: they allocate in the memory-side cache
    x ^= (uint32_t)(v[0] ^ v[1] ^ v[2] ^ v[3]);
  }
  if (x == never) sink[0] = x;
}

// Sustained MFMA rate: the shape of the large GEMM's inner loop without its
// memory traffic.  Every wave (8 per CU, 2 per SIMD) holds 8 A and 4 B
// operand fragments in registers and runs `iters` rounds of 32 independent
// v_mfma_i32_16x16x64_i8 (accumulators acc[i][j] += a[i] * b[j], 128
// accumulator registers), with no LDS, barrier or memory access in the loop.
// The fragments are built from the 256 words at `seed` (random or zero
// bytes, chosen by the caller).  The accumulators are folded into sink[0]
// only if they equal `never`, so the work cannot be dropped.
__global__ __launch_bounds__(512) void mfma_peak_kernel(const int32_t* __restrict__ seed, int64_t iters,
                                                        int32_t never, int32_t* __restrict__ sink) {
  const int l = threadIdx.x;
  v4i a[8], b[4], acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; i++)
    a[i] = v4i{seed[(l + i) & 255], seed[(l + 3 * i + 1) & 255], seed[(l + 5 * i + 2) & 255],
               seed[(l + 7 * i + 3) & 255]};
#pragma unroll
  for (int j = 0; j < 4; j++)
    b[j] = v4i{seed[(l + 11 * j) & 255], seed[(l + 13 * j + 5) & 255], seed[(l + 17 * j + 6) & 255],
               seed[(l + 19 * j + 7) & 255]};
#pragma unroll
  for (int i = 0; i < 8; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) acc[i][j] = v4i{0, 0, 0, 0};
  for (int64_t it = 0; it < iters; it++) {
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
      for (int j = 0; j < 4; j++) acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[i], b[j], acc[i][j], 0, 0, 0);
  }
  int32_t x = 0;
#pragma unroll
  for (int i = 0; i < 8; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) x ^= acc[i][j][0] ^ acc[i][j][1] ^ acc[i][j][2] ^ acc[i][j][3];
  if (x == never) sink[0] = x;
}

double probe_mfma_rate(const void* ops, int64_t iters, int32_t* sink, int64_t* macs_out, hipStream_t s) {
  int dev = 0, cus = 256;
  (void)hipGetDevice(&dev);
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
  const int64_t blocks = cus;  // one 8-wave workgroup per CU, as the large GEMM
  hipEvent_t e0, e1;
  if (hipEventCreate(&e0) != hipSuccess) return -1.0;
  if (hipEventCreate(&e1) != hipSuccess) {
    (void)hipEventDestroy(e0);
    return -1.0;
  }
  (void)hipEventRecord(e0, s);
  hipLaunchKernelGGL(mfma_peak_kernel, dim3((unsigned)blocks), dim3(512), 0, s, reinterpret_cast<const int32_t*>(ops),
                     iters, (int32_t)0x5bd1e995, sink);
  (void)hipEventRecord(e1, s);
  float ms = -1.0f;
  if (hipGetLastError() == hipSuccess && hipEventSynchronize(e1) == hipSuccess) (void)hipEventElapsedTime(&ms, e0, e1);
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  *macs_out = blocks * 8 * iters * 32 * (int64_t)(16 * 16 * 64);
  return ms;
}

void launch_evict(const void* p, int64_t bytes, uint32_t* sink, hipStream_t s) {
  const int64_t n = bytes / 16;
  if (n <= 0) return;
  RG_LAUNCH(evict_kernel, dim3(4096), dim3(256), 0, s, reinterpret_cast<const v4i*>(p), n, 0x9e3779b9u, sink);
}

// ---------------------------------------------------------------------------
// absmax: QuantTensor::from_f32's `fold(0, max(|v|))` (quantize.rs:19) as a
// grid reduction.  Non-negative f32 order equals u32 bit order, so a u32
// atomicMax of |v| bits is exact; NaN keys are dropped like f32::max does.
// The unmasked form streams 16-byte loads; the masked form (conv inputs whose
// rows/columns are not all read by a window) tests each element's position.
// ---------------------------------------------------------------------------

// One atomic per block: into `slot` itself, or (spread) into the block's
// partial of a spread slot.
__device__ __forceinline__ void block_max_atomic(uint32_t m, uint32_t* slot, bool spread) {
  m = wave_max_u32(m);
  __shared__ uint32_t red[4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) red[wave] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t r = red[0];
    for (int i = 1; i < (int)(blockDim.x >> 6); i++) r = red[i] > r ? red[i] : r;
    if (r) atomicMax(spread ? slot + (blockIdx.x & (kSpread - 1)) * kSpreadStride : slot, r);
  }
}

__global__ __launch_bounds__(256) void absmax_kernel(const float* __restrict__ x, int64_t per_img,
                                                     uint32_t* __restrict__ slots, int spread, SlotClear clear) {
  clear_slots(clear);
  const int64_t img = blockIdx.y;
  const float* xi = x + img * per_img;
  uint32_t m = 0;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  // Aligned images: each thread reads contiguous 64-byte chunks (a wave
  // covers 4 KiB), two chunks per iteration; then the tail.  The running
  // max is kept as f32 (NaN ignored, like f32::max) and its bits are the key.
  const bool al = (reinterpret_cast<uintptr_t>(xi) & 15) == 0;
  const int64_t n16 = al ? per_img / 16 : 0;
  const float4* x4 = reinterpret_cast<const float4*>(xi);
  float fm = 0.0f;
  auto take4 = [&](float4 v) {
    fm = __builtin_fmaxf(fm, __builtin_fabsf(v.x));
    fm = __builtin_fmaxf(fm, __builtin_fabsf(v.y));
    fm = __builtin_fmaxf(fm, __builtin_fabsf(v.z));
    fm = __builtin_fmaxf(fm, __builtin_fabsf(v.w));
  };
  int64_t c = tid;
  for (; c + stride < n16; c += 2 * stride) {
    const float4* p = x4 + c * 4;
    const float4* q = x4 + (c + stride) * 4;
    const float4 a0 = p[0], a1 = p[1], a2 = p[2], a3 = p[3];
    const float4 b0 = q[0], b1 = q[1], b2 = q[2], b3 = q[3];
    take4(a0); take4(a1); take4(a2); take4(a3);
    take4(b0); take4(b1); take4(b2); take4(b3);
  }
  if (c < n16) {
    const float4* p = x4 + c * 4;
    take4(p[0]); take4(p[1]); take4(p[2]); take4(p[3]);
  }
  for (int64_t e = n16 * 16 + tid; e < per_img; e += stride) fm = __builtin_fmaxf(fm, __builtin_fabsf(xi[e]));
  m = rgmath::fbits(fm);
  block_max_atomic(m, spread ? slots : &slots[img], spread != 0);
}

__global__ __launch_bounds__(256) void absmax_masked_kernel(const float* __restrict__ x, int64_t per_img,
                                                            uint32_t* __restrict__ slots,
                                                            const uint8_t* __restrict__ rowmask,
                                                            const uint8_t* __restrict__ colmask, int H, int W,
                                                            SlotClear clear) {
  clear_slots(clear);
  const int64_t img = blockIdx.y;
  const float* xi = x + img * per_img;
  uint32_t m = 0;
  const uint32_t hw = (uint32_t)(H * W);
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < per_img; e += (int64_t)gridDim.x * blockDim.x) {
    const uint32_t p = (uint32_t)(e % hw);
    const uint32_t iy = p / (uint32_t)W, ix = p % (uint32_t)W;
    if (rowmask[iy] && colmask[ix]) {
      const uint32_t k = rgmath::absmax_key(xi[e]);
      m = k > m ? k : m;
    }
  }
  block_max_atomic(m, &slots[img], false);
}

void launch_absmax(const float* x, int64_t per_img, int64_t n_img, uint32_t* slots, bool spread,
                   const uint8_t* rowmask, const uint8_t* colmask, int64_t H, int64_t W, hipStream_t s,
                   SlotClear clear) {
  if (per_img <= 0 || n_img <= 0) return;
  if (spread && (n_img != 1 || rowmask)) throw std::logic_error("spread absmax takes one unmasked tensor");
  int64_t bx = (per_img + 256 * 32 - 1) / (256 * 32);
  const int64_t cap = n_img >= 64 ? 8 : 4096;
  if (bx > cap) bx = cap;
  if (bx < 1) bx = 1;
  if (rowmask)
    RG_LAUNCH(absmax_masked_kernel, dim3((unsigned)bx, (unsigned)n_img), dim3(256), 0, s, x, per_img, slots,
                       rowmask, colmask, (int)H, (int)W, clear);
  else
    RG_LAUNCH(absmax_kernel, dim3((unsigned)bx, (unsigned)n_img), dim3(256), 0, s, x, per_img, slots,
                       spread ? 1 : 0, clear);
}

// ---------------------------------------------------------------------------
// quantize rows: x f32 [M,K] -> q i8 [Mpad,Kpad].  One thread per 16 output
// bytes (one 16-byte store); padding rows and columns are written as zeros.
// Rows whose K is a multiple of 4 are read with 16-byte loads.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t pack4(float a, float b, float c, float d, float inv) {
  return (uint32_t)(uint8_t)rgmath::quantize_one(a, inv) | ((uint32_t)(uint8_t)rgmath::quantize_one(b, inv) << 8) |
         ((uint32_t)(uint8_t)rgmath::quantize_one(c, inv) << 16) |
         ((uint32_t)(uint8_t)rgmath::quantize_one(d, inv) << 24);
}

template <bool VEC>
__global__ __launch_bounds__(256) void quant_rows_kernel(const float* __restrict__ x, int64_t M, int64_t K,
                                                         int64_t Mpad, int64_t Kpad, const uint32_t* __restrict__ slot,
                                                         int8_t* __restrict__ q, float* scale_out) {
  const float scale = tensor_scale(slot);
  const float inv = 1.0f / scale;
  const uint32_t chunks = (uint32_t)(Kpad / 16);
  const int64_t total = Mpad * (int64_t)chunks;
  for (int64_t w = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; w < total; w += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = w / chunks;
    const uint32_t c0 = (uint32_t)(w - r * chunks) * 16u;
    v4i out = v4i{0, 0, 0, 0};
    if (r < M) {
      const float* xr = x + r * K;
      if (VEC && c0 + 16 <= (uint32_t)K) {
        const float4* p = reinterpret_cast<const float4*>(xr + c0);
        const float4 a = p[0], b = p[1], c = p[2], d = p[3];
        out[0] = (int)pack4(a.x, a.y, a.z, a.w, inv);
        out[1] = (int)pack4(b.x, b.y, b.z, b.w, inv);
        out[2] = (int)pack4(c.x, c.y, c.z, c.w, inv);
        out[3] = (int)pack4(d.x, d.y, d.z, d.w, inv);
      } else {
#pragma unroll
        for (int g = 0; g < 4; g++) {
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const uint32_t c = c0 + (uint32_t)(g * 4 + e);
            v[e] = c < (uint32_t)K ? xr[c] : 0.0f;
          }
          out[g] = (int)pack4(v[0], v[1], v[2], v[3], inv);
        }
      }
    }
    reinterpret_cast<v4i*>(q)[w] = out;
  }
  if (scale_out && blockIdx.x == 0 && threadIdx.x == 0) *scale_out = scale;
}

void launch_quant_rows(const float* x, int64_t M, int64_t K, int64_t Mpad, int64_t Kpad, const uint32_t* slot,
                       int8_t* q, float* scale_out, hipStream_t s) {
  const int64_t chunks = Mpad * (Kpad / 16);
  if (chunks <= 0) return;
  int64_t blocks = (chunks + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  const bool vec = (K % 4) == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0;
  if (vec)
    RG_LAUNCH(quant_rows_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, s, x, M, K, Mpad, Kpad, slot, q,
                       scale_out);
  else
    RG_LAUNCH(quant_rows_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, s, x, M, K, Mpad, Kpad, slot, q,
                       scale_out);
}

// ---------------------------------------------------------------------------
// FP16 operands (NpuPrecision::Fp16): round_fp16 (quantize.rs:50-64) of each
// f32 activation, stored as IEEE binary16 (exact, see rgmath::fp16_bits).
// Rows: x [M, K] -> h [Mpad, Kpad_h], one thread per 8 halves (16 bytes),
// zero padding.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t half2_of(float a, float b) {
  return (uint32_t)rgmath::fp16_bits(rgmath::round_fp16(a)) | ((uint32_t)rgmath::fp16_bits(rgmath::round_fp16(b)) << 16);
}

template <bool VEC>
__global__ __launch_bounds__(256) void half_rows_kernel(const float* __restrict__ x, int64_t M, int64_t K,
                                                        int64_t Mpad, int64_t Kpad_h, uint16_t* __restrict__ h) {
  const uint32_t chunks = (uint32_t)(Kpad_h / 8);
  const int64_t total = Mpad * (int64_t)chunks;
  for (int64_t w = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; w < total; w += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = w / chunks;
    const uint32_t c0 = (uint32_t)(w - r * chunks) * 8u;
    v4i out = v4i{0, 0, 0, 0};
    if (r < M) {
      const float* xr = x + r * K;
      float v[8];
      if (VEC && c0 + 8 <= (uint32_t)K) {
        const float4 p = reinterpret_cast<const float4*>(xr + c0)[0], q = reinterpret_cast<const float4*>(xr + c0)[1];
        v[0] = p.x; v[1] = p.y; v[2] = p.z; v[3] = p.w; v[4] = q.x; v[5] = q.y; v[6] = q.z; v[7] = q.w;
      } else {
#pragma unroll
        for (int e = 0; e < 8; e++) v[e] = c0 + (uint32_t)e < (uint32_t)K ? xr[c0 + e] : 0.0f;
      }
#pragma unroll
      for (int g = 0; g < 4; g++) out[g] = (int)half2_of(v[2 * g], v[2 * g + 1]);
    }
    reinterpret_cast<v4i*>(h)[w] = out;
  }
}

// Rows whose K is a multiple of 4 on a 16-byte aligned base are read with
// 16-byte loads.
void launch_half_rows(const float* x, int64_t M, int64_t K, int64_t Mpad, int64_t Kpad_h, uint16_t* h, hipStream_t s) {
  const int64_t chunks = Mpad * (Kpad_h / 8);
  if (chunks <= 0) return;
  int64_t blocks = (chunks + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  const bool vec = (K % 4) == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0;
  if (vec)
    RG_LAUNCH(half_rows_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, s, x, M, K, Mpad, Kpad_h, h);
  else
    RG_LAUNCH(half_rows_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, s, x, M, K, Mpad, Kpad_h, h);
}

// im2col in binary16 for the FP16 conv (npu.rs:341-355): row img*L + oy*OW + ox,
// column kk = (c*k + ki)*k + kj as in im2col_into (kernels.rs:28-96), value
// round_fp16(x) or 0 for padding; rows past n*L and columns past C*k*k are 0.
__global__ __launch_bounds__(256) void im2col_half_kernel(const float* __restrict__ x, ConvShape cs, int64_t Mpad,
                                                          int64_t Kpad_h, uint16_t* __restrict__ h) {
  const uint32_t k = (uint32_t)cs.k, kk2 = k * k, ckk = (uint32_t)cs.C * kk2;
  const uint32_t L = (uint32_t)(cs.OH * cs.OW), OW = (uint32_t)cs.OW;
  const uint32_t H = (uint32_t)cs.H, W = (uint32_t)cs.W;
  const int64_t rows = cs.n * (int64_t)L;
  const uint32_t chunks = (uint32_t)(Kpad_h / 8);
  const int64_t total = Mpad * (int64_t)chunks;
  for (int64_t w = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; w < total; w += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = w / chunks;
    const uint32_t c0 = (uint32_t)(w - r * chunks) * 8u;
    v4i out = v4i{0, 0, 0, 0};
    if (r < rows) {
      const int64_t img = r / L;
      const uint32_t p = (uint32_t)(r - img * L);
      const uint32_t oy = p / OW, ox = p - oy * OW;
      const float* xi = x + img * (int64_t)(cs.C * cs.H * cs.W);
      float v[8];
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const uint32_t kk = c0 + (uint32_t)e;
        float val = 0.0f;
        if (kk < ckk) {
          const uint32_t c = kk / kk2, t = kk - c * kk2, ki = t / k, kj = t - ki * k;
          const int iy = (int)(oy * (uint32_t)cs.stride + ki) - (int)cs.pad;
          const int ix = (int)(ox * (uint32_t)cs.stride + kj) - (int)cs.pad;
          if (iy >= 0 && iy < (int)H && ix >= 0 && ix < (int)W) val = xi[(c * H + (uint32_t)iy) * W + (uint32_t)ix];
        }
        v[e] = val;
      }
#pragma unroll
      for (int g = 0; g < 4; g++) out[g] = (int)half2_of(v[2 * g], v[2 * g + 1]);
    }
    reinterpret_cast<v4i*>(h)[w] = out;
  }
}

void launch_im2col_half(const float* x, const ConvShape& cs, int64_t Mpad, int64_t Kpad_h, uint16_t* h,
                        hipStream_t s) {
  const int64_t chunks = Mpad * (Kpad_h / 8);
  if (chunks <= 0) return;
  int64_t blocks = (chunks + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  RG_LAUNCH(im2col_half_kernel, dim3((unsigned)blocks), dim3(256), 0, s, x, cs, Mpad, Kpad_h, h);
}

// y_lo [n*L, O] (row stride O) -> NCHW [n, O, L] (transpose2d_into per image,
// npu.rs:356).  One thread per output element, consecutive l per thread.
__global__ __launch_bounds__(256) void nlo_to_nchw_kernel(const float* __restrict__ ylo, int64_t n, int64_t O,
                                                          int64_t L, float* __restrict__ y) {
  const int64_t total = n * O * L;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t img = e / (O * L);
    const int64_t rem = e - img * O * L;
    const int64_t o = rem / L, l = rem - o * L;
    y[e] = ylo[(img * L + l) * O + o];
  }
}

// Direct convolution for the FP16 and FP32 providers when a window holds at
// most kDirectConvTaps values (C * k * k: the CNN's first conv has 27).  The
// im2col matrix would be written to HBM and fed to an MFMA tile whose
// columns the few output channels barely fill; here one thread computes
// every output channel of one output pixel, summing the taps serially in
// the reference's im2col order (ch * k + ki) * k + kj, padding taps (zeros)
// included, as fp16_gemm_fused (npu.rs:425-445) and the serial matmul of
// conv2d_forward (kernels.rs:218-265) do.  FP16: each input is round_fp16'd
// and each product of two binary16 values is exact in f32, so fma gives the
// reference's multiply-then-add; the output is act(round_fp16(sum + bias)).
// FP32: multiply, then add (no contraction); the output is sum + bias (the
// activation is a layer of its own).  The weights of one output channel are
// read at a wave-uniform address.
// FP16 direct conv outputs: act(round_fp16(acc + bias)) per output channel.
template <int ACT, int OMAX>
__device__ __forceinline__ void conv_direct_store_f16(const float (&acc)[OMAX], const float* __restrict__ bias,
                                                      float* yb, int64_t L, int O, float act_param) {
#pragma unroll
  for (int o = 0; o < OMAX; o++)
    if (o < O) yb[(int64_t)o * L] = act_fixed<ACT>(rgmath::round_fp16(acc[o] + bias[o]), act_param);
}

// The max pool's window step: NaN propagates and ties keep the earlier
// element (kernels.rs:180-191).
__device__ __forceinline__ float pool_take(float best, float v) { return (v > best || v != v) ? v : best; }

// Direct conv -> MaxPool2d(2, 2) (npu.rs:384-390): the outputs as in
// conv_direct_store_f16 (FP16) or the FP32 store followed by the
// activation op's act_fixed (FP32: conv, Act, pool), pooled in registers.  OW is 16 or 32 and OH even
// (host-checked), so a wave's 64 pixels are whole pairs of output rows:
// pixel p + 1 is in lane ^ 1 and p + OW in lane ^ OW.  The even-row,
// even-column lanes take the window in the reference's order with
// pool_take and store the pooled value; every lane takes part in the
// shuffles (lanes past the last pixel computed a clamped one).
template <int ACT, int OMAX, int MODE>
__device__ __forceinline__ void conv_direct_pool(const float (&acc)[OMAX], const float* __restrict__ bias,
                                                     float* __restrict__ y, int64_t b, int O, int OH, int OW,
                                                     int64_t pix, bool live, float act_param) {
  const int oy = (int)(pix / OW), ox = (int)(pix - (int64_t)oy * OW);
  const bool lead = live && (oy & 1) == 0 && (ox & 1) == 0;
  const int64_t PL = (int64_t)(OH >> 1) * (OW >> 1);
  float* const yb = y + b * (int64_t)O * PL + (oy >> 1) * (OW >> 1) + (ox >> 1);
#pragma unroll
  for (int o = 0; o < OMAX; o++) {
    if (o < O) {  // O is the same for the whole wave (no break: it put acc on the stack)
      const float s = acc[o] + bias[o];
      const float v = act_fixed<ACT>(MODE == kModeF16 ? rgmath::round_fp16(s) : s, act_param);
      const float h = __shfl_xor(v, 1);
      const float d = __shfl_xor(v, OW);
      const float dh = __shfl_xor(h, OW);
      float best = -__builtin_inff();
      best = pool_take(best, v);
      best = pool_take(best, h);
      best = pool_take(best, d);
      best = pool_take(best, dh);
      if (lead) yb[(int64_t)o * PL] = best;
    }
  }
}

template <int OMAX, int MODE>
__global__ __launch_bounds__(256) void conv_direct_kernel(const float* __restrict__ x, const void* __restrict__ wv,
                                                          const float* __restrict__ bias, float* __restrict__ y,
                                                          ConvShape cs, int act, float act_param, int pool2) {
  // weights as f32, tap-major [tap][OMAX] (channels past O are zero), so a
  // tap's weights are OMAX / 4 broadcast 16-byte LDS reads
  __shared__ __attribute__((aligned(16))) float ws[kDirectConvTaps * OMAX];
  const int taps = (int)(cs.C * cs.k * cs.k), O = (int)cs.O, k = (int)cs.k;
  for (int i = threadIdx.x; i < taps * OMAX; i += blockDim.x) {
    const int kk = i / OMAX, o = i - kk * OMAX;
    float w = 0.0f;
    if (o < O) {
      if constexpr (MODE == kModeF16)
        w = (float)reinterpret_cast<const _Float16*>(wv)[(int64_t)o * cs.Kpad + kk];
      else
        w = reinterpret_cast<const float*>(wv)[(int64_t)o * cs.Kpad + kk];
    }
    ws[i] = w;
  }
  __syncthreads();
  const int64_t b = blockIdx.y;
  const int64_t L = cs.OH * cs.OW;
  const int64_t pix_raw = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const bool live = pix_raw < L;
  if (!live && !pool2) return;
  const int64_t pix = live ? pix_raw : L - 1;  // pooled: every lane joins the shuffles
  const int oy = (int)(pix / cs.OW), ox = (int)(pix - (int64_t)oy * cs.OW);
  const int iy0 = oy * (int)cs.stride - (int)cs.pad, ix0 = ox * (int)cs.stride - (int)cs.pad;
  const int H = (int)cs.H, W = (int)cs.W;
  const float* xb = x + b * cs.C * cs.H * cs.W;
  float acc[OMAX];
#pragma unroll
  for (int o = 0; o < OMAX; o++) acc[o] = 0.0f;
  int kk = 0;
  for (int ch = 0; ch < (int)cs.C; ch++)
    for (int ki = 0; ki < k; ki++) {
      const int iy = iy0 + ki;
      const bool row_ok = iy >= 0 && iy < H;
      const float* xr = xb + ((int64_t)ch * H + iy) * W;
      for (int kj = 0; kj < k; kj++, kk++) {
        const int ix = ix0 + kj;
        float v = (row_ok && ix >= 0 && ix < W) ? xr[ix] : 0.0f;
        const float4* wr = reinterpret_cast<const float4*>(ws + kk * OMAX);
        if constexpr (MODE == kModeF16) {
          v = rgmath::round_fp16(v);
#pragma unroll
          for (int q = 0; q < OMAX / 4; q++) {
            const float4 w4 = wr[q];
            acc[4 * q] = __builtin_fmaf(v, w4.x, acc[4 * q]);
            acc[4 * q + 1] = __builtin_fmaf(v, w4.y, acc[4 * q + 1]);
            acc[4 * q + 2] = __builtin_fmaf(v, w4.z, acc[4 * q + 2]);
            acc[4 * q + 3] = __builtin_fmaf(v, w4.w, acc[4 * q + 3]);
          }
        } else {
#pragma unroll
          for (int q = 0; q < OMAX / 4; q++) {
            const float4 w4 = wr[q];
            const float p0 = v * w4.x, p1 = v * w4.y, p2 = v * w4.z, p3 = v * w4.w;
            acc[4 * q] = acc[4 * q] + p0;
            acc[4 * q + 1] = acc[4 * q + 1] + p1;
            acc[4 * q + 2] = acc[4 * q + 2] + p2;
            acc[4 * q + 3] = acc[4 * q + 3] + p3;
          }
        }
      }
    }
  if (pool2) {
    if (act == rgmath::ACT_RELU)
      conv_direct_pool<rgmath::ACT_RELU, OMAX, MODE>(acc, bias, y, b, O, (int)cs.OH, (int)cs.OW, pix, live, act_param);
    else
      conv_direct_pool<rgmath::ACT_NONE, OMAX, MODE>(acc, bias, y, b, O, (int)cs.OH, (int)cs.OW, pix, live, act_param);
    return;
  }
  float* yb = y + b * (int64_t)O * L + pix;
  if constexpr (MODE == kModeF16) {
    // one activation per unrolled store loop: with the activation switch
    // inside the loop, the accumulators ended up on the stack
#define RG_CDS(ACTV) conv_direct_store_f16<ACTV, OMAX>(acc, bias, yb, L, O, act_param)
    switch (act) {
      case rgmath::ACT_RELU: RG_CDS(rgmath::ACT_RELU); break;
      case rgmath::ACT_SIGMOID: RG_CDS(rgmath::ACT_SIGMOID); break;
      case rgmath::ACT_TANH: RG_CDS(rgmath::ACT_TANH); break;
      case rgmath::ACT_GELU: RG_CDS(rgmath::ACT_GELU); break;
      case rgmath::ACT_LEAKY_RELU: RG_CDS(rgmath::ACT_LEAKY_RELU); break;
      case rgmath::ACT_SILU: RG_CDS(rgmath::ACT_SILU); break;
      default: RG_CDS(rgmath::ACT_NONE); break;
    }
#undef RG_CDS
  } else {
#pragma unroll
    for (int o = 0; o < OMAX; o++)
      if (o < O) yb[(int64_t)o * L] = acc[o] + bias[o];
  }
}

template <int MODE>
static void launch_conv_direct_t(const float* x, const void* w, const float* bias, float* y, const ConvShape& cs,
                                 int act, float act_param, int pool2, hipStream_t s) {
  if (cs.C * cs.k * cs.k > kDirectConvTaps || cs.O > 64 || cs.O <= 0)
    throw std::logic_error("direct conv: window or output channels too large");
  if (pool2 && ((pool2 != 16 && pool2 != 32) || cs.OW != pool2 || cs.OH % 2 != 0 ||
                (act != rgmath::ACT_RELU && act != rgmath::ACT_NONE)))
    throw std::logic_error("direct conv: the fused pool needs ReLU or none, even height, width 16 or 32");
  const int64_t L = cs.OH * cs.OW;
  if (L <= 0 || cs.n <= 0) return;
  if (cs.n > 65535) throw std::logic_error("direct conv: too many images for one launch");
  const dim3 grid((unsigned)((L + 255) / 256), (unsigned)cs.n);
  if (cs.O <= 16)
    RG_LAUNCH((conv_direct_kernel<16, MODE>), grid, dim3(256), 0, s, x, w, bias, y, cs, act, act_param, pool2);
  else if (cs.O <= 32)
    RG_LAUNCH((conv_direct_kernel<32, MODE>), grid, dim3(256), 0, s, x, w, bias, y, cs, act, act_param, pool2);
  else
    RG_LAUNCH((conv_direct_kernel<64, MODE>), grid, dim3(256), 0, s, x, w, bias, y, cs, act, act_param, pool2);
}

void launch_conv_direct_f16(const float* x, const uint16_t* w, const float* bias, float* y, const ConvShape& cs,
                            int act, float act_param, int pool_ow, hipStream_t s) {
  launch_conv_direct_t<kModeF16>(x, w, bias, y, cs, act, act_param, pool_ow, s);
}

void launch_conv_direct_f32(const float* x, const float* w, const float* bias, float* y, const ConvShape& cs,
                            int pool_act, int pool_ow, hipStream_t s) {
  launch_conv_direct_t<kModeF32>(x, w, bias, y, cs, pool_ow ? pool_act : rgmath::ACT_NONE, 0.0f, pool_ow, s);
}

void launch_nlo_to_nchw(const float* ylo, int64_t n, int64_t O, int64_t L, float* y, hipStream_t s) {
  const int64_t total = n * O * L;
  if (total <= 0) return;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  RG_LAUNCH(nlo_to_nchw_kernel, dim3((unsigned)blocks), dim3(256), 0, s, ylo, n, O, L, y);
}

// ---------------------------------------------------------------------------
// Standard FP32 path operands: x [M, K] -> A [Mpad, Kpad_f] f32 zero padded
// (one thread per 4 floats), and im2col in f32 with the reference's column
// order (kernels.rs:28-96).
// ---------------------------------------------------------------------------
template <bool VEC>
__global__ __launch_bounds__(256) void pad_rows_f32_kernel(const float* __restrict__ x, int64_t M, int64_t K,
                                                           int64_t Mpad, int64_t Kpad_f, float* __restrict__ a) {
  const uint32_t chunks = (uint32_t)(Kpad_f / 4);
  const int64_t total = Mpad * (int64_t)chunks;
  for (int64_t w = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; w < total; w += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = w / chunks;
    const uint32_t c0 = (uint32_t)(w - r * chunks) * 4u;
    float4 out = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (r < M) {
      const float* xr = x + r * K;
      if (VEC && c0 + 4 <= (uint32_t)K) {
        out = *reinterpret_cast<const float4*>(xr + c0);
      } else {
        out.x = c0 < (uint32_t)K ? xr[c0] : 0.0f;
        out.y = c0 + 1 < (uint32_t)K ? xr[c0 + 1] : 0.0f;
        out.z = c0 + 2 < (uint32_t)K ? xr[c0 + 2] : 0.0f;
        out.w = c0 + 3 < (uint32_t)K ? xr[c0 + 3] : 0.0f;
      }
    }
    reinterpret_cast<float4*>(a)[w] = out;
  }
}

void launch_pad_rows_f32(const float* x, int64_t M, int64_t K, int64_t Mpad, int64_t Kpad_f, float* a, hipStream_t s) {
  const int64_t chunks = Mpad * (Kpad_f / 4);
  if (chunks <= 0) return;
  int64_t blocks = (chunks + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  if ((K % 4) == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0)
    RG_LAUNCH(pad_rows_f32_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, s, x, M, K, Mpad, Kpad_f, a);
  else
    RG_LAUNCH(pad_rows_f32_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, s, x, M, K, Mpad, Kpad_f, a);
}

__global__ __launch_bounds__(256) void im2col_f32_kernel(const float* __restrict__ x, ConvShape cs, int64_t Mpad,
                                                         int64_t Kpad_f, float* __restrict__ a) {
  const uint32_t k = (uint32_t)cs.k, kk2 = k * k, ckk = (uint32_t)cs.C * kk2;
  const uint32_t L = (uint32_t)(cs.OH * cs.OW), OW = (uint32_t)cs.OW;
  const uint32_t H = (uint32_t)cs.H, W = (uint32_t)cs.W;
  const int64_t rows = cs.n * (int64_t)L;
  const int64_t total = Mpad * Kpad_f;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = e / Kpad_f;
    const uint32_t kk = (uint32_t)(e - r * Kpad_f);
    float val = 0.0f;
    if (r < rows && kk < ckk) {
      const int64_t img = r / L;
      const uint32_t p = (uint32_t)(r - img * L);
      const uint32_t oy = p / OW, ox = p - oy * OW;
      const uint32_t c = kk / kk2, t = kk - c * kk2, ki = t / k, kj = t - ki * k;
      const int iy = (int)(oy * (uint32_t)cs.stride + ki) - (int)cs.pad;
      const int ix = (int)(ox * (uint32_t)cs.stride + kj) - (int)cs.pad;
      if (iy >= 0 && iy < (int)H && ix >= 0 && ix < (int)W)
        val = x[img * (int64_t)(cs.C * cs.H * cs.W) + (c * H + (uint32_t)iy) * W + (uint32_t)ix];
    }
    a[e] = val;
  }
}

void launch_im2col_f32(const float* x, const ConvShape& cs, int64_t Mpad, int64_t Kpad_f, float* a, hipStream_t s) {
  const int64_t total = Mpad * Kpad_f;
  if (total <= 0) return;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 16384) blocks = 16384;
  RG_LAUNCH(im2col_f32_kernel, dim3((unsigned)blocks), dim3(256), 0, s, x, cs, Mpad, Kpad_f, a);
}

// ChannelAffine of the standard path (mod.rs:295-306): channel axis 1,
// inner = product of the dimensions after it; y = x * scale[ch] + shift[ch]
// (multiply, then add).
__global__ __launch_bounds__(256) void channel_affine_kernel(const float* __restrict__ x, int64_t n, int64_t C,
                                                             int64_t inner, const float* __restrict__ scale,
                                                             const float* __restrict__ shift, float* __restrict__ y) {
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n; e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t ch = (e / inner) % C;
    const float prod = x[e] * scale[ch];
    y[e] = prod + shift[ch];
  }
}

void launch_channel_affine(const float* x, int64_t n, int64_t C, int64_t inner, const float* scale, const float* shift,
                           float* y, hipStream_t s) {
  if (n <= 0) return;
  int64_t blocks = (n + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  RG_LAUNCH(channel_affine_kernel, dim3((unsigned)blocks), dim3(256), 0, s, x, n, C, inner, scale, shift, y);
}

// Lone ChannelAffine in FP16: the diagonal FusedLinear's serial sum has a
// single non-zero term, the product with the raw scale (npu.rs:254-270,
// 433-445), so y = round_fp16(fl(round_fp16(x) * scale[c]) + shift[c]).
__global__ __launch_bounds__(256) void affine_f16_kernel(const float* __restrict__ x, int64_t n, int64_t C,
                                                         const float* __restrict__ scale,
                                                         const float* __restrict__ shift, float* __restrict__ y) {
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n; e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t c = e % C;
    const float prod = rgmath::round_fp16(x[e]) * scale[c];
    const float t = prod + shift[c];
    y[e] = rgmath::round_fp16(t);
  }
}

void launch_affine_f16(const float* x, int64_t n, int64_t C, const float* scale, const float* shift, float* y,
                       hipStream_t s) {
  if (n <= 0) return;
  int64_t blocks = (n + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  RG_LAUNCH(affine_f16_kernel, dim3((unsigned)blocks), dim3(256), 0, s, x, n, C, scale, shift, y);
}

// ---------------------------------------------------------------------------
// quantize images (conv input): per-image scale, same element layout.
// quantize(im2col(x)) == im2col(quantize(x)) elementwise, and padding zeros
// quantize to 0, so the conv kernel gathers from the quantized image.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void quant_images_kernel(const float* __restrict__ x, int64_t per_img,
                                                           const uint32_t* __restrict__ slots, int8_t* __restrict__ q,
                                                           float* scales_out) {
  const int64_t img = blockIdx.y;
  const float scale = slot_scale(slots + img);
  const float inv = 1.0f / scale;
  const float* xi = x + img * per_img;
  int8_t* qi = q + img * per_img;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < per_img; e += (int64_t)gridDim.x * blockDim.x)
    qi[e] = rgmath::quantize_one(xi[e], inv);
  if (scales_out && blockIdx.x == 0 && threadIdx.x == 0) scales_out[img] = scale;
}

void launch_quant_images(const float* x, int64_t per_img, int64_t n_img, const uint32_t* slots, int8_t* q,
                         float* scales_out, hipStream_t s) {
  if (per_img <= 0 || n_img <= 0) return;
  int64_t bx = (per_img + 255) / 256;
  if (bx > 1024) bx = 1024;
  RG_LAUNCH(quant_images_kernel, dim3((unsigned)bx, (unsigned)n_img), dim3(256), 0, s, x, per_img, slots, q,
                     scales_out);
}

// ---------------------------------------------------------------------------
// Tile epilogue.  The block's i32 accumulators are staged in LDS as
// Cs[TM][CLD]; 256 threads then walk the tile row-major so consecutive
// threads store consecutive f32 (coalesced) and each element is dequantized,
// biased and activated once.  CONV selects the NCHW conv indexing
// (rows = output channels, columns = pixels of image b).
// ---------------------------------------------------------------------------
struct TileCoords {
  int64_t m0, n0;     // tile origin
  int64_t M, N;       // valid extent (GEMM rows/cols or conv channels/pixels)
  int64_t img;        // conv image index
};

template <int TM, int TN, int CLD, bool CONV, int ACT>
__device__ __forceinline__ uint32_t epilogue_tile_act(const int32_t* Cs, const TileCoords& tc, float cs,
                                                      const Epilogue& ep) {
  uint32_t amax = 0;
  for (int e = threadIdx.x; e < TM * TN; e += 256) {
    const int r = e / TN, c = e % TN;
    const int64_t row = tc.m0 + r, col = tc.n0 + c;
    if (row < tc.M && col < tc.N) {
      const int32_t a = Cs[r * CLD + c];
      const float b = CONV ? ep.bias[row] : ep.bias[col];
      const float v = epi_value<ACT>(a, cs, b, ep.act_param);
      if (CONV) {
        ep.y[(tc.img * tc.M + row) * tc.N + col] = v;
        if (ep.acc_out) ep.acc_out[(tc.img * tc.N + col) * tc.M + row] = a;
      } else {
        ep.y[row * tc.N + col] = v;
        if (ep.acc_out) ep.acc_out[row * tc.N + col] = a;
      }
      const uint32_t k = rgmath::absmax_key(v);
      amax = k > amax ? k : amax;
    }
  }
  return amax;
}

template <int TM, int TN, int CLD, bool CONV>
__device__ __forceinline__ void epilogue_tile(const int32_t* Cs, const TileCoords& tc, float cs, const Epilogue& ep) {
  uint32_t amax = 0;
  switch (ep.act) {
    case rgmath::ACT_RELU: amax = epilogue_tile_act<TM, TN, CLD, CONV, rgmath::ACT_RELU>(Cs, tc, cs, ep); break;
    case rgmath::ACT_SIGMOID: amax = epilogue_tile_act<TM, TN, CLD, CONV, rgmath::ACT_SIGMOID>(Cs, tc, cs, ep); break;
    case rgmath::ACT_TANH: amax = epilogue_tile_act<TM, TN, CLD, CONV, rgmath::ACT_TANH>(Cs, tc, cs, ep); break;
    case rgmath::ACT_GELU: amax = epilogue_tile_act<TM, TN, CLD, CONV, rgmath::ACT_GELU>(Cs, tc, cs, ep); break;
    case rgmath::ACT_LEAKY_RELU:
      amax = epilogue_tile_act<TM, TN, CLD, CONV, rgmath::ACT_LEAKY_RELU>(Cs, tc, cs, ep);
      break;
    case rgmath::ACT_SILU: amax = epilogue_tile_act<TM, TN, CLD, CONV, rgmath::ACT_SILU>(Cs, tc, cs, ep); break;
    default: amax = epilogue_tile_act<TM, TN, CLD, CONV, rgmath::ACT_NONE>(Cs, tc, cs, ep); break;
  }
  if (ep.absmax_out) {
    amax = wave_max_u32(amax);
    if (CONV && ep.absmax_out_per_image) {
      if ((threadIdx.x & 63) == 0 && amax) atomicMax(ep.absmax_out + tc.img, amax);
    } else if ((threadIdx.x & 63) == 0) {
      spread_max(ep.absmax_out, amax);
    }
  }
}

// One staged 16-row slab: rows (wave-uniform) outputs per lane, row r at
// yrow + r N, byte offset col_bytes.  The stores are buffer stores with the
// row's byte offset r N 4 in a scalar register and the lane's column in a
// 32-bit vector offset (both fit: N <= 2^26), so the loop counter and all
// row addressing stay scalar.  Returns the running max of |y| (NaN ignored,
// like f32::max), as f32.
template <int ACT, bool CAP, int MODE>
__device__ __forceinline__ float big_epilogue_slab(const int32_t* slab, int rows, float* yrow, int32_t* arow,
                                                   int64_t N, uint32_t col_bytes, float cs, float b, float p,
                                                   int lane, float amax, bool stream) {
  const __amdgpu_buffer_rsrc_t ry = raw_rsrc(yrow);
  const __amdgpu_buffer_rsrc_t ra = raw_rsrc(arow);
  const uint32_t row_bytes = (uint32_t)N * 4u;
#pragma unroll 4
  for (int r = 0; r < rows; r++) {
    const int32_t a = slab[r * big::SLAB_LD + lane];
    const float v = epi_word<ACT, MODE>(a, cs, b, p);
    // The program's own output is not read again on the device: the
    // non-temporal hint keeps it from displacing operands in the caches.
    if (stream)
      __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), ry, (int)col_bytes, (int)(r * row_bytes), 2);
    else
      __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), ry, (int)col_bytes, (int)(r * row_bytes), 0);
    if (CAP) __builtin_amdgcn_raw_buffer_store_b32((uint32_t)a, ra, (int)col_bytes, (int)(r * row_bytes), 0);
    amax = __builtin_fmaxf(amax, __builtin_fabsf(v));
  }
  return amax;
}

// Stages the wave's (16 FM) x 64 accumulator tile through LDS 16 rows at a
// time and stores it row-major: lane l owns column n0 + wn*64 + l, so each
// store instruction writes 256 contiguous bytes.  The bias and scale were
// loaded before the K loop.
// FP16 hand-off (ep.h_out): the same slabs read back with 4 consecutive
// columns per lane; each output y = act(round_fp16(acc + b)) (npu.rs:442)
// becomes the consumer's binary16 operand fp16_bits(round_fp16(y)), exactly
// what the consumer's own conversion (half_rows_kernel) would write, with the
// operand's zero padding for rows past M and columns past N.  N % 4 == 0, so
// a lane's 4 columns are all outputs or all padding; columns at or past ldh
// are not part of the operand.  No f32 output is stored (capture runs do not
// hand off).
typedef unsigned int v2u __attribute__((ext_vector_type(2)));

// The binary16 operand of an FP16 output value (what half_rows_kernel writes).
__device__ __forceinline__ uint32_t h16(float y) { return rgmath::fp16_bits(rgmath::round_fp16(y)); }

// Certified GELU for the hand-off (ACT == GELU): the operand of
// gelu(pre) is h16 of it, and h16 never decreases (as the value it encodes)
// and never gives -0 over the finite f32 values (host check,
// tests/support/gelu_shape_check.cpp).  gelu_approx(pre) is within
// kGeluApproxRel |pre| + kGeluApproxAbs of gelu(pre) (device check), so when
// h16 agrees at both ends of that interval, widened for the roundings of its
// ends, it is the exact value's operand.  pre = round_fp16(acc + b) is always
// finite.  The values the test cannot decide go to a per-wave queue in LDS
// and get the exact GELU after the walk; a queue that overflows sends the
// wave through the exact walk again.
namespace f16c {
constexpr int kQueue = 512;        // entries per wave
constexpr int kQueueBase = 36864;  // bytes from the LDS array's start: past the 8 epilogue slabs
static_assert(kQueueBase >= 8 * big::SLAB, "the queues follow the slabs");
}  // namespace f16c

struct F16Cert {
  float c1, c2, c3;  // interval half-width e = c1 |pre| + c3 |g| + c2
};

__device__ __forceinline__ F16Cert f16_cert_const(int mode) {
  F16Cert c;
  c.c1 = rgmath::kGeluApproxRel * 1.001f;
  c.c2 = mode == 2 ? __builtin_inff() : rgmath::kGeluApproxAbs * 2.0f;
  c.c3 = mode == 3 ? 0x1p-18f : 0x1p-22f;  // 2^-22: the roundings of g -+ e; mode 3 queues ~1% of the values
  return c;
}

__device__ __forceinline__ uint32_t cert_h16(float pre, const F16Cert& c, bool& ok) {
  const float g = rgmath::gelu_approx(pre);
  const float e = __builtin_fmaf(c.c1, __builtin_fabsf(pre), __builtin_fmaf(c.c3, __builtin_fabsf(g), c.c2));
  const uint32_t lo = h16(g - e), hi = h16(g + e);
  ok = lo == hi;
  return lo;
}

__device__ __forceinline__ void f16_push(uint32_t* qx, uint32_t* qo, uint32_t& n, bool need, float pre,
                                         uint32_t off) {
  const uint64_t m = __builtin_amdgcn_ballot_w64(need);
  if (m == 0) return;
  if (need) {
    const uint32_t pos = n + __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
    if (pos < (uint32_t)f16c::kQueue) {
      qx[pos] = __float_as_uint(pre);
      qo[pos] = off;
    }
  }
  n += (uint32_t)__builtin_popcountll(m);
}

// FP16 hand-off (ep.h_out): the same slabs read back with 4 consecutive
// columns per lane; each output y = act(round_fp16(acc + b)) (npu.rs:442)
// becomes the consumer's binary16 operand fp16_bits(round_fp16(y)), exactly
// what the consumer's own conversion (half_rows_kernel) would write, with the
// operand's zero padding for rows past M and columns past N.  N % 4 == 0, so
// a lane's 4 columns are all outputs or all padding; columns at or past ldh
// are not part of the operand.  No f32 output is stored (capture runs do not
// hand off).  CERT: the certified GELU above.
template <int ACT, int FM, bool CERT>
__device__ __forceinline__ void big_epilogue_f16_handoff(int8_t* smem, int32_t* slab, const v4i (&acc)[FM][4],
                                                         int64_t m0, int64_t n0, int64_t M, int64_t N,
                                                         const Epilogue& ep, int wave, int wm, int wn, int lane) {
  const int sub = lane >> 4, c4 = (lane & 15) * 4;
  const int64_t row0 = m0 + wm * (16 * FM), col0 = n0 + wn * 64;
  const int64_t col = col0 + c4;
  const bool col_ok = col < N, h_ok = col < ep.ldh;
  const float4 b4 = col_ok ? *reinterpret_cast<const float4*>(ep.bias + col) : float4{0.0f, 0.0f, 0.0f, 0.0f};
  const float bb[4] = {b4.x, b4.y, b4.z, b4.w};
  // wave-uniform bases, 32-bit lane offsets (the plan bounds the operand and
  // output below 2^31 bytes per 128 rows), row offsets in the scalar offset
  const __amdgpu_buffer_rsrc_t rh = raw_rsrc(ep.h_out + row0 * ep.ldh + col0);
  const uint32_t hoff = (uint32_t)((sub * ep.ldh + c4) * 2), hrow = (uint32_t)ep.ldh * 2u;
  const int32_t rows_left = (int32_t)(M - row0 - sub);  // row 16 i + 4 p (+ sub) is an output iff 16 i + 4 p < rows_left
  uint32_t* const qx = reinterpret_cast<uint32_t*>(smem + f16c::kQueueBase) + wave * 2 * f16c::kQueue;
  uint32_t* const qo = qx + f16c::kQueue;
  uint32_t n = 0;
  const F16Cert cc = f16_cert_const(ep.gelu_cert);
#pragma unroll
  for (int i = 0; i < FM; i++) {
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int r = 0; r < 4; r++) slab[((lane >> 4) * 4 + r) * big::SLAB_LD + j * 16 + (lane & 15)] = acc[i][j][r];
    // the rows are read back from the slab in a rolled loop: acc is indexed
    // only by the unrolled staging above, so it stays in registers
#pragma unroll 1
    for (int p = 0; p < 4; p++) {
      const int ro = i * 16 + p * 4;
      const v4i a = *reinterpret_cast<const v4i*>(slab + (p * 4 + sub) * big::SLAB_LD + c4);
      const bool ok = ro < rows_left && col_ok;
      uint32_t hv[4];
      if constexpr (CERT) {
        bool o[4];
        float pre[4];
#pragma unroll
        for (int c = 0; c < 4; c++) {
          pre[c] = rgmath::round_fp16(__int_as_float(a[c]) + bb[c]);
          hv[c] = cert_h16(pre[c], cc, o[c]);
        }
        const bool valid = ok && h_ok;
        if (__builtin_amdgcn_ballot_w64(valid && !(o[0] && o[1] && o[2] && o[3]))) {
          const uint32_t off = hoff + (uint32_t)ro * hrow;
#pragma unroll
          for (int c = 0; c < 4; c++) f16_push(qx, qo, n, valid && !o[c], pre[c], off + 2u * c);
        }
      } else {
#pragma unroll
        for (int c = 0; c < 4; c++) hv[c] = h16(epi_word<ACT, kModeF16>(a[c], 1.0f, bb[c], ep.act_param));
      }
      if (h_ok) {
        const uint32_t lo = ok ? (hv[0] | (hv[1] << 16)) : 0u, hi = ok ? (hv[2] | (hv[3] << 16)) : 0u;
        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(v2u, make_uint2(lo, hi)), rh, (int)hoff,
                                              (int)((uint32_t)ro * hrow), 0);
      }
    }
  }
  if constexpr (CERT) {
    if (n == 0) return;
    if (n > (uint32_t)f16c::kQueue) {
      // overflow: the exact walk again (acc is unchanged)
      big_epilogue_f16_handoff<ACT, FM, false>(smem, slab, acc, m0, n0, M, N, ep, wave, wm, wn, lane);
      return;
    }
    // the walk's word stores have completed, so these 2-byte stores land
    // after them whichever lane makes them
    wait_vmcnt<0>();
    for (uint32_t j = (uint32_t)lane; j < n; j += 64)
      __builtin_amdgcn_raw_buffer_store_b16((uint16_t)h16(rgmath::gelu_fast(__uint_as_float(qx[j]))), rh,
                                            (int)qo[j], 0, 0);
  }
}

template <int ACT, bool CAP, int FM, int MODE>
__device__ __forceinline__ uint32_t big_epilogue(int8_t* smem, const v4i (&acc)[FM][4], int64_t m0, int64_t n0,
                                                 int64_t M, int64_t N, float cs, float b, const Epilogue& ep,
                                                 int wave, int wm, int wn, int lane) {
  int32_t* slab = reinterpret_cast<int32_t*>(smem + wave * big::SLAB);
  if constexpr (MODE == kModeF16) {
    if (ep.h_out) {
      if constexpr (ACT == rgmath::ACT_GELU) {
        if (ep.gelu_cert) {
          big_epilogue_f16_handoff<ACT, FM, true>(smem, slab, acc, m0, n0, M, N, ep, wave, wm, wn, lane);
          return 0u;
        }
      }
      big_epilogue_f16_handoff<ACT, FM, false>(smem, slab, acc, m0, n0, M, N, ep, wave, wm, wn, lane);
      return 0u;
    }
  }
  float amax = 0.0f;
  const int64_t col = n0 + wn * 64 + lane;
  // Every lane stages its accumulators (the slab is shared by the wave);
  // lanes past the last column then skip the slab loop.
  const bool col_ok = col < N;
#pragma unroll
  for (int i = 0; i < FM; i++) {
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int r = 0; r < 4; r++) slab[((lane >> 4) * 4 + r) * big::SLAB_LD + j * 16 + (lane & 15)] = acc[i][j][r];
    const int64_t row0 = m0 + wm * (16 * FM) + i * 16;
    const int rows = (int)(M - row0 < 16 ? (M - row0 > 0 ? M - row0 : 0) : 16);
    if (col_ok)
      amax = big_epilogue_slab<ACT, CAP, MODE>(slab, rows, ep.y + row0 * N, CAP ? ep.acc_out + row0 * N : nullptr, N,
                                               (uint32_t)col * 4u, cs, b, ep.act_param, lane, amax, ep.y_stream != 0);
  }
  return rgmath::fbits(amax);
}

template <int ACT, int FM, int MODE>
__device__ __forceinline__ uint32_t big_epilogue_any(int8_t* smem, const v4i (&acc)[FM][4], int64_t m0, int64_t n0,
                                                     int64_t M, int64_t N, float cs, float b, const Epilogue& ep,
                                                     int wave, int wm, int wn, int lane) {
  return ep.acc_out ? big_epilogue<ACT, true, FM, MODE>(smem, acc, m0, n0, M, N, cs, b, ep, wave, wm, wn, lane)
                    : big_epilogue<ACT, false, FM, MODE>(smem, acc, m0, n0, M, N, cs, b, ep, wave, wm, wn, lane);
}

// Split K: gridDim.y > 1 gives block (x, y) the K steps [y*ks, (y+1)*ks) and
// it stores its raw sums to ws[y][Mpad][Npad] for splitk_epilogue_kernel.
template <int BM, int BN, int WAVES_M, int WAVES_N, int STAGES, int OCC, int FM, int MODE>
__global__ __launch_bounds__(WAVES_M * WAVES_N * 64, OCC) void gemm_big_kernel(
    const int8_t* __restrict__ A, const int8_t* __restrict__ B, int64_t M, int64_t N, int64_t Kpad, int tiles_m,
    int tiles_n, Epilogue ep, int ks, int32_t* __restrict__ ws) {
  using namespace big;
  constexpr int NW = WAVES_M * WAVES_N;
  static_assert(BM == 16 * FM * WAVES_M && BN == 64 * WAVES_N, "wave tile is (16 FM) x 64");
  constexpr int ST = (BM + BN) * BK;
  static_assert(NW * SLAB <= STAGES * ST, "epilogue slabs reuse the ring");
  static_assert(MODE != kModeF16 || f16c::kQueueBase + NW * 8 * f16c::kQueue <= STAGES * ST,
                "the FP16 hand-off queues fit in the ring");
  __shared__ __attribute__((aligned(1024))) int8_t smem[STAGES * ST];
  // wave index read through a scalar register: the compiler then keeps the
  // wave's tile coordinates and row bases scalar
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;

  int tile_m, tile_n;
  tile_coords(blockIdx.x, tiles_m, tiles_n, tile_m, tile_n);
  const int64_t m0 = (int64_t)tile_m * BM, n0 = (int64_t)tile_n * BN;
  // Epilogue operands are fetched now; they arrive while the K loop runs.
  const int64_t my_col = n0 + wn * 64 + lane;
  const float bias_v = my_col < N ? ep.bias[my_col] : 0.0f;
  // Partial of the input absmax; folded after the K loop so the fold does not
  // wait on the prologue DMA.  (FP16 has no activation scale.)
  uint32_t absmax_part = 0;
  if constexpr (MODE == kModeI8) absmax_part = tensor_absmax_part(ep.absmax_in);

  // This block's K steps [kbeg, kbeg + nk).
  const int nk_all = (int)(Kpad / BK);
  const int kbeg = (int)blockIdx.y * ks;
  const int nk = min(ks, nk_all - kbeg);
  v4i acc[FM][4];
  big_kloop<BM, BN, WAVES_M, WAVES_N, STAGES, FM, MODE>(smem, A, B, Kpad, m0, n0, kbeg, nk, wave, wm, wn, lane, acc);
  if (gridDim.y > 1) {
    // Split K: raw sums for splitk_epilogue_kernel (padded extent, no masks).
    const int64_t Npad = (int64_t)tiles_n * BN;
    int32_t* w = ws + ((int64_t)blockIdx.y * tiles_m * BM + m0 + wm * 16 * FM + (lane >> 4) * 4) * Npad + n0 +
                 wn * 64 + (lane & 15);
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
      for (int j = 0; j < 4; j++)
#pragma unroll
        for (int r = 0; r < 4; r++) w[(int64_t)(i * 16 + r) * Npad + j * 16] = acc[i][j][r];
    (void)absmax_part;
    return;
  }
  const float cs =
      MODE != kModeI8 ? 1.0f : rgmath::scale_from_absmax(rgmath::bitsf(wave_max_u32(absmax_part))) * ep.w_scale;
  uint32_t amax = 0;
#define RG_BIG_EPI(ACTV) big_epilogue_any<ACTV, FM, MODE>(smem, acc, m0, n0, M, N, cs, bias_v, ep, wave, wm, wn, lane)
  switch (ep.act) {
    case rgmath::ACT_RELU: amax = RG_BIG_EPI(rgmath::ACT_RELU); break;
    case rgmath::ACT_SIGMOID: amax = RG_BIG_EPI(rgmath::ACT_SIGMOID); break;
    case rgmath::ACT_TANH: amax = RG_BIG_EPI(rgmath::ACT_TANH); break;
    case rgmath::ACT_GELU: amax = RG_BIG_EPI(rgmath::ACT_GELU); break;
    case rgmath::ACT_LEAKY_RELU: amax = RG_BIG_EPI(rgmath::ACT_LEAKY_RELU); break;
    case rgmath::ACT_SILU: amax = RG_BIG_EPI(rgmath::ACT_SILU); break;
    default: amax = RG_BIG_EPI(rgmath::ACT_NONE); break;
  }
#undef RG_BIG_EPI
  if (ep.absmax_out) {
    amax = wave_max_u32(amax);
    if (lane == 0) spread_max(ep.absmax_out, amax);
  }
}

// Split-K epilogue: the S partial sums added in slice order, then the fused
// epilogue (INT8: exact i32 sum; FP16: f32 sum).
template <int ACT, int MODE>
__global__ __launch_bounds__(256) void splitk_epilogue_kernel(const int32_t* __restrict__ ws, int S, int64_t M,
                                                              int64_t N, int64_t Mpad, int64_t Npad, Epilogue ep) {
  const int64_t n4 = Npad / 4, total = M * n4;
  uint32_t amax = 0;
  float cs = 1.0f;
  if constexpr (MODE == kModeI8) cs = tensor_scale(ep.absmax_in) * ep.w_scale;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = e / n4, c0 = (e - row * n4) * 4;
    const v4f bias = *reinterpret_cast<const v4f*>(ep.bias + c0);  // padded to Npad
    // The partials are loaded KB at a time, all issued before any is added
    // (a load-add loop waits for each in turn), then added in slice order;
    // past S a lane re-reads the last partial and does not add it.
    constexpr int KB = 8;
    v4i sum = v4i{0, 0, 0, 0};
    v4f f = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    for (int sp0 = 0; sp0 < S; sp0 += KB) {
      v4i part[KB];
#pragma unroll
      for (int u = 0; u < KB; u++) {
        const int sp = sp0 + u < S ? sp0 + u : S - 1;
        part[u] = *reinterpret_cast<const v4i*>(ws + ((int64_t)sp * Mpad + row) * Npad + c0);
      }
#pragma unroll
      for (int u = 0; u < KB; u++) {
        const bool ok = sp0 + u < S;  // a select, not a branch, so no load waits alone
        if constexpr (MODE != kModeI8) {
          const v4f g = f + __builtin_bit_cast(v4f, part[u]);
          f = ok ? g : f;
        } else {
          const v4i g = sum + part[u];
          sum = ok ? g : sum;
        }
      }
    }
    if constexpr (MODE != kModeI8) sum = __builtin_bit_cast(v4i, f);
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const int64_t col = c0 + q;
      if (col < N) {
        const float v = epi_word<ACT, MODE>(sum[q], cs, bias[q], ep.act_param);
        ep.y[row * N + col] = v;
        if (ep.acc_out) ep.acc_out[row * N + col] = sum[q];
        const uint32_t k = rgmath::absmax_key(v);
        amax = k > amax ? k : amax;
      }
    }
  }
  if (ep.absmax_out) {
    amax = wave_max_u32(amax);
    if ((threadIdx.x & 63) == 0) spread_max(ep.absmax_out, amax);
  }
}

template <int MODE>
static void launch_splitk_epilogue(const int32_t* ws, int S, int64_t M, int64_t N, int64_t Mpad, int64_t Npad,
                                   const Epilogue& ep, hipStream_t s) {
  int64_t blocks = (M * (Npad / 4) + 255) / 256;
  if (blocks > 2048) blocks = 2048;
  if (blocks < 1) blocks = 1;
#define RG_SKE(ACTV) \
  RG_LAUNCH((splitk_epilogue_kernel<ACTV, MODE>), dim3((unsigned)blocks), dim3(256), 0, s, ws, S, M, N, Mpad, Npad, ep)
  switch (ep.act) {
    case rgmath::ACT_RELU: RG_SKE(rgmath::ACT_RELU); break;
    case rgmath::ACT_SIGMOID: RG_SKE(rgmath::ACT_SIGMOID); break;
    case rgmath::ACT_TANH: RG_SKE(rgmath::ACT_TANH); break;
    case rgmath::ACT_GELU: RG_SKE(rgmath::ACT_GELU); break;
    case rgmath::ACT_LEAKY_RELU: RG_SKE(rgmath::ACT_LEAKY_RELU); break;
    case rgmath::ACT_SILU: RG_SKE(rgmath::ACT_SILU); break;
    default: RG_SKE(rgmath::ACT_NONE); break;
  }
#undef RG_SKE
}

template <int BM, int BN, int WAVES_M, int WAVES_N, int STAGES, int OCC, int FM, int MODE>
static void launch_big(const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t Mpad, int64_t Npad,
                       int64_t Kpad, const Epilogue& ep, int splits, int32_t* ws, hipStream_t s) {
  const int tm = (int)(Mpad / BM), tn = (int)(Npad / BN);
  const int nk = (int)(Kpad / big::BK);
  const int ks = (nk + splits - 1) / splits;
  RG_LAUNCH((gemm_big_kernel<BM, BN, WAVES_M, WAVES_N, STAGES, OCC, FM, MODE>), dim3((unsigned)(tm * tn), (unsigned)splits),
            dim3(WAVES_M * WAVES_N * 64), 0, s, A, B, M, N, Kpad, tm, tn, ep, ks, ws);
}

// Kernel choice.  Problems with at least 256 tiles of 256 x 256 (or 256 x 128)
// fill the CUs with the large kernels; smaller ones use 128 x 128 tiles and,
// below 128 tiles (fewer than half the CUs busy), split K over up to 512
// blocks of at least 4 K steps each through the workspace.
GemmChoice choose_gemm(int64_t Mpad, int64_t Npad, int64_t Kpad) {
  if (Mpad % 256 == 0 && Npad % 256 == 0 && (Mpad / 256) * (Npad / 256) >= 256) return {0, 1};
  if (Mpad % 256 == 0 && Npad % 128 == 0 && (Mpad / 256) * (Npad / 128) >= 256) return {1, 1};
  const int64_t tiles = (Mpad / 128) * (Npad / 128), nk = Kpad / big::BK;
  if (tiles >= 128) return {2, 1};
  int64_t S = 512 / (tiles > 0 ? tiles : 1);
  if (S > nk / 4) S = nk / 4;
  if (S < 1) S = 1;
  const int64_t ks = (nk + S - 1) / S;
  return {2, (int)((nk + ks - 1) / ks)};
}

int64_t gemm_workspace_bytes(int64_t Mpad, int64_t Npad, int64_t Kpad) {
  const GemmChoice g = choose_gemm(Mpad, Npad, Kpad);
  return g.kind == 2 && g.splits > 1 ? (int64_t)g.splits * Mpad * Npad * 4 : 0;
}

template <int MODE>
static void launch_gemm_t(const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t Mpad, int64_t Npad,
                          int64_t Kpad, const Epilogue& ep, int32_t* ws, int64_t ws_bytes, hipStream_t s) {
  if (Kpad % big::BK || Mpad % 128 || Npad % 128 || Kpad <= 0)
    throw std::logic_error("GEMM operands must be padded to 128 rows and 64-byte K steps");
  const GemmChoice g = choose_gemm(Mpad, Npad, Kpad);
  if (g.kind == 0) {
    launch_big<256, 256, 2, 4, 4, 1, 8, MODE>(A, B, M, N, Mpad, Npad, Kpad, ep, 1, nullptr, s);
  } else if (g.kind == 1) {
    launch_big<256, 128, 2, 2, 3, 2, 8, MODE>(A, B, M, N, Mpad, Npad, Kpad, ep, 1, nullptr, s);
  } else if (g.splits > 1 && ws && ws_bytes >= (int64_t)g.splits * Mpad * Npad * 4) {
    launch_big<128, 128, 2, 2, 4, 2, 4, MODE>(A, B, M, N, Mpad, Npad, Kpad, ep, g.splits, ws, s);
    launch_splitk_epilogue<MODE>(ws, g.splits, M, N, Mpad, Npad, ep, s);
  } else {
    launch_big<128, 128, 2, 2, 4, 2, 4, MODE>(A, B, M, N, Mpad, Npad, Kpad, ep, 1, nullptr, s);
  }
}

void launch_gemm(const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t Mpad, int64_t Npad, int64_t Kpad,
                 const Epilogue& ep, int32_t* ws, int64_t ws_bytes, hipStream_t s) {
  launch_gemm_t<kModeI8>(A, B, M, N, Mpad, Npad, Kpad, ep, ws, ws_bytes, s);
}

void launch_gemm_f32(const float* A, const float* B, int64_t M, int64_t N, int64_t Mpad, int64_t Npad,
                     int64_t Kpad_f, const Epilogue& ep, int32_t* ws, int64_t ws_bytes, hipStream_t s) {
  launch_gemm_t<kModeF32>(reinterpret_cast<const int8_t*>(A), reinterpret_cast<const int8_t*>(B), M, N, Mpad, Npad,
                          4 * Kpad_f, ep, ws, ws_bytes, s);
}

void launch_gemm_f16(const uint16_t* A, const uint16_t* B, int64_t M, int64_t N, int64_t Mpad, int64_t Npad,
                     int64_t Kpad_h, const Epilogue& ep, int32_t* ws, int64_t ws_bytes, hipStream_t s) {
  launch_gemm_t<kModeF16>(reinterpret_cast<const int8_t*>(A), reinterpret_cast<const int8_t*>(B), M, N, Mpad, Npad,
                          2 * Kpad_h, ep, ws, ws_bytes, s);
}

// ---------------------------------------------------------------------------
// GEMV for M <= 8: weight streaming, HBM-bound.
//
// A wave owns a group of R consecutive output features and walks all of K:
// per loop trip each lane issues U x R non-temporal 16-byte weight loads
// (U x 1 KiB coalesced per feature) before consuming any, plus the matching
// activation bytes (cache resident), and accumulates with v_dot4_i32_i8.
// The grid is persistent: it holds as many workgroups as fit on the device
// at once and each wave strides over feature groups, so the whole weight
// stream runs in one generation of waves with no tail.
//
// The MR x R partial sums are combined with a reduce-scatter butterfly:
// at each xor step a lane keeps one half of its sums and sends the other,
// so S sums cost S - 1 + log2(64 / S) shuffles instead of 6 S.  Afterwards
// lane L holds sum L / (64 / S), i.e. output (m, n + r) with m * R + r =
// L / (64 / S).
// ---------------------------------------------------------------------------
// Cross-lane exchange partners.  Offsets 32 and 16 use the gfx950
// v_permlane32_swap / v_permlane16_swap (lane l <-> l ^ 32 / l ^ 16); the
// smaller ones DPP within a 16-lane row: row_mirror (l ^ 15),
// row_half_mirror (l ^ 7) and quad permutes (l ^ 2, l ^ 1).  Each partner
// differs from l in bit OFF and agrees on every higher bit, which is all
// the butterfly below needs.
template <int OFF>
__device__ __forceinline__ int32_t dpp_partner(int32_t v) {
  static_assert(OFF == 8 || OFF == 4 || OFF == 2 || OFF == 1, "DPP partner offsets are 8, 4, 2, 1");
  constexpr int ctrl = OFF == 8 ? 0x140 : OFF == 4 ? 0x141 : OFF == 2 ? 0x4E : 0xB1;
  return __builtin_amdgcn_update_dpp(0, v, ctrl, 0xf, 0xf, false);
}

// Sum of two 32-bit words: i32 (INT8 sums) or the f32 values they hold (FP16).
template <bool F>
__device__ __forceinline__ int32_t add_word(int32_t a, int32_t b) {
  if constexpr (F)
    return __float_as_int(__int_as_float(a) + __int_as_float(b));
  else
    return a + b;
}

// Lanes with bit OFF clear get lo + partner's lo, the others hi + partner's hi.
template <int OFF, bool F = false>
__device__ __forceinline__ int32_t pair_combine(int32_t lo, int32_t hi, int lane) {
  if constexpr (OFF == 32) {
    const auto p = __builtin_amdgcn_permlane32_swap(lo, hi, false, false);
    return add_word<F>((int32_t)p[0], (int32_t)p[1]);
  } else if constexpr (OFF == 16) {
    const auto p = __builtin_amdgcn_permlane16_swap(lo, hi, false, false);
    return add_word<F>((int32_t)p[0], (int32_t)p[1]);
  } else {
    const bool up = (lane & OFF) != 0;
    return add_word<F>(up ? hi : lo, dpp_partner<OFF>(up ? lo : hi));
  }
}

template <int OFF, bool F = false>
__device__ __forceinline__ int32_t fold(int32_t t, int lane) { return pair_combine<OFF, F>(t, t, lane); }

// Reduce-scatter butterfly over the wave: S partial sums per lane in, one
// finished sum out; lane l holds sum l / (64 / S).  S - 1 exchanges while
// the sums halve, then log2(64 / S) folds of the last one.
template <int S, bool F = false>
__device__ __forceinline__ int32_t wave_reduce_scatter(int32_t (&v)[S], int lane) {
  static_assert(S >= 1 && S <= 64 && (S & (S - 1)) == 0, "S must be a power of two <= 64");
#define RG_RS_STEP(OFF, DIV)                                                  \
  if constexpr (S >= DIV) {                                                   \
    _Pragma("unroll") for (int i = 0; i < S / DIV; i++)                       \
      v[i] = pair_combine<OFF, F>(v[i], v[i + S / DIV], lane);                \
  }
  RG_RS_STEP(32, 2)
  RG_RS_STEP(16, 4)
  RG_RS_STEP(8, 8)
  RG_RS_STEP(4, 16)
  RG_RS_STEP(2, 32)
  RG_RS_STEP(1, 64)
#undef RG_RS_STEP
  int32_t t = v[0];
  if constexpr (S < 2) t = fold<32, F>(t, lane);
  if constexpr (S < 4) t = fold<16, F>(t, lane);
  if constexpr (S < 8) t = fold<8, F>(t, lane);
  if constexpr (S < 16) t = fold<4, F>(t, lane);
  if constexpr (S < 32) t = fold<2, F>(t, lane);
  if constexpr (S < 64) t = fold<1, F>(t, lane);
  return t;
}

constexpr int pow2_at_least(int v) { return v <= 1 ? 1 : 2 * pow2_at_least((v + 1) / 2); }

// F16 (NpuPrecision::Fp16): A and B hold binary16 values (8 per 16-byte
// chunk), the partial sums are f32 from v_dot2_f32_f16 (exact products; the
// summation order differs from the reference's serial one), and the
// epilogue is act(round_fp16(acc + bias)).
template <int MR, int R, int U, int MODE>
__global__ __launch_bounds__(256) void gemv_kernel(const int8_t* __restrict__ A, const int8_t* __restrict__ B,
                                                   int64_t N, int64_t groups, int64_t Kpad, Epilogue ep) {
  constexpr int S = pow2_at_least(MR * R);
  constexpr int SPREAD = 64 / S;  // lanes holding the same finished sum
  const int lane = threadIdx.x & 63;
  const int64_t waves = (int64_t)gridDim.x * 4;
  float cs = 1.0f;
  if constexpr (MODE == kModeI8) cs = tensor_scale(ep.absmax_in) * ep.w_scale;
  const int sidx = lane / SPREAD;
  const int om = sidx / R, orr = sidx % R;
  const bool owner = (lane % SPREAD) == 0 && sidx < MR * R;
  // Uniform trip count; past the end of K a lane re-reads the last chunk
  // (in bounds, cache resident) and pairs it with zero activations.
  const int64_t ntrip = (Kpad + 1024 * U - 1) / (1024 * U);
  const int64_t klast = Kpad - 16;
  uint32_t amax = 0;
  for (int64_t g = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); g < groups; g += waves) {
    const int64_t nb = g * R;
    const int64_t col = nb + orr;
    // Loaded and consumed by every lane (clamped column): a masked load would
    // leave its register pending on the skip path and force a full memory
    // wait at the next group.
    const float bias_v = ep.bias[col < N ? col : N - 1];
    int32_t acc[S];
#pragma unroll
    for (int i = 0; i < S; i++) acc[i] = 0;
    const int8_t* wrow = B + nb * Kpad;
    for (int64_t t = 0; t < ntrip; t++) {
      v4i w[U][R];
      v4i x[U][MR];
      bool ok[U];
#pragma unroll
      for (int u = 0; u < U; u++) {
        const int64_t k = (t * U + u) * 1024 + lane * 16;
        ok[u] = k < Kpad;
        const int64_t kk = ok[u] ? k : klast;
#pragma unroll
        for (int r = 0; r < R; r++)
          w[u][r] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(wrow + r * Kpad + kk));
#pragma unroll
        for (int m = 0; m < MR; m++) x[u][m] = *reinterpret_cast<const v4i*>(A + (int64_t)m * Kpad + kk);
      }
#pragma unroll
      for (int u = 0; u < U; u++)
#pragma unroll
        for (int m = 0; m < MR; m++) {
          const v4i xv = ok[u] ? x[u][m] : v4i{0, 0, 0, 0};
#pragma unroll
          for (int r = 0; r < R; r++) {
            int32_t a = acc[m * R + r];
            if constexpr (MODE == kModeF32) {
              const v4f xf = __builtin_bit_cast(v4f, xv), wf = __builtin_bit_cast(v4f, w[u][r]);
              float f = __int_as_float(a);
#pragma unroll
              for (int q = 0; q < 4; q++) f = __builtin_fmaf(xf[q], wf[q], f);
              a = __float_as_int(f);
            } else if constexpr (MODE == kModeF16) {
              const v8h xh = __builtin_bit_cast(v8h, xv), wh = __builtin_bit_cast(v8h, w[u][r]);
              float f = __int_as_float(a);
#pragma unroll
              for (int q = 0; q < 4; q++)
                f = __builtin_amdgcn_fdot2(v2h{xh[2 * q], xh[2 * q + 1]}, v2h{wh[2 * q], wh[2 * q + 1]}, f, false);
              a = __float_as_int(f);
            } else {
              a = __builtin_amdgcn_sdot4(xv[0], w[u][r][0], a, false);
              a = __builtin_amdgcn_sdot4(xv[1], w[u][r][1], a, false);
              a = __builtin_amdgcn_sdot4(xv[2], w[u][r][2], a, false);
              a = __builtin_amdgcn_sdot4(xv[3], w[u][r][3], a, false);
            }
            acc[m * R + r] = a;
          }
        }
    }
    const int32_t mine = wave_reduce_scatter<S, MODE != kModeI8>(acc, lane);
    // INT8: (acc as f32) * cs + bias with separate roundings, as in
    // epi_value.  FP16: round_fp16(acc + bias).
    float pre;
    if constexpr (MODE == kModeF16) {
      pre = rgmath::round_fp16(__int_as_float(mine) + bias_v);
    } else if constexpr (MODE == kModeF32) {
      pre = __int_as_float(mine) + bias_v;
    } else {
      const float prod = (float)mine * cs;
      pre = prod + bias_v;
    }
    if (owner && col < N) {
      float v;
      switch (ep.act) {
        case rgmath::ACT_RELU: v = act_fixed<rgmath::ACT_RELU>(pre, ep.act_param); break;
        case rgmath::ACT_SIGMOID: v = act_fixed<rgmath::ACT_SIGMOID>(pre, ep.act_param); break;
        case rgmath::ACT_TANH: v = act_fixed<rgmath::ACT_TANH>(pre, ep.act_param); break;
        case rgmath::ACT_GELU: v = act_fixed<rgmath::ACT_GELU>(pre, ep.act_param); break;
        case rgmath::ACT_LEAKY_RELU: v = act_fixed<rgmath::ACT_LEAKY_RELU>(pre, ep.act_param); break;
        case rgmath::ACT_SILU: v = act_fixed<rgmath::ACT_SILU>(pre, ep.act_param); break;
        default: v = pre; break;
      }
      ep.y[om * N + col] = v;
      if (ep.acc_out) ep.acc_out[om * N + col] = mine;
      const uint32_t key = rgmath::absmax_key(v);
      amax = key > amax ? key : amax;
    }
  }
  if (ep.absmax_out) {
    amax = wave_max_u32(amax);
    if (lane == 0) spread_max(ep.absmax_out, amax);
  }
}


template <int MR, int R, int U, int MODE>
void launch_gemv_t(const int8_t* A, const int8_t* B, int64_t N, int64_t Npad, int64_t Kpad, const Epilogue& ep,
                   hipStream_t s, int64_t max_blocks) {
  const void* fn = reinterpret_cast<const void*>(&gemv_kernel<MR, R, U, MODE>);
  static const int64_t cap = resident_blocks(fn);
  const int64_t groups = Npad / R;  // Npad is a multiple of 256, so of every R used
  int64_t blocks = (groups + 3) / 4;
  const int64_t lim = max_blocks > 0 ? max_blocks : cap;
  if (blocks > lim) blocks = lim;
  RG_LAUNCH((gemv_kernel<MR, R, U, MODE>), dim3((unsigned)blocks), dim3(256), 0, s, A, B, N, groups, Kpad, ep);
}

template <int MODE>
static void launch_gemv_any(const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t Npad, int64_t Kpad,
                            const Epilogue& ep, hipStream_t s) {
  // (R, U) from a sweep on the decode shapes (8192 x 28672 and 28672 x
  // 8192): more rows share each activation load as M grows; long K rows
  // favour 8 rows per wave.
  const bool long_k = Kpad >= 16384;
  switch (M) {
    case 1:
      // binary16 / f32 rows are 2-4x longer in bytes: two rows per wave with
      // 8 KiB of each in flight (FP16 layer 1 84 -> 70 us, FP32 168 -> 145 us;
      // the same per-lane order, so the same bits)
      if constexpr (MODE == kModeI8)
        launch_gemv_t<1, 4, 4, MODE>(A, B, N, Npad, Kpad, ep, s, 0);
      else
        launch_gemv_t<1, 2, 8, MODE>(A, B, N, Npad, Kpad, ep, s, 0);
      break;
    case 2: launch_gemv_t<2, 4, 4, MODE>(A, B, N, Npad, Kpad, ep, s, 0); break;
    case 3: launch_gemv_t<3, 4, 1, MODE>(A, B, N, Npad, Kpad, ep, s, 0); break;
    case 4: launch_gemv_t<4, 4, 1, MODE>(A, B, N, Npad, Kpad, ep, s, 0); break;
    case 5:
      long_k ? launch_gemv_t<5, 8, 1, MODE>(A, B, N, Npad, Kpad, ep, s, 0) : launch_gemv_t<5, 4, 1, MODE>(A, B, N, Npad, Kpad, ep, s, 0);
      break;
    case 6:
      long_k ? launch_gemv_t<6, 8, 1, MODE>(A, B, N, Npad, Kpad, ep, s, 0) : launch_gemv_t<6, 4, 1, MODE>(A, B, N, Npad, Kpad, ep, s, 0);
      break;
    case 7:
      long_k ? launch_gemv_t<7, 8, 1, MODE>(A, B, N, Npad, Kpad, ep, s, 0) : launch_gemv_t<7, 4, 1, MODE>(A, B, N, Npad, Kpad, ep, s, 0);
      break;
    default:
      long_k ? launch_gemv_t<8, 8, 1, MODE>(A, B, N, Npad, Kpad, ep, s, 0) : launch_gemv_t<8, 4, 1, MODE>(A, B, N, Npad, Kpad, ep, s, 0);
      break;
  }
}

// One-row INT8 GEMV that quantizes its own f32 input (QuantTensor::from_f32,
// quantize.rs:18-24 at npu.rs:312, then quantize.rs:104-113), so no
// quantize launch precedes it.  Each thread reads its share of the row into
// registers, then each wave issues the weight loads of its first trip; while
// they are in flight the workgroup stages the quantized row in LDS (the
// same quantize_one rule as quant_rows_kernel),
// with the scale from the spread slot the producer raised or, for a Linear
// whose input has no absmax yet (SELF), from the input's absmax, which every
// workgroup reduces itself from L2.  The weights then stream as in
// gemv_kernel<1, 4, 4, 0> (same lanes, same per-lane sdot4 order, same
// reduce-scatter and epilogue).  Workgroup 0 writes the i8 row and the
// scale to the capture taps when they are given.
constexpr int kGemvXqR = 4, kGemvXqU = 4;

template <bool SELF>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void gemv_xq_kernel(const float* __restrict__ x, const int8_t* __restrict__ B,
                                                      int64_t N, int64_t groups, int64_t K, int64_t Kpad, Epilogue ep,
                                                      int8_t* q_out, float* scale_out, SlotClear clear) {
  constexpr int R = kGemvXqR, U = kGemvXqU;
  constexpr int S = pow2_at_least(R);
  constexpr int SPREAD = 64 / S;
  __shared__ __attribute__((aligned(16))) int8_t xl[kGemvXqMaxK];
  __shared__ uint32_t red[4];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t waves = (int64_t)gridDim.x * 4;
  const int64_t g0 = (int64_t)blockIdx.x * 4 + wave;
  const int64_t ntrip = (Kpad + 1024 * U - 1) / (1024 * U);
  const int64_t klast = Kpad - 16;
  auto load_w = [&](int64_t g, int64_t t, v4i (&w)[U][R]) {
    const int8_t* wrow = B + g * R * Kpad;
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int64_t k = (t * U + u) * 1024 + lane * 16;
      const int64_t kk = k < Kpad ? k : klast;
#pragma unroll
      for (int r = 0; r < R; r++)
        w[u][r] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(wrow + r * Kpad + kk));
    }
  };
  // The whole row is read into registers first (8 float4 per thread, zeros
  // past K), then the slot partial, then the first trip's weights: vector
  // loads complete in issue order, so the row and the slot are usable while
  // the weights are still in flight.
  constexpr int XB = kGemvXqMaxK / 1024;
  const v4f* const x4 = reinterpret_cast<const v4f*>(x);
  const int K4 = (int)(K >> 2), Kp4 = (int)(Kpad >> 2);
  v4f v[XB];
#pragma unroll
  for (int j = 0; j < XB; j++) {
    const int c = (int)threadIdx.x + 256 * j;
    v[j] = c < K4 ? x4[c] : v4f{0.f, 0.f, 0.f, 0.f};
  }
  uint32_t part = 0;
  if constexpr (!SELF) part = tensor_absmax_part(ep.absmax_in);
  // (issued unconditionally, clamped to the last group, so the waits below
  // count exactly these 16 loads as the newer ones)
  v4i w[U][R];
  load_w(g0 < groups ? g0 : groups - 1, 0, w);
  // The row is used only after this point, so its wait (vmcnt(16)) and the
  // staging arithmetic stay behind the weight loads.
#pragma unroll
  for (int j = 0; j < XB; j++) asm volatile("" : "+v"(v[j]));
  // A workgroup barrier without the fence of __syncthreads, whose vmcnt(0)
  // would wait for the weights: LDS writes complete first, then s_barrier.
  auto lds_barrier = [] {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };

  uint32_t m;
  if constexpr (SELF) {
    m = 0;
#pragma unroll
    for (int j = 0; j < XB; j++) {
      const uint32_t a = max(rgmath::absmax_key(v[j][0]), rgmath::absmax_key(v[j][1]));
      const uint32_t b = max(rgmath::absmax_key(v[j][2]), rgmath::absmax_key(v[j][3]));
      m = max(m, max(a, b));
    }
    m = wave_max_u32(m);
    if (lane == 0) red[wave] = m;
    lds_barrier();
    m = max(max(red[0], red[1]), max(red[2], red[3]));
  } else {
    m = wave_max_u32(part);
  }
  const float scale = rgmath::scale_from_absmax(rgmath::bitsf(m));
  const float inv = 1.0f / scale;
  uint32_t* const xw = reinterpret_cast<uint32_t*>(xl);
#pragma unroll
  for (int j = 0; j < XB; j++) {
    const int c = (int)threadIdx.x + 256 * j;
    if (c < Kp4) xw[c] = pack4(v[j][0], v[j][1], v[j][2], v[j][3], inv);
  }
  lds_barrier();
  // (after the staging: clear_slots reads the block size from the dispatch
  // packet with a vector load, whose wait would also wait for the weights)
  if constexpr (SELF) clear_slots(clear);
  if (blockIdx.x == 0) {
    if (q_out)
      for (int64_t i = threadIdx.x; i < Kp4; i += 256) reinterpret_cast<uint32_t*>(q_out)[i] = xw[i];
    if (scale_out && threadIdx.x == 0) *scale_out = scale;
  }

  const float cs = scale * ep.w_scale;
  const int sidx = lane / SPREAD;
  const int orr = sidx % R;
  const bool owner = (lane % SPREAD) == 0 && sidx < R;
  uint32_t amax = 0;
  for (int64_t g = g0; g < groups; g += waves) {
    const int64_t col = g * R + orr;
    const float bias_v = ep.bias[col < N ? col : N - 1];
    int32_t acc[S];
#pragma unroll
    for (int i = 0; i < S; i++) acc[i] = 0;
    for (int64_t t = 0; t < ntrip; t++) {
      // the first trip of the first group was issued before the staging
      if (g != g0 || t != 0) load_w(g, t, w);
#pragma unroll
      for (int u = 0; u < U; u++) {
        const int64_t k = (t * U + u) * 1024 + lane * 16;
        const bool ok = k < Kpad;
        const v4i xr = *reinterpret_cast<const v4i*>(xl + (ok ? k : klast));
        const v4i xv = ok ? xr : v4i{0, 0, 0, 0};
#pragma unroll
        for (int r = 0; r < R; r++) {
          int32_t a = acc[r];
          a = __builtin_amdgcn_sdot4(xv[0], w[u][r][0], a, false);
          a = __builtin_amdgcn_sdot4(xv[1], w[u][r][1], a, false);
          a = __builtin_amdgcn_sdot4(xv[2], w[u][r][2], a, false);
          a = __builtin_amdgcn_sdot4(xv[3], w[u][r][3], a, false);
          acc[r] = a;
        }
      }
    }
    const int32_t mine = wave_reduce_scatter<S, false>(acc, lane);
    const float prod = (float)mine * cs;
    const float pre = prod + bias_v;
    if (owner && col < N) {
      float v;
      switch (ep.act) {
        case rgmath::ACT_RELU: v = act_fixed<rgmath::ACT_RELU>(pre, ep.act_param); break;
        case rgmath::ACT_SIGMOID: v = act_fixed<rgmath::ACT_SIGMOID>(pre, ep.act_param); break;
        case rgmath::ACT_TANH: v = act_fixed<rgmath::ACT_TANH>(pre, ep.act_param); break;
        case rgmath::ACT_GELU: v = act_fixed<rgmath::ACT_GELU>(pre, ep.act_param); break;
        case rgmath::ACT_LEAKY_RELU: v = act_fixed<rgmath::ACT_LEAKY_RELU>(pre, ep.act_param); break;
        case rgmath::ACT_SILU: v = act_fixed<rgmath::ACT_SILU>(pre, ep.act_param); break;
        default: v = pre; break;
      }
      ep.y[col] = v;
      if (ep.acc_out) ep.acc_out[col] = mine;
      const uint32_t key = rgmath::absmax_key(v);
      amax = key > amax ? key : amax;
    }
  }
  if (ep.absmax_out) {
    amax = wave_max_u32(amax);
    if (lane == 0) spread_max(ep.absmax_out, amax);
  }
}

bool gemv_xq_supported(int64_t M, int64_t K, int64_t Kpad, const void* x) {
  return M == 1 && K % 4 == 0 && Kpad <= kGemvXqMaxK && (reinterpret_cast<uintptr_t>(x) & 15) == 0;
}

void launch_gemv_xq(const float* x, const int8_t* B, int64_t N, int64_t Npad, int64_t K, int64_t Kpad,
                    const Epilogue& ep, bool self_absmax, int8_t* q_out, float* scale_out, const SlotClear& clear,
                    hipStream_t s) {
  const int64_t groups = Npad / kGemvXqR;
  const int64_t want = (groups + 3) / 4;
  if (self_absmax) {
    static const int64_t cap = resident_blocks(reinterpret_cast<const void*>(&gemv_xq_kernel<true>));
    RG_LAUNCH(gemv_xq_kernel<true>, dim3((unsigned)(want < cap ? want : cap)), dim3(256), 0, s, x, B, N, groups, K,
              Kpad, ep, q_out, scale_out, clear);
  } else {
    static const int64_t cap = resident_blocks(reinterpret_cast<const void*>(&gemv_xq_kernel<false>));
    RG_LAUNCH(gemv_xq_kernel<false>, dim3((unsigned)(want < cap ? want : cap)), dim3(256), 0, s, x, B, N, groups,
              K, Kpad, ep, q_out, scale_out, clear);
  }
}

// INT8 GEMV on the matrix cores for a few rows (quantize.rs:104-113 with
// M <= 8): y[m][n] = act(fl(float(sum_k x[m][k] w[n][k]) * cs) + b[n]).
//
// The weights stream through LDS: an item is 16 weight rows x one 512-byte
// K piece (8 KiB), copied by 8 global_load_lds instructions of two 512-byte
// row pieces each, so every instruction reads whole 128-byte lines.  Each
// wave owns a three-stage ring and streams its own items (no workgroup
// barrier in the loop): while it consumes item i the copies of items i + 1
// and i + 2 are in flight.  A piece's activations (M <= 8 rows x 512 bytes)
// travel the same way, into the stage of the piece's first item, so no
// register is the target of a load in flight and the waits are exactly the
// counted ones.  v_mfma_i32_16x16x64_i8 takes the weights as A (row n = lane %
// 16) and the activations as B (column m = lane % 16, zero for m >= M), so
// D[n][m] is the exact i32 sum; the activation fragments of a piece (8 K
// steps x 16 bytes per lane) are loaded once per piece and serve every row
// block of the workgroup.
//
// Workgroup g owns row blocks [g NB / G, (g + 1) NB / G) (at most kGmvBlocks)
// and its 4 waves split K into contiguous ranges of pieces; each wave walks
// its pieces, and within a piece the row blocks, keeping one accumulator per
// block.  The waves' partial sums are added in LDS (integer adds: exact in
// any order), and the workgroup applies the epilogue.
//
// LDS swizzle: row r's 16-byte chunk c lands at position c ^ r (the DMA lane
// that writes position i fetches chunk i ^ r), so the 16 rows of a fragment
// read hit 16 different bank groups.
namespace gmv {
constexpr int kWaves = 4;
constexpr int kPiece = 512;                // K bytes per piece
constexpr int kItem = 16 * kPiece;         // 16 rows x one piece
constexpr int kDma = kItem / 1024;         // copy instructions per item
constexpr int kSteps = kPiece / 64;        // MFMA K steps per piece
constexpr int kXBytes = 8 * kPiece;             // a piece's activations, 8 rows
constexpr int kXDma = kXBytes / 1024;           // their copy instructions
constexpr int kStage = kItem + kXBytes;         // 12 KiB
constexpr int kStages = 3;
constexpr int kRing = kWaves * kStages * kStage;  // 144 KiB
constexpr int kRedWords = kGmvBlocks * 16 * 8;
constexpr int kLds = kRing + kRedWords * 4;
// Past half of the CU's 160 KiB, so the grid spreads one workgroup per CU.
static_assert(kLds > 80 * 1024 && kLds <= 160 * 1024, "LDS plan");
}  // namespace gmv

__global__ __launch_bounds__(256) void gemv_mfma_kernel(const int8_t* __restrict__ A, const int8_t* __restrict__ B,
                                                        int M, int64_t N, int NB, int Kpad, Epilogue ep) {
  using namespace gmv;
  __shared__ __attribute__((aligned(1024))) int8_t smem[kLds];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int bb = (int)((int64_t)blockIdx.x * NB / gridDim.x);
  const int nbl = (int)((int64_t)(blockIdx.x + 1) * NB / gridDim.x) - bb;
  const int KP = Kpad / kPiece;
  const int p0 = wave * KP / kWaves, p1 = (wave + 1) * KP / kWaves;
  const int nitems = (p1 - p0) * nbl;
  int32_t* red = reinterpret_cast<int32_t*>(smem + kRing);  // [block][row][m]
  for (int i = threadIdx.x; i < kRedWords; i += 256) red[i] = 0;
  __syncthreads();

  int8_t* const ring = smem + wave * kStages * kStage;
  const int8_t* const wbase = B + (int64_t)bb * 16 * Kpad;
  const int drow = lane >> 5, dchunk = lane & 31;  // copy: two 512-byte row pieces per instruction
  const int r = lane & 15, q = lane >> 4;          // fragment: row / column r, K quarter q
  v4i xc[kSteps], acc[kGmvBlocks];
#pragma unroll
  for (int b = 0; b < kGmvBlocks; b++) acc[b] = v4i{0, 0, 0, 0};
  // Item (p, b) into stage `stage`: for b == 0 first the piece's activation
  // rows (rows past M repeat row M - 1; their columns are never used), then
  // the weights.  Row rr's chunk c lands at position c ^ rr.
  auto issue = [&](int p, int b, int stage) {
    int8_t* dst = ring + stage * kStage;
    if (b == 0) {
#pragma unroll
      for (int j = 0; j < kXDma; j++) {
        const int rr = 2 * j + drow;
        dma16(A + (int64_t)(rr < M ? rr : M - 1) * Kpad + p * kPiece + ((dchunk ^ rr) << 4),
              dst + kItem + j * 1024);
      }
    }
    const int8_t* src = wbase + (int64_t)b * 16 * Kpad + p * kPiece;
#pragma unroll
    for (int j = 0; j < kDma; j++) {
      const int rr = 2 * j + drow;
      dma16(src + (int64_t)rr * Kpad + ((dchunk ^ rr) << 4), dst + j * 1024);
    }
  };
  // Item k is (piece p0 + k / nbl, row block k % nbl) in stage k % kStages;
  // two items are in flight ahead of the one consumed.
  const int dist = 2;
  int issued = 0, ip = p0, ib = 0;  // next item to issue and its (piece, block)
  auto issue_next = [&]() {
    issue(ip, ib, issued % kStages);
    issued++;
    if (++ib == nbl) {
      ib = 0;
      ip++;
    }
  };
  while (issued < dist && issued < nitems) issue_next();
  int i = 0;
  for (int p = p0; p < p1; p++) {
#pragma unroll
    for (int b = 0; b < kGmvBlocks; b++) {
      if (b < nbl) {
        // Wait for item i: what was issued after it may stay in flight --
        // item i + 1's weight copies (kDma) and, when that item starts a
        // piece, its activation copies (kXDma).  Loads complete in order.
        if (issued > i + 1) {
          if (b + 1 == nbl)
            wait_vmcnt<kDma + kXDma>();
          else
            wait_vmcnt<kDma>();
        } else {
          wait_vmcnt<0>();
        }
        const int8_t* const sb = ring + (i % kStages) * kStage;
        if (b == 0) {
          // the piece's activation fragments (zero for rows past M)
          const int8_t* const xr = sb + kItem + (r < M ? r : 0) * kPiece;
#pragma unroll
          for (int s = 0; s < kSteps; s++) {
            const v4i v = *reinterpret_cast<const v4i*>(xr + (((4 * s + q) ^ (r < M ? r : 0)) << 4));
            xc[s] = r < M ? v : v4i{0, 0, 0, 0};
          }
        }
        if (issued < nitems) issue_next();
        const int8_t* st = sb + r * kPiece;
#pragma unroll
        for (int s = 0; s < kSteps; s++) {
          const v4i wf = *reinterpret_cast<const v4i*>(st + (((4 * s + q) ^ r) << 4));
          acc[b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wf, xc[s], acc[b], 0, 0, 0);
        }
        // this stage's reads are done before a later copy refills it
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        i++;
      }
    }
  }
  // lane l holds D[4 q + e][r]: rows 4q..4q+3 of each block, column r
  if (r < M) {
#pragma unroll
    for (int b = 0; b < kGmvBlocks; b++)
      if (b < nbl) {
#pragma unroll
        for (int e = 0; e < 4; e++) atomicAdd(&red[(b * 16 + 4 * q + e) * 8 + r], acc[b][e]);
      }
  }
  __syncthreads();

  const float cs = tensor_scale(ep.absmax_in) * ep.w_scale;
  const int rows = nbl * 16;
  uint32_t amax = 0;
  for (int idx = threadIdx.x; idx < rows * M; idx += 256) {
    const int m = idx / rows, nl = idx - m * rows;
    const int64_t col = (int64_t)bb * 16 + nl;
    if (col < N) {
      const int32_t sum = red[nl * 8 + m];
      const float prod = (float)sum * cs;
      const float pre = prod + ep.bias[col];
      float v;
      switch (ep.act) {
        case rgmath::ACT_RELU: v = act_fixed<rgmath::ACT_RELU>(pre, ep.act_param); break;
        case rgmath::ACT_SIGMOID: v = act_fixed<rgmath::ACT_SIGMOID>(pre, ep.act_param); break;
        case rgmath::ACT_TANH: v = act_fixed<rgmath::ACT_TANH>(pre, ep.act_param); break;
        case rgmath::ACT_GELU: v = act_fixed<rgmath::ACT_GELU>(pre, ep.act_param); break;
        case rgmath::ACT_LEAKY_RELU: v = act_fixed<rgmath::ACT_LEAKY_RELU>(pre, ep.act_param); break;
        case rgmath::ACT_SILU: v = act_fixed<rgmath::ACT_SILU>(pre, ep.act_param); break;
        default: v = pre; break;
      }
      ep.y[m * N + col] = v;
      if (ep.acc_out) ep.acc_out[m * N + col] = sum;
      const uint32_t key = rgmath::absmax_key(v);
      amax = key > amax ? key : amax;
    }
  }
  if (ep.absmax_out) {
    amax = wave_max_u32(amax);
    if (lane == 0) spread_max(ep.absmax_out, amax);
  }
}

bool gemv_mfma_supported(int64_t M, int64_t Npad, int64_t Kpad) {
  // Row counts and shapes where the matrix-core form beats the dot4 form:
  // enough row blocks for every CU and whole 512-byte K pieces, at least
  // one per wave.
  return M >= kGmvMinRows && M <= 8 && Kpad % gmv::kPiece == 0 && Kpad >= gmv::kWaves * gmv::kPiece &&
         Kpad <= INT32_MAX && Npad / 16 >= 256;
}

static void launch_gemv_mfma(const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t Npad, int64_t Kpad,
                             const Epilogue& ep, hipStream_t s) {
  const void* fn = reinterpret_cast<const void*>(&gemv_mfma_kernel);
  static const int64_t cap = resident_blocks(fn);
  const int64_t NB = Npad / 16;
  int64_t grid = cap < NB ? cap : NB;
  const int64_t need = (NB + kGmvBlocks - 1) / kGmvBlocks;  // at most kGmvBlocks blocks per workgroup
  if (grid < need) grid = need;
  RG_LAUNCH(gemv_mfma_kernel, dim3((unsigned)grid), dim3(256), 0, s, A, B, (int)M, N, (int)NB, (int)Kpad, ep);
}

// Linear with at most 16 outputs per row (the classifier heads: D's
// 1024 -> 10, C's 256 -> 10, Q's 32 -> 3).  A 128 x 128 MFMA tile would waste
// most of its columns, so a wave takes one row at a time instead: lane l
// holds 16 bytes of every 1 KiB K chunk of the row and of the N weight rows
// (those are a few KiB and stay in L1), sums them (INT8: sdot4, exact; FP16:
// fdot2, FP32: FMA, in gemv_kernel's order), and the wave's N sums are
// reduce-scattered as in gemv_kernel before the fused epilogue.  Kpad is in
// bytes.  With XQ (INT8) A is the f32 input [M, xk] (xk % 4 == 0, 16-byte
// aligned rows), quantized as it is read (QuantTensor::from_f32 with the
// spread slot's scale, quantize.rs:18-24): each value is read once, so the
// separate quantize pass over it is gone; q_out (capture) receives the i8
// operand [M, Kpad] and scale_out the scale.
template <int NN, int MODE, bool XQ = false>
__global__ __launch_bounds__(256) void gemm_narrow_kernel(const int8_t* __restrict__ A, const int8_t* __restrict__ B,
                                                          int64_t M, int64_t N, int64_t Kpad, Epilogue ep, int64_t xk,
                                                          int8_t* q_out, float* scale_out) {
  constexpr int S = pow2_at_least(NN);
  constexpr int SPREAD = 64 / S;
  const int lane = threadIdx.x & 63;
  float cs = 1.0f, inv = 0.0f;
  if constexpr (MODE == kModeI8) {
    const float sa = tensor_scale(ep.absmax_in);
    cs = sa * ep.w_scale;
    inv = 1.0f / sa;
    if (XQ && scale_out && blockIdx.x == 0 && threadIdx.x == 0) *scale_out = sa;
  }
  const int sidx = lane / SPREAD;
  const bool owner = (lane % SPREAD) == 0 && sidx < N;
  const float bias_v = ep.bias[sidx < N ? sidx : N - 1];
  const int64_t ntrip = (Kpad + 1023) / 1024;
  const int64_t klast = Kpad - 16;
  uint32_t amax = 0;
  for (int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); row < M; row += (int64_t)gridDim.x * 4) {
    int32_t acc[S];
#pragma unroll
    for (int i = 0; i < S; i++) acc[i] = 0;
    for (int64_t t = 0; t < ntrip; t++) {
      const int64_t k = t * 1024 + lane * 16;
      const bool ok = k < Kpad;
      const int64_t kk = ok ? k : klast;
      v4i av;
      if constexpr (XQ) {
        // 16 inputs of the row from k on: zeros past its xk values
        const float* xr = reinterpret_cast<const float*>(A) + row * xk;
        v4f f[4];
#pragma unroll
        for (int g = 0; g < 4; g++)
          f[g] = k + 4 * g < xk ? *reinterpret_cast<const v4f*>(xr + k + 4 * g) : v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int g = 0; g < 4; g++) {
          const uint32_t b0 = (uint32_t)rgmath::quantize_rz_bounded(f[g][0] * inv) & 0xffu;
          const uint32_t b1 = (uint32_t)rgmath::quantize_rz_bounded(f[g][1] * inv) & 0xffu;
          const uint32_t b2 = (uint32_t)rgmath::quantize_rz_bounded(f[g][2] * inv) & 0xffu;
          const uint32_t b3 = (uint32_t)rgmath::quantize_rz_bounded(f[g][3] * inv) & 0xffu;
          av[g] = (int32_t)(b0 | (b1 << 8) | (b2 << 16) | (b3 << 24));
        }
        if (q_out && ok) *reinterpret_cast<v4i*>(q_out + row * Kpad + k) = av;
      } else {
        const v4i al = *reinterpret_cast<const v4i*>(A + row * Kpad + kk);
        av = ok ? al : v4i{0, 0, 0, 0};
      }
#pragma unroll
      for (int n = 0; n < NN; n++) {
        const v4i w = *reinterpret_cast<const v4i*>(B + (int64_t)n * Kpad + kk);
        int32_t c = acc[n];
        if constexpr (MODE == kModeF32) {
          const v4f xf = __builtin_bit_cast(v4f, av), wf = __builtin_bit_cast(v4f, w);
          float f = __int_as_float(c);
#pragma unroll
          for (int q = 0; q < 4; q++) f = __builtin_fmaf(xf[q], wf[q], f);
          c = __float_as_int(f);
        } else if constexpr (MODE == kModeF16) {
          const v8h xh = __builtin_bit_cast(v8h, av), wh = __builtin_bit_cast(v8h, w);
          float f = __int_as_float(c);
#pragma unroll
          for (int q = 0; q < 4; q++)
            f = __builtin_amdgcn_fdot2(v2h{xh[2 * q], xh[2 * q + 1]}, v2h{wh[2 * q], wh[2 * q + 1]}, f, false);
          c = __float_as_int(f);
        } else {
          c = __builtin_amdgcn_sdot4(av[0], w[0], c, false);
          c = __builtin_amdgcn_sdot4(av[1], w[1], c, false);
          c = __builtin_amdgcn_sdot4(av[2], w[2], c, false);
          c = __builtin_amdgcn_sdot4(av[3], w[3], c, false);
        }
        acc[n] = c;
      }
    }
    const int32_t mine = wave_reduce_scatter<S, MODE != kModeI8>(acc, lane);
    float pre;
    if constexpr (MODE == kModeF16) {
      pre = rgmath::round_fp16(__int_as_float(mine) + bias_v);
    } else if constexpr (MODE == kModeF32) {
      pre = __int_as_float(mine) + bias_v;
    } else {
      const float prod = (float)mine * cs;
      pre = prod + bias_v;
    }
    if (owner) {
      float v;
      switch (ep.act) {
        case rgmath::ACT_RELU: v = act_fixed<rgmath::ACT_RELU>(pre, ep.act_param); break;
        case rgmath::ACT_SIGMOID: v = act_fixed<rgmath::ACT_SIGMOID>(pre, ep.act_param); break;
        case rgmath::ACT_TANH: v = act_fixed<rgmath::ACT_TANH>(pre, ep.act_param); break;
        case rgmath::ACT_GELU: v = act_fixed<rgmath::ACT_GELU>(pre, ep.act_param); break;
        case rgmath::ACT_LEAKY_RELU: v = act_fixed<rgmath::ACT_LEAKY_RELU>(pre, ep.act_param); break;
        case rgmath::ACT_SILU: v = act_fixed<rgmath::ACT_SILU>(pre, ep.act_param); break;
        default: v = pre; break;
      }
      ep.y[row * N + sidx] = v;
      if (ep.acc_out) ep.acc_out[row * N + sidx] = mine;
      const uint32_t key = rgmath::absmax_key(v);
      amax = key > amax ? key : amax;
    }
  }
  if (ep.absmax_out) {
    amax = wave_max_u32(amax);
    if (lane == 0) spread_max(ep.absmax_out, amax);
  }
}

template <int MODE, bool XQ = false>
static void launch_gemm_narrow_t(const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t Kpad_bytes,
                                 const Epilogue& ep, hipStream_t s, int64_t xk = 0, int8_t* q_out = nullptr,
                                 float* scale_out = nullptr) {
  if (N <= 0 || N > kNarrowMaxN || Kpad_bytes % 16 || Kpad_bytes <= 0)
    throw std::logic_error("narrow GEMM: N must be 1..16 and K padded to 16 bytes");
  if (M <= 0) return;
  const int64_t blocks = std::min<int64_t>((M + 3) / 4, 8192);
  if (N <= 4)
    RG_LAUNCH((gemm_narrow_kernel<4, MODE, XQ>), dim3((unsigned)blocks), dim3(256), 0, s, A, B, M, N, Kpad_bytes, ep,
              xk, q_out, scale_out);
  else if (N <= 8)
    RG_LAUNCH((gemm_narrow_kernel<8, MODE, XQ>), dim3((unsigned)blocks), dim3(256), 0, s, A, B, M, N, Kpad_bytes, ep,
              xk, q_out, scale_out);
  else if (N <= 12)  // the 10-class heads: 12 weight rows per lane instead of 16
    RG_LAUNCH((gemm_narrow_kernel<12, MODE, XQ>), dim3((unsigned)blocks), dim3(256), 0, s, A, B, M, N, Kpad_bytes,
              ep, xk, q_out, scale_out);
  else
    RG_LAUNCH((gemm_narrow_kernel<16, MODE, XQ>), dim3((unsigned)blocks), dim3(256), 0, s, A, B, M, N, Kpad_bytes, ep,
              xk, q_out, scale_out);
}

void launch_gemm_narrow(const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t Kpad, const Epilogue& ep,
                        hipStream_t s) {
  launch_gemm_narrow_t<kModeI8>(A, B, M, N, Kpad, ep, s);
}

bool gemm_narrow_xq_supported(int64_t K, int64_t Kpad) { return K > 0 && K % 4 == 0 && K <= Kpad && Kpad % 16 == 0; }

void launch_gemm_narrow_xq(const float* x, const int8_t* B, int64_t M, int64_t N, int64_t K, int64_t Kpad,
                           const Epilogue& ep, int8_t* q_out, float* scale_out, hipStream_t s) {
  if (!gemm_narrow_xq_supported(K, Kpad) || (reinterpret_cast<uintptr_t>(x) & 15) || !ep.absmax_in)
    throw std::logic_error("narrow GEMM: the quantizing form needs K % 4 == 0, an aligned input and a slot");
  launch_gemm_narrow_t<kModeI8, true>(reinterpret_cast<const int8_t*>(x), B, M, N, Kpad, ep, s, K, q_out, scale_out);
}

// ---------------------------------------------------------------------------
// INT8 Linear with few output tiles (C's 4096 -> 256 on 256 images): instead
// of quantizing the input in a pass of its own, running a few 128 x 128 tiles
// (K split over more workgroups, the slices added by another kernel), one
// workgroup of 16 waves owns a 16 x TN output block (TN 16 or 64) and a
// slice of K (usually all of it).
//  * Its waves take the slice's K steps of 64, one per wave at a time.  A
//    lane's operand is 16 f32 inputs of row l % 16, columns 16 g + 4 (l / 16)
//    of the step (g = 0..3), quantized as quant_rows_kernel does
//    (QuantTensor::from_f32 with the producer's absmax, quantize.rs:18-24;
//    quantize_rz_bounded, since the scale comes from the absmax of these
//    very values); a 4 x 4 transpose over the lane quads (v_permlane32_swap,
//    v_permlane16_swap) then gives lane l the K bytes [16 (l / 16), +16) of
//    its row, the v_mfma_i32_16x16x64_i8 operand layout, in which the
//    weight rows are read directly.
//  * Slices of 16 or more steps go through LDS in chunks of 16 steps copied
//    by buffer loads with the LDS as destination, each instruction one
//    contiguous KiB of a row; shorter slices load the fragments straight
//    into registers.  The loads are issued before the scale is folded from
//    its slot, so the two round trips overlap.
//  * The waves' exact i32 sums are added in LDS (integer addition: any
//    order gives the same sum), one output per thread.
//  * With one slice the thread applies the fused epilogue of the large GEMM
//    (quantize.rs:104-113), stores y and raises the next op's absmax.  With
//    S slices (few blocks and a long K) each thread adds its sum to its
//    output's 64-bit word in acc64 (zero at the start of the run) with one
//    device-scope atomic that returns the word's old value: the word's high
//    bits count the slices added, its low 40 bits the sums plus 2^31 each
//    (every term in [0, 2^32), so S <= 16 of them cannot carry into the
//    count), and the thread whose slice completes the count applies the
//    epilogue to the full sum.  No workgroup waits for another, and the
//    slices' sums meet in one atomic round trip, with no fence (on this GPU
//    an agent-scope fence writes back or invalidates the XCD's whole L2).
// Inputs past K and rows past M read zeros (buffer loads with the input's
// extent as their limit).  Workgroups are numbered so that the 8 XCDs each
// take a contiguous run of (slice, block) pairs: the blocks of one row strip
// and slice, which read the same inputs, share an XCD's L2.
// ---------------------------------------------------------------------------
namespace xqs {
constexpr int kWaves = 16, kThreads = kWaves * 64, kTM = 16;
constexpr int kMaxBlocks = 512, kTargetGrid = 256, kMaxSlices = 16;
// LDS staging: a chunk of kChunk K steps (1 KiB of weights per row, 4 KiB of
// f32 inputs per row), rows padded by 16 bytes so that the 16 rows of a
// fragment read fall in different banks
constexpr int kChunk = 16, kALd = kChunk * 64 * 4 + 16, kBLd = kChunk * 64 + 16;
constexpr int kStageBytes = kTM * kALd + 64 * kBLd;
}  // namespace xqs

// Dword g of lane quad q (lanes 16 q .. 16 q + 15) <-> dword q of lane quad g.
__device__ __forceinline__ void quad_transpose(v4i& d) {
  const auto a = __builtin_amdgcn_permlane32_swap((uint32_t)d[0], (uint32_t)d[2], false, false);
  const auto b = __builtin_amdgcn_permlane32_swap((uint32_t)d[1], (uint32_t)d[3], false, false);
  const auto c = __builtin_amdgcn_permlane16_swap(a[0], b[0], false, false);
  const auto e = __builtin_amdgcn_permlane16_swap(a[1], b[1], false, false);
  d = v4i{(int32_t)c[0], (int32_t)c[1], (int32_t)e[0], (int32_t)e[1]};
}

template <int TN>
__global__ __launch_bounds__(xqs::kThreads) void gemm_xq_small_kernel(
    const float* __restrict__ x, const int8_t* __restrict__ B, int M, int N, int xk, int Kpad, int tiles_m,
    int tiles_n, int ks, Epilogue ep, uint64_t* __restrict__ acc64) {
  using namespace xqs;
  constexpr int NB = TN / 16, LD = TN + 4, OUT = kTM * TN;  // LD: the 4 lane quads' rows in different banks
  static_assert(OUT <= kThreads, "one output per thread");
  static_assert(kWaves * kTM * LD * 4 <= kStageBytes, "the wave sums reuse the staging area");
  __shared__ __attribute__((aligned(16))) int8_t smem[kStageBytes];
  int8_t* const sa = smem;                  // [16 rows][kALd]: f32 inputs of a chunk
  int8_t* const sb = smem + kTM * kALd;     // [TN rows][kBLd]: weight bytes of a chunk
  int32_t* const red = reinterpret_cast<int32_t*>(smem);
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = (int)gridDim.x, tiles = tiles_m * tiles_n, S = G / tiles;
  int t = (int)blockIdx.x;
  if ((G & 7) == 0) t = (t & 7) * (G >> 3) + (t >> 3);
  const int z = t / tiles, tile = t - z * tiles;
  const int tm = tile / tiles_n, tn = tile - tm * tiles_n;
  const int m0 = tm * kTM, n0 = tn * TN;
  const int rows = min(kTM, M - m0);
  const uint32_t part = tensor_absmax_part(ep.absmax_in);
  const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(x + (int64_t)m0 * xk), 0, (int)((uint32_t)(rows * xk) * 4u), 0x00020000);
  const __amdgpu_buffer_rsrc_t rb =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(B + (int64_t)n0 * Kpad), 0, TN * Kpad, 0x00020000);
  const int r = lane & 15, q = lane >> 4;
  const int nk = Kpad / 64, kb = z * ks, ke = min(nk, kb + ks);
  v4i acc[NB];
#pragma unroll
  for (int j = 0; j < NB; j++) acc[j] = v4i{0, 0, 0, 0};
  // A lane's 16 inputs of a K step (row l % 16, columns 16 g + 4 (l / 16) of
  // the step, g = 0..3), quantized (quant_rows_kernel's rule with the
  // producer's scale) and transposed over the lane quads into the MFMA
  // operand layout.
  auto quantize_frag = [&](const v4f (&f)[4], float inv) {
    v4i av;
#pragma unroll
    for (int g = 0; g < 4; g++) {
      const uint32_t b0 = (uint32_t)rgmath::quantize_rz_bounded(f[g][0] * inv);
      const uint32_t b1 = (uint32_t)rgmath::quantize_rz_bounded(f[g][1] * inv);
      const uint32_t b2 = (uint32_t)rgmath::quantize_rz_bounded(f[g][2] * inv);
      const uint32_t b3 = (uint32_t)rgmath::quantize_rz_bounded(f[g][3] * inv);
      const uint32_t lo = __builtin_amdgcn_perm(b1, b0, 0x0c0c0400u), hi = __builtin_amdgcn_perm(b3, b2, 0x0c0c0400u);
      av[g] = (int32_t)__builtin_amdgcn_perm(hi, lo, 0x05040100u);
    }
    quad_transpose(av);
    return av;
  };
  float sa_scale;
  if (ke - kb < kChunk) {
    // A slice of fewer than kChunk steps (at most one per wave): each lane
    // loads its fragments straight into registers -- four 16-byte loads of
    // its inputs, one 16-byte load per weight row block -- all issued before
    // the scale is folded.
    const int s = kb + wave;
    v4f f[4];
    v4i bfr[NB];
    if (s < ke) {
      const uint32_t aoff = (uint32_t)(r * xk) * 4u + (uint32_t)q * 16u;
#pragma unroll
      for (int g = 0; g < 4; g++)
        f[g] = __builtin_bit_cast(
            v4f, __builtin_amdgcn_raw_buffer_load_b128(
                     ra, (int)(s * 64 + 16 * g + 4 * q < xk ? aoff + (uint32_t)(s * 64 + 16 * g) * 4u : kDropOffset), 0,
                     0));
#pragma unroll
      for (int j = 0; j < NB; j++)
        bfr[j] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(
                                             rb, (int)((uint32_t)((j * 16 + r) * Kpad + s * 64 + 16 * q)), 0, 0));
    }
    sa_scale = rgmath::scale_from_absmax(rgmath::bitsf(wave_max_u32(part)));
    if (s < ke) {
      const v4i av = quantize_frag(f, 1.0f / sa_scale);
#pragma unroll
      for (int j = 0; j < NB; j++) acc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bfr[j], acc[j], 0, 0, 0);
    }
  } else {
    // Chunks of kChunk K steps through LDS.  The copies are buffer loads
    // with the LDS as their destination, 1 KiB per instruction (64 lanes x
    // 16 bytes): wave w copies input row w (up to four 1 KiB quarters of 256
    // floats, the ones the slice reaches; floats past K get an offset past
    // the buffer, so they land as zeros, as do rows past M) and weight rows
    // w, w + 16, ... (1 KiB each).  Every instruction reads one contiguous
    // KiB, where register loads of the fragments read 64 bytes of each of 16
    // rows (C's fc layer: 9.1 -> 8.0 us).
    float inv = 0.0f;
    sa_scale = 0.0f;
    for (int c0 = kb; c0 < ke; c0 += kChunk) {
      const int kf0 = c0 * 64;  // first input column of the chunk
#pragma unroll
      for (int u = 0; u < 4; u++) {
        if (kf0 + u * 256 >= ke * 64) break;  // past the slice
        const int k = kf0 + u * 256 + lane * 4;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            ra, (RG_LDS_AS void*)(sa + wave * kALd + u * 1024), 16,
            (int)(k < xk ? (uint32_t)(wave * xk + k) * 4u : kDropOffset), 0, 0, 0);
      }
#pragma unroll
      for (int u = 0; u < TN / kWaves; u++) {
        const int row = wave + u * kWaves;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (RG_LDS_AS void*)(sb + row * kBLd), 16,
                                                 (int)((uint32_t)(row * Kpad + kf0 + lane * 16)), 0, 0, 0);
      }
      if (c0 == kb) {  // the scale, folded while the first chunk is in flight
        sa_scale = rgmath::scale_from_absmax(rgmath::bitsf(wave_max_u32(part)));
        inv = 1.0f / sa_scale;
      }
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      const int s = c0 + wave;  // this wave's K step of the chunk
      if (s < ke) {
        const int ko = (s - c0) * 64;  // its first column within the chunk
        v4f f[4];
#pragma unroll
        for (int g = 0; g < 4; g++) f[g] = *reinterpret_cast<const v4f*>(sa + r * kALd + (ko + 16 * g + 4 * q) * 4);
        const v4i av = quantize_frag(f, inv);
#pragma unroll
        for (int j = 0; j < NB; j++) {
          const v4i bf = *reinterpret_cast<const v4i*>(sb + (j * 16 + r) * kBLd + ko + 16 * q);
          acc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bf, acc[j], 0, 0, 0);
        }
      }
      __syncthreads();  // the chunk's reads are done before the next copies (or the sums) overwrite it
    }
  }
  // result register i of lane l: D[4 (l / 16) + i][l % 16] of block j
#pragma unroll
  for (int j = 0; j < NB; j++)
#pragma unroll
    for (int i = 0; i < 4; i++) red[wave * (kTM * LD) + (4 * q + i) * LD + j * 16 + r] = acc[j][i];
  __syncthreads();
  const float sa_s = sa_scale;
  const int orow = tid / TN, ocol = tid % TN;
  const bool mine = tid < OUT;
  int32_t sum = 0;
  if (mine) {
#pragma unroll
    for (int w = 0; w < kWaves; w++) sum += red[w * (kTM * LD) + orow * LD + ocol];
  }
  bool done = mine;
  if (S > 1 && mine) {
    constexpr uint64_t kLow = (uint64_t(1) << 40) - 1;
    const uint64_t add = (uint64_t(1) << 40) + (uint64_t)((int64_t)sum + (int64_t(1) << 31));
    const uint64_t old =
        __hip_atomic_fetch_add(acc64 + (int64_t)tile * OUT + tid, add, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    done = (old >> 40) == (uint64_t)(S - 1);
    // the low 32 bits of sum(terms) - S 2^31: the i32 sum, wrapped as i32 accumulation wraps
    sum = (int32_t)(uint32_t)((old & kLow) + (add & kLow) - ((uint64_t)S << 31));
  }
  uint32_t amax = 0;
  const int row = m0 + orow, col = n0 + ocol;
  if (done && row < M && col < N) {
    const float cs = sa_s * ep.w_scale, b = ep.bias[col];
    float v;
    switch (ep.act) {
      case rgmath::ACT_RELU: v = epi_value<rgmath::ACT_RELU>(sum, cs, b, ep.act_param); break;
      case rgmath::ACT_SIGMOID: v = epi_value<rgmath::ACT_SIGMOID>(sum, cs, b, ep.act_param); break;
      case rgmath::ACT_TANH: v = epi_value<rgmath::ACT_TANH>(sum, cs, b, ep.act_param); break;
      case rgmath::ACT_GELU: v = epi_value<rgmath::ACT_GELU>(sum, cs, b, ep.act_param); break;
      case rgmath::ACT_LEAKY_RELU: v = epi_value<rgmath::ACT_LEAKY_RELU>(sum, cs, b, ep.act_param); break;
      case rgmath::ACT_SILU: v = epi_value<rgmath::ACT_SILU>(sum, cs, b, ep.act_param); break;
      default: v = epi_value<rgmath::ACT_NONE>(sum, cs, b, ep.act_param); break;
    }
    ep.y[(int64_t)row * N + col] = v;
    amax = rgmath::absmax_key(v);
  }
  if (ep.absmax_out) {
    amax = wave_max_u32(amax);
    if (lane == 0) spread_max(ep.absmax_out, amax);
  }
}

// Block width (16 or 64), blocks and K slices: a workgroup's loads are
// bound by the latency of its CU's outstanding misses, so the choice
// minimises the bytes one CU loads -- per workgroup the slice's K steps times
// 64 bytes times (16 rows x 4 bytes of input + TN weight rows), times the
// workgroups per CU -- plus a charge for the slices' atomic round trip.  At
// most kMaxSlices slices and kMaxBlocks blocks.  RGNPU_XQS_TN (16 or 64) and
// RGNPU_XQS_SLICES (a power of two) force a geometry (measurement aids).
struct XqsGeom {
  int TN, tiles_m, tiles_n, S, ks;
};
static XqsGeom xqs_geom(int64_t M, int64_t Npad, int64_t Kpad) {
  const int tiles_m = (int)((M + xqs::kTM - 1) / xqs::kTM), nk = (int)(Kpad / 64);
  int force_tn = 0, force_s = 0;
  if (const char* e = getenv("RGNPU_XQS_TN")) force_tn = atoi(e);
  if (const char* e = getenv("RGNPU_XQS_SLICES")) force_s = atoi(e);
  XqsGeom best{0, tiles_m, 0, 0, 0};
  double best_cost = 0.0;
  for (int TN : {16, 64}) {
    if ((force_tn == 16 || force_tn == 64) && TN != force_tn) continue;
    const int tiles_n = (int)(Npad / TN);
    const int64_t tiles = (int64_t)tiles_m * tiles_n;
    if (tiles > xqs::kMaxBlocks) continue;
    for (int S = 1; S <= xqs::kMaxSlices; S *= 2) {
      if (force_s > 0 && S != std::min(force_s, xqs::kMaxSlices)) continue;
      const int ks = (nk + S - 1) / S, Se = (nk + ks - 1) / ks;
      if (Se != S && S > 1) continue;  // fewer K steps than slices
      const int64_t wgs = tiles * S, per_cu = (wgs + xqs::kTargetGrid - 1) / xqs::kTargetGrid;
      const double cost = (double)per_cu * ks * 64.0 * (xqs::kTM * 4 + TN) + (S > 1 ? 32768.0 + 4096.0 * S : 0.0);
      if (best.TN == 0 || cost < best_cost) {
        best = XqsGeom{TN, tiles_m, tiles_n, S, ks};
        best_cost = cost;
      }
    }
  }
  if (best.TN == 0) best = XqsGeom{64, tiles_m, (int)(Npad / 64), 1, nk};
  return best;
}

bool gemm_xq_small_supported(int64_t M, int64_t N, int64_t Npad, int64_t K, int64_t Kpad) {
  if (!(M > 0 && M < (int64_t(1) << 30) && N > 0 && N <= Npad && Npad % 64 == 0 && K > 0 && K % 4 == 0 &&
        K <= Kpad && Kpad % 64 == 0 && Kpad * 64 < (int64_t(1) << 31) && K * xqs::kTM * 4 < (int64_t(1) << 31)))
    return false;
  const XqsGeom g = xqs_geom(M, Npad, Kpad);
  return (int64_t)g.tiles_m * g.tiles_n <= xqs::kMaxBlocks;
}

int64_t gemm_xq_small_sync_words(int64_t M, int64_t Npad, int64_t Kpad) {
  const XqsGeom g = xqs_geom(M, Npad, Kpad);
  return g.S > 1 ? (int64_t)g.tiles_m * g.tiles_n * xqs::kTM * g.TN * 2 : 0;
}

void launch_gemm_xq_small(const float* x, const int8_t* B, int64_t M, int64_t N, int64_t Npad, int64_t K,
                          int64_t Kpad, const Epilogue& ep, uint32_t* sync, hipStream_t s) {
  if (!gemm_xq_small_supported(M, N, Npad, K, Kpad) || (reinterpret_cast<uintptr_t>(x) & 15) || !ep.absmax_in ||
      ep.acc_out || ep.h_out || ep.pool2)
    throw std::logic_error("small GEMM: unsupported shape, unaligned input, no slot or capture outputs");
  const XqsGeom g = xqs_geom(M, Npad, Kpad);
  if (g.S > 1 && (!sync || (reinterpret_cast<uintptr_t>(sync) & 7)))
    throw std::logic_error("small GEMM: K slices need zeroed, 8-byte aligned sum words");
  uint64_t* const acc64 = reinterpret_cast<uint64_t*>(sync);
  const dim3 grid((unsigned)(g.S * g.tiles_m * g.tiles_n));
  if (g.TN == 16)
    RG_LAUNCH((gemm_xq_small_kernel<16>), grid, dim3(xqs::kThreads), 0, s, x, B, (int)M, (int)N, (int)K,
              (int)Kpad, g.tiles_m, g.tiles_n, g.ks, ep, acc64);
  else
    RG_LAUNCH((gemm_xq_small_kernel<64>), grid, dim3(xqs::kThreads), 0, s, x, B, (int)M, (int)N, (int)K,
              (int)Kpad, g.tiles_m, g.tiles_n, g.ks, ep, acc64);
}

// ---------------------------------------------------------------------------
// A whole program of small INT8 Linears in one workgroup (npu.rs:307-318 op
// after op).  The input, every layer's weights and biases are copied into LDS
// by global_load_lds (every copy in flight at once, one memory round trip).
// Each layer then
//  * folds its input's absmax with absmax_key (NaN ignored, as absmax_kernel
//    and the producing epilogues do) and takes scale_from_absmax of it
//    (quantize.rs:19-21);
//  * quantizes the input with quantize_one into an i8 operand [rows, Kpad]
//    with zero padding, the rule of quant_rows_kernel (quantize.rs:22);
//  * forms each exact i32 sum with v_dot4_i32_i8 and applies the fused
//    epilogue epi_value, fl(fl(float(acc) * fl(scale * w_scale)) + b) and the
//    activation (quantize.rs:104-113), into the other activation buffer or,
//    for the last layer, into y.
// The arithmetic is that of the per-op kernels, so the output is the same bit
// for bit; what goes is the launches between the ops, which are most of the
// time of a program this small.
// ---------------------------------------------------------------------------
namespace tiny {
constexpr int kThreads = 1024;  // 4 waves per SIMD of the one CU: they hide each other's LDS latency
// LDS row strides: f32 activations odd (a wave's lanes store one column of
// consecutive rows without bank conflicts), the i8 operand 16 bytes past
// Kpad (16 consecutive rows start in 16 different 4-bank groups)
constexpr int kActLd = kTinyWidth + 1;
constexpr int kActWords = kTinyRows * kActLd;
constexpr int kQaLd = kTinyWidth + 16;
constexpr int kBiasWords = kTinyMaxLayers * kTinyWidth;
}  // namespace tiny

// One global_load_lds_dword: 4 bytes per lane, lane i lands at lds + 4 i.
__device__ __forceinline__ void dma4(const void* g, void* lds) {
  __builtin_amdgcn_global_load_lds(g, (RG_LDS_AS void*)lds, 4, 0, 0);
}

// Copies n 4-byte words (unit 4) or 16-byte pieces (unit 16) from src to the
// LDS array dst, 64 units per wave instruction; lanes past n copy nothing.
template <int UNIT>
__device__ __forceinline__ void tiny_copy(const void* src, void* dst, int n, int wave, int lane) {
  for (int c = wave; c * 64 < n; c += tiny::kThreads / 64) {
    const int u = c * 64 + lane;
    const char* g = static_cast<const char*>(src) + (int64_t)u * UNIT;
    char* l = static_cast<char*>(dst) + c * 64 * UNIT;
    if (u < n) {
      if constexpr (UNIT == 16)
        dma16(reinterpret_cast<const int8_t*>(g), reinterpret_cast<int8_t*>(l));
      else
        dma4(g, l);
    }
  }
}

// Max over the wave's 64 lanes, in every lane, without LDS: partners l ^ 32
// and l ^ 16 by the gfx950 lane swaps, then l ^ 15, l ^ 7, l ^ 2, l ^ 1 by
// DPP (dpp_partner); those six offsets span all 64 lanes under XOR.
__device__ __forceinline__ uint32_t wave_max_xlane(uint32_t v) {
  {
    const auto p = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    v = p[0] > p[1] ? p[0] : p[1];
  }
  {
    const auto p = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    v = p[0] > p[1] ? p[0] : p[1];
  }
  uint32_t t = (uint32_t)dpp_partner<8>((int32_t)v);
  v = t > v ? t : v;
  t = (uint32_t)dpp_partner<4>((int32_t)v);
  v = t > v ? t : v;
  t = (uint32_t)dpp_partner<2>((int32_t)v);
  v = t > v ? t : v;
  t = (uint32_t)dpp_partner<1>((int32_t)v);
  return t > v ? t : v;
}

// n / d for a divisor d the whole block shares, as a high multiply:
// mag = ceil(2^32 / d) (div_magic), exact whenever n * d < 2^32.
__device__ __forceinline__ uint32_t div_magic(uint32_t d) { return d <= 1 ? 0u : 0xffffffffu / d + 1u; }
__device__ __forceinline__ int udiv(int n, uint32_t mag) { return mag ? (int)__umulhi((uint32_t)n, mag) : n; }

__device__ __forceinline__ float tiny_epi(int32_t acc, float cs, float b, int act, float p) {
  switch (act) {
    case rgmath::ACT_RELU: return epi_value<rgmath::ACT_RELU>(acc, cs, b, p);
    case rgmath::ACT_SIGMOID: return epi_value<rgmath::ACT_SIGMOID>(acc, cs, b, p);
    case rgmath::ACT_TANH: return epi_value<rgmath::ACT_TANH>(acc, cs, b, p);
    case rgmath::ACT_GELU: return epi_value<rgmath::ACT_GELU>(acc, cs, b, p);
    case rgmath::ACT_LEAKY_RELU: return epi_value<rgmath::ACT_LEAKY_RELU>(acc, cs, b, p);
    case rgmath::ACT_SILU: return epi_value<rgmath::ACT_SILU>(acc, cs, b, p);
    default: return epi_value<rgmath::ACT_NONE>(acc, cs, b, p);
  }
}

__global__ __launch_bounds__(tiny::kThreads) void mlp_tiny_kernel(const float* __restrict__ x, float* __restrict__ y,
                                                                  TinyChain ch, SlotClear clear) {
  __shared__ __attribute__((aligned(16))) float act[2][tiny::kActWords];
  __shared__ __attribute__((aligned(16))) float bias[tiny::kBiasWords];
  __shared__ __attribute__((aligned(16))) int8_t wl[kTinyWeightBytes];
  __shared__ __attribute__((aligned(16))) int8_t qa[kTinyRows * tiny::kQaLd];
  __shared__ uint32_t red[tiny::kThreads / 64];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rows = ch.rows;
  // the input lands as it is laid out in memory (row stride in_f)
  tiny_copy<4>(x, act[0], rows * ch.l[0].in_f, wave, lane);
  for (int l = 0, woff = 0; l < ch.n; l++) {
    tiny_copy<16>(ch.l[l].w, wl + woff, ch.l[l].out_f * ch.l[l].kpad / 16, wave, lane);
    tiny_copy<4>(ch.l[l].bias, bias + l * kTinyWidth, ch.l[l].out_f, wave, lane);
    woff += ch.l[l].out_f * ch.l[l].kpad;
  }
  // the other slot set (clear_slots without its block-size read, whose wait
  // would also wait for the copies above)
  for (int64_t i = tid; i < clear.n; i += tiny::kThreads) clear.p[i] = 0u;
  // the i8 operand starts as zeros: each layer then writes only the words
  // that hold its inputs or that an earlier layer left nonzero
  for (int i = tid; i < kTinyRows * tiny::kQaLd / 16; i += tiny::kThreads) reinterpret_cast<v4i*>(qa)[i] = v4i{0, 0, 0, 0};
  wait_vmcnt<0>();
  __syncthreads();
  int cur = 0, ld = ch.l[0].in_f;  // the current activation buffer and its row stride
  int qw = 0;                      // operand words per row that may be nonzero
  const uint32_t rows_mag = div_magic((uint32_t)rows);
  for (int l = 0, woff = 0; l < ch.n; l++) {
    const TinyLayer L = ch.l[l];
    const float* src = act[cur];
    // The input's absmax: the first layer folds its input; a later layer's
    // per-wave partials were left in red by the previous layer's epilogue.
    if (l == 0) {
      uint32_t m0 = 0;
      const uint32_t in_mag = div_magic((uint32_t)L.in_f);
      for (int e = tid; e < rows * L.in_f; e += tiny::kThreads) {
        const int r = udiv(e, in_mag), k = e - r * L.in_f;
        const uint32_t key = rgmath::absmax_key(src[r * ld + k]);
        m0 = key > m0 ? key : m0;
      }
      m0 = wave_max_xlane(m0);
      if (lane == 0) red[wave] = m0;
      __syncthreads();
    }
    uint32_t m = 0;
#pragma unroll
    for (int w = 0; w < tiny::kThreads / 64; w++) m = red[w] > m ? red[w] : m;
    const float scale = rgmath::scale_from_absmax(rgmath::bitsf(m));
    const float inv = 1.0f / scale;
    if (tid == 0 && L.slot) L.slot[0] = m;
    // words [0, kq) hold the inputs (zeros past in_f); words up to the
    // previous layer's kq are rewritten as zeros; the rest are still zero
    const int kq = (L.in_f + 3) / 4, wq = kq > qw ? kq : qw;
    const uint32_t wq_mag = div_magic((uint32_t)wq);
    for (int e = tid; e < rows * wq; e += tiny::kThreads) {
      const int r = udiv(e, wq_mag), w = e - r * wq, k = 4 * w;
      float v[4];
#pragma unroll
      for (int c = 0; c < 4; c++) v[c] = k + c < L.in_f ? src[r * ld + k + c] : 0.0f;
      reinterpret_cast<uint32_t*>(qa + r * tiny::kQaLd)[w] = pack4(v[0], v[1], v[2], v[3], inv);
    }
    qw = kq;
    __syncthreads();
    const int ks = (L.in_f + 15) / 16;  // 16-byte steps that hold inputs; the rest of Kpad is zero
    const float cs = scale * L.w_scale;
    const bool last = l + 1 == ch.n;
    float* const dst = act[cur ^ 1];
    // output-major: a wave's lanes share a weight row (broadcast reads) and
    // take consecutive operand rows
    uint32_t mo = 0;  // absmax of the outputs this thread writes (the next layer's input)
    for (int e = tid; e < rows * L.out_f; e += tiny::kThreads) {
      const int n = udiv(e, rows_mag), r = e - n * rows;
      const v4i* qr = reinterpret_cast<const v4i*>(qa + r * tiny::kQaLd);
      const v4i* wr = reinterpret_cast<const v4i*>(wl + woff + n * kTinyWidth);
      // the steps that hold inputs (the zero ones add nothing to the exact
      // sum); every fragment read is issued before the sums
      v4i a[kTinyWidth / 16], b[kTinyWidth / 16];
#pragma unroll
      for (int k = 0; k < kTinyWidth / 16; k++) {
        if (k < ks) {
          a[k] = qr[k];
          b[k] = wr[k];
        }
      }
      int32_t acc = 0;
#pragma unroll
      for (int k = 0; k < kTinyWidth / 16; k++) {
        if (k < ks) {
          acc = __builtin_amdgcn_sdot4(a[k][0], b[k][0], acc, false);
          acc = __builtin_amdgcn_sdot4(a[k][1], b[k][1], acc, false);
          acc = __builtin_amdgcn_sdot4(a[k][2], b[k][2], acc, false);
          acc = __builtin_amdgcn_sdot4(a[k][3], b[k][3], acc, false);
        }
      }
      const float v = tiny_epi(acc, cs, bias[l * kTinyWidth + n], L.act, L.act_param);
      if (last) {
        y[r * L.out_f + n] = v;
      } else {
        dst[r * tiny::kActLd + n] = v;
        const uint32_t key = rgmath::absmax_key(v);
        mo = key > mo ? key : mo;
      }
    }
    // every thread read red before the barrier after the quantization
    if (!last) {
      mo = wave_max_xlane(mo);
      if (lane == 0) red[wave] = mo;
    }
    woff += L.out_f * L.kpad;
    cur ^= 1;
    ld = tiny::kActLd;
    __syncthreads();
  }
}

void launch_mlp_tiny(const float* x, float* y, const TinyChain& ch, SlotClear clear, hipStream_t s) {
  int wbytes = 0;
  bool ok = ch.n >= 1 && ch.n <= kTinyMaxLayers && ch.rows >= 1 && ch.rows <= kTinyRows;
  for (int l = 0; ok && l < ch.n; l++) {
    const TinyLayer& L = ch.l[l];
    ok = L.in_f >= 1 && L.in_f <= kTinyWidth && L.out_f >= 1 && L.out_f <= kTinyWidth && L.kpad == kTinyWidth &&
         (l == 0 || L.in_f == ch.l[l - 1].out_f) && L.w && L.bias && (reinterpret_cast<uintptr_t>(L.w) & 15) == 0;
    wbytes += L.out_f * L.kpad;
  }
  if (!ok || wbytes > kTinyWeightBytes || (reinterpret_cast<uintptr_t>(x) & 3) || (reinterpret_cast<uintptr_t>(y) & 3))
    throw std::logic_error("mlp_tiny: the chain does not fit the one-workgroup kernel");
  RG_LAUNCH(mlp_tiny_kernel, dim3(1), dim3(tiny::kThreads), 0, s, x, y, ch, clear);
}

void launch_gemm_narrow_f16(const uint16_t* A, const uint16_t* B, int64_t M, int64_t N, int64_t Kpad_h,
                            const Epilogue& ep, hipStream_t s) {
  launch_gemm_narrow_t<kModeF16>(reinterpret_cast<const int8_t*>(A), reinterpret_cast<const int8_t*>(B), M, N,
                                 2 * Kpad_h, ep, s);
}

void launch_gemm_narrow_f32(const float* A, const float* B, int64_t M, int64_t N, int64_t Kpad_f, const Epilogue& ep,
                            hipStream_t s) {
  launch_gemm_narrow_t<kModeF32>(reinterpret_cast<const int8_t*>(A), reinterpret_cast<const int8_t*>(B), M, N,
                                 4 * Kpad_f, ep, s);
}

void launch_gemv(const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t Npad, int64_t Kpad,
                 const Epilogue& ep, hipStream_t s) {
  if (gemv_mfma_supported(M, Npad, Kpad))
    launch_gemv_mfma(A, B, M, N, Npad, Kpad, ep, s);
  else
    launch_gemv_any<kModeI8>(A, B, M, N, Npad, Kpad, ep, s);
}

void launch_gemv_f32(const float* A, const float* B, int64_t M, int64_t N, int64_t Npad, int64_t Kpad_f,
                     const Epilogue& ep, hipStream_t s) {
  launch_gemv_any<kModeF32>(reinterpret_cast<const int8_t*>(A), reinterpret_cast<const int8_t*>(B), M, N, Npad,
                            4 * Kpad_f, ep, s);
}

void launch_gemv_f16(const uint16_t* A, const uint16_t* B, int64_t M, int64_t N, int64_t Npad, int64_t Kpad_h,
                     const Epilogue& ep, hipStream_t s) {
  launch_gemv_any<kModeF16>(reinterpret_cast<const int8_t*>(A), reinterpret_cast<const int8_t*>(B), M, N, Npad,
                            2 * Kpad_h, ep, s);
}

// ---------------------------------------------------------------------------
// Implicit-GEMM conv.  MFMA "A" = weights [Opad, Kpad] (TM output channels,
// tap-major K, see ConvShape), "B" = im2col columns of one image (output
// pixels), so D[o][l] maps onto the NCHW output with pixels contiguous.
//
// Main kernel (conv_band_kernel): block = image b (grid.z) x TM channels
// (grid.y) x TN pixels (grid.x); wave w owns pixels [p0 + w TN/4, +TN/4).
// LDS holds the block's weights (row stride Kpad + 16) and the input rows its
// pixels read, zero padded and channel-last: band[r][x][c], r < R,
// x < W + 2 pad, c < cp.  With XF the input is the f32 image and the band
// is filled with its quantized values (quantize_into's per-image scale,
// quantize.rs:27-35, from the image's absmax slot): a thread quantizes 4
// channels of one pixel and writes them as one 32-bit word, and no i8 image
// exists in memory.  With self_absmax (the run's first conv, an image of at
// most kConvSelfAbsmaxMax floats whose every pixel a window reads) each
// block also measures the absmax of its whole image first, so no absmax
// pass runs before the conv; block (0, 0) of each image publishes it in the
// image's slot (read only after this kernel: the capture tap).  A 16-byte K chunk of an im2col column is then 16
// channels of one tap (cp >= 16: one ds_read_b128) or 4 channels of 4 taps
// (cp == 4: four ds_read_b32); taps past k*k read a zero block.  Outputs are
// stored straight from the accumulators (16 consecutive pixels per store).
// ---------------------------------------------------------------------------
struct ConvBand {
  int rows_max;    // band rows for the worst block
  int lds_bytes;   // dynamic LDS
};

static ConvBand conv_band_geom(const ConvShape& cs, int TM, int TN) {
  const int64_t Wp = cs.W + 2 * cs.pad;
  const int64_t rows = ((TN - 1) / cs.OW + 1) * cs.stride + cs.k;
  const int64_t band = round_up(rows * Wp * cs.cp, 16) + 16;
  const int64_t bytes = (int64_t)TM * (cs.Kpad + 16) + band;
  return ConvBand{(int)rows, bytes > (1 << 30) ? (1 << 30) : (int)bytes};
}


// The block's absmax for the next op: the 4 waves' maxima meet in LDS and
// one atomic per block raises the image's slot (per image) or one partial of
// the spread slot (per tensor), so an image slot takes one atomic per block
// rather than one per wave.  Every thread of the block (NW waves) calls it.
template <int NW = 4>
__device__ __forceinline__ void conv_block_absmax(const Epilogue& ep, int b, uint32_t amax, uint32_t* red, int lane) {
  if (!ep.absmax_out) return;
  amax = wave_max_u32(amax);
  if (lane == 0) red[threadIdx.x >> 6] = amax;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t m = red[0];
#pragma unroll
    for (int w = 1; w < NW; w++) m = red[w] > m ? red[w] : m;
    if (m) {
      if (ep.absmax_out_per_image) {
        atomicMax(ep.absmax_out + b, m);
      } else {
        const uint32_t block = (blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x;
        atomicMax(ep.absmax_out + (block & (kSpread - 1)) * kSpreadStride, m);
      }
    }
  }
}

template <int TM, int TN, bool CP4, int ACT>
__device__ __forceinline__ void conv_band_epilogue(const v4i (&acc)[TM / 16][TN / 64], const ConvShape& cs,
                                                   const Epilogue& ep, int b, int o0, const int (&pix)[TN / 64],
                                                   float csc, int lane, uint32_t* red) {
  constexpr int FM = TM / 16, FN = TN / 64;
  const int O = (int)cs.O, L = (int)(cs.OH * cs.OW);
  // the image's output plane set through a bounded resource: 32-bit offsets
  // o * L + p (host-checked: O * L * 4 < 2^31), invalid ones dropped
  const __amdgpu_buffer_rsrc_t ry = bounded_rsrc(ep.y + (int64_t)b * O * L);
  uint32_t amax = 0;
#pragma unroll
  for (int i = 0; i < FM; i++)
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int o = o0 + i * 16 + (lane >> 4) * 4 + r;
      const float bias = ep.bias[o];  // padded to Opad
      const bool o_ok = o < O;
#pragma unroll
      for (int j = 0; j < FN; j++) {
        const int p = pix[j];
        const bool ok = o_ok && p < L;
        const int32_t a = acc[i][j][r];
        const float v = epi_value<ACT>(a, csc, bias, ep.act_param);
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), ry,
                                              (int)(ok ? (uint32_t)(o * L + p) * 4u : kDropOffset), 0, 0);
        if (ep.acc_out && ok) ep.acc_out[((int64_t)b * L + p) * O + o] = a;
        const uint32_t key = ok ? rgmath::absmax_key(v) : 0u;
        amax = key > amax ? key : amax;
      }
    }
  conv_block_absmax(ep, b, amax, red, lane);
}

// Conv -> MaxPool2d(2, 2) (npu.rs:384-390 on the output of npu.rs:319-383)
// in the conv's epilogue: only the pooled output is stored.  Host-checked
// shape: OH, OW even, OW = 16 R16, and every wave's TN/4 pixels are whole
// pairs of output rows, so fragment j of an even row (j / R16 even) has the
// next row in fragment j + R16 of the same lane and pixel p + 1 in lane ^ 1.
// An even lane takes its window in the reference's order (0,0), (0,1),
// (1,0), (1,1) with pool_take from -inf (maxpool2_kernel's rule), and the
// absmax for the next op is over the pooled values.  LDS: the pooled values
// go to the image's planes lout [O, OH/2, OW/2] in LDS instead, and the
// block's absmax is left to the caller (the lane's key is returned).
// With ReLU the window is pooled on the i32 sums: relu(fl(fl(s * csc) + b))
// is non-decreasing in s for every scale product csc the reference can
// form (positive, +inf, or NaN, where every value is +0), and ReLU leaves
// no NaN and no -0, so the largest value of the window is the value of its
// largest sum, bit for bit, and one epilogue evaluation serves four outputs.

template <int TM, int TN, int ACT, int R16, bool LDS = false, int NW = 4, bool LBIAS = false>
__device__ __forceinline__ uint32_t conv_band_epilogue_pool2(const v4i (&acc)[TM / 16][TN / 64], const ConvShape& cs,
                                                             const Epilogue& ep, int b, int o0,
                                                             const int (&pix)[TN / 64], float csc, int lane,
                                                             uint32_t* red, float* lout = nullptr,
                                                             const float* lbias = nullptr) {
  constexpr int FM = TM / 16, FN = TN / 64;
  static_assert(FN % (2 * R16) == 0, "a wave's pixels are whole pairs of output rows");
  const int O = (int)cs.O;
  const int OW = (int)cs.OW, L = (int)(cs.OH * cs.OW), POW = OW >> 1;
  const int PL = (int)(cs.OH >> 1) * POW;
  const bool even = (lane & 1) == 0;
  // the pooled pixel of each even-row fragment (once per lane), stored
  // through a bounded resource over the image's pooled planes with 32-bit
  // offsets o * PL + pp (host-checked: O * PL * 4 < 2^31)
  const __amdgpu_buffer_rsrc_t ry = bounded_rsrc(LDS ? nullptr : ep.y + (int64_t)b * O * PL);
  // the lane's 4 output channels of each row block (bias padded to Opad;
  // LBIAS: a copy in LDS, staged before the K loop, so no global load sits
  // between the MFMAs and the stores)
  float4 b4[FM];
#pragma unroll
  for (int i = 0; i < FM; i++)
    b4[i] = *reinterpret_cast<const float4*>((LBIAS ? lbias : ep.bias) + o0 + i * 16 + (lane >> 4) * 4);
  int pp[FN];
  const uint32_t owmag = div_magic((uint32_t)OW);
#pragma unroll
  for (int j = 0; j < FN; j++) {
    const int p = pix[j];
    const int oy = udiv(p, owmag), ox = p - oy * OW;
    pp[j] = (even && p < L) ? (oy >> 1) * POW + (ox >> 1) : -1;
  }
  uint32_t amax = 0;
  if constexpr (ACT == rgmath::ACT_RELU) {
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int o = o0 + i * 16 + (lane >> 4) * 4 + r;
        int32_t h[FN];
#pragma unroll
        for (int j = 0; j < FN; j++) h[j] = dpp_partner<1>(acc[i][j][r]);  // lane ^ 1
#pragma unroll
        for (int j = 0; j < FN; j++) {
          if ((j / R16) % 2 != 0) continue;
          const int jn = j + R16 < FN ? j + R16 : j;
          const int32_t mx = max(max(acc[i][j][r], h[j]), max(acc[i][jn][r], h[jn]));
          const float best = epi_value<ACT>(mx, csc, b4[i][r], ep.act_param);
          const bool ok = pp[j] >= 0 && o < O;
          if constexpr (LDS) {
            if (ok) lout[o * PL + pp[j]] = best;
          } else {
            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, best), ry,
                                                  (int)(ok ? (uint32_t)(o * PL + pp[j]) * 4u : kDropOffset), 0, 0);
          }
          const uint32_t key = ok ? rgmath::fbits(best) : 0u;
          amax = key > amax ? key : amax;
        }
      }
    if constexpr (!LDS) conv_block_absmax<NW>(ep, b, amax, red, lane);
    return amax;
  }
#pragma unroll
  for (int i = 0; i < FM; i++)
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int o = o0 + i * 16 + (lane >> 4) * 4 + r;
      const float bias = b4[i][r];  // padded to Opad
      float v[FN], h[FN];
#pragma unroll
      for (int j = 0; j < FN; j++) v[j] = epi_value<ACT>(acc[i][j][r], csc, bias, ep.act_param);
#pragma unroll
      for (int j = 0; j < FN; j++) h[j] = __int_as_float(dpp_partner<1>(__float_as_int(v[j])));  // lane ^ 1
#pragma unroll
      for (int j = 0; j < FN; j++) {
        if ((j / R16) % 2 != 0) continue;
        const int jn = j + R16 < FN ? j + R16 : j;  // j + R16 whenever j's row is even
        float best;
        if constexpr (ACT == rgmath::ACT_RELU) {
          // ReLU leaves no NaN and no -0 (x > 0 ? x : +0), so pool_take's
          // first-maximum rule is the plain maximum of the four values
          best = __builtin_fmaxf(__builtin_fmaxf(v[j], h[j]), __builtin_fmaxf(v[jn], h[jn]));
        } else {
          best = v[j];  // pool_take(-inf, v) == v for every v
          best = pool_take(best, h[j]);
          best = pool_take(best, v[jn]);
          best = pool_take(best, h[jn]);
        }
        const bool ok = pp[j] >= 0 && o < O;
        if constexpr (LDS) {
          if (ok) lout[o * PL + pp[j]] = best;
        } else {
          __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, best), ry,
                                                (int)(ok ? (uint32_t)(o * PL + pp[j]) * 4u : kDropOffset), 0, 0);
        }
        const uint32_t key = ok ? (ACT == rgmath::ACT_RELU ? rgmath::fbits(best) : rgmath::absmax_key(best)) : 0u;
        amax = key > amax ? key : amax;
      }
    }
  if constexpr (!LDS) conv_block_absmax<NW>(ep, b, amax, red, lane);
  return amax;
}

// The band conv's MFMA part: wave `wave`'s TN / 4 pixels of the block from
// output pixel p0 (pix[j]: fragment j's pixel in this lane), summed over the
// LDS band (output row oy0's band row first, channel-last with cp channels
// per pixel, Wp pixels per row) against TM weight rows of wstride bytes.
// Each MFMA B fragment is one ds_read_b128 (cp >= 16) or four ds_read_b32
// (CP4) of the band; taps past k * k and pixels past L read zero16.
struct BandGeom {
  int OW, L, oy0, st, Wp, cp, k, kk, KP, wstride;
};

template <int TM, int TN, bool CP4>
__device__ __forceinline__ void conv_band_mma(const int8_t* wts, const int8_t* band, const int8_t* zero16,
                                              const BandGeom& g, int p0, int wave, int lane, int (&pix)[TN / 64],
                                              v4i (&acc)[TM / 16][TN / 64]) {
  constexpr int WTN = TN / 4, FM = TM / 16, FN = WTN / 16;
  const int OW = g.OW, L = g.L, oy0 = g.oy0, st = g.st, Wp = g.Wp, cp = g.cp, k = g.k, kk = g.kk, KP = g.KP,
            wstride = g.wstride;
  // the byte offset of each pixel's tap (0, 0), channel 0
  const uint32_t owmag_k = div_magic((uint32_t)OW), kmag = div_magic((uint32_t)k), cpmag = div_magic((uint32_t)cp);
  int rowoff[FN];
#pragma unroll
  for (int j = 0; j < FN; j++) {
    pix[j] = p0 + wave * WTN + j * 16 + (lane & 15);
    const int oy = udiv(pix[j], owmag_k), ox = pix[j] - oy * OW;
    rowoff[j] = pix[j] < L ? ((oy - oy0) * st * Wp + ox * st) * cp : -1;
  }
#pragma unroll
  for (int i = 0; i < FM; i++)
#pragma unroll
    for (int j = 0; j < FN; j++) acc[i][j] = v4i{0, 0, 0, 0};
  for (int k0 = 0; k0 < KP; k0 += 64) {
    const int kb = k0 + (lane >> 4) * 16;  // this lane's 16-byte K chunk
    v4i af[FM], bf[FN];
#pragma unroll
    for (int i = 0; i < FM; i++) af[i] = *reinterpret_cast<const v4i*>(wts + (i * 16 + (lane & 15)) * wstride + kb);
    if (!CP4) {
      const int tap = udiv(kb, cpmag), c0 = kb - tap * cp;
      const int ki = udiv(tap, kmag), kj = tap - ki * k;
      const int toff = (ki * Wp + kj) * cp + c0;
#pragma unroll
      for (int j = 0; j < FN; j++) {
        const int8_t* a = (rowoff[j] >= 0 && tap < kk) ? band + rowoff[j] + toff : zero16;
        bf[j] = *reinterpret_cast<const v4i*>(a);
      }
    } else {
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int tap = (kb >> 2) + e;
        const int ki = udiv(tap, kmag), kj = tap - ki * k;
        const int toff = (ki * Wp + kj) * 4;
#pragma unroll
        for (int j = 0; j < FN; j++) {
          const int8_t* a = (rowoff[j] >= 0 && tap < kk) ? band + rowoff[j] + toff : zero16;
          bf[j][e] = *reinterpret_cast<const int*>(a);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
      for (int j = 0; j < FN; j++)
        acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
  }
}

// conv_band_mma with every dimension known at compile time and every pixel
// of the block inside the output, oy0 = 0 and stride 1 (the pair kernel's
// two convs): the divisions, the tap offsets and the K loop fold to
// constants and immediates.
template <int TM, int TN, bool CP4, int OW, int WP, int CP, int K, int KP, int WSTRIDE>
__device__ __forceinline__ void conv_band_mma_fixed(const int8_t* wts, const int8_t* band, const int8_t* zero16, int p0,
                                                    int wave, int lane, int (&pix)[TN / 64],
                                                    v4i (&acc)[TM / 16][TN / 64]) {
  constexpr int WTN = TN / 4, FM = TM / 16, FN = WTN / 16, KK = K * K;
  static_assert(KP % 64 == 0 && (OW & (OW - 1)) == 0, "whole K steps; a power-of-two row");
  int rowoff[FN];
#pragma unroll
  for (int j = 0; j < FN; j++) {
    pix[j] = p0 + wave * WTN + j * 16 + (lane & 15);
    rowoff[j] = ((pix[j] / OW) * WP + pix[j] % OW) * CP;
  }
#pragma unroll
  for (int i = 0; i < FM; i++)
#pragma unroll
    for (int j = 0; j < FN; j++) acc[i][j] = v4i{0, 0, 0, 0};
  const int q16 = (lane >> 4) * 16;  // this lane's 16-byte K chunk within a step
#pragma unroll
  for (int k0 = 0; k0 < KP; k0 += 64) {
    const int kb = k0 + q16;
    v4i af[FM], bf[FN];
#pragma unroll
    for (int i = 0; i < FM; i++) af[i] = *reinterpret_cast<const v4i*>(wts + (i * 16 + (lane & 15)) * WSTRIDE + kb);
    if constexpr (!CP4) {
      const int tap = kb / CP, c0 = kb % CP;
      const int toff = ((tap / K) * WP + tap % K) * CP + c0;
#pragma unroll
      for (int j = 0; j < FN; j++)
        bf[j] = *reinterpret_cast<const v4i*>(tap < KK ? band + rowoff[j] + toff : zero16);
    } else {
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int tap = (kb >> 2) + e;
        const int toff = ((tap / K) * WP + tap % K) * 4;
#pragma unroll
        for (int j = 0; j < FN; j++) bf[j][e] = *reinterpret_cast<const int*>(tap < KK ? band + rowoff[j] + toff : zero16);
      }
    }
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
      for (int j = 0; j < FN; j++)
        acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
  }
}

constexpr int64_t kConvSelfAbsmaxMax = 16384;

// Publishes a block-measured per-image absmax in the image's slot (zeroed
// at the start of the run, read only after the kernel).
__device__ __forceinline__ void ep_absmax_publish(const uint32_t* slots, int b, uint32_t v) {
  const_cast<uint32_t*>(slots)[b] = v;
}

// CP4 (3- or 4-channel images, the run's first conv) keeps within 128
// registers, so four of its workgroups share a CU.
template <int TM, int TN, bool CP4, bool XF = false>
__global__ __launch_bounds__(256, CP4 ? 4 : 1) void conv_band_kernel(const int8_t* __restrict__ xq, const int8_t* __restrict__ Wt,
                                                        ConvShape cs, Epilogue ep, int self_absmax, SlotClear clear) {
  extern __shared__ __attribute__((aligned(16))) int8_t dsm[];
  constexpr int WTN = TN / 4, FM = TM / 16, FN = WTN / 16;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // grid (images, channel blocks, pixel blocks): the blocks of one image are
  // dealt to the same XCD (linear workgroup id = image mod 8 for image counts
  // that are multiples of 8), so they share its L2 for the image's reads
  const int b = blockIdx.x, o0 = blockIdx.y * TM, p0 = blockIdx.z * TN;
  const int C = (int)cs.C, H = (int)cs.H, W = (int)cs.W, k = (int)cs.k, st = (int)cs.stride, pad = (int)cs.pad;
  const int OW = (int)cs.OW, L = (int)(cs.OH * cs.OW), KP = (int)cs.Kpad, cp = (int)cs.cp, kk = k * k;
  const int wstride = KP + 16, Wp = W + 2 * pad;
  int8_t* const wts = dsm;
  int8_t* const band = dsm + TM * wstride;
  const int oy0 = p0 / OW, oy1 = (min(p0 + TN, L) - 1) / OW;
  const int R = (oy1 - oy0) * st + k;
  const int band_bytes = R * Wp * cp;
  int8_t* const zero16 = band + ((band_bytes + 15) & ~15);

  // The f32 input's first band batch (see step 2), loaded up front.
  const int iy_base = oy0 * st - pad;
  float img_scale = 0.0f;
  // units in flight per thread: with 4 channels (CP4: the run's first conv
  // of 3-channel images) a band holds few units, fewer registers suffice
  constexpr int BATCH = CP4 ? 2 : 8;
  float v[BATCH][4];  // unused (and removed) in the i8 form
  int dst[BATCH];
  const float* imgf = reinterpret_cast<const float*>(xq) + (int64_t)b * C * H * W;
  const int per_g = R * W, total = (cp / 4) * per_g;  // channel groups of 4 (cp is 4 or a multiple of 16)
  auto load_batch = [&](int e0) {
#pragma unroll
    for (int u = 0; u < BATCH; u++) {
      const int e = e0 + u * 256;
      const int g = e / per_g, t = e - g * per_g, r = t / W, x = t - r * W;
      const int iy = iy_base + r;
      const bool ok = e < total && iy >= 0 && iy < H;
      dst[u] = ok ? (r * Wp + x + pad) * cp + 4 * g : -1;
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const int c = 4 * g + q;
        v[u][q] = ok && c < C ? imgf[((int64_t)c * H + iy) * W + x] : 0.0f;
      }
    }
  };
  // The image's scale comes from its own absmax (over every pixel a window
  // reads), so the clamp cannot act on those pixels (quantize_rz_bounded);
  // pixels no window reads are never used.  Four bytes pack with v_perm.
  auto pack4b = [](float a, float b_, float c, float d, float inv) -> uint32_t {
    const uint32_t b0 = (uint32_t)rgmath::quantize_rz_bounded(a * inv), b1 = (uint32_t)rgmath::quantize_rz_bounded(b_ * inv);
    const uint32_t b2 = (uint32_t)rgmath::quantize_rz_bounded(c * inv), b3 = (uint32_t)rgmath::quantize_rz_bounded(d * inv);
    const uint32_t lo = __builtin_amdgcn_perm(b1, b0, 0x0c0c0400u);  // bytes b0.0, b1.0
    const uint32_t hi = __builtin_amdgcn_perm(b3, b2, 0x0c0c0400u);
    return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
  };
  auto store_batch = [&](float inv) {
#pragma unroll
    for (int u = 0; u < BATCH; u++) {
      if (dst[u] < 0) continue;
      *reinterpret_cast<uint32_t*>(band + dst[u]) = pack4b(v[u][0], v[u][1], v[u][2], v[u][3], inv);
    }
  };
  // The vector form of the same fill (rows of a multiple of 4 floats on a
  // 16-byte boundary): a unit is 4 channels x 4 pixels of one band row, read
  // with four 16-byte loads through a resource bounded by the image (channels
  // past C read zeros; rows outside the image get the dropped offset), and
  // written as four 32-bit LDS words.  A thread's units are 256 apart; their
  // (channel group, row, pixel quad) advance by the uniform step of 256 units
  // without divisions.
  constexpr int B4 = CP4 ? 1 : 4;
  const bool vec4 = XF && (W & 3) == 0 && (reinterpret_cast<uintptr_t>(xq) & 15) == 0 && C * H * W < (1 << 29);
  const int wq = W >> 2, per_g4 = R * wq, g4 = cp >> 2, total4 = g4 * per_g4;
  int ug = 0, ur = 0, ux = 0, sg = 0, sr = 0, sx = 0;
  if (vec4) {
    ug = tid / per_g4;
    const int rem = tid - ug * per_g4;
    ur = rem / wq;
    ux = rem - ur * wq;
    sg = 256 / per_g4;
    const int srem = 256 - sg * per_g4;
    sr = srem / wq;
    sx = srem - sr * wq;
  }
  const __amdgpu_buffer_rsrc_t rimg = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(imgf), 0, (int)((uint32_t)(C * H * W) * 4u), 0x00020000);
  v4f w4[B4][4];
  int d4[B4];
  auto load4 = [&]() {
#pragma unroll
    for (int u = 0; u < B4; u++) {
      const int iy = iy_base + ur;
      const bool ok = ug < g4 && iy >= 0 && iy < H;
      d4[u] = ok ? ((ur * Wp + 4 * ux + pad) * cp + 4 * ug) : -1;
      const uint32_t off = (uint32_t)(((4 * ug) * H + iy) * W + 4 * ux) * 4u;
#pragma unroll
      for (int q = 0; q < 4; q++)
        w4[u][q] = __builtin_bit_cast(
            v4f, __builtin_amdgcn_raw_buffer_load_b128(rimg, (int)(ok ? off + (uint32_t)(q * H * W) * 4u : kDropOffset),
                                                       0, 0));
      ux += sx;
      if (ux >= wq) {
        ux -= wq;
        ur++;
      }
      ur += sr;
      if (ur >= R) {
        ur -= R;
        ug++;
      }
      ug += sg;
    }
  };
  auto store4 = [&](float inv) {
#pragma unroll
    for (int u = 0; u < B4; u++) {
      if (d4[u] < 0) continue;
#pragma unroll
      for (int xx = 0; xx < 4; xx++)
        *reinterpret_cast<uint32_t*>(band + d4[u] + xx * cp) =
            pack4b(w4[u][0][xx], w4[u][1][xx], w4[u][2][xx], w4[u][3][xx], inv);
    }
  };
  // The image's absmax comes first: with self_absmax the first 4 x 256
  // 16-byte pieces of the image, else the image's slot, are loaded before the
  // band and the weights, so all three share one memory round trip.
  __shared__ uint32_t red[4];
  const int n_img = C * H * W;
  const bool am_vec = XF && self_absmax && (n_img & 3) == 0 && (reinterpret_cast<uintptr_t>(imgf) & 15) == 0;
  float4 am4[4];
  uint32_t slot_bits = 0;
  if constexpr (XF) {
    if (am_vec) {
      const float4* f4 = reinterpret_cast<const float4*>(imgf);
#pragma unroll
      for (int u = 0; u < 4; u++)
        am4[u] = tid + u * 256 < (n_img >> 2) ? f4[tid + u * 256] : float4{0.0f, 0.0f, 0.0f, 0.0f};
    } else if (!self_absmax) {
      slot_bits = ep.absmax_in[b];
    }
    if (vec4)
      load4();
    else
      load_batch(tid);
  }

  // 1. zero the band and the zero block; copy this block's weights.
  for (int i = tid; i <= (band_bytes + 15) / 16; i += 256) *reinterpret_cast<v4i*>(band + 16 * i) = v4i{0, 0, 0, 0};
  const int kc = KP / 16;
  const uint32_t kcmag = div_magic((uint32_t)kc);
  for (int i = tid; i < TM * kc; i += 256) {
    const int row = udiv(i, kcmag), c16 = i - row * kc;
    *reinterpret_cast<v4i*>(wts + row * wstride + c16 * 16) =
        *reinterpret_cast<const v4i*>(Wt + (int64_t)(o0 + row) * KP + c16 * 16);
  }
  __syncthreads();
  // 2. input rows iy = oy0*st - pad + r of every channel, channel-last.  The
  // f32 input: with self_absmax the image's absmax first (its loads overlap
  // the first batch's), then the batches are quantized into the band.
  if constexpr (XF) {
    if (self_absmax) {
      clear_slots(clear);
      float m = 0.0f;  // NaN ignored, like f32::max
      if (am_vec) {
        const float4* f4 = reinterpret_cast<const float4*>(imgf);
        const int n4 = n_img >> 2;
        for (int e = tid;; e += 4 * 256) {
#pragma unroll
          for (int u = 0; u < 4; u++) {
            m = __builtin_fmaxf(__builtin_fmaxf(m, __builtin_fabsf(am4[u].x)), __builtin_fabsf(am4[u].y));
            m = __builtin_fmaxf(__builtin_fmaxf(m, __builtin_fabsf(am4[u].z)), __builtin_fabsf(am4[u].w));
          }
          if (e + 4 * 256 >= n4) break;
#pragma unroll
          for (int u = 0; u < 4; u++)
            am4[u] = e + 4 * 256 + u * 256 < n4 ? f4[e + 4 * 256 + u * 256] : float4{0.0f, 0.0f, 0.0f, 0.0f};
        }
      } else {
        for (int e = tid; e < n_img; e += 256) m = __builtin_fmaxf(m, __builtin_fabsf(imgf[e]));
      }
      const uint32_t w = wave_max_u32(rgmath::fbits(m));
      if (lane == 0) red[wave] = w;
      __syncthreads();
      const uint32_t t = max(max(red[0], red[1]), max(red[2], red[3]));
      if (tid == 0 && blockIdx.z == 0 && blockIdx.y == 0) ep_absmax_publish(ep.absmax_in, b, t);
      img_scale = rgmath::scale_from_absmax(rgmath::bitsf(t));
      __syncthreads();  // red is reused by the epilogue's absmax
    } else {
      img_scale = rgmath::scale_from_absmax(rgmath::bitsf(slot_bits));
    }
    const float inv = 1.0f / img_scale;
    if (vec4) {
      store4(inv);
      for (int e0 = 256 * B4; e0 < total4; e0 += 256 * B4) {
        load4();
        store4(inv);
      }
    } else {
      store_batch(inv);
      for (int e0 = tid + 256 * BATCH; e0 < total; e0 += 256 * BATCH) {
        load_batch(e0);
        store_batch(inv);
      }
    }
  } else if ((W & 3) == 0) {
    const int8_t* img = xq + (int64_t)b * C * H * W;
    const int wq = W >> 2, per_c = R * wq;
    for (int e = tid; e < C * per_c; e += 256) {
      const int c = e / per_c, t = e - c * per_c, r = t / wq, x = (t - r * wq) * 4;
      const int iy = iy_base + r;
      if (iy >= 0 && iy < H) {
        const uint32_t v = *reinterpret_cast<const uint32_t*>(img + ((int64_t)c * H + iy) * W + x);
        int8_t* d = band + (r * Wp + x + pad) * cp + c;
        d[0] = (int8_t)v;
        d[cp] = (int8_t)(v >> 8);
        d[2 * cp] = (int8_t)(v >> 16);
        d[3 * cp] = (int8_t)(v >> 24);
      }
    }
  } else {
    const int8_t* img = xq + (int64_t)b * C * H * W;
    const int per_c = R * W;
    for (int e = tid; e < C * per_c; e += 256) {
      const int c = e / per_c, t = e - c * per_c, r = t / W, x = t - r * W;
      const int iy = iy_base + r;
      if (iy >= 0 && iy < H) band[(r * Wp + x + pad) * cp + c] = img[((int64_t)c * H + iy) * W + x];
    }
  }
  __syncthreads();

  // 3. per-lane pixels and their sums over the band
  const BandGeom geo{OW, L, oy0, st, Wp, cp, k, kk, KP, wstride};
  int pix[FN];
  v4i acc[FM][FN];
  conv_band_mma<TM, TN, CP4>(wts, band, zero16, geo, p0, wave, lane, pix, acc);
  float csc;
  if constexpr (XF)
    csc = img_scale * ep.w_scale;
  else
    csc = slot_scale(ep.absmax_in + b) * ep.w_scale;
  if constexpr (XF && TN / 64 >= 2) {
    // the fused 2 x 2 pool (ReLU or no activation; try_conv_band checks the shape)
    if (ep.pool2) {
      const bool relu = ep.act == rgmath::ACT_RELU;
      if constexpr (TN / 64 >= 4) {
        if (ep.pool2 == 2) {
          relu ? conv_band_epilogue_pool2<TM, TN, rgmath::ACT_RELU, 2>(acc, cs, ep, b, o0, pix, csc, lane, red)
               : conv_band_epilogue_pool2<TM, TN, rgmath::ACT_NONE, 2>(acc, cs, ep, b, o0, pix, csc, lane, red);
          return;
        }
      }
      relu ? conv_band_epilogue_pool2<TM, TN, rgmath::ACT_RELU, 1>(acc, cs, ep, b, o0, pix, csc, lane, red)
           : conv_band_epilogue_pool2<TM, TN, rgmath::ACT_NONE, 1>(acc, cs, ep, b, o0, pix, csc, lane, red);
      return;
    }
  }
  switch (ep.act) {
    case rgmath::ACT_RELU: conv_band_epilogue<TM, TN, CP4, rgmath::ACT_RELU>(acc, cs, ep, b, o0, pix, csc, lane, red); break;
    case rgmath::ACT_SIGMOID: conv_band_epilogue<TM, TN, CP4, rgmath::ACT_SIGMOID>(acc, cs, ep, b, o0, pix, csc, lane, red); break;
    case rgmath::ACT_TANH: conv_band_epilogue<TM, TN, CP4, rgmath::ACT_TANH>(acc, cs, ep, b, o0, pix, csc, lane, red); break;
    case rgmath::ACT_GELU: conv_band_epilogue<TM, TN, CP4, rgmath::ACT_GELU>(acc, cs, ep, b, o0, pix, csc, lane, red); break;
    case rgmath::ACT_LEAKY_RELU:
      conv_band_epilogue<TM, TN, CP4, rgmath::ACT_LEAKY_RELU>(acc, cs, ep, b, o0, pix, csc, lane, red);
      break;
    case rgmath::ACT_SILU: conv_band_epilogue<TM, TN, CP4, rgmath::ACT_SILU>(acc, cs, ep, b, o0, pix, csc, lane, red); break;
    default: conv_band_epilogue<TM, TN, CP4, rgmath::ACT_NONE>(acc, cs, ep, b, o0, pix, csc, lane, red); break;
  }
}

// Fallback for shapes whose band or weights do not fit in LDS: the im2col
// tile is gathered byte by byte from the quantized image (tap-major K).
template <int TM, int TN>
__global__ __launch_bounds__(256) void conv_i8_kernel(const int8_t* __restrict__ xq, const int8_t* __restrict__ Wq,
                                                      ConvShape cs, Epilogue ep) {
  constexpr int STAGE = (TM + TN) * kLdsStride;
  constexpr int CLD = TN + 4;
  constexpr int EPI = TM * CLD * 4;
  __shared__ __attribute__((aligned(16))) int8_t smem[STAGE > EPI ? STAGE : EPI];
  int8_t* const As = smem;
  int8_t* const Bs = smem + TM * kLdsStride;
  constexpr int WTN = TN / 4, FM = TM / 16, FN = WTN / 16;
  constexpr int A_CHUNKS = TM * kTK / 16;
  constexpr int A_CH = (A_CHUNKS + 255) / 256;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t b = blockIdx.z;
  const int64_t o0 = (int64_t)blockIdx.y * TM, p0 = (int64_t)blockIdx.x * TN;
  const int64_t L = cs.OH * cs.OW;
  const int C = (int)cs.C, H = (int)cs.H, W = (int)cs.W, k = (int)cs.k, cp = (int)cs.cp, kk = k * k;
  const int8_t* img = xq + b * cs.C * cs.H * cs.W;

  v4i acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; i++)
#pragma unroll
    for (int j = 0; j < FN; j++) acc[i][j] = v4i{0, 0, 0, 0};

  // B gather mapping: thread -> pixel (tid % TN), K bytes [(tid/TN)*KB, +KB).
  constexpr int KB = kTK * TN / 256;
  const int gp = tid % TN, gk = (tid / TN) * KB;
  const int64_t pix = p0 + gp;
  const int oy = (int)(pix / cs.OW), ox = (int)(pix % cs.OW);
  const bool pix_ok = pix < L;
  const int koff = (lane >> 4) * 16;

  for (int64_t k0 = 0; k0 < cs.Kpad; k0 += kTK) {
#pragma unroll
    for (int i = 0; i < A_CH; i++) {
      const int c = tid + i * 256;
      if (c < A_CHUNKS)
        *reinterpret_cast<v4i*>(&As[(c >> 2) * kLdsStride + (c & 3) * 16]) =
            *reinterpret_cast<const v4i*>(Wq + (o0 + (c >> 2)) * cs.Kpad + k0 + (c & 3) * 16);
    }
#pragma unroll
    for (int w4 = 0; w4 < KB / 4; w4++) {
      uint32_t word = 0;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int kq = (int)k0 + gk + w4 * 4 + e;  // tap-major index
        const int tap = kq / cp, ch = kq - tap * cp;
        int8_t v = 0;
        if (pix_ok && tap < kk && ch < C) {
          const int ki = tap / k, kj = tap - ki * k;
          const int iy = oy * (int)cs.stride + ki - (int)cs.pad, ix = ox * (int)cs.stride + kj - (int)cs.pad;
          if (iy >= 0 && iy < H && ix >= 0 && ix < W) v = img[((int64_t)ch * H + iy) * W + ix];
        }
        word |= (uint32_t)(uint8_t)v << (8 * e);
      }
      *reinterpret_cast<uint32_t*>(&Bs[gp * kLdsStride + gk + w4 * 4]) = word;
    }
    __syncthreads();
    v4i af[FM], bf[FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
      af[i] = *reinterpret_cast<const v4i*>(&As[(i * 16 + (lane & 15)) * kLdsStride + koff]);
#pragma unroll
    for (int j = 0; j < FN; j++)
      bf[j] = *reinterpret_cast<const v4i*>(&Bs[(wave * WTN + j * 16 + (lane & 15)) * kLdsStride + koff]);
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
      for (int j = 0; j < FN; j++)
        acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
    __syncthreads();
  }

  int32_t* Cs = reinterpret_cast<int32_t*>(smem);
#pragma unroll
  for (int i = 0; i < FM; i++)
#pragma unroll
    for (int j = 0; j < FN; j++)
#pragma unroll
      for (int r = 0; r < 4; r++)
        Cs[(i * 16 + (lane >> 4) * 4 + r) * CLD + wave * WTN + j * 16 + (lane & 15)] = acc[i][j][r];
  __syncthreads();
  const float csc = slot_scale(ep.absmax_in + b) * ep.w_scale;
  const TileCoords tc{o0, p0, cs.O, L, b};
  epilogue_tile<TM, TN, CLD, true>(Cs, tc, csc, ep);
}

// The band kernel divides by the block's shape with high multiplies
// (div_magic), exact when dividend x divisor < 2^32: pixels by OW, taps by k,
// K bytes by cp, weight chunks by Kpad / 16.
static bool conv_band_indexable(const ConvShape& cs, int TM, int TN) {
  const int64_t lim = (int64_t)1 << 32, L = cs.OH * cs.OW, kc = cs.Kpad / 16;
  return (L + TN) * cs.OW < lim && (cs.Kpad / 4 + 4) * cs.k < lim && cs.Kpad * cs.cp < lim && (TM * kc + 256) * kc < lim;
}

template <int TM, int TN, bool CP4, bool XF>
static bool try_conv_band(const int8_t* xq, const int8_t* Wq, const ConvShape& cs, const Epilogue& ep, hipStream_t s,
                          int self_absmax = 0, SlotClear clear = SlotClear{}) {
  if (!conv_band_indexable(cs, TM, TN)) return false;
  // the fused pool needs whole pairs of output rows per wave (TN / 4 pixels)
  if (ep.pool2 && (!XF || (TN / 4) % (32 * ep.pool2) != 0)) return false;
  // 32-bit output offsets within one image (o * L + p), pixel blocks in grid.z
  if (cs.O * cs.OH * cs.OW * 4 >= ((int64_t)1 << 31) || (cs.OH * cs.OW + TN - 1) / TN > 65535 ||
      cs.n >= ((int64_t)1 << 31))
    return false;
  const ConvBand g = conv_band_geom(cs, TM, TN);
  constexpr int kStatic = 64;  // the kernel's few words of static LDS
  constexpr int kMaxLds = 160 * 1024 - kStatic;
  if (g.lds_bytes > kMaxLds) return false;
  const void* fn = reinterpret_cast<const void*>(&conv_band_kernel<TM, TN, CP4, XF>);
  static bool attr_set = false;
  if (!attr_set) {
    if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, kMaxLds) != hipSuccess) return false;
    attr_set = true;
  }
  const int64_t L = cs.OH * cs.OW;
  dim3 grid((unsigned)cs.n, (unsigned)(cs.Opad / TM), (unsigned)((L + TN - 1) / TN));
  RG_LAUNCH((conv_band_kernel<TM, TN, CP4, XF>), grid, dim3(256), (unsigned)g.lds_bytes, s, xq, Wq, cs, ep,
            self_absmax, clear);
  return true;
}

template <int TM, bool CP4, bool XF>
static bool try_conv_band_tn(const int8_t* xq, const int8_t* Wq, const ConvShape& cs, const Epilogue& ep,
                             hipStream_t s, int self_absmax = 0, SlotClear clear = SlotClear{}) {
  // 256-pixel blocks unless that leaves fewer than two workgroups per CU
  // (512 on the MI355X's 256 CUs): then 128-pixel blocks first, whose bands
  // add only their halo rows, so more CUs hold two blocks' latency chains
  const int64_t L = cs.OH * cs.OW;
  // RGNPU_CONV_TN (64, 128 or 256) tries that block width first (measurement aid)
  static const int forced = [] {
    const char* e = getenv("RGNPU_CONV_TN");
    return e ? atoi(e) : 0;
  }();
  if (forced == 64 && try_conv_band<TM, 64, CP4, XF>(xq, Wq, cs, ep, s, self_absmax, clear)) return true;
  if (forced == 128 && try_conv_band<TM, 128, CP4, XF>(xq, Wq, cs, ep, s, self_absmax, clear)) return true;
  if (forced == 256 && try_conv_band<TM, 256, CP4, XF>(xq, Wq, cs, ep, s, self_absmax, clear)) return true;
  const bool small_grid = cs.n * (cs.Opad / TM) * ((L + 255) / 256) < 512;
  if (small_grid && try_conv_band<TM, 128, CP4, XF>(xq, Wq, cs, ep, s, self_absmax, clear)) return true;
  return try_conv_band<TM, 256, CP4, XF>(xq, Wq, cs, ep, s, self_absmax, clear) ||
         try_conv_band<TM, 128, CP4, XF>(xq, Wq, cs, ep, s, self_absmax, clear) ||
         try_conv_band<TM, 64, CP4, XF>(xq, Wq, cs, ep, s, self_absmax, clear);
}

bool conv_self_absmax_supported(const ConvShape& cs) { return cs.C * cs.H * cs.W <= kConvSelfAbsmaxMax; }

bool conv_pool_supported(const ConvShape& cs, int r16) {
  if (r16 != 1 && r16 != 2) return false;
  if (cs.n >= ((int64_t)1 << 31) || cs.C * cs.H * cs.W >= ((int64_t)1 << 31) || cs.OH * cs.OW >= ((int64_t)1 << 31) ||
      cs.O * cs.OH * cs.OW * 4 >= ((int64_t)1 << 31) || (cs.OH * cs.OW + 127) / 128 > 65535)
    return false;
  const int TM = cs.Opad % 64 == 0 ? 64 : 32;
  constexpr int kMaxLds = 160 * 1024 - 64;  // try_conv_band's bound for the f32-input form
  for (const int TN : {256, 128})
    if ((TN / 4) % (32 * r16) == 0 && conv_band_geom(cs, TM, TN).lds_bytes <= kMaxLds && conv_band_indexable(cs, TM, TN))
      return true;
  return false;
}

bool launch_conv_f32in(const float* x, const int8_t* Wq, const ConvShape& cs, const Epilogue& ep, hipStream_t s,
                       bool self_absmax, SlotClear clear) {
  if (cs.n > 65535 || cs.C * cs.H * cs.W >= ((int64_t)1 << 31) || cs.OH * cs.OW >= ((int64_t)1 << 31))
    throw std::logic_error("conv: shape too large for the kernel's indexing");
  if (self_absmax && !conv_self_absmax_supported(cs)) throw std::logic_error("conv: image too large for self_absmax");
  const int8_t* xb = reinterpret_cast<const int8_t*>(x);
  const bool cp4 = cs.cp == 4;
  const int sa = self_absmax ? 1 : 0;
  if (cs.Opad % 64 == 0)
    return cp4 ? try_conv_band_tn<64, true, true>(xb, Wq, cs, ep, s, sa, clear)
               : try_conv_band_tn<64, false, true>(xb, Wq, cs, ep, s, sa, clear);
  return cp4 ? try_conv_band_tn<32, true, true>(xb, Wq, cs, ep, s, sa, clear)
             : try_conv_band_tn<32, false, true>(xb, Wq, cs, ep, s, sa, clear);
}

// ---------------------------------------------------------------------------
// Two INT8 conv + 2 x 2 max pool stages on one image per workgroup
// (npu.rs:319-390, op after op): conv A (C <= 4 channels, 3 x 3, stride 1,
// pad 1, on a 32 x 32 image) with ReLU or no activation, its pool, then
// conv B (OA -> OB channels, the same window) and its pool.  A conv's
// activation scale is per image (npu.rs:341-351), and conv B's is the absmax
// of this image's pooled conv A output, which the workgroup holds in LDS:
// nothing crosses workgroups, the pooled intermediate never leaves LDS, and
// one launch replaces two.  Every step is the arithmetic of conv_band_kernel
// (the band quantized with the image's own scale, conv_band_mma, the pooled
// epilogue's window rule), so the outputs are the same bit for bit.
// The workgroup is 16 waves in four groups of 4 (four waves per SIMD).
//  0. Each thread loads one unit of the image (4 channels x 4 pixels of one
//     row: 256 units cover 32 x 32; threads 256.. load them again),
//     and a share of both convs' weights.
//  1. The image's absmax from those registers (every pixel is in a window);
//     its key goes to conv A's slot, as the separate conv would publish it.
//  2. The unit, quantized, fills conv A's channel-last band (all 34 rows).
//  3. Conv A in four 256-pixel blocks, one per wave group, each pooled into
//     the LDS planes.
//  4. The planes' absmax (conv B's per-image scale; its key goes to conv B's
//     slot, as pool A's epilogue would have raised it).
//  5. The planes, quantized, fill conv B's band.
//  6. Conv B over all 256 pixels, each wave group taking a quarter of the
//     output channels, pooled into y with the block's absmax raised for the
//     next op (conv_block_absmax).
// ---------------------------------------------------------------------------
constexpr int kPairSide = 32;  // conv A's image side; conv B's is half of it

struct PairLds {
  int wa, wb, band_a, zero_a, band_b, zero_b, plane, total;
};

// LDS byte offsets (each 16-byte aligned): the weights (rows of Kpad + 16
// bytes, as conv_band_kernel stages them), the bands with a zero block each,
// and the pooled planes [OA, 16, 16] f32.
static __host__ __device__ inline PairLds pair_lds(int OA, int OB, int KPA, int KPB) {
  const int sa = kPairSide + 2, sb = kPairSide / 2 + 2;
  PairLds l{};
  l.wa = 0;
  l.wb = (OA * (KPA + 16) + 15) & ~15;
  l.band_a = l.wb + ((OB * (KPB + 16) + 15) & ~15);
  l.zero_a = l.band_a + ((sa * sa * 4 + 15) & ~15);
  l.band_b = l.zero_a + 16;
  l.zero_b = l.band_b + ((sb * sb * OA + 15) & ~15);
  l.plane = l.zero_b + 16;
  l.total = l.plane + OA * (kPairSide / 2) * (kPairSide / 2) * 4;
  return l;
}

constexpr int kPairThreads = 1024;  // 16 waves: four groups of 4, four waves per SIMD
// the two convs' K padding (conv_kpad: 9 taps x 4 channel bytes, 9 taps x 32)
constexpr int kPairKpA = 64, kPairKpB = 320;
// static LDS of the pair kernel (wave maxima, the two convs' biases) stays under this bound
constexpr int kPairStaticLds = 512;
constexpr int kPairWbUnits = 2;     // 16-byte weight units of conv B per thread at most (OB * KPB <= 2 * 1024 * 16)

template <int OA, int OB, int ACTA, int ACTB>
__global__ __launch_bounds__(kPairThreads) void conv_pool_pair_kernel(const float* __restrict__ x,
                                                                      const int8_t* __restrict__ WA,
                                                                      const int8_t* __restrict__ WB, ConvShape csA,
                                                                      ConvShape csB, Epilogue epA, Epilogue epB,
                                                                      SlotClear clear) {
  constexpr int S = kPairSide, PS = S / 2, SA = S + 2, SB = PS + 2, PL = PS * PS, NT = kPairThreads, NW = NT / 64;
  constexpr int NG = NW / 4;  // wave groups
  static_assert(OA % 16 == 0 && OB % (16 * NG) == 0, "channel blocks of 16; conv B's channels split over the groups");
  extern __shared__ __attribute__((aligned(16))) int8_t dsm[];
  __shared__ uint32_t red[NW];
  __shared__ __attribute__((aligned(16))) float lbias[OA + OB];  // both convs' biases
  static_assert(sizeof(red) + sizeof(lbias) <= kPairStaticLds, "static LDS bound");
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, grp = wave >> 2, wl = wave & 3, b = blockIdx.x;
  const int C = (int)csA.C;
  constexpr int KPA = kPairKpA, KPB = kPairKpB;  // host-checked against the shapes
  // the shapes with their sides as constants, so the epilogues' divisions fold
  ConvShape sa = csA, sb = csB;
  sa.O = OA;
  sa.OH = sa.OW = S;
  sb.O = OB;
  sb.OH = sb.OW = PS;
  const PairLds ly = pair_lds(OA, OB, KPA, KPB);
  int8_t* const wa = dsm + ly.wa;
  int8_t* const wb = dsm + ly.wb;
  int8_t* const band_a = dsm + ly.band_a;
  int8_t* const band_b = dsm + ly.band_b;
  float* const plane = reinterpret_cast<float*>(dsm + ly.plane);

  // 0. unit tid % 256 of the image (channels 0-3 of pixels x4 .. x4 + 3 of
  // row y; channels past C read zeros through the bounded resource), which
  // threads 256.. load again and do not store, and the weights.  Weight rows
  // are contiguous in memory (KPA, KPB bytes): unit i of a conv's weights is
  // bytes [16 i, 16 i + 16).  Every load is issued (a unit past the end is
  // clamped and not stored), so no branch leaves a register pending.
  const int unit = tid & 255, y = unit >> 3, x4 = (unit & 7) * 4;
  const float* img = x + (int64_t)b * C * S * S;
  const __amdgpu_buffer_rsrc_t rimg =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(img), 0, (int)((uint32_t)(C * S * S) * 4u), 0x00020000);
  v4f u[4];
#pragma unroll
  for (int q = 0; q < 4; q++)
    u[q] = __builtin_bit_cast(
        v4f, __builtin_amdgcn_raw_buffer_load_b128(rimg, (int)((uint32_t)((q * S + y) * S + x4) * 4u), 0, 0));
  const int kca = KPA / 16, kcb = KPB / 16, na = OA * kca, nb = OB * kcb;
  const uint32_t kcamag = div_magic((uint32_t)kca), kcbmag = div_magic((uint32_t)kcb);
  const v4i wav = reinterpret_cast<const v4i*>(WA)[tid < na ? tid : na - 1];
  v4i wbv[kPairWbUnits];
#pragma unroll
  for (int t = 0; t < kPairWbUnits; t++) {
    const int i = tid + NT * t;
    wbv[t] = reinterpret_cast<const v4i*>(WB)[i < nb ? i : nb - 1];
  }
  // the biases (padded to Opad), read with the image and weights
  const float bv = tid < OA ? epA.bias[tid] : epB.bias[tid < OA + OB ? tid - OA : 0];
  // both bands and their zero blocks to zero (they are contiguous)
  for (int i = tid; i < (ly.plane - ly.band_a) / 16; i += NT) reinterpret_cast<v4i*>(band_a)[i] = v4i{0, 0, 0, 0};
  clear_slots(clear);
  if (tid < na) {
    const int row = udiv(tid, kcamag), c16 = tid - row * kca;
    *reinterpret_cast<v4i*>(wa + row * (KPA + 16) + c16 * 16) = wav;
  }
#pragma unroll
  for (int t = 0; t < kPairWbUnits; t++) {
    const int i = tid + NT * t;
    if (i < nb) {
      const int row = udiv(i, kcbmag), c16 = i - row * kcb;
      *reinterpret_cast<v4i*>(wb + row * (KPB + 16) + c16 * 16) = wbv[t];
    }
  }
  if (tid < OA + OB) lbias[tid] = bv;
  // 1. the image's absmax (NaN ignored, like f32::max)
  float m = 0.0f;
#pragma unroll
  for (int q = 0; q < 4; q++) {
    m = __builtin_fmaxf(__builtin_fmaxf(m, __builtin_fabsf(u[q][0])), __builtin_fabsf(u[q][1]));
    m = __builtin_fmaxf(__builtin_fmaxf(m, __builtin_fabsf(u[q][2])), __builtin_fabsf(u[q][3]));
  }
  uint32_t w = wave_max_u32(rgmath::fbits(m));
  if (lane == 0) red[wave] = w;
  __syncthreads();
  uint32_t ta = red[0];
#pragma unroll
  for (int i = 1; i < NW; i++) ta = red[i] > ta ? red[i] : ta;
  if (tid == 0) ep_absmax_publish(epA.absmax_in, b, ta);
  const float scale_a = rgmath::scale_from_absmax(rgmath::bitsf(ta));
  // 2. conv A's band: pixel (y, x) at word (y + 1) * SA + x + 1, channels 0-3
  if (tid < 256) {
    const float inv = 1.0f / scale_a;
    uint32_t* const bw = reinterpret_cast<uint32_t*>(band_a) + (y + 1) * SA + x4 + 1;
#pragma unroll
    for (int xx = 0; xx < 4; xx++) {
      const uint32_t b0 = (uint32_t)rgmath::quantize_rz_bounded(u[0][xx] * inv);
      const uint32_t b1 = (uint32_t)rgmath::quantize_rz_bounded(u[1][xx] * inv);
      const uint32_t b2 = (uint32_t)rgmath::quantize_rz_bounded(u[2][xx] * inv);
      const uint32_t b3 = (uint32_t)rgmath::quantize_rz_bounded(u[3][xx] * inv);
      const uint32_t lo = __builtin_amdgcn_perm(b1, b0, 0x0c0c0400u), hi = __builtin_amdgcn_perm(b3, b2, 0x0c0c0400u);
      bw[xx] = __builtin_amdgcn_perm(hi, lo, 0x05040100u);
    }
  }
  __syncthreads();
  // 3. conv A, pooled into the planes: the wave groups take the 256-pixel
  // blocks in turn
  const float csc_a = scale_a * epA.w_scale;
  uint32_t ma = 0;
#pragma unroll 1
  for (int blk = grp; blk < (S * S) / 256; blk += NG) {
    int pix[4];
    v4i acc[OA / 16][4];
    conv_band_mma_fixed<OA, 256, true, S, SA, 4, 3, kPairKpA, kPairKpA + 16>(wa, band_a, dsm + ly.zero_a, blk * 256, wl,
                                                                             lane, pix, acc);
    const uint32_t t = conv_band_epilogue_pool2<OA, 256, ACTA, 2, true, 4, true>(acc, sa, epA, b, 0, pix, csc_a, lane,
                                                                                 red, plane, lbias);
    ma = t > ma ? t : ma;
  }
  // 4. conv B's scale: the absmax of the pooled planes
  w = wave_max_u32(ma);
  __syncthreads();  // every plane value is written, and red is free again
  if (lane == 0) red[wave] = w;
  __syncthreads();
  uint32_t tb = red[0];
#pragma unroll
  for (int i = 1; i < NW; i++) tb = red[i] > tb ? red[i] : tb;
  if (tid == 0) ep_absmax_publish(epB.absmax_in, b, tb);
  const float scale_b = rgmath::scale_from_absmax(rgmath::bitsf(tb));
  // 5. conv B's band: pixel p of the planes, channel group g at word
  // ((p / 16 + 1) * SB + p % 16 + 1) * (OA / 4) + g
  {
    const float inv = 1.0f / scale_b;
    uint32_t* const bw = reinterpret_cast<uint32_t*>(band_b);
#pragma unroll
    for (int t = 0; t < (OA / 4) * PL / NT; t++) {
      const int e = tid + NT * t, p = e & (PL - 1), g = e / PL;
      const float* src = plane + (4 * g) * PL + p;
      const uint32_t b0 = (uint32_t)rgmath::quantize_rz_bounded(src[0] * inv);
      const uint32_t b1 = (uint32_t)rgmath::quantize_rz_bounded(src[PL] * inv);
      const uint32_t b2 = (uint32_t)rgmath::quantize_rz_bounded(src[2 * PL] * inv);
      const uint32_t b3 = (uint32_t)rgmath::quantize_rz_bounded(src[3 * PL] * inv);
      const uint32_t lo = __builtin_amdgcn_perm(b1, b0, 0x0c0c0400u), hi = __builtin_amdgcn_perm(b3, b2, 0x0c0c0400u);
      bw[((p / PS + 1) * SB + (p % PS) + 1) * (OA / 4) + g] = __builtin_amdgcn_perm(hi, lo, 0x05040100u);
    }
  }
  __syncthreads();
  // 6. conv B, pooled into y: each wave group takes OB / NG output channels
  constexpr int OH = OB / NG;
  int pix[4];
  v4i acc[OH / 16][4];
  conv_band_mma_fixed<OH, 256, false, PS, SB, OA, 3, kPairKpB, kPairKpB + 16>(wb + grp * OH * (kPairKpB + 16), band_b,
                                                                              dsm + ly.zero_b, 0, wl, lane, pix, acc);
  conv_band_epilogue_pool2<OH, 256, ACTB, 1, false, NW, true>(acc, sb, epB, b, grp * OH, pix, scale_b * epB.w_scale,
                                                              lane, red, nullptr, lbias + OA);
}

bool conv_pool_pair_supported(const ConvShape& a, const ConvShape& b) {
  constexpr int S = kPairSide;
  const bool ok_a = a.C >= 1 && a.C <= 4 && a.cp == 4 && a.H == S && a.W == S && a.k == 3 && a.stride == 1 &&
                    a.pad == 1 && a.OH == S && a.OW == S && a.O == 32 && a.Opad == 32 && a.Kpad == conv_kpad(a.C, 3);
  const bool ok_b = b.C == 32 && b.cp == 32 && b.H == S / 2 && b.W == S / 2 && b.k == 3 && b.stride == 1 &&
                    b.pad == 1 && b.OH == S / 2 && b.OW == S / 2 && b.O == 64 && b.Opad == 64 &&
                    b.Kpad == conv_kpad(32, 3) && b.n == a.n;
  return ok_a && ok_b && a.Kpad == kPairKpA && b.Kpad == kPairKpB && a.n >= 1 && a.n <= 65535 &&
         64 * (b.Kpad / 16) <= kPairThreads * kPairWbUnits &&
         pair_lds(32, 64, (int)a.Kpad, (int)b.Kpad).total <= 160 * 1024 - kPairStaticLds;
}

template <int ACTA, int ACTB>
static void launch_pair_t(const float* x, const int8_t* WA, const int8_t* WB, const ConvShape& a, const ConvShape& b,
                          const Epilogue& ea, const Epilogue& eb, SlotClear clear, hipStream_t s) {
  const int lds = pair_lds(32, 64, (int)a.Kpad, (int)b.Kpad).total;
  const void* fn = reinterpret_cast<const void*>(&conv_pool_pair_kernel<32, 64, ACTA, ACTB>);
  static bool attr_set = false;
  if (!attr_set) {
    if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024 - kPairStaticLds) != hipSuccess)
      throw std::runtime_error("conv pair: the dynamic LDS limit could not be raised");
    attr_set = true;
  }
  RG_LAUNCH((conv_pool_pair_kernel<32, 64, ACTA, ACTB>), dim3((unsigned)a.n), dim3(kPairThreads), (unsigned)lds, s, x,
            WA, WB, a, b, ea, eb, clear);
}

void launch_conv_pool_pair(const float* x, const int8_t* WA, const int8_t* WB, const ConvShape& a, const ConvShape& b,
                           const Epilogue& ea, const Epilogue& eb, SlotClear clear, hipStream_t s) {
  const bool acts_ok = (ea.act == rgmath::ACT_RELU || ea.act == rgmath::ACT_NONE) &&
                       (eb.act == rgmath::ACT_RELU || eb.act == rgmath::ACT_NONE);
  if (!conv_pool_pair_supported(a, b) || !acts_ok || ea.pool2 != 2 || eb.pool2 != 1 || !ea.absmax_in ||
      !eb.absmax_in || (reinterpret_cast<uintptr_t>(x) & 15) || (reinterpret_cast<uintptr_t>(WA) & 15) ||
      (reinterpret_cast<uintptr_t>(WB) & 15))
    throw std::logic_error("conv pair: the two convs do not fit the one-image kernel");
  const bool ra = ea.act == rgmath::ACT_RELU, rb = eb.act == rgmath::ACT_RELU;
  if (ra && rb)
    launch_pair_t<rgmath::ACT_RELU, rgmath::ACT_RELU>(x, WA, WB, a, b, ea, eb, clear, s);
  else if (ra)
    launch_pair_t<rgmath::ACT_RELU, rgmath::ACT_NONE>(x, WA, WB, a, b, ea, eb, clear, s);
  else if (rb)
    launch_pair_t<rgmath::ACT_NONE, rgmath::ACT_RELU>(x, WA, WB, a, b, ea, eb, clear, s);
  else
    launch_pair_t<rgmath::ACT_NONE, rgmath::ACT_NONE>(x, WA, WB, a, b, ea, eb, clear, s);
}

void launch_conv(const int8_t* xq, const int8_t* Wq, const ConvShape& cs, const Epilogue& ep, hipStream_t s) {
  if (ep.pool2) throw std::logic_error("conv: the fused pool needs the f32-input conv");
  if (cs.n > 65535 || cs.C * cs.H * cs.W >= ((int64_t)1 << 31) || cs.OH * cs.OW >= ((int64_t)1 << 31))
    throw std::logic_error("conv: shape too large for the kernel's indexing");
  const bool cp4 = cs.cp == 4;
  bool done;
  if (cs.Opad % 64 == 0)
    done = cp4 ? try_conv_band_tn<64, true, false>(xq, Wq, cs, ep, s) : try_conv_band_tn<64, false, false>(xq, Wq, cs, ep, s);
  else
    done = cp4 ? try_conv_band_tn<32, true, false>(xq, Wq, cs, ep, s) : try_conv_band_tn<32, false, false>(xq, Wq, cs, ep, s);
  if (done) return;
  constexpr int TN = 128;
  const int64_t L = cs.OH * cs.OW;
  const unsigned gx = (unsigned)((L + TN - 1) / TN);
  if (cs.Opad % 64 == 0) {
    dim3 grid(gx, (unsigned)(cs.Opad / 64), (unsigned)cs.n);
    RG_LAUNCH((conv_i8_kernel<64, TN>), grid, dim3(256), 0, s, xq, Wq, cs, ep);
  } else {
    dim3 grid(gx, (unsigned)(cs.Opad / 32), (unsigned)cs.n);
    RG_LAUNCH((conv_i8_kernel<32, TN>), grid, dim3(256), 0, s, xq, Wq, cs, ep);
  }
}

// ---------------------------------------------------------------------------
// Max pool: window scan in (ki, kj) order from -inf with `v > best || NaN`
// (kernels.rs:180-191), so NaN propagates and ties keep the first element.
// ---------------------------------------------------------------------------
// Grid: y = image, x = contiguous chunks of that image's C*OH*OW outputs
// (32-bit index math within an image).  The next op's absmax is reduced per
// block and raised with one atomic: per image when a conv consumes it, else
// into the block's partial of a spread slot.  Per-wave atomics on one image
// slot were the pool's bottleneck (memory-side atomics serialise).
__global__ __launch_bounds__(256) void maxpool_kernel(const float* __restrict__ x, float* __restrict__ y, uint32_t C,
                                                      uint32_t H, uint32_t W, uint32_t k, uint32_t st, uint32_t OH,
                                                      uint32_t OW, uint32_t chunk, uint32_t* absmax_out,
                                                      int per_image) {
  const int64_t b = blockIdx.y;
  const uint32_t hw = OH * OW, per = C * hw;
  const float* xi = x + b * (int64_t)C * H * W;
  float* yi = y + b * (int64_t)per;
  const uint32_t e0 = blockIdx.x * chunk;
  const uint32_t e1 = per - e0 < chunk ? per : e0 + chunk;
  uint32_t amax = 0;
  for (uint32_t e = e0 + threadIdx.x; e < e1; e += blockDim.x) {
    const uint32_t c = e / hw, r = e - c * hw;
    const uint32_t oy = r / OW, ox = r - oy * OW;
    const float* pl = xi + (size_t)c * H * W + (size_t)(oy * st) * W + ox * st;
    float best = -__builtin_inff();
    for (uint32_t ki = 0; ki < k; ki++)
      for (uint32_t kj = 0; kj < k; kj++) {
        const float v = pl[ki * W + kj];
        if (v > best || v != v) best = v;
      }
    yi[e] = best;
    const uint32_t kk = rgmath::absmax_key(best);
    amax = kk > amax ? kk : amax;
  }
  if (absmax_out) {
    amax = wave_max_u32(amax);
    __shared__ uint32_t red[4];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) red[wave] = amax;
    __syncthreads();
    if (wave == 0) {
      uint32_t m = lane < (int)(blockDim.x >> 6) ? red[lane] : 0u;
      m = wave_max_u32(m);
      if (lane == 0) {
        if (per_image) {
          if (m) atomicMax(absmax_out + b, m);
        } else {
          spread_max(absmax_out, m);
        }
      }
    }
  }
}

// The 2 x 2, stride 2 window on rows of a multiple of 4 floats: a thread
// takes pairs of neighbouring outputs, two 16-byte loads (one per window
// row) each, all issued before any is used.  A block of 1024 threads covers
// up to 4096 pairs of one image (a whole image of the CNN's first pool), so
// a per-image absmax costs one device-scope atomic per block: many blocks
// raising neighbouring slots serialise at the memory side.  Each output takes
// its window in the reference's order (0,0), (0,1), (1,0), (1,1) with the
// same rule as maxpool_kernel, so ties and NaNs resolve alike.
constexpr int kPool2Threads = 1024, kPool2PerThread = 4;

__global__ __launch_bounds__(kPool2Threads) void maxpool2_kernel(const float* __restrict__ x, float* __restrict__ y,
                                                                 uint32_t C, uint32_t H, uint32_t W, uint32_t OH,
                                                                 uint32_t OW, uint32_t pairs, uint32_t* absmax_out,
                                                                 int per_image) {
  const int64_t b = blockIdx.y;
  const uint32_t half = OW >> 1, plane = OH * half;
  uint32_t amax = 0;
  float4 u[kPool2PerThread], v[kPool2PerThread];
  int64_t yo[kPool2PerThread];
  bool ok[kPool2PerThread];
#pragma unroll
  for (int i = 0; i < kPool2PerThread; i++) {
    const uint32_t p = (blockIdx.x * kPool2PerThread + i) * kPool2Threads + threadIdx.x;
    ok[i] = p < pairs;
    const uint32_t q = ok[i] ? p : 0u;
    const uint32_t c = q / plane, r = q - c * plane;
    const uint32_t oy = r / half, ox = (r - oy * half) * 2;
    const float* row0 = x + ((b * C + c) * (int64_t)H + 2 * oy) * (int64_t)W + 2 * ox;
    if (ok[i]) {
      u[i] = *reinterpret_cast<const float4*>(row0);
      v[i] = *reinterpret_cast<const float4*>(row0 + W);
    }
    yo[i] = b * (int64_t)pairs * 2 + (int64_t)c * OH * OW + (int64_t)oy * OW + ox;
  }
#pragma unroll
  for (int i = 0; i < kPool2PerThread; i++) {
    if (!ok[i]) continue;
    float o0 = -__builtin_inff(), o1 = -__builtin_inff();
    o0 = pool_take(o0, u[i].x); o0 = pool_take(o0, u[i].y); o0 = pool_take(o0, v[i].x); o0 = pool_take(o0, v[i].y);
    o1 = pool_take(o1, u[i].z); o1 = pool_take(o1, u[i].w); o1 = pool_take(o1, v[i].z); o1 = pool_take(o1, v[i].w);
    *reinterpret_cast<float2*>(y + yo[i]) = make_float2(o0, o1);
    const uint32_t k0 = rgmath::absmax_key(o0), k1 = rgmath::absmax_key(o1);
    const uint32_t k = k0 > k1 ? k0 : k1;
    amax = k > amax ? k : amax;
  }
  if (absmax_out) {
    __shared__ uint32_t red[kPool2Threads / 64];
    amax = wave_max_u32(amax);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) red[wave] = amax;
    __syncthreads();
    if (wave == 0) {
      uint32_t m = lane < kPool2Threads / 64 ? red[lane] : 0u;
      m = wave_max_u32(m);
      if (lane == 0) {
        if (per_image) {
          if (m) atomicMax(absmax_out + b, m);
        } else {
          spread_max(absmax_out, m);
        }
      }
    }
  }
}

void launch_maxpool(const float* x, float* y, int64_t n, int64_t C, int64_t H, int64_t W, int64_t k, int64_t stride,
                    int64_t OH, int64_t OW, uint32_t* absmax_out, int absmax_per_image, hipStream_t s) {
  const int64_t per = C * OH * OW;
  if (per <= 0 || n <= 0) return;
  if (C * H * W >= ((int64_t)1 << 32) || n > 65535)
    throw std::logic_error("max pool: image or batch too large for the 32-bit kernel indexing");
  if (k == 2 && stride == 2 && W % 4 == 0 && OW * 2 == W && OH * 2 <= H &&
      (reinterpret_cast<uintptr_t>(x) & 15) == 0 && (reinterpret_cast<uintptr_t>(y) & 7) == 0) {
    const int64_t pairs = per / 2, per_block = (int64_t)kPool2Threads * kPool2PerThread;
    RG_LAUNCH(maxpool2_kernel, dim3((unsigned)((pairs + per_block - 1) / per_block), (unsigned)n), dim3(kPool2Threads), 0, s, x, y,
              (uint32_t)C, (uint32_t)H, (uint32_t)W, (uint32_t)OH, (uint32_t)OW, (uint32_t)pairs, absmax_out,
              absmax_per_image);
    return;
  }
  // about 16 outputs per thread, at most 64 blocks per image
  int64_t bx = (per + 256 * 16 - 1) / (256 * 16);
  if (bx > 64) bx = 64;
  const int64_t chunk = (per + bx - 1) / bx;
  bx = (per + chunk - 1) / chunk;
  RG_LAUNCH(maxpool_kernel, dim3((unsigned)bx, (unsigned)n), dim3(256), 0, s, x, y, (uint32_t)C, (uint32_t)H,
               (uint32_t)W, (uint32_t)k, (uint32_t)stride, (uint32_t)OH, (uint32_t)OW, (uint32_t)chunk, absmax_out,
               absmax_per_image);
}

// ---------------------------------------------------------------------------
// standalone activation (npu.rs:395-399)
// ---------------------------------------------------------------------------
template <int ACT>
__device__ __forceinline__ uint32_t activation_loop(const float* __restrict__ x, float* __restrict__ y, int64_t n,
                                                    float p) {
  uint32_t amax = 0;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const float v = act_fixed<ACT>(x[i], p);
    y[i] = v;
    const uint32_t k = rgmath::absmax_key(v);
    amax = k > amax ? k : amax;
  }
  return amax;
}

__global__ __launch_bounds__(256) void activation_kernel(const float* __restrict__ x, float* __restrict__ y, int64_t n,
                                                         int act, float p, uint32_t* absmax_out) {
  uint32_t amax = 0;
  switch (act) {
    case rgmath::ACT_RELU: amax = activation_loop<rgmath::ACT_RELU>(x, y, n, p); break;
    case rgmath::ACT_SIGMOID: amax = activation_loop<rgmath::ACT_SIGMOID>(x, y, n, p); break;
    case rgmath::ACT_TANH: amax = activation_loop<rgmath::ACT_TANH>(x, y, n, p); break;
    case rgmath::ACT_GELU: amax = activation_loop<rgmath::ACT_GELU>(x, y, n, p); break;
    case rgmath::ACT_LEAKY_RELU: amax = activation_loop<rgmath::ACT_LEAKY_RELU>(x, y, n, p); break;
    case rgmath::ACT_SILU: amax = activation_loop<rgmath::ACT_SILU>(x, y, n, p); break;
    default: amax = activation_loop<rgmath::ACT_NONE>(x, y, n, p); break;
  }
  if (absmax_out) {
    amax = wave_max_u32(amax);
    if ((threadIdx.x & 63) == 0) spread_max(absmax_out, amax);
  }
}

void launch_activation(const float* x, float* y, int64_t n, int act, float p, uint32_t* absmax_out, hipStream_t s) {
  if (n <= 0) return;
  int64_t blocks = (n + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  RG_LAUNCH(activation_kernel, dim3((unsigned)blocks), dim3(256), 0, s, x, y, n, act, p, absmax_out);
}

// ---------------------------------------------------------------------------
// softmax_raw (tensor/ops.rs:1058-1076): one thread per row so the f32 sum
// is accumulated in the reference's sequential order.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void softmax_kernel(const float* __restrict__ x, float* __restrict__ y, int64_t outer,
                                                      int64_t size) {
  const int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (o >= outer) return;
  const float* xr = x + o * size;
  float* yr = y + o * size;
  float mx = -__builtin_inff();
  for (int64_t j = 0; j < size; j++) mx = rgmath::fmax_nan_ignoring(mx, xr[j]);
  float s = 0.0f;
  for (int64_t j = 0; j < size; j++) {
    const float d = xr[j] - mx;
    const float e = rgmath::expf_aor(d);
    yr[j] = e;
    s = s + e;
  }
  for (int64_t j = 0; j < size; j++) yr[j] = yr[j] / s;
}

void launch_softmax(const float* x, float* y, int64_t outer, int64_t size, hipStream_t s) {
  if (outer <= 0 || size <= 0) return;
  RG_LAUNCH(softmax_kernel, dim3((unsigned)((outer + 255) / 256)), dim3(256), 0, s, x, y, outer, size);
}

}  // namespace rgnpu
