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
#include <hip/hip_runtime.h>

#include "devmath.h"
#include "rgnpu_internal.h"

namespace rgnpu {

typedef int v4i __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// small helpers
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    uint32_t o = (uint32_t)__shfl_xor((int)v, off, 64);
    v = o > v ? o : v;
  }
  return v;
}

__device__ __forceinline__ int32_t wave_sum_i32(int32_t v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ float slot_scale(const uint32_t* slot) {
  return rgmath::scale_from_absmax(rgmath::bitsf(*slot));
}

template <int ACT>
__device__ __forceinline__ float act_fixed(float x, float p) {
  return rgmath::act_apply(ACT, p, x);
}

// (acc as f32) * cs + bias, then the activation: separate roundings, no FMA
// (quantize.rs:110-111).
template <int ACT>
__device__ __forceinline__ float epi_value(int32_t acc, float cs, float b, float p) {
  const float prod = (float)acc * cs;
  const float val = prod + b;
  return act_fixed<ACT>(val, p);
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
  hipLaunchKernelGGL(fill_u32_kernel, dim3((unsigned)blocks), dim3(256), 0, s, p, n, v);
}

// ---------------------------------------------------------------------------
// absmax: QuantTensor::from_f32's `fold(0, max(|v|))` (quantize.rs:19) as a
// grid reduction.  Non-negative f32 order equals u32 bit order, so a u32
// atomicMax of |v| bits is exact; NaN keys are dropped like f32::max does.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void absmax_kernel(const float* __restrict__ x, int64_t per_img,
                                                     uint32_t* __restrict__ slots,
                                                     const uint8_t* __restrict__ rowmask,
                                                     const uint8_t* __restrict__ colmask, int64_t H,
                                                     int64_t W) {
  const int64_t img = blockIdx.y;
  const float* xi = x + img * per_img;
  uint32_t m = 0;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  if (rowmask) {
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < per_img; e += stride) {
      const int64_t hw = e % (H * W);
      const int64_t iy = hw / W, ix = hw % W;
      if (rowmask[iy] && colmask[ix]) {
        const uint32_t k = rgmath::absmax_key(xi[e]);
        m = k > m ? k : m;
      }
    }
  } else {
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < per_img; e += stride) {
      const uint32_t k = rgmath::absmax_key(xi[e]);
      m = k > m ? k : m;
    }
  }
  m = wave_max_u32(m);
  __shared__ uint32_t red[4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) red[wave] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t r = red[0];
    for (int i = 1; i < (int)(blockDim.x >> 6); i++) r = red[i] > r ? red[i] : r;
    if (r) atomicMax(&slots[img], r);
  }
}

void launch_absmax(const float* x, int64_t per_img, int64_t n_img, uint32_t* slots, const uint8_t* rowmask,
                   const uint8_t* colmask, int64_t H, int64_t W, hipStream_t s) {
  if (per_img <= 0 || n_img <= 0) return;
  int64_t bx = (per_img + 256 * 8 - 1) / (256 * 8);
  if (bx > 2048) bx = 2048;
  if (bx < 1) bx = 1;
  hipLaunchKernelGGL(absmax_kernel, dim3((unsigned)bx, (unsigned)n_img), dim3(256), 0, s, x, per_img, slots, rowmask,
                     colmask, H, W);
}

// ---------------------------------------------------------------------------
// quantize rows: x f32 [M,K] -> q i8 [Mpad,Kpad].  One thread per 4 output
// bytes; padding rows and columns are written as zeros.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void quant_rows_kernel(const float* __restrict__ x, int64_t M, int64_t K,
                                                         int64_t Mpad, int64_t Kpad, const uint32_t* __restrict__ slot,
                                                         int8_t* __restrict__ q, float* scale_out) {
  const float scale = slot_scale(slot);
  const float inv = 1.0f / scale;
  const int64_t words_per_row = Kpad / 4;
  const int64_t total = Mpad * words_per_row;
  for (int64_t w = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; w < total; w += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = w / words_per_row;
    const int64_t c0 = (w % words_per_row) * 4;
    uint32_t packed = 0;
    if (r < M) {
      const float* xr = x + r * K;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int64_t c = c0 + e;
        const int8_t v = c < K ? rgmath::quantize_one(xr[c], inv) : (int8_t)0;
        packed |= (uint32_t)(uint8_t)v << (8 * e);
      }
    }
    reinterpret_cast<uint32_t*>(q)[w] = packed;
  }
  if (scale_out && blockIdx.x == 0 && threadIdx.x == 0) *scale_out = scale;
}

void launch_quant_rows(const float* x, int64_t M, int64_t K, int64_t Mpad, int64_t Kpad, const uint32_t* slot,
                       int8_t* q, float* scale_out, hipStream_t s) {
  const int64_t words = Mpad * (Kpad / 4);
  if (words <= 0) return;
  int64_t blocks = (words + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL(quant_rows_kernel, dim3((unsigned)blocks), dim3(256), 0, s, x, M, K, Mpad, Kpad, slot, q,
                     scale_out);
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
  hipLaunchKernelGGL(quant_images_kernel, dim3((unsigned)bx, (unsigned)n_img), dim3(256), 0, s, x, per_img, slots, q,
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
    if ((threadIdx.x & 63) == 0 && amax)
      atomicMax(ep.absmax_out + (CONV && ep.absmax_out_per_image ? tc.img : 0), amax);
  }
}

// ---------------------------------------------------------------------------
// i8 MFMA GEMM.  Block tile TM x TN, K step 64 bytes, 4 waves in a 2x2 grid,
// each wave owns (TM/2) x (TN/2) built from 16x16 v_mfma_i32_16x16x64_i8
// blocks.  Operands are K-contiguous; LDS rows are padded to 80 bytes so the
// 16 row reads of one MFMA operand fetch hit distinct banks.  Two LDS stages:
// the next K step is loaded to registers while the current one is consumed.
//
// MFMA operand/result layout (16x16x64): lane l supplies row (l%16) of A and
// column (l%16) of B, K bytes [16*(l/16), 16*(l/16)+16); result register r
// of lane l holds D[4*(l/16)+r][l%16].
// ---------------------------------------------------------------------------
constexpr int kTK = 64;
constexpr int kLdsStride = kTK + 16;

template <int TM, int TN>
__global__ __launch_bounds__(256) void gemm_i8_kernel(const int8_t* __restrict__ A, const int8_t* __restrict__ B,
                                                      int64_t M, int64_t N, int64_t Kpad, Epilogue ep) {
  constexpr int STAGE = 2 * (TM + TN) * kLdsStride;
  constexpr int CLD = TN + 4;
  constexpr int EPI = TM * CLD * 4;
  __shared__ __attribute__((aligned(16))) int8_t smem[STAGE > EPI ? STAGE : EPI];
  int8_t* const As = smem;
  int8_t* const Bs = smem + 2 * TM * kLdsStride;
  constexpr int WTM = TM / 2, WTN = TN / 2, FM = WTM / 16, FN = WTN / 16;
  constexpr int A_CH = TM * kTK / 16 / 256, B_CH = TN * kTK / 16 / 256;
  static_assert(A_CH >= 1 && B_CH >= 1, "tile too small");
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t m0 = (int64_t)blockIdx.y * TM, n0 = (int64_t)blockIdx.x * TN;

  v4i acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; i++)
#pragma unroll
    for (int j = 0; j < FN; j++) acc[i][j] = v4i{0, 0, 0, 0};

  // Global -> register -> LDS staging; thread t moves 16-byte chunks
  // (row = c/4, col = 16*(c%4)) of the TM x 64 and TN x 64 tiles.
  v4i ra[A_CH], rb[B_CH];
#pragma unroll
  for (int i = 0; i < A_CH; i++) {
    const int c = tid + i * 256;
    ra[i] = *reinterpret_cast<const v4i*>(A + (m0 + (c >> 2)) * Kpad + (c & 3) * 16);
  }
#pragma unroll
  for (int i = 0; i < B_CH; i++) {
    const int c = tid + i * 256;
    rb[i] = *reinterpret_cast<const v4i*>(B + (n0 + (c >> 2)) * Kpad + (c & 3) * 16);
  }
#pragma unroll
  for (int i = 0; i < A_CH; i++) {
    const int c = tid + i * 256;
    *reinterpret_cast<v4i*>(&As[(c >> 2) * kLdsStride + (c & 3) * 16]) = ra[i];
  }
#pragma unroll
  for (int i = 0; i < B_CH; i++) {
    const int c = tid + i * 256;
    *reinterpret_cast<v4i*>(&Bs[(c >> 2) * kLdsStride + (c & 3) * 16]) = rb[i];
  }
  __syncthreads();

  const int64_t nk = Kpad / kTK;
  const int koff = (lane >> 4) * 16;
  for (int64_t kt = 0; kt < nk; kt++) {
    const int cur = (int)(kt & 1);
    const bool more = kt + 1 < nk;
    if (more) {
      const int64_t k0 = (kt + 1) * kTK;
#pragma unroll
      for (int i = 0; i < A_CH; i++) {
        const int c = tid + i * 256;
        ra[i] = *reinterpret_cast<const v4i*>(A + (m0 + (c >> 2)) * Kpad + k0 + (c & 3) * 16);
      }
#pragma unroll
      for (int i = 0; i < B_CH; i++) {
        const int c = tid + i * 256;
        rb[i] = *reinterpret_cast<const v4i*>(B + (n0 + (c >> 2)) * Kpad + k0 + (c & 3) * 16);
      }
    }
    const int8_t* Ac = As + cur * TM * kLdsStride;
    const int8_t* Bc = Bs + cur * TN * kLdsStride;
    v4i af[FM], bf[FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
      af[i] = *reinterpret_cast<const v4i*>(&Ac[(wm * WTM + i * 16 + (lane & 15)) * kLdsStride + koff]);
#pragma unroll
    for (int j = 0; j < FN; j++)
      bf[j] = *reinterpret_cast<const v4i*>(&Bc[(wn * WTN + j * 16 + (lane & 15)) * kLdsStride + koff]);
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
      for (int j = 0; j < FN; j++)
        acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
    if (more) {
      int8_t* An = As + (cur ^ 1) * TM * kLdsStride;
      int8_t* Bn = Bs + (cur ^ 1) * TN * kLdsStride;
#pragma unroll
      for (int i = 0; i < A_CH; i++) {
        const int c = tid + i * 256;
        *reinterpret_cast<v4i*>(&An[(c >> 2) * kLdsStride + (c & 3) * 16]) = ra[i];
      }
#pragma unroll
      for (int i = 0; i < B_CH; i++) {
        const int c = tid + i * 256;
        *reinterpret_cast<v4i*>(&Bn[(c >> 2) * kLdsStride + (c & 3) * 16]) = rb[i];
      }
    }
    __syncthreads();
  }

  // Stage accumulators in LDS (the stage buffers are free after the barrier).
  int32_t* Cs = reinterpret_cast<int32_t*>(smem);
#pragma unroll
  for (int i = 0; i < FM; i++)
#pragma unroll
    for (int j = 0; j < FN; j++)
#pragma unroll
      for (int r = 0; r < 4; r++)
        Cs[(wm * WTM + i * 16 + (lane >> 4) * 4 + r) * CLD + wn * WTN + j * 16 + (lane & 15)] = acc[i][j][r];
  __syncthreads();
  const float cs = slot_scale(ep.absmax_in) * ep.w_scale;
  const TileCoords tc{m0, n0, M, N, 0};
  epilogue_tile<TM, TN, CLD, false>(Cs, tc, cs, ep);
}

void launch_gemm(const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t Mpad, int64_t Npad, int64_t Kpad,
                 const Epilogue& ep, hipStream_t s) {
  constexpr int TM = 128, TN = 128;
  dim3 grid((unsigned)(Npad / TN), (unsigned)(Mpad / TM));
  hipLaunchKernelGGL((gemm_i8_kernel<TM, TN>), grid, dim3(256), 0, s, A, B, M, N, Kpad, ep);
}

// ---------------------------------------------------------------------------
// GEMV for M <= 8: weight streaming.  Each wave owns R consecutive output
// features; per 1 KiB K chunk every lane loads 16 weight bytes per feature
// (one coalesced 1 KiB read per feature) and 16 activation bytes per row,
// and accumulates with v_dot4_i32_i8.  Lane sums are reduced at the end and
// lane (m*R + r) finishes output (m, n+r).
// ---------------------------------------------------------------------------
constexpr int kGemvR = 4;
constexpr int kGemvMaxM = 8;

template <int MR>
__global__ __launch_bounds__(256) void gemv_i8_kernel(const int8_t* __restrict__ A, const int8_t* __restrict__ B,
                                                      int64_t M, int64_t N, int64_t Npad, int64_t Kpad, Epilogue ep) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t nb = ((int64_t)blockIdx.x * 4 + wave) * kGemvR;
  if (nb >= Npad) return;
  int32_t acc[MR][kGemvR];
#pragma unroll
  for (int m = 0; m < MR; m++)
#pragma unroll
    for (int r = 0; r < kGemvR; r++) acc[m][r] = 0;

  for (int64_t k = (int64_t)lane * 16; k < Kpad; k += 1024) {
    v4i w[kGemvR];
#pragma unroll
    for (int r = 0; r < kGemvR; r++) w[r] = *reinterpret_cast<const v4i*>(B + (nb + r) * Kpad + k);
#pragma unroll
    for (int m = 0; m < MR; m++) {
      if (m < M) {
        const v4i x = *reinterpret_cast<const v4i*>(A + (int64_t)m * Kpad + k);
#pragma unroll
        for (int r = 0; r < kGemvR; r++) {
          int32_t t = acc[m][r];
          t = __builtin_amdgcn_sdot4(x[0], w[r][0], t, false);
          t = __builtin_amdgcn_sdot4(x[1], w[r][1], t, false);
          t = __builtin_amdgcn_sdot4(x[2], w[r][2], t, false);
          t = __builtin_amdgcn_sdot4(x[3], w[r][3], t, false);
          acc[m][r] = t;
        }
      }
    }
  }
  // Reduce; afterwards every lane holds every sum and lane L keeps sum L.
  int32_t mine = 0;
#pragma unroll
  for (int m = 0; m < MR; m++)
#pragma unroll
    for (int r = 0; r < kGemvR; r++) {
      const int32_t t = wave_sum_i32(acc[m][r]);
      if (lane == m * kGemvR + r) mine = t;
    }
  const int64_t m = lane / kGemvR, col = nb + lane % kGemvR;
  const bool ok = lane < MR * kGemvR && m < M && col < N;
  const float cs = slot_scale(ep.absmax_in) * ep.w_scale;
  float v = 0.0f;
  if (ok) {
    const float b = ep.bias[col];
    switch (ep.act) {
      case rgmath::ACT_RELU: v = epi_value<rgmath::ACT_RELU>(mine, cs, b, ep.act_param); break;
      case rgmath::ACT_SIGMOID: v = epi_value<rgmath::ACT_SIGMOID>(mine, cs, b, ep.act_param); break;
      case rgmath::ACT_TANH: v = epi_value<rgmath::ACT_TANH>(mine, cs, b, ep.act_param); break;
      case rgmath::ACT_GELU: v = epi_value<rgmath::ACT_GELU>(mine, cs, b, ep.act_param); break;
      case rgmath::ACT_LEAKY_RELU: v = epi_value<rgmath::ACT_LEAKY_RELU>(mine, cs, b, ep.act_param); break;
      case rgmath::ACT_SILU: v = epi_value<rgmath::ACT_SILU>(mine, cs, b, ep.act_param); break;
      default: v = epi_value<rgmath::ACT_NONE>(mine, cs, b, ep.act_param); break;
    }
    ep.y[m * N + col] = v;
    if (ep.acc_out) ep.acc_out[m * N + col] = mine;
  }
  if (ep.absmax_out) {
    const uint32_t amax = wave_max_u32(ok ? rgmath::absmax_key(v) : 0u);
    if (lane == 0 && amax) atomicMax(ep.absmax_out, amax);
  }
}

void launch_gemv(const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t Npad, int64_t Kpad,
                 const Epilogue& ep, hipStream_t s) {
  const int64_t waves = Npad / kGemvR;
  const int64_t blocks = (waves + 3) / 4;
  hipLaunchKernelGGL((gemv_i8_kernel<kGemvMaxM>), dim3((unsigned)blocks), dim3(256), 0, s, A, B, M, N, Npad, Kpad,
                     ep);
}

// ---------------------------------------------------------------------------
// Implicit-GEMM conv.  MFMA "A" = weights [Opad, Kpad] (TM output channels),
// "B" = im2col columns of one image (TN output pixels), so D[o][l] maps onto
// the NCHW output with pixels contiguous.  The B tile is gathered from the
// quantized image while it is written to LDS; out-of-image taps and K padding
// are zeros.  Each of the 4 waves owns all TM channels x TN/4 pixels.
// ---------------------------------------------------------------------------
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
  const int64_t L = cs.OH * cs.OW, KK = cs.C * cs.k * cs.k, kk2 = cs.k * cs.k;
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
  const int64_t oy = pix / cs.OW, ox = pix % cs.OW;
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
        const int64_t kk = k0 + gk + w4 * 4 + e;
        int8_t v = 0;
        if (pix_ok && kk < KK) {
          const int64_t ch = kk / kk2, rem = kk % kk2;
          const int64_t ki = rem / cs.k, kj = rem % cs.k;
          const int64_t iy = oy * cs.stride + ki - cs.pad, ix = ox * cs.stride + kj - cs.pad;
          if (iy >= 0 && iy < cs.H && ix >= 0 && ix < cs.W) v = img[(ch * cs.H + iy) * cs.W + ix];
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

void launch_conv(const int8_t* xq, const int8_t* Wq, const ConvShape& cs, const Epilogue& ep, hipStream_t s) {
  constexpr int TN = 128;
  const int64_t L = cs.OH * cs.OW;
  const unsigned gx = (unsigned)((L + TN - 1) / TN);
  if (cs.Opad % 64 == 0) {
    dim3 grid(gx, (unsigned)(cs.Opad / 64), (unsigned)cs.n);
    hipLaunchKernelGGL((conv_i8_kernel<64, TN>), grid, dim3(256), 0, s, xq, Wq, cs, ep);
  } else {
    dim3 grid(gx, (unsigned)(cs.Opad / 32), (unsigned)cs.n);
    hipLaunchKernelGGL((conv_i8_kernel<32, TN>), grid, dim3(256), 0, s, xq, Wq, cs, ep);
  }
}

// ---------------------------------------------------------------------------
// Max pool: window scan in (ki, kj) order from -inf with `v > best || NaN`
// (kernels.rs:180-191), so NaN propagates and ties keep the first element.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void maxpool_kernel(const float* __restrict__ x, float* __restrict__ y, int64_t C,
                                                      int64_t H, int64_t W, int64_t k, int64_t st, int64_t OH,
                                                      int64_t OW, uint32_t* absmax_out, int per_image) {
  const int64_t b = blockIdx.y;
  const int64_t per = C * OH * OW;
  uint32_t amax = 0;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < per; e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t c = e / (OH * OW), rem = e % (OH * OW);
    const int64_t oy = rem / OW, ox = rem % OW;
    const float* plane = x + (b * C + c) * H * W;
    float best = -__builtin_inff();
    for (int64_t ki = 0; ki < k; ki++)
      for (int64_t kj = 0; kj < k; kj++) {
        const float v = plane[(oy * st + ki) * W + ox * st + kj];
        if (v > best || v != v) best = v;
      }
    y[b * per + e] = best;
    const uint32_t kk = rgmath::absmax_key(best);
    amax = kk > amax ? kk : amax;
  }
  if (absmax_out) {
    amax = wave_max_u32(amax);
    if ((threadIdx.x & 63) == 0 && amax) atomicMax(absmax_out + (per_image ? b : 0), amax);
  }
}

void launch_maxpool(const float* x, float* y, int64_t n, int64_t C, int64_t H, int64_t W, int64_t k, int64_t stride,
                    int64_t OH, int64_t OW, uint32_t* absmax_out, int absmax_per_image, hipStream_t s) {
  const int64_t per = C * OH * OW;
  if (per <= 0 || n <= 0) return;
  int64_t bx = (per + 255) / 256;
  if (bx > 1024) bx = 1024;
  hipLaunchKernelGGL(maxpool_kernel, dim3((unsigned)bx, (unsigned)n), dim3(256), 0, s, x, y, C, H, W, k, stride, OH,
                     OW, absmax_out, absmax_per_image);
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
    if ((threadIdx.x & 63) == 0 && amax) atomicMax(absmax_out, amax);
  }
}

void launch_activation(const float* x, float* y, int64_t n, int act, float p, uint32_t* absmax_out, hipStream_t s) {
  if (n <= 0) return;
  int64_t blocks = (n + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(activation_kernel, dim3((unsigned)blocks), dim3(256), 0, s, x, y, n, act, p, absmax_out);
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
  hipLaunchKernelGGL(softmax_kernel, dim3((unsigned)((outer + 255) / 256)), dim3(256), 0, s, x, y, outer, size);
}

}  // namespace rgnpu
