// requant.hip — the next Linear's activation quantization fused into the
// producing Linear's GEMM (Linear -> Linear on the INT8 path).
//
// NpuProgram::execute quantizes every Linear's input per tensor (npu.rs:312,
// QuantTensor::from_f32, quantize.rs:18-24): the scale is absmax/127 over
// the previous layer's whole f32 output, so no tile of that output can be
// quantized before every tile of it exists.  This kernel runs the producing
// GEMM as a persistent grid: G workgroups, all resident at once, each walking
// tiles b, b + G, ... with the fused dequant/bias/activation epilogue of
// quantize.rs:109-111.  Each raises the spread absmax slot of its outputs,
// then the grid meets at a barrier; after it the absmax is final and every
// workgroup quantizes its own tiles into the next layer's i8 operand: its last
// tile straight from the registers that hold its activations, earlier tiles
// from the f32 outputs they stored.  The separate pass that re-read the whole
// f32 output (and its launch) is gone, and the f32 output of the last tile of
// each workgroup is not written at all unless a capture asks for it.
//
// The barrier wait is bounded.  On an otherwise idle device the G <= occupancy
// workgroups are resident together, but a kernel on another stream may hold
// CUs.  A workgroup that has polled spin_limit times (about 1 us each)
// stores its last tile's f32 outputs, marks itself deferred and exits; the
// workgroup whose arrival completed the barrier (the finisher) waits for
// every workgroup to settle (they are all running, so this is short) and
// quantizes the deferred workgroups' tiles from memory.  No wait is
// unbounded, so two such kernels can never deadlock each other.
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <stdexcept>

#include "devmath.h"
#include "gemm_core.h"
#include "rgnpu_internal.h"

namespace rgnpu {

namespace rqk {
constexpr uint32_t kOwn = 1, kDeferred = 2;
constexpr int kFinisherExtraPolls = 20000;  // settle budget of the finisher beyond spin_limit
}  // namespace rqk

// One wave's (16 FM) x 64 tile of the fused epilogue, staged through the
// wave's LDS slab 16 rows at a time.  Lane l takes the 4 consecutive columns
// col0 .. col0 + 3 (col0 = n0 + wn 64 + 4 (l & 15)) of rows 4 p + (l >> 4),
// p = 0..3, of each slab, so its f32 stores are 16 bytes and its 4 quantized
// bytes form one word.  The activations are left in acc[i][p] (f32 bits) in
// that layout.  Returns the max |y| over the valid outputs (NaN ignored, like
// f32::max); columns past N (zero weights, zero bias) are not outputs.
template <int ACT, int FM>
__device__ __forceinline__ float requant_epilogue(int8_t* smem, v4i (&acc)[FM][4], int64_t row0, int64_t col0,
                                                  int64_t M, int64_t N, float cs, const float4 b4, const Epilogue& ep,
                                                  bool store, bool vec, int wave, int lane) {
  int32_t* slab = reinterpret_cast<int32_t*>(smem + wave * big::SLAB);
  const int sub = lane >> 4, c4 = (lane & 15) * 4;
  const float bb[4] = {b4.x, b4.y, b4.z, b4.w};
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < FM; i++) {
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int r = 0; r < 4; r++) slab[((lane >> 4) * 4 + r) * big::SLAB_LD + j * 16 + (lane & 15)] = acc[i][j][r];
#pragma unroll
    for (int p = 0; p < 4; p++) {
      const int rr = p * 4 + sub;
      const v4i a = *reinterpret_cast<const v4i*>(slab + rr * big::SLAB_LD + c4);
      const int64_t row = row0 + i * 16 + rr;
      v4f v;
#pragma unroll
      for (int c = 0; c < 4; c++) v[c] = epi_value<ACT>(a[c], cs, bb[c], ep.act_param);
      if (row < M) {
        float* yr = ep.y + row * N + col0;
        if (vec && col0 + 4 <= N) {
          if (store) *reinterpret_cast<v4f*>(yr) = v;
#pragma unroll
          for (int c = 0; c < 4; c++) amax = __builtin_fmaxf(amax, __builtin_fabsf(v[c]));
        } else {
#pragma unroll
          for (int c = 0; c < 4; c++)
            if (col0 + c < N) {
              if (store) yr[c] = v[c];
              amax = __builtin_fmaxf(amax, __builtin_fabsf(v[c]));
            }
        }
        if (ep.acc_out) {
#pragma unroll
          for (int c = 0; c < 4; c++)
            if (col0 + c < N) ep.acc_out[row * N + col0 + c] = a[c];
        }
      }
      acc[i][p] = __builtin_bit_cast(v4i, v);
    }
  }
  return amax;
}

// Stores the activations requant_epilogue left in acc as f32 (a workgroup
// that defers its quantization leaves them for the finisher).
template <int FM>
__device__ __forceinline__ void store_kept_f32(const v4i (&acc)[FM][4], float* y, int64_t row0, int64_t col0,
                                               int64_t M, int64_t N, bool vec, int lane) {
  const int sub = lane >> 4;
#pragma unroll
  for (int i = 0; i < FM; i++)
#pragma unroll
    for (int p = 0; p < 4; p++) {
      const int64_t row = row0 + i * 16 + p * 4 + sub;
      if (row >= M) continue;
      const v4f v = __builtin_bit_cast(v4f, acc[i][p]);
      float* yr = y + row * N + col0;
      if (vec && col0 + 4 <= N) {
        *reinterpret_cast<v4f*>(yr) = v;
      } else {
#pragma unroll
        for (int c = 0; c < 4; c++)
          if (col0 + c < N) yr[c] = v[c];
      }
    }
}

// Four quantized bytes of row `row`, columns col0 .. col0 + 3; positions
// outside [0, M) x [0, N) are the zero padding of the next operand.
__device__ __forceinline__ uint32_t quant_word(v4f v, int64_t row, int64_t col0, int64_t M, int64_t N, float inv) {
  uint32_t w = 0;
  if (row < M) {
#pragma unroll
    for (int c = 0; c < 4; c++)
      if (col0 + c < N) w |= (uint32_t)(uint8_t)rgmath::quantize_one(v[c], inv) << (8 * c);
  }
  return w;
}

// Quantizes the activations kept in acc (requant_epilogue layout) into
// q [.., ldq].  Columns at or past ldq (the producer's Npad may exceed the
// consumer's Kpad) are not part of the operand.
template <int FM>
__device__ __forceinline__ void quantize_kept(const v4i (&acc)[FM][4], int8_t* q, int64_t ldq, int64_t row0,
                                              int64_t col0, int64_t M, int64_t N, float inv, int lane) {
  if (col0 >= ldq) return;
  const int sub = lane >> 4;
#pragma unroll
  for (int i = 0; i < FM; i++)
#pragma unroll
    for (int p = 0; p < 4; p++) {
      const int64_t row = row0 + i * 16 + p * 4 + sub;
      *reinterpret_cast<uint32_t*>(q + row * ldq + col0) =
          quant_word(__builtin_bit_cast(v4f, acc[i][p]), row, col0, M, N, inv);
    }
}

// Quantizes one wave's (16 FM) x 64 part of a tile from its stored f32
// outputs, in the same lane layout.
template <int FM>
__device__ __forceinline__ void quantize_stored(const float* y, int8_t* q, int64_t ldq, int64_t row0, int64_t col0,
                                                int64_t M, int64_t N, float inv, bool vec, int lane) {
  if (col0 >= ldq) return;
  const int sub = lane >> 4;
#pragma unroll
  for (int i = 0; i < FM; i++) {
    v4f v[4];
#pragma unroll
    for (int p = 0; p < 4; p++) {
      const int64_t row = row0 + i * 16 + p * 4 + sub;
      v[p] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
      if (row < M) {
        const float* yr = y + row * N + col0;
        if (vec && col0 + 4 <= N) {
          v[p] = *reinterpret_cast<const v4f*>(yr);
        } else {
#pragma unroll
          for (int c = 0; c < 4; c++)
            if (col0 + c < N) v[p][c] = yr[c];
        }
      }
    }
#pragma unroll
    for (int p = 0; p < 4; p++) {
      const int64_t row = row0 + i * 16 + p * 4 + sub;
      *reinterpret_cast<uint32_t*>(q + row * ldq + col0) = quant_word(v[p], row, col0, M, N, inv);
    }
  }
}

template <int BM, int BN, int WAVES_M, int WAVES_N, int STAGES, int OCC, int FM, int ACT>
__global__ __launch_bounds__(WAVES_M * WAVES_N * 64, OCC) void gemm_requant_kernel(
    const int8_t* __restrict__ A, const int8_t* __restrict__ B, int64_t M, int64_t N, int64_t Kpad, int tiles_m,
    int tiles_n, Epilogue ep, Requant rq) {
  using namespace big;
  constexpr int NW = WAVES_M * WAVES_N;
  static_assert(BM == 16 * FM * WAVES_M && BN == 64 * WAVES_N, "wave tile is (16 FM) x 64");
  constexpr int ST = (BM + BN) * BK;
  static_assert(NW * SLAB <= STAGES * ST, "epilogue slabs reuse the ring");
  __shared__ __attribute__((aligned(1024))) int8_t smem[STAGES * ST];
  __shared__ uint32_t s_flag, s_ndef;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  const int T = tiles_m * tiles_n, G = (int)gridDim.x, b = (int)blockIdx.x;
  const int ntile = (T - b + G - 1) / G;  // >= 1: the grid never exceeds the tile count
  const int nk = (int)(Kpad / BK);
  const int64_t wrow = (int64_t)wm * 16 * FM, wcol = (int64_t)wn * 64 + 4 * (lane & 15);
  const bool vec = (N & 3) == 0 && (reinterpret_cast<uintptr_t>(ep.y) & 15) == 0;
  // partial of the input absmax, folded after the first K loop
  const uint32_t absmax_part = tensor_absmax_part(ep.absmax_in);
  float cs = 0.0f, amax = 0.0f;
  int64_t m0 = 0, n0 = 0;
  v4i acc[FM][4];
  for (int it = 0; it < ntile; it++) {
    int tm, tn;
    tile_coords(b + it * G, tiles_m, tiles_n, tm, tn);
    m0 = (int64_t)tm * BM;
    n0 = (int64_t)tn * BN;
    const float4 b4 = *reinterpret_cast<const float4*>(ep.bias + n0 + wcol);  // bias is padded to Npad
    if (it > 0) {
      // the previous epilogue's slabs live in the ring the K loop refills
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
    }
    big_kloop<BM, BN, WAVES_M, WAVES_N, STAGES, FM, kModeI8>(smem, A, B, Kpad, m0, n0, 0, nk, wave, wm, wn, lane,
                                                             acc);
    if (it == 0) cs = rgmath::scale_from_absmax(rgmath::bitsf(wave_max_u32(absmax_part))) * ep.w_scale;
    const bool store = it + 1 < ntile || rq.keep_f32;
    const float t = requant_epilogue<ACT, FM>(smem, acc, m0 + wrow, n0 + wcol, M, N, cs, b4, ep, store, vec, wave,
                                              lane);
    amax = __builtin_fmaxf(amax, t);
  }

  // Publish this workgroup's absmax, then arrive.  The release fence orders
  // the absmax atomics and the f32 stores above before the arrival.
  {
    const uint32_t m = wave_max_u32(rgmath::fbits(amax));
    if (lane == 0) spread_max(ep.absmax_out, m);
  }
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(rq.sync, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
    uint32_t flag = prev + 1 == (uint32_t)G ? 2u : 0u;  // 2: this arrival completed the barrier
    for (int k = 0; flag == 0 && k < rq.spin_limit; k++) {
      __builtin_amdgcn_s_sleep(32);
      if (__hip_atomic_load(rq.sync, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT) >= (uint32_t)G) flag = 1;
    }
    s_flag = flag;
  }
  __syncthreads();
  const uint32_t flag = s_flag;
  if (flag == 0) {
    // Waited too long: the finisher quantizes this workgroup's tiles.
    if (!rq.keep_f32) store_kept_f32<FM>(acc, ep.y, m0 + wrow, n0 + wcol, M, N, vec, lane);
    __threadfence();
    __syncthreads();
    if (tid == 0)
      __hip_atomic_store(rq.sync + kRequantStateBase + b, rqk::kDeferred, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  __threadfence();  // acquire: every workgroup's absmax partials and stores
  if (tid == 0)
    __hip_atomic_store(rq.sync + kRequantStateBase + b, rqk::kOwn, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const uint32_t part =
      __hip_atomic_load(ep.absmax_out + lane * kSpreadStride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const float scale = rgmath::scale_from_absmax(rgmath::bitsf(wave_max_u32(part)));
  const float inv = 1.0f / scale;
  // earlier tiles from their stored outputs, the last one from registers
  for (int it = 0; it + 1 < ntile; it++) {
    int tm, tn;
    tile_coords(b + it * G, tiles_m, tiles_n, tm, tn);
    quantize_stored<FM>(ep.y, rq.q, rq.ldq, (int64_t)tm * BM + wrow, (int64_t)tn * BN + wcol, M, N, inv, vec, lane);
  }
  quantize_kept<FM>(acc, rq.q, rq.ldq, m0 + wrow, n0 + wcol, M, N, inv, lane);
  if (flag != 2) return;

  // Finisher: the scale tap, then the tiles of every deferred workgroup.
  if (tid == 0 && rq.scale_out) *rq.scale_out = scale;
  uint32_t* list = reinterpret_cast<uint32_t*>(smem);  // the ring is free: no K loop follows
  if (tid == 0) s_ndef = 0;
  __syncthreads();
  for (int w = tid; w < G; w += blockDim.x) {
    uint32_t st = 0;
    for (int k = 0; k < rq.spin_limit + rqk::kFinisherExtraPolls; k++) {
      st = __hip_atomic_load(rq.sync + kRequantStateBase + w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (st != 0) break;
      __builtin_amdgcn_s_sleep(32);
    }
    if (st == 0) __hip_atomic_store(rq.sync + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (st == rqk::kDeferred) list[atomicAdd(&s_ndef, 1u)] = (uint32_t)w;
  }
  __threadfence();  // acquire: the deferred workgroups' stored outputs
  __syncthreads();
  const int ndef = (int)s_ndef;
  for (int d = 0; d < ndef; d++) {
    const int w = (int)list[d];
    const int wt = (T - w + G - 1) / G;
    for (int it = 0; it < wt; it++) {
      int tm, tn;
      tile_coords(w + it * G, tiles_m, tiles_n, tm, tn);
      quantize_stored<FM>(ep.y, rq.q, rq.ldq, (int64_t)tm * BM + wrow, (int64_t)tn * BN + wcol, M, N, inv, vec,
                          lane);
    }
  }
}

template <int BM, int BN, int WAVES_M, int WAVES_N, int STAGES, int OCC, int FM, int ACT>
static void launch_requant_act(const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t Mpad, int64_t Npad,
                               int64_t Kpad, const Epilogue& ep, const Requant& rq, hipStream_t s) {
  constexpr int threads = WAVES_M * WAVES_N * 64;
  const void* fn = reinterpret_cast<const void*>(&gemm_requant_kernel<BM, BN, WAVES_M, WAVES_N, STAGES, OCC, FM, ACT>);
  static const int64_t cap = resident_blocks(fn, threads);
  const int tm = (int)(Mpad / BM), tn = (int)(Npad / BN);
  const int64_t T = (int64_t)tm * tn;
  const int64_t G = T < cap ? T : cap;
  if (G > requant_sync_words(Mpad, Npad, Kpad) - kRequantStateBase)
    throw std::logic_error("requant: more workgroups than sync words");
  RG_LAUNCH((gemm_requant_kernel<BM, BN, WAVES_M, WAVES_N, STAGES, OCC, FM, ACT>), dim3((unsigned)G), dim3(threads), 0,
            s, A, B, M, N, Kpad, tm, tn, ep, rq);
}

template <int BM, int BN, int WAVES_M, int WAVES_N, int STAGES, int OCC, int FM>
static void launch_requant_shape(const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t Mpad, int64_t Npad,
                                 int64_t Kpad, const Epilogue& ep, const Requant& rq, hipStream_t s) {
#define RG_RQ(ACTV) \
  launch_requant_act<BM, BN, WAVES_M, WAVES_N, STAGES, OCC, FM, ACTV>(A, B, M, N, Mpad, Npad, Kpad, ep, rq, s)
  switch (ep.act) {
    case rgmath::ACT_RELU: RG_RQ(rgmath::ACT_RELU); break;
    case rgmath::ACT_SIGMOID: RG_RQ(rgmath::ACT_SIGMOID); break;
    case rgmath::ACT_TANH: RG_RQ(rgmath::ACT_TANH); break;
    case rgmath::ACT_GELU: RG_RQ(rgmath::ACT_GELU); break;
    case rgmath::ACT_LEAKY_RELU: RG_RQ(rgmath::ACT_LEAKY_RELU); break;
    case rgmath::ACT_SILU: RG_RQ(rgmath::ACT_SILU); break;
    default: RG_RQ(rgmath::ACT_NONE); break;
  }
#undef RG_RQ
}

bool gemm_requant_supported(int64_t Mpad, int64_t Npad, int64_t Kpad) {
  if (Kpad % big::BK || Mpad % 128 || Npad % 128 || Kpad <= 0) return false;
  return choose_gemm(Mpad, Npad, Kpad).splits == 1;
}

int64_t requant_sync_words(int64_t Mpad, int64_t Npad, int64_t Kpad) {
  // the grid never exceeds the tile count or two workgroups per CU of 256
  const GemmChoice g = choose_gemm(Mpad, Npad, Kpad);
  const int64_t bm = g.kind == 2 ? 128 : 256, bn = g.kind == 0 ? 256 : 128;
  int64_t T = (Mpad / bm) * (Npad / bn);
  if (T > 4096) T = 4096;
  return round_up(kRequantStateBase + T, 32);
}

void launch_gemm_requant(const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t Mpad, int64_t Npad,
                         int64_t Kpad, const Epilogue& ep, const Requant& rq, hipStream_t s) {
  if (!gemm_requant_supported(Mpad, Npad, Kpad)) throw std::logic_error("requant: the GEMM must be unsplit");
  if (!ep.absmax_out || !rq.q || !rq.sync || rq.ldq <= 0 || rq.ldq > Npad || rq.ldq % 16)
    throw std::logic_error("requant: absmax slot, operand and sync words are required");
  if (M <= 0) return;
  const GemmChoice g = choose_gemm(Mpad, Npad, Kpad);
  if (g.kind == 0)
    launch_requant_shape<256, 256, 2, 4, 4, 1, 8>(A, B, M, N, Mpad, Npad, Kpad, ep, rq, s);
  else if (g.kind == 1)
    launch_requant_shape<256, 128, 2, 2, 3, 2, 8>(A, B, M, N, Mpad, Npad, Kpad, ep, rq, s);
  else
    launch_requant_shape<128, 128, 2, 2, 4, 2, 4>(A, B, M, N, Mpad, Npad, Kpad, ep, rq, s);
}

}  // namespace rgnpu
