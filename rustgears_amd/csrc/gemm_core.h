// gemm_core.h -- device code shared by the HIP translation units of the
// MI355X provider: vector types, the launch macro, absmax-slot and epilogue
// helpers, and the large MFMA GEMM's tile order and K loop.  Included by
// kernels.hip and requant.hip only.
#pragma once
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include "devmath.h"
#include "rgnpu_internal.h"

namespace rgnpu {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));

// The stop event for the next launch while a launch-event sink is set on this
// thread (set_launch_events), else null.
hipEvent_t next_launch_event();

#define RG_LAUNCH(kernel, grid, block, shmem, stream, ...)                                                   \
  do {                                                                                                     \
    hipEvent_t rg_ev_ = next_launch_event();                                                               \
    if (rg_ev_) {                                                                                          \
      hipExtLaunchKernelGGL(kernel, grid, block, shmem, stream, nullptr, rg_ev_, 0, __VA_ARGS__);          \
    } else {                                                                                               \
      hipLaunchKernelGGL(kernel, grid, block, shmem, stream, __VA_ARGS__);                                 \
    }                                                                                                      \
  } while (0)

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

// Zeroes the other run's slot set (the plan's slots are double-buffered by
// run parity and the first kernel of a run clears the set the next run
// uses).  Every thread of the grid takes a share.
__device__ __forceinline__ void clear_slots(const SlotClear& c) {
  if (!c.p) return;
  const int64_t nthreads = (int64_t)gridDim.x * gridDim.y * blockDim.x;
  for (int64_t i = ((int64_t)blockIdx.y * gridDim.x + blockIdx.x) * blockDim.x + threadIdx.x; i < c.n; i += nthreads)
    c.p[i] = 0u;
}

__device__ __forceinline__ float slot_scale(const uint32_t* slot) {
  return rgmath::scale_from_absmax(rgmath::bitsf(*slot));
}

// Per-tensor absmax from a spread slot: every lane loads one partial and the
// wave folds them.  All 64 lanes of the wave must be active for the fold.
__device__ __forceinline__ uint32_t tensor_absmax_part(const uint32_t* slot) {
  static_assert(kSpread == 64, "one partial per lane");
  return slot[(threadIdx.x & 63) * kSpreadStride];
}

__device__ __forceinline__ uint32_t tensor_absmax_bits(const uint32_t* slot) {
  return wave_max_u32(tensor_absmax_part(slot));
}

__device__ __forceinline__ float tensor_scale(const uint32_t* slot) {
  return rgmath::scale_from_absmax(rgmath::bitsf(tensor_absmax_bits(slot)));
}

// Raise the partial of a spread slot that belongs to this wave (linear
// wave index over the whole grid, modulo kSpread).
__device__ __forceinline__ void spread_max(uint32_t* slot, uint32_t v) {
  const uint32_t block = (blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x;
  const uint32_t part = (block * (blockDim.x >> 6) + (threadIdx.x >> 6)) & (kSpread - 1);
  if (v) atomicMax(slot + part * kSpreadStride, v);
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

// Operand modes of the MFMA GEMM and the GEMV: i8 (NpuPrecision::Int8),
// binary16 (NpuPrecision::Fp16) and f32 (the standard FP32 path).
constexpr int kModeI8 = 0, kModeF16 = 1, kModeF32 = 2;

// One accumulator word to its output.  INT8: the i32 sum, y = act(fl(float(acc)
// * cs) + b).  FP16: the bits of the f32 sum, y = act(round_fp16(acc + b))
// (npu.rs:442).  FP32: y = act(acc + b) (mod.rs:267-272: matmul, then bias).
template <int ACT, int MODE>
__device__ __forceinline__ float epi_word(int32_t w, float cs, float b, float p) {
  if constexpr (MODE == kModeF16) {
    const float t = __int_as_float(w) + b;
    return act_fixed<ACT>(rgmath::round_fp16(t), p);
  } else if constexpr (MODE == kModeF32) {
    return act_fixed<ACT>(__int_as_float(w) + b, p);
  } else {
    return epi_value<ACT>(w, cs, b, p);
  }
}

// ---------------------------------------------------------------------------
// MFMA operand/result layout (v_mfma_i32_16x16x64_i8): lane l supplies row
// (l%16) of A and column (l%16) of B, K bytes [16*(l/16), 16*(l/16)+16);
// result register r of lane l holds D[4*(l/16)+r][l%16].
// ---------------------------------------------------------------------------
constexpr int kTK = 64;
constexpr int kLdsStride = kTK + 16;

// ---------------------------------------------------------------------------
// Large-problem i8 GEMM.
//
// Every wave owns a 128 x 64 output tile built from 8 x 4
// v_mfma_i32_16x16x64_i8 blocks (128 accumulator registers, two waves per
// SIMD).  A block tile is BM x BN from WAVES_M x WAVES_N waves, K step 64
// bytes.  Two shapes are used: 256 x 128 (4 waves, two workgroups per CU)
// and 256 x 256 (8 waves, one workgroup per CU), which moves a third fewer
// operand bytes per MAC and leaves LDS for a deeper ring.
//
// Operand tiles move global -> LDS with global_load_lds_dwordx4 (no VGPR
// staging) through a STAGES-deep ring: the loads for steps k+1 .. k+STAGES-1
// are in flight while step k is consumed.  Each DMA instruction fills 1 KiB
// = 16 rows x 64 bytes; lane i lands at byte 16*i, so the XOR swizzle of
// 16-byte chunks (chunk ^ ((row >> 1) & 3)) is applied by choosing which
// global chunk each lane fetches.  With that swizzle the MFMA operand reads
// (16 rows, one chunk) are bank-conflict free on gfx950.  The stage barrier
// is a raw s_barrier: each wave first waits for its own DMA loads (vmcnt),
// so no fence-induced vmcnt(0) drains the pipeline.
//
// Tiles are ordered so the workgroups resident on one XCD (hardware deals
// workgroups round-robin over the 8 XCDs) cover a compact group of GROUP_M
// M-tiles, which keeps their A and B panels in that XCD's L2.
// ---------------------------------------------------------------------------
#define RG_LDS_AS __attribute__((address_space(3)))

namespace big {
constexpr int BK = 64;
constexpr int SLAB_LD = 68;  // i32 words per staged epilogue row (64 + 4 pad)
constexpr int SLAB = 16 * SLAB_LD * 4;
constexpr int GROUP_M = 8;
}  // namespace big

// Workgroups of `threads` threads of `fn` that are resident on the current
// device at once.
inline int64_t resident_blocks(const void* fn, int threads = 256) {
  int dev = 0, cus = 0, per_cu = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    cus = 256;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, threads, 0) != hipSuccess || per_cu <= 0) per_cu = 1;
  return (int64_t)per_cu * cus;
}

// XCD-aware, M-grouped tile order: hardware deals workgroups round-robin
// over the 8 XCDs, so tile index t runs on XCD t & 7; the tiles of one XCD
// are numbered contiguously (L) and walk groups of GROUP_M M-tiles, which
// keeps their A and B panels in that XCD's L2.
__device__ __forceinline__ void tile_coords(int t, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int total = tiles_m * tiles_n;
  const int xcd = t & 7, local = t >> 3;
  const int q = total >> 3, rem = total & 7;
  const int L = (xcd < rem ? xcd * (q + 1) : rem * (q + 1) + (xcd - rem) * q) + local;
  const int group_span = big::GROUP_M * tiles_n;
  const int group = L / group_span;
  const int first_m = group * big::GROUP_M;
  const int gsize = min(tiles_m - first_m, big::GROUP_M);
  const int in_group = L - group * group_span;
  tm = first_m + in_group % gsize;
  tn = in_group / gsize;
}

// One global_load_lds_dwordx4: 16 bytes per lane, lane i lands at lds + 16 i
// (the LDS address is wave-uniform).  Kept out of the kernel templates: the
// LDS address-space cast does not survive the host compilation pass of a
// template body, which would silently drop the kernel's host stub.
__device__ __forceinline__ void dma16(const int8_t* g, int8_t* lds) {
  __builtin_amdgcn_global_load_lds(g, (RG_LDS_AS void*)lds, 16, 0, 0);
}

// s_waitcnt vmcnt(N) for a compile-time N (gfx9 encoding: vmcnt bits 3:0 and
// 15:14, expcnt and lgkmcnt left at their no-wait maxima).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

__device__ __forceinline__ int lds_swz(int r) { return (r >> 1) & 3; }

// Masked stores without branches: raw buffer stores over a wave-uniform
// base with a record limit of 2^31 bytes; an element outside the output gets
// the per-lane offset 2^31, which the hardware's bounds check drops, and a
// row offset can travel in the scalar offset.
constexpr uint32_t kDropOffset = 0x80000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t bounded_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)kDropOffset, 0x00020000);
}

// Raw buffer resource over base (gfx9 word 3: 32-bit data format); the
// record count is left at its maximum, so no store is clipped.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t raw_rsrc(void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(base, 0, -1, 0x00020000);
}

// The K loop shared by the large GEMM kernels: block tile (m0, n0) of BM x BN
// from WAVES_M x WAVES_N waves, K steps [kbeg, kbeg + nk) of 64 bytes, into
// acc (zeroed here).  Ends with every wave's DMA and LDS traffic drained and
// a barrier, so the ring may be reused (epilogue slabs, the next tile).
//
// F16 (NpuPrecision::Fp16): A and B hold IEEE binary16 values, a K step of
// 64 bytes is 32 of them and one v_mfma_f32_16x16x32_f16 per 16 x 16 block,
// whose per-lane operand layout matches the i8 instruction's byte for byte,
// so the DMA ring, swizzle and LDS reads are shared.  The f32 sums travel in
// the same 32-bit accumulator words.
template <int BM, int BN, int WAVES_M, int WAVES_N, int STAGES, int FM, int MODE>
__device__ __forceinline__ void big_kloop(int8_t* smem, const int8_t* __restrict__ A, const int8_t* __restrict__ B,
                                          int64_t Kpad, int64_t m0, int64_t n0, int kbeg, int nk, int wave, int wm,
                                          int wn, int lane, v4i (&acc)[FM][4]) {
  using namespace big;
  constexpr int NW = WAVES_M * WAVES_N;
  constexpr int IA = BM / 16 / NW, IB = BN / 16 / NW;  // DMA instructions per wave per stage
  static_assert(IA * 16 * NW == BM && IB * 16 * NW == BN && IA >= 1 && IB >= 1, "DMA split");
  static_assert(STAGES >= 3, "ring depth");
  constexpr int A_ST = BM * BK, ST = (BM + BN) * BK;
  // DMA addressing: uniform tile base pointers plus 32-bit per-lane offsets.
  // Wave w fills A rows [16 IA w, 16 IA (w+1)) and B rows [16 IB w, ...).
  const uint32_t kp = (uint32_t)Kpad;
  const int8_t* const abase = A + m0 * Kpad;
  const int8_t* const bbase = B + n0 * Kpad;
  const int lr = lane >> 2, lp = lane & 3;
  uint32_t offa[IA], offb[IB];
#pragma unroll
  for (int j = 0; j < IA; j++) {
    const int r = (wave * IA + j) * 16 + lr;
    offa[j] = (uint32_t)r * kp + (uint32_t)((lp ^ lds_swz(r)) << 4);
  }
#pragma unroll
  for (int j = 0; j < IB; j++) {
    const int r = (wave * IB + j) * 16 + lr;
    offb[j] = (uint32_t)r * kp + (uint32_t)((lp ^ lds_swz(r)) << 4);
  }
  // The DMA offsets address K from kbeg.
  const int8_t* const abase_k = abase + (int64_t)kbeg * BK;
  const int8_t* const bbase_k = bbase + (int64_t)kbeg * BK;
  auto issue = [&](uint32_t st_off, uint32_t k0) {
    int8_t* sa = smem + st_off;
#pragma unroll
    for (int j = 0; j < IA; j++) dma16(abase_k + (offa[j] + k0), sa + (wave * IA + j) * 16 * BK);
#pragma unroll
    for (int j = 0; j < IB; j++) dma16(bbase_k + (offb[j] + k0), sa + A_ST + (wave * IB + j) * 16 * BK);
  };

#pragma unroll
  for (int i = 0; i < FM; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) acc[i][j] = v4i{0, 0, 0, 0};

  // MFMA operand read offset: row (lane & 15) of a 16-row block, chunk lane>>4.
  const uint32_t rd = (uint32_t)((lane & 15) * BK + (((lane >> 4) ^ lds_swz(lane & 15)) << 4));
  const uint32_t rda = rd + (uint32_t)(wm * 16 * FM * BK), rdb = rd + (uint32_t)(A_ST + wn * 64 * BK);
  // STAGES - 1 groups in flight before the loop (clamped to the last step,
  // so short K still issues the same number of groups).
#pragma unroll
  for (int s = 0; s < STAGES - 1; s++) issue((uint32_t)(s * ST), (uint32_t)(s < nk ? s : nk - 1) * BK);
  uint32_t st_rd = 0, st_is = (uint32_t)((STAGES - 1) * ST);
  for (int kt = 0; kt < nk; kt++) {
    // Loads of the STAGES - 2 later steps may stay in flight; step kt's
    // DMA instructions must have landed.
    wait_vmcnt<(STAGES - 2) * (IA + IB)>();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    const int8_t* sa = smem + st_rd;
    // B fragments first, then A in consumption order, so each MFMA row
    // block waits only for its own A fragment (lgkmcnt counts in order).
    v4i bf[4], af[FM];
#pragma unroll
    for (int j = 0; j < 4; j++) bf[j] = *reinterpret_cast<const v4i*>(sa + rdb + j * 16 * BK);
#pragma unroll
    for (int i = 0; i < FM; i++) af[i] = *reinterpret_cast<const v4i*>(sa + rda + i * 16 * BK);
    // Always issue (the last steps re-fetch step nk-1 into the stage that is
    // free), so every path keeps the same counter state and the MFMAs below
    // wait for their own fragments only.
    issue(st_is, (uint32_t)(kt + STAGES - 1 < nk ? kt + STAGES - 1 : nk - 1) * BK);
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
      for (int j = 0; j < 4; j++) {
        if constexpr (MODE == kModeF16) {
          acc[i][j] = __builtin_bit_cast(
              v4i, __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, af[i]), __builtin_bit_cast(v8h, bf[j]),
                                                           __builtin_bit_cast(v4f, acc[i][j]), 0, 0, 0));
        } else if constexpr (MODE == kModeF32) {
          // Each lane's 16 bytes are 4 floats of its row, k = 4 (lane / 16) + c;
          // one v_mfma_f32_16x16x4_f32 per c covers the step's 16 k values
          // (the same products, grouped by c).
          v4f a4 = __builtin_bit_cast(v4f, acc[i][j]);
          const v4f fa = __builtin_bit_cast(v4f, af[i]), fb = __builtin_bit_cast(v4f, bf[j]);
#pragma unroll
          for (int c = 0; c < 4; c++) a4 = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[c], fb[c], a4, 0, 0, 0);
          acc[i][j] = __builtin_bit_cast(v4i, a4);
        } else
          acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
      }
    st_rd = st_rd == (uint32_t)((STAGES - 1) * ST) ? 0 : st_rd + ST;
    st_is = st_is == (uint32_t)((STAGES - 1) * ST) ? 0 : st_is + ST;
  }
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

}  // namespace rgnpu
