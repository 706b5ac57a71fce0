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
// CUs.  A workgroup that has polled spin_limit times (kBarrierPollUs each)
// stores its last tile's f32 outputs, marks itself deferred and exits; the
// workgroup whose arrival completed the barrier (the finisher) waits for
// every workgroup to settle (they have all arrived, so they are running and
// each stores its state within spin_limit polls) and quantizes the deferred
// workgroups' tiles from memory.  No wait is unbounded, so two such kernels
// can never deadlock each other.  The context's counters (Requant::stats)
// count deferrals, launches, and workgroups a finisher found unsettled after
// its own, larger bound: the host turns the last into RGNPU_ERR_DEVICE.
//
// Memory ordering.  Everything that crosses workgroups on the common path is
// an agent-scope atomic read-modify-write or atomic load: the absmax
// partials, the arrival counters, the go lines and the state words.  On
// gfx942/gfx950 these are performed with sc1 set, at the memory side where
// every XCD sees them (LLVM AMDGPU memory model, GFX942 table: "atomicrmw /
// load atomic, agent scope: sc1=1"), and a wave's earlier atomic has
// completed before its next is issued once s_waitcnt vmcnt(0) has returned
// (atomics without return are counted by vmcnt).  The partial's atomicMax is
// waited for before the arrival, the finisher has observed every arrival
// before it stores a go line, and a released workgroup loads the partials
// only after it has observed its go line: each cross-workgroup value is read
// by an atomic load after the atomic that wrote it has completed at the
// memory side.  No plain (cached) load reads another workgroup's data except
// on the deferral path, which fences (release before the deferred state,
// acquire in the finisher).  Release/acquire orderings on the go lines
// would make the compiler write back (buffer_wbl2) or invalidate
// (buffer_inv) the XCD's L2 around every poll; the tests that force every
// workgroup through the deferral path (spin limit 0) check the fenced path.
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cstdlib>
#include <stdexcept>

#include "devmath.h"
#include "gemm_core.h"
#include "rgnpu_internal.h"

namespace rgnpu {

// Barrier words (u32 offsets into Requant::sync, zeroed before every run):
// eight group arrival counters and the count of complete groups, each on a
// 128-byte line of its own; the error flag; one state word per workgroup;
// and one "go" line per workgroup, written by the finisher and polled by that
// workgroup alone, so no line is polled by more than one workgroup and no
// poll competes with the arrivals.
namespace rqk {
constexpr uint32_t kOwn = 1, kDeferred = 2;
constexpr int kGroups = 8;                      // arrival groups: workgroup b joins group b % 8
constexpr int64_t kLine = 32;                   // u32 words per 128-byte line
constexpr int64_t kGroupDone = kGroups * kLine; // complete groups
constexpr int64_t kError = kGroupDone + kLine;  // the finisher saw a workgroup that never settled
constexpr int64_t kMaxGrid = 1024;              // workgroups of one launch at most
constexpr int64_t kGoBase = kRequantStateBase + kMaxGrid;
constexpr int kPollSleep = 8;                   // s_sleep units (64 clocks) between polls
constexpr int kFinisherExtraPolls = 100000;     // settle budget of the finisher beyond spin_limit
static_assert(kError < kRequantStateBase, "state words follow the counters");
}  // namespace rqk

// Arrival at the grid barrier of a persistent launch; every thread of the
// workgroup calls it after the workgroup's absmax atomic has completed.
// Two-level arrival: the last of a group counts the group, and the arrival
// that completes the last group is the finisher, which releases every other
// workgroup through its go line.  Returns 2 for the finisher, 1 for a
// released workgroup, 0 for one that gave up after spin_limit polls.
// blk_flag is a word of the workgroup's LDS.
// One barrier poll loop: up to `limit` polls of a go line; true once set.
__device__ __forceinline__ bool poll_go(const uint32_t* go, int limit) {
  for (int k = 0; k < limit; k++) {
    __builtin_amdgcn_s_sleep(rqk::kPollSleep);
    if (__hip_atomic_load(go, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) return true;
  }
  return false;
}

__device__ __forceinline__ uint32_t grid_arrive(uint32_t* sync, int b, int G, int spin_limit, uint32_t* blk_flag) {
  if (threadIdx.x == 0) {
    const int g = b % rqk::kGroups;
    const uint32_t in_group = (uint32_t)((G - g + rqk::kGroups - 1) / rqk::kGroups);
    const uint32_t groups = (uint32_t)(G < rqk::kGroups ? G : rqk::kGroups);
    uint32_t flag = 0;
    if (__hip_atomic_fetch_add(sync + g * rqk::kLine, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1 ==
            in_group &&
        __hip_atomic_fetch_add(sync + rqk::kGroupDone, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1 == groups)
      flag = 2;
    if (flag == 0 && poll_go(sync + rqk::kGoBase + (int64_t)b * rqk::kLine, spin_limit)) flag = 1;
    *blk_flag = flag;
  }
  __syncthreads();
  const uint32_t flag = *blk_flag;
  if (flag == 2) {
    // release every other workgroup: one line each
    for (int w = threadIdx.x; w < G; w += blockDim.x)
      if (w != b)
        __hip_atomic_store(sync + rqk::kGoBase + (int64_t)w * rqk::kLine, 1u, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
  }
  return flag;
}

// The finisher's wait for every workgroup's state word (each has arrived and
// stores its state within spin_limit polls, so this is short; one that never
// settles raises the error flag and the context's unsettled counter): the
// indices of the deferred ones go to list[0 .. *count).  Every thread calls
// it; count is a word of LDS.  Also counts the finished launch.
__device__ __forceinline__ int collect_deferred(uint32_t* sync, int G, int spin_limit, uint32_t* list,
                                                uint32_t* count, uint32_t* stats) {
  if (threadIdx.x == 0) {
    *count = 0;
    if (stats) atomicAdd(stats + kStatLaunches, 1u);
  }
  __syncthreads();
  for (int w = threadIdx.x; w < G; w += blockDim.x) {
    uint32_t st = 0;
    for (int k = 0; k < spin_limit + rqk::kFinisherExtraPolls; k++) {
      st = __hip_atomic_load(sync + kRequantStateBase + w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (st != 0) break;
      __builtin_amdgcn_s_sleep(rqk::kPollSleep);
    }
    if (st == 0) {
      __hip_atomic_store(sync + rqk::kError, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (stats) atomicAdd(stats + kStatUnsettled, 1u);
    }
    if (st == rqk::kDeferred) list[atomicAdd(count, 1u)] = (uint32_t)w;
  }
  __syncthreads();
  return (int)*count;
}

// The lane layout of the requant epilogue and quantization: lane l of a
// wave owning rows [wrow0, wrow0 + 16 FM) and columns [wcol0, wcol0 + 64)
// takes the 4 consecutive columns wcol0 + 4 (l & 15) .. + 3 of rows
// wrow0 + 16 i + 4 p + (l >> 4), i < FM, p < 4.  N is a multiple of 4 (the
// plan fuses only then), so a lane's 4 columns are all outputs or all
// padding.  Which rows are outputs is fixed per lane: 16 i + 4 p < rows_left.
struct LaneSpan {
  int32_t rows_left;  // rows of this lane's column group that are outputs, counted from its first row
  bool cols_ok;       // the lane's 4 columns are outputs (< N)
};

__device__ __forceinline__ LaneSpan lane_span(int32_t wrow0, int32_t wcol0, int32_t M, int32_t N, int lane) {
  LaneSpan s;
  const int32_t rl = M - wrow0 - (lane >> 4);
  s.rows_left = rl < 0 ? 0 : rl;
  s.cols_ok = wcol0 + 4 * (lane & 15) < N;
  return s;
}

// quantize_one (quantize.rs:22) without branches, for a value of the tensor
// whose absmax gave inv: the clamp to +-127 cannot act (rgmath::quantize_rz_bounded).
__device__ __forceinline__ int32_t q8(float v, float inv) { return rgmath::quantize_rz_bounded(v * inv); }

// Four quantized bytes of one row, little-endian by column.
__device__ __forceinline__ uint32_t q8x4(v4f v, float inv) {
  const uint32_t b0 = (uint32_t)q8(v[0], inv), b1 = (uint32_t)q8(v[1], inv);
  const uint32_t b2 = (uint32_t)q8(v[2], inv), b3 = (uint32_t)q8(v[3], inv);
  const uint32_t lo = __builtin_amdgcn_perm(b1, b0, 0x0c0c0400u);  // bytes b0.0, b1.0
  const uint32_t hi = __builtin_amdgcn_perm(b3, b2, 0x0c0c0400u);
  return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
}

typedef unsigned int v4u __attribute__((ext_vector_type(4)));

// Quantizes 4 values into q's row (byte offset qoff from the wave's q base):
// rows past M and columns past N are the operand's zero padding.
__device__ __forceinline__ void quant_store(__amdgpu_buffer_rsrc_t rq, v4f v, float inv, uint32_t qoff, uint32_t soff,
                                            bool row_ok, bool cols_ok, bool q_ok) {
  const uint32_t w = row_ok && cols_ok ? q8x4(v, inv) : 0u;
  __builtin_amdgcn_raw_buffer_store_b32(w, rq, (int)(q_ok ? qoff : kDropOffset), (int)soff, 0);
}

// One wave's (16 FM) x 64 tile of the fused epilogue (quantize.rs:109-111),
// staged through the wave's LDS slab 16 rows at a time and read back in the
// lane layout above, so the f32 stores (when `store`) are 16 bytes.  The
// activations are left in acc[i][p] (f32 bits); with CAP the i32 sums are
// stored too.  Returns the max |y| over the outputs (NaN ignored, like
// f32::max); padding columns (zero weights and bias) are not outputs.
template <int ACT, int FM, bool CAP>
__device__ __forceinline__ float requant_epilogue(int8_t* smem, v4i (&acc)[FM][4], int32_t wrow0, int32_t wcol0,
                                                  int32_t N, const LaneSpan& sp, float cs, const float4 b4,
                                                  const Epilogue& ep, bool store, int wave, int lane) {
  int32_t* slab = reinterpret_cast<int32_t*>(smem + wave * big::SLAB);
  const int sub = lane >> 4, c4 = (lane & 15) * 4;
  const float bb[4] = {b4.x, b4.y, b4.z, b4.w};
  const int64_t base = (int64_t)wrow0 * N + wcol0;
  const __amdgpu_buffer_rsrc_t ry = bounded_rsrc(ep.y + base);
  const uint32_t voff = (uint32_t)((sub * N + c4) * 4);
  const uint32_t row_bytes = (uint32_t)N * 4u;
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < FM; i++) {
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int r = 0; r < 4; r++) slab[((lane >> 4) * 4 + r) * big::SLAB_LD + j * 16 + (lane & 15)] = acc[i][j][r];
#pragma unroll
    for (int p = 0; p < 4; p++) {
      const int rr = p * 4 + sub, ro = i * 16 + p * 4;
      const v4i a = *reinterpret_cast<const v4i*>(slab + rr * big::SLAB_LD + c4);
      v4f v;
#pragma unroll
      for (int c = 0; c < 4; c++) v[c] = epi_value<ACT>(a[c], cs, bb[c], ep.act_param);
      const bool ok = ro < sp.rows_left && sp.cols_ok;
      const float m4 = __builtin_fmaxf(__builtin_fmaxf(__builtin_fabsf(v[0]), __builtin_fabsf(v[1])),
                                       __builtin_fmaxf(__builtin_fabsf(v[2]), __builtin_fabsf(v[3])));
      amax = __builtin_fmaxf(amax, ok ? m4 : 0.0f);
      const uint32_t soff = (uint32_t)ro * row_bytes;
      if (store || CAP)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u, v), ry, (int)(ok ? voff : kDropOffset),
                                               (int)soff, 0);
      if constexpr (CAP)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u, a), bounded_rsrc(ep.acc_out + base),
                                               (int)(ok ? voff : kDropOffset), (int)soff, 0);
      acc[i][p] = __builtin_bit_cast(v4i, v);
    }
  }
  return amax;
}

// Stores the activations requant_epilogue left in acc as f32 (a workgroup
// that defers its quantization leaves them for the finisher).
template <int FM>
__device__ __forceinline__ void store_kept_f32(const v4i (&acc)[FM][4], float* y, int32_t wrow0, int32_t wcol0,
                                               int32_t N, const LaneSpan& sp, int lane) {
  const __amdgpu_buffer_rsrc_t ry = bounded_rsrc(y + (int64_t)wrow0 * N + wcol0);
  const uint32_t voff = (uint32_t)(((lane >> 4) * N + 4 * (lane & 15)) * 4);
#pragma unroll
  for (int i = 0; i < FM; i++)
#pragma unroll
    for (int p = 0; p < 4; p++) {
      const int ro = i * 16 + p * 4;
      const bool ok = ro < sp.rows_left && sp.cols_ok;
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u, acc[i][p]), ry, (int)(ok ? voff : kDropOffset),
                                             (int)((uint32_t)ro * (uint32_t)N * 4u), 0);
    }
}

// Quantizes the activations kept in acc into q [.., ldq]: every row of the
// wave's part is written (zero rows past M and zero columns past N are the
// operand's padding); columns at or past ldq (the producer's Npad may exceed
// the consumer's Kpad) are not part of the operand.
template <int FM>
__device__ __forceinline__ void quantize_kept(const v4i (&acc)[FM][4], int8_t* q, int32_t ldq, int32_t wrow0,
                                              int32_t wcol0, const LaneSpan& sp, float inv, int lane) {
  const __amdgpu_buffer_rsrc_t rq = bounded_rsrc(q + (int64_t)wrow0 * ldq + wcol0);
  const uint32_t qoff = (uint32_t)((lane >> 4) * ldq + 4 * (lane & 15));
  const bool q_ok = wcol0 + 4 * (lane & 15) < ldq;
#pragma unroll
  for (int i = 0; i < FM; i++)
#pragma unroll
    for (int p = 0; p < 4; p++) {
      const int ro = i * 16 + p * 4;
      quant_store(rq, __builtin_bit_cast(v4f, acc[i][p]), inv, qoff, (uint32_t)ro * (uint32_t)ldq, ro < sp.rows_left,
                  sp.cols_ok, q_ok);
    }
}

// Quantizes a whole BM x BN tile (rows m0.., columns n0..) from its stored
// f32 outputs, the workgroup's threads walking it row-major: one load of a
// wave reads 64 consecutive float4 (a 1 KiB row when BN = 256) and one store
// writes 256 consecutive bytes.  Rows past M and columns past N are the
// operand's zero padding; columns at or past ldq are not part of it.  BATCH
// loads per thread are in flight before the first is used.
template <int BM, int BN, int NTHREADS>
__device__ __forceinline__ void quantize_stored_flat(const float* y, int8_t* q, int32_t ldq, int32_t m0, int32_t n0,
                                                     int32_t M, int32_t N, float inv, int tid) {
  constexpr int C4 = BN / 4, PER = BM * C4 / NTHREADS, BATCH = PER < 16 ? PER : 16;
  static_assert(PER * NTHREADS == BM * C4 && PER % BATCH == 0 && NTHREADS % C4 == 0, "tile walk");
  const __amdgpu_buffer_rsrc_t ry = bounded_rsrc(y + (int64_t)m0 * N + n0);
  const __amdgpu_buffer_rsrc_t rq = bounded_rsrc(q + (int64_t)m0 * ldq + n0);
  const int c4 = tid % C4, rt = tid / C4;  // a thread keeps its column; its rows step by NTHREADS / C4
  constexpr int RSTEP = NTHREADS / C4;
  const bool col_ok = n0 + 4 * c4 < N, q_ok = n0 + 4 * c4 < ldq;
  const int32_t rows_left = M - m0 - rt;  // row rt + RSTEP k is an output iff RSTEP k < rows_left
  const uint32_t voff = (uint32_t)((rt * N + 4 * c4) * 4), qoff = (uint32_t)(rt * ldq + 4 * c4);
#pragma unroll
  for (int k0 = 0; k0 < PER; k0 += BATCH) {
    v4f v[BATCH];
#pragma unroll
    for (int k = 0; k < BATCH; k++) {
      const int rr = (k0 + k) * RSTEP;
      const bool ok = rr < rows_left && col_ok;
      v[k] = __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(
                                         ry, (int)(ok ? voff : kDropOffset), (int)((uint32_t)rr * (uint32_t)N * 4u), 2));
    }
#pragma unroll
    for (int k = 0; k < BATCH; k++) {
      const int rr = (k0 + k) * RSTEP;
      quant_store(rq, v[k], inv, qoff, (uint32_t)rr * (uint32_t)ldq, rr < rows_left, col_ok, q_ok);
    }
  }
}

// ---------------------------------------------------------------------------
// Certified GELU requantization (GELU producer, no capture).  The epilogue
// keeps and stores the pre-activations x = fl(fl(acc * cs) + b); a lane's
// exact absmax is gelu(xmax) over its outputs (rgmath::kGeluNegAbsMax and the
// monotonicity of the f32 GELU on [0, +inf]) when that clears the bound, and
// a lane below it cannot hold the workgroup's absmax unless no lane of the
// workgroup clears it, in which case the workgroup walks all of its outputs
// with the exact GELU (cert_exact_absmax).  After the barrier each
// value is quantized from gelu_approx(x): t = fl(g * inv) and q = round(t)
// stand when |t - q| + m < 1/2, where m = fl(mc |x|) + m0 covers
// (kGeluApproxRel |x| + kGeluApproxAbs) inv plus the roundings of t (|t| is
// at most about |x| inv, since |gelu(x)| <= |x|) and of the test itself.
// The values that miss the test (a few per 10^5; NaN and infinite x always
// miss it: their m is not finite) go to a per-wave queue in LDS and get the
// exact GELU once the walk is done, one queued value per lane; a queue that
// overflows sends its wave through every value again.
// ---------------------------------------------------------------------------
struct CertConst {
  float mc, m0;  // m = mc |x| + m0, in quantization steps
};

// Mode 1: the certified test.  Mode 2: every value misses it (each wave's
// queue overflows: the full re-walk).  Mode 3: m0 raised by 1/256, so a few
// values in a thousand miss it and go through the queue.
__device__ __forceinline__ CertConst cert_const(float inv, int mode) {
  CertConst c;
  c.mc = ((rgmath::kGeluApproxRel + 0x1p-23f) * 1.0001f) * inv;
  c.m0 = (rgmath::kGeluApproxAbs * 1.0001f) * inv + 0x1p-24f;
  if (mode == 2) c.m0 = __builtin_inff();
  if (mode == 3) c.m0 = c.m0 + 0x1p-8f;
  return c;
}

// The certified quantization of one pre-activation: the quantized integer,
// and in ok whether it is certain.
__device__ __forceinline__ int32_t cert_q(float x, float inv, const CertConst& c, bool& ok) {
  const float t = rgmath::gelu_approx(x) * inv;
  const int32_t q = rgmath::quantize_rz_bounded(t);
  const float r = __builtin_fabsf(t - (float)q);
  const float m = c.mc * __builtin_fabsf(x) + c.m0;
  ok = r + m < 0.5f;
  return q;
}

// The exact quantized integer (the clamp cannot act: |gelu(x)| <= absmax).
__device__ __forceinline__ int32_t exact_q(float x, float inv) {
  return rgmath::quantize_rz_bounded(rgmath::gelu_fast(x) * inv);
}

// Per-wave queue of uncertain values in LDS: x bits, and the byte offset of
// its q byte from the walk's buffer base, in two arrays.  n counts every
// value pushed (it is wave-uniform) and may exceed the capacity.
constexpr int kCertQueue = 512;      // entries per wave (4 KiB)
constexpr int kCertQueueBase = 8192; // bytes from the LDS array's start (the finisher's list comes first)
struct CertQueue {
  uint32_t* x;
  uint32_t* off;
  uint32_t n;
};

__device__ __forceinline__ CertQueue cert_queue(int8_t* smem, int wave) {
  uint32_t* const base = reinterpret_cast<uint32_t*>(smem + kCertQueueBase) + wave * 2 * kCertQueue;
  return CertQueue{base, base + kCertQueue, 0u};
}

__device__ __forceinline__ void cert_push(CertQueue& qu, bool need, float x, uint32_t off) {
  const uint64_t m = __builtin_amdgcn_ballot_w64(need);
  if (m == 0) return;
  if (need) {
    const uint32_t pos =
        qu.n + __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
    if (pos < (uint32_t)kCertQueue) {
      qu.x[pos] = __float_as_uint(x);
      qu.off[pos] = off;
    }
  }
  qu.n += (uint32_t)__builtin_popcountll(m);
}

// Four certified bytes of one row (little-endian by column); the uncertain
// ones among the valid values are queued (off: the first byte's offset).
__device__ __forceinline__ uint32_t cert_q8x4(v4f v, float inv, const CertConst& c, bool valid, uint32_t off,
                                              CertQueue& qu) {
  bool o0, o1, o2, o3;
  const uint32_t b0 = (uint32_t)cert_q(v[0], inv, c, o0), b1 = (uint32_t)cert_q(v[1], inv, c, o1);
  const uint32_t b2 = (uint32_t)cert_q(v[2], inv, c, o2), b3 = (uint32_t)cert_q(v[3], inv, c, o3);
  if (__builtin_amdgcn_ballot_w64(valid && !(o0 && o1 && o2 && o3))) {
    cert_push(qu, valid && !o0, v[0], off);
    cert_push(qu, valid && !o1, v[1], off + 1u);
    cert_push(qu, valid && !o2, v[2], off + 2u);
    cert_push(qu, valid && !o3, v[3], off + 3u);
  }
  const uint32_t lo = __builtin_amdgcn_perm(b1, b0, 0x0c0c0400u);
  const uint32_t hi = __builtin_amdgcn_perm(b3, b2, 0x0c0c0400u);
  return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
}

// Rewrites the queued bytes with the exact GELU, one entry per lane.  The
// word stores of the walk have completed first (vmcnt(0)), so these byte
// stores, from any lane, land after them.  Returns false when the queue
// overflowed (nothing is rewritten then).
__device__ __forceinline__ bool cert_drain(const CertQueue& qu, __amdgpu_buffer_rsrc_t rq, float inv, int lane) {
  if (qu.n == 0) return true;
  if (qu.n > (uint32_t)kCertQueue) return false;
  wait_vmcnt<0>();
  for (uint32_t j = (uint32_t)lane; j < qu.n; j += 64)
    __builtin_amdgcn_raw_buffer_store_b8((uint8_t)exact_q(__uint_as_float(qu.x[j]), inv), rq, (int)qu.off[j], 0, 0);
  return true;
}

// The uncertain bytes of 4 values, rewritten with the exact GELU (the
// overflow path: a byte store after the word store of the same thread).
__device__ __forceinline__ void cert_fix4(__amdgpu_buffer_rsrc_t rq, v4f v, float inv, const CertConst& c, uint32_t qoff,
                                          uint32_t soff) {
#pragma unroll 1
  for (int e = 0; e < 4; e++) {
    bool ok;
    (void)cert_q(v[e], inv, c, ok);
    if (!ok)
      __builtin_amdgcn_raw_buffer_store_b8((uint8_t)exact_q(v[e], inv), rq, (int)(qoff + (uint32_t)e), (int)soff, 0);
  }
}

// The epilogue of the certified path: x = fl(fl(acc * cs) + b) in acc
// (f32 bits) and, when `store`, in y; returns the exact max |gelu(x)| over
// the lane's outputs.
template <int FM>
__device__ __forceinline__ float cert_epilogue(int8_t* smem, v4i (&acc)[FM][4], int32_t wrow0, int32_t wcol0, int32_t N,
                                               const LaneSpan& sp, float cs, const float4 b4, const Epilogue& ep,
                                               bool store, float thr, int wave, int lane) {
  int32_t* slab = reinterpret_cast<int32_t*>(smem + wave * big::SLAB);
  const int sub = lane >> 4, c4 = (lane & 15) * 4;
  const float bb[4] = {b4.x, b4.y, b4.z, b4.w};
  const __amdgpu_buffer_rsrc_t ry = bounded_rsrc(ep.y + (int64_t)wrow0 * N + wcol0);
  const uint32_t voff = (uint32_t)((sub * N + c4) * 4);
  const uint32_t row_bytes = (uint32_t)N * 4u;
  float xmax = 0.0f;  // a phantom 0 output: gelu(0) = 0 is no larger than the absmax
#pragma unroll
  for (int i = 0; i < FM; i++) {
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int r = 0; r < 4; r++) slab[((lane >> 4) * 4 + r) * big::SLAB_LD + j * 16 + (lane & 15)] = acc[i][j][r];
#pragma unroll
    for (int p = 0; p < 4; p++) {
      const int rr = p * 4 + sub, ro = i * 16 + p * 4;
      const v4i a = *reinterpret_cast<const v4i*>(slab + rr * big::SLAB_LD + c4);
      v4f v;
#pragma unroll
      for (int c = 0; c < 4; c++) v[c] = epi_value<rgmath::ACT_NONE>(a[c], cs, bb[c], 0.0f);
      const bool ok = ro < sp.rows_left && sp.cols_ok;
      const float m4 = __builtin_fmaxf(__builtin_fmaxf(v[0], v[1]), __builtin_fmaxf(v[2], v[3]));
      xmax = __builtin_fmaxf(xmax, ok ? m4 : 0.0f);
      if (store)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u, v), ry, (int)(ok ? voff : kDropOffset),
                                               (int)((uint32_t)ro * row_bytes), 0);
      acc[i][p] = __builtin_bit_cast(v4i, v);
    }
  }
  // The lane's exact max |gelu| when gelu(xmax) clears the bound, else 0:
  // such a lane's outputs are all within kGeluNegAbsMax, which any lane of
  // the workgroup that clears the bound dominates (see cert_exact_absmax).
  const float gx = rgmath::gelu_fast(xmax);
  return gx >= thr ? gx : 0.0f;
}

// The workgroup's exact max |gelu| over all of its outputs, when no lane's
// gelu(xmax) cleared the bound (every output of the workgroup is small or not
// finite; with thr = +inf, the test mode, always): the kept tile's
// pre-activations go to y beside the stored ones, then the workgroup walks
// every one of its tiles with the exact GELU.  Every thread calls it; red is
// NW words of LDS.
template <int BM, int BN, int NTHREADS, int FM>
__device__ __forceinline__ float cert_exact_absmax(const v4i (&acc)[FM][4], float* y, int32_t wrow0, int32_t wcol0,
                                                   int32_t M, int32_t N, const LaneSpan& sp_last, int b, int G,
                                                   int tiles_m, int tiles_n, int ntile, uint32_t* red, int tid) {
  constexpr int C4 = BN / 4, RSTEP = NTHREADS / C4;
  const int lane = tid & 63;
  store_kept_f32<FM>(acc, y, wrow0, wcol0, N, sp_last, lane);
  wait_vmcnt<0>();
  __syncthreads();
  float amax = 0.0f;
  const int c4 = tid % C4, rt = tid / C4;
  for (int it = 0; it < ntile; it++) {
    int tm, tn;
    tile_coords(b + it * G, tiles_m, tiles_n, tm, tn);
    const int32_t m0 = tm * BM, n0 = tn * BN;
    if (!(n0 + 4 * c4 < N)) continue;
    const __amdgpu_buffer_rsrc_t ry = bounded_rsrc(y + (int64_t)m0 * N + n0);
#pragma unroll 1
    for (int r = rt; r < BM && m0 + r < M; r += RSTEP) {
      const v4f v = __builtin_bit_cast(
          v4f, __builtin_amdgcn_raw_buffer_load_b128(ry, (int)((uint32_t)(r * N + 4 * c4) * 4u), 0, 0));
#pragma unroll
      for (int c = 0; c < 4; c++) amax = __builtin_fmaxf(amax, __builtin_fabsf(rgmath::gelu_fast(v[c])));
    }
  }
  const uint32_t m = wave_max_u32(rgmath::fbits(amax));
  __syncthreads();
  if (lane == 0) red[tid >> 6] = m;
  __syncthreads();
  uint32_t r = red[0];
  for (int w = 1; w < NTHREADS / 64; w++) r = red[w] > r ? red[w] : r;
  return rgmath::bitsf(r);
}

// quantize_kept for the certified path: acc holds the pre-activations.
template <int FM>
__device__ __forceinline__ void cert_quantize_kept(const v4i (&acc)[FM][4], float* y, int8_t* q, int32_t ldq,
                                                   int32_t wrow0, int32_t wcol0, int32_t N, const LaneSpan& sp,
                                                   float inv, const CertConst& c, CertQueue qu, int lane) {
  const __amdgpu_buffer_rsrc_t rq = bounded_rsrc(q + (int64_t)wrow0 * ldq + wcol0);
  const uint32_t qoff = (uint32_t)((lane >> 4) * ldq + 4 * (lane & 15));
  const bool q_ok = wcol0 + 4 * (lane & 15) < ldq;
#pragma unroll
  for (int i = 0; i < FM; i++)
#pragma unroll
    for (int p = 0; p < 4; p++) {
      const int ro = i * 16 + p * 4;
      const bool row_ok = ro < sp.rows_left;
      const uint32_t soff = (uint32_t)ro * (uint32_t)ldq;
      const uint32_t w =
          cert_q8x4(__builtin_bit_cast(v4f, acc[i][p]), inv, c, row_ok && sp.cols_ok && q_ok, qoff + soff, qu);
      __builtin_amdgcn_raw_buffer_store_b32(row_ok && sp.cols_ok ? w : 0u, rq, (int)(q_ok ? qoff : kDropOffset),
                                            (int)soff, 0);
    }
  if (cert_drain(qu, rq, inv, lane)) return;
  // Overflow: store the pre-activations (outputs only), then rewrite every
  // uncertain byte from them.
  const __amdgpu_buffer_rsrc_t ry = bounded_rsrc(y + (int64_t)wrow0 * N + wcol0);
  const uint32_t voff = (uint32_t)(((lane >> 4) * N + 4 * (lane & 15)) * 4);
  const bool lane_ok = sp.cols_ok && q_ok;
#pragma unroll
  for (int i = 0; i < FM; i++)
#pragma unroll
    for (int p = 0; p < 4; p++) {
      const int ro = i * 16 + p * 4;
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u, acc[i][p]), ry,
                                             (int)(ro < sp.rows_left && lane_ok ? voff : kDropOffset),
                                             (int)((uint32_t)ro * (uint32_t)N * 4u), 0);
    }
  if (!lane_ok) return;
#pragma unroll 1
  for (int k = 0; k < FM * 4; k++) {
    const int ro = (k >> 2) * 16 + (k & 3) * 4;
    if (!(ro < sp.rows_left)) continue;
    const v4f v = __builtin_bit_cast(
        v4f, __builtin_amdgcn_raw_buffer_load_b128(ry, (int)voff, (int)((uint32_t)ro * (uint32_t)N * 4u), 0));
    cert_fix4(rq, v, inv, c, qoff, (uint32_t)ro * (uint32_t)ldq);
  }
}

// quantize_stored_flat for the certified path: y holds the pre-activations.
template <int BM, int BN, int NTHREADS>
__device__ __forceinline__ void cert_quantize_stored_flat(const float* y, int8_t* q, int32_t ldq, int32_t m0,
                                                          int32_t n0, int32_t M, int32_t N, float inv,
                                                          const CertConst& cc, CertQueue qu, int tid) {
  constexpr int C4 = BN / 4, PER = BM * C4 / NTHREADS, BATCH = PER < 16 ? PER : 16;
  static_assert(PER * NTHREADS == BM * C4 && PER % BATCH == 0 && NTHREADS % C4 == 0, "tile walk");
  const __amdgpu_buffer_rsrc_t ry = bounded_rsrc(y + (int64_t)m0 * N + n0);
  const __amdgpu_buffer_rsrc_t rq = bounded_rsrc(q + (int64_t)m0 * ldq + n0);
  const int c4 = tid % C4, rt = tid / C4;
  constexpr int RSTEP = NTHREADS / C4;
  const bool col_ok = n0 + 4 * c4 < N, q_ok = n0 + 4 * c4 < ldq;
  const int32_t rows_left = M - m0 - rt;
  const uint32_t voff = (uint32_t)((rt * N + 4 * c4) * 4), qoff = (uint32_t)(rt * ldq + 4 * c4);
#pragma unroll
  for (int k0 = 0; k0 < PER; k0 += BATCH) {
    v4f v[BATCH];
#pragma unroll
    for (int k = 0; k < BATCH; k++) {
      const int rr = (k0 + k) * RSTEP;
      const bool ok = rr < rows_left && col_ok;
      v[k] = __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(
                                         ry, (int)(ok ? voff : kDropOffset), (int)((uint32_t)rr * (uint32_t)N * 4u), 2));
    }
#pragma unroll
    for (int k = 0; k < BATCH; k++) {
      const int rr = (k0 + k) * RSTEP;
      const bool row_ok = rr < rows_left;
      const uint32_t soff = (uint32_t)rr * (uint32_t)ldq;
      const uint32_t w = cert_q8x4(v[k], inv, cc, row_ok && col_ok && q_ok, qoff + soff, qu);
      __builtin_amdgcn_raw_buffer_store_b32(row_ok && col_ok ? w : 0u, rq, (int)(q_ok ? qoff : kDropOffset),
                                            (int)soff, 0);
    }
  }
  if (cert_drain(qu, rq, inv, tid & 63)) return;
  // Overflow: rewrite every uncertain byte from the stored pre-activations.
  if (!(col_ok && q_ok)) return;
#pragma unroll 1
  for (int k = 0; k < PER; k++) {
    const int rr = k * RSTEP;
    if (!(rr < rows_left)) continue;
    const v4f v = __builtin_bit_cast(
        v4f, __builtin_amdgcn_raw_buffer_load_b128(ry, (int)voff, (int)((uint32_t)rr * (uint32_t)N * 4u), 0));
    cert_fix4(rq, v, inv, cc, qoff, (uint32_t)rr * (uint32_t)ldq);
  }
}

// Per-launch constants of the fused kernel, 32-bit where the plan bounds
// them (the fused path requires N % 4 == 0 and 128 N * 4 < 2^31).
struct RequantShape {
  int32_t M, N, ldq, nk, tiles_m, tiles_n;
};

// CERT: the certified GELU path (ACT == GELU, no capture): the f32 tiles
// stored for the quantization hold pre-activations, and the GELU is
// evaluated exactly only where the certified bound cannot decide.
template <int BM, int BN, int WAVES_M, int WAVES_N, int STAGES, int OCC, int FM, int ACT, bool CAP, bool CERT>
__global__ __launch_bounds__(WAVES_M * WAVES_N * 64, OCC) void gemm_requant_kernel(
    const int8_t* __restrict__ A, const int8_t* __restrict__ B, RequantShape sh, Epilogue ep, Requant rq) {
  using namespace big;
  static_assert(!CERT || (ACT == rgmath::ACT_GELU && !CAP), "certified path: GELU without capture");
  const float cert_thr = rq.gelu_cert == 2 ? __builtin_inff() : rgmath::kGeluNegAbsMax;
  constexpr int NW = WAVES_M * WAVES_N;
  static_assert(BM == 16 * FM * WAVES_M && BN == 64 * WAVES_N, "wave tile is (16 FM) x 64");
  constexpr int ST = (BM + BN) * BK;
  static_assert(NW * SLAB <= STAGES * ST, "epilogue slabs reuse the ring");
  static_assert(!CERT || kCertQueueBase + 8 * kCertQueue * NW <= STAGES * ST, "certified queues fit in the ring");
  static_assert(rqk::kMaxGrid * 4 <= kCertQueueBase, "the finisher's list precedes the queues");
  // One LDS array only, the few words of block state at its end: with a
  // second __shared__ variable the compiler no longer tells the ring's DMA
  // writes (global_load_lds) apart from the K loop's LDS reads and waits for
  // every outstanding load (vmcnt(0)) in each K step, serializing the ring.
  __shared__ __attribute__((aligned(1024))) int8_t smem[STAGES * ST + 64];
  uint32_t* const blk = reinterpret_cast<uint32_t*>(smem + STAGES * ST);  // [0] flag, [1] deferred, [2..] wave maxima
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  const int T = sh.tiles_m * sh.tiles_n, G = (int)gridDim.x, b = (int)blockIdx.x;
  const int ntile = (T - b + G - 1) / G;  // >= 1: the grid never exceeds the tile count
  const int32_t M = sh.M, N = sh.N, wrow = wm * 16 * FM, wcolw = wn * 64;
  // partial of the input absmax, folded after the first K loop
  const uint32_t absmax_part = tensor_absmax_part(ep.absmax_in);
  float cs = 0.0f, amax = 0.0f;
  int32_t m0 = 0, n0 = 0;
  v4i acc[FM][4];
  for (int it = 0; it < ntile; it++) {
    int tm, tn;
    tile_coords(b + it * G, sh.tiles_m, sh.tiles_n, tm, tn);
    m0 = tm * BM;
    n0 = tn * BN;
    if (it > 0) {
      // the previous epilogue's slabs live in the ring the K loop refills;
      // its stores are drained once here rather than left to the K loop
      wait_vmcnt<0>();
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
    }
    const float4 b4 = *reinterpret_cast<const float4*>(ep.bias + n0 + wcolw + 4 * (lane & 15));  // padded to Npad
    big_kloop<BM, BN, WAVES_M, WAVES_N, STAGES, FM, kModeI8>(smem, A, B, (int64_t)sh.nk * BK, m0, n0, 0, sh.nk, wave,
                                                             wm, wn, lane, acc);
    if (it == 0) cs = rgmath::scale_from_absmax(rgmath::bitsf(wave_max_u32(absmax_part))) * ep.w_scale;
    const LaneSpan sp = lane_span(m0 + wrow, n0 + wcolw, M, N, lane);
    float t;
    if constexpr (CERT)
      t = cert_epilogue<FM>(smem, acc, m0 + wrow, n0 + wcolw, N, sp, cs, b4, ep, it + 1 < ntile, cert_thr, wave,
                            lane);
    else
      t = requant_epilogue<ACT, FM, CAP>(smem, acc, m0 + wrow, n0 + wcolw, N, sp, cs, b4, ep,
                                         it + 1 < ntile || rq.keep_f32, wave, lane);
    amax = __builtin_fmaxf(amax, t);
  }

  // Publish this workgroup's absmax (one atomic), then arrive.  Everything
  // crossing workgroups on this path is a device-scope atomic (the absmax
  // partials, the arrival counts, the go lines, the states), performed where
  // all XCDs see it; the atomic has completed before the arrival (vmcnt
  // counts atomics without return on gfx9), and a workgroup reads back only
  // its own f32 stores.  No cache writeback or invalidation is needed, so
  // none is done: agent-scope fences here would flush the L2 of an XCD for
  // every wave.
  {
    const uint32_t m = wave_max_u32(rgmath::fbits(amax));
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();  // the epilogue slabs are done with
    if (lane == 0) blk[2 + wave] = m;
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    uint32_t r = blk[2];
    for (int w = 1; w < NW; w++) r = blk[2 + w] > r ? blk[2 + w] : r;
    if constexpr (CERT) {
      // no lane cleared the bound: the exact walk (every thread; rare)
      if (!(rgmath::bitsf(r) >= cert_thr))
        r = rgmath::fbits(cert_exact_absmax<BM, BN, NW * 64, FM>(acc, ep.y, m0 + wrow, n0 + wcolw, M, N,
                                                                  lane_span(m0 + wrow, n0 + wcolw, M, N, lane), b, G,
                                                                  sh.tiles_m, sh.tiles_n, ntile, blk + 2, tid));
    }
    if (tid == 0) {
      if (r) atomicMax(ep.absmax_out + (b & (kSpread - 1)) * kSpreadStride, r);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the atomic has completed before the arrival
    }
  }
  __builtin_amdgcn_s_barrier();
  const uint32_t flag = grid_arrive(rq.sync, b, G, rq.spin_limit, &blk[0]);
  const LaneSpan sp_last = lane_span(m0 + wrow, n0 + wcolw, M, N, lane);
  if (flag == 0) {
    // Waited too long: the finisher quantizes this workgroup's tiles from the
    // f32 outputs, which it reads from another XCD -- so here, and only on
    // this path, a release fence writes them back before the state says so.
    if (!rq.keep_f32 && !CAP) store_kept_f32<FM>(acc, ep.y, m0 + wrow, n0 + wcolw, N, sp_last, lane);
    __threadfence();
    __syncthreads();
    if (tid == 0) {
      __hip_atomic_store(rq.sync + kRequantStateBase + b, rqk::kDeferred, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (rq.stats) atomicAdd(rq.stats + kStatDeferred, 1u);
    }
    return;
  }
  if (tid == 0)
    __hip_atomic_store(rq.sync + kRequantStateBase + b, rqk::kOwn, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const uint32_t part =
      __hip_atomic_load(ep.absmax_out + lane * kSpreadStride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const float scale = rgmath::scale_from_absmax(rgmath::bitsf(wave_max_u32(part)));
  const float inv = 1.0f / scale;
  const CertConst cc = cert_const(inv, rq.gelu_cert);
  // the last tile from registers, then the earlier tiles from their stored outputs
  if constexpr (CERT)
    cert_quantize_kept<FM>(acc, ep.y, rq.q, sh.ldq, m0 + wrow, n0 + wcolw, N, sp_last, inv, cc,
                           cert_queue(smem, wave), lane);
  else
    quantize_kept<FM>(acc, rq.q, sh.ldq, m0 + wrow, n0 + wcolw, sp_last, inv, lane);
  __builtin_amdgcn_sched_barrier(0);
  for (int it = 0; it + 1 < ntile; it++) {
    int tm, tn;
    tile_coords(b + it * G, sh.tiles_m, sh.tiles_n, tm, tn);
    if constexpr (CERT)
      cert_quantize_stored_flat<BM, BN, NW * 64>(ep.y, rq.q, sh.ldq, tm * BM, tn * BN, M, N, inv, cc,
                                                 cert_queue(smem, wave), tid);
    else
      quantize_stored_flat<BM, BN, NW * 64>(ep.y, rq.q, sh.ldq, tm * BM, tn * BN, M, N, inv, tid);
  }
  if (flag != 2) return;

  // Finisher: the scale tap, then the tiles of every deferred workgroup.
  if (tid == 0 && rq.scale_out) *rq.scale_out = scale;
  uint32_t* list = reinterpret_cast<uint32_t*>(smem);  // the ring is free: no K loop follows
  const int ndef = collect_deferred(rq.sync, G, rq.spin_limit, list, &blk[1], rq.stats);
  if (ndef > 0) __threadfence();  // acquire: the deferred workgroups' stored outputs
  for (int d = 0; d < ndef; d++) {
    const int w = (int)list[d];
    const int wt = (T - w + G - 1) / G;
    for (int it = 0; it < wt; it++) {
      int tm, tn;
      tile_coords(w + it * G, sh.tiles_m, sh.tiles_n, tm, tn);
      if constexpr (CERT)
        cert_quantize_stored_flat<BM, BN, NW * 64>(ep.y, rq.q, sh.ldq, tm * BM, tn * BN, M, N, inv, cc,
                                                   cert_queue(smem, wave), tid);
      else
        quantize_stored_flat<BM, BN, NW * 64>(ep.y, rq.q, sh.ldq, tm * BM, tn * BN, M, N, inv, tid);
    }
  }
}

template <int BM, int BN, int WAVES_M, int WAVES_N, int STAGES, int OCC, int FM, int ACT, bool CAP, bool CERT = false>
static void launch_requant_act(const int8_t* A, const int8_t* B, const RequantShape& sh, int64_t Mpad, int64_t Npad,
                               int64_t Kpad, const Epilogue& ep, const Requant& rq, hipStream_t s) {
  constexpr int threads = WAVES_M * WAVES_N * 64;
  const void* fn =
      reinterpret_cast<const void*>(&gemm_requant_kernel<BM, BN, WAVES_M, WAVES_N, STAGES, OCC, FM, ACT, CAP, CERT>);
  static const int64_t cap = resident_blocks(fn, threads);
  const int64_t T = (int64_t)sh.tiles_m * sh.tiles_n;
  int64_t G = T < cap ? T : cap;
  if (G > rqk::kMaxGrid) G = rqk::kMaxGrid;
  if (rqk::kGoBase + G * rqk::kLine > requant_sync_words(Mpad, Npad, Kpad))
    throw std::logic_error("requant: more workgroups than sync words");
  RG_LAUNCH((gemm_requant_kernel<BM, BN, WAVES_M, WAVES_N, STAGES, OCC, FM, ACT, CAP, CERT>), dim3((unsigned)G),
            dim3(threads), 0, s, A, B, sh, ep, rq);
}

template <int BM, int BN, int WAVES_M, int WAVES_N, int STAGES, int OCC, int FM, bool CAP>
static void launch_requant_shape(const int8_t* A, const int8_t* B, const RequantShape& sh, int64_t Mpad, int64_t Npad,
                                 int64_t Kpad, const Epilogue& ep, const Requant& rq, hipStream_t s) {
#define RG_RQ(ACTV) \
  launch_requant_act<BM, BN, WAVES_M, WAVES_N, STAGES, OCC, FM, ACTV, CAP>(A, B, sh, Mpad, Npad, Kpad, ep, rq, s)
  switch (ep.act) {
    case rgmath::ACT_RELU: RG_RQ(rgmath::ACT_RELU); break;
    case rgmath::ACT_SIGMOID: RG_RQ(rgmath::ACT_SIGMOID); break;
    case rgmath::ACT_TANH: RG_RQ(rgmath::ACT_TANH); break;
    case rgmath::ACT_GELU:
      if constexpr (!CAP) {
        if (rq.gelu_cert) {
          launch_requant_act<BM, BN, WAVES_M, WAVES_N, STAGES, OCC, FM, rgmath::ACT_GELU, false, true>(
              A, B, sh, Mpad, Npad, Kpad, ep, rq, s);
          break;
        }
      }
      RG_RQ(rgmath::ACT_GELU);
      break;
    case rgmath::ACT_LEAKY_RELU: RG_RQ(rgmath::ACT_LEAKY_RELU); break;
    case rgmath::ACT_SILU: RG_RQ(rgmath::ACT_SILU); break;
    default: RG_RQ(rgmath::ACT_NONE); break;
  }
#undef RG_RQ
}

// ---------------------------------------------------------------------------
// A Linear's input quantization in one pass: QuantTensor::from_f32
// (quantize.rs:18-24) at npu.rs:312 for an input that no fused producer has
// quantized (the run's input, or the output of an op that does not emit the
// absmax).  The operand q [Mpad, Kpad] is cut into 4-byte units (4 inputs of
// one row; padding rows and columns are zero).  Workgroup b of G keeps the
// U * 512 consecutive units from b * U * 512 on, thread t of it units
// b U 512 + 512 j + t (j < U), so one load of a wave reads 1 KiB of
// consecutive inputs, one store writes 256 consecutive bytes, and a
// workgroup's reads stay within one contiguous range (few pages, long DRAM
// bursts).  Units past G U 512 (an input larger than the resident grid
// keeps) are shared out as G U 512 + gtid + k G 512.  A persistent grid
// reads its units once and keeps U of them per thread (the
// smallest U of 4, 8, ..., 64 whose grid is resident; at U = 64 the first 19
// in LDS and 45 in registers, 1 KiB of input per thread: the whole 134 MB
// input of an 8192 x 4096 batch on 256 CUs), raises the spread absmax slot,
// meets at the grid barrier and quantizes what it kept; units beyond those
// (inputs larger than the resident grid keeps) are read a second time.  The separate absmax pass
// over the input, and its launch, are gone.  A workgroup that waits too long
// at the barrier just exits: the finisher quantizes its units from the
// input, which nothing has changed.  A grid of one workgroup needs no
// barrier.
// ---------------------------------------------------------------------------
namespace iq {
constexpr int kThreads = 512;
constexpr int kMaxRegUnits = 45;  // units per thread in registers at most (180 VGPRs)
constexpr int kFirst = 30;        // register units loaded together with the LDS units
// units kept per thread: U, of which lds_units(U) in LDS (152 KiB per workgroup at U = 64)
constexpr int lds_units(int U) { return U > kMaxRegUnits ? U - kMaxRegUnits : 0; }
}  // namespace iq

struct InputQuantShape {
  int32_t M, K;     // input rows and row length (floats)
  uint32_t upr;     // units per operand row (Kpad / 4)
  uint32_t W;       // units of the operand (Mpad * Kpad / 4)
  uint32_t kr, kc;  // 512 = kr * upr + kc: the (row, unit-column) step between a thread's kept units
  uint32_t nr, nc;  // NT = G * 512 in the same form: the step between its remaining units
};

// w += (dr * upr + dc) in (row, unit-column) form.
__device__ __forceinline__ void iq_step(uint32_t& r, uint32_t& c, uint32_t dr, uint32_t dc, uint32_t upr) {
  c += dc;
  r += dr;
  const bool carry = c >= upr;
  c = carry ? c - upr : c;
  r = carry ? r + 1 : r;
}

// The 4 inputs of unit (r, c): zeros outside [M, K] (loads out of the input
// are dropped, and a dropped buffer load returns 0).
template <bool VEC>
__device__ __forceinline__ v4f iq_load(__amdgpu_buffer_rsrc_t rx, uint32_t r, uint32_t c, const InputQuantShape& s) {
  const uint32_t c0 = c * 4u;
  const bool row_ok = r < (uint32_t)s.M;
  const uint32_t base = (r * (uint32_t)s.K + c0) * 4u;  // used only in bounds (input < 2^31 bytes)
  if constexpr (VEC) {
    const bool ok = row_ok && c0 < (uint32_t)s.K;  // K % 4 == 0: a unit is all in or all out
    return __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(rx, (int)(ok ? base : kDropOffset), 0, 2));
  } else {
    v4f v;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const bool ok = row_ok && c0 + e < (uint32_t)s.K;
      v[e] = __builtin_bit_cast(float,
                                __builtin_amdgcn_raw_buffer_load_b32(rx, (int)(ok ? base + 4u * e : kDropOffset), 0, 0));
    }
    return v;
  }
}

__device__ __forceinline__ float iq_absmax(float m, v4f v) {
  m = __builtin_fmaxf(m, __builtin_fabsf(v[0]));  // NaN ignored, like f32::max
  m = __builtin_fmaxf(m, __builtin_fabsf(v[1]));
  m = __builtin_fmaxf(m, __builtin_fabsf(v[2]));
  return __builtin_fmaxf(m, __builtin_fabsf(v[3]));
}

// Unit w of the operand (byte offset 4 w) through a resource whose record
// count is the operand's size: the hardware drops units past the operand.
__device__ __forceinline__ void iq_store(__amdgpu_buffer_rsrc_t rq, v4f v, float inv, uint32_t w) {
  __builtin_amdgcn_raw_buffer_store_b32(q8x4(v, inv), rq, (int)(w * 4u), 0, 0);
}

// Quantizes `count` units w, w + (dr upr + dc), ... of one thread from the
// input (starting at row r, unit-column c); units past the operand are
// dropped.
template <bool VEC>
__device__ __forceinline__ void iq_quantize_from(__amdgpu_buffer_rsrc_t rx, __amdgpu_buffer_rsrc_t rq,
                                                 const InputQuantShape& s, uint32_t w, uint32_t count, uint32_t r,
                                                 uint32_t c, uint32_t dr, uint32_t dc, float inv) {
  const uint32_t dw = dr * s.upr + dc;
  for (uint32_t k = 0; k < count && w < s.W; k++, w += dw) {
    iq_store(rq, iq_load<VEC>(rx, r, c, s), inv, w);
    iq_step(r, c, dr, dc, s.upr);
  }
}

// The units a thread (workgroup b, thread t) owns: U kept ones from
// b U 512 + t, 512 apart, then the remaining ones from G U 512 + b 512 + t,
// G 512 apart.
__device__ __forceinline__ uint32_t iq_kept0(uint32_t b, uint32_t t, int U) { return b * (uint32_t)U * 512u + t; }
// The unit range of workgroup b: hardware deals workgroups round-robin over
// the 8 XCDs (b on XCD b & 7), so with G a multiple of 8 the workgroups of
// XCD x take the x-th contiguous eighth of the input (and write that eighth
// of the operand, about half of the rows the consuming GEMM's XCD-grouped
// tile order sends to XCD x).  On S (256 workgroups) the quantization went
// from 34.2-34.4 to 31.7-31.8 us against ranges dealt round-robin.
__device__ __forceinline__ uint32_t iq_range(uint32_t b, uint32_t G) {
  return (G & 7u) == 0 ? (b & 7u) * (G >> 3) + (b >> 3) : b;
}
__device__ __forceinline__ uint32_t iq_rest0(uint32_t b, uint32_t t, int U, uint32_t G) {
  return G * (uint32_t)U * 512u + b * 512u + t;
}

template <bool VEC, int U>
__global__ __launch_bounds__(iq::kThreads) void input_quant_kernel(const float* __restrict__ x, InputQuantShape sh,
                                                                   uint32_t* __restrict__ slot, int8_t* q,
                                                                   float* scale_out, uint32_t* sync, int spin_limit,
                                                                   uint32_t* stats, SlotClear clear) {
  using namespace iq;
  constexpr int KL = lds_units(U), KR = U - KL;
  static_assert(KR <= kMaxRegUnits && (KL == 0 || KR >= kFirst) && (KL == 0 || KL % 2 == 1), "unit split");
  // one LDS array: the LDS units as [kThreads][KL] 16-byte words (one
  // address register per thread, immediate offsets; KL is odd, so a wave's
  // 16-byte accesses spread over all banks), 16 words of block state, then
  // the finisher's list of deferred workgroups
  constexpr int kListWords = (int)rqk::kMaxGrid;
  __shared__ __attribute__((aligned(16))) v4f lds[KL * kThreads + 4 + kListWords / 4];
  uint32_t* const blk = reinterpret_cast<uint32_t*>(lds + KL * kThreads);  // [0] flag, [1] count, [2..] wave maxima
  clear_slots(clear);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int G = (int)gridDim.x, b = (int)blockIdx.x;
  static_assert(kThreads == 512, "unit layout");
  const uint32_t rb = iq_range((uint32_t)b, (uint32_t)G);
  const uint32_t w0 = iq_kept0(rb, (uint32_t)tid, U);
  const __amdgpu_buffer_rsrc_t rx = bounded_rsrc(x);
  const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(q, 0, (int)(sh.W * 4u), 0x00020000);
  const uint32_t r0 = w0 / sh.upr, c0 = w0 - r0 * sh.upr;

  // Pass 1: read every unit once (units past the operand have r >= Mpad >=
  // M and read as zeros).  Units 0 .. KL-1 of the thread go to LDS, the next
  // KR stay in registers, later ones are only measured.  The LDS units'
  // loads and the first kFirst register units' are in flight together; the
  // LDS units are retired before the other register units are loaded, so at
  // most KR units occupy registers at a time.
  v4f keep[KR];
  float m = 0.0f;
  uint32_t r = r0, c = c0;
  if constexpr (KL > 0) {
    v4f part[KL];
#pragma unroll
    for (int j = 0; j < KL; j++) {
      part[j] = iq_load<VEC>(rx, r, c, sh);
      iq_step(r, c, sh.kr, sh.kc, sh.upr);
    }
#pragma unroll
    for (int j = 0; j < kFirst; j++) {
      keep[j] = iq_load<VEC>(rx, r, c, sh);
      iq_step(r, c, sh.kr, sh.kc, sh.upr);
    }
#pragma unroll
    for (int j = 0; j < KL; j++) {
      m = iq_absmax(m, part[j]);
      lds[tid * KL + j] = part[j];
    }
  }
#pragma unroll
  for (int j = KL > 0 ? kFirst : 0; j < KR; j++) {
    keep[j] = iq_load<VEC>(rx, r, c, sh);
    iq_step(r, c, sh.kr, sh.kc, sh.upr);
  }
#pragma unroll
  for (int j = 0; j < KR; j++) m = iq_absmax(m, keep[j]);
  // the remaining units (an input larger than the grid keeps)
  const uint32_t NT = (uint32_t)G * kThreads;
  const uint32_t rest_w = iq_rest0(rb, (uint32_t)tid, U, (uint32_t)G);
  const uint32_t rest_r = rest_w / sh.upr, rest_c = rest_w - rest_r * sh.upr;
  r = rest_r;
  c = rest_c;
  for (uint32_t w = rest_w; w < sh.W; w += NT) {
    m = iq_absmax(m, iq_load<VEC>(rx, r, c, sh));
    iq_step(r, c, sh.nr, sh.nc, sh.upr);
  }
  // the workgroup's absmax: one atomic into its partial of the spread slot
  const uint32_t mw = wave_max_u32(rgmath::fbits(m));
  if (lane == 0) blk[2 + wave] = mw;
  __syncthreads();
  uint32_t t = blk[2];
  for (int w = 1; w < kThreads / 64; w++) t = blk[2 + w] > t ? blk[2 + w] : t;
  if (tid == 0) {
    if (t) atomicMax(slot + (b & (kSpread - 1)) * kSpreadStride, t);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the atomic has completed before the arrival
  }
  uint32_t flag = 2;  // a grid of one is its own finisher, and its absmax is t
  float scale;
  if (G == 1) {
    scale = rgmath::scale_from_absmax(rgmath::bitsf(t));
  } else {
    flag = grid_arrive(sync, b, G, spin_limit, &blk[0]);
    if (flag == 0) {
      // waited too long: the finisher quantizes this workgroup's units
      if (tid == 0) {
        __hip_atomic_store(sync + kRequantStateBase + b, rqk::kDeferred, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (stats) atomicAdd(stats + kStatDeferred, 1u);
      }
      return;
    }
    if (tid == 0)
      __hip_atomic_store(sync + kRequantStateBase + b, rqk::kOwn, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t pm = __hip_atomic_load(slot + lane * kSpreadStride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    scale = rgmath::scale_from_absmax(rgmath::bitsf(wave_max_u32(pm)));
  }
  const float inv = 1.0f / scale;
  // pass 2: the kept units, then the rest from the input
#pragma unroll
  for (int j = 0; j < KL; j++) iq_store(rq, lds[tid * KL + j], inv, w0 + (uint32_t)j * kThreads);
#pragma unroll
  for (int j = 0; j < KR; j++) iq_store(rq, keep[j], inv, w0 + (uint32_t)(KL + j) * kThreads);
  iq_quantize_from<VEC>(rx, rq, sh, rest_w, ~0u, rest_r, rest_c, sh.nr, sh.nc, inv);
  if (flag != 2) return;

  // Finisher: the scale tap, then the units of every deferred workgroup.
  if (tid == 0 && scale_out) *scale_out = scale;
  if (G == 1) return;
  uint32_t* const list = blk + 16;  // kListWords words after the block state
  const int ndef = collect_deferred(sync, G, spin_limit, list, &blk[1], stats);
  // the thread index again, from the wave index (scalar) and the lane count,
  // rather than a register held across the whole kernel
  const uint32_t tid2 = (uint32_t)__builtin_amdgcn_readfirstlane(wave) * 64u +
                        __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
  for (int d = 0; d < ndef; d++) {
    const uint32_t rd = iq_range(list[d], (uint32_t)G);
    const uint32_t k0 = iq_kept0(rd, tid2, U), kr0 = k0 / sh.upr;
    iq_quantize_from<VEC>(rx, rq, sh, k0, (uint32_t)U, kr0, k0 - kr0 * sh.upr, sh.kr, sh.kc, inv);
    const uint32_t q0 = iq_rest0(rd, tid2, U, (uint32_t)G), qr0 = q0 / sh.upr;
    iq_quantize_from<VEC>(rx, rq, sh, q0, ~0u, qr0, q0 - qr0 * sh.upr, sh.nr, sh.nc, inv);
  }
}

bool input_quant_supported(int64_t M, int64_t K, int64_t Mpad, int64_t Kpad) {
  // 32-bit byte offsets into the input, the operand, and past them
  return M > 0 && K > 0 && Kpad % 16 == 0 && M <= Mpad && K <= Kpad && Mpad * Kpad * 4 < ((int64_t)1 << 31);
}

// The launch: the smallest U (units kept per thread) whose grid of
// ceil(W / (512 U)) workgroups is resident with at most one workgroup per CU
// (fewer workgroups meet at the barrier: the deep MLP's 4096 x 896 operand
// runs 224 workgroups of U = 8 instead of 448 of U = 4, 0.0470 -> 0.0457 ms
// per step); else the smallest U whose grid is resident; else U = 64 on every
// resident slot (capped by the barrier's kMaxGrid), the rest read twice.
struct IqLaunch {
  int U;
  int64_t G;
};

template <bool VEC, int U>
static const void* iq_fn() {
  return reinterpret_cast<const void*>(&input_quant_kernel<VEC, U>);
}

template <int U>
static int64_t iq_cap() {
  static const int64_t cap = resident_blocks(iq_fn<true, U>(), iq::kThreads);
  return cap < rqk::kMaxGrid ? cap : rqk::kMaxGrid;
}

static int64_t iq_cus() {
  static const int64_t cus = [] {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    return (int64_t)n;
  }();
  return cus;
}

static IqLaunch input_quant_choice(int64_t Mpad, int64_t Kpad) {
  const int64_t W = Mpad * Kpad / 4;
  const int64_t caps[5] = {iq_cap<4>(), iq_cap<8>(), iq_cap<16>(), iq_cap<32>(), iq_cap<64>()};
  // RGNPU_IQ_U (4 .. 64, measurement): no U below it
  static const int min_u = [] {
    const char* e = getenv("RGNPU_IQ_U");
    return e ? atoi(e) : 0;
  }();
  for (int pass = 0; pass < 2; pass++)
    for (int i = 0, U = 4; i < 5; i++, U *= 2) {
      if (U < min_u) continue;
      const int64_t per_block = (int64_t)iq::kThreads * U, G = (W + per_block - 1) / per_block;
      const int64_t limit = pass == 0 && iq_cus() < caps[i] ? iq_cus() : caps[i];
      if (G <= limit) return IqLaunch{U, G < 1 ? 1 : G};
    }
  return IqLaunch{64, caps[4]};
}

int64_t input_quant_sync_words(int64_t Mpad, int64_t Kpad) {
  return rqk::kGoBase + input_quant_choice(Mpad, Kpad).G * rqk::kLine;
}

template <bool VEC, int U>
static void launch_iq(const float* x, const InputQuantShape& sh, int64_t G, uint32_t* slot, int8_t* q,
                      float* scale_out, uint32_t* sync, int spin_limit, uint32_t* stats, SlotClear clear,
                      hipStream_t s) {
  RG_LAUNCH((input_quant_kernel<VEC, U>), dim3((unsigned)G), dim3(iq::kThreads), 0, s, x, sh, slot, q, scale_out, sync,
            spin_limit, stats, clear);
}

template <bool VEC>
static void launch_iq_u(int U, const float* x, const InputQuantShape& sh, int64_t G, uint32_t* slot, int8_t* q,
                        float* scale_out, uint32_t* sync, int spin_limit, uint32_t* stats, SlotClear clear,
                        hipStream_t s) {
  switch (U) {
    case 4: launch_iq<VEC, 4>(x, sh, G, slot, q, scale_out, sync, spin_limit, stats, clear, s); break;
    case 8: launch_iq<VEC, 8>(x, sh, G, slot, q, scale_out, sync, spin_limit, stats, clear, s); break;
    case 16: launch_iq<VEC, 16>(x, sh, G, slot, q, scale_out, sync, spin_limit, stats, clear, s); break;
    case 32: launch_iq<VEC, 32>(x, sh, G, slot, q, scale_out, sync, spin_limit, stats, clear, s); break;
    default: launch_iq<VEC, 64>(x, sh, G, slot, q, scale_out, sync, spin_limit, stats, clear, s); break;
  }
}

void launch_input_quant(const float* x, int64_t M, int64_t K, int64_t Mpad, int64_t Kpad, uint32_t* slot, int8_t* q,
                        float* scale_out, uint32_t* sync, int spin_limit, uint32_t* stats, SlotClear clear,
                        hipStream_t s) {
  if (!input_quant_supported(M, K, Mpad, Kpad) || !slot || !q || !sync || (reinterpret_cast<uintptr_t>(q) & 15))
    throw std::logic_error("input_quant: unsupported shape or missing buffers");
  const bool vec = K % 4 == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0;
  const IqLaunch lc = input_quant_choice(Mpad, Kpad);
  const int64_t W = Mpad * Kpad / 4, NT = lc.G * iq::kThreads, upr = Kpad / 4;
  const InputQuantShape sh{(int32_t)M,          (int32_t)K,          (uint32_t)upr,       (uint32_t)W,
                           (uint32_t)(iq::kThreads / upr), (uint32_t)(iq::kThreads % upr),
                           (uint32_t)(NT / upr), (uint32_t)(NT % upr)};
  if (vec)
    launch_iq_u<true>(lc.U, x, sh, lc.G, slot, q, scale_out, sync, spin_limit, stats, clear, s);
  else
    launch_iq_u<false>(lc.U, x, sh, lc.G, slot, q, scale_out, sync, spin_limit, stats, clear, s);
}

// The poll probe: thread 0 of each workgroup runs the barrier's poll loop
// `polls` times on a line of its own that nothing sets (zeroed by the
// caller), so every poll runs; the other threads wait at the end.
__global__ __launch_bounds__(256) void barrier_poll_probe_kernel(uint32_t* lines, int polls) {
  if (threadIdx.x == 0 && poll_go(lines + (int64_t)blockIdx.x * rqk::kLine, polls)) lines[0] = 2u;
}

double probe_barrier_poll(uint32_t* lines, int blocks, int polls, hipStream_t s) {
  hipEvent_t e0, e1;
  if (hipEventCreate(&e0) != hipSuccess) return -1.0;
  if (hipEventCreate(&e1) != hipSuccess) {
    (void)hipEventDestroy(e0);
    return -1.0;
  }
  (void)hipEventRecord(e0, s);
  hipLaunchKernelGGL(barrier_poll_probe_kernel, dim3((unsigned)blocks), dim3(256), 0, s, lines, polls);
  (void)hipEventRecord(e1, s);
  float ms = -1.0f;
  if (hipGetLastError() == hipSuccess && hipEventSynchronize(e1) == hipSuccess) (void)hipEventElapsedTime(&ms, e0, e1);
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  return ms;
}

// This translation unit is its own code object: loaded at program creation
// with the rest (see load_code_object).
__global__ void requant_load_probe_kernel() {}

void load_requant_code_object(hipStream_t s) {
  hipLaunchKernelGGL(requant_load_probe_kernel, dim3(1), dim3(64), 0, s);
}

bool gemm_requant_supported(int64_t Mpad, int64_t Npad, int64_t Kpad) {
  if (Kpad % big::BK || Mpad % 128 || Npad % 128 || Kpad <= 0) return false;
  // 32-bit offsets: whole rows and 128-row spans of the f32 output and of q
  if (Mpad * Npad * 4 >= ((int64_t)1 << 31) * 64 || Npad * 4 * 128 >= ((int64_t)1 << 31)) return false;
  return choose_gemm(Mpad, Npad, Kpad).splits == 1;
}

int64_t requant_sync_words(int64_t Mpad, int64_t Npad, int64_t Kpad) {
  // the grid never exceeds the tile count or kMaxGrid
  const GemmChoice g = choose_gemm(Mpad, Npad, Kpad);
  const int64_t bm = g.kind == 2 ? 128 : 256, bn = g.kind == 0 ? 256 : 128;
  int64_t T = (Mpad / bm) * (Npad / bn);
  if (T > rqk::kMaxGrid) T = rqk::kMaxGrid;
  return rqk::kGoBase + T * rqk::kLine;
}

void launch_gemm_requant(const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t Mpad, int64_t Npad,
                         int64_t Kpad, const Epilogue& ep, const Requant& rq, hipStream_t s) {
  if (!gemm_requant_supported(Mpad, Npad, Kpad) || N % 4 || M >= ((int64_t)1 << 31))
    throw std::logic_error("requant: the GEMM must be unsplit and N a multiple of 4");
  if (!ep.absmax_out || !rq.q || !rq.sync || rq.ldq <= 0 || rq.ldq > Npad || rq.ldq % 16 ||
      (reinterpret_cast<uintptr_t>(ep.y) & 15) || (reinterpret_cast<uintptr_t>(rq.q) & 15))
    throw std::logic_error("requant: absmax slot, aligned operand and output, and sync words are required");
  if (M <= 0) return;
  const GemmChoice g = choose_gemm(Mpad, Npad, Kpad);
  const int64_t bm = g.kind == 2 ? 128 : 256, bn = g.kind == 0 ? 256 : 128;
  const RequantShape sh{(int32_t)M, (int32_t)N, (int32_t)rq.ldq, (int32_t)(Kpad / big::BK), (int32_t)(Mpad / bm),
                        (int32_t)(Npad / bn)};
  const bool cap = ep.acc_out != nullptr;
  if (g.kind == 0) {
    cap ? launch_requant_shape<256, 256, 2, 4, 4, 1, 8, true>(A, B, sh, Mpad, Npad, Kpad, ep, rq, s)
        : launch_requant_shape<256, 256, 2, 4, 4, 1, 8, false>(A, B, sh, Mpad, Npad, Kpad, ep, rq, s);
  } else if (g.kind == 1) {
    cap ? launch_requant_shape<256, 128, 2, 2, 3, 2, 8, true>(A, B, sh, Mpad, Npad, Kpad, ep, rq, s)
        : launch_requant_shape<256, 128, 2, 2, 3, 2, 8, false>(A, B, sh, Mpad, Npad, Kpad, ep, rq, s);
  } else {
    cap ? launch_requant_shape<128, 128, 2, 2, 4, 2, 4, true>(A, B, sh, Mpad, Npad, Kpad, ep, rq, s)
        : launch_requant_shape<128, 128, 2, 2, 4, 2, 4, false>(A, B, sh, Mpad, Npad, Kpad, ep, rq, s);
  }
}

}  // namespace rgnpu
