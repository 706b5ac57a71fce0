// program.cpp — host runtime of the MI355X INT8 execution provider.
//
// compile  (npu::compile, src/inference/npu.rs:188-276): fold_batch_norm
//          (src/inference/mod.rs:225-257), Linear/Conv2d + Activation fusion,
//          per-tensor i8 weight quantization (quantize.rs:18-24), weight
//          upload in the padded [Npad, Kpad] device layout.
// run      (NpuProgram::execute, npu.rs:296-421): a per-input-shape plan fixes
//          buffers, absmax slots and kernel choices; every op is enqueued on
//          the program's single HIP stream.
// The host arithmetic here (BN folding, weight quantization) is written as
// separate f32 operations and compiled with -ffp-contract=off so it rounds
// exactly like the reference.
#include <hip/hip_runtime_api.h>

#include <charconv>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <array>
#include <condition_variable>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/rgnpu.h"
#include "devmath.h"
#include "hostcopy.h"
#include "rgnpu_internal.h"

namespace rgnpu {

thread_local std::string g_last_error;

struct Error : std::runtime_error {
  int code;
  Error(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

#define RG_HIP(expr)                                                                       \
  do {                                                                                     \
    hipError_t e_ = (expr);                                                                \
    if (e_ != hipSuccess)                                                                  \
      throw Error(RGNPU_ERR_DEVICE, std::string(#expr) + ": " + hipGetErrorString(e_));   \
  } while (0)

struct DevBuf {
  void* p = nullptr;
  size_t bytes = 0;
  bool borrowed = false;  // a view into memory the buffer does not own (the device scratch)
  DevBuf() = default;
  DevBuf(const DevBuf&) = delete;
  DevBuf& operator=(const DevBuf&) = delete;
  ~DevBuf() { release(); }
  void release() {
    if (p && !borrowed) (void)hipFree(p);
    p = nullptr;
    bytes = 0;
    borrowed = false;
  }
  void borrow(void* base, size_t n) {
    release();
    p = base;
    bytes = n;
    borrowed = true;
  }
  void ensure(size_t n) {
    if (n <= bytes && p) return;
    if (borrowed) throw Error(RGNPU_ERR_INVALID, "internal: growing a view into the device scratch");
    release();
    size_t b = n ? n : 16;
    RG_HIP(hipMalloc(&p, b));
    bytes = b;
  }
  template <class T>
  T* as() const { return static_cast<T*>(p); }
};

// ---- label formatting (Display impls, mod.rs:56-67, npu.rs:83-104) ---------
static std::string rust_f32(float v) {
  if (v != v) return "NaN";
  if (std::isinf(v)) return v < 0 ? "-inf" : "inf";
  char buf[128];
  auto res = std::to_chars(buf, buf + sizeof buf, v, std::chars_format::fixed);
  return std::string(buf, res.ptr);
}

static std::string act_display(int act, float p) {
  switch (act) {
    case rgmath::ACT_NONE: return "none";
    case rgmath::ACT_RELU: return "ReLU";
    case rgmath::ACT_SIGMOID: return "Sigmoid";
    case rgmath::ACT_TANH: return "Tanh";
    case rgmath::ACT_GELU: return "GELU";
    case rgmath::ACT_LEAKY_RELU: return "LeakyReLU(" + rust_f32(p) + ")";
    case rgmath::ACT_SILU: return "SiLU";
  }
  return "?";
}

enum OpKind { OP_LINEAR = 1, OP_CONV = 2, OP_AFFINE = 3, OP_POOL = 4, OP_FLATTEN = 5, OP_ACT = 6, OP_SOFTMAX = 7 };

struct Op {
  int kind = 0;
  int64_t in_f = 0, out_f = 0;  // Linear features / Conv2d channels
  int64_t k = 0, s = 0, p = 0;  // Conv2d kernel/stride/pad, MaxPool2d kernel/stride
  int act = 0;
  float act_param = 0.0f;
  std::vector<int8_t> wq;  // [out, K] as the reference holds it (INT8)
  float w_scale = 1.0f;
  std::vector<float> wh;   // FP16: round_fp16 weights [out, K] (npu.rs:210, 232); FP32: the f32 weights [out, K]
  bool diag = false;       // FP16 lone ChannelAffine: elementwise, scale kept as is (npu.rs:254-270)
  std::vector<float> diag_scale;
  std::vector<float> bias;
  int64_t K = 0, Kpad = 0, Npad = 0;  // Kpad in bytes (INT8) or binary16 elements (FP16)
  DevBuf d_w, d_bias, d_scale;
  std::string label;
};

enum { BUF_INPUT = -1, BUF_OUTPUT = -2 };

struct OpPlan {
  std::vector<int64_t> in_shape, out_shape;
  int64_t in_len = 0, out_len = 0;
  int in_buf = BUF_INPUT, out_buf = BUF_OUTPUT;
  uint64_t macs = 0;
  int64_t rows = 0, Mpad = 0;
  bool gemv = false;
  ConvShape cs{};
  bool full_cov = true;
  int64_t mask_off = 0;       // offset of row/col coverage masks in Plan::masks
  int64_t slot_base = -1, slot_count = 0;  // slot words offset; scales this op quantizes with
  int64_t scale_base = -1;                  // index of its first scale in Plan::scales
  bool explicit_absmax = true;
  int64_t emit_slot = -1;     // this op's kernel writes absmax into slots[emit_slot..]
  int emit_per_image = 0;
  // INT8 Linear -> Linear: the producer's GEMM also quantizes the consumer's
  // input (requant.hip); the consumer then skips its quantize pass.
  bool requant = false;       // this op's GEMM writes the next Linear's i8 operand
  int consumer = -1;          // that Linear's op index
  int64_t sync_base = -1;     // its barrier words in the slot set
  bool q_ready = false;       // this op's i8 operand was written by its producer
  int q_in = 0;               // which of the two i8 operand buffers this op's GEMM reads
  // INT8 Linear quantizing its own input (explicit absmax): the one-pass
  // kernel's barrier words in the slot set, or -1 for the absmax + quantize
  // kernel pair.
  int64_t iq_sync_base = -1;
  // FP16 Linear -> FP16 Linear: the producer's GEMM epilogue writes the
  // consumer's binary16 operand (q_ready / q_in of the consumer as above).
  bool handoff = false;
  // Conv -> MaxPool2d(2, 2) in the conv (FP32: conv -> Act -> pool):
  // pool_r16 (OW / 16) on the conv, which writes the pooled output to its
  // out_buf; pool_fused on the ops it absorbs, which launch nothing and pass
  // that buffer on.
  int pool_r16 = 0;
  int pool_act = 0;  // FP32: the activation of the Act op it absorbs
  bool pool_fused = false;
  // INT8 conv + pool, conv + pool on one image per workgroup
  // (launch_conv_pool_pair): 1 on the first conv, which launches it, 2 on
  // the second, which launches nothing; no_out on the first pool, whose
  // output stays in LDS.
  int pair = 0;
  bool no_out = false;
  // INT8 Linear with few output tiles reading its f32 input and quantizing
  // it as it reads it (launch_gemm_xq_small): no quantize pass before it.
  bool small_xq = false;
  int64_t xq_sync_base = -1;  // its 64-bit sum words in the slot set (K slices), or -1
};

struct Plan {
  std::vector<int64_t> in_shape, out_shape;
  bool capture = false;  // made for capture runs (no conv-pool fusion)
  // made while persistent grids (fused requantization, one-pass input
  // quantization) were allowed
  bool persistent = true;
  bool tiny = false;       // the whole program is one mlp_tiny_kernel launch (by the first op)
  int64_t in_len = 0, out_len = 0;
  std::vector<OpPlan> ops;
  size_t f32_elems = 0, q_bytes = 0, ylo_elems = 0;
  int64_t n_slots = 0;
  // Slot sets: with clear_by_first the slots are two sets of n_slots words;
  // run k uses set `parity` and its first kernel (the input absmax) zeroes
  // the other one for run k + 1.  Otherwise one set, filled with zeros at
  // the start of every run.
  bool clear_by_first = false;
  int parity = 0;
  int64_t slot_set_words = 0;  // n_slots rounded up to a 128-byte multiple
  DevBuf f32[2], q, slots, scales, masks, host_in, host_out;
  DevBuf q_alt;  // second i8 operand buffer: a fused producer writes the one its GEMM does not read
  int spin_limit = 0;  // requant barrier polls before a workgroup defers (RGNPU_REQUANT_SPIN_LIMIT)
  int gelu_cert = 1;   // GELU requantization (RGNPU_GELU_CERT): 1 certified, 0 exact; 2, 3 test modes (requant.hip)
  DevBuf ylo;  // FP16 conv: GEMM output [n*L, O] before the NCHW transpose
  DevBuf ws;  // split-K partial sums
  int64_t ws_bytes = 0;
  // Allocation-free plan: every buffer above is a view into the device
  // scratch, which other calls overwrite, so each run zeroes its slots and
  // uploads the coverage masks again (kept here).
  bool in_scratch = false;
  std::vector<uint8_t> mask_host;
  std::vector<std::unique_ptr<DevBuf>> cap_q, cap_acc, cap_out;
  bool capture_ready = false;
  // Production taps (test only): per op, a copy of its absmax slot words and
  // whether its i8 operand (cap_q) and f32 output (cap_out) exist in memory
  // on the production path.
  std::vector<std::unique_ptr<DevBuf>> tap_slot;
  std::vector<uint8_t> tap_q_ok, tap_out_ok, tap_scale_ok;
  bool taps_ready = false;
  // Per op, indices into the run's launch events (-1 = the run-start event):
  // [0] last launch before the op, [1] last launch before its main kernel,
  // [2] its main kernel (== [1] when the op launches none).
  std::vector<std::array<int, 3>> roles;
};

}  // namespace rgnpu

using namespace rgnpu;

struct rgnpu_program {
  int device = 0;
  int precision = RGNPU_PRECISION_INT8;
  hipStream_t stream = nullptr;
  int64_t original_layers = 0;
  int64_t fp32_bytes = 0, npu_bytes = 0;
  std::vector<std::shared_ptr<Op>> ops;  // device weights; shared with the workers
  std::unique_ptr<Plan> plan;
  std::unique_ptr<Plan> scratch_plan;  // plan of rgnpu_program_run_device_noalloc
  void* scratch = nullptr;             // this device's scratch array (scratch.hip)
  int profiling = 1;
  bool capture = false;
  bool capture_valid = false;
  // Production taps: the production plan and kernels run unchanged, and the
  // operands, absmax slots and outputs that exist in memory are copied after
  // each op (rgnpu_program_set_capture(prog, RGNPU_CAPTURE_PRODUCTION)).
  bool taps = false;
  bool taps_valid = false;
  std::vector<hipEvent_t> ev;  // run start/end + launch events
  bool profile_pending = false;
  bool have_profile = false;
  rgnpu_profile prof{};
  std::vector<rgnpu_op_record> records;
  std::mutex mu;
  // Concurrent host runs (InferenceSession::run takes &self and is Sync,
  // mod.rs:146-151, 212-221): each call borrows a worker -- the same ops
  // (weights), its own stream, plans and events -- so calls on one handle
  // run side by side on the device, their copies overlapping other calls'
  // kernels.  The handle's own stream serves run_device, benchmark and
  // capture.
  std::mutex pool_mu;
  std::condition_variable pool_cv;
  std::vector<std::unique_ptr<rgnpu_program>> workers;
  std::vector<char> worker_busy;
  rgnpu::Staging staging;  // pinned ring for this stream's host copies
  DevBuf evict;            // zero buffer read between benchmark runs on request
  // This context's cumulative barrier counters (kStat*, requant.hip), a
  // pinned copy of them read after each synchronization, and the unsettled
  // count already reported.
  DevBuf stats;
  uint32_t* stats_host = nullptr;
  uint32_t unsettled_seen = 0;
  // Whether this context's next run may use persistent grids (make_plan):
  // the handle's runs always; a worker's runs until the program has once had
  // two host runs in flight together (concurrent_seen, set by the handle
  // and sticky).  The plan of the other kind is kept in plan_other, so a
  // change of kind does not rebuild plans.
  bool use_persistent = true;
  bool concurrent_seen = false;
  std::unique_ptr<Plan> plan_other;
};

// Bytes read between benchmark runs to displace the 256 MB memory-side cache.
static constexpr int64_t kEvictBytes = int64_t(512) << 20;

// Upper bound on workers (concurrent host runs) per handle.
static constexpr size_t kMaxWorkers = 8;

namespace rgnpu {

static void check_layer(const rgnpu_layer& l, int64_t idx) {
  auto bad = [&](const std::string& m) { throw Error(RGNPU_ERR_INVALID, "layer " + std::to_string(idx) + ": " + m); };
  // Every size the kernels index with fits 31 bits; the ABI fields are 64-bit
  // only so that any u32 of an .rtim file reads back unchanged.
  constexpr int64_t kMaxField = INT32_MAX;
  auto too_big = [&](std::initializer_list<int64_t> v) {
    for (int64_t x : v)
      if (x > kMaxField) bad("size field above 2^31 - 1 is not supported");
  };
  switch (l.kind) {
    case RGNPU_LAYER_LINEAR:
      too_big({l.in_features, l.out_features});
      if (l.in_features <= 0 || l.out_features <= 0) bad("Linear needs positive in/out features");
      // the GEMM epilogue addresses 16 output rows with 32-bit byte offsets
      if (l.out_features > (1 << 26)) bad("Linear out_features above 2^26 are not supported");
      if (l.weight_len != l.in_features * l.out_features || !l.weight) bad("Linear weight must be [in, out]");
      if (l.bias_len != l.out_features || !l.bias) bad("Linear bias must have out_features elements");
      break;
    case RGNPU_LAYER_CONV2D:
      too_big({l.in_channels, l.out_channels, l.kernel, l.stride, l.padding});
      if (l.in_channels <= 0 || l.out_channels <= 0 || l.kernel <= 0 || l.stride <= 0 || l.padding < 0)
        bad("Conv2d needs positive channels/kernel/stride and padding >= 0");
      if ((__int128)l.weight_len != (__int128)l.out_channels * l.in_channels * l.kernel * l.kernel || !l.weight)
        bad("Conv2d weight must be [out, in, k, k]");
      if (l.bias_len != l.out_channels || !l.bias) bad("Conv2d bias must have out_channels elements");
      break;
    case RGNPU_LAYER_CHANNEL_AFFINE:
      too_big({l.scale_len});
      if (l.scale_len <= 0 || !l.scale || !l.shift) bad("ChannelAffine needs scale and shift");
      // fold_batch_norm and the lone affine read shift[c] for c < scale.len()
      // (mod.rs:236-237, 246, 302; npu.rs:254-268): a shorter shift panics there
      if (l.shift_len < l.scale_len) bad("ChannelAffine shift is shorter than its scale");
      break;
    case RGNPU_LAYER_MAXPOOL2D:
      too_big({l.pool_kernel, l.pool_stride});
      if (l.pool_kernel <= 0 || l.pool_stride <= 0) bad("MaxPool2d needs positive kernel and stride");
      break;
    case RGNPU_LAYER_FLATTEN:
    case RGNPU_LAYER_SOFTMAX:
      break;
    case RGNPU_LAYER_ACTIVATION:
      if (l.act < RGNPU_ACT_NONE || l.act > RGNPU_ACT_SILU) bad("unknown activation code");
      break;
    default:
      bad("unknown layer kind");
  }
}

// Folded layer (owning copies), fold_batch_norm (inference/mod.rs:225-257).
struct FLayer {
  rgnpu_layer spec{};
  std::vector<float> w, b, scale, shift;
};

static std::vector<FLayer> fold_batch_norm(const rgnpu_layer* L, int64_t n) {
  std::vector<FLayer> out;
  out.reserve((size_t)n);
  for (int64_t i = 0; i < n; i++) {
    const rgnpu_layer& l = L[i];
    if (l.kind == RGNPU_LAYER_CHANNEL_AFFINE && !out.empty()) {
      FLayer& last = out.back();
      if (last.spec.kind == RGNPU_LAYER_LINEAR && last.spec.out_features == l.scale_len) {
        const int64_t in = last.spec.in_features, of = last.spec.out_features;
        for (int64_t r = 0; r < in; r++)
          for (int64_t c = 0; c < of; c++) last.w[r * of + c] = last.w[r * of + c] * l.scale[c];
        for (int64_t c = 0; c < of; c++) {
          const float t = last.b[c] * l.scale[c];
          last.b[c] = t + l.shift[c];
        }
        continue;
      }
      if (last.spec.kind == RGNPU_LAYER_CONV2D && last.spec.out_channels == l.scale_len) {
        const int64_t plane = (int64_t)last.spec.in_channels * last.spec.kernel * last.spec.kernel;
        for (int64_t o = 0; o < last.spec.out_channels; o++) {
          for (int64_t j = 0; j < plane; j++) last.w[o * plane + j] = last.w[o * plane + j] * l.scale[o];
          const float t = last.b[o] * l.scale[o];
          last.b[o] = t + l.shift[o];
        }
        continue;
      }
    }
    FLayer f;
    f.spec = l;
    if (l.kind == RGNPU_LAYER_LINEAR || l.kind == RGNPU_LAYER_CONV2D) {
      f.w.assign(l.weight, l.weight + l.weight_len);
      f.b.assign(l.bias, l.bias + l.bias_len);
    } else if (l.kind == RGNPU_LAYER_CHANNEL_AFFINE) {
      // entries of a longer shift past scale.len() are never read
      f.scale.assign(l.scale, l.scale + l.scale_len);
      f.shift.assign(l.shift, l.shift + l.scale_len);
    }
    out.push_back(std::move(f));
  }
  return out;
}

// QuantTensor::from_f32 (quantize.rs:18-24) on the host.
static float quantize_host(const float* v, int64_t n, int8_t* out) {
  float max_abs = 0.0f;
  for (int64_t i = 0; i < n; i++) max_abs = std::fmax(max_abs, std::fabs(v[i]));
  const float scale = rgmath::scale_from_absmax(max_abs);
  const float inv = 1.0f / scale;
  for (int64_t i = 0; i < n; i++) out[i] = rgmath::quantize_one(v[i], inv);
  return scale;
}

// FP16: binary16 [Npad, Kpad] from the rounded weights in the reference
// order (Linear [out, in], Conv [out, c*k*k]), zero padded.
static void upload_weights_f16(Op& op, hipStream_t s) {
  std::vector<float> bpad((size_t)std::max<int64_t>(op.Npad, (int64_t)op.bias.size()), 0.0f);
  std::memcpy(bpad.data(), op.bias.data(), sizeof(float) * op.bias.size());
  op.d_bias.ensure(bpad.size() * sizeof(float));
  RG_HIP(hipMemcpyAsync(op.d_bias.p, bpad.data(), bpad.size() * sizeof(float), hipMemcpyHostToDevice, s));
  if (op.diag) {
    op.d_scale.ensure(op.diag_scale.size() * sizeof(float));
    RG_HIP(hipMemcpyAsync(op.d_scale.p, op.diag_scale.data(), op.diag_scale.size() * sizeof(float),
                          hipMemcpyHostToDevice, s));
  } else {
    std::vector<uint16_t> h((size_t)(op.Npad * op.Kpad), 0);
    for (int64_t r = 0; r < op.out_f; r++)
      for (int64_t c = 0; c < op.K; c++) h[(size_t)(r * op.Kpad + c)] = rgmath::fp16_bits(op.wh[(size_t)(r * op.K + c)]);
    op.d_w.ensure(h.size() * sizeof(uint16_t));
    RG_HIP(hipMemcpyAsync(op.d_w.p, h.data(), h.size() * sizeof(uint16_t), hipMemcpyHostToDevice, s));
  }
  RG_HIP(hipStreamSynchronize(s));
}

static void upload_weights(Op& op, hipStream_t s) {
  // Linear: [N, K] host -> [Npad, Kpad] device, zero padded.  Conv: the
  // reference [O, C*k*k] order becomes tap-major [Opad, Kpad], kk' =
  // (ki*k + kj)*cp + c (see ConvShape).
  std::vector<int8_t> pad((size_t)(op.Npad * op.Kpad), 0);
  if (op.kind == OP_CONV) {
    const int64_t C = op.in_f, k = op.k, cp = conv_cp(C);
    for (int64_t o = 0; o < op.out_f; o++)
      for (int64_t c = 0; c < C; c++)
        for (int64_t ki = 0; ki < k; ki++)
          for (int64_t kj = 0; kj < k; kj++)
            pad[(size_t)(o * op.Kpad + (ki * k + kj) * cp + c)] = op.wq[(size_t)(o * op.K + (c * k + ki) * k + kj)];
  } else {
    for (int64_t r = 0; r < op.out_f; r++)
      std::memcpy(&pad[(size_t)(r * op.Kpad)], &op.wq[(size_t)(r * op.K)], (size_t)op.K);
  }
  std::vector<float> bpad((size_t)op.Npad, 0.0f);
  std::memcpy(bpad.data(), op.bias.data(), sizeof(float) * op.bias.size());
  op.d_w.ensure(pad.size());
  op.d_bias.ensure(bpad.size() * sizeof(float));
  RG_HIP(hipMemcpyAsync(op.d_w.p, pad.data(), pad.size(), hipMemcpyHostToDevice, s));
  RG_HIP(hipMemcpyAsync(op.d_bias.p, bpad.data(), bpad.size() * sizeof(float), hipMemcpyHostToDevice, s));
  RG_HIP(hipStreamSynchronize(s));
}

static std::string op_label(const Op& op) {
  const std::string a = act_display(op.act, op.act_param);
  char buf[256];
  switch (op.kind) {
    case OP_LINEAR:
      if (op.act == rgmath::ACT_NONE)
        snprintf(buf, sizeof buf, "NPU::Gemm(%lld->%lld)", (long long)op.in_f, (long long)op.out_f);
      else
        snprintf(buf, sizeof buf, "NPU::FusedGemmAct(%lld->%lld, %s)", (long long)op.in_f, (long long)op.out_f, a.c_str());
      break;
    case OP_CONV:
      if (op.act == rgmath::ACT_NONE)
        snprintf(buf, sizeof buf, "NPU::Conv2d(%lld->%lld, k=%lld)", (long long)op.in_f, (long long)op.out_f, (long long)op.k);
      else
        snprintf(buf, sizeof buf, "NPU::FusedConv2dAct(%lld->%lld, k=%lld, %s)", (long long)op.in_f, (long long)op.out_f,
                 (long long)op.k, a.c_str());
      break;
    case OP_POOL: snprintf(buf, sizeof buf, "NPU::MaxPool2d(k=%lld)", (long long)op.k); break;
    case OP_FLATTEN: snprintf(buf, sizeof buf, "NPU::Flatten"); break;
    case OP_ACT: snprintf(buf, sizeof buf, "NPU::Act(%s)", a.c_str()); break;
    case OP_SOFTMAX: snprintf(buf, sizeof buf, "NPU::Softmax"); break;
    default: snprintf(buf, sizeof buf, "?");
  }
  return buf;
}

// FP32 weights [Npad, Kpad_f] (Linear transposed to [out, in], Conv [O, c*k*k]), zero padded.
static void upload_weights_f32(Op& op, hipStream_t s) {
  std::vector<float> bpad((size_t)std::max<int64_t>(op.Npad, (int64_t)op.bias.size()), 0.0f);
  std::memcpy(bpad.data(), op.bias.data(), sizeof(float) * op.bias.size());
  op.d_bias.ensure(bpad.size() * sizeof(float));
  RG_HIP(hipMemcpyAsync(op.d_bias.p, bpad.data(), bpad.size() * sizeof(float), hipMemcpyHostToDevice, s));
  if (op.kind == OP_AFFINE) {
    op.d_scale.ensure(op.diag_scale.size() * sizeof(float));
    RG_HIP(hipMemcpyAsync(op.d_scale.p, op.diag_scale.data(), op.diag_scale.size() * sizeof(float),
                          hipMemcpyHostToDevice, s));
  } else {
    std::vector<float> w((size_t)(op.Npad * op.Kpad), 0.0f);
    for (int64_t r = 0; r < op.out_f; r++)
      std::memcpy(&w[(size_t)(r * op.Kpad)], &op.wh[(size_t)(r * op.K)], sizeof(float) * (size_t)op.K);
    op.d_w.ensure(w.size() * sizeof(float));
    RG_HIP(hipMemcpyAsync(op.d_w.p, w.data(), w.size() * sizeof(float), hipMemcpyHostToDevice, s));
  }
  RG_HIP(hipStreamSynchronize(s));
}

// The standard FP32 program of ExecutionProvider::Gpu(i): the folded layers
// (InferenceSession::from_layers, mod.rs:168-171) run one by one as
// run_standard does (mod.rs:260-331) -- no Linear/Activation fusion, and a
// ChannelAffine that did not fold stays an elementwise affine.
static void compile_standard(rgnpu_program* P, const std::vector<FLayer>& F) {
  for (const FLayer& f : F) {
    auto op = std::make_unique<Op>();
    char buf[160];
    switch (f.spec.kind) {
      case RGNPU_LAYER_LINEAR: {
        op->kind = OP_LINEAR;
        op->in_f = f.spec.in_features;
        op->out_f = f.spec.out_features;
        op->K = op->in_f;
        op->wh.resize((size_t)(op->in_f * op->out_f));
        for (int64_t r = 0; r < op->in_f; r++)
          for (int64_t c = 0; c < op->out_f; c++) op->wh[(size_t)(c * op->in_f + r)] = f.w[(size_t)(r * op->out_f + c)];
        op->bias = f.b;
        op->Npad = round_up(op->out_f, kRowPad);
        op->Kpad = round_up(op->K, kKPadF32);
        snprintf(buf, sizeof buf, "GPU::Linear(%lld->%lld)", (long long)op->in_f, (long long)op->out_f);
        break;
      }
      case RGNPU_LAYER_CONV2D:
        op->kind = OP_CONV;
        op->in_f = f.spec.in_channels;
        op->out_f = f.spec.out_channels;
        op->k = f.spec.kernel;
        op->s = f.spec.stride;
        op->p = f.spec.padding;
        op->K = op->in_f * op->k * op->k;
        op->wh = f.w;  // [O, c*k*k]
        op->bias = f.b;
        op->Npad = round_up(op->out_f, 128);
        op->Kpad = round_up(op->K, kKPadF32);
        snprintf(buf, sizeof buf, "GPU::Conv2d(%lld->%lld, k=%lld)", (long long)op->in_f, (long long)op->out_f,
                 (long long)op->k);
        break;
      case RGNPU_LAYER_CHANNEL_AFFINE:
        op->kind = OP_AFFINE;
        op->in_f = op->out_f = (int64_t)f.scale.size();
        op->diag_scale = f.scale;
        op->bias = f.shift;
        snprintf(buf, sizeof buf, "GPU::ChannelAffine(%lld)", (long long)op->in_f);
        break;
      case RGNPU_LAYER_MAXPOOL2D:
        op->kind = OP_POOL;
        op->k = f.spec.pool_kernel;
        op->s = f.spec.pool_stride;
        snprintf(buf, sizeof buf, "GPU::MaxPool2d(k=%lld)", (long long)op->k);
        break;
      case RGNPU_LAYER_FLATTEN:
        op->kind = OP_FLATTEN;
        snprintf(buf, sizeof buf, "GPU::Flatten");
        break;
      case RGNPU_LAYER_ACTIVATION:
        op->kind = OP_ACT;
        op->act = f.spec.act;
        op->act_param = f.spec.act_param;
        snprintf(buf, sizeof buf, "GPU::Act(%s)", act_display(op->act, op->act_param).c_str());
        break;
      default:
        op->kind = OP_SOFTMAX;
        snprintf(buf, sizeof buf, "GPU::Softmax");
        break;
    }
    if (op->kind == OP_LINEAR || op->kind == OP_CONV) P->fp32_bytes += (int64_t)(f.w.size() + f.b.size()) * 4;
    if (op->kind == OP_LINEAR || op->kind == OP_CONV || op->kind == OP_AFFINE) upload_weights_f32(*op, P->stream);
    op->label = buf;
    P->ops.push_back(std::move(op));
  }
  P->npu_bytes = P->fp32_bytes;
}

// npu::compile (npu.rs:188-276).
static void compile(rgnpu_program* P, const rgnpu_layer* layers, int64_t n) {
  const bool f16 = P->precision == RGNPU_PRECISION_FP16;
  P->original_layers = n;  // every layer passed check_layer in rgnpu_program_create
  std::vector<FLayer> F = fold_batch_norm(layers, n);
  if (P->precision == RGNPU_PRECISION_FP32) {
    compile_standard(P, F);
    return;
  }
  size_t i = 0;
  while (i < F.size()) {
    const bool has_act = i + 1 < F.size() && F[i + 1].spec.kind == RGNPU_LAYER_ACTIVATION;
    auto op = std::make_unique<Op>();
    const FLayer& f = F[i];
    if (f.spec.kind == RGNPU_LAYER_LINEAR || f.spec.kind == RGNPU_LAYER_CONV2D) {
      op->act = has_act ? F[i + 1].spec.act : rgmath::ACT_NONE;
      op->act_param = has_act ? F[i + 1].spec.act_param : 0.0f;
      if (has_act) i++;
    }
    if (f.spec.kind == RGNPU_LAYER_LINEAR) {
      op->kind = OP_LINEAR;
      op->in_f = f.spec.in_features;
      op->out_f = f.spec.out_features;
      op->K = op->in_f;
      // transpose2d [in,out] -> [out,in] (npu.rs:208), then per-tensor quantize.
      std::vector<float> wt((size_t)(op->in_f * op->out_f));
      for (int64_t r = 0; r < op->in_f; r++)
        for (int64_t c = 0; c < op->out_f; c++) wt[(size_t)(c * op->in_f + r)] = f.w[(size_t)(r * op->out_f + c)];
      op->bias = f.b;
      P->fp32_bytes += (int64_t)(f.w.size() + f.b.size()) * 4;
      op->Npad = round_up(op->out_f, kRowPad);
      if (f16) {
        op->wh.resize(wt.size());
        for (size_t j = 0; j < wt.size(); j++) op->wh[j] = rgmath::round_fp16(wt[j]);
        P->npu_bytes += (int64_t)(f.w.size() + f.b.size()) * 2;
        op->Kpad = round_up(op->K, kKPadHalf);
      } else {
        op->wq.resize(wt.size());
        op->w_scale = quantize_host(wt.data(), (int64_t)wt.size(), op->wq.data());
        P->npu_bytes += ((int64_t)op->wq.size() + 4) + (int64_t)f.b.size() * 4;
        op->Kpad = round_up(op->K, kKPad);
      }
    } else if (f.spec.kind == RGNPU_LAYER_CONV2D) {
      op->kind = OP_CONV;
      op->in_f = f.spec.in_channels;
      op->out_f = f.spec.out_channels;
      op->k = f.spec.kernel;
      op->s = f.spec.stride;
      op->p = f.spec.padding;
      op->K = op->in_f * op->k * op->k;
      op->bias = f.b;
      P->fp32_bytes += (int64_t)(f.w.size() + f.b.size()) * 4;
      if (f16) {
        // the conv runs as im2col + GEMM: output channels are the GEMM's N
        op->wh.resize(f.w.size());
        for (size_t j = 0; j < f.w.size(); j++) op->wh[j] = rgmath::round_fp16(f.w[j]);
        P->npu_bytes += (int64_t)(f.w.size() + f.b.size()) * 2;
        op->Npad = round_up(op->out_f, 128);  // the GEMM's smallest N tile
        op->Kpad = round_up(op->K, kKPadHalf);
      } else {
        op->wq.resize(f.w.size());
        op->w_scale = quantize_host(f.w.data(), (int64_t)f.w.size(), op->wq.data());  // [out, c*k*k] (npu.rs:231)
        P->npu_bytes += ((int64_t)op->wq.size() + 4) + (int64_t)f.b.size() * 4;
        op->Npad = round_up(op->out_f, kConvOPad);
        op->Kpad = conv_kpad(op->in_f, op->k);
      }
    } else if (f.spec.kind == RGNPU_LAYER_CHANNEL_AFFINE) {
      // Lone ChannelAffine -> diagonal Linear, no byte accounting (npu.rs:254-270).
      const int64_t c = (int64_t)f.scale.size();
      std::vector<float> w((size_t)(c * c), 0.0f);
      for (int64_t j = 0; j < c; j++) w[(size_t)(j * c + j)] = f.scale[(size_t)j];
      op->kind = OP_LINEAR;
      op->in_f = op->out_f = op->K = c;
      op->act = rgmath::ACT_NONE;
      op->bias = f.shift;
      op->Npad = round_up(c, kRowPad);
      if (f16) {
        op->diag = true;
        op->diag_scale = f.scale;
        op->Kpad = round_up(c, kKPadHalf);
      } else {
        op->wq.resize(w.size());
        op->w_scale = quantize_host(w.data(), (int64_t)w.size(), op->wq.data());
        op->Kpad = round_up(c, kKPad);
      }
    } else if (f.spec.kind == RGNPU_LAYER_MAXPOOL2D) {
      op->kind = OP_POOL;
      op->k = f.spec.pool_kernel;
      op->s = f.spec.pool_stride;
    } else if (f.spec.kind == RGNPU_LAYER_FLATTEN) {
      op->kind = OP_FLATTEN;
    } else if (f.spec.kind == RGNPU_LAYER_ACTIVATION) {
      op->kind = OP_ACT;
      op->act = f.spec.act;
      op->act_param = f.spec.act_param;
    } else if (f.spec.kind == RGNPU_LAYER_SOFTMAX) {
      op->kind = OP_SOFTMAX;
    }
    if (op->kind == OP_LINEAR || op->kind == OP_CONV) {
      if (f16)
        upload_weights_f16(*op, P->stream);
      else
        upload_weights(*op, P->stream);
    }
    op->label = op_label(*op);
    P->ops.push_back(std::move(op));
    i++;
  }
}

static int64_t out_size(int64_t input, int64_t k, int64_t s, int64_t pad) {  // kernels.rs:10-15
  const int64_t padded = input + 2 * pad;
  if (padded < k) throw Error(RGNPU_ERR_SHAPE, "kernel " + std::to_string(k) + " larger than padded input " + std::to_string(padded));
  return (padded - k) / s + 1;
}

// Coverage of one spatial axis by the conv windows: position i is read by
// some window iff i = o*s + t - pad for o < out, t < k.
static std::vector<uint8_t> coverage(int64_t size, int64_t k, int64_t s, int64_t pad, int64_t out) {
  std::vector<uint8_t> m((size_t)size, 0);
  for (int64_t o = 0; o < out; o++)
    for (int64_t t = 0; t < k; t++) {
      const int64_t i = o * s + t - pad;
      if (i >= 0 && i < size) m[(size_t)i] = 1;
    }
  return m;
}

static int64_t numel(const std::vector<int64_t>& s) {
  int64_t n = 1;
  for (int64_t v : s) n *= v;
  return n;
}

// Conv i followed by MaxPool2d(2, 2) that the conv can do itself: ReLU or
// no activation, even output height and width of 16 or 32, no capture
// (which keeps the conv's own output); INT8 on the band kernel
// (conv_band_epilogue_pool2, when a tile width fits), FP16 and FP32 on the
// direct conv (conv_direct_pool).  FP32 convs carry no activation: there
// the pattern is conv, Act (ReLU or none), pool.  Returns OW / 16, or 0,
// with *span the number of ops after the conv that it absorbs and *act the
// activation it applies.  RGNPU_CONV_POOL=0 turns the fusion off.
static int conv_pool_fusion(const rgnpu_program* P, const std::vector<OpPlan>& plan_ops, size_t i, int* span,
                            int* act) {
  const char* e = getenv("RGNPU_CONV_POOL");
  const bool f32 = P->precision == RGNPU_PRECISION_FP32;
  const size_t n = f32 ? 2 : 1;
  if ((e && atoi(e) == 0) || P->capture || i + n >= P->ops.size()) return 0;
  const Op& op = *P->ops[i];
  const Op& pool = *P->ops[i + n];
  if (op.kind != OP_CONV || pool.kind != OP_POOL || pool.k != 2 || pool.s != 2) return 0;
  int a = op.act;
  if (f32) {
    if (P->ops[i + 1]->kind != OP_ACT) return 0;
    a = P->ops[i + 1]->act;
  }
  if (a != rgmath::ACT_NONE && a != rgmath::ACT_RELU) return 0;
  const ConvShape& c = plan_ops[i].cs;
  if (c.OH % 2 != 0 || (c.OW != 16 && c.OW != 32) || c.n <= 0) return 0;
  const int r16 = (int)(c.OW / 16);
  *span = (int)n;
  *act = a;
  if (P->precision != RGNPU_PRECISION_INT8)  // the direct conv, as enqueue picks it
    return plan_ops[i].rows > 0 && op.K <= kDirectConvTaps && op.out_f <= 64 ? r16 : 0;
  return conv_pool_supported(c, r16) ? r16 : 0;
}

// With `scratch` the plan's buffers are views into that device array (of
// kScratchBytes) instead of allocations of their own.

static std::unique_ptr<Plan> make_plan(rgnpu_program* P, const int64_t* shape, int ndim, void* scratch = nullptr) {
  if (ndim < 1 || ndim > 8) throw Error(RGNPU_ERR_SHAPE, "input rank must be 1..8");
  auto plan = std::make_unique<Plan>();
  plan->in_shape.assign(shape, shape + ndim);
  for (int64_t v : plan->in_shape)
    if (v < 0) throw Error(RGNPU_ERR_SHAPE, "negative dimension");
  plan->in_len = numel(plan->in_shape);
  std::vector<int64_t> cur = plan->in_shape;
  std::vector<uint8_t> mask_host;
  const size_t nops = P->ops.size();
  plan->ops.resize(nops);
  for (size_t i = 0; i < nops; i++) {
    const Op& op = *P->ops[i];
    OpPlan& pl = plan->ops[i];
    pl.in_shape = cur;
    pl.in_len = numel(cur);
    switch (op.kind) {
      case OP_LINEAR: {  // npu.rs:307-318
        if (pl.in_len % op.in_f != 0)
          throw Error(RGNPU_ERR_SHAPE, "Linear(" + std::to_string(op.in_f) + "): input length " + std::to_string(pl.in_len) +
                                           " is not a multiple of in_features");
        pl.rows = pl.in_len / op.in_f;
        pl.macs = (uint64_t)(pl.rows * op.in_f * op.out_f);
        pl.gemv = pl.rows <= 8;
        // the GEMV reads exactly `rows` activation rows; the MFMA GEMM reads
        // whole 256-row tiles
        pl.Mpad = pl.gemv ? (pl.rows > 0 ? pl.rows : 1) : round_up(pl.rows > 0 ? pl.rows : 1, kRowPad);
        cur.back() = op.out_f;
        break;
      }
      case OP_CONV: {  // npu.rs:319-383
        if (cur.size() < 4) throw Error(RGNPU_ERR_SHAPE, "Conv2d expects NCHW input");
        const int64_t n = cur[0], c = cur[1], h = cur[2], w = cur[3];
        if (c != op.in_f)
          throw Error(RGNPU_ERR_SHAPE, "Conv2d: input has " + std::to_string(c) + " channels, expected " + std::to_string(op.in_f));
        const int64_t oh = out_size(h, op.k, op.s, op.p), ow = out_size(w, op.k, op.s, op.p);
        pl.cs = ConvShape{n, c, h, w, op.out_f, op.Npad, op.k, op.s, op.p, oh, ow, op.Kpad, conv_cp(c)};
        pl.macs = (uint64_t)(n * op.out_f * op.K * oh * ow);
        pl.rows = n * oh * ow;  // FP16: GEMM rows of the im2col matrix
        pl.Mpad = round_up(pl.rows > 0 ? pl.rows : 1, kRowPad);
        auto rm = coverage(h, op.k, op.s, op.p, oh), cm = coverage(w, op.k, op.s, op.p, ow);
        pl.full_cov = true;
        for (auto v : rm) pl.full_cov &= v != 0;
        for (auto v : cm) pl.full_cov &= v != 0;
        pl.mask_off = (int64_t)mask_host.size();
        mask_host.insert(mask_host.end(), rm.begin(), rm.end());
        mask_host.insert(mask_host.end(), cm.begin(), cm.end());
        cur = {n, op.out_f, oh, ow};
        break;
      }
      case OP_POOL: {  // npu.rs:384-390
        if (cur.size() < 4) throw Error(RGNPU_ERR_SHAPE, "MaxPool2d expects NCHW input");
        const int64_t oh = out_size(cur[2], op.k, op.s, 0), ow = out_size(cur[3], op.k, op.s, 0);
        cur = {cur[0], cur[1], oh, ow};
        break;
      }
      case OP_FLATTEN: {  // npu.rs:391-394
        int64_t rest = 1;
        for (size_t d = 1; d < cur.size(); d++) rest *= cur[d];
        cur = {cur[0], rest};
        break;
      }
      case OP_AFFINE: {  // mod.rs:295-306: channels on axis 1
        if (cur.size() < 2 || cur[1] != op.in_f)
          throw Error(RGNPU_ERR_SHAPE, "ChannelAffine(" + std::to_string(op.in_f) + "): input axis 1 must have " +
                                           std::to_string(op.in_f) + " channels");
        break;
      }
      default:
        break;
    }
    pl.out_shape = cur;
    pl.out_len = numel(cur);
  }
  plan->out_shape = cur;
  plan->out_len = numel(cur);

  // Buffers: f32 ping-pong between ops, the last computing op writes the
  // caller's output.
  plan->capture = P->capture;
  for (size_t i = 0; i + 1 < nops; i++) {
    int span = 0, act = 0;
    plan->ops[i].pool_r16 = conv_pool_fusion(P, plan->ops, i, &span, &act);
    if (!plan->ops[i].pool_r16) continue;
    plan->ops[i].pool_act = act;
    for (int k = 1; k <= span; k++) plan->ops[i + k].pool_fused = true;
  }
  int last = -1;
  for (size_t i = 0; i < nops; i++)
    if (P->ops[i]->kind != OP_FLATTEN && !plan->ops[i].pool_fused) last = (int)i;
  int curbuf = BUF_INPUT;
  for (size_t i = 0; i < nops; i++) {
    OpPlan& pl = plan->ops[i];
    pl.in_buf = curbuf;
    if (P->ops[i]->kind == OP_FLATTEN || pl.pool_fused) {
      pl.out_buf = curbuf;
    } else if ((int)i == last) {
      pl.out_buf = BUF_OUTPUT;
    } else {
      pl.out_buf = curbuf == 0 ? 1 : 0;
      plan->f32_elems = std::max(plan->f32_elems, (size_t)pl.out_len);
    }
    curbuf = pl.out_buf;
  }

  // Absmax slots for quantizing consumers, and producer fusion.  A Linear
  // consumer gets a spread per-tensor slot (kTensorSlotWords words, 128-byte
  // aligned), a conv consumer one word per image.
  int64_t slots = 0, n_scales = 0;
  for (size_t i = 0; i < nops; i++) {
    const Op& op = *P->ops[i];
    OpPlan& pl = plan->ops[i];
    if (op.kind != OP_LINEAR && op.kind != OP_CONV) continue;
    if (P->precision != RGNPU_PRECISION_INT8) {
      // No activation quantization: binary16 (FP16) or f32 (FP32) operands,
      // the split-K workspace, and the conv's [n*L, O] GEMM output.
      if (op.diag) continue;
      const int64_t es = P->precision == RGNPU_PRECISION_FP16 ? 2 : 4;
      plan->q_bytes = std::max(plan->q_bytes, (size_t)(pl.Mpad * op.Kpad * es));
      if (!pl.gemv && !(op.kind == OP_LINEAR && op.out_f <= kNarrowMaxN))
        plan->ws_bytes = std::max(plan->ws_bytes, gemm_workspace_bytes(pl.Mpad, op.Npad, es * op.Kpad));
      if (op.kind == OP_CONV) plan->ylo_elems = std::max(plan->ylo_elems, (size_t)(pl.rows * op.out_f));
      continue;
    }
    pl.slot_count = op.kind == OP_LINEAR ? 1 : pl.cs.n;
    if (op.kind == OP_LINEAR) {
      pl.slot_base = round_up(slots, kSpreadStride);
      slots = pl.slot_base + kTensorSlotWords;
    } else {
      pl.slot_base = slots;
      slots += pl.slot_count;
    }
    pl.scale_base = n_scales;
    n_scales += pl.slot_count;
    int j = (int)i - 1;
    while (j >= 0 && P->ops[j]->kind == OP_FLATTEN) j--;
    pl.explicit_absmax = true;
    if (j >= 0) {
      const int pk = P->ops[j]->kind;
      OpPlan& prod = plan->ops[j];
      if (op.kind == OP_LINEAR && (pk == OP_LINEAR || pk == OP_CONV || pk == OP_POOL || pk == OP_ACT)) {
        prod.emit_slot = pl.slot_base;
        prod.emit_per_image = 0;
        pl.explicit_absmax = false;
      } else if (op.kind == OP_CONV && pl.full_cov && (pk == OP_CONV || pk == OP_POOL)) {
        prod.emit_slot = pl.slot_base;
        prod.emit_per_image = 1;
        pl.explicit_absmax = false;
      }
    }
    if (op.kind == OP_LINEAR && !pl.gemv && op.out_f > kNarrowMaxN)
      plan->ws_bytes = std::max(plan->ws_bytes, gemm_workspace_bytes(pl.Mpad, op.Npad, op.Kpad));
    size_t qb = op.kind == OP_LINEAR ? (size_t)(pl.Mpad * op.Kpad) : (size_t)pl.in_len;
    plan->q_bytes = std::max(plan->q_bytes, qb);
  }
  // A program of small INT8 Linears on the same rows runs as one kernel in
  // one workgroup (launch_mlp_tiny, the same arithmetic op by op): the first
  // op launches it and the others launch nothing.  Not in capture plans,
  // which store every op's operand and output; RGNPU_TINY_MLP=0 turns it off.
  {
    const char* te = getenv("RGNPU_TINY_MLP");
    bool tiny = P->precision == RGNPU_PRECISION_INT8 && !plan->capture && !(te && atoi(te) == 0) && nops >= 1 &&
                nops <= (size_t)kTinyMaxLayers;
    int64_t wbytes = 0;
    for (size_t i = 0; tiny && i < nops; i++) {
      const Op& op = *P->ops[i];
      const OpPlan& pl = plan->ops[i];
      tiny = op.kind == OP_LINEAR && pl.rows >= 1 && pl.rows <= kTinyRows && pl.rows == plan->ops[0].rows &&
             op.in_f <= kTinyWidth && op.out_f <= kTinyWidth && op.Kpad == kTinyWidth;
      wbytes += op.out_f * op.Kpad;
    }
    plan->tiny = tiny && wbytes <= kTinyWeightBytes;
  }
  // Two INT8 conv + pool stages, the first on the run's input (it measures
  // its images' absmax itself), run as one kernel per image when their shapes
  // fit it; not in capture plans, which store every op's operand and output.
  // RGNPU_CONV_PAIR=0 turns it off.
  {
    const char* ce = getenv("RGNPU_CONV_PAIR");
    const bool on = P->precision == RGNPU_PRECISION_INT8 && !plan->capture && !(ce && atoi(ce) == 0);
    for (size_t i = 0; on && i + 3 < nops; i++) {
      OpPlan &a = plan->ops[i], &b = plan->ops[i + 2];
      if (P->ops[i]->kind != OP_CONV || P->ops[i + 2]->kind != OP_CONV || a.pool_r16 != 2 || b.pool_r16 != 1 ||
          !plan->ops[i + 1].pool_fused || !plan->ops[i + 3].pool_fused || P->ops[i + 1]->kind != OP_POOL ||
          P->ops[i + 3]->kind != OP_POOL)
        continue;
      if (!a.explicit_absmax || !a.full_cov || !conv_self_absmax_supported(a.cs) || b.explicit_absmax ||
          !conv_pool_pair_supported(a.cs, b.cs))
        continue;
      a.pair = 1;
      b.pair = 2;
      plan->ops[i + 1].no_out = true;
      break;
    }
  }
  // Requantization fused into the producing GEMM: an INT8 Linear on the
  // unsplit MFMA GEMM whose next computing op is a Linear reading the same
  // rows (its absmax is this op's emitted slot).  Its barrier words join the
  // slot set, which every run zeroes.
  //
  // Persistent grids (this fusion and the one-pass input quantization below)
  // take every resident workgroup slot and meet at a grid barrier, so they
  // need the whole GPU to themselves.  Host-pointer runs of several threads
  // run on worker streams at once, and there the other streams' kernels
  // (GEMMs, copies) keep taking the slots such a grid waits for: its
  // workgroups then wait out the barrier's bound (~32 ms) and defer.  Once
  // two host runs of a program have overlapped, its worker runs therefore use
  // plans with the separate quantize kernels (the same arithmetic); those
  // runs are bound by their host copies anyway.
  const bool persistent_ok = P->use_persistent && !plan->tiny;
  plan->persistent = P->use_persistent;
  bool any_requant = false;
  for (size_t i = 0; i < nops && P->precision == RGNPU_PRECISION_INT8 && persistent_ok; i++) {
    const Op& op = *P->ops[i];
    OpPlan& pl = plan->ops[i];
    if (op.kind != OP_LINEAR || pl.gemv || op.out_f <= kNarrowMaxN || pl.rows <= 0 || op.out_f % 4) continue;
    if (!gemm_requant_supported(pl.Mpad, op.Npad, op.Kpad)) continue;
    size_t j = i + 1;
    while (j < nops && P->ops[j]->kind == OP_FLATTEN) j++;
    if (j >= nops || P->ops[j]->kind != OP_LINEAR) continue;
    const Op& cop = *P->ops[j];
    OpPlan& cpl = plan->ops[j];
    if (cop.in_f != op.out_f || cpl.rows != pl.rows || cpl.gemv || cpl.explicit_absmax ||
        pl.emit_slot != cpl.slot_base || cop.Kpad > op.Npad)
      continue;
    pl.requant = true;
    pl.consumer = (int)j;
    pl.sync_base = round_up(slots, kSpreadStride);
    slots = pl.sync_base + requant_sync_words(pl.Mpad, op.Npad, op.Kpad);
    cpl.q_ready = true;
    cpl.q_in = pl.q_in ^ 1;
    any_requant = true;
  }
  // FP16: a Linear on the unsplit MFMA GEMM whose next computing op is an
  // FP16 Linear on the same rows hands it its binary16 operand from the GEMM
  // epilogue, so the consumer runs no conversion pass (RGNPU_F16_HANDOFF=0
  // turns this off).
  const char* hoff = getenv("RGNPU_F16_HANDOFF");
  const bool handoff_on = !(hoff && atoi(hoff) == 0);
  for (size_t i = 0; i < nops && P->precision == RGNPU_PRECISION_FP16 && handoff_on; i++) {
    const Op& op = *P->ops[i];
    OpPlan& pl = plan->ops[i];
    if (op.kind != OP_LINEAR || op.diag || pl.gemv || op.out_f <= kNarrowMaxN || pl.rows <= 0 || op.out_f % 4) continue;
    if (choose_gemm(pl.Mpad, op.Npad, 2 * op.Kpad).splits != 1) continue;
    size_t j = i + 1;
    while (j < nops && P->ops[j]->kind == OP_FLATTEN) j++;
    if (j >= nops || P->ops[j]->kind != OP_LINEAR) continue;
    const Op& cop = *P->ops[j];
    OpPlan& cpl = plan->ops[j];
    if (cop.diag || cop.in_f != op.out_f || cpl.rows != pl.rows || cpl.gemv || cpl.Mpad != pl.Mpad ||
        cop.Kpad > op.Npad)
      continue;
    pl.handoff = true;
    pl.consumer = (int)j;
    cpl.q_ready = true;
    cpl.q_in = pl.q_in ^ 1;
    any_requant = true;  // the second operand buffer
  }
  // A Linear that quantizes its own input does so in one pass when the
  // shapes fit the kernel's 32-bit offsets (RGNPU_INPUT_QUANT=0, for
  // measurement: the absmax and quantize kernels instead).
  const char* iqe = getenv("RGNPU_INPUT_QUANT");
  const bool one_pass = !(iqe && atoi(iqe) == 0);
  for (size_t i = 0; i < nops && P->precision == RGNPU_PRECISION_INT8 && persistent_ok && one_pass; i++) {
    const Op& op = *P->ops[i];
    OpPlan& pl = plan->ops[i];
    if (op.kind != OP_LINEAR || !pl.explicit_absmax || pl.rows <= 0 ||
        !input_quant_supported(pl.rows, op.in_f, pl.Mpad, op.Kpad))
      continue;
    pl.iq_sync_base = round_up(slots, kSpreadStride);
    slots = pl.iq_sync_base + input_quant_sync_words(pl.Mpad, op.Kpad);
  }
  // An INT8 Linear with fewer than 128 output tiles of 128 x 128 (the tile
  // GEMM would split K or leave most CUs idle) whose input's absmax a
  // producer emitted quantizes that input as it reads it, one workgroup per
  // small output block and K slice: no quantize pass and no kernel adding
  // the slices (they meet in one 64-bit word per output in the slot set).
  // Not in capture plans, which store the i8 operand.  RGNPU_SMALL_XQ=0
  // turns it off.
  {
    const char* xe = getenv("RGNPU_SMALL_XQ");
    const bool on = P->precision == RGNPU_PRECISION_INT8 && !plan->capture && !plan->tiny && !(xe && atoi(xe) == 0);
    for (size_t i = 0; on && i < nops; i++) {
      const Op& op = *P->ops[i];
      OpPlan& pl = plan->ops[i];
      pl.small_xq = op.kind == OP_LINEAR && !pl.gemv && op.out_f > kNarrowMaxN && pl.rows > 0 &&
                    !pl.explicit_absmax && !pl.q_ready && !pl.requant &&
                    (pl.Mpad / 128) * (op.Npad / 128) < 128 &&
                    gemm_xq_small_supported(pl.rows, op.out_f, op.Npad, op.in_f, op.Kpad);
      if (!pl.small_xq) continue;
      const int64_t words = gemm_xq_small_sync_words(pl.rows, op.Npad, op.Kpad);
      if (words > 0) {
        pl.xq_sync_base = round_up(slots, kSpreadStride);
        slots = pl.xq_sync_base + words;
      }
    }
  }
  if (const char* e = getenv("RGNPU_REQUANT_SPIN_LIMIT")) plan->spin_limit = std::max(0, atoi(e));
  else plan->spin_limit = 100000;  // x kBarrierPollUs (0.32 us) = ~32 ms
  if (const char* e = getenv("RGNPU_GELU_CERT")) plan->gelu_cert = std::min(3, std::max(0, atoi(e)));
  plan->n_slots = slots;
  // The first computing op quantizes the input itself (its absmax is the
  // run's first kernel) unless the input is empty.
  for (size_t i = 0; i < nops; i++) {
    const Op& op = *P->ops[i];
    if (op.kind == OP_FLATTEN) continue;
    const OpPlan& pl = plan->ops[i];
    plan->clear_by_first =
        slots > 0 && (op.kind == OP_LINEAR || op.kind == OP_CONV) && pl.explicit_absmax && pl.in_len > 0;
    break;
  }
  if (scratch) {
    // One call's buffers, 256-byte aligned, one after the other.  A new
    // call finds whatever the previous one (of any program on this device)
    // left, so the slots are zeroed by every run rather than by the first
    // kernel of the run before.
    plan->clear_by_first = false;
    plan->slot_set_words = round_up(std::max<int64_t>(slots, 1), kSpreadStride);
    DevBuf* const bufs[] = {&plan->f32[0], &plan->f32[1], &plan->q,     &plan->q_alt, &plan->ylo,
                            &plan->ws,     &plan->slots,  &plan->scales, &plan->masks};
    const size_t sizes[] = {plan->f32_elems * sizeof(float),
                            plan->f32_elems * sizeof(float),
                            plan->q_bytes,
                            any_requant ? plan->q_bytes : 0,
                            plan->ylo_elems * sizeof(float),
                            (size_t)plan->ws_bytes,
                            (size_t)plan->slot_set_words * sizeof(uint32_t),
                            (size_t)std::max<int64_t>(n_scales, 1) * sizeof(float),
                            mask_host.size()};
    size_t need = 0;
    for (size_t b : sizes) need += round_up((int64_t)std::max<size_t>(b, 1), 256);
    if (need > (size_t)kScratchBytes)
      throw Error(RGNPU_ERR_CAPACITY, "this input shape needs " + std::to_string(need) +
                                          " bytes of intermediate buffers; the allocation-free entry point's "
                                          "device scratch holds " + std::to_string(kScratchBytes) +
                                          " (use rgnpu_program_run_device)");
    size_t off = 0;
    for (size_t k = 0; k < sizeof sizes / sizeof sizes[0]; k++) {
      const size_t b = std::max<size_t>(sizes[k], 1);
      bufs[k]->borrow(static_cast<char*>(scratch) + off, b);
      off += round_up((int64_t)b, 256);
    }
    plan->in_scratch = true;
    plan->mask_host = std::move(mask_host);
    return plan;
  }

  plan->f32[0].ensure(plan->f32_elems * sizeof(float));
  plan->f32[1].ensure(plan->f32_elems * sizeof(float));
  plan->q.ensure(plan->q_bytes);
  if (any_requant) plan->q_alt.ensure(plan->q_bytes);
  if (plan->ylo_elems > 0) plan->ylo.ensure(plan->ylo_elems * sizeof(float));
  if (plan->ws_bytes > 0) plan->ws.ensure((size_t)plan->ws_bytes);
  plan->slot_set_words = round_up(std::max<int64_t>(slots, 1), kSpreadStride);
  const size_t slot_bytes = (size_t)plan->slot_set_words * sizeof(uint32_t) * (plan->clear_by_first ? 2 : 1);
  plan->slots.ensure(slot_bytes);
  RG_HIP(hipMemsetAsync(plan->slots.p, 0, slot_bytes, P->stream));
  plan->scales.ensure((size_t)std::max<int64_t>(n_scales, 1) * sizeof(float));
  plan->masks.ensure(std::max<size_t>(mask_host.size(), 1));
  if (!mask_host.empty())
    RG_HIP(hipMemcpyAsync(plan->masks.p, mask_host.data(), mask_host.size(), hipMemcpyHostToDevice, P->stream));
  RG_HIP(hipStreamSynchronize(P->stream));
  return plan;
}

static void ensure_capture_buffers(rgnpu_program* P, Plan& plan) {
  if (plan.capture_ready) return;
  const size_t n = P->ops.size();
  plan.cap_q.resize(n);
  plan.cap_acc.resize(n);
  plan.cap_out.resize(n);
  for (size_t i = 0; i < n; i++) {
    const Op& op = *P->ops[i];
    const OpPlan& pl = plan.ops[i];
    plan.cap_out[i] = std::make_unique<DevBuf>();
    plan.cap_out[i]->ensure((size_t)pl.out_len * sizeof(float));
    if ((op.kind == OP_LINEAR || op.kind == OP_CONV) && P->precision == RGNPU_PRECISION_INT8) {
      plan.cap_q[i] = std::make_unique<DevBuf>();
      plan.cap_acc[i] = std::make_unique<DevBuf>();
      plan.cap_q[i]->ensure(op.kind == OP_LINEAR ? (size_t)(pl.Mpad * op.Kpad) : (size_t)pl.in_len);
      const size_t accn = op.kind == OP_LINEAR ? (size_t)(pl.rows * op.out_f)
                                               : (size_t)(pl.cs.n * pl.cs.OH * pl.cs.OW * op.out_f);
      plan.cap_acc[i]->ensure(accn * sizeof(int32_t));
    }
  }
  plan.capture_ready = true;
}

// Buffers of the production taps: the INT8 Linear operands, the absmax slot
// words of every quantizing op, and every f32 output.
static void ensure_tap_buffers(rgnpu_program* P, Plan& plan) {
  if (plan.taps_ready) return;
  const size_t n = P->ops.size();
  plan.cap_q.resize(n);
  plan.cap_out.resize(n);
  plan.tap_slot.resize(n);
  plan.tap_q_ok.assign(n, 0);
  plan.tap_out_ok.assign(n, 0);
  plan.tap_scale_ok.assign(n, 1);
  for (size_t i = 0; i < n; i++) {
    const Op& op = *P->ops[i];
    const OpPlan& pl = plan.ops[i];
    plan.cap_out[i] = std::make_unique<DevBuf>();
    plan.cap_out[i]->ensure((size_t)pl.out_len * sizeof(float));
    if (pl.slot_base < 0) continue;
    plan.tap_slot[i] = std::make_unique<DevBuf>();
    plan.tap_slot[i]->ensure((size_t)(op.kind == OP_LINEAR ? kTensorSlotWords : pl.slot_count) * sizeof(uint32_t));
    if (op.kind == OP_LINEAR) {
      plan.cap_q[i] = std::make_unique<DevBuf>();
      plan.cap_q[i]->ensure((size_t)(pl.Mpad * op.Kpad));
    }
  }
  plan.taps_ready = true;
}

static void finalize_profile(rgnpu_program* P);

// The barrier counters of a context: device words zeroed once, a pinned copy.
static void init_stats(rgnpu_program* P) {
  P->stats.ensure(kStatWords * sizeof(uint32_t));
  launch_fill_u32(P->stats.as<uint32_t>(), kStatWords, 0u, P->stream);
  RG_HIP(hipGetLastError());
  RG_HIP(hipHostMalloc(reinterpret_cast<void**>(&P->stats_host), kStatWords * sizeof(uint32_t)));
  for (int k = 0; k < kStatWords; k++) P->stats_host[k] = 0;
}

// After P's stream has drained past a copy of the counters into
// stats_host: a finisher that met an unsettled workgroup left that
// workgroup's share of the next operand unquantized, so the run is reported
// as failed (once per occurrence).
static void check_stats(rgnpu_program* P) {
  const uint32_t u = P->stats_host[kStatUnsettled];
  if (u != P->unsettled_seen) {
    P->unsettled_seen = u;
    throw Error(RGNPU_ERR_DEVICE, "a grid barrier workgroup never settled: the run's output is incomplete");
  }
}

// Synchronous variant for the synchronizing entry points.
static void read_stats(rgnpu_program* P) {
  RG_HIP(hipMemcpyAsync(P->stats_host, P->stats.p, kStatWords * sizeof(uint32_t), hipMemcpyDeviceToHost, P->stream));
  RG_HIP(hipStreamSynchronize(P->stream));
}

static bool plan_fits(const Plan* pl, const rgnpu_program* P, const int64_t* shape, int ndim) {
  return pl && (int)pl->in_shape.size() == ndim && pl->capture == P->capture &&
         pl->persistent == P->use_persistent && std::equal(pl->in_shape.begin(), pl->in_shape.end(), shape);
}

static Plan& get_plan(rgnpu_program* P, const int64_t* shape, int ndim) {
  if (plan_fits(P->plan.get(), P, shape, ndim)) return *P->plan;
  // A pending profile reads the roles and events of the plan it ran with:
  // settle it before that plan stops being the current one.
  if (P->plan && P->profile_pending) finalize_profile(P);
  if (plan_fits(P->plan_other.get(), P, shape, ndim)) {
    std::swap(P->plan, P->plan_other);
    return *P->plan;
  }
  // keep the current plan as the other kind when only the kind changes
  const bool same_shape = P->plan && (int)P->plan->in_shape.size() == ndim && P->plan->capture == P->capture &&
                          std::equal(P->plan->in_shape.begin(), P->plan->in_shape.end(), shape);
  P->plan_other = same_shape ? std::move(P->plan) : nullptr;
  P->plan.reset();
  P->plan = make_plan(P, shape, ndim);
  return *P->plan;
}

// Events of one run: [0], [1] bracket the run (markers, default flags; the
// host waits on [1]); [2 ..] are launch events: the stop event of each kernel
// the run launches, recorded by that kernel's own dispatch.  Launch events
// skip the system-scope fence, which is not needed for timing.  A run
// launches one fill at most plus at most kMaxLaunchesPerOp kernels per op
// (an FP16 im2col conv with split K launches four: im2col, GEMM, split-K
// epilogue, NCHW transpose); enqueue() checks the bound.
static constexpr size_t kMaxLaunchesPerOp = 6;
static size_t launch_event_cap(const rgnpu_program* P) { return 1 + kMaxLaunchesPerOp * P->ops.size(); }
static size_t events_per_run(const rgnpu_program* P) { return 2 + launch_event_cap(P); }

static void create_run_event(hipEvent_t* e, size_t index_in_set) {
  if (index_in_set < 2)
    RG_HIP(hipEventCreate(e));
  else
    RG_HIP(hipEventCreateWithFlags(e, hipEventDisableSystemFence));
}

static void ensure_events(rgnpu_program* P) {
  const size_t need = events_per_run(P);
  while (P->ev.size() < need) {
    hipEvent_t e;
    create_run_event(&e, P->ev.size());
    P->ev.push_back(e);
  }
}

// Per-op (op ns, kernel ns) of one run from its event set.
static void op_times(const rgnpu_program* P, const Plan& plan, const hipEvent_t* set, size_t i, double* op_ms,
                     double* kernel_ms) {
  auto at = [&](int idx) { return idx < 0 ? set[0] : set[2 + idx]; };
  const auto& r = plan.roles[i];
  float a = 0, b = 0;
  if (r[2] != r[0]) RG_HIP(hipEventElapsedTime(&a, at(r[0]), at(r[2])));
  if (r[2] != r[1]) RG_HIP(hipEventElapsedTime(&b, at(r[1]), at(r[2])));
  *op_ms = a;
  *kernel_ms = b;
  (void)P;
}

// Enqueue one run; x and y are device pointers.  `ev` is one run's event set
// (events_per_run): [0] and [1] are recorded when it is given; with `timed`
// every kernel also records its launch event and plan.roles says which ones
// bound each op.  A null `ev` records nothing (back-to-back throughput runs).
static void enqueue(rgnpu_program* P, Plan& plan, const float* x, float* y, hipEvent_t* ev, bool timed) {
  hipStream_t s = P->stream;
  const bool f16 = P->precision == RGNPU_PRECISION_FP16;
  const bool f32 = P->precision == RGNPU_PRECISION_FP32;
  const bool cap = P->capture;
  // production taps: copies between the unchanged launches (not in the
  // allocation-free plan, whose buffers other calls share)
  const bool tap = P->taps && !cap && !plan.in_scratch;
  struct SinkOff {
    ~SinkOff() { set_launch_events(nullptr, 0); }
  } sink_off;
  timed = timed && ev;
  set_launch_events(timed ? ev + 2 : nullptr, timed ? (int)launch_event_cap(P) : 0);
  if (cap) ensure_capture_buffers(P, plan);
  if (tap) ensure_tap_buffers(P, plan);
  plan.roles.assign(P->ops.size(), std::array<int, 3>{-1, -1, -1});
  if (ev) RG_HIP(hipEventRecord(ev[0], s));
  if (plan.in_scratch && !plan.mask_host.empty())
    RG_HIP(hipMemcpyAsync(plan.masks.p, plan.mask_host.data(), plan.mask_host.size(), hipMemcpyHostToDevice, s));
  uint32_t* const slot_sets = plan.slots.as<uint32_t>();
  uint32_t* slots = slot_sets;
  SlotClear clear{};  // handed to the run's first kernel, then reset
  if (plan.clear_by_first) {
    slots = slot_sets + plan.parity * plan.slot_set_words;
    clear = SlotClear{slot_sets + (1 - plan.parity) * plan.slot_set_words, plan.n_slots};
  } else if (plan.n_slots > 0) {
    launch_fill_u32(slots, plan.n_slots, 0u, s);
  }
  // The other set is zero once the first kernel is enqueued: from then on
  // the next run uses it, whatever happens later in this one.
  auto first_launched = [&]() {
    if (clear.p) {
      clear = SlotClear{};
      plan.parity ^= 1;
    }
  };
  float* scales = plan.scales.as<float>();
  int8_t* q = plan.q.as<int8_t>();
  auto buf = [&](int id) -> float* {
    if (id == BUF_INPUT) return const_cast<float*>(x);
    if (id == BUF_OUTPUT) return y;
    return plan.f32[id].as<float>();
  };
  for (size_t i = 0; i < P->ops.size(); i++) {
    const Op& op = *P->ops[i];
    const OpPlan& pl = plan.ops[i];
    const int first = launch_events_used();
    int pre = first;  // launches before the op's main kernel
    const float* in = buf(pl.in_buf);
    float* out = buf(pl.out_buf);
    uint32_t* emit = pl.emit_slot >= 0 ? slots + pl.emit_slot : nullptr;
    switch (op.kind) {
      case OP_LINEAR: {
        if (plan.tiny) {
          pre = launch_events_used();
          if (i == 0) {
            TinyChain ch;
            ch.n = (int32_t)P->ops.size();
            ch.rows = (int32_t)pl.rows;
            for (size_t l = 0; l < P->ops.size(); l++) {
              const Op& o = *P->ops[l];
              TinyLayer& t = ch.l[l];
              t.w = o.d_w.as<int8_t>();
              t.bias = o.d_bias.as<float>();
              t.slot = slots + plan.ops[l].slot_base;
              t.in_f = (int32_t)o.in_f;
              t.out_f = (int32_t)o.out_f;
              t.kpad = (int32_t)o.Kpad;
              t.act = o.act;
              t.act_param = o.act_param;
              t.w_scale = o.w_scale;
            }
            launch_mlp_tiny(in, y, ch, clear, s);
            first_launched();
          }
          break;
        }
        if (f32) {  // mod.rs:263-273: matmul, then the bias
          pre = launch_events_used();
          if (pl.rows > 0) {
            // the GEMM reads [Mpad, Kpad] rows: an input of exactly that shape
            // on a 16-byte boundary is read in place
            const float* a = in;
            if (pl.rows != pl.Mpad || op.K != op.Kpad || (reinterpret_cast<uintptr_t>(in) & 15) != 0) {
              float* pa = plan.q.as<float>();
              launch_pad_rows_f32(in, pl.rows, op.K, pl.Mpad, op.Kpad, pa, s);
              a = pa;
            }
            Epilogue ep;
            ep.bias = op.d_bias.as<float>();
            ep.y = out;
            ep.y_stream = pl.out_buf == BUF_OUTPUT;
            pre = launch_events_used();
            if (pl.gemv)
              launch_gemv_f32(a, op.d_w.as<float>(), pl.rows, op.out_f, op.Npad, op.Kpad, ep, s);
            else if (op.out_f <= kNarrowMaxN)
              launch_gemm_narrow_f32(a, op.d_w.as<float>(), pl.rows, op.out_f, op.Kpad, ep, s);
            else
              launch_gemm_f32(a, op.d_w.as<float>(), pl.rows, op.out_f, pl.Mpad, op.Npad, op.Kpad, ep,
                              plan.ws.as<int32_t>(), plan.ws_bytes, s);
          }
          break;
        }
        if (f16) {  // npu.rs:315
          pre = launch_events_used();
          if (op.diag) {
            launch_affine_f16(in, pl.in_len, op.in_f, op.d_scale.as<float>(), op.d_bias.as<float>(), out, s);
          } else if (pl.rows > 0) {
            // Capture runs store every f32 output and convert every input
            // (no hand-off); each op still reads its own operand buffer.
            uint16_t* h = pl.q_in ? plan.q_alt.as<uint16_t>() : plan.q.as<uint16_t>();
            if (!pl.q_ready || cap) launch_half_rows(in, pl.rows, op.K, pl.Mpad, op.Kpad, h, s);
            Epilogue ep;
            ep.bias = op.d_bias.as<float>();
            ep.act = op.act;
            ep.act_param = op.act_param;
            ep.y = out;
            ep.y_stream = pl.out_buf == BUF_OUTPUT;
            if (pl.handoff && !cap) {
              const OpPlan& cpl = plan.ops[(size_t)pl.consumer];
              ep.h_out = cpl.q_in ? plan.q_alt.as<uint16_t>() : plan.q.as<uint16_t>();
              ep.ldh = P->ops[(size_t)pl.consumer]->Kpad;
              ep.gelu_cert = plan.gelu_cert;
              ep.y = nullptr;  // nothing reads the f32 output
            }
            pre = launch_events_used();
            if (pl.gemv)
              launch_gemv_f16(h, op.d_w.as<uint16_t>(), pl.rows, op.out_f, op.Npad, op.Kpad, ep, s);
            else if (op.out_f <= kNarrowMaxN)
              launch_gemm_narrow_f16(h, op.d_w.as<uint16_t>(), pl.rows, op.out_f, op.Kpad, ep, s);
            else
              launch_gemm_f16(h, op.d_w.as<uint16_t>(), pl.rows, op.out_f, pl.Mpad, op.Npad, op.Kpad, ep,
                              plan.ws.as<int32_t>(), plan.ws_bytes, s);
          }
          break;
        }
        uint32_t* slot = slots + pl.slot_base;
        int8_t* const qa = pl.q_in ? plan.q_alt.as<int8_t>() : q;
        // A narrow GEMM after a producer that emitted the absmax quantizes
        // its input as it reads it (an unaligned input takes quant_rows).
        const bool narrow_xq = !pl.gemv && op.out_f <= kNarrowMaxN && !pl.explicit_absmax && !pl.q_ready &&
                               pl.rows > 0 && gemm_narrow_xq_supported(op.in_f, op.Kpad) &&
                               (reinterpret_cast<uintptr_t>(in) & 15) == 0;
        // A one-row GEMV quantizes its input itself, with the producer's
        // absmax or, when its input has none yet, the input's own.
        const bool gemv_xq = pl.gemv && !pl.q_ready && gemv_xq_supported(pl.rows, op.in_f, op.Kpad, in);
        const bool small_xq = pl.small_xq && !cap && (reinterpret_cast<uintptr_t>(in) & 15) == 0;
        // a one-row GEMV that measures its input's absmax itself keeps it in
        // registers: no slot holds it
        if (tap) plan.tap_scale_ok[i] = !(gemv_xq && pl.explicit_absmax);
        if (narrow_xq || gemv_xq || small_xq) {
          // nothing before the GEMM
        } else if (pl.iq_sync_base >= 0) {
          launch_input_quant(in, pl.rows, op.K, pl.Mpad, op.Kpad, slot, qa, scales + pl.scale_base,
                             slots + pl.iq_sync_base, plan.spin_limit, P->stats.as<uint32_t>(), clear, s);
          first_launched();
        } else if (!pl.q_ready) {
          if (pl.explicit_absmax) {
            launch_absmax(in, pl.in_len, 1, slot, true, nullptr, nullptr, 0, 0, s, clear);
            first_launched();
          }
          launch_quant_rows(in, pl.rows, op.K, pl.Mpad, op.Kpad, slot, qa, scales + pl.scale_base, s);
        }
        Epilogue ep;
        ep.bias = op.d_bias.as<float>();
        ep.act = op.act;
        ep.act_param = op.act_param;
        ep.absmax_in = slot;
        ep.w_scale = op.w_scale;
        ep.y = out;
        ep.y_stream = pl.out_buf == BUF_OUTPUT;
        ep.absmax_out = emit;
        ep.absmax_out_per_image = 0;
        ep.acc_out = cap ? plan.cap_acc[i]->as<int32_t>() : nullptr;
        pre = launch_events_used();
        if (pl.rows > 0) {
          if (pl.requant) {
            const OpPlan& cpl = plan.ops[(size_t)pl.consumer];
            Requant rq;
            rq.q = cpl.q_in ? plan.q_alt.as<int8_t>() : q;
            rq.ldq = P->ops[(size_t)pl.consumer]->Kpad;
            rq.sync = slots + pl.sync_base;
            rq.scale_out = scales + cpl.scale_base;
            rq.keep_f32 = cap ? 1 : 0;
            rq.spin_limit = plan.spin_limit;
            rq.gelu_cert = plan.gelu_cert;
            rq.stats = P->stats.as<uint32_t>();
            launch_gemm_requant(qa, op.d_w.as<int8_t>(), pl.rows, op.out_f, pl.Mpad, op.Npad, op.Kpad, ep, rq, s);
          } else if (gemv_xq) {
            launch_gemv_xq(in, op.d_w.as<int8_t>(), op.out_f, op.Npad, op.in_f, op.Kpad, ep, pl.explicit_absmax,
                           cap ? qa : nullptr, cap ? scales + pl.scale_base : nullptr,
                           pl.explicit_absmax ? clear : SlotClear{}, s);
            if (pl.explicit_absmax) first_launched();
          } else if (pl.gemv) {
            launch_gemv(qa, op.d_w.as<int8_t>(), pl.rows, op.out_f, op.Npad, op.Kpad, ep, s);
          } else if (small_xq) {
            launch_gemm_xq_small(in, op.d_w.as<int8_t>(), pl.rows, op.out_f, op.Npad, op.in_f, op.Kpad, ep,
                                 pl.xq_sync_base >= 0 ? slots + pl.xq_sync_base : nullptr, s);
          } else if (narrow_xq) {
            launch_gemm_narrow_xq(in, op.d_w.as<int8_t>(), pl.rows, op.out_f, op.in_f, op.Kpad, ep, cap ? qa : nullptr,
                                  cap ? scales + pl.scale_base : nullptr, s);
          } else if (op.out_f <= kNarrowMaxN) {
            launch_gemm_narrow(qa, op.d_w.as<int8_t>(), pl.rows, op.out_f, op.Kpad, ep, s);
          } else {
            launch_gemm(qa, op.d_w.as<int8_t>(), pl.rows, op.out_f, pl.Mpad, op.Npad, op.Kpad, ep,
                        plan.ws.as<int32_t>(), plan.ws_bytes, s);
          }
        }
        if (cap) RG_HIP(hipMemcpyAsync(plan.cap_q[i]->p, qa, (size_t)(pl.Mpad * op.Kpad), hipMemcpyDeviceToDevice, s));
        // the one-row GEMV and the narrow and small GEMMs that quantize as
        // they read leave no i8 operand in memory
        if (tap && pl.rows > 0 && !narrow_xq && !gemv_xq && !small_xq) {
          RG_HIP(hipMemcpyAsync(plan.cap_q[i]->p, qa, (size_t)(pl.Mpad * op.Kpad), hipMemcpyDeviceToDevice, s));
          plan.tap_q_ok[i] = 1;
        }
        break;
      }
      case OP_CONV: {
        const ConvShape& c = pl.cs;
        if (f32) {  // mod.rs:274-290: conv2d_forward (im2col + matmul), then the bias
          pre = launch_events_used();
          if (pl.rows > 0 && op.K <= kDirectConvTaps && op.out_f <= 64) {
            launch_conv_direct_f32(in, op.d_w.as<float>(), op.d_bias.as<float>(), out, c, pl.pool_act,
                                   pl.pool_r16 ? (int)c.OW : 0, s);
          } else if (pl.rows > 0) {
            float* a = plan.q.as<float>();
            launch_im2col_f32(in, c, pl.Mpad, op.Kpad, a, s);
            Epilogue ep;
            ep.bias = op.d_bias.as<float>();
            ep.y = plan.ylo.as<float>();
            pre = launch_events_used();
            launch_gemm_f32(a, op.d_w.as<float>(), pl.rows, op.out_f, pl.Mpad, op.Npad, op.Kpad, ep,
                            plan.ws.as<int32_t>(), plan.ws_bytes, s);
            launch_nlo_to_nchw(plan.ylo.as<float>(), c.n, op.out_f, c.OH * c.OW, out, s);
          }
          break;
        }
        if (f16) {  // npu.rs:341-376: im2col, GEMM, transpose per image
          pre = launch_events_used();
          if (pl.rows > 0 && op.K <= kDirectConvTaps && op.out_f <= 64) {
            launch_conv_direct_f16(in, op.d_w.as<uint16_t>(), op.d_bias.as<float>(), out, c, op.act, op.act_param,
                                   pl.pool_r16 ? (int)c.OW : 0, s);
          } else if (pl.rows > 0) {
            uint16_t* h = plan.q.as<uint16_t>();
            launch_im2col_half(in, c, pl.Mpad, op.Kpad, h, s);
            Epilogue ep;
            ep.bias = op.d_bias.as<float>();
            ep.act = op.act;
            ep.act_param = op.act_param;
            ep.y = plan.ylo.as<float>();
            pre = launch_events_used();
            launch_gemm_f16(h, op.d_w.as<uint16_t>(), pl.rows, op.out_f, pl.Mpad, op.Npad, op.Kpad, ep,
                            plan.ws.as<int32_t>(), plan.ws_bytes, s);
            launch_nlo_to_nchw(plan.ylo.as<float>(), c.n, op.out_f, c.OH * c.OW, out, s);
          }
          break;
        }
        if (pl.pair == 2) {  // run by the first conv of the pair
          pre = launch_events_used();
          break;
        }
        uint32_t* sl = slots + pl.slot_base;
        const int64_t per = c.C * c.H * c.W;
        if (pl.pair == 1) {
          const Op& ob = *P->ops[i + 2];
          const OpPlan &pb = plan.ops[i + 2], &pool_b = plan.ops[i + 3];
          Epilogue ea, eb;
          ea.bias = op.d_bias.as<float>();
          ea.act = op.act;
          ea.act_param = op.act_param;
          ea.absmax_in = sl;
          ea.w_scale = op.w_scale;
          ea.pool2 = pl.pool_r16;
          eb.bias = ob.d_bias.as<float>();
          eb.act = ob.act;
          eb.act_param = ob.act_param;
          eb.absmax_in = slots + pb.slot_base;
          eb.w_scale = ob.w_scale;
          eb.y = buf(pb.out_buf);
          eb.y_stream = pb.out_buf == BUF_OUTPUT;
          eb.pool2 = pb.pool_r16;
          eb.absmax_out = pool_b.emit_slot >= 0 ? slots + pool_b.emit_slot : nullptr;
          eb.absmax_out_per_image = pool_b.emit_per_image;
          pre = launch_events_used();
          launch_conv_pool_pair(in, op.d_w.as<int8_t>(), ob.d_w.as<int8_t>(), c, pb.cs, ea, eb, clear, s);
          first_launched();
          break;
        }
        // a small, fully covered first image: the conv measures its absmax itself
        const bool self_absmax = pl.explicit_absmax && pl.full_cov && conv_self_absmax_supported(c);
        if (pl.explicit_absmax && !self_absmax) {
          const uint8_t* mk = plan.masks.as<uint8_t>() + pl.mask_off;
          if (pl.full_cov)
            launch_absmax(in, per, c.n, sl, false, nullptr, nullptr, 0, 0, s, clear);
          else
            launch_absmax(in, per, c.n, sl, false, mk, mk + c.H, c.H, c.W, s, clear);
          first_launched();
        }
        Epilogue ep;
        ep.bias = op.d_bias.as<float>();
        ep.act = op.act;
        ep.act_param = op.act_param;
        ep.absmax_in = sl;
        ep.w_scale = op.w_scale;
        ep.y = out;
        ep.y_stream = pl.out_buf == BUF_OUTPUT;
        ep.absmax_out = emit;
        ep.absmax_out_per_image = pl.emit_per_image;
        ep.acc_out = cap ? plan.cap_acc[i]->as<int32_t>() : nullptr;
        // Conv -> MaxPool2d(2, 2): the conv's epilogue pools, stores only the
        // pool's output (in this op's out buffer) and raises its absmax for
        // the next op; the pool op then launches nothing.
        if (pl.pool_r16) {
          const OpPlan& ppl = plan.ops[i + 1];
          ep.pool2 = pl.pool_r16;
          ep.absmax_out = ppl.emit_slot >= 0 ? slots + ppl.emit_slot : nullptr;
          ep.absmax_out_per_image = ppl.emit_per_image;
        }
        // The conv quantizes the f32 image into its LDS band itself; the
        // separate i8 image is made only for the capture tap (after the conv
        // when the conv measures the absmax), or when the band does not fit
        // in LDS.
        if (cap && !self_absmax) launch_quant_images(in, per, c.n, sl, q, scales + pl.scale_base, s);
        pre = launch_events_used();
        bool fused = false;
        if (c.n > 0 && c.OH * c.OW > 0) {
          fused = launch_conv_f32in(in, op.d_w.as<int8_t>(), c, ep, s, self_absmax, clear);
          if (ep.pool2 && !fused) throw std::logic_error("conv with pool: no tile width fits (plan said one does)");
          if (self_absmax && fused) first_launched();
          if (!fused) {
            if (self_absmax) {  // the band does not fit: the absmax pass after all
              launch_absmax(in, per, c.n, sl, false, nullptr, nullptr, 0, 0, s, clear);
              first_launched();
            }
            if (!cap || self_absmax) launch_quant_images(in, per, c.n, sl, q, scales + pl.scale_base, s);
            pre = launch_events_used();
            launch_conv(q, op.d_w.as<int8_t>(), c, ep, s);
          }
        } else if (self_absmax) {
          launch_absmax(in, per, c.n, sl, false, nullptr, nullptr, 0, 0, s, clear);
          first_launched();
        }
        if (cap && self_absmax && fused) launch_quant_images(in, per, c.n, sl, q, scales + pl.scale_base, s);
        if (cap) RG_HIP(hipMemcpyAsync(plan.cap_q[i]->p, q, (size_t)pl.in_len, hipMemcpyDeviceToDevice, s));
        break;
      }
      case OP_POOL: {
        const auto& is = pl.in_shape;
        pre = launch_events_used();
        if (pl.pool_fused) break;  // done in the conv's epilogue
        launch_maxpool(in, out, is[0], is[1], is[2], is[3], op.k, op.s, pl.out_shape[2], pl.out_shape[3], emit,
                       pl.emit_per_image, s);
        break;
      }
      case OP_FLATTEN:
        pre = launch_events_used();
        break;
      case OP_ACT:
        pre = launch_events_used();
        if (pl.pool_fused) break;  // applied by the conv before its pool
        launch_activation(in, out, pl.in_len, op.act, op.act_param, emit, s);
        break;
      case OP_AFFINE: {
        int64_t inner = 1;
        for (size_t d = 2; d < pl.in_shape.size(); d++) inner *= pl.in_shape[d];
        pre = launch_events_used();
        launch_channel_affine(in, pl.in_len, op.in_f, inner, op.d_scale.as<float>(), op.d_bias.as<float>(), out, s);
        break;
      }
      case OP_SOFTMAX: {
        const int64_t last = pl.in_shape.back();
        pre = launch_events_used();
        if (last > 0) launch_softmax(in, out, pl.in_len / last, last, s);
        break;
      }
    }
    RG_HIP(hipGetLastError());
    if (cap)
      RG_HIP(hipMemcpyAsync(plan.cap_out[i]->p, buf(pl.out_buf), (size_t)pl.out_len * sizeof(float),
                            hipMemcpyDeviceToDevice, s));
    if (tap) {
      if (pl.slot_base >= 0) {
        const int64_t words = op.kind == OP_LINEAR ? kTensorSlotWords : pl.slot_count;
        RG_HIP(hipMemcpyAsync(plan.tap_slot[i]->p, slots + pl.slot_base, (size_t)words * sizeof(uint32_t),
                              hipMemcpyDeviceToDevice, s));
      }
      // The op's own f32 output exists unless its GEMM hands the next op its
      // operand instead (INT8 requantization, FP16 hand-off), or the conv
      // pools in its epilogue (its buffer then holds the pool's output, which
      // is the output of the MaxPool2d op; an FP32 conv's absorbed Act op
      // likewise has none of its own), or the program runs as one tiny
      // kernel (only the last op's output leaves its LDS), or the pool is
      // the first of a conv pair's (its output stays in LDS).
      const bool has_out = !pl.requant && !pl.handoff && !pl.pool_r16 && !(pl.pool_fused && op.kind != OP_POOL) &&
                           !(plan.tiny && pl.out_buf != BUF_OUTPUT) && !pl.no_out;
      plan.tap_out_ok[i] = has_out;
      if (has_out && pl.out_len > 0)
        RG_HIP(hipMemcpyAsync(plan.cap_out[i]->p, buf(pl.out_buf), (size_t)pl.out_len * sizeof(float),
                              hipMemcpyDeviceToDevice, s));
    }
    const int end = launch_events_used();
    plan.roles[i] = {first - 1, pre - 1, end > pre ? end - 1 : pre - 1};
  }
  if (timed && (size_t)launch_events_used() >= launch_event_cap(P))
    throw Error(RGNPU_ERR_INVALID, "internal: a run launched more kernels than its event budget");
  // A program with no computing op returns its input (Flatten only).
  bool any = false;
  for (auto& o : P->ops) any |= o->kind != OP_FLATTEN;
  if (!any && plan.out_len > 0)
    RG_HIP(hipMemcpyAsync(y, x, (size_t)plan.out_len * sizeof(float), hipMemcpyDeviceToDevice, s));
  if (ev) RG_HIP(hipEventRecord(ev[1], s));
  P->capture_valid = cap || tap;
  P->taps_valid = tap;
}

static void enqueue_profiled(rgnpu_program* P, Plan& plan, const float* x, float* y) {
  ensure_events(P);
  enqueue(P, plan, x, y, P->ev.data(), P->profiling > 0);
  P->profile_pending = true;
}

static void finalize_profile(rgnpu_program* P) {
  if (!P->profile_pending) return;
  RG_HIP(hipEventSynchronize(P->ev[1]));
  Plan& plan = *P->plan;
  rgnpu_profile pr{};
  pr.precision = P->precision;
  pr.original_layers = (int32_t)P->original_layers;
  pr.fused_ops = (int32_t)P->ops.size();
  pr.fp32_weight_bytes = (uint64_t)P->fp32_bytes;
  pr.npu_weight_bytes = (uint64_t)P->npu_bytes;
  float ms = 0.0f;
  RG_HIP(hipEventElapsedTime(&ms, P->ev[0], P->ev[1]));
  pr.total_ns = (uint64_t)((double)ms * 1e6);
  P->records.assign(P->ops.size(), rgnpu_op_record{});
  uint64_t total_macs = 0;
  for (size_t i = 0; i < P->ops.size(); i++) {
    rgnpu_op_record& r = P->records[i];
    snprintf(r.op, sizeof r.op, "%s", P->ops[i]->label.c_str());
    r.macs = plan.ops[i].macs;
    total_macs += r.macs;
    if (P->profiling > 0) {
      double a = 0, b = 0;
      op_times(P, plan, P->ev.data(), i, &a, &b);
      r.ns = (uint64_t)(a * 1e6);
      r.kernel_ns = (uint64_t)(b * 1e6);
    }
  }
  pr.total_macs = total_macs;
  pr.n_records = (int32_t)P->ops.size();
  P->prof = pr;
  P->have_profile = true;
  P->profile_pending = false;
}

static void write_shape(const Plan& plan, int64_t* y_shape, int32_t* y_ndim) {
  if (y_ndim) *y_ndim = (int32_t)plan.out_shape.size();
  if (y_shape)
    for (size_t d = 0; d < plan.out_shape.size(); d++) y_shape[d] = plan.out_shape[d];
}

}  // namespace rgnpu

// ===================== C ABI =================================================
#define RG_API_BEGIN try {
#define RG_API_END                                  \
  }                                                 \
  catch (const rgnpu::Error& e) {                   \
    rgnpu::g_last_error = e.what();                 \
    return e.code;                                  \
  }                                                 \
  catch (const std::bad_alloc&) {                   \
    rgnpu::g_last_error = "host allocation failed"; \
    return RGNPU_ERR_DEVICE;                        \
  }                                                 \
  catch (const std::exception& e) {                 \
    rgnpu::g_last_error = e.what();                 \
    return RGNPU_ERR_INVALID;                       \
  }                                                 \
  return RGNPU_OK;

extern "C" {

const char* rgnpu_last_error(void) { return rgnpu::g_last_error.c_str(); }

int rgnpu_program_create(const rgnpu_layer* layers, int64_t n_layers, int32_t precision, int32_t device,
                         rgnpu_program** out) {
  RG_API_BEGIN
  if (!out) throw Error(RGNPU_ERR_INVALID, "out is NULL");
  *out = nullptr;
  if (n_layers < 0 || (n_layers > 0 && !layers)) throw Error(RGNPU_ERR_INVALID, "invalid layer list");
  if (precision != RGNPU_PRECISION_INT8 && precision != RGNPU_PRECISION_FP16 && precision != RGNPU_PRECISION_FP32)
    throw Error(RGNPU_ERR_INVALID, "unknown precision");
  // the layer list is checked before any device work, so a bad spec gives
  // RGNPU_ERR_INVALID on any machine
  for (int64_t i = 0; i < n_layers; i++) check_layer(layers[i], i);
  int count = 0;
  RG_HIP(hipGetDeviceCount(&count));
  if (device < 0 || device >= count) throw Error(RGNPU_ERR_DEVICE, "device index out of range");
  auto P = std::make_unique<rgnpu_program>();
  P->device = device;
  P->precision = precision;
  RG_HIP(hipSetDevice(device));
  RG_HIP(hipStreamCreateWithFlags(&P->stream, hipStreamNonBlocking));
  try {
    load_code_object(P->stream);
    RG_HIP(hipGetLastError());
    RG_HIP(hipStreamSynchronize(P->stream));
    // this device's copy of the allocation-free entry point's scratch
    RG_HIP(scratch_address(device, &P->scratch));
    init_stats(P.get());
    compile(P.get(), layers, n_layers);
  } catch (...) {
    (void)hipStreamDestroy(P->stream);
    P->stream = nullptr;
    throw;
  }
  *out = P.release();
  RG_API_END
}

void rgnpu_program_destroy(rgnpu_program* P) {
  if (!P) return;
  for (auto& w : P->workers) {
    rgnpu_program* W = w.release();
    rgnpu_program_destroy(W);
  }
  (void)hipSetDevice(P->device);
  if (P->stream) (void)hipStreamSynchronize(P->stream);
  P->plan.reset();
  P->ops.clear();
  for (auto e : P->ev) (void)hipEventDestroy(e);
  if (P->stream) (void)hipStreamDestroy(P->stream);
  if (P->stats_host) (void)hipHostFree(P->stats_host);
  delete P;
}

}  // extern "C"

namespace rgnpu {

// One host-pointer run on P's own stream and plan (P is the handle or one of
// its workers).
static void run_host(rgnpu_program* P, const float* x, const int64_t* shape, int32_t ndim, float* y, int64_t y_cap,
                     int64_t* y_shape, int32_t* y_ndim) {
  std::lock_guard<std::mutex> lk(P->mu);
  RG_HIP(hipSetDevice(P->device));
  Plan& plan = get_plan(P, shape, ndim);
  write_shape(plan, y_shape, y_ndim);
  if (!y) return;
  if (!x && plan.in_len > 0) throw Error(RGNPU_ERR_INVALID, "x is NULL");
  if (y_cap < plan.out_len) throw Error(RGNPU_ERR_CAPACITY, "output buffer too small");
  plan.host_in.ensure((size_t)plan.in_len * sizeof(float));
  plan.host_out.ensure((size_t)plan.out_len * sizeof(float));
  // On any exit the stream drains, so no DMA still reads or writes the
  // staging ring (or the caller's buffers) once this call has returned.
  struct Drain {
    hipStream_t s;
    ~Drain() { (void)hipStreamSynchronize(s); }
  } drain{P->stream};
  if (plan.in_len > 0)
    RG_HIP(copy_to_device(P->staging, plan.host_in.p, x, (size_t)plan.in_len * sizeof(float), P->stream));
  enqueue_profiled(P, plan, plan.host_in.as<float>(), plan.host_out.as<float>());
  if (plan.out_len > 0)
    RG_HIP(copy_to_host(P->staging, y, plan.host_out.p, (size_t)plan.out_len * sizeof(float), P->stream));
  RG_HIP(hipMemcpyAsync(P->stats_host, P->stats.p, kStatWords * sizeof(uint32_t), hipMemcpyDeviceToHost, P->stream));
  RG_HIP(hipStreamSynchronize(P->stream));
  finalize_profile(P);
  check_stats(P);
}

static rgnpu_program* acquire_worker(rgnpu_program* P) {
  std::unique_lock<std::mutex> lk(P->pool_mu);
  for (;;) {
    for (size_t i = 0; i < P->workers.size(); i++)
      if (!P->worker_busy[i]) {
        P->worker_busy[i] = 1;
        return P->workers[i].get();
      }
    if (P->workers.size() < kMaxWorkers) {
      auto W = std::make_unique<rgnpu_program>();
      W->device = P->device;
      W->precision = P->precision;
      W->original_layers = P->original_layers;
      W->fp32_bytes = P->fp32_bytes;
      W->npu_bytes = P->npu_bytes;
      W->ops = P->ops;
      RG_HIP(hipSetDevice(P->device));
      RG_HIP(hipStreamCreateWithFlags(&W->stream, hipStreamNonBlocking));
      init_stats(W.get());
      P->workers.push_back(std::move(W));
      P->worker_busy.push_back(1);
      return P->workers.back().get();
    }
    P->pool_cv.wait(lk);
  }
}

static void release_worker(rgnpu_program* P, rgnpu_program* W) {
  {
    std::lock_guard<std::mutex> lk(P->pool_mu);
    for (size_t i = 0; i < P->workers.size(); i++)
      if (P->workers[i].get() == W) P->worker_busy[i] = 0;
  }
  P->pool_cv.notify_one();
}

}  // namespace rgnpu

extern "C" {

int rgnpu_program_run(rgnpu_program* P, const float* x, const int64_t* shape, int32_t ndim, float* y, int64_t y_cap,
                      int64_t* y_shape, int32_t* y_ndim) {
  RG_API_BEGIN
  if (!P || !shape) throw Error(RGNPU_ERR_INVALID, "NULL argument");
  bool capture;
  int profiling;
  {
    std::lock_guard<std::mutex> lk(P->mu);
    capture = P->capture || P->taps;
    profiling = P->profiling;
  }
  if (capture) {
    // capture and production taps live on the handle's own plan
    run_host(P, x, shape, ndim, y, y_cap, y_shape, y_ndim);
    return RGNPU_OK;
  }
  rgnpu_program* W = acquire_worker(P);
  struct Release {
    rgnpu_program *P, *W;
    ~Release() { release_worker(P, W); }
  } rel{P, W};
  W->profiling = profiling;
  {
    // persistent grids until two host runs of this program have overlapped
    std::lock_guard<std::mutex> lk(P->pool_mu);
    int busy = 0;
    for (char b : P->worker_busy) busy += b != 0;
    if (busy > 1) P->concurrent_seen = true;
    W->use_persistent = !P->concurrent_seen;
  }
  run_host(W, x, shape, ndim, y, y_cap, y_shape, y_ndim);
  if (y && W->have_profile) {
    // the last completed run's profile (mod.rs:217)
    std::lock_guard<std::mutex> lk(P->mu);
    P->prof = W->prof;
    P->records = W->records;
    P->have_profile = true;
    // this completed run supersedes a device run still awaiting its profile
    P->profile_pending = false;
  }
  RG_API_END
}

int rgnpu_program_run_device(rgnpu_program* P, const float* d_x, const int64_t* shape, int32_t ndim, float* d_y,
                             int64_t y_cap, int64_t* y_shape, int32_t* y_ndim) {
  RG_API_BEGIN
  if (!P || !shape) throw Error(RGNPU_ERR_INVALID, "NULL argument");
  std::lock_guard<std::mutex> lk(P->mu);
  RG_HIP(hipSetDevice(P->device));
  Plan& plan = get_plan(P, shape, ndim);
  write_shape(plan, y_shape, y_ndim);
  if (!d_y) return RGNPU_OK;
  if (!d_x && plan.in_len > 0) throw Error(RGNPU_ERR_INVALID, "x is NULL");
  if (y_cap < plan.out_len) throw Error(RGNPU_ERR_CAPACITY, "output buffer too small");
  enqueue_profiled(P, plan, d_x, d_y);
  RG_API_END
}

static_assert(kScratchBytes == RGNPU_NOALLOC_SCRATCH_BYTES, "the header states the scratch size");

int rgnpu_program_run_device_noalloc(rgnpu_program* P, const float* d_x, const int64_t* shape, int32_t ndim,
                                     float* d_y, int64_t y_cap, int64_t* y_shape, int32_t* y_ndim) {
  RG_API_BEGIN
  if (!P || !shape) throw Error(RGNPU_ERR_INVALID, "NULL argument");
  std::lock_guard<std::mutex> lk(P->mu);
  if (P->capture || P->taps)
    throw Error(RGNPU_ERR_INVALID, "capture mode allocates its tap buffers: use rgnpu_program_run_device");
  if (!P->scratch) throw Error(RGNPU_ERR_DEVICE, "no device scratch for this program");
  RG_HIP(hipSetDevice(P->device));
  Plan* plan = P->scratch_plan.get();
  if (!plan || (int)plan->in_shape.size() != ndim || !std::equal(plan->in_shape.begin(), plan->in_shape.end(), shape)) {
    // the previous plan's mask upload may still read its host copy
    if (plan) RG_HIP(hipStreamSynchronize(P->stream));
    P->scratch_plan.reset();
    P->scratch_plan = make_plan(P, shape, ndim, P->scratch);
    plan = P->scratch_plan.get();
  }
  write_shape(*plan, y_shape, y_ndim);
  if (!d_y) return RGNPU_OK;
  if (!d_x && plan->in_len > 0) throw Error(RGNPU_ERR_INVALID, "x is NULL");
  if (y_cap < plan->out_len) throw Error(RGNPU_ERR_CAPACITY, "output buffer too small");
  enqueue(P, *plan, d_x, d_y, nullptr, false);
  RG_API_END
}

int rgnpu_program_benchmark(rgnpu_program* P, const float* d_x, const int64_t* shape, int32_t ndim, float* d_y,
                            int64_t y_cap, int32_t iters, int32_t flags, double* total_ms,
                            rgnpu_op_record* avg, int32_t cap) {
  RG_API_BEGIN
  if (!P || !shape || !d_y || iters <= 0) throw Error(RGNPU_ERR_INVALID, "invalid arguments");
  const bool per_kernel_events = (flags & RGNPU_BENCH_KERNEL_EVENTS) != 0;
  std::lock_guard<std::mutex> lk(P->mu);
  if (P->capture || P->taps) throw Error(RGNPU_ERR_INVALID, "capture mode is on: benchmark times the production path only");
  RG_HIP(hipSetDevice(P->device));
  Plan& plan = get_plan(P, shape, ndim);
  if (y_cap < plan.out_len) throw Error(RGNPU_ERR_CAPACITY, "output buffer too small");
  const size_t per = events_per_run(P);
  const size_t sets = per_kernel_events ? (size_t)iters : 1;
  std::vector<hipEvent_t> evs(per * sets + 2, nullptr);
  struct Guard {
    std::vector<hipEvent_t>& v;
    ~Guard() {
      for (auto e : v)
        if (e) (void)hipEventDestroy(e);
    }
  } guard{evs};
  for (size_t i = 0; i < evs.size(); i++) {
    if (i >= (size_t)(per * sets))
      RG_HIP(hipEventCreate(&evs[i]));  // the region's own start/end
    else
      create_run_event(&evs[i], i % (size_t)per);
  }
  hipEvent_t t0 = evs[per * sets], t1 = evs[per * sets + 1];
  const bool evict = (flags & RGNPU_BENCH_EVICT_CACHE) != 0;
  if (evict && !P->evict.p) {
    P->evict.ensure(kEvictBytes + 256);
    launch_fill_u32(P->evict.as<uint32_t>(), (kEvictBytes + 256) / 4, 0u, P->stream);
  }
  RG_HIP(hipStreamSynchronize(P->stream));
  RG_HIP(hipEventRecord(t0, P->stream));
  for (int32_t it = 0; it < iters; it++) {
    hipEvent_t* set = per_kernel_events ? evs.data() + per * (size_t)it : nullptr;
    // before the run's start marker: no op interval includes it
    if (evict)
      launch_evict(P->evict.p, kEvictBytes,
                   reinterpret_cast<uint32_t*>(static_cast<char*>(P->evict.p) + kEvictBytes), P->stream);
    enqueue(P, plan, d_x, d_y, set, per_kernel_events);
  }
  RG_HIP(hipEventRecord(t1, P->stream));
  RG_HIP(hipEventSynchronize(t1));
  float ms = 0.0f;
  RG_HIP(hipEventElapsedTime(&ms, t0, t1));
  if (total_ms) *total_ms = ms;
  read_stats(P);
  check_stats(P);
  if (avg) {
    for (size_t i = 0; i < P->ops.size() && (int32_t)i < cap; i++) {
      rgnpu_op_record r{};
      snprintf(r.op, sizeof r.op, "%s", P->ops[i]->label.c_str());
      r.macs = plan.ops[i].macs;
      if (per_kernel_events) {
        double a = 0, b = 0;
        for (int32_t it = 0; it < iters; it++) {
          double x = 0, y = 0;
          op_times(P, plan, evs.data() + per * (size_t)it, i, &x, &y);
          a += x;
          b += y;
        }
        r.ns = (uint64_t)(a / iters * 1e6);
        r.kernel_ns = (uint64_t)(b / iters * 1e6);
      }
      avg[i] = r;
    }
  }
  RG_API_END
}

int rgnpu_program_synchronize(rgnpu_program* P) {
  RG_API_BEGIN
  if (!P) throw Error(RGNPU_ERR_INVALID, "NULL program");
  std::lock_guard<std::mutex> lk(P->mu);
  RG_HIP(hipSetDevice(P->device));
  RG_HIP(hipStreamSynchronize(P->stream));
  if (P->plan) finalize_profile(P);
  read_stats(P);
  check_stats(P);
  RG_API_END
}

int rgnpu_program_set_profiling(rgnpu_program* P, int32_t level) {
  RG_API_BEGIN
  if (!P) throw Error(RGNPU_ERR_INVALID, "NULL program");
  std::lock_guard<std::mutex> lk(P->mu);
  P->profiling = level > 0 ? 1 : 0;
  RG_API_END
}

int rgnpu_program_profile(rgnpu_program* P, rgnpu_profile* out, rgnpu_op_record* records, int32_t cap) {
  RG_API_BEGIN
  if (!P || !out) throw Error(RGNPU_ERR_INVALID, "NULL argument");
  std::lock_guard<std::mutex> lk(P->mu);
  RG_HIP(hipSetDevice(P->device));
  if (P->plan) finalize_profile(P);
  if (!P->have_profile) throw Error(RGNPU_ERR_INVALID, "no run has completed yet");
  *out = P->prof;
  if (records)
    for (int32_t i = 0; i < cap && i < (int32_t)P->records.size(); i++) records[i] = P->records[(size_t)i];
  RG_API_END
}

int64_t rgnpu_program_num_ops(const rgnpu_program* P) { return P ? (int64_t)P->ops.size() : -1; }

int64_t rgnpu_program_op_label(const rgnpu_program* P, int64_t i, char* buf, int64_t cap) {
  if (!P || i < 0 || i >= (int64_t)P->ops.size()) return -1;
  const std::string& l = P->ops[(size_t)i]->label;
  if (buf && cap > 0) snprintf(buf, (size_t)cap, "%s", l.c_str());
  return (int64_t)l.size();
}

int64_t rgnpu_program_op_weight(const rgnpu_program* P, int64_t i, int8_t* dst, int64_t cap, float* scale) {
  if (!P || i < 0 || i >= (int64_t)P->ops.size()) return -1;
  const Op& op = *P->ops[(size_t)i];
  if (scale) *scale = op.w_scale;
  if (dst) std::memcpy(dst, op.wq.data(), (size_t)std::min<int64_t>(cap, (int64_t)op.wq.size()));
  return (int64_t)op.wq.size();
}

int64_t rgnpu_program_summary(const rgnpu_program* P, char* buf, int64_t cap) {
  if (!P) return -1;
  // NpuProgram::summary (npu.rs:280-293)
  const float ratio = P->npu_bytes == 0 ? 1.0f : (float)P->fp32_bytes / (float)P->npu_bytes;
  std::string names;
  for (size_t i = 0; i < P->ops.size(); i++) {
    if (i) names += " -> ";
    names += P->ops[i]->label;
  }
  char head[512];
  if (P->precision == RGNPU_PRECISION_FP32) {
    // compilation_report of a Standard program (mod.rs:198-204)
    snprintf(head, sizeof head, "InferenceSession [provider = GPU:%d (FP32), device = gpu:%d, ops = %zu (from %lld raw layers)]",
             P->device, P->device, P->ops.size(), (long long)P->original_layers);
    const std::string st(head);
    if (buf && cap > 0) snprintf(buf, (size_t)cap, "%s", st.c_str());
    return (int64_t)st.size();
  }
  snprintf(head, sizeof head,
           "InferenceSession [provider = MI355X (%s), layers: %lld -> %zu fused ops, weights: %lld B -> %lld B (%.2fx "
           "compression)]\n  Pipeline: ",
           P->precision == RGNPU_PRECISION_FP16 ? "FP16" : "INT8", (long long)P->original_layers, P->ops.size(), (long long)P->fp32_bytes, (long long)P->npu_bytes, (double)ratio);
  std::string s = std::string(head) + names;
  if (buf && cap > 0) snprintf(buf, (size_t)cap, "%s", s.c_str());
  return (int64_t)s.size();
}

int rgnpu_program_set_capture(rgnpu_program* P, int32_t on) {
  RG_API_BEGIN
  if (!P) throw Error(RGNPU_ERR_INVALID, "NULL program");
  if (on < RGNPU_CAPTURE_OFF || on > RGNPU_CAPTURE_PRODUCTION) throw Error(RGNPU_ERR_INVALID, "unknown capture mode");
  std::lock_guard<std::mutex> lk(P->mu);
  P->capture = on == RGNPU_CAPTURE_FULL;
  P->taps = on == RGNPU_CAPTURE_PRODUCTION;
  P->capture_valid = false;
  P->taps_valid = false;
  RG_API_END
}

int64_t rgnpu_program_capture(rgnpu_program* P, int64_t i, int32_t what, void* dst, int64_t cap_bytes) {
  try {
    if (!P) {
      rgnpu::g_last_error = "no capture available";
      return -1;
    }
    std::lock_guard<std::mutex> lk(P->mu);
    if (!P->plan || !P->capture_valid || i < 0 || i >= (int64_t)P->ops.size()) {
      rgnpu::g_last_error = "no capture available";
      return -1;
    }
    RG_HIP(hipSetDevice(P->device));
    RG_HIP(hipStreamSynchronize(P->stream));
    Plan& plan = *P->plan;
    const Op& op = *P->ops[(size_t)i];
    const OpPlan& pl = plan.ops[(size_t)i];
    // FP16 and FP32 have no quantized activations, scales or integer sums to expose.
    const bool gemm = (op.kind == OP_LINEAR || op.kind == OP_CONV) && P->precision == RGNPU_PRECISION_INT8;
    auto copy_out = [&](const void* src, int64_t count, size_t elem) -> int64_t {
      if (dst) {
        const int64_t bytes = std::min<int64_t>(cap_bytes, count * (int64_t)elem);
        if (bytes > 0) RG_HIP(hipMemcpy(dst, src, (size_t)bytes, hipMemcpyDeviceToHost));
      }
      return count;
    };
    if (P->taps_valid) {
      switch (what) {
        case RGNPU_CAP_OUT:
          if (!plan.tap_out_ok[(size_t)i]) return 0;
          return copy_out(plan.cap_out[(size_t)i]->p, pl.out_len, sizeof(float));
        case RGNPU_CAP_ACC:
          return 0;  // the i32 sums never leave the GEMM's registers
        case RGNPU_CAP_SCALE: {
          if (!gemm || !plan.tap_scale_ok[(size_t)i]) return 0;
          // the scale each consumer derives from the absmax slot that its
          // producer (or its own absmax pass) filled
          const bool lin = op.kind == OP_LINEAR;
          std::vector<uint32_t> w((size_t)(lin ? kTensorSlotWords : pl.slot_count));
          RG_HIP(hipMemcpy(w.data(), plan.tap_slot[(size_t)i]->p, w.size() * sizeof(uint32_t), hipMemcpyDeviceToHost));
          std::vector<float> sc;
          if (lin) {
            uint32_t m = 0;
            for (int k = 0; k < kSpread; k++) m = std::max(m, w[(size_t)k * kSpreadStride]);
            sc.push_back(rgmath::scale_from_absmax(rgmath::bitsf(m)));
          } else {
            for (uint32_t m : w) sc.push_back(rgmath::scale_from_absmax(rgmath::bitsf(m)));
          }
          const int64_t b = std::min<int64_t>(cap_bytes, (int64_t)(sc.size() * sizeof(float)));
          if (dst && b > 0) std::memcpy(dst, sc.data(), (size_t)b);
          return (int64_t)sc.size();
        }
        case RGNPU_CAP_QACT:
          if (!gemm || op.kind != OP_LINEAR || !plan.tap_q_ok[(size_t)i]) return 0;
          break;  // the Linear operand, read back as in capture mode
        default:
          return -1;
      }
    }
    switch (what) {
      case RGNPU_CAP_OUT:
        return copy_out(plan.cap_out[(size_t)i]->p, pl.out_len, sizeof(float));
      case RGNPU_CAP_ACC: {
        if (!gemm) return 0;
        const int64_t n = op.kind == OP_LINEAR ? pl.rows * op.out_f : pl.cs.n * pl.cs.OH * pl.cs.OW * op.out_f;
        return copy_out(plan.cap_acc[(size_t)i]->p, n, sizeof(int32_t));
      }
      case RGNPU_CAP_SCALE:
        if (!gemm) return 0;
        return copy_out(plan.scales.as<float>() + pl.scale_base, pl.slot_count, sizeof(float));
      case RGNPU_CAP_QACT: {
        if (!gemm) return 0;
        if (op.kind == OP_LINEAR) {
          std::vector<int8_t> full((size_t)(pl.Mpad * op.Kpad));
          RG_HIP(hipMemcpy(full.data(), plan.cap_q[(size_t)i]->p, full.size(), hipMemcpyDeviceToHost));
          const int64_t n = pl.rows * op.K;
          if (dst) {
            int8_t* d = static_cast<int8_t*>(dst);
            for (int64_t r = 0; r < pl.rows; r++)
              for (int64_t c = 0; c < op.K; c++) {
                const int64_t o = r * op.K + c;
                if (o < cap_bytes) d[o] = full[(size_t)(r * op.Kpad + c)];
              }
          }
          return n;
        }
        // Conv: transposed im2col [n, L, C*k*k] of the quantized image.
        const ConvShape& c = pl.cs;
        std::vector<int8_t> img((size_t)pl.in_len);
        RG_HIP(hipMemcpy(img.data(), plan.cap_q[(size_t)i]->p, img.size(), hipMemcpyDeviceToHost));
        const int64_t L = c.OH * c.OW, KK = op.K;
        const int64_t n = c.n * L * KK;
        if (dst) {
          int8_t* d = static_cast<int8_t*>(dst);
          for (int64_t b = 0; b < c.n; b++)
            for (int64_t l = 0; l < L; l++)
              for (int64_t kk = 0; kk < KK; kk++) {
                const int64_t o = (b * L + l) * KK + kk;
                if (o >= cap_bytes) continue;
                const int64_t ch = kk / (c.k * c.k), rem = kk % (c.k * c.k), ki = rem / c.k, kj = rem % c.k;
                const int64_t iy = (l / c.OW) * c.stride + ki - c.pad, ix = (l % c.OW) * c.stride + kj - c.pad;
                int8_t v = 0;
                if (iy >= 0 && iy < c.H && ix >= 0 && ix < c.W) v = img[(size_t)(((b * c.C + ch) * c.H + iy) * c.W + ix)];
                d[o] = v;
              }
        }
        return n;
      }
    }
    return -1;
  } catch (const std::exception& e) {
    rgnpu::g_last_error = e.what();
    return -1;
  }
}

int rgnpu_program_barrier_stats(rgnpu_program* P, uint64_t* deferred, uint64_t* unsettled, uint64_t* launches) {
  RG_API_BEGIN
  if (!P) throw Error(RGNPU_ERR_INVALID, "NULL program");
  uint64_t d = 0, u = 0, l = 0;
  auto add = [&](rgnpu_program* C) {
    RG_HIP(hipSetDevice(C->device));
    RG_HIP(hipStreamSynchronize(C->stream));
    uint32_t w[kStatWords];
    RG_HIP(hipMemcpy(w, C->stats.p, sizeof w, hipMemcpyDeviceToHost));
    d += w[kStatDeferred];
    u += w[kStatUnsettled];
    l += w[kStatLaunches];
  };
  {
    std::lock_guard<std::mutex> lk(P->mu);
    add(P);
  }
  {
    // idle workers only: a busy one is mid-run on another thread
    std::lock_guard<std::mutex> lk(P->pool_mu);
    for (size_t i = 0; i < P->workers.size(); i++)
      if (!P->worker_busy[i]) add(P->workers[i].get());
  }
  if (deferred) *deferred = d;
  if (unsettled) *unsettled = u;
  if (launches) *launches = l;
  RG_API_END
}

int rgnpu_probe_barrier_poll(int32_t device, int32_t blocks, int32_t polls, double* us_per_poll) {
  RG_API_BEGIN
  if (!us_per_poll || blocks <= 0 || blocks > 4096 || polls <= 0) throw Error(RGNPU_ERR_INVALID, "invalid arguments");
  RG_HIP(hipSetDevice(device));
  DevBuf lines;
  const int64_t words = (int64_t)blocks * 32;  // one 128-byte line per workgroup
  lines.ensure((size_t)words * sizeof(uint32_t));
  hipStream_t s = nullptr;
  RG_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  struct Destroy {
    hipStream_t s;
    ~Destroy() { (void)hipStreamDestroy(s); }
  } destroy{s};
  load_code_object(s);
  launch_fill_u32(lines.as<uint32_t>(), words, 0u, s);
  RG_HIP(hipGetLastError());
  RG_HIP(hipStreamSynchronize(s));
  const double ms = probe_barrier_poll(lines.as<uint32_t>(), blocks, polls, s);
  RG_HIP(hipStreamSynchronize(s));
  if (ms <= 0) throw Error(RGNPU_ERR_DEVICE, "barrier poll probe failed");
  *us_per_poll = ms * 1000.0 / polls;
  RG_API_END
}

int rgnpu_probe_mfma_rate(int32_t device, int64_t iters, int32_t random_operands, double* ms, double* tops) {
  RG_API_BEGIN
  if (!ms || !tops || iters <= 0) throw Error(RGNPU_ERR_INVALID, "invalid arguments");
  RG_HIP(hipSetDevice(device));
  std::vector<uint8_t> host(256 * 16 + 16, 0);
  if (random_operands) {
    uint64_t z = 0x9e3779b97f4a7c15ull;  // SplitMix64 stream
    for (auto& b : host) {
      z += 0x9e3779b97f4a7c15ull;
      uint64_t t = z;
      t = (t ^ (t >> 30)) * 0xbf58476d1ce4e5b9ull;
      t = (t ^ (t >> 27)) * 0x94d049bb133111ebull;
      b = (uint8_t)(t ^ (t >> 31));
    }
  }
  DevBuf buf;
  buf.ensure(host.size());
  RG_HIP(hipMemcpy(buf.p, host.data(), host.size(), hipMemcpyHostToDevice));
  hipStream_t s = nullptr;
  RG_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  int64_t macs = 0;
  const double t = probe_mfma_rate(buf.p, iters, reinterpret_cast<int32_t*>(buf.as<uint8_t>() + 256 * 16), &macs, s);
  (void)hipStreamDestroy(s);
  if (t <= 0) throw Error(RGNPU_ERR_DEVICE, "MFMA probe launch failed");
  *ms = t;
  *tops = 2.0 * (double)macs / (t * 1e-3) / 1e12;
  RG_API_END
}

int rgnpu_device_count(int32_t* count) {
  RG_API_BEGIN
  int c = 0;
  RG_HIP(hipGetDeviceCount(&c));
  if (count) *count = c;
  RG_API_END
}

int rgnpu_device_alloc(int32_t device, int64_t bytes, void** out) {
  RG_API_BEGIN
  if (!out || bytes < 0) throw Error(RGNPU_ERR_INVALID, "invalid arguments");
  RG_HIP(hipSetDevice(device));
  RG_HIP(hipMalloc(out, (size_t)(bytes ? bytes : 16)));
  RG_API_END
}

int rgnpu_device_free(void* p) {
  RG_API_BEGIN
  if (p) RG_HIP(hipFree(p));
  RG_API_END
}

int rgnpu_memcpy_h2d(void* dst, const void* src, int64_t bytes) {
  RG_API_BEGIN
  if (bytes > 0) RG_HIP(hipMemcpy(dst, src, (size_t)bytes, hipMemcpyHostToDevice));
  RG_API_END
}

int rgnpu_memcpy_d2h(void* dst, const void* src, int64_t bytes) {
  RG_API_BEGIN
  if (bytes > 0) RG_HIP(hipMemcpy(dst, src, (size_t)bytes, hipMemcpyDeviceToHost));
  RG_API_END
}

int rgnpu_device_synchronize(void) {
  RG_API_BEGIN
  RG_HIP(hipDeviceSynchronize());
  RG_API_END
}

}  // extern "C"
