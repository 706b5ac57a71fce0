// rgnpu_internal.h — declarations shared by the host runtime (program.cpp)
// and the HIP kernels (kernels.hip).  Nothing here is part of the C ABI.
#pragma once
#include <hip/hip_runtime_api.h>
#include <stdint.h>

namespace rgnpu {

// Padding rules for device operands.  Weights are stored [Npad, Kpad] with
// zero rows/columns so every MFMA tile load stays in bounds.
constexpr int64_t kRowPad = 256;   // Linear output features and activation rows
constexpr int64_t kKPad = 128;     // reduction dimension (bytes)
constexpr int64_t kKPadHalf = 32;  // FP16 reduction dimension (binary16 elements: one 64-byte K step)
constexpr int64_t kKPadF32 = 16;   // FP32 reduction dimension (f32 elements: one 64-byte K step)
constexpr int64_t kConvOPad = 32;  // conv output channels

inline int64_t round_up(int64_t v, int64_t m) { return (v + m - 1) / m * m; }

// Absmax slots.  A per-image absmax (conv consumers) is one u32 per image.
// A per-tensor absmax (Linear consumers) is spread over kSpread partial
// maxima kSpreadStride words (128 bytes) apart: each producing wave or
// block raises the partial picked by its index, and consumers fold all
// kSpread partials with one load per lane.  Device-scope atomics on one
// address are serialised at the memory side on MI355X (the eight XCD L2s
// are not coherent), so thousands of waves ending together on a single
// slot would cost tens of microseconds.
constexpr int kSpread = 64;
constexpr int kSpreadStride = 32;
constexpr int64_t kTensorSlotWords = (int64_t)kSpread * kSpreadStride;

// A plan's absmax slots are double-buffered by run parity when the run's
// first kernel is an input absmax: that kernel also zeroes the other set
// (p[0 .. n)), which the next run then uses.
struct SlotClear {
  uint32_t* p = nullptr;
  int64_t n = 0;
};

// Fused epilogue parameters: y = act(float(acc) * (sa * sw) + bias[n]).
struct Epilogue {
  const float* bias = nullptr;        // [N] (padded)
  int act = 0;
  float act_param = 0.0f;
  const uint32_t* absmax_in = nullptr; // activation absmax: spread slot (Linear) or per image (conv)
  float w_scale = 1.0f;
  float* y = nullptr;                  // f32 output
  uint32_t* absmax_out = nullptr;      // nullable: absmax of y for the next op
  int absmax_out_per_image = 0;        // 1: slot per image; 0: spread per-tensor slot
  int32_t* acc_out = nullptr;          // nullable: i32 accumulator capture
  int y_stream = 0;                    // 1: y is the program's output, stored with the non-temporal hint
  // FP16 Linear -> FP16 Linear: the consumer's binary16 operand [Mpad, ldh]
  // (zero padded), written by this GEMM's epilogue in place of the consumer's
  // conversion pass; no f32 output is stored then.
  uint16_t* h_out = nullptr;
  int64_t ldh = 0;
  int gelu_cert = 0;  // with h_out and GELU: 1 certified (2, 3 test modes as in Requant), 0 exact
  // INT8 conv -> MaxPool2d(2, 2): y is the pool's output [n, O, OH/2, OW/2]
  // and absmax_out its absmax; the value is OW / 16 (1 or 2), 0 = no pool.
  int pool2 = 0;
};

// Requantization fused into a producing Linear's GEMM (requant.hip): the
// next Linear's i8 operand q [Mpad, ldq] is written by this GEMM once the
// absmax of its whole output (ep.absmax_out) is known.  sync points at
// requant_sync_words() zeroed words (arrival counters, per-workgroup states
// from kRequantStateBase on, and per-workgroup release lines).
struct Requant {
  int8_t* q = nullptr;        // next op's activations [Mpad, ldq], zero padded
  int64_t ldq = 0;            // next op's Kpad (<= the producer's Npad)
  uint32_t* sync = nullptr;
  float* scale_out = nullptr; // nullable: the scale used (capture tap)
  int keep_f32 = 0;           // also store every f32 output (capture)
  int spin_limit = 0;         // barrier polls (kBarrierPollUs each) before a workgroup defers its quantization
  int gelu_cert = 1;          // GELU without capture: 1 certified path, 0 exact; 2 and 3 test modes (cert_const)
  uint32_t* stats = nullptr;  // the context's cumulative barrier counters (kStat*)
};
constexpr int64_t kRequantStateBase = 320;

// Cumulative counters of the persistent grids' barriers, one block per
// program context (handle or worker), never cleared by a run: workgroups
// that gave up waiting and deferred their quantization to the finisher,
// workgroups a finisher found unsettled (their tiles were not quantized:
// the run's result is incomplete and the host reports RGNPU_ERR_DEVICE), and
// finished barrier launches.
constexpr int kStatDeferred = 0, kStatUnsettled = 1, kStatLaunches = 2, kStatWords = 4;

// One barrier poll (an s_sleep of 8 x 64 clocks and one agent-scope load of
// the workgroup's go line), measured on the MI355X with
// rgnpu_probe_barrier_poll over 256 workgroups: 0.32 us.  The default bound
// of 100000 polls is therefore ~32 ms before a workgroup defers; a finisher
// waits at most that plus 100000 polls (~64 ms in all) for a workgroup to
// settle.
constexpr double kBarrierPollUs = 0.32;
// Times `polls` barrier polls of one thread in each of `blocks` workgroups on
// lines that are never set (requant.hip); returns ms (negative on failure).
double probe_barrier_poll(uint32_t* lines, int blocks, int polls, hipStream_t s);

// ---- launchers (kernels.hip) -------------------------------------------
// Launch events: while set_launch_events(events, cap) is active on this
// thread, the i-th kernel launched by the launchers below records events[i]
// as the stop event of its own dispatch (hipExtLaunchKernelGGL), i.e. the
// completion timestamp of that kernel, with no marker packet and no bubble
// before the next kernel.  launch_events_used() counts the launches so far.
// set_launch_events(nullptr, 0) turns it off.
void set_launch_events(hipEvent_t* events, int cap);
int launch_events_used();

void launch_fill_u32(uint32_t* p, int64_t n, uint32_t v, hipStream_t s);
// Loads the library's kernels on the current device (one empty launch per
// code object: kernels.hip and requant.hip).
void load_code_object(hipStream_t s);

// Times one launch of the register-only MFMA probe (kernels.hip): 8 waves
// per CU, `iters` rounds of 32 i8 16x16x64 MFMAs per wave on operands built
// from the 256 words at ops.  Returns the elapsed ms (negative on failure)
// and the MACs performed.
double probe_mfma_rate(const void* ops, int64_t iters, int32_t* sink, int64_t* macs_out, hipStream_t s);
void load_requant_code_object(hipStream_t s);

// Device scratch of the allocation-free run entry point (scratch.hip): one
// file-scope array of kScratchBytes per device.  scratch_address looks up
// this device's copy (the device must be current) on its first call for the
// device and returns the cached address afterwards.
constexpr int64_t kScratchBytes = int64_t(64) << 20;
hipError_t scratch_address(int device, void** out);
// Reads `bytes` (a zero-filled buffer) to displace the memory-side cache.
void launch_evict(const void* p, int64_t bytes, uint32_t* sink, hipStream_t s);

// Absmax of x (f32) (atomic max of |x| bits, NaN ignored): per image into
// slots[img], or with n_img == 1 and `spread` into a spread per-tensor slot.
// per_img elements per image, n_img images; optional coverage masks select
// which (row, col) positions of a [C,H,W] image participate.
void launch_absmax(const float* x, int64_t per_img, int64_t n_img, uint32_t* slots, bool spread,
                   const uint8_t* rowmask, const uint8_t* colmask, int64_t H, int64_t W,
                   hipStream_t s,
                   SlotClear clear = SlotClear{});

// x f32 [M,K] -> q i8 [Mpad,Kpad] (zero padded), scale from a spread slot.
// scale_out (nullable) receives the scale used.
void launch_quant_rows(const float* x, int64_t M, int64_t K, int64_t Mpad, int64_t Kpad,
                       const uint32_t* slot, int8_t* q, float* scale_out, hipStream_t s);

// x f32 [n_img, per_img] -> q i8, per-image scale from slots[img].
void launch_quant_images(const float* x, int64_t per_img, int64_t n_img, const uint32_t* slots,
                         int8_t* q, float* scales_out, hipStream_t s);

// C[M,N] = A[Mpad,Kpad] . B[Npad,Kpad]^T with the fused epilogue.  Mpad and
// Npad are multiples of 128, Kpad of 64.  Shapes with few tiles split K
// through `ws` (i32 partial sums, gemm_workspace_bytes() bytes); without a
// large enough workspace they run unsplit.
void launch_gemm(const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t Mpad,
                 int64_t Npad, int64_t Kpad, const Epilogue& ep, int32_t* ws, int64_t ws_bytes,
                 hipStream_t s);
int64_t gemm_workspace_bytes(int64_t Mpad, int64_t Npad, int64_t Kpad);
// Tile shape of the large GEMM for a padded problem: 0 = 256 x 256,
// 1 = 256 x 128, 2 = 128 x 128; splits > 1 when K is split.
struct GemmChoice {
  int kind;
  int splits;
};
GemmChoice choose_gemm(int64_t Mpad, int64_t Npad, int64_t Kpad);

// The same GEMM with the next Linear's quantization fused (requant.hip):
// a persistent grid computes every tile and its fused epilogue, raises
// ep.absmax_out, meets at a grid barrier, then quantizes its tiles into
// rq.q with the scale of the whole output.  Only for unsplit problems
// (choose_gemm(...).splits == 1).  ep.y receives the f32 outputs the
// quantization reads back (all of them when rq.keep_f32).
bool gemm_requant_supported(int64_t Mpad, int64_t Npad, int64_t Kpad);
int64_t requant_sync_words(int64_t Mpad, int64_t Npad, int64_t Kpad);
void launch_gemm_requant(const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t Mpad, int64_t Npad,
                         int64_t Kpad, const Epilogue& ep, const Requant& rq, hipStream_t s);

// A Linear input's quantization in one pass (requant.hip): x f32 [M, K] ->
// q i8 [Mpad, Kpad] (padding zero) with the per-tensor absmax raised into the
// spread slot and its scale written to scale_out; a persistent grid that
// keeps its share of x in registers and LDS across a grid barrier (sync:
// input_quant_sync_words() zeroed words).  The run's first kernel also
// zeroes `clear`.  Requires input_quant_supported.
bool input_quant_supported(int64_t M, int64_t K, int64_t Mpad, int64_t Kpad);
int64_t input_quant_sync_words(int64_t Mpad, int64_t Kpad);
void launch_input_quant(const float* x, int64_t M, int64_t K, int64_t Mpad, int64_t Kpad, uint32_t* slot, int8_t* q,
                        float* scale_out, uint32_t* sync, int spin_limit, uint32_t* stats, SlotClear clear,
                        hipStream_t s);

// Same contract for M <= 8 rows (weight-streaming GEMV).
// INT8 Linear with N <= kNarrowMaxN outputs per row: one wave per row, the
// weights from L1 (A [M,Kpad], B [>= N, Kpad]).
constexpr int64_t kNarrowMaxN = 16;
void launch_gemm_narrow(const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t Kpad, const Epilogue& ep,
                        hipStream_t s);
// The same reading the f32 input x [M, K] and quantizing it as it is read,
// with the scale of the spread slot ep.absmax_in (a producer emitted it);
// q_out / scale_out (nullable) receive the i8 operand [M, Kpad] and the
// scale (capture).
bool gemm_narrow_xq_supported(int64_t K, int64_t Kpad);
void launch_gemm_narrow_xq(const float* x, const int8_t* B, int64_t M, int64_t N, int64_t K, int64_t Kpad,
                           const Epilogue& ep, int8_t* q_out, float* scale_out, hipStream_t s);
// INT8 Linear with few output tiles, reading the f32 input x [M, K] and
// quantizing it as it is read with the scale of the spread slot
// ep.absmax_in: one workgroup per 16 x 16 or 16 x 64 output block and K
// slice, the slice's K steps spread over its waves and their sums added in
// LDS; the fused epilogue of launch_gemm.  B [Npad, Kpad].  With more than
// one K slice, sync (gemm_xq_small_sync_words, zero at launch, 8-byte
// aligned) holds a 64-bit word per output in which the slices meet.  No
// capture outputs.
bool gemm_xq_small_supported(int64_t M, int64_t N, int64_t Npad, int64_t K, int64_t Kpad);
int64_t gemm_xq_small_sync_words(int64_t M, int64_t Npad, int64_t Kpad);
void launch_gemm_xq_small(const float* x, const int8_t* B, int64_t M, int64_t N, int64_t Npad, int64_t K,
                          int64_t Kpad, const Epilogue& ep, uint32_t* sync, hipStream_t s);
// A whole program of small INT8 Linears (npu.rs:307-318 per op: the input
// quantized per tensor with its own absmax, quantize.rs:18-24, then the
// fused GEMM, quantize.rs:93-118) in one workgroup, for programs whose every
// op is a Linear on the same rows: at most kTinyMaxLayers layers, kTinyRows
// rows, kTinyWidth input and output features, Kpad == kTinyWidth (the INT8
// Kpad of any K <= kTinyWidth), and kTinyWeightBytes of weights (out_f x Kpad
// per layer) in all.  Layer l reads
// w [out_f, Kpad] (i8, zero K padding) and writes its input's absmax key into
// slot[0] (a spread slot the run zeroed); the last layer writes y [rows, out_f].
constexpr int kTinyMaxLayers = 8, kTinyRows = 64, kTinyWidth = 128, kTinyWeightBytes = 48 * 1024;
static_assert(kTinyWidth == kKPad, "one Kpad for every layer of a tiny program");
struct TinyLayer {
  const int8_t* w = nullptr;
  const float* bias = nullptr;
  uint32_t* slot = nullptr;
  int32_t in_f = 0, out_f = 0, kpad = 0, act = 0;
  float act_param = 0.0f, w_scale = 1.0f;
};
struct TinyChain {
  TinyLayer l[kTinyMaxLayers];
  int32_t n = 0, rows = 0;
};
void launch_mlp_tiny(const float* x, float* y, const TinyChain& ch, SlotClear clear, hipStream_t s);
void launch_gemm_narrow_f16(const uint16_t* A, const uint16_t* B, int64_t M, int64_t N, int64_t Kpad_h,
                            const Epilogue& ep, hipStream_t s);
void launch_gemm_narrow_f32(const float* A, const float* B, int64_t M, int64_t N, int64_t Kpad_f, const Epilogue& ep,
                            hipStream_t s);
// INT8 GEMV for M <= 8 rows: the matrix-core form (row blocks of 16
// weights streamed through LDS) where gemv_mfma_supported, else the dot4
// form.  kGmvBlocks: most 16-row blocks one workgroup of the matrix-core
// form keeps accumulators for; kGmvMinRows: fewest rows it is used for.
constexpr int kGmvBlocks = 8;
constexpr int kGmvMinRows = 2;
bool gemv_mfma_supported(int64_t M, int64_t Npad, int64_t Kpad);
// One-row INT8 GEMV reading its f32 input x [K] and quantizing it itself:
// with the scale of the spread slot ep.absmax_in (a producer raised it) or,
// with self_absmax, from x's own absmax (then it also takes the run's slot
// clearing).  q_out [Kpad] / scale_out (nullable): capture taps.
constexpr int kGemvXqMaxK = 8192;  // the row a workgroup holds in registers (8 float4 per thread)
bool gemv_xq_supported(int64_t M, int64_t K, int64_t Kpad, const void* x);
void launch_gemv_xq(const float* x, const int8_t* B, int64_t N, int64_t Npad, int64_t K, int64_t Kpad,
                    const Epilogue& ep, bool self_absmax, int8_t* q_out, float* scale_out, const SlotClear& clear,
                    hipStream_t s);
void launch_gemv(const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t Npad,
                 int64_t Kpad, const Epilogue& ep, hipStream_t s);

// Implicit-GEMM conv: per image b, y[b,o,l] = act(sum_kk W[o,kk]*im2col(xq_b)[kk,l]
// * (sa_b*sw) + bias[o]).  xq is i8 NCHW.  On the device W is [Opad, Kpad] in
// tap-major order, kk' = (ki*k + kj)*cp + c with the channels padded to cp
// (4 when C <= 4, else a multiple of 16) and zero weights for c >= C: the i32
// sums do not depend on the order of the K terms, and this order makes the
// im2col operand of one tap a contiguous run of channels.
struct ConvShape {
  int64_t n, C, H, W, O, Opad, k, stride, pad, OH, OW, Kpad, cp;
};
inline int64_t conv_cp(int64_t C) { return C <= 4 ? 4 : round_up(C, 16); }
inline int64_t conv_kpad(int64_t C, int64_t k) { return round_up(k * k * conv_cp(C), 64); }
// Two INT8 conv + MaxPool2d(2, 2) stages in one launch, one workgroup per
// image (kernels.hip conv_pool_pair_kernel): conv A on 32 x 32 images with
// at most 4 channels -> 32, 3 x 3, stride 1, pad 1, then conv B 32 -> 64 with
// the same window, each with ReLU or no activation.  The first conv measures
// its image's absmax itself and writes its key to ea.absmax_in[b]; conv B's
// per-image absmax (over the pooled conv A output) goes to eb.absmax_in[b];
// the pooled conv B output goes to eb.y and its absmax to eb.absmax_out.
bool conv_pool_pair_supported(const ConvShape& a, const ConvShape& b);
void launch_conv_pool_pair(const float* x, const int8_t* WA, const int8_t* WB, const ConvShape& a, const ConvShape& b,
                           const Epilogue& ea, const Epilogue& eb, SlotClear clear, hipStream_t s);
void launch_conv(const int8_t* xq, const int8_t* Wq, const ConvShape& cs, const Epilogue& ep,
                 hipStream_t s);
// The same conv reading the f32 image and quantizing its band in LDS with
// the image's scale (ep.absmax_in, one slot per image); false when the
// band does not fit in LDS (then quantize the image and use launch_conv).
// With self_absmax (conv_self_absmax_supported: small, fully covered
// images) the kernel measures each image's absmax itself, publishes it in
// ep.absmax_in, and zeroes `clear` (the run's first kernel).  With
// ep.pool2 (see Epilogue) it also returns false when no tile width fits
// the pool; then launch it without.
bool conv_self_absmax_supported(const ConvShape& cs);
// Whether launch_conv_f32in can pool 2 x 2 in its epilogue (ep.pool2 = r16 =
// OW / 16): some tile width it tries holds whole pairs of output rows per
// wave and fits in LDS.
bool conv_pool_supported(const ConvShape& cs, int r16);
bool launch_conv_f32in(const float* x, const int8_t* Wq, const ConvShape& cs, const Epilogue& ep, hipStream_t s,
                       bool self_absmax = false, SlotClear clear = SlotClear{});

// ---- NpuPrecision::Fp16 ----------------------------------------------------
// GEMM on IEEE binary16 operands (A [Mpad, Kpad_h], B [Npad, Kpad_h], Kpad_h a
// multiple of 32), f32 accumulation, epilogue y = act(round_fp16(acc + bias))
// (npu.rs:433-445).  Same tile choice and split-K workspace as launch_gemm
// with Kpad = 2 * Kpad_h bytes.
void launch_gemm_f16(const uint16_t* A, const uint16_t* B, int64_t M, int64_t N, int64_t Mpad, int64_t Npad,
                     int64_t Kpad_h, const Epilogue& ep, int32_t* ws, int64_t ws_bytes, hipStream_t s);
// GEMV for M <= 8 on binary16 operands (A [M, Kpad_h]), same epilogue.
void launch_gemv_f16(const uint16_t* A, const uint16_t* B, int64_t M, int64_t N, int64_t Npad, int64_t Kpad_h,
                     const Epilogue& ep, hipStream_t s);
// x f32 [M, K] -> binary16 round_fp16(x) [Mpad, Kpad_h], zero padded.
void launch_half_rows(const float* x, int64_t M, int64_t K, int64_t Mpad, int64_t Kpad_h, uint16_t* h,
                      hipStream_t s);
// im2col of an NCHW batch in binary16: [Mpad >= n*L, Kpad_h >= C*k*k], reference column order.
void launch_im2col_half(const float* x, const ConvShape& cs, int64_t Mpad, int64_t Kpad_h, uint16_t* h,
                        hipStream_t s);
// [n*L, O] -> NCHW [n, O, L].
void launch_nlo_to_nchw(const float* ylo, int64_t n, int64_t O, int64_t L, float* y, hipStream_t s);
// Direct convolution (FP16 / FP32) for windows of at most kDirectConvTaps
// values and at most 64 output channels: taps summed serially in im2col
// order; w is [O, Kpad] (binary16 or f32), y NCHW.  With pool_ow = OW
// (16 or 32; OH even; ReLU or no activation): y is the output of the
// MaxPool2d(2, 2) that follows, [n, O, OH/2, OW/2]; 0 = no pool.  FP32 has
// no activation of its own: pool_act is that of the Act op between the conv
// and the pool.
constexpr int64_t kDirectConvTaps = 32;
void launch_conv_direct_f16(const float* x, const uint16_t* w, const float* bias, float* y, const ConvShape& cs,
                            int act, float act_param, int pool_ow, hipStream_t s);
void launch_conv_direct_f32(const float* x, const float* w, const float* bias, float* y, const ConvShape& cs,
                            int pool_act, int pool_ow, hipStream_t s);
// Lone ChannelAffine: y = round_fp16(fl(round_fp16(x) * scale[c]) + shift[c]), c = index % C.
void launch_affine_f16(const float* x, int64_t n, int64_t C, const float* scale, const float* shift, float* y,
                       hipStream_t s);

// ---- Standard FP32 path (ExecutionProvider::Gpu, run_standard) ------------
// f32 MFMA GEMM (v_mfma_f32_16x16x4_f32: full f32 products and sums, no
// reduced-precision inputs), epilogue y = act(acc + bias); A [Mpad, Kpad_f],
// B [Npad, Kpad_f], Kpad_f a multiple of 16 (one 64-byte K step).
void launch_gemm_f32(const float* A, const float* B, int64_t M, int64_t N, int64_t Mpad, int64_t Npad,
                     int64_t Kpad_f, const Epilogue& ep, int32_t* ws, int64_t ws_bytes, hipStream_t s);
void launch_gemv_f32(const float* A, const float* B, int64_t M, int64_t N, int64_t Npad, int64_t Kpad_f,
                     const Epilogue& ep, hipStream_t s);
void launch_pad_rows_f32(const float* x, int64_t M, int64_t K, int64_t Mpad, int64_t Kpad_f, float* a,
                         hipStream_t s);
void launch_im2col_f32(const float* x, const ConvShape& cs, int64_t Mpad, int64_t Kpad_f, float* a, hipStream_t s);
// y = x * scale[ch] + shift[ch] with ch = (index / inner) % C.
void launch_channel_affine(const float* x, int64_t n, int64_t C, int64_t inner, const float* scale,
                           const float* shift, float* y, hipStream_t s);

// Max pool (kernels.rs:165-213 semantics) with optional absmax of the output.
void launch_maxpool(const float* x, float* y, int64_t n, int64_t C, int64_t H, int64_t W,
                    int64_t k, int64_t stride, int64_t OH, int64_t OW, uint32_t* absmax_out,
                    int absmax_per_image, hipStream_t s);

// Standalone activation (in place allowed) with optional per-tensor absmax.
void launch_activation(const float* x, float* y, int64_t n, int act, float p, uint32_t* absmax_out,
                       hipStream_t s);

// Row softmax (tensor/ops.rs:1058-1076), sequential per row.
void launch_softmax(const float* x, float* y, int64_t outer, int64_t size, hipStream_t s);

}  // namespace rgnpu
