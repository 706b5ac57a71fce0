/*
 * rgnpu.h — C ABI of the MI355X-native INT8 execution provider for
 * RustGears' InferenceSession (elandice/RustGears).
 *
 * The reference dispatches inference through Rust enums, not an FFI:
 *   ExecutionProvider / CompiledProgram   src/inference/mod.rs:104-111, 140-143
 *   InferenceSession::from_layers          src/inference/mod.rs:162-180
 *     -> npu::compile(&[LayerSpec], NpuPrecision) -> NpuProgram   src/inference/npu.rs:188
 *   InferenceSession::run                   src/inference/mod.rs:212-221
 *     -> NpuProgram::execute(&Tensor) -> (Tensor, NpuProfile)     src/inference/npu.rs:296
 * Each function below replaces one of those calls for a new provider
 * variant (ExecutionProvider::Mi355x(NpuPrecision)), bound from Rust by an
 * extern "C" block.  All functions are thread-safe: rgnpu_program_run calls
 * from several threads on one program run side by side on worker streams;
 * the other calls on one program are serialized on that program's HIP stream.
 * No function panics or throws across the ABI; failures return a nonzero
 * status and set a thread-local message readable with rgnpu_last_error().
 */
#ifndef RGNPU_H
#define RGNPU_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------- */
enum {
  RGNPU_OK = 0,
  RGNPU_ERR_INVALID = 1,     /* bad argument / layer spec */
  RGNPU_ERR_SHAPE = 2,       /* input shape the reference would panic on */
  RGNPU_ERR_DEVICE = 3,      /* HIP runtime failure */
  RGNPU_ERR_UNSUPPORTED = 4, /* precision or feature not provided */
  RGNPU_ERR_IO = 5,          /* RTIM file I/O */
  RGNPU_ERR_FORMAT = 6,      /* RTIM InvalidData (bad magic, unknown tag) */
  RGNPU_ERR_CAPACITY = 7     /* caller buffer too small */
};

/* ---- layer IR: LayerSpec (src/inference/mod.rs:71-100) ------------------ */
enum {
  RGNPU_LAYER_LINEAR = 1, RGNPU_LAYER_CONV2D = 2, RGNPU_LAYER_CHANNEL_AFFINE = 3,
  RGNPU_LAYER_MAXPOOL2D = 4, RGNPU_LAYER_FLATTEN = 5, RGNPU_LAYER_ACTIVATION = 6,
  RGNPU_LAYER_SOFTMAX = 7
};
/* Activation codes = RTIM codes (src/save.rs:201-208).  RGNPU_ACT_SILU is an
 * extension: the reference has no SiLU in its inference IR
 * (src/inference/mod.rs:26-33); it computes x * sigmoid(x) as nn::Silu does
 * (src/nn/layers.rs:341-343). */
enum {
  RGNPU_ACT_NONE = 0, RGNPU_ACT_RELU = 1, RGNPU_ACT_SIGMOID = 2, RGNPU_ACT_TANH = 3,
  RGNPU_ACT_GELU = 4, RGNPU_ACT_LEAKY_RELU = 5, RGNPU_ACT_SILU = 6
};
/* NpuPrecision (src/inference/npu.rs:25-30), plus RGNPU_PRECISION_FP32: the
 * standard FP32 path of ExecutionProvider::Cpu / Gpu(i) (run_standard,
 * src/inference/mod.rs:260-331) on the MI355X, replacing the wgpu matmul
 * (src/device/gpu/wgpu_impl.rs:7-50). */
enum { RGNPU_PRECISION_INT8 = 0, RGNPU_PRECISION_FP16 = 1, RGNPU_PRECISION_FP32 = 2 };

/* One LayerSpec.  Weight layouts are exactly as Module::export produces
 * them: Linear weight [in_features, out_features] row-major
 * (src/nn/layers.rs:74-81), Conv2d weight [out, in, k, k]
 * (src/nn/layers.rs:151-161).  Fields a kind does not use are ignored.
 * The size fields are 64-bit so that every u32 an .rtim file holds reads
 * back unchanged, as the reference's `usize` fields do (src/save.rs:233-255).
 * A ChannelAffine's scale and shift carry their own lengths: the reference
 * loads them as two independent vectors (src/save.rs:254) and indexes shift
 * only below scale.len() (src/inference/mod.rs:236-237, 246, 302). */
typedef struct rgnpu_layer {
  int32_t kind;
  int32_t act; float act_param;                                /* Activation */
  int64_t in_features, out_features;                           /* Linear */
  int64_t in_channels, out_channels, kernel, stride, padding;  /* Conv2d */
  int64_t pool_kernel, pool_stride;                            /* MaxPool2d */
  const float* weight; int64_t weight_len;
  const float* bias; int64_t bias_len;
  const float* scale; int64_t scale_len;                       /* ChannelAffine */
  const float* shift; int64_t shift_len;
} rgnpu_layer;

typedef struct rgnpu_program rgnpu_program;

/* OpRecord (src/inference/npu.rs:109-116).  ns is device time from HIP
 * events around the op's kernels; kernel_ns brackets the op's main kernel
 * (GEMM / GEMV / conv / pool) only. */
typedef struct rgnpu_op_record {
  char op[96];
  uint64_t macs;
  uint64_t ns;
  uint64_t kernel_ns;
} rgnpu_op_record;

/* NpuProfile (src/inference/npu.rs:120-176). */
typedef struct rgnpu_profile {
  int32_t precision;
  int32_t original_layers;
  int32_t fused_ops;
  int32_t n_records;
  uint64_t fp32_weight_bytes;
  uint64_t npu_weight_bytes;
  uint64_t total_macs;
  uint64_t total_ns;
} rgnpu_profile;

/* Compile a layer list (fold_batch_norm, Linear/Conv2d+Activation fusion,
 * per-tensor i8 weight quantization, or round_fp16 weights for
 * RGNPU_PRECISION_FP16) and upload the weights to `device`.  Replaces
 * npu::compile (src/inference/npu.rs:188-276) as called from
 * InferenceSession::from_layers (src/inference/mod.rs:172).  INT8 results
 * are bit-exact with the reference; FP16 sums in a different order than the
 * reference's serial f32 loop (npu.rs:433-445), so its results agree within
 * that reordering (see the test suite's bound), and an activation or weight
 * whose round_fp16 value is +-65536 (inputs in [65520, 65536)) saturates to
 * +-65504, the largest binary16 value.  A Linear layer may have at most
 * 2^26 output features (RGNPU_ERR_INVALID above that; the reference has no
 * such limit), and every size field at most 2^31 - 1.  A ChannelAffine whose
 * shift is shorter than its scale gives RGNPU_ERR_INVALID (the reference
 * indexes shift[c] for every channel and panics); a longer shift is used up
 * to the scale's length, as the reference does. */
int rgnpu_program_create(const rgnpu_layer* layers, int64_t n_layers, int32_t precision,
                         int32_t device, rgnpu_program** out);

/* Run on host buffers: x is contiguous f32 with `shape[ndim]` (row-major /
 * NCHW).  The output (f32) is written to y (capacity y_cap elements) and its
 * shape to y_shape / y_ndim.  With y == NULL only the output shape is
 * computed.  Replaces NpuProgram::execute (src/inference/npu.rs:296-421) as
 * called by InferenceSession::run (src/inference/mod.rs:212-221); the
 * profile of the call is kept as last_npu_profile (mod.rs:193-195).
 * Thread-safe like the reference's run(&self) on a Sync session: concurrent
 * calls on one program each borrow a worker context (own stream and
 * activation buffers, shared weights; at most 8, further callers wait), so
 * their copies and kernels overlap and their results do not depend on the
 * interleaving.  The last call to finish sets the profile.  In capture mode
 * calls run one at a time on the program's own stream. */
int rgnpu_program_run(rgnpu_program* prog, const float* x, const int64_t* shape, int32_t ndim,
                      float* y, int64_t y_cap, int64_t* y_shape, int32_t* y_ndim);

/* Same on device buffers (d_x, d_y allocated on the program's device).  The
 * work is enqueued on the program's stream; call rgnpu_program_synchronize
 * before reading d_y from another stream or the host.  No counterpart in the
 * reference (its tensors live on the host); used for device-resident
 * throughput measurement. */
int rgnpu_program_run_device(rgnpu_program* prog, const float* d_x, const int64_t* shape, int32_t ndim,
                             float* d_y, int64_t y_cap, int64_t* y_shape, int32_t* y_ndim);
int rgnpu_program_synchronize(rgnpu_program* prog);

/* Allocation-free variant of rgnpu_program_run_device, with the same
 * arguments and results.  No counterpart in the reference: it is for callers
 * that cannot allocate device memory (serving loops and harnesses that forbid
 * hipMalloc).  It allocates no device memory but is not capture-safe: every
 * call uploads the conv programs' coverage masks from host memory the plan
 * owns, and a new input shape synchronizes the stream.  The call makes no hipMalloc or
 * hipFree: every intermediate buffer of the run (activations between ops,
 * the i8 / binary16 GEMM operands, absmax slots, scales, conv coverage
 * masks, split-K partial sums) is a view into one device array of
 * RGNPU_NOALLOC_SCRATCH_BYTES per GPU, which the library looks up when a
 * program is created on that GPU and keeps until the process ends.  A shape
 * whose buffers do not fit gives RGNPU_ERR_CAPACITY (nothing is enqueued);
 * capture mode gives RGNPU_ERR_INVALID.  Every call on a GPU shares that GPU's
 * array and finds the previous call's contents (each call clears what must
 * start at zero), so calls whose device work overlaps on one GPU race:
 * calls on one program are ordered by its stream, calls on different
 * programs must be ordered by the caller.  The call records no profile
 * (last_npu_profile is unchanged).  Host-side bookkeeping for a new input
 * shape (the plan) uses the host heap. */
#define RGNPU_NOALLOC_SCRATCH_BYTES (64ll << 20)
int rgnpu_program_run_device_noalloc(rgnpu_program* prog, const float* d_x, const int64_t* shape, int32_t ndim,
                                     float* d_y, int64_t y_cap, int64_t* y_shape, int32_t* y_ndim);

/* Throughput measurement on device buffers: enqueues `iters` runs back to
 * back on the program's stream, bracketed by two HIP events, waits, and
 * returns the elapsed device time.  `flags`:
 *  - 0: the runs record no events of their own;
 *  - RGNPU_BENCH_KERNEL_EVENTS: each run also records a start and an end
 *    marker, every kernel of every run records the completion timestamp of
 *    its own dispatch (no marker packet per kernel), and avg[i] receives op
 *    i's mean op time (ns, from the previous kernel's completion to its last
 *    kernel's) and main-kernel time (kernel_ns) over the iterations;
 *  - RGNPU_BENCH_EVICT_CACHE (with or without the above): before each run a
 *    kernel reads 512 MiB of a zero buffer, so the run finds none of its own
 *    data in the 256 MB memory-side cache.  That read is outside every op
 *    interval but inside total_ms.
 * No counterpart in the reference; this is the bench harness's timed region. */
#define RGNPU_BENCH_KERNEL_EVENTS 1
#define RGNPU_BENCH_EVICT_CACHE 2
int rgnpu_program_benchmark(rgnpu_program* prog, const float* d_x, const int64_t* shape, int32_t ndim, float* d_y,
                            int64_t y_cap, int32_t iters, int32_t flags, double* total_ms,
                            rgnpu_op_record* avg, int32_t cap);

/* Profiling level: 0 = total time only, 1 = per-op and per-kernel HIP events.
 * Default 1 (the reference always records per-op durations, npu.rs:303-407). */
int rgnpu_program_set_profiling(rgnpu_program* prog, int32_t level);

/* last_npu_profile (src/inference/mod.rs:193-195): header plus up to `cap`
 * op records of the most recent run. */
int rgnpu_program_profile(rgnpu_program* prog, rgnpu_profile* out, rgnpu_op_record* records, int32_t cap);

/* compilation_report (src/inference/mod.rs:198-209) -> NpuProgram::summary
 * (src/inference/npu.rs:280-293).  Returns the string length; writes at most
 * cap-1 bytes plus a terminating NUL. */
int64_t rgnpu_program_summary(const rgnpu_program* prog, char* buf, int64_t cap);

/* Number of fused ops and the label of op i (NpuOp::label, npu.rs:83-104). */
int64_t rgnpu_program_num_ops(const rgnpu_program* prog);
int64_t rgnpu_program_op_label(const rgnpu_program* prog, int64_t i, char* buf, int64_t cap);

/* Quantized weight of op i as the reference holds it (QuantTensor of
 * weight_q_t [out,in] or weight_q [out, c*k*k], npu.rs:208-209, 231):
 * copies up to cap bytes, returns the element count, writes the scale. */
int64_t rgnpu_program_op_weight(const rgnpu_program* prog, int64_t i, int8_t* dst, int64_t cap, float* scale);

/* Capture taps for bit-exactness checks (no counterpart in the reference,
 * which fuses these values away, quantize.rs:109-111).
 *  - RGNPU_CAPTURE_FULL: the next runs use the capture forms of the kernels
 *    (every value stored) and keep per op: the i8 activations the GEMM
 *    consumed (Linear [rows,in]; Conv2d [n, L, C*k*k] = transposed im2col
 *    per image), the activation scale(s) (1 or n f32), the i32 accumulators
 *    (Linear [rows,out]; Conv2d [n, L, out]) and the op's f32 output.
 *  - RGNPU_CAPTURE_PRODUCTION: the next runs use the production plan and
 *    kernels unchanged (fused requantization with the certified GELU,
 *    conv + pool fusion, operand hand-offs); after each op its i8 operand,
 *    absmax slot and f32 output are copied device to device where they exist
 *    in memory: the i8 activations of a Linear whose operand buffer was
 *    written (not for the GEMMs that quantize as they read, nor for convs,
 *    which quantize into LDS), the scale(s) from the absmax the consumer
 *    read (none for a one-row GEMV that measures its own input's absmax in
 *    registers), and the f32 output of ops that store theirs (not of a GEMM that
 *    writes the next op's operand instead, nor of a conv that pools in its
 *    epilogue: the MaxPool2d op then shows the pooled output).  The i32
 *    accumulators are never available; what is not available reads as 0
 *    elements.
 * rgnpu_program_capture copies up to cap_bytes into dst and returns the
 * element count (dst may be NULL). */
enum { RGNPU_CAP_QACT = 0, RGNPU_CAP_SCALE = 1, RGNPU_CAP_ACC = 2, RGNPU_CAP_OUT = 3 };
enum { RGNPU_CAPTURE_OFF = 0, RGNPU_CAPTURE_FULL = 1, RGNPU_CAPTURE_PRODUCTION = 2 };
int rgnpu_program_set_capture(rgnpu_program* prog, int32_t mode);
int64_t rgnpu_program_capture(rgnpu_program* prog, int64_t op, int32_t what, void* dst, int64_t cap_bytes);

void rgnpu_program_destroy(rgnpu_program* prog);

/* Thread-local message of the last failing call on this thread. */
const char* rgnpu_last_error(void);

/* ---- RTIM (src/save.rs:165-279) ----------------------------------------- */
/* Reads an .rtim file (load_inference_layers, src/save.rs:227-279).  The
 * returned layers and their arrays are owned by *out_handle; free with
 * rgnpu_rtim_free.  Bad magic / unknown tags give RGNPU_ERR_FORMAT
 * (io::ErrorKind::InvalidData), truncation RGNPU_ERR_IO. */
typedef struct rgnpu_rtim rgnpu_rtim;
int rgnpu_rtim_load(const char* path, rgnpu_rtim** out_handle, const rgnpu_layer** layers, int64_t* n_layers);
void rgnpu_rtim_free(rgnpu_rtim* handle);
/* Writes layers as .rtim (save_layers, src/save.rs:172-224), atomically
 * (temporary file in the same directory, then rename; src/save.rs:21-32). */
int rgnpu_rtim_save(const char* path, const rgnpu_layer* layers, int64_t n_layers);

/* ---- seeded synthetic data (src/rng.rs:10-98) ----------------------------- */
/* SplitMix64 generator with the reference's global-seed semantics, used to
 * build the reference's seeded weights and inputs (Tensor::rand/uniform/randn,
 * src/tensor/mod.rs:116-131) without a Rust toolchain. */
void rgnpu_manual_seed(uint64_t seed);
void rgnpu_fill_uniform(float* out, int64_t n);                          /* Tensor::rand */
void rgnpu_fill_uniform_range(float* out, int64_t n, float lo, float hi); /* Tensor::uniform */
void rgnpu_fill_normal(float* out, int64_t n);                           /* Tensor::randn */

/* ---- device buffers for callers without their own allocator -------------- */
/* Sustained i8 MFMA rate of the device: one launch of a register-only loop
 * of independent v_mfma_i32_16x16x64_i8 (8 waves per CU, `iters` rounds of
 * 32 per wave, no memory traffic in the loop) on random or all-zero operand
 * bytes, timed with HIP events.  Writes the elapsed ms and the rate in
 * TOPS (2 ops per MAC).  No counterpart in the reference: it measures the
 * ceiling that the GEMM kernels' MFMA utilization is compared against. */
int rgnpu_probe_mfma_rate(int32_t device, int64_t iters, int32_t random_operands, double* ms, double* tops);

/* Cost of one poll of the persistent grids' barrier (one s_sleep of 512
 * clocks and one agent-scope atomic load of a 128-byte line): thread 0 of
 * each of `blocks` workgroups polls a line of its own that is never set,
 * `polls` times, in one launch timed with HIP events.  No counterpart in the
 * reference: it states in microseconds the barrier's wait bound
 * (RGNPU_REQUANT_SPIN_LIMIT polls, default 100000). */
int rgnpu_probe_barrier_poll(int32_t device, int32_t blocks, int32_t polls, double* us_per_poll);

/* Cumulative counters of the persistent grids' barriers (the fused
 * requantization and the one-pass input quantization) over a program's
 * handle and its idle workers since creation: workgroups that gave up
 * waiting and deferred their quantization to the finisher (correct results,
 * later), workgroups a finisher found unsettled (their outputs were not
 * quantized; the synchronizing call of that run -- rgnpu_program_run,
 * rgnpu_program_synchronize, rgnpu_program_benchmark -- returns
 * RGNPU_ERR_DEVICE), and finished barrier launches.  Synchronizes the
 * streams it reads.  No counterpart in the reference; a diagnostic for
 * concurrent runs. */
int rgnpu_program_barrier_stats(rgnpu_program* prog, uint64_t* deferred, uint64_t* unsettled, uint64_t* launches);

int rgnpu_device_count(int32_t* count);
int rgnpu_device_alloc(int32_t device, int64_t bytes, void** out);
int rgnpu_device_free(void* p);
int rgnpu_memcpy_h2d(void* dst, const void* src, int64_t bytes);
int rgnpu_memcpy_d2h(void* dst, const void* src, int64_t bytes);
int rgnpu_device_synchronize(void);

#ifdef __cplusplus
}
#endif
#endif /* RGNPU_H */
