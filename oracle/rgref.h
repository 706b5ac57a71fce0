/*
 * rgref — CPU oracle for the RustGears NPU inference path (INT8 and FP16).
 *
 * TEST INFRASTRUCTURE ONLY.  This is a plain-C restatement of the reference
 * Rust code (elandice/RustGears) for `InferenceSession` with
 * `ExecutionProvider::Npu(NpuPrecision::Int8)` and `::Fp16`.  It exists to check the HIP
 * execution provider and to time the reference algorithm on host cores.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it; the product library never links or calls it.
 *
 * Every function cites the reference file:line it restates.  Arithmetic
 * follows Rust semantics: strict left-to-right f32 evaluation without FMA
 * contraction (build with -ffp-contract=off), f32::max ignores NaN (fmaxf),
 * f32::round is half-away-from-zero (roundf), `as i8` saturates with NaN -> 0,
 * and f32::{exp,tanh,ln,cos} are the host libm expf/tanhf/logf/cosf.
 *
 * Parity pins (see tests/test_oracle.py): SplitMix64 published vector,
 * closed forms for uniform/quantize/epilogue, brute-force integer GEMM,
 * im2col/max-pool/transpose brute force, the reference's own structural
 * test (integration.rs:127-164) and USAGE.md:377-381 pipeline example.
 *
 * Parity unpinned at the bit level: the GELU, Sigmoid, Tanh and SiLU values
 * of rgref_act_apply.  They call the host glibc tanhf/expf, as the Rust
 * reference does, but nothing the reference ships fixes their bits; the
 * tests pin the formulas to <= 2e-6 relative against double precision only.
 */
#ifndef RGREF_H
#define RGREF_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- layer IR: mirrors LayerSpec (src/inference/mod.rs:71-100) ---------- */
enum {
  RGREF_LINEAR = 1, RGREF_CONV2D = 2, RGREF_CHANNEL_AFFINE = 3,
  RGREF_MAXPOOL2D = 4, RGREF_FLATTEN = 5, RGREF_ACTIVATION = 6,
  RGREF_SOFTMAX = 7
};
/* Activation codes follow the RTIM encoding (src/save.rs:201-208); 6 = SiLU
 * is a build extension (x * sigmoid(x), src/nn/layers.rs:341-343). */
enum { RGREF_ACT_NONE = 0, RGREF_ACT_RELU = 1, RGREF_ACT_SIGMOID = 2,
       RGREF_ACT_TANH = 3, RGREF_ACT_GELU = 4, RGREF_ACT_LEAKY_RELU = 5,
       RGREF_ACT_SILU = 6 };

typedef struct {
  int32_t kind;
  int32_t in_features, out_features;                 /* Linear */
  int32_t in_channels, out_channels, kernel, stride, padding; /* Conv2d */
  int32_t pool_kernel, pool_stride;                  /* MaxPool2d */
  int32_t act; float act_param;                      /* Activation */
  const float* weight; int64_t weight_len;           /* Linear [in,out]; Conv [out,in,k,k] */
  const float* bias;   int64_t bias_len;
  const float* scale;  const float* shift; int64_t affine_len; /* ChannelAffine */
} rgref_layer;

/* ---- rng.rs restatement --------------------------------------------------- */
typedef struct { uint64_t state; } rgref_rng;
void     rgref_rng_new(rgref_rng* r, uint64_t seed);          /* rng.rs:16-18 */
uint64_t rgref_rng_next_u64(rgref_rng* r);                    /* rng.rs:21-27 */
float    rgref_rng_uniform(rgref_rng* r);                     /* rng.rs:30-32 */
float    rgref_rng_uniform_range(rgref_rng* r, float lo, float hi); /* rng.rs:35-37 */
float    rgref_rng_normal(rgref_rng* r);                      /* rng.rs:40-44 */
void     rgref_manual_seed(uint64_t seed);                    /* rng.rs:71-73 */
void     rgref_fill_uniform(float* out, int64_t n);           /* Tensor::rand, tensor/mod.rs:122-125 */
void     rgref_fill_uniform_range(float* out, int64_t n, float lo, float hi); /* Tensor::uniform :128-131 */
void     rgref_fill_normal(float* out, int64_t n);            /* Tensor::randn :116-119 */

/* ---- elementwise / primitives ---------------------------------------------- */
float rgref_act_apply(int act, float param, float x);         /* mod.rs:37-53, backend.rs:66-78 */
void  rgref_act_apply_array(int act, float param, const float* x, float* y, int64_t n);
float rgref_quantize(const float* v, int64_t n, int8_t* out); /* quantize.rs:18-35, returns scale */
int32_t rgref_dot_i8(const int8_t* a, const int8_t* b, int64_t len); /* quantize.rs:68-88 */
/* quantize.rs:93-144; acc_out (nullable) receives the i32 accumulators. */
void rgref_int8_gemm_fused(const int8_t* a, float a_scale, const int8_t* b_t, float b_scale,
                           int64_t m, int64_t k, int64_t n, const float* bias,
                           int act, float act_param, float* out, int32_t* acc_out, int parallel);
int64_t rgref_out_size(int64_t input, int64_t kernel, int64_t stride, int64_t pad); /* kernels.rs:10-15 */
void rgref_im2col(const float* x, int64_t c, int64_t h, int64_t w, int64_t k, int64_t stride,
                  int64_t pad, int64_t oh, int64_t ow, float* cols);          /* kernels.rs:28-96 */
void rgref_transpose2d(const float* data, int64_t rows, int64_t cols, float* out); /* shape.rs:105-123 */
void rgref_max_pool2d(const float* x, int64_t n, int64_t c, int64_t h, int64_t w,
                      int64_t k, int64_t stride, float* out, int parallel); /* kernels.rs:165-213 */
void rgref_softmax_rows(const float* x, int64_t outer, int64_t size, float* y); /* ops.rs:1058-1076 */

/* ---- compile / execute (npu.rs:188-276, 296-421) --------------------------- */
typedef struct rgref_program rgref_program;
enum { RGREF_INT8 = 0, RGREF_FP16 = 1, RGREF_FP32 = 2 }; /* NpuPrecision (npu.rs:25-30); FP32 = run_standard (mod.rs:260-331) */
void rgref_matmul_f32(const float* a, const float* b, int64_t m, int64_t k, int64_t n, float* c, int parallel);
float rgref_round_fp16(float x);                              /* quantize.rs:50-64 */
void rgref_round_fp16_array(const float* x, float* y, int64_t n);
void rgref_fp16_gemm_fused(const float* a, const float* b_t, int64_t m, int64_t k, int64_t n,
                           const float* bias, int act, float p, float* out, int parallel); /* npu.rs:433-445 */
rgref_program* rgref_compile(const rgref_layer* layers, int64_t n_layers); /* INT8 */
rgref_program* rgref_compile_precision(const rgref_layer* layers, int64_t n_layers, int precision);
/* FP16 weights of op i ([out, K] row-major, as round_fp16'd by compile); 0 when none. */
int64_t rgref_program_op_weight_fp16(const rgref_program* p, int64_t i, const float** w, int64_t* rows);
void    rgref_program_free(rgref_program* p);
int64_t rgref_program_num_ops(const rgref_program* p);
int64_t rgref_program_fp32_bytes(const rgref_program* p);
int64_t rgref_program_npu_bytes(const rgref_program* p);
int64_t rgref_program_original_layers(const rgref_program* p);
/* Writes the op label (npu.rs:83-104) of op i into buf; returns its length. */
int64_t rgref_program_op_label(const rgref_program* p, int64_t i, char* buf, int64_t cap);
/* Quantized weight of op i ([out, in] or [out, c*k*k]) and its scale. */
int64_t rgref_program_op_weight(const rgref_program* p, int64_t i, const int8_t** w, float* scale,
                                const float** bias);

/* Capture taps: per op, the quantized activations fed to the GEMM
 * (Linear [rows,in]; Conv2d [n,L,ckk] = transposed im2col per image), the
 * activation scale(s) (1 or n), the i32 accumulators (Linear [rows,out];
 * Conv2d [n,L,out]) and the op's f32 output. */
enum { RGREF_CAP_QACT = 0, RGREF_CAP_SCALE = 1, RGREF_CAP_ACC = 2, RGREF_CAP_OUT = 3 };
void    rgref_program_set_capture(rgref_program* p, int on);
int64_t rgref_program_capture(const rgref_program* p, int64_t op, int what, const void** data);

/* Runs the program on x (shape[ndim]).  On success returns 0 and the output
 * is available through rgref_program_output.  Returns nonzero (and sets an
 * error string) on shapes the reference would panic on. */
int rgref_execute(rgref_program* p, const float* x, const int64_t* shape, int ndim, int parallel);
int64_t rgref_program_output(const rgref_program* p, const float** y, int64_t* shape, int* ndim);
int64_t rgref_program_op_macs(const rgref_program* p, int64_t i);
int64_t rgref_program_total_macs(const rgref_program* p);
const char* rgref_last_error(void);

/* Parallel region width used when `parallel` is nonzero (OpenMP). */
void rgref_set_threads(int n);
int  rgref_get_threads(void);

#ifdef __cplusplus
}
#endif
#endif
