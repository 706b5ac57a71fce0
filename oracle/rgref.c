/*
 * rgref.c — CPU oracle (test infrastructure only) restating the RustGears
 * NPU INT8 inference path.  See rgref.h for the contract and the list of
 * parity pins.  Build: oracle/Makefile (gcc -O3 -ffp-contract=off, baseline
 * x86-64, OpenMP for the rayon-equivalent splits).
 */
#include "rgref.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static __thread char g_err[256];
static void set_err(const char* m) { snprintf(g_err, sizeof g_err, "%s", m); }
const char* rgref_last_error(void) { return g_err; }

static int g_threads = 0;
void rgref_set_threads(int n) { g_threads = n; }
int rgref_get_threads(void) {
#ifdef _OPENMP
  return g_threads > 0 ? g_threads : omp_get_max_threads();
#else
  return 1;
#endif
}

/* ======================= rng.rs:10-98 ===================================== */
#define GOLDEN 0x9E3779B97F4A7C15ull
void rgref_rng_new(rgref_rng* r, uint64_t seed) { r->state = seed ^ GOLDEN; } /* rng.rs:16-18 */
uint64_t rgref_rng_next_u64(rgref_rng* r) {                                 /* rng.rs:21-27 */
  r->state += GOLDEN;
  uint64_t z = r->state;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
float rgref_rng_uniform(rgref_rng* r) {                                     /* rng.rs:30-32 */
  return (float)(rgref_rng_next_u64(r) >> 40) / (float)(1ull << 24);
}
float rgref_rng_uniform_range(rgref_rng* r, float lo, float hi) {           /* rng.rs:35-37 */
  float d = hi - lo;
  float u = rgref_rng_uniform(r);
  float p = d * u;
  return lo + p;
}
float rgref_rng_normal(rgref_rng* r) {                                      /* rng.rs:40-44 */
  float u1 = fmaxf(rgref_rng_uniform(r), 1e-7f);
  float u2 = rgref_rng_uniform(r);
  float a = -2.0f * logf(u1);
  float s = sqrtf(a);
  float two_pi = 2.0f * 3.14159274101257324f; /* 2.0 * std::f32::consts::PI */
  float c = cosf(two_pi * u2);
  return s * c;
}
/* Global generator, default seed 0x5EED (rng.rs:61-73). */
static rgref_rng g_rng = {0x5EEDull ^ GOLDEN};
void rgref_manual_seed(uint64_t seed) { rgref_rng_new(&g_rng, seed); }
void rgref_fill_uniform(float* out, int64_t n) {
  for (int64_t i = 0; i < n; i++) out[i] = rgref_rng_uniform(&g_rng);
}
void rgref_fill_uniform_range(float* out, int64_t n, float lo, float hi) {
  for (int64_t i = 0; i < n; i++) out[i] = rgref_rng_uniform_range(&g_rng, lo, hi);
}
void rgref_fill_normal(float* out, int64_t n) {
  for (int64_t i = 0; i < n; i++) out[i] = rgref_rng_normal(&g_rng);
}

/* ======================= activations ====================================== */
/* Activation::apply (inference/mod.rs:37-53) -> UnaryOp::apply
 * (device/backend.rs:66-78); GELU_C = 0.797_884_6 (backend.rs:61). */
static float sigmoid_f(float x) { float e = expf(-x); float d = 1.0f + e; return 1.0f / d; }
/* ReLU = x.max(0.0) (backend.rs:71) as the reference's x86-64 build computes
 * it.  Rust lowers f32::max to llvm.maxnum, which leaves the sign of an
 * equal-zero result open; with a constant operand that cannot be NaN, LLVM's
 * x86 backend emits one maxss with the constant as the source operand
 * (x > 0 ? x : 0), so NaN and -0.0 both give +0.0. */
static float rust_relu(float x) { return x > 0.0f ? x : 0.0f; }
float rgref_act_apply(int act, float p, float x) {
  switch (act) {
    case RGREF_ACT_NONE: return x;
    case RGREF_ACT_RELU: return rust_relu(x);
    case RGREF_ACT_SIGMOID: return sigmoid_f(x);
    case RGREF_ACT_TANH: return tanhf(x);
    case RGREF_ACT_GELU: {
      float x3 = 0.044715f * x; x3 = x3 * x; x3 = x3 * x;
      float inner = x + x3;
      float u = 0.7978846f * inner;
      float t = tanhf(u);
      float h = 0.5f * x;
      float one_t = 1.0f + t;
      return h * one_t;
    }
    case RGREF_ACT_LEAKY_RELU: return x > 0.0f ? x : p * x;
    case RGREF_ACT_SILU: { float s = sigmoid_f(x); return x * s; } /* layers.rs:341-343 */
    default: return x;
  }
}

void rgref_act_apply_array(int act, float p, const float* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; i++) y[i] = rgref_act_apply(act, p, x[i]);
}

/* ======================= quantize.rs ====================================== */
/* QuantTensor::from_f32 / quantize_into (quantize.rs:18-35). */
static inline int8_t q_one(float v, float inv) {
  float t = roundf(v * inv);
  if (t < -127.0f) t = -127.0f;
  if (t > 127.0f) t = 127.0f;
  if (t != t) return 0; /* `as i8` maps NaN to 0 */
  return (int8_t)t;
}
float rgref_quantize(const float* v, int64_t n, int8_t* out) {
  float max_abs = 0.0f;
  for (int64_t i = 0; i < n; i++) max_abs = fmaxf(max_abs, fabsf(v[i]));
  float scale = max_abs < 1e-12f ? 1.0f : max_abs / 127.0f;
  float inv = 1.0f / scale;
  for (int64_t i = 0; i < n; i++) out[i] = q_one(v[i], inv);
  return scale;
}

/* round_fp16 (quantize.rs:50-64): keeps the top 10 mantissa bits after
 * adding half an ulp to the magnitude (ties round up, not to even),
 * flushes exponents below -14 to +0 (the sign is dropped) and clamps
 * exponents above 15 to +-65504 (NaN and +-inf included, with their sign
 * bit).  The exponent is read before rounding, so [65520, 65536) rounds to
 * 65536. */
float rgref_round_fp16(float x) {
  uint32_t bits;
  memcpy(&bits, &x, 4);
  const uint32_t sign = bits & 0x80000000u;
  const int32_t e = (int32_t)((bits >> 23) & 0xffu) - 127;
  if (e < -14) return 0.0f;
  uint32_t r = e > 15 ? (sign | 0x477fe000u) : ((bits + (1u << 12)) & ~0x1fffu);
  float y;
  memcpy(&y, &r, 4);
  return y;
}

void rgref_round_fp16_array(const float* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; i++) y[i] = rgref_round_fp16(x[i]);
}

/* dot_i8 (quantize.rs:68-88): four i32 lanes then a tail.  i32 adds wrap in
 * release Rust; the order only matters on overflow, where wrapping sums are
 * still order-independent. */
int32_t rgref_dot_i8(const int8_t* a, const int8_t* b, int64_t len) {
  uint32_t acc0 = 0, acc1 = 0, acc2 = 0, acc3 = 0;
  int64_t i = 0;
  for (; i + 4 <= len; i += 4) {
    acc0 += (uint32_t)((int32_t)a[i] * (int32_t)b[i]);
    acc1 += (uint32_t)((int32_t)a[i + 1] * (int32_t)b[i + 1]);
    acc2 += (uint32_t)((int32_t)a[i + 2] * (int32_t)b[i + 2]);
    acc3 += (uint32_t)((int32_t)a[i + 3] * (int32_t)b[i + 3]);
  }
  uint32_t total = (acc0 + acc1) + (acc2 + acc3);
  for (; i < len; i++) total += (uint32_t)((int32_t)a[i] * (int32_t)b[i]);
  return (int32_t)total;
}

static void gemm_row(const int8_t* arow, const int8_t* b_t, int64_t k, int64_t n, float cs,
                     const float* bias, int act, float p, float* orow, int32_t* accrow) {
  for (int64_t c = 0; c < n; c++) {
    int32_t acc = rgref_dot_i8(arow, b_t + c * k, k);
    if (accrow) accrow[c] = acc;
    float prod = (float)acc * cs;      /* (acc as f32) * combined_scale */
    float val = prod + bias[c];        /* + bias[c], no FMA */
    orow[c] = rgref_act_apply(act, p, val);
  }
}
/* fp16_gemm_fused_into (npu.rs:433-445): each output is a serial f32 sum,
 * k ascending, of round_fp16(a) * w (multiply then add, no FMA), then
 * act(round_fp16(acc + bias[c])).  The reference runs rows serially; rows
 * are independent, so the optional row-parallel loop gives the same bits. */
static void fp16_gemm_row(const float* arow, const float* b_t, int64_t k, int64_t n, const float* bias, int act,
                          float p, float* orow, float* ah) {
  for (int64_t j = 0; j < k; j++) ah[j] = rgref_round_fp16(arow[j]);
  for (int64_t c = 0; c < n; c++) {
    const float* brow = b_t + c * k;
    float acc = 0.0f;
    for (int64_t j = 0; j < k; j++) {
      float prod = ah[j] * brow[j];
      acc = acc + prod;
    }
    float t = acc + bias[c];
    orow[c] = rgref_act_apply(act, p, rgref_round_fp16(t));
  }
}
void rgref_fp16_gemm_fused(const float* a, const float* b_t, int64_t m, int64_t k, int64_t n, const float* bias,
                           int act, float p, float* out, int parallel) {
#pragma omp parallel for schedule(dynamic, 4) num_threads(rgref_get_threads()) if (parallel && m * k * n >= 32 * 1024)
  for (int64_t r = 0; r < m; r++) {
    float* ah = (float*)malloc(sizeof(float) * (size_t)(k > 0 ? k : 1));
    fp16_gemm_row(a + r * k, b_t, k, n, bias, act, p, out + r * n, ah);
    free(ah);
  }
}

/* int8_gemm_fused (quantize.rs:93-118) / int8_gemm_fused_serial (122-144).
 * The parallel split is over output rows when m*k*n >= 32768 (quantize.rs:104). */
void rgref_int8_gemm_fused(const int8_t* a, float a_scale, const int8_t* b_t, float b_scale,
                           int64_t m, int64_t k, int64_t n, const float* bias, int act, float p,
                           float* out, int32_t* acc_out, int parallel) {
  float cs = a_scale * b_scale;
  if (parallel && m * k * n >= 32 * 1024) {
#pragma omp parallel for schedule(dynamic, 1) num_threads(rgref_get_threads())
    for (int64_t r = 0; r < m; r++)
      gemm_row(a + r * k, b_t, k, n, cs, bias, act, p, out + r * n, acc_out ? acc_out + r * n : NULL);
  } else {
    for (int64_t r = 0; r < m; r++)
      gemm_row(a + r * k, b_t, k, n, cs, bias, act, p, out + r * n, acc_out ? acc_out + r * n : NULL);
  }
}

/* ======================= kernels.rs / shape.rs ============================ */
int64_t rgref_out_size(int64_t input, int64_t kernel, int64_t stride, int64_t pad) { /* kernels.rs:10-15 */
  if (kernel <= 0 || stride <= 0) return -1;
  int64_t padded = input + 2 * pad;
  if (padded < kernel) return -1;
  return (padded - kernel) / stride + 1;
}

/* im2col_into (kernels.rs:28-96): rows (ch*k+ki)*k+kj, columns oy*ow+ox,
 * zero padding.  Both reference branches produce the same matrix; the
 * general-stride branch is used for all strides here. */
void rgref_im2col(const float* x, int64_t c, int64_t h, int64_t w, int64_t k, int64_t stride,
                  int64_t pad, int64_t oh, int64_t ow, float* cols) {
  int64_t l = oh * ow;
  memset(cols, 0, sizeof(float) * (size_t)(c * k * k * l));
  for (int64_t ch = 0; ch < c; ch++)
    for (int64_t ki = 0; ki < k; ki++)
      for (int64_t kj = 0; kj < k; kj++) {
        int64_t base = ((ch * k + ki) * k + kj) * l;
        for (int64_t oy = 0; oy < oh; oy++) {
          int64_t iy = oy * stride + ki - pad;
          if (iy < 0 || iy >= h) continue;
          for (int64_t ox = 0; ox < ow; ox++) {
            int64_t ix = ox * stride + kj - pad;
            if (ix < 0 || ix >= w) continue;
            cols[base + oy * ow + ox] = x[(ch * h + iy) * w + ix];
          }
        }
      }
}

void rgref_transpose2d(const float* data, int64_t rows, int64_t cols, float* out) { /* shape.rs:105-123 */
  for (int64_t r = 0; r < rows; r++)
    for (int64_t c = 0; c < cols; c++) out[c * rows + r] = data[r * cols + c];
}

static void pool_plane(const float* x, int64_t plane, int64_t h, int64_t w, int64_t k, int64_t stride,
                       int64_t oh, int64_t ow, float* out_plane) {
  int64_t base = plane * h * w;
  for (int64_t oy = 0; oy < oh; oy++)
    for (int64_t ox = 0; ox < ow; ox++) {
      float best = -INFINITY;
      for (int64_t ki = 0; ki < k; ki++)
        for (int64_t kj = 0; kj < k; kj++) {
          float v = x[base + (oy * stride + ki) * w + ox * stride + kj];
          if (v > best || v != v) best = v; /* kernels.rs:187 */
        }
      out_plane[oy * ow + ox] = best;
    }
}
/* max_pool2d (kernels.rs:165-213): planes in parallel when total >= 8192. */
void rgref_max_pool2d(const float* x, int64_t n, int64_t c, int64_t h, int64_t w, int64_t k,
                      int64_t stride, float* out, int parallel) {
  int64_t oh = rgref_out_size(h, k, stride, 0), ow = rgref_out_size(w, k, stride, 0);
  int64_t l = oh * ow, planes = n * c;
  if (l <= 0) return;
  if (parallel && planes * l >= 8192) {
#pragma omp parallel for schedule(static) num_threads(rgref_get_threads())
    for (int64_t pl = 0; pl < planes; pl++) pool_plane(x, pl, h, w, k, stride, oh, ow, out + pl * l);
  } else {
    for (int64_t pl = 0; pl < planes; pl++) pool_plane(x, pl, h, w, k, stride, oh, ow, out + pl * l);
  }
}

/* softmax_raw (tensor/ops.rs:1058-1076) with inner = 1. */
void rgref_softmax_rows(const float* x, int64_t outer, int64_t size, float* y) {
  for (int64_t o = 0; o < outer; o++) {
    const float* xr = x + o * size;
    float* yr = y + o * size;
    float mx = -INFINITY;
    for (int64_t j = 0; j < size; j++) mx = fmaxf(mx, xr[j]);
    float s = 0.0f;
    for (int64_t j = 0; j < size; j++) { float e = expf(xr[j] - mx); yr[j] = e; s += e; }
    for (int64_t j = 0; j < size; j++) yr[j] = yr[j] / s;
  }
}

/* ======================= compile (npu.rs:188-276) ========================= */
typedef struct {
  int kind; /* RGREF_LINEAR (FusedLinear), RGREF_CONV2D (FusedConv2d), MAXPOOL, FLATTEN, ACTIVATION, SOFTMAX */
  int64_t in_f, out_f;              /* Linear: in/out features; Conv: in/out channels */
  int64_t kernel, stride, padding;
  int8_t* wq; float w_scale; int64_t w_len;
  float* wh;  /* FP16: round_fp16 weights [out, in] / [out, c*k*k]; the raw diagonal for a lone ChannelAffine.
                FP32 (standard path): the f32 weights as exported (Linear [in, out], Conv [out, c*k*k]) */
  float* aff_scale; int64_t aff_len; /* FP32: a ChannelAffine that did not fold (shift in bias) */
  float* bias;
  int act; float act_param;
  /* captures */
  int8_t* cap_q; int64_t cap_q_len;
  float* cap_scale; int64_t cap_scale_len;
  int32_t* cap_acc; int64_t cap_acc_len;
  float* cap_out; int64_t cap_out_len;
  int64_t macs;
} ref_op;

struct rgref_program {
  int precision; /* RGREF_INT8 or RGREF_FP16 (NpuPrecision, npu.rs:25-30) */
  ref_op* ops; int64_t n_ops;
  int64_t original_layers, fp32_bytes, npu_bytes;
  int capture;
  float* out; int64_t out_len; int64_t out_shape[8]; int out_ndim;
  int64_t total_macs;
};

typedef struct {
  int kind;
  int64_t in_f, out_f, in_c, out_c, k, s, p, pk, ps;
  int act; float act_param;
  float* w; int64_t w_len; float* b; int64_t b_len;
  float* scale; float* shift; int64_t aff_len;
} folded_layer;

static float* dupf(const float* src, int64_t n) {
  float* d = (float*)malloc(sizeof(float) * (size_t)(n > 0 ? n : 1));
  if (n > 0) memcpy(d, src, sizeof(float) * (size_t)n);
  return d;
}

/* fold_batch_norm (inference/mod.rs:225-257). */
static folded_layer* fold_batch_norm(const rgref_layer* L, int64_t n, int64_t* out_n) {
  folded_layer* out = (folded_layer*)calloc((size_t)(n > 0 ? n : 1), sizeof(folded_layer));
  int64_t m = 0;
  for (int64_t i = 0; i < n; i++) {
    const rgref_layer* l = &L[i];
    if (l->kind == RGREF_CHANNEL_AFFINE && m > 0) {
      folded_layer* last = &out[m - 1];
      if (last->kind == RGREF_LINEAR && last->out_f == l->affine_len) {
        for (int64_t r = 0; r < last->in_f; r++)
          for (int64_t c = 0; c < last->out_f; c++) last->w[r * last->out_f + c] *= l->scale[c];
        for (int64_t c = 0; c < last->out_f; c++) {
          float t = last->b[c] * l->scale[c];
          last->b[c] = t + l->shift[c];
        }
        continue;
      }
      if (last->kind == RGREF_CONV2D && last->out_c == l->affine_len) {
        int64_t plane = last->in_c * last->k * last->k;
        for (int64_t o = 0; o < last->out_c; o++) {
          for (int64_t j = 0; j < plane; j++) last->w[o * plane + j] *= l->scale[o];
          float t = last->b[o] * l->scale[o];
          last->b[o] = t + l->shift[o];
        }
        continue;
      }
    }
    folded_layer* f = &out[m++];
    f->kind = l->kind;
    f->in_f = l->in_features; f->out_f = l->out_features;
    f->in_c = l->in_channels; f->out_c = l->out_channels;
    f->k = l->kernel; f->s = l->stride; f->p = l->padding;
    f->pk = l->pool_kernel; f->ps = l->pool_stride;
    f->act = l->act; f->act_param = l->act_param;
    if (l->kind == RGREF_LINEAR || l->kind == RGREF_CONV2D) {
      f->w = dupf(l->weight, l->weight_len); f->w_len = l->weight_len;
      f->b = dupf(l->bias, l->bias_len); f->b_len = l->bias_len;
    } else if (l->kind == RGREF_CHANNEL_AFFINE) {
      f->scale = dupf(l->scale, l->affine_len); f->shift = dupf(l->shift, l->affine_len);
      f->aff_len = l->affine_len;
    }
  }
  *out_n = m;
  return out;
}

static void free_folded(folded_layer* f, int64_t n) {
  for (int64_t i = 0; i < n; i++) { free(f[i].w); free(f[i].b); free(f[i].scale); free(f[i].shift); }
  free(f);
}

static float* round_fp16_copy(const float* w, int64_t n) {
  float* r = (float*)malloc(sizeof(float) * (size_t)(n > 0 ? n : 1));
  for (int64_t i = 0; i < n; i++) r[i] = rgref_round_fp16(w[i]);
  return r;
}

rgref_program* rgref_compile(const rgref_layer* layers, int64_t n_layers) {
  return rgref_compile_precision(layers, n_layers, RGREF_INT8);
}

rgref_program* rgref_compile_precision(const rgref_layer* layers, int64_t n_layers, int precision) {
  int64_t nf = 0;
  folded_layer* F = fold_batch_norm(layers, n_layers, &nf);
  rgref_program* P = (rgref_program*)calloc(1, sizeof(rgref_program));
  P->precision = precision;
  P->ops = (ref_op*)calloc((size_t)(nf > 0 ? nf : 1), sizeof(ref_op));
  P->original_layers = n_layers;
  if (precision == RGREF_FP32) {
    /* Standard program (mod.rs:164-171): the folded layers, run one by one. */
    for (int64_t j = 0; j < nf; j++) {
      folded_layer* f = &F[j];
      ref_op* op = &P->ops[P->n_ops++];
      op->kind = f->kind;
      op->act = f->act; op->act_param = f->act_param;
      if (f->kind == RGREF_LINEAR) {
        op->in_f = f->in_f; op->out_f = f->out_f;
        op->wh = dupf(f->w, f->w_len); op->w_len = f->w_len; op->bias = dupf(f->b, f->b_len);
        P->fp32_bytes += (f->w_len + f->b_len) * 4;
      } else if (f->kind == RGREF_CONV2D) {
        op->in_f = f->in_c; op->out_f = f->out_c;
        op->kernel = f->k; op->stride = f->s; op->padding = f->p;
        op->wh = dupf(f->w, f->w_len); op->w_len = f->w_len; op->bias = dupf(f->b, f->b_len);
        P->fp32_bytes += (f->w_len + f->b_len) * 4;
      } else if (f->kind == RGREF_CHANNEL_AFFINE) {
        op->in_f = op->out_f = f->aff_len;
        op->aff_scale = dupf(f->scale, f->aff_len); op->aff_len = f->aff_len;
        op->bias = dupf(f->shift, f->aff_len);
      } else {
        op->kernel = f->pk; op->stride = f->ps;
      }
    }
    P->npu_bytes = P->fp32_bytes;
    free_folded(F, nf);
    return P;
  }
  int64_t i = 0;
  while (i < nf) {
    int has_act = (i + 1 < nf) && F[i + 1].kind == RGREF_ACTIVATION;
    ref_op* op = &P->ops[P->n_ops];
    memset(op, 0, sizeof *op);
    folded_layer* f = &F[i];
    if (f->kind == RGREF_LINEAR) {
      op->kind = RGREF_LINEAR;
      op->act = has_act ? F[i + 1].act : RGREF_ACT_NONE;
      op->act_param = has_act ? F[i + 1].act_param : 0.0f;
      if (has_act) i++;
      op->in_f = f->in_f; op->out_f = f->out_f;
      /* transpose2d [in,out] -> [out,in], then per-tensor quantize (npu.rs:208-209) */
      float* wt = (float*)malloc(sizeof(float) * (size_t)(f->in_f * f->out_f > 0 ? f->in_f * f->out_f : 1));
      rgref_transpose2d(f->w, f->in_f, f->out_f, wt);
      op->w_len = f->in_f * f->out_f;
      op->wq = (int8_t*)malloc((size_t)(op->w_len > 0 ? op->w_len : 1));
      op->w_scale = rgref_quantize(wt, op->w_len, op->wq);
      op->wh = round_fp16_copy(wt, op->w_len); /* npu.rs:210 */
      free(wt);
      op->bias = dupf(f->b, f->b_len);
      P->fp32_bytes += (f->w_len + f->b_len) * 4;
      P->npu_bytes += precision == RGREF_FP16 ? f->w_len * 2 + f->b_len * 2 : (op->w_len + 4) + f->b_len * 4;
      P->n_ops++;
    } else if (f->kind == RGREF_CONV2D) {
      op->kind = RGREF_CONV2D;
      op->act = has_act ? F[i + 1].act : RGREF_ACT_NONE;
      op->act_param = has_act ? F[i + 1].act_param : 0.0f;
      if (has_act) i++;
      op->in_f = f->in_c; op->out_f = f->out_c;
      op->kernel = f->k; op->stride = f->s; op->padding = f->p;
      op->w_len = f->w_len;
      op->wq = (int8_t*)malloc((size_t)(op->w_len > 0 ? op->w_len : 1));
      op->w_scale = rgref_quantize(f->w, op->w_len, op->wq); /* [out, c*k*k] (npu.rs:231) */
      op->wh = round_fp16_copy(f->w, op->w_len);             /* npu.rs:232 */
      op->bias = dupf(f->b, f->b_len);
      P->fp32_bytes += (f->w_len + f->b_len) * 4;
      P->npu_bytes += precision == RGREF_FP16 ? f->w_len * 2 + f->b_len * 2 : (op->w_len + 4) + f->b_len * 4;
      P->n_ops++;
    } else if (f->kind == RGREF_CHANNEL_AFFINE) {
      /* lone ChannelAffine -> diagonal FusedLinear, no byte accounting (npu.rs:254-270) */
      int64_t c = f->aff_len;
      float* w = (float*)calloc((size_t)(c * c > 0 ? c * c : 1), sizeof(float));
      for (int64_t j = 0; j < c; j++) w[j * c + j] = f->scale[j];
      op->kind = RGREF_LINEAR; op->in_f = c; op->out_f = c; op->act = RGREF_ACT_NONE;
      op->w_len = c * c;
      op->wq = (int8_t*)malloc((size_t)(op->w_len > 0 ? op->w_len : 1));
      op->w_scale = rgref_quantize(w, op->w_len, op->wq);
      op->wh = w; /* weight_fp16_t: w as is, not rounded (npu.rs:266) */
      op->bias = dupf(f->shift, c);
      P->n_ops++;
    } else {
      op->kind = f->kind;
      op->kernel = f->pk; op->stride = f->ps;
      op->act = f->act; op->act_param = f->act_param;
      P->n_ops++;
    }
    i++;
  }
  free_folded(F, nf);
  return P;
}

static void free_caps(ref_op* op) {
  free(op->cap_q); free(op->cap_scale); free(op->cap_acc); free(op->cap_out);
  op->cap_q = NULL; op->cap_scale = NULL; op->cap_acc = NULL; op->cap_out = NULL;
  op->cap_q_len = op->cap_scale_len = op->cap_acc_len = op->cap_out_len = 0;
}

void rgref_program_free(rgref_program* p) {
  if (!p) return;
  for (int64_t i = 0; i < p->n_ops; i++) {
    free(p->ops[i].wq); free(p->ops[i].wh); free(p->ops[i].aff_scale); free(p->ops[i].bias); free_caps(&p->ops[i]);
  }
  free(p->ops); free(p->out); free(p);
}
int64_t rgref_program_num_ops(const rgref_program* p) { return p->n_ops; }
int64_t rgref_program_fp32_bytes(const rgref_program* p) { return p->fp32_bytes; }
int64_t rgref_program_npu_bytes(const rgref_program* p) { return p->npu_bytes; }
int64_t rgref_program_original_layers(const rgref_program* p) { return p->original_layers; }
int64_t rgref_program_op_macs(const rgref_program* p, int64_t i) { return p->ops[i].macs; }
int64_t rgref_program_total_macs(const rgref_program* p) { return p->total_macs; }
void rgref_program_set_capture(rgref_program* p, int on) { p->capture = on; }

int64_t rgref_program_op_weight_fp16(const rgref_program* p, int64_t i, const float** w, int64_t* rows) {
  const ref_op* op = &p->ops[i];
  *w = op->wh;
  *rows = op->out_f;
  return op->wh ? op->w_len : 0;
}

int64_t rgref_program_op_weight(const rgref_program* p, int64_t i, const int8_t** w, float* scale,
                                const float** bias) {
  const ref_op* op = &p->ops[i];
  *w = op->wq; *scale = op->w_scale; *bias = op->bias;
  return op->w_len;
}

int64_t rgref_program_capture(const rgref_program* p, int64_t i, int what, const void** data) {
  const ref_op* op = &p->ops[i];
  switch (what) {
    case RGREF_CAP_QACT: *data = op->cap_q; return op->cap_q_len;
    case RGREF_CAP_SCALE: *data = op->cap_scale; return op->cap_scale_len;
    case RGREF_CAP_ACC: *data = op->cap_acc; return op->cap_acc_len;
    case RGREF_CAP_OUT: *data = op->cap_out; return op->cap_out_len;
  }
  *data = NULL;
  return 0;
}

/* Rust's `Display` for f32: the shortest digit string that reads back as the
 * same f32, written positionally (no exponent): 0.01 -> "0.01", 1 -> "1",
 * 1e-5 -> "0.00001", NaN -> "NaN", inf -> "inf". */
static void fmt_f32_rust(float v, char* out, size_t cap) {
  if (v != v) { snprintf(out, cap, "NaN"); return; }
  if (isinf(v)) { snprintf(out, cap, v < 0 ? "-inf" : "inf"); return; }
  char sci[64];
  int prec = 1;
  for (; prec <= 9; prec++) {
    snprintf(sci, sizeof sci, "%.*e", prec - 1, (double)v);
    if (strtof(sci, NULL) == v) break;
  }
  /* sci = [-]d[.ddd]e[+-]XX */
  char digits[32]; int nd = 0; int neg = sci[0] == '-';
  const char* s = sci + neg;
  for (; *s && *s != 'e'; s++) if (*s >= '0' && *s <= '9') digits[nd++] = *s;
  int exp10 = atoi(s + 1);
  while (nd > 1 && digits[nd - 1] == '0') nd--; /* trailing zeros of the mantissa */
  char buf[128]; int o = 0;
  if (neg) buf[o++] = '-';
  int point = exp10 + 1; /* digits before the decimal point */
  if (point <= 0) {
    buf[o++] = '0'; buf[o++] = '.';
    for (int i = 0; i < -point; i++) buf[o++] = '0';
    for (int i = 0; i < nd; i++) buf[o++] = digits[i];
  } else if (point >= nd) {
    for (int i = 0; i < nd; i++) buf[o++] = digits[i];
    for (int i = nd; i < point; i++) buf[o++] = '0';
  } else {
    for (int i = 0; i < point; i++) buf[o++] = digits[i];
    buf[o++] = '.';
    for (int i = point; i < nd; i++) buf[o++] = digits[i];
  }
  buf[o] = 0;
  snprintf(out, cap, "%s", buf);
}

/* Activation Display (inference/mod.rs:56-67). */
static void act_name(int act, float p, char* buf, size_t cap) {
  switch (act) {
    case RGREF_ACT_NONE: snprintf(buf, cap, "none"); break;
    case RGREF_ACT_RELU: snprintf(buf, cap, "ReLU"); break;
    case RGREF_ACT_SIGMOID: snprintf(buf, cap, "Sigmoid"); break;
    case RGREF_ACT_TANH: snprintf(buf, cap, "Tanh"); break;
    case RGREF_ACT_GELU: snprintf(buf, cap, "GELU"); break;
    case RGREF_ACT_SILU: snprintf(buf, cap, "SiLU"); break;
    case RGREF_ACT_LEAKY_RELU: {
      char num[64];
      fmt_f32_rust(p, num, sizeof num);
      snprintf(buf, cap, "LeakyReLU(%s)", num);
      break;
    }
    default: snprintf(buf, cap, "?");
  }
}

/* NpuOp::label (npu.rs:83-104). */
int64_t rgref_program_op_label(const rgref_program* p, int64_t i, char* buf, int64_t cap) {
  const ref_op* op = &p->ops[i];
  char a[128];
  act_name(op->act, op->act_param, a, sizeof a);
  int n = 0;
  switch (op->kind) {
    case RGREF_LINEAR:
      n = op->act == RGREF_ACT_NONE
              ? snprintf(buf, (size_t)cap, "NPU::Gemm(%lld->%lld)", (long long)op->in_f, (long long)op->out_f)
              : snprintf(buf, (size_t)cap, "NPU::FusedGemmAct(%lld->%lld, %s)", (long long)op->in_f,
                         (long long)op->out_f, a);
      break;
    case RGREF_CONV2D:
      n = op->act == RGREF_ACT_NONE
              ? snprintf(buf, (size_t)cap, "NPU::Conv2d(%lld->%lld, k=%lld)", (long long)op->in_f,
                         (long long)op->out_f, (long long)op->kernel)
              : snprintf(buf, (size_t)cap, "NPU::FusedConv2dAct(%lld->%lld, k=%lld, %s)", (long long)op->in_f,
                         (long long)op->out_f, (long long)op->kernel, a);
      break;
    case RGREF_MAXPOOL2D: n = snprintf(buf, (size_t)cap, "NPU::MaxPool2d(k=%lld)", (long long)op->kernel); break;
    case RGREF_FLATTEN: n = snprintf(buf, (size_t)cap, "NPU::Flatten"); break;
    case RGREF_ACTIVATION: n = snprintf(buf, (size_t)cap, "NPU::Act(%s)", a); break;
    case RGREF_SOFTMAX: n = snprintf(buf, (size_t)cap, "NPU::Softmax"); break;
  }
  return n;
}

/* ================ standard FP32 path (run_standard, mod.rs:260-331) ======== */
/* Backend matmul C[m,n] = A[m,k] @ B[k,n] as the GPU provider's WGSL shader
 * orders it (wgpu_impl.rs:20-48): per output a serial f32 sum over k in
 * order, multiply then add.  (The CPU backend's AVX2/FMA blocking,
 * cpu.rs:43-160, orders the same products differently.) */
/* c[r, j] = fl(... fl(fl(0 + fl(a[r,0] b[0,j])) + fl(a[r,1] b[1,j])) ...): each
   output sums its products serially in increasing p.  The loop keeps one
   accumulator per output column of a block and walks b along its rows, so
   the work is spread over (row, column block) pairs and b is read with unit
   stride; every accumulator still adds its products in the same order. */
#define RGREF_MM_JB 256
void rgref_matmul_f32(const float* a, const float* b, int64_t m, int64_t k, int64_t n, float* c, int parallel) {
  const int64_t nb = (n + RGREF_MM_JB - 1) / RGREF_MM_JB;
#pragma omp parallel for schedule(dynamic, 1) num_threads(rgref_get_threads()) if (parallel && m * k * n >= 32 * 1024)
  for (int64_t t = 0; t < m * nb; t++) {
    const int64_t r = t / nb, j0 = (t % nb) * RGREF_MM_JB;
    const int64_t w = n - j0 < RGREF_MM_JB ? n - j0 : RGREF_MM_JB;
    float acc[RGREF_MM_JB];
    for (int64_t j = 0; j < w; j++) acc[j] = 0.0f;
    for (int64_t p = 0; p < k; p++) {
      const float av = a[r * k + p];
      const float* br = b + p * n + j0;
      for (int64_t j = 0; j < w; j++) {
        const float prod = av * br[j];
        acc[j] = acc[j] + prod;
      }
    }
    for (int64_t j = 0; j < w; j++) c[r * n + j0 + j] = acc[j];
  }
}

static int standard_layer(ref_op* op, float** pdata, int64_t* plen, int64_t* shape, int* pnd, int parallel) {
  float* data = *pdata; int64_t len = *plen; int nd = *pnd;
  if (op->kind == RGREF_LINEAR) {                                      /* mod.rs:264-273 */
    int64_t in = op->in_f, out = op->out_f;
    if (in <= 0 || len % in != 0) { set_err("Linear: input length not a multiple of in_features"); return 1; }
    int64_t rows = len / in;
    op->macs = rows * in * out;
    float* y = (float*)malloc(sizeof(float) * (size_t)(rows * out > 0 ? rows * out : 1));
    rgref_matmul_f32(data, op->wh, rows, in, out, y, parallel);
    for (int64_t r = 0; r < rows; r++)
      for (int64_t c = 0; c < out; c++) y[r * out + c] = y[r * out + c] + op->bias[c];
    free(data); data = y; len = rows * out; shape[nd - 1] = out;
  } else if (op->kind == RGREF_CONV2D) {                               /* mod.rs:274-290, kernels.rs:218-265 */
    if (nd < 4) { set_err("Conv2d: input must be NCHW"); return 1; }
    int64_t n = shape[0], c = shape[1], h = shape[2], w = shape[3];
    if (c != op->in_f) { set_err("Conv2d: channel mismatch"); return 1; }
    int64_t k = op->kernel, s = op->stride, pd = op->padding, O = op->out_f;
    int64_t oh = rgref_out_size(h, k, s, pd), ow = rgref_out_size(w, k, s, pd);
    if (oh < 0 || ow < 0) { set_err("Conv2d: kernel larger than padded input"); return 1; }
    int64_t l = oh * ow, ckk = c * k * k;
    op->macs = n * O * ckk * l;
    float* out = (float*)malloc(sizeof(float) * (size_t)(n * O * l > 0 ? n * O * l : 1));
    float* cols = (float*)malloc(sizeof(float) * (size_t)(ckk * l > 0 ? ckk * l : 1));
    for (int64_t b = 0; b < n; b++) {
      rgref_im2col(data + b * c * h * w, c, h, w, k, s, pd, oh, ow, cols);
      rgref_matmul_f32(op->wh, cols, O, ckk, l, out + b * O * l, parallel); /* W[O,ckk] @ cols[ckk,L] */
      for (int64_t o = 0; o < O; o++)
        for (int64_t q = 0; q < l; q++) out[(b * O + o) * l + q] = out[(b * O + o) * l + q] + op->bias[o];
    }
    free(cols); free(data); data = out; len = n * O * l;
    shape[0] = n; shape[1] = O; shape[2] = oh; shape[3] = ow; nd = 4;
  } else if (op->kind == RGREF_CHANNEL_AFFINE) {                       /* mod.rs:292-306 */
    if (nd < 2 || shape[1] != op->aff_len) { set_err("ChannelAffine: channel mismatch"); return 1; }
    int64_t inner = 1;
    for (int i = 2; i < nd; i++) inner *= shape[i];
    for (int64_t b = 0; b < shape[0]; b++)
      for (int64_t ch = 0; ch < op->aff_len; ch++)
        for (int64_t q = 0; q < inner; q++) {
          float* v = &data[(b * op->aff_len + ch) * inner + q];
          float prod = *v * op->aff_scale[ch];
          *v = prod + op->bias[ch];
        }
  } else if (op->kind == RGREF_MAXPOOL2D) {                            /* mod.rs:307-313 */
    if (nd < 4) { set_err("MaxPool2d: input must be NCHW"); return 1; }
    int64_t n = shape[0], c = shape[1], h = shape[2], w = shape[3];
    int64_t oh = rgref_out_size(h, op->kernel, op->stride, 0), ow = rgref_out_size(w, op->kernel, op->stride, 0);
    if (oh < 0 || ow < 0) { set_err("MaxPool2d: kernel larger than input"); return 1; }
    float* out = (float*)malloc(sizeof(float) * (size_t)(n * c * oh * ow > 0 ? n * c * oh * ow : 1));
    rgref_max_pool2d(data, n, c, h, w, op->kernel, op->stride, out, parallel);
    free(data); data = out; len = n * c * oh * ow; shape[2] = oh; shape[3] = ow; nd = 4;
  } else if (op->kind == RGREF_FLATTEN) {                              /* mod.rs:314-317 */
    int64_t rest = 1;
    for (int i = 1; i < nd; i++) rest *= shape[i];
    shape[1] = rest; nd = 2;
  } else if (op->kind == RGREF_ACTIVATION) {                           /* mod.rs:318-322 */
    for (int64_t i = 0; i < len; i++) data[i] = rgref_act_apply(op->act, op->act_param, data[i]);
  } else if (op->kind == RGREF_SOFTMAX) {                              /* mod.rs:323-327 */
    int64_t last = shape[nd - 1];
    float* y = (float*)malloc(sizeof(float) * (size_t)(len > 0 ? len : 1));
    if (last > 0) rgref_softmax_rows(data, len / last, last, y);
    free(data); data = y;
  }
  *pdata = data; *plen = len; *pnd = nd;
  return 0;
}

/* ======================= execute (npu.rs:296-421) ========================= */
static void* xmalloc(size_t n) { return malloc(n ? n : 1); }

int rgref_execute(rgref_program* P, const float* x, const int64_t* shape_in, int ndim, int parallel) {
  if (ndim < 1 || ndim > 8) { set_err("rank must be 1..8"); return 1; }
  int64_t shape[8]; int nd = ndim; int64_t len = 1;
  for (int i = 0; i < ndim; i++) { shape[i] = shape_in[i]; len *= shape_in[i]; }
  float* data = (float*)xmalloc(sizeof(float) * (size_t)len);
  memcpy(data, x, sizeof(float) * (size_t)len);
  P->total_macs = 0;
  for (int64_t oi = 0; oi < P->n_ops; oi++) {
    ref_op* op = &P->ops[oi];
    free_caps(op);
    op->macs = 0;
    if (P->precision == RGREF_FP32) {
      if (standard_layer(op, &data, &len, shape, &nd, parallel)) { free(data); return 1; }
      goto op_done;
    }
    if (op->kind == RGREF_LINEAR) {                                    /* npu.rs:307-318 */
      int64_t in = op->in_f, out = op->out_f;
      if (in <= 0 || len % in != 0) { free(data); set_err("Linear: input length not a multiple of in_features"); return 1; }
      int64_t rows = len / in;
      op->macs = rows * in * out;
      if (P->precision == RGREF_FP16) {                                /* npu.rs:315 */
        float* y = (float*)xmalloc(sizeof(float) * (size_t)(rows * out));
        /* serial, as the reference runs it (no rayon split for FP16 Linear) */
        rgref_fp16_gemm_fused(data, op->wh, rows, in, out, op->bias, op->act, op->act_param, y, 0);
        free(data); data = y; len = rows * out;
        shape[nd - 1] = out;
        goto op_done;
      }
      int8_t* aq = (int8_t*)xmalloc((size_t)(rows * in));
      float sa = rgref_quantize(data, rows * in, aq);
      float* y = (float*)xmalloc(sizeof(float) * (size_t)(rows * out));
      int32_t* acc = P->capture ? (int32_t*)xmalloc(sizeof(int32_t) * (size_t)(rows * out)) : NULL;
      rgref_int8_gemm_fused(aq, sa, op->wq, op->w_scale, rows, in, out, op->bias, op->act, op->act_param, y, acc,
                            parallel);
      if (P->capture) {
        op->cap_q = aq; op->cap_q_len = rows * in;
        op->cap_scale = (float*)xmalloc(sizeof(float)); op->cap_scale[0] = sa; op->cap_scale_len = 1;
        op->cap_acc = acc; op->cap_acc_len = rows * out;
      } else {
        free(aq);
      }
      free(data); data = y; len = rows * out;
      shape[nd - 1] = out;
    } else if (op->kind == RGREF_CONV2D) {                             /* npu.rs:319-383 */
      if (nd < 4) { free(data); set_err("Conv2d: input must be NCHW"); return 1; }
      int64_t n = shape[0], c = shape[1], h = shape[2], w = shape[3];
      if (c != op->in_f) { free(data); set_err("Conv2d: channel mismatch"); return 1; }
      int64_t k = op->kernel, s = op->stride, pd = op->padding, O = op->out_f;
      int64_t oh = rgref_out_size(h, k, s, pd), ow = rgref_out_size(w, k, s, pd);
      if (oh < 0 || ow < 0) { free(data); set_err("Conv2d: kernel larger than padded input"); return 1; }
      int64_t l = oh * ow, ckk = c * k * k, img = c * h * w, ostr = O * l;
      op->macs = n * O * ckk * l;
      float* out = (float*)xmalloc(sizeof(float) * (size_t)(n * ostr));
      if (P->precision == RGREF_FP16) {                                /* npu.rs:353-355, 374-376 */
#pragma omp parallel for schedule(dynamic, 1) num_threads(rgref_get_threads()) if (parallel && n >= 2 && ostr > 0)
        for (int64_t b = 0; b < n; b++) {
          float* cols = (float*)xmalloc(sizeof(float) * (size_t)(ckk * l));
          float* cols_t = (float*)xmalloc(sizeof(float) * (size_t)(l * ckk));
          float* ylo = (float*)xmalloc(sizeof(float) * (size_t)(l * O));
          rgref_im2col(data + b * img, c, h, w, k, s, pd, oh, ow, cols);
          rgref_transpose2d(cols, ckk, l, cols_t);
          rgref_fp16_gemm_fused(cols_t, op->wh, l, ckk, O, op->bias, op->act, op->act_param, ylo, 0);
          rgref_transpose2d(ylo, l, O, out + b * ostr);
          free(cols); free(cols_t); free(ylo);
        }
        free(data); data = out; len = n * ostr;
        shape[0] = n; shape[1] = O; shape[2] = oh; shape[3] = ow; nd = 4;
        goto op_done;
      }
      if (P->capture) {
        op->cap_q = (int8_t*)xmalloc((size_t)(n * l * ckk)); op->cap_q_len = n * l * ckk;
        op->cap_scale = (float*)xmalloc(sizeof(float) * (size_t)n); op->cap_scale_len = n;
        op->cap_acc = (int32_t*)xmalloc(sizeof(int32_t) * (size_t)(n * l * O)); op->cap_acc_len = n * l * O;
      }
#pragma omp parallel for schedule(dynamic, 1) num_threads(rgref_get_threads()) if (parallel && n >= 2 && ostr > 0)
      for (int64_t b = 0; b < n; b++) {
        float* cols = (float*)xmalloc(sizeof(float) * (size_t)(ckk * l));
        float* cols_t = (float*)xmalloc(sizeof(float) * (size_t)(l * ckk));
        int8_t* aq = (int8_t*)xmalloc((size_t)(l * ckk));
        float* ylo = (float*)xmalloc(sizeof(float) * (size_t)(l * O));
        rgref_im2col(data + b * img, c, h, w, k, s, pd, oh, ow, cols);
        rgref_transpose2d(cols, ckk, l, cols_t);
        float sa = rgref_quantize(cols_t, l * ckk, aq);
        int32_t* acc = P->capture ? op->cap_acc + b * l * O : NULL;
        rgref_int8_gemm_fused(aq, sa, op->wq, op->w_scale, l, ckk, O, op->bias, op->act, op->act_param, ylo, acc, 0);
        rgref_transpose2d(ylo, l, O, out + b * ostr);
        if (P->capture) { memcpy(op->cap_q + b * l * ckk, aq, (size_t)(l * ckk)); op->cap_scale[b] = sa; }
        free(cols); free(cols_t); free(aq); free(ylo);
      }
      free(data); data = out; len = n * ostr;
      shape[0] = n; shape[1] = O; shape[2] = oh; shape[3] = ow; nd = 4;
    } else if (op->kind == RGREF_MAXPOOL2D) {                          /* npu.rs:384-390 */
      if (nd < 4) { free(data); set_err("MaxPool2d: input must be NCHW"); return 1; }
      int64_t n = shape[0], c = shape[1], h = shape[2], w = shape[3];
      int64_t oh = rgref_out_size(h, op->kernel, op->stride, 0), ow = rgref_out_size(w, op->kernel, op->stride, 0);
      if (oh < 0 || ow < 0) { free(data); set_err("MaxPool2d: kernel larger than input"); return 1; }
      float* out = (float*)xmalloc(sizeof(float) * (size_t)(n * c * oh * ow));
      rgref_max_pool2d(data, n, c, h, w, op->kernel, op->stride, out, parallel);
      free(data); data = out; len = n * c * oh * ow;
      shape[2] = oh; shape[3] = ow; nd = 4;
    } else if (op->kind == RGREF_FLATTEN) {                            /* npu.rs:391-394 */
      int64_t rest = 1;
      for (int i = 1; i < nd; i++) rest *= shape[i];
      shape[1] = rest; nd = 2;
    } else if (op->kind == RGREF_ACTIVATION) {                         /* npu.rs:395-399 */
      for (int64_t i = 0; i < len; i++) data[i] = rgref_act_apply(op->act, op->act_param, data[i]);
    } else if (op->kind == RGREF_SOFTMAX) {                            /* npu.rs:400-404 */
      int64_t last = shape[nd - 1];
      float* y = (float*)xmalloc(sizeof(float) * (size_t)len);
      if (last > 0) rgref_softmax_rows(data, len / last, last, y);
      free(data); data = y;
    }
  op_done:
    if (P->capture) {
      op->cap_out = (float*)xmalloc(sizeof(float) * (size_t)len);
      memcpy(op->cap_out, data, sizeof(float) * (size_t)len);
      op->cap_out_len = len;
    }
    P->total_macs += op->macs;
  }
  free(P->out);
  P->out = data; P->out_len = len; P->out_ndim = nd;
  for (int i = 0; i < nd; i++) P->out_shape[i] = shape[i];
  return 0;
}

int64_t rgref_program_output(const rgref_program* p, const float** y, int64_t* shape, int* ndim) {
  *y = p->out;
  *ndim = p->out_ndim;
  for (int i = 0; i < p->out_ndim; i++) shape[i] = p->out_shape[i];
  return p->out_len;
}
