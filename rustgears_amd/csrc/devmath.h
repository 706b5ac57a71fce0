// devmath.h — activation math shared by the HIP kernels and the host side,
// bit-identical to what the reference computes on its host.
//
// The reference applies activations with f32 arithmetic and host libm
// (src/device/backend.rs:66-78, src/inference/mod.rs:37-53):
//   ReLU  x.max(0)          Sigmoid 1/(1+exp(-x))      Tanh x.tanh()
//   GELU  0.5*x*(1+tanh(0.7978846*(x+0.044715*x*x*x)))   LeakyReLU x>0?x:s*x
// and SiLU (build extension, src/nn/layers.rs:341-343) is x*sigmoid(x).
// Rust lowers f32::tanh / f32::exp to glibc tanhf / expf.  The two functions
// below restate the published algorithms glibc 2.35 uses for them so the GPU
// reproduces glibc's results exactly (not merely to within an ulp):
//   * tanhf: fdlibm s_tanhf.c on top of fdlibm s_expm1f.c (Sun Microsystems,
//     permissive licence), as shipped in glibc sysdeps/ieee754/flt-32.
//   * expf:  ARM optimized-routines expf (Szabolcs Nagy, MIT/Apache-2.0),
//     glibc sysdeps/ieee754/flt-32/e_expf.c, in the form glibc's x86-64 FMA
//     ifunc variant computes it (fused multiply-add in the double-precision
//     argument reduction and polynomial).  The 2^(i/32) table is generated
//     from its definition, asuint64(2^(i/32)) - (i << 47).
// Both restatements were compared against glibc 2.35 on every one of the 2^32
// f32 inputs with zero mismatches; tests/test_host.py re-checks the host build
// against the local libm and tests/test_gpu_devmath.py the GPU build.
//
// Everything here must be compiled with -ffp-contract=off: the reference does
// not contract a*b+c, and neither may we outside the explicit fma() calls.
#pragma once
#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__)
#define RG_HD __host__ __device__ __forceinline__
#else
#define RG_HD static inline
#endif

namespace rgmath {

RG_HD uint32_t fbits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
RG_HD float bitsf(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
RG_HD uint64_t dbits(double f) { uint64_t u; memcpy(&u, &f, 8); return u; }
RG_HD double bitsd(uint64_t u) { double f; memcpy(&f, &u, 8); return f; }

// f32::max(self, 0.0): NaN-ignoring maximum.
RG_HD float fmax_nan_ignoring(float a, float b) {
  if (a != a) return b;
  if (b != b) return a;
  return a > b ? a : (b > a ? b : a);
}

// x.max(0.0) as the reference's x86-64 build computes it (backend.rs:71):
// llvm.maxnum with a constant operand that cannot be NaN becomes one maxss
// with the constant as its source operand, x > 0 ? x : 0, so NaN and -0.0
// both give +0.0.
RG_HD float relu(float x) { return x > 0.0f ? x : 0.0f; }

// ---------------------------------------------------------------------------
// The constants and steps of expm1f / tanhf below restate fdlibm's
// s_expm1f.c and s_tanhf.c, which carry this notice:
//   Copyright (C) 1993 by Sun Microsystems, Inc. All rights reserved.
//   Developed at SunPro, a Sun Microsystems, Inc. business.
//   Permission to use, copy, modify, and distribute this
//   software is freely granted, provided that this notice
//   is preserved.
// (float versions by Ian Lance Taylor, Cygnus Support).
// ---------------------------------------------------------------------------

// fdlibm expm1f.  Branches are kept in the published order; the tanh path
// only reaches k in {0,-1,-2,-3} (|x|<1) and k in [3,63] (1<=|x|<22).
RG_HD float expm1f_fdlibm(float x) {
  const float ln2_hi = bitsf(0x3f317180u), ln2_lo = bitsf(0x3717f7d1u), invln2 = bitsf(0x3fb8aa3bu);
  const float Q1 = bitsf(0xbd088889u), Q2 = bitsf(0x3ad00d01u), Q3 = bitsf(0xb8a670cdu),
              Q4 = bitsf(0x36867e54u), Q5 = bitsf(0xb457edbbu);
  float y, hi, lo, c = 0.0f, t, e, hxs, hfx, r1;
  int32_t k;
  uint32_t hx = fbits(x);
  const uint32_t xsb = hx & 0x80000000u;
  hx &= 0x7fffffffu;
  if (hx >= 0x4195b844u) {            // |x| >= 27*ln2
    if (hx >= 0x42b17218u) {          // |x| >= 88.72
      if (hx > 0x7f800000u) return x + x;
      if (hx == 0x7f800000u) return xsb == 0 ? x : -1.0f;
      if (x > bitsf(0x42b17180u)) return bitsf(0x7f800000u);
    }
    if (xsb != 0) return -1.0f;
  }
  if (hx > 0x3eb17218u) {             // |x| > 0.5 ln2
    if (hx < 0x3F851592u) {           // |x| < 1.5 ln2
      if (xsb == 0) { hi = x - ln2_hi; lo = ln2_lo; k = 1; }
      else { hi = x + ln2_hi; lo = -ln2_lo; k = -1; }
    } else {
      float kf = invln2 * x;
      kf = kf + (xsb == 0 ? 0.5f : -0.5f);
      k = (int32_t)kf;
      t = (float)k;
      float th = t * ln2_hi;
      hi = x - th;
      lo = t * ln2_lo;
    }
    x = hi - lo;
    c = (hi - x) - lo;
  } else if (hx < 0x33000000u) {      // |x| < 2^-25
    return x;
  } else {
    k = 0;
  }
  hfx = 0.5f * x;
  hxs = x * hfx;
  float p = hxs * Q5; p = Q4 + p;
  p = hxs * p; p = Q3 + p;
  p = hxs * p; p = Q2 + p;
  p = hxs * p; p = Q1 + p;
  p = hxs * p; r1 = 1.0f + p;
  float rh = r1 * hfx; t = 3.0f - rh;
  float xt = x * t; float den = 6.0f - xt;
  float num = r1 - t;
  float q = num / den;
  e = hxs * q;
  if (k == 0) { float xe = x * e; xe = xe - hxs; return x - xe; }
  float ec = e - c; e = x * ec; e = e - c;
  e = e - hxs;
  if (k == -1) { float d = x - e; d = 0.5f * d; return d - 0.5f; }
  if (k == 1) {
    if (x < -0.25f) { float xh = x + 0.5f; float d = e - xh; return -2.0f * d; }
    float d = x - e; d = 2.0f * d; return 1.0f + d;
  }
  if (k <= -2 || k > 56) {
    float d = e - x; y = 1.0f - d;
    y = bitsf(fbits(y) + ((uint32_t)k << 23));
    return y - 1.0f;
  }
  if (k < 23) {
    t = bitsf(0x3f800000u - (0x1000000u >> k));
    float d = e - x; y = t - d;
    y = bitsf(fbits(y) + ((uint32_t)k << 23));
  } else {
    t = bitsf((uint32_t)(0x7f - k) << 23);
    float d = e + t; y = x - d;
    y = y + 1.0f;
    y = bitsf(fbits(y) + ((uint32_t)k << 23));
  }
  return y;
}

// fdlibm tanhf.
RG_HD float tanhf_fdlibm(float x) {
  const uint32_t jx = fbits(x), ix = jx & 0x7fffffffu;
  float t, z;
  if (ix >= 0x7f800000u) {
    float r = 1.0f / x;
    return (jx >> 31) == 0 ? r + 1.0f : r - 1.0f;
  }
  if (ix < 0x41b00000u) {             // |x| < 22
    if (ix == 0) return x;
    if (ix < 0x24000000u) { float o = 1.0f + x; return x * o; }
    float ax = bitsf(ix);
    if (ix >= 0x3f800000u) {          // |x| >= 1
      t = expm1f_fdlibm(2.0f * ax);
      float d = t + 2.0f; float q = 2.0f / d; z = 1.0f - q;
    } else {
      t = expm1f_fdlibm(-2.0f * ax);
      float d = t + 2.0f; float nt = -t; z = nt / d;
    }
  } else {
    z = 1.0f;
  }
  return (jx >> 31) ? -z : z;
}

// ---------------------------------------------------------------------------
// Branch-free forms of the same two fdlibm functions, used in the GEMM
// epilogues.  They perform the identical sequence of f32 roundings; only the
// control flow differs: every case of expm1f's argument reduction and
// reconstruction is computed and the right one selected, so the 64 lanes of
// a wave never diverge.  The reduction is shared (k = 0 and k = +-1 are the
// general formula with t = 0 and t = +-1: t*ln2_hi is exact and
// x - (-a) == x + a), and tanhf's two divisions 2/(t+2) and -t/(t+2) share
// their denominator.  On the GPU the correctly rounded division is
// computed as q0 = n*rcp(d), q = fma(fma(-d, q0, n), rcp(d), q0); the
// exhaustive device check in tests/support/devmath_gpu_check.hip confirms
// tanhf_fast == tanhf_fdlibm for all 2^32 inputs.  On
// the host the division is the IEEE one, so the host build of these
// functions is compared with glibc by tests/support/devmath_host_check.cpp.
// ---------------------------------------------------------------------------
RG_HD float div_fast(float n, float d) {
#if defined(__HIP_DEVICE_COMPILE__)
  const float r = __builtin_amdgcn_rcpf(d);
  const float q0 = n * r;
  const float rem = __builtin_fmaf(-d, q0, n);
  return __builtin_fmaf(rem, r, q0);
#else
  return n / d;
#endif
}

// expm1f_fdlibm restricted to the arguments tanhf passes: x in (-2, 0) and
// x in [2, 44].  (k = 1 and the |x| >= 27 ln2 negative exit never occur.)
RG_HD float expm1f_tanh_domain(float x) {
  const float ln2_hi = bitsf(0x3f317180u), ln2_lo = bitsf(0x3717f7d1u), invln2 = bitsf(0x3fb8aa3bu);
  const float Q1 = bitsf(0xbd088889u), Q2 = bitsf(0x3ad00d01u), Q3 = bitsf(0xb8a670cdu),
              Q4 = bitsf(0x36867e54u), Q5 = bitsf(0xb457edbbu);
  const uint32_t bx = fbits(x);
  const uint32_t hx = bx & 0x7fffffffu;
  const bool neg = (bx >> 31) != 0;
  // argument reduction: k = 0 (|x| <= 0.5 ln2), -1 (|x| < 1.5 ln2, x < 0), else rounded
  float kf = invln2 * x;
  kf = kf + (neg ? -0.5f : 0.5f);
  const int32_t kgen = (int32_t)kf;
  const int32_t k = hx > 0x3eb17218u ? (hx < 0x3F851592u ? (neg ? -1 : 1) : kgen) : 0;
  const float t = (float)k;
  const float th = t * ln2_hi;
  const float hi = x - th;
  const float lo = t * ln2_lo;
  const float xr = hi - lo;
  const float c = (hi - xr) - lo;
  const float hfx = 0.5f * xr;
  const float hxs = xr * hfx;
  float p = hxs * Q5; p = Q4 + p;
  p = hxs * p; p = Q3 + p;
  p = hxs * p; p = Q2 + p;
  p = hxs * p; p = Q1 + p;
  p = hxs * p;
  const float r1 = 1.0f + p;
  const float rh = r1 * hfx;
  const float tt = 3.0f - rh;
  const float xt = xr * tt;
  const float den = 6.0f - xt;
  const float num = r1 - tt;
  const float e = hxs * div_fast(num, den);
  // k == 0
  const float xe = xr * e;
  const float r0 = xr - (xe - hxs);
  // k != 0 share e2 = x*(e-c) - c - hxs
  const float ec = e - c;
  float e2 = xr * ec;
  e2 = e2 - c;
  e2 = e2 - hxs;
  const float em = e2 - xr;
  // k == -1
  const float d1 = xr - e2;
  const float rm1 = 0.5f * d1 - 0.5f;
  // k <= -2 or k > 56
  const uint32_t kshift = (uint32_t)k << 23;
  const float ylow = 1.0f - em;
  const float rlow = bitsf(fbits(ylow) + kshift) - 1.0f;
  // 2 <= k < 23: t = 1 - 2^-k
  const float tk = bitsf(0x3f800000u - (0x1000000u >> (k & 31)));
  const float rmid = bitsf(fbits(tk - em) + kshift);
  // 23 <= k <= 56: t = 2^-k
  const float t2 = bitsf(((uint32_t)(0x7f - k) & 0x1ffu) << 23);
  const float yh = (xr - (e2 + t2)) + 1.0f;
  const float rhigh = bitsf(fbits(yh) + kshift);
  float r = k == 0 ? r0 : (k == -1 ? rm1 : ((k <= -2 || k > 56) ? rlow : (k < 23 ? rmid : rhigh)));
  return hx < 0x33000000u ? x : r;
}

RG_HD float tanhf_fast(float x) {
  const uint32_t jx = fbits(x), ix = jx & 0x7fffffffu;
  const float ax = bitsf(ix);
  const bool ge1 = ix >= 0x3f800000u;
  const float two_ax = 2.0f * ax;
  // |x| >= 22 selects z = 1 below; capping keeps the unused lanes in range.
  const float arg = ge1 ? (two_ax < 44.0f ? two_ax : 44.0f) : -two_ax;
  const float t = expm1f_tanh_domain(arg);
  const float d = t + 2.0f;
  const float q = div_fast(ge1 ? 2.0f : -t, d);
  float z = ge1 ? 1.0f - q : q;
  z = ix >= 0x41b00000u ? 1.0f : z;                // |x| >= 22 (and +-inf)
  const float signed_z = (jx >> 31) ? -z : z;
  const float tiny = x * (1.0f + x);               // |x| < 2^-55, and +-0
  float r = ix < 0x24000000u ? tiny : signed_z;
  return ix > 0x7f800000u ? x + x : r;             // NaN
}

// GELU for the GEMM epilogues: the same f32 roundings as gelu() (fdlibm
// tanhf over fdlibm expm1f), restricted to the arguments GELU produces and
// with every case that cannot change the result folded away:
//  * |u| >= 9.25: fdlibm returns z = 1 - 2/(t+2) with t + 2 >= 2^26, which
//    rounds to 1; capping expm1's argument 2|u| at 18.5 keeps t + 2 above
//    2^26, so the general path also yields exactly 1 (this covers fdlibm's
//    |u| >= 22 and +-inf exits too);
//  * |u| < 2^-55 (fdlibm's u*(1+u)) and |arg| < 2^-25 (expm1's x exit):
//    the polynomial path returns the same value to within half an ulp of 1,
//    which 1 + t absorbs;
//  * expm1's k selection: k = 0 below 0.5 ln2 comes out of the rounded
//    reduction except at its boundary, where the result is unchanged;
//  * expm1's reconstruction for k <= -2, k == 0 and 3 <= k <= 27 is one
//    formula y = T - (e - x), y * 2^k, minus 1 when k < 0 (T = 1, 0 or
//    1 - 2^-k); for k == 0 it is fdlibm's x - (x*e - hxs) exactly, and the
//    23 <= k form x - (e + 2^-k) + 1 gives the same GELU.
// The exhaustive device check (every f32 input) confirms gelu_fast == gelu.
RG_HD float gelu_fast(float x) {
  float x3 = 0.044715f * x; x3 = x3 * x; x3 = x3 * x;
  const float inner = x + x3;
  const float u = 0.7978846f * inner;
  const uint32_t ju = fbits(u);
  const float au = __builtin_fabsf(u);
  const bool ge1 = !(au < 1.0f);  // |u| >= 1 or NaN, as the integer test of |u|'s bits
  const float two_au = 2.0f * au;
  // tanhf: t = expm1(2|u|) for |u| >= 1, expm1(-2|u|) below
  const float arg = ge1 ? __builtin_fminf(two_au, 18.5f) : -two_au;
  const float ln2_hi = bitsf(0x3f317180u), ln2_lo = bitsf(0x3717f7d1u), invln2 = bitsf(0x3fb8aa3bu);
  const float Q1 = bitsf(0xbd088889u), Q2 = bitsf(0x3ad00d01u), Q3 = bitsf(0xb8a670cdu),
              Q4 = bitsf(0x36867e54u), Q5 = bitsf(0xb457edbbu);
  float kf = invln2 * arg;
  kf = kf + (ge1 ? 0.5f : -0.5f);
  const int32_t k = (int32_t)kf;
  const float tk = (float)k;
  const float th = tk * ln2_hi;
  const float hi = arg - th;
  const float lo = tk * ln2_lo;
  const float xr = hi - lo;
  const float c = (hi - xr) - lo;
  const float hfx = 0.5f * xr;
  const float hxs = xr * hfx;
  float p = hxs * Q5; p = Q4 + p;
  p = hxs * p; p = Q3 + p;
  p = hxs * p; p = Q2 + p;
  p = hxs * p; p = Q1 + p;
  p = hxs * p;
  const float r1 = 1.0f + p;
  const float rh = r1 * hfx;
  const float tt = 3.0f - rh;
  const float xt = xr * tt;
  const float den = 6.0f - xt;
  const float num = r1 - tt;
  const float e = hxs * div_fast(num, den);
  // e2 = x*(e-c) - c - hxs, em = e2 - x.  For k == 0, c is exactly 0, so
  // -em is fdlibm's x - (x*e - hxs) bit for bit.
  const float ec = e - c;
  float e2 = xr * ec;
  e2 = e2 - c;
  e2 = e2 - hxs;
  const float em = e2 - xr;
  // k == -1
  const float d1 = xr - e2;
  const float rm1 = 0.5f * d1 - 0.5f;
  // k <= -2, k == 0 and 3 <= k <= 27: y = T - em scaled by 2^k, minus 1
  // when k < 0, with T = 1 - 2^-k (0 for k == 0, exact up to k = 24, 1 from
  // k = 25 on) and T = 1 for k < 0 (the shift by k & 31 >= 29 gives 0)
  const float T = bitsf(0x3f800000u - (0x1000000u >> (k & 31)));
  const float y = (k == 0 ? 0.0f : T) - em;
  const float ys = bitsf(fbits(y) + ((uint32_t)k << 23));
  const float rk = k < 0 ? ys - 1.0f : ys;
  const float t = k == -1 ? rm1 : rk;
  // tanhf: z = 1 - 2/(t+2) for |u| >= 1, -t/(t+2) below; sign of u
  const float d = t + 2.0f;
  const float q = div_fast(ge1 ? 2.0f : -t, d);
  const float z = ge1 ? 1.0f - q : q;
  const float tanh_u = bitsf(fbits(z) ^ (ju & 0x80000000u));
  const float h = 0.5f * x;
  const float one_t = 1.0f + tanh_u;
  return h * one_t;
}

// ---------------------------------------------------------------------------
// The table, constants and steps of expf below restate the expf of Arm's
// optimized-routines (as used by glibc's e_expf.c):
//   Copyright (c) 2017-2018, Arm Limited.
//   SPDX-License-Identifier: MIT OR Apache-2.0 WITH LLVM-exception
// ---------------------------------------------------------------------------

// 2^(i/32) table of ARM optimized-routines expf: asuint64(2^(i/32)) - (i<<47).
#if defined(__HIPCC__)
__host__ __device__
#endif
static inline uint64_t exp2f_tab(uint32_t i) {
  // Values of double(2^(i/32)) with i<<47 subtracted (see header comment).
  constexpr uint64_t T[32] = {
      0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
      0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
      0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
      0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
      0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
      0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
      0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
      0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull};
  return T[i & 31];
}

RG_HD float expf_aor(float x) {
  const double C0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
  const double C1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
  const double C2 = 0x1.62e42ff0c52d6p-1 / 32;
  const double SHIFT = 0x1.8p+52;
  const double INVLN2N = 0x1.71547652b82fep+0 * 32;
  const uint32_t abstop = (fbits(x) >> 20) & 0x7ffu;
  if (abstop >= 0x42bu) {             // |x| >= 88 or NaN (top12(88.0f))
    if (fbits(x) == 0xff800000u) return 0.0f;
    if (abstop >= 0x7f8u) return x + x;
    if (x > 0x1.62e42ep6f) return bitsf(0x7f800000u);
    if (x < -0x1.9fe368p6f) return 0.0f;
  }
  const double xd = (double)x;
  double kd = __builtin_fma(INVLN2N, xd, SHIFT);
  const uint64_t ki = dbits(kd);
  kd = kd - SHIFT;
  const double r = __builtin_fma(INVLN2N, xd, -kd);
  uint64_t t = exp2f_tab((uint32_t)(ki % 32));
  t += ki << 47;
  const double s = bitsd(t);
  double z = __builtin_fma(C0, r, C1);
  const double r2 = r * r;
  double y = __builtin_fma(C2, r, 1.0);
  y = __builtin_fma(z, r2, y);
  y = y * s;
  return (float)y;
}

// Activation codes (RTIM encoding, src/save.rs:201-208; 6 = SiLU extension).
enum : int { ACT_NONE = 0, ACT_RELU = 1, ACT_SIGMOID = 2, ACT_TANH = 3, ACT_GELU = 4,
             ACT_LEAKY_RELU = 5, ACT_SILU = 6 };

RG_HD float sigmoid(float x) { float e = expf_aor(-x); float d = 1.0f + e; return 1.0f / d; }

RG_HD float gelu(float x) {
  float x3 = 0.044715f * x; x3 = x3 * x; x3 = x3 * x;
  float inner = x + x3;
  float u = 0.7978846f * inner;
  float t = tanhf_fdlibm(u);
  float h = 0.5f * x;
  float one_t = 1.0f + t;
  return h * one_t;
}

// Certified GELU for the INT8 requantization (a GELU output that only feeds
// the next Linear's QuantTensor::from_f32, quantize.rs:18-24).  Only the
// tensor's absmax and each value's quantized integer leave such a layer, and
// both can be had exactly without evaluating the exact GELU on every value:
//  * absmax: on [0, +inf] the f32 GELU never decreases, and over every
//    negative input |gelu(x)| <= kGeluNegAbsMax (both checked exhaustively
//    on the host, tests/support/gelu_shape_check.cpp).  So over a set of
//    pre-activations whose largest value xmax has gelu(xmax) >= that bound,
//    the absmax of the outputs is gelu(xmax), and any other set whose
//    gelu(xmax) is below the bound cannot exceed it.  (Below 0 the f32 GELU
//    is not monotonic on either side of its minimum: rounding in 1 + tanh
//    makes it wiggle, so no such shortcut exists for negative values.)
//  * quantization: gelu_approx(x) is within kGeluApproxRel * |x| +
//    kGeluApproxAbs of gelu(x) for every finite x (checked on the device for
//    all 2^32 inputs, tests/support/devmath_gpu_check.hip).  Rounding
//    fl(v * inv) half away from zero is monotonic in v, so when the whole
//    interval around gelu_approx(x) rounds to one integer, that integer is
//    the exact value's; otherwise the exact GELU is evaluated.
constexpr float kGeluNegAbsMax = 0x1.5c3e58p-3f;  // |gelu(-0x1.8138e0p-1)|, the largest over x < 0
constexpr float kGeluApproxRel = 0x1p-21f;        // bound on |gelu_approx(x) - gelu(x)| / |x|
constexpr float kGeluApproxAbs = 0x1p-126f;       // plus this absolute term (subnormal results)

#if defined(__HIPCC__)
// x * sigmoid(2u) = 0.5 x (1 + tanh(u)) with u = sqrt(2/pi) (x + 0.044715 x^3)
// written as u = x (c1 + c3 x^2), exp(-2u) = 2^(x (k1 + k3 x^2)), by the
// hardware exp2 and reciprocal.  Device only: the bound is a property of
// those instructions.
__device__ __forceinline__ float gelu_approx(float x) {
  const float x2 = x * x;
  const float p = __builtin_fmaf(-0.10294324f, x2, -2.3022084f);  // -2 log2(e) c1 (0.044715, 1), c1 = 0.7978846
  const float e = __builtin_amdgcn_exp2f(x * p);
  return x * __builtin_amdgcn_rcpf(1.0f + e);
}
#endif

RG_HD float act_apply(int act, float p, float x) {
  switch (act) {
    case ACT_RELU: return relu(x);
    case ACT_SIGMOID: return sigmoid(x);
    case ACT_TANH: return tanhf_fast(x);
    case ACT_GELU: return gelu_fast(x);
    case ACT_LEAKY_RELU: return x > 0.0f ? x : p * x;
    case ACT_SILU: { float s = sigmoid(x); return x * s; }
    default: return x;
  }
}

// QuantTensor scale rule (src/inference/quantize.rs:19-21):
// scale = max_abs < 1e-12 ? 1 : max_abs / 127, inv = 1 / scale.
RG_HD float scale_from_absmax(float max_abs) { return max_abs < 1e-12f ? 1.0f : max_abs / 127.0f; }

// (v * inv).round().clamp(-127, 127) as i8 (quantize.rs:22): half away from
// zero, NaN -> 0.
RG_HD int8_t quantize_one(float v, float inv) {
  float t = __builtin_roundf(v * inv);
  t = t < -127.0f ? -127.0f : t;
  t = t > 127.0f ? 127.0f : t;
  if (t != t) return 0;
  return (int8_t)(int)t;
}

// quantize_one's integer for t = v * inv in fewer operations (the fused
// requantization's form): s = t + copysign(0.5 - 2^-25, t), rounded to f32,
// then truncated toward zero, is round-half-away(t) for every t.  The
// addition is exact or rounds to the correct side of each integer boundary;
// checked on all 2^32 inputs on the host (tests/support/quant_host_check.cpp).
// The conversion saturates and maps NaN to 0 (the device's v_cvt_i32_f32;
// restated on the host), and the clamp to +-127 is done on the integer.
RG_HD int32_t quantize_rz(float t) {
  const float s = t + __builtin_copysignf(bitsf(0x3effffffu), t);
#if defined(__HIP_DEVICE_COMPILE__)
  int32_t i;
  asm("v_cvt_i32_f32 %0, %1" : "=v"(i) : "v"(s));
#else
  const int32_t i = s != s ? 0 : (s >= 2147483648.0f ? 2147483647 : (s <= -2147483648.0f ? (-2147483647 - 1) : (int32_t)s));
#endif
  return i < -127 ? -127 : (i > 127 ? 127 : i);
}

// quantize_rz without the clamp, for t = v * inv with |v| at most the absmax
// the scale was taken from (a tensor quantized with its own absmax): with
// scale = fl(absmax / 127) and inv = fl(1 / scale), |t| <= 127 (1 + 3 * 2^-24)
// < 127.5, so the rounded integer is already within +-127 (checked for every
// finite absmax by tests/support/quant_host_check.cpp).  NaN gives 0.
RG_HD int32_t quantize_rz_bounded(float t) {
  const float s = t + __builtin_copysignf(bitsf(0x3effffffu), t);
#if defined(__HIP_DEVICE_COMPILE__)
  int32_t i;
  asm("v_cvt_i32_f32 %0, %1" : "=v"(i) : "v"(s));
  return i;
#else
  return s != s ? 0 : (int32_t)s;
#endif
}

// round_fp16 (quantize.rs:50-64): half an ulp added to the magnitude, then
// the low 13 mantissa bits cleared (ties away from zero); exponents below
// -14 give +0 and above 15 give +-65504 (NaN and inf included).  The
// exponent is read before rounding, so [65520, 65536) gives 65536.
RG_HD float round_fp16(float x) {
  const uint32_t bits = fbits(x);
  const int32_t e = (int32_t)((bits >> 23) & 0xffu) - 127;
  const uint32_t r = e > 15 ? ((bits & 0x80000000u) | 0x477fe000u) : ((bits + (1u << 12)) & ~0x1fffu);
  return e < -14 ? 0.0f : bitsf(r);
}

// IEEE binary16 bits of a round_fp16 result (exact: 10 mantissa bits and an
// exponent in [-14, 15]), except +-65536, which binary16 cannot hold and
// which saturates to +-65504.
RG_HD uint16_t fp16_bits(float r) {
  const uint32_t b = fbits(r);
  const uint32_t sign = (b >> 16) & 0x8000u;
  const uint32_t mag = b & 0x7fffffffu;
  if (mag == 0) return (uint16_t)sign;
  if (mag >= 0x47800000u) return (uint16_t)(sign | 0x7bffu);
  return (uint16_t)(sign | (((mag >> 23) - 112u) << 10) | ((mag >> 13) & 0x3ffu));
}

// |v| as an ordered integer for atomicMax; NaN is ignored (f32::max).
RG_HD uint32_t absmax_key(float v) {
  uint32_t b = fbits(v) & 0x7fffffffu;
  return b > 0x7f800000u ? 0u : b;
}

}  // namespace rgmath
