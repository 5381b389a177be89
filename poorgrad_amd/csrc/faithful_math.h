// Host-libm-faithful single-precision transcendentals for the exact posture.
//
// The reference interpreter computes `exp`, `ln` and `tanh` of an `f32` by
// calling the host C library (`src/payload/elementary.rs:117-135`: Rust's
// `f32::exp/ln/tanh` lower to `expf/logf/tanhf`). Bit identity with the
// interpreter therefore means bit identity with the host glibc (2.35 on this
// image), including its x86-64 ifunc choice: on a CPU with FMA, glibc runs the
// `-mfma` build of `expf`/`logf`, in which GCC contracted several
// multiply-adds into fused ones. The functions below restate those published
// algorithms with every contraction spelled out as an explicit `fma`, so one
// source compiles to the same bits with g++ on the host and hipcc on gfx950
// (both with -ffp-contract=off):
//
//   expf  — ARM optimized-routines `expf` (glibc sysdeps/ieee754/flt-32/e_expf.c
//           since 2.27): 2^(k/32) table lookup plus a cubic in double.
//   logf  — ARM optimized-routines `logf` (e_logf.c): 16-interval table of
//           (1/c, log c) plus a cubic in double.
//   powf  — ARM optimized-routines `powf` (e_powf.c since 2.27): log2 x from the
//           same 16 subintervals (1/c, log2 c) and a quintic in double, times
//           y in double, then 2^(y log2 x) from the exp table and a cubic.
//   tanhf — fdlibm `tanhf` over fdlibm `expm1f` (s_tanhf.c, s_expm1f.c), pure
//           single precision, built without FMA in glibc.
//
// Notices of the restated sources. ARM optimized-routines (the expf/logf
// algorithms and their tables) is Copyright (c) 2017-2018 Arm Limited,
// distributed under the MIT License or the Apache License 2.0 with LLVM
// exception (SPDX: MIT OR Apache-2.0 WITH LLVM-exception), as contributed to
// glibc. fdlibm (tanhf, expm1f): "Copyright (C) 1993 by Sun Microsystems, Inc.
// All rights reserved. Developed at SunPro, a Sun Microsystems, Inc. business.
// Permission to use, copy, modify, and distribute this software is freely
// granted, provided that this notice is preserved."
//
// Each function is checked against the host glibc on every one of the 2^32
// single-precision inputs (tests/native/faithful_check.cpp, run by the CPU tests),
// and the device build is checked the same way on the GPU.
#pragma once
#if defined(__HIPCC_RTC__)
// Generated chain kernels include this text through hipRTC, which has no C
// library headers.
typedef unsigned int uint32_t;
typedef int int32_t;
typedef unsigned long long uint64_t;
#ifndef __HIPCC__
#define __HIPCC__ 1
#endif
#else
#include <stdint.h>
#endif

#if defined(__HIPCC__)
#define TOPOS_HD __host__ __device__ inline
#else
#define TOPOS_HD inline
#endif

namespace topos_faithful {

TOPOS_HD uint32_t bits_of(float value) { return __builtin_bit_cast(uint32_t, value); }
TOPOS_HD float float_of(uint32_t bits) { return __builtin_bit_cast(float, bits); }
TOPOS_HD uint64_t bits_of(double value) { return __builtin_bit_cast(uint64_t, value); }
TOPOS_HD double double_of(uint64_t bits) { return __builtin_bit_cast(double, bits); }

// exp: bits(RN(2^(i/32))) - (i << 52) / 32 for i in 0..32. Derivable from the
// definition alone (tests/native/faithful_check.cpp recomputes every entry in
// extended precision and compares).
#if defined(__HIPCC__)
static __device__ __constant__ uint64_t kExpTableDevice[32] = {
#else
static const uint64_t kExpTableHost[32] = {
#endif
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

// logf: for the 16 subintervals of [0x3f330000, 2 * 0x3f330000), the double
// 1/c and RN(log c) of a point c near the subinterval's centre (logc equals
// RN(-log(invc)) for every row; the check recomputes it).
struct LogRow {
  double invc, logc;
};
#if defined(__HIPCC__)
static __device__ __constant__ LogRow kLogTableDevice[16] = {
#else
static const LogRow kLogTableHost[16] = {
#endif
    {0x1.661ec79f8f3bep+0, -0x1.57bf7808caadep-2}, {0x1.571ed4aaf883dp+0, -0x1.2bef0a7c06ddbp-2},
    {0x1.49539f0f010bp+0, -0x1.01eae7f513a67p-2},  {0x1.3c995b0b80385p+0, -0x1.b31d8a68224e9p-3},
    {0x1.30d190c8864a5p+0, -0x1.6574f0ac07758p-3}, {0x1.25e227b0b8eap+0, -0x1.1aa2bc79c81p-3},
    {0x1.1bb4a4a1a343fp+0, -0x1.a4e76ce8c0e5ep-4}, {0x1.12358f08ae5bap+0, -0x1.1973c5a611cccp-4},
    {0x1.0953f419900a7p+0, -0x1.252f438e10c1ep-5}, {0x1p+0, 0x0p+0},
    {0x1.e608cfd9a47acp-1, 0x1.aa5aa5df25984p-5},  {0x1.ca4b31f026aap-1, 0x1.c5e53aa362eb4p-4},
    {0x1.b2036576afce6p-1, 0x1.526e57720db08p-3},  {0x1.9c2d163a1aa2dp-1, 0x1.bc2860d22477p-3},
    {0x1.886e6037841edp-1, 0x1.1058bc8a07ee1p-2},  {0x1.767dcf5534862p-1, 0x1.4043057b6ee09p-2},
};

// powf's log2: the same 1/c column, and RN(log2 c) = RN(-log2(invc)) (the check
// recomputes it).
#if defined(__HIPCC__)
static __device__ __constant__ LogRow kLog2TableDevice[16] = {
#else
static const LogRow kLog2TableHost[16] = {
#endif
    {0x1.661ec79f8f3bep+0, -0x1.efec65b963019p-2}, {0x1.571ed4aaf883dp+0, -0x1.b0b6832d4fca4p-2},
    {0x1.49539f0f010bp+0, -0x1.7418b0a1fb77bp-2},  {0x1.3c995b0b80385p+0, -0x1.39de91a6dcf7bp-2},
    {0x1.30d190c8864a5p+0, -0x1.01d9bf3f2b631p-2}, {0x1.25e227b0b8eap+0, -0x1.97c1d1b3b7afp-3},
    {0x1.1bb4a4a1a343fp+0, -0x1.2f9e393af3c9fp-3}, {0x1.12358f08ae5bap+0, -0x1.960cbbf788d5cp-4},
    {0x1.0953f419900a7p+0, -0x1.a6f9db6475fcep-5}, {0x1p+0, 0x0p+0},
    {0x1.e608cfd9a47acp-1, 0x1.338ca9f24f53dp-4},  {0x1.ca4b31f026aap-1, 0x1.476a9543891bap-3},
    {0x1.b2036576afce6p-1, 0x1.e840b4ac4e4d2p-3},  {0x1.9c2d163a1aa2dp-1, 0x1.40645f0c6651cp-2},
    {0x1.886e6037841edp-1, 0x1.88e9c2c1b9ff8p-2},  {0x1.767dcf5534862p-1, 0x1.ce0a44eb17bccp-2},
};

#if defined(__HIPCC__)
#define TOPOS_EXP_TABLE kExpTableDevice
#define TOPOS_LOG_TABLE kLogTableDevice
#define TOPOS_LOG2_TABLE kLog2TableDevice
#else
#define TOPOS_EXP_TABLE kExpTableHost
#define TOPOS_LOG_TABLE kLogTableHost
#define TOPOS_LOG2_TABLE kLog2TableHost
#endif

// e^x. Reduction x * 32/ln2 = k + r, |r| <= 1/2, with k rounded by the
// 1.5 * 2^52 shift; 2^(k/32) = table[k mod 32] with k/32 added to the exponent
// field; 2^(r/32) by a cubic. The product x * 32/ln2 is fused into both the
// shift addition and the remainder subtraction, as the FMA build of glibc does.
// glibc's special cases need no branch and no select but NaN's: the argument
// is clamped to [-104, 89] first, and the arithmetic itself gives glibc's
// values beyond its thresholds. Above 0x1.62e42ep6 (the largest f32 whose
// e^x stays below 2^128) the next f32 already has e^x > 2^128 (1 + 2.4e-7),
// and e^89, so the double rounds to +inf (e^+inf = +inf). Below -0x1.9fe368p6
// the next f32 has e^x < 2^-150 (1 - 7e-6), and e^-104 < 2^-150, so it rounds
// to +0 (e^-inf = +0). The double's relative error (below 2^-40) is far inside
// both margins. A NaN argument gives x + x, the quieted NaN, as glibc does;
// the arithmetic on it stays harmless (the table index is still k mod 32).
TOPOS_HD float exp_f32_table(float x, const uint64_t *table) {
  const double inv_ln2_scaled = 0x1.71547652b82fep+0 * 32;
  const double shift = 0x1.8p+52;
  const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
  const double c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
  const double c2 = 0x1.62e42ff0c52d6p-1 / 32;
#if defined(__HIP_DEVICE_COMPILE__) || defined(__HIPCC_RTC__)
  const float clamped = __builtin_amdgcn_fmed3f(x, -104.0f, 89.0f);
#else
  const float clamped = x < -104.0f ? -104.0f : (x > 89.0f ? 89.0f : x);
#endif
  const double xd = (double)clamped;
  double kd = __builtin_fma(inv_ln2_scaled, xd, shift);
  const uint32_t k = (uint32_t)bits_of(kd);  // k mod 2^32: the low word of the shifted sum
  kd -= shift;
  const double r = __builtin_fma(inv_ln2_scaled, xd, -kd);
  // table[k mod 32] + (k << 47): the shifted k has a zero low word, so only
  // the entry's high word changes, by (k << 15) mod 2^32.
  const uint64_t entry = table[k % 32];
  const uint32_t s_low = (uint32_t)entry, s_high = (uint32_t)(entry >> 32) + (k << 15);
#if defined(__HIP_DEVICE_COMPILE__) || defined(__HIPCC_RTC__)
  typedef uint32_t word_pair __attribute__((ext_vector_type(2)));
  const double s = __builtin_bit_cast(double, word_pair{s_low, s_high});
#else
  const double s = double_of((uint64_t)s_high << 32 | s_low);
#endif
  const double z = __builtin_fma(c0, r, c1);
  const double r2 = r * r;
  double y = __builtin_fma(c2, r, 1.0);
  y = __builtin_fma(z, r2, y);
  y = y * s;
  const float result = (float)y, quiet = x + x;
  return x != x ? quiet : result;
}

// e^x with the built-in table (a kernel may pass a copy it keeps in LDS).
TOPOS_HD float exp_f32(float x) { return exp_f32_table(x, TOPOS_EXP_TABLE); }

// ln x. x = 2^k z with z in [0x3f330000, 2 * 0x3f330000); the top four
// mantissa bits of z pick c; ln x = log1p(z/c - 1) + ln c + k ln2 with a cubic
// for log1p, evaluated with the fused multiply-adds of glibc's FMA build.
TOPOS_HD float ln_f32_table(float x, const LogRow *table) {
  const double ln2 = 0x1.62e42fefa39efp-1;
  const double a0 = -0x1.00ea348b88334p-2, a1 = 0x1.5575b0be00b6ap-2, a2 = -0x1.ffffef20a4123p-2;
  uint32_t ix = bits_of(x);
  if (ix == 0x3f800000u) return 0.0f;  // ln 1 = +0 in every rounding mode
  if (ix - 0x00800000u >= 0x7f800000u - 0x00800000u) {
    if (ix * 2 == 0) return float_of(0xff800000u);  // ln(+-0) = -inf
    if (ix == 0x7f800000u) return x;               // ln(inf) = inf
    if ((ix & 0x80000000u) || ix * 2 >= 0xff000000u) {
      // Negative or NaN: the invalid result, (x - x) / (x - x).
      const float d = x - x;
      return d / d;
    }
    ix = bits_of(x * 0x1p23f);  // subnormal: normalise
    ix -= 23u << 23;
  }
  const uint32_t tmp = ix - 0x3f330000u;
  const int i = (int)((tmp >> (23 - 4)) % 16);
  const int k = (int32_t)tmp >> 23;
  const uint32_t iz = ix - (tmp & 0xff800000u);
  const double invc = table[i].invc;
  const double logc = table[i].logc;
  const double z = (double)float_of(iz);
  const double r = __builtin_fma(z, invc, -1.0);
  const double y0 = __builtin_fma((double)k, ln2, logc);
  const double r2 = r * r;
  double y = __builtin_fma(a1, r, a2);
  y = __builtin_fma(a0, r2, y);
  y = __builtin_fma(y, r2, y0 + r);
  return (float)y;
}

TOPOS_HD float ln_f32(float x) { return ln_f32_table(x, TOPOS_LOG_TABLE); }

// e^x - 1 in single precision (fdlibm): reduce by k ln2 with a hi/lo split
// of ln2, rational approximation on the primary range, then rescale.
TOPOS_HD float expm1_f32(float x) {
  const float one = 1.0f, huge = 1.0e+30f, tiny = 1.0e-30f;
  const float o_threshold = 8.8721679688e+01f;
  const float ln2_hi = 6.9313812256e-01f, ln2_lo = 9.0580006145e-06f;
  const float invln2 = 1.4426950216e+00f;
  const float q1 = -3.3333335072e-02f, q2 = 1.5873016091e-03f, q3 = -7.9365076090e-05f,
              q4 = 4.0082177293e-06f, q5 = -2.0109921195e-07f;
  float hi, lo, c = 0.0f, t, e, hxs, hfx, r1, y;
  int32_t k;
  uint32_t hx = bits_of(x);
  const uint32_t negative = hx & 0x80000000u;
  hx &= 0x7fffffffu;
  if (hx >= 0x4195b844u) {  // |x| >= 27 ln2
    if (hx >= 0x42b17218u) {
      if (hx > 0x7f800000u) return x + x;  // NaN
      if (hx == 0x7f800000u) return negative == 0 ? x : -1.0f;
      if (x > o_threshold) return huge * huge;  // overflow
    }
    if (negative != 0) return tiny - one;  // x < -27 ln2: -1 (inexact)
  }
  if (hx > 0x3eb17218u) {  // |x| > ln2 / 2
    if (hx < 0x3f851592u) {  // and |x| < 3 ln2 / 2
      if (negative == 0) {
        hi = x - ln2_hi;
        lo = ln2_lo;
        k = 1;
      } else {
        hi = x + ln2_hi;
        lo = -ln2_lo;
        k = -1;
      }
    } else {
      k = (int32_t)(invln2 * x + (negative == 0 ? 0.5f : -0.5f));
      t = (float)k;
      hi = x - t * ln2_hi;
      lo = t * ln2_lo;
    }
    x = hi - lo;
    c = (hi - x) - lo;
  } else if (hx < 0x33000000u) {  // |x| < 2^-25: x itself
    t = huge + x;
    return x - (t - (huge + x));
  } else {
    k = 0;
  }
  hfx = 0.5f * x;
  hxs = x * hfx;
  r1 = one + hxs * (q1 + hxs * (q2 + hxs * (q3 + hxs * (q4 + hxs * q5))));
  t = 3.0f - r1 * hfx;
  e = hxs * ((r1 - t) / (6.0f - x * t));
  if (k == 0) return x - (x * e - hxs);
  e = (x * (e - c) - c);
  e -= hxs;
  if (k == -1) return 0.5f * (x - e) - 0.5f;
  if (k == 1) {
    if (x < -0.25f) return -2.0f * (e - (x + 0.5f));
    return one + 2.0f * (x - e);
  }
  if (k <= -2 || k > 56) {
    y = one - (e - x);
    if (k == 128)
      y = y * 2.0f * 0x1p127f;
    else
      y = float_of(bits_of(y) + ((uint32_t)k << 23));
    return y - one;
  }
  if (k < 23) {
    t = float_of(0x3f800000u - (0x1000000u >> k));  // 1 - 2^-k
    y = t - (e - x);
  } else {
    t = float_of((uint32_t)(0x7f - k) << 23);  // 2^-k
    y = x - (e + t);
    y += one;
  }
  return float_of(bits_of(y) + ((uint32_t)k << 23));
}

// tanh x (fdlibm): sign-symmetric, through expm1 of -2|x| below one and of
// 2|x| above, saturating to +-1 from 22.
TOPOS_HD float tanh_f32(float x) {
  const float one = 1.0f, two = 2.0f, tiny = 1.0e-30f;
  const int32_t jx = (int32_t)bits_of(x);
  const int32_t ix = jx & 0x7fffffff;
  float t, z;
  if (ix >= 0x7f800000) {  // inf or NaN
    return jx >= 0 ? one / x + one : one / x - one;
  }
  if (ix < 0x41b00000) {  // |x| < 22
    if (ix == 0) return x;
    if (ix < 0x24000000) return x * (one + x);  // |x| < 2^-55
    const float ax = __builtin_fabsf(x);
    // One expm1 for both ranges (its argument and the quotient selected per
    // lane), so lanes of a wave on either side of 1 share one evaluation.
    const bool large = ix >= 0x3f800000;
    t = expm1_f32(large ? two * ax : -two * ax);
    const float q = (large ? two : -t) / (t + two);
    z = large ? one - q : q;
  } else {
    z = one - tiny;
  }
  return jx >= 0 ? z : -z;
}

// Whether a non-zero finite f32 (by its bits) is an integer: 0 if not, 1 if
// odd, 2 if even.
TOPOS_HD int pow_integer_class(uint32_t iy) {
  const int e = (int)(iy >> 23 & 0xff);
  if (e < 0x7f) return 0;
  if (e > 0x7f + 23) return 2;
  if (iy & ((1u << (0x7f + 23 - e)) - 1)) return 0;
  if (iy & (1u << (0x7f + 23 - e))) return 1;
  return 2;
}

// Whether an f32 (by its bits) is zero, infinite or NaN.
TOPOS_HD bool pow_zero_inf_nan(uint32_t i) { return 2 * i - 1 >= 2u * 0x7f800000u - 1; }

// x^y. log2 x = k + log2 c + log1p(z/c - 1)/ln 2 (x = 2^k z, z in
// [0x3f330000, 2 * 0x3f330000), c from the top four mantissa bits of z) with a
// quintic for log1p(r)/ln 2; y log2 x rounded to double; 2^(y log2 x) =
// 2^(k'/32) 2^r by the exp table and a cubic, the result's sign folded into
// the table entry's exponent. The multiply-adds are fused as in glibc's FMA
// build. Special cases follow glibc: y = +-0 or x = 1 give 1 (NaN included);
// NaN operands propagate; |x| = 1 with y = +-inf gives 1; 0 and inf bases
// square through; a finite negative base needs an integer exponent (else
// NaN), an odd one carrying the sign; overflow gives +-inf and underflow
// +-0, with the sign of the result.
TOPOS_HD float pow_f32_tables(float x, float y, const LogRow *log2_table, const uint64_t *exp_table) {
  const double a0 = 0x1.27616c9496e0bp-2, a1 = -0x1.71969a075c67ap-2, a2 = 0x1.ec70a6ca7baddp-2,
               a3 = -0x1.7154748bef6c8p-1, a4 = 0x1.71547652ab82bp0;
  const double c0 = 0x1.c6af84b912394p-5, c1 = 0x1.ebfce50fac4f3p-3, c2 = 0x1.62e42ff0c52d6p-1;
  const double shift = 0x1.8p+52 / 32;
  uint32_t sign_bias = 0;
  uint32_t ix = bits_of(x);
  const uint32_t iy = bits_of(y);
  if (ix - 0x00800000u >= 0x7f800000u - 0x00800000u || pow_zero_inf_nan(iy)) {
    // x subnormal, zero, negative, infinite or NaN; or y zero, infinite or NaN.
    if (pow_zero_inf_nan(iy)) {
      if (2 * iy == 0) return (ix & 0x7fc00000u) == 0x7f800000u && (ix & 0x003fffffu) ? x + y : 1.0f;
      if (ix == 0x3f800000u) return (iy & 0x7fc00000u) == 0x7f800000u && (iy & 0x003fffffu) ? x + y : 1.0f;
      if (2 * ix > 2u * 0x7f800000u || 2 * iy > 2u * 0x7f800000u) return x + y;
      if (2 * ix == 2u * 0x3f800000u) return 1.0f;
      if ((2 * ix < 2u * 0x3f800000u) == !(iy & 0x80000000u)) return 0.0f;  // |x| < 1, y = inf; |x| > 1, y = -inf
      return y * y;
    }
    if (pow_zero_inf_nan(ix)) {
      float x2 = x * x;
      if ((ix & 0x80000000u) && pow_integer_class(iy) == 1) x2 = -x2;
      return (iy & 0x80000000u) ? 1.0f / x2 : x2;
    }
    // x and y are non-zero finite.
    if (ix & 0x80000000u) {
      const int yint = pow_integer_class(iy);
      if (yint == 0) {
        const float d = x - x;  // the invalid result, (x - x) / (x - x)
        return d / d;
      }
      if (yint == 1) sign_bias = 1u << (5 + 11);
      ix &= 0x7fffffffu;
    }
    if (ix < 0x00800000u) {  // subnormal x: normalise, the exponent goes negative
      ix = bits_of(x * 0x1p23f);
      ix &= 0x7fffffffu;
      ix -= 23u << 23;
    }
  }
  // log2 x.
  const uint32_t tmp = ix - 0x3f330000u;
  const int i = (int)((tmp >> (23 - 4)) % 16);
  const uint32_t top = tmp & 0xff800000u;
  const uint32_t iz = ix - top;
  const int k = (int32_t)top >> 23;
  const double invc = log2_table[i].invc;
  const double logc = log2_table[i].logc;
  const double z = (double)float_of(iz);
  const double r = __builtin_fma(z, invc, -1.0);
  const double y0 = logc + (double)k;
  const double r2 = r * r;
  double p = __builtin_fma(a0, r, a1);
  const double q0 = __builtin_fma(a2, r, a3);
  const double r4 = r2 * r2;
  double q = __builtin_fma(a4, r, y0);
  q = __builtin_fma(q0, r2, q);
  const double logx = __builtin_fma(p, r4, q);
  const double ylogx = (double)y * logx;
  if ((bits_of(ylogx) >> 47 & 0xffff) >= bits_of(126.0) >> 47) {
    // |y log2 x| >= 126.
    if (ylogx > 0x1.fffffffd1d571p+6) return sign_bias ? -float_of(0x7f800000u) : float_of(0x7f800000u);
    if (ylogx <= -150.0) return sign_bias ? -0.0f : 0.0f;
  }
  // 2^ylogx.
  double kd = ylogx + shift;
  const uint64_t ki = bits_of(kd);
  kd -= shift;
  const double rr = ylogx - kd;
  uint64_t t = exp_table[ki % 32];
  const uint64_t ski = ki + sign_bias;
  t += ski << (52 - 5);
  const double s = double_of(t);
  const double zz = __builtin_fma(c0, rr, c1);
  const double rr2 = rr * rr;
  double yy = __builtin_fma(c2, rr, 1.0);
  yy = __builtin_fma(zz, rr2, yy);
  yy = yy * s;
  return (float)yy;
}

TOPOS_HD float pow_f32(float x, float y) { return pow_f32_tables(x, y, TOPOS_LOG2_TABLE, TOPOS_EXP_TABLE); }

// Rust's f32::max as compiled for x86-64 (llvm.maxnum): a NaN operand loses
// to the other, and a tie between +0 and -0 answers the first operand.
TOPOS_HD float max_f32(float a, float b) {
  if (a != a) return b;
  if (b != b) return a;
  return b > a ? b : a;
}

// The Heaviside step of `src/payload/elementary.rs:141-143`: one where
// x >= threshold (ties answer one), else zero; NaN compares false.
TOPOS_HD float step_f32(float x, float threshold) { return x >= threshold ? 1.0f : 0.0f; }

}  // namespace topos_faithful
