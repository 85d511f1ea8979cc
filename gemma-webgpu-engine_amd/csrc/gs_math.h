// Scalar math shared by the gfx950 kernels and the host code of libgsample.
//
// js_exp / js_log reproduce the JavaScript engine's Math.exp / Math.log bit
// for bit (the reference sampler calls them at src/runtime/sampling.ts:39,
// 50,51,77,79). V8 implements both with the fdlibm method (Sun fdlibm 5.3,
// e_exp.c / e_log.c): exp reduces x = k*ln2 + r and evaluates
// 1 + r + r*c/(2-c) with a degree-5 Remez polynomial c(r^2); log reduces
// x = 2^k*(1+f) and evaluates the series in s = f/(2+f). Only IEEE binary64
// + - * / are used, and this file is compiled with -ffp-contract=off, so GPU
// and CPU round every step identically.
//
// mulberry32_draw is SeededRandom.next() (src/runtime/sampling.ts:3-16) as a
// counter-based function of (seed, draw number).
//
// The exp and log routines restate fdlibm's published method and carry its
// notice:
//   ====================================================
//   Copyright (C) 1993 by Sun Microsystems, Inc. All rights reserved.
//   (e_exp.c: Copyright (C) 2004 by Sun Microsystems, Inc.)
//
//   Developed at SunSoft, a Sun Microsystems, Inc. business.
//   Permission to use, copy, modify, and distribute this
//   software is freely granted, provided that this notice
//   is preserved.
//   ====================================================

#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define GS_HD __host__ __device__ __forceinline__
#else
#define GS_HD static inline
#endif

namespace gsm {

GS_HD uint64_t bits_of(double x) { return __builtin_bit_cast(uint64_t, x); }
GS_HD double double_of(uint64_t u) { return __builtin_bit_cast(double, u); }
GS_HD int32_t high_word(double x) { return (int32_t)(bits_of(x) >> 32); }
GS_HD uint32_t low_word(double x) { return (uint32_t)bits_of(x); }
GS_HD double with_high_word(double x, int32_t hi) {
  return double_of(((uint64_t)(uint32_t)hi << 32) | (bits_of(x) & 0xffffffffull));
}

GS_HD double js_exp(double x) {
  const double kLn2Hi = 6.93147180369123816490e-01;
  const double kLn2Lo = 1.90821492927058770002e-10;
  const double kInvLn2 = 1.44269504088896338700e+00;
  const double kP1 = 1.66666666666666019037e-01;
  const double kP2 = -2.77777777770155933842e-03;
  const double kP3 = 6.61375632143793436117e-05;
  const double kP4 = -1.65339022054652515390e-06;
  const double kP5 = 4.13813679705723846039e-08;
  const double kOverflow = 7.09782712893383973096e+02;
  const double kUnderflow = -7.45133219101941108420e+02;
  const double kTwoM1000 = 9.33263618503218878990e-302;
  const double kHuge = 1.0e300;

  int32_t hx = high_word(x);
  const bool neg = hx < 0;
  hx &= 0x7fffffff;
  double hi = 0.0, lo = 0.0;
  int k = 0;
  if (hx >= 0x40862E42) {
    if (hx >= 0x7ff00000) {
      if (((hx & 0xfffff) | low_word(x)) != 0) return x + x;
      return neg ? 0.0 : x;
    }
    if (x > kOverflow) return kHuge * kHuge;
    if (x < kUnderflow) return kTwoM1000 * kTwoM1000;
  }
  if (hx > 0x3fd62e42) {
    if (hx < 0x3FF0A2B2) {
      hi = neg ? x + kLn2Hi : x - kLn2Hi;
      lo = neg ? -kLn2Lo : kLn2Lo;
      k = neg ? -1 : 1;
    } else {
      k = (int)(kInvLn2 * x + (neg ? -0.5 : 0.5));
      const double t = (double)k;
      hi = x - t * kLn2Hi;
      lo = t * kLn2Lo;
    }
    x = hi - lo;
  } else if (hx < 0x3e300000) {
    if (kHuge + x > 1.0) return 1.0 + x;
  }
  const double t = x * x;
  const double c = x - t * (kP1 + t * (kP2 + t * (kP3 + t * (kP4 + t * kP5))));
  if (k == 0) return 1.0 - ((x * c) / (c - 2.0) - x);
  double y = 1.0 - ((lo - (x * c) / (2.0 - c)) - hi);
  if (k >= -1021) return with_high_word(y, high_word(y) + (k << 20));
  y = with_high_word(y, high_word(y) + ((k + 1000) << 20));
  return y * kTwoM1000;
}

GS_HD double js_log(double x) {
  const double kLn2Hi = 6.93147180369123816490e-01;
  const double kLn2Lo = 1.90821492927058770002e-10;
  const double kTwo54 = 1.80143985094819840000e+16;
  const double kLg1 = 6.666666666666735130e-01;
  const double kLg2 = 3.999999999940941908e-01;
  const double kLg3 = 2.857142874366239149e-01;
  const double kLg4 = 2.222219843214978396e-01;
  const double kLg5 = 1.818357216161805012e-01;
  const double kLg6 = 1.531383769920937332e-01;
  const double kLg7 = 1.479819860511658591e-01;
  const double kZero = 0.0;

  int32_t hx = high_word(x);
  const uint32_t lx = low_word(x);
  int k = 0;
  if (hx < 0x00100000) {
    if (((hx & 0x7fffffff) | lx) == 0) return -kTwo54 / kZero;
    if (hx < 0) return (x - x) / kZero;
    k -= 54;
    x *= kTwo54;
    hx = high_word(x);
  }
  if (hx >= 0x7ff00000) return x + x;
  k += (hx >> 20) - 1023;
  hx &= 0x000fffff;
  int32_t i = (hx + 0x95f64) & 0x100000;
  x = with_high_word(x, hx | (i ^ 0x3ff00000));
  k += (i >> 20);
  const double f = x - 1.0;
  if ((0x000fffff & (2 + hx)) < 3) {
    if (f == kZero) {
      if (k == 0) return kZero;
      const double dk = (double)k;
      return dk * kLn2Hi + dk * kLn2Lo;
    }
    const double r = f * f * (0.5 - 0.33333333333333333 * f);
    if (k == 0) return f - r;
    const double dk = (double)k;
    return dk * kLn2Hi - ((r - dk * kLn2Lo) - f);
  }
  const double s = f / (2.0 + f);
  const double dk = (double)k;
  const double z = s * s;
  i = hx - 0x6147a;
  const double w = z * z;
  const int32_t j = 0x6b851 - hx;
  const double t1 = w * (kLg2 + w * (kLg4 + w * kLg6));
  const double t2 = z * (kLg1 + w * (kLg3 + w * (kLg5 + w * kLg7)));
  i |= j;
  const double r = t2 + t1;
  if (i > 0) {
    const double hfsq = 0.5 * f * f;
    if (k == 0) return f - (hfsq - s * (hfsq + r));
    return dk * kLn2Hi - ((hfsq - (s * (hfsq + r) + dk * kLn2Lo)) - f);
  }
  if (k == 0) return f - s * (f - r);
  return dk * kLn2Hi - ((s * (f - r) - dk * kLn2Lo) - f);
}

// Math.max semantics for two doubles (NaN wins, +0 beats -0).
GS_HD double js_max(double a, double b) {
  if (a != a || b != b) return a + b;
  if (a == b) return (bits_of(a) >> 63) ? b : a;
  return a > b ? a : b;
}

constexpr uint32_t kMulberryStep = 0x6d2b79f5u;

GS_HD uint32_t mulberry32_start(int64_t seed) {
  const uint32_t s = (uint32_t)(uint64_t)seed;
  return s ? s : kMulberryStep;
}

// The `index`-th value (0 = first) of SeededRandom(seed).next().
GS_HD double mulberry32_draw(int64_t seed, uint64_t index) {
  uint32_t z = mulberry32_start(seed) + (uint32_t)((index + 1) * (uint64_t)kMulberryStep);
  z = (z ^ (z >> 15)) * (z | 1u);
  z ^= z + (z ^ (z >> 7)) * (z | 61u);
  return (double)(z ^ (z >> 14)) / 4294967296.0;
}

// Draws up to this index reproduce the JS double state exactly.
GS_HD uint64_t mulberry32_index_limit(int64_t seed) {
  return ((1ull << 53) - mulberry32_start(seed)) / kMulberryStep - 1;
}

// softcap(x) = cap * tanh(x / cap), evaluated in binary64 from js_exp and
// rounded once to binary32, so host and device agree bit for bit.
GS_HD float softcap_f32(float x, double cap) {
  const double y = (double)x / cap;
  const double a = y < 0 ? -y : y;
  double t;
  if (a > 40.0) {
    t = 1.0;
  } else if (a < 1.0e-4) {
    t = a - (a * a * a) / 3.0;  // tanh series; next term 2a^5/15 < 1e-20 relative
  } else {
    const double e = js_exp(2.0 * a);
    t = (e - 1.0) / (e + 1.0);
  }
  if (y < 0) t = -t;
  if (y != y) t = y;
  return (float)(cap * t);
}

}  // namespace gsm
