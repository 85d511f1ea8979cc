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
// exp_neg_fast is NOT bit-compatible with Math.exp: it is the throughput
// exponential the streaming kernels use for partial softmax sums
// (2^(j/64) table + degree-5 polynomial, ~2 ulp), whose result only enters
// the normaliser, never an ordering.
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

// 2^(j/64), j = 0..63, correctly rounded.
#define GSM_EXP2_TABLE_64                                                                     \
  0x1.0000000000000p+0, 0x1.02c9a3e778061p+0, 0x1.059b0d3158574p+0, 0x1.0874518759bc8p+0,   \
  0x1.0b5586cf9890fp+0, 0x1.0e3ec32d3d1a2p+0, 0x1.11301d0125b51p+0, 0x1.1429aaea92de0p+0,   \
  0x1.172b83c7d517bp+0, 0x1.1a35beb6fcb75p+0, 0x1.1d4873168b9aap+0, 0x1.2063b88628cd6p+0,   \
  0x1.2387a6e756238p+0, 0x1.26b4565e27cddp+0, 0x1.29e9df51fdee1p+0, 0x1.2d285a6e4030bp+0,   \
  0x1.306fe0a31b715p+0, 0x1.33c08b26416ffp+0, 0x1.371a7373aa9cbp+0, 0x1.3a7db34e59ff7p+0,   \
  0x1.3dea64c123422p+0, 0x1.4160a21f72e2ap+0, 0x1.44e086061892dp+0, 0x1.486a2b5c13cd0p+0,   \
  0x1.4bfdad5362a27p+0, 0x1.4f9b2769d2ca7p+0, 0x1.5342b569d4f82p+0, 0x1.56f4736b527dap+0,   \
  0x1.5ab07dd485429p+0, 0x1.5e76f15ad2148p+0, 0x1.6247eb03a5585p+0, 0x1.6623882552225p+0,   \
  0x1.6a09e667f3bcdp+0, 0x1.6dfb23c651a2fp+0, 0x1.71f75e8ec5f74p+0, 0x1.75feb564267c9p+0,   \
  0x1.7a11473eb0187p+0, 0x1.7e2f336cf4e62p+0, 0x1.82589994cce13p+0, 0x1.868d99b4492edp+0,   \
  0x1.8ace5422aa0dbp+0, 0x1.8f1ae99157736p+0, 0x1.93737b0cdc5e5p+0, 0x1.97d829fde4e50p+0,   \
  0x1.9c49182a3f090p+0, 0x1.a0c667b5de565p+0, 0x1.a5503b23e255dp+0, 0x1.a9e6b5579fdbfp+0,   \
  0x1.ae89f995ad3adp+0, 0x1.b33a2b84f15fbp+0, 0x1.b7f76f2fb5e47p+0, 0x1.bcc1e904bc1d2p+0,   \
  0x1.c199bdd85529cp+0, 0x1.c67f12e57d14bp+0, 0x1.cb720dcef9069p+0, 0x1.d072d4a07897cp+0,   \
  0x1.d5818dcfba487p+0, 0x1.da9e603db3285p+0, 0x1.dfc97337b9b5fp+0, 0x1.e502ee78b3ff6p+0,   \
  0x1.ea4afa2a490dap+0, 0x1.efa1bee615a27p+0, 0x1.f50765b6e4540p+0, 0x1.fa7c1819e90d8p+0

// e^x for x <= 0 with ~2 ulp error; `tab` is GSM_EXP2_TABLE_64.
// x = (64k + j) ln2/64 + r, |r| <= ln2/128, e^r by its degree-5 Taylor
// polynomial (truncation < 4e-17 relative), then scale by 2^(j/64) and 2^k.
GS_HD double exp_neg_fast(double x, const double* tab) {
  if (!(x > -745.0)) return 0.0;  // also maps NaN to 0; callers test finiteness first
  const double kInvLn2x64 = 0x1.71547652b82fep+6;
  const double kLn2d64Hi = 0x1.62e42fee00000p-7;
  const double kLn2d64Lo = 0x1.a39ef35793c76p-39;
  const double n = __builtin_rint(x * kInvLn2x64);
  double r = __builtin_fma(-n, kLn2d64Hi, x);
  r = __builtin_fma(-n, kLn2d64Lo, r);
  double p = __builtin_fma(r, 1.0 / 120.0, 1.0 / 24.0);
  p = __builtin_fma(r, p, 1.0 / 6.0);
  p = __builtin_fma(r, p, 0.5);
  p = __builtin_fma(r, p, 1.0);
  p = r * p;
  const int ni = (int)n;
  const double t = tab[ni & 63];
  const double y = __builtin_fma(t, p, t);
  const int e = ni >> 6;  // floor division, e in [-1075, 0]
  if (e >= -1022) return y * double_of((uint64_t)(e + 1023) << 52);
  return (y * double_of((uint64_t)(e + 1023 + 200) << 52)) * double_of((uint64_t)(1023 - 200) << 52);
}

}  // namespace gsm
