/*
 * ORACLE — test infrastructure only. Nothing in the product path may include,
 * link or call this file; only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg use it, and only as the checker.
 *
 * JavaScript-engine arithmetic that the reference sampler depends on:
 *
 *  - js_exp / js_log: the reference calls Math.exp and Math.log
 *    (src/runtime/sampling.ts:39,50,51,77,79). V8 implements both with its
 *    port of the fdlibm / FreeBSD msun routines e_exp.c and e_log.c. This is a
 *    restatement of those published methods (Sun Microsystems fdlibm 5.3:
 *    argument reduction x = k*ln2 + r, Remez rational approximation of
 *    r*(e^r+1)/(e^r-1) for exp; x = 2^k*(1+f), s = f/(2+f) series for log).
 *    Pinned by tests/test_oracle_vs_node.py against Node's own Math.exp /
 *    Math.log.
 *
 *  - mulberry32_draw: SeededRandom (src/runtime/sampling.ts:3-16). The state is
 *    an unbounded JS double advanced by 0x6d2b79f5 per draw, so the n-th draw
 *    (0-based) mixes (s0 + (n+1)*0x6d2b79f5) mod 2^32 where
 *    s0 = (seed >>> 0) || 0x6d2b79f5. Exact while s0 + (n+1)*C <= 2^53.
 *
 * All arithmetic here uses IEEE-754 binary64 basic operations only; compile
 * with -ffp-contract=off so no fused multiply-add changes a rounding. *
 * The exp and log routines restate fdlibm's published method and carry its
 * notice:
 *   ====================================================
 *   Copyright (C) 1993 by Sun Microsystems, Inc. All rights reserved.
 *   (e_exp.c: Copyright (C) 2004 by Sun Microsystems, Inc.)
 *
 *   Developed at SunSoft, a Sun Microsystems, Inc. business.
 *   Permission to use, copy, modify, and distribute this
 *   software is freely granted, provided that this notice
 *   is preserved.
 *   ====================================================
 */
#ifndef ORACLE_JSMATH_H
#define ORACLE_JSMATH_H

#include <stdint.h>
#include <string.h>

static inline uint64_t orj_bits(double x) { uint64_t u; memcpy(&u, &x, 8); return u; }
static inline double orj_from_bits(uint64_t u) { double x; memcpy(&x, &u, 8); return x; }
static inline int32_t orj_hi(double x) { return (int32_t)(orj_bits(x) >> 32); }
static inline uint32_t orj_lo(double x) { return (uint32_t)orj_bits(x); }
static inline double orj_with_hi(double x, int32_t hi) {
  return orj_from_bits(((uint64_t)(uint32_t)hi << 32) | (orj_bits(x) & 0xffffffffull));
}

/* e^x by the fdlibm method. */
static inline double js_exp(double x) {
  const double LN2_HI = 6.93147180369123816490e-01;
  const double LN2_LO = 1.90821492927058770002e-10;
  const double INV_LN2 = 1.44269504088896338700e+00;
  const double P1 = 1.66666666666666019037e-01;
  const double P2 = -2.77777777770155933842e-03;
  const double P3 = 6.61375632143793436117e-05;
  const double P4 = -1.65339022054652515390e-06;
  const double P5 = 4.13813679705723846039e-08;
  const double OVER = 7.09782712893383973096e+02;
  const double UNDER = -7.45133219101941108420e+02;
  const double TWO_M1000 = 9.33263618503218878990e-302; /* 2^-1000 */
  const double HUGE_V = 1.0e300;

  int32_t hx = orj_hi(x);
  int negative = (hx >> 31) & 1;
  hx &= 0x7fffffff;
  double hi = 0.0, lo = 0.0;
  int k = 0;

  if (hx >= 0x40862E42) {               /* |x| >= 709.78 */
    if (hx >= 0x7ff00000) {
      if (((hx & 0xfffff) | orj_lo(x)) != 0) return x + x;   /* NaN */
      return negative ? 0.0 : x;                            /* exp(+-inf) */
    }
    if (x > OVER) return HUGE_V * HUGE_V;                   /* overflow */
    if (x < UNDER) return TWO_M1000 * TWO_M1000;            /* underflow */
  }
  if (hx > 0x3fd62e42) {                /* |x| > 0.5 ln2 */
    if (hx < 0x3FF0A2B2) {              /* and |x| < 1.5 ln2 */
      hi = negative ? x + LN2_HI : x - LN2_HI;
      lo = negative ? -LN2_LO : LN2_LO;
      k = negative ? -1 : 1;
    } else {
      k = (int)(INV_LN2 * x + (negative ? -0.5 : 0.5));
      double t = (double)k;
      hi = x - t * LN2_HI;
      lo = t * LN2_LO;
    }
    x = hi - lo;
  } else if (hx < 0x3e300000) {         /* |x| < 2^-28 */
    if (HUGE_V + x > 1.0) return 1.0 + x;
  } else {
    k = 0;
  }

  double t = x * x;
  double c = x - t * (P1 + t * (P2 + t * (P3 + t * (P4 + t * P5))));
  if (k == 0) return 1.0 - ((x * c) / (c - 2.0) - x);
  double y = 1.0 - ((lo - (x * c) / (2.0 - c)) - hi);
  if (k >= -1021) {
    return orj_with_hi(y, orj_hi(y) + (k << 20));
  }
  y = orj_with_hi(y, orj_hi(y) + ((k + 1000) << 20));
  return y * TWO_M1000;
}

/* natural logarithm by the fdlibm method. */
static inline double js_log(double x) {
  const double LN2_HI = 6.93147180369123816490e-01;
  const double LN2_LO = 1.90821492927058770002e-10;
  const double TWO54 = 1.80143985094819840000e+16;
  const double LG1 = 6.666666666666735130e-01;
  const double LG2 = 3.999999999940941908e-01;
  const double LG3 = 2.857142874366239149e-01;
  const double LG4 = 2.222219843214978396e-01;
  const double LG5 = 1.818357216161805012e-01;
  const double LG6 = 1.531383769920937332e-01;
  const double LG7 = 1.479819860511658591e-01;
  const double zero = 0.0;

  int32_t hx = orj_hi(x);
  uint32_t lx = orj_lo(x);
  int k = 0;
  if (hx < 0x00100000) {                         /* x < 2^-1022 */
    if (((hx & 0x7fffffff) | lx) == 0) return -TWO54 / zero;   /* log(+-0) = -inf */
    if (hx < 0) return (x - x) / zero;                         /* log(-#) = NaN */
    k -= 54;
    x *= TWO54;
    hx = orj_hi(x);
  }
  if (hx >= 0x7ff00000) return x + x;
  k += (hx >> 20) - 1023;
  hx &= 0x000fffff;
  int32_t i = (hx + 0x95f64) & 0x100000;
  x = orj_with_hi(x, hx | (i ^ 0x3ff00000));      /* normalise x or x/2 */
  k += (i >> 20);
  double f = x - 1.0;
  if ((0x000fffff & (2 + hx)) < 3) {             /* -2^-20 <= f < 2^-20 */
    if (f == zero) {
      if (k == 0) return zero;
      double dk = (double)k;
      return dk * LN2_HI + dk * LN2_LO;
    }
    double r = f * f * (0.5 - 0.33333333333333333 * f);
    if (k == 0) return f - r;
    double dk = (double)k;
    return dk * LN2_HI - ((r - dk * LN2_LO) - f);
  }
  double s = f / (2.0 + f);
  double dk = (double)k;
  double z = s * s;
  i = hx - 0x6147a;
  double w = z * z;
  int32_t j = 0x6b851 - hx;
  double t1 = w * (LG2 + w * (LG4 + w * LG6));
  double t2 = z * (LG1 + w * (LG3 + w * (LG5 + w * LG7)));
  i |= j;
  double r = t2 + t1;
  if (i > 0) {
    double hfsq = 0.5 * f * f;
    if (k == 0) return f - (hfsq - s * (hfsq + r));
    return dk * LN2_HI - ((hfsq - (s * (hfsq + r) + dk * LN2_LO)) - f);
  }
  if (k == 0) return f - s * (f - r);
  return dk * LN2_HI - ((s * (f - r) - dk * LN2_LO) - f);
}

#define ORJ_MULBERRY_STEP 0x6d2b79f5u

/* s0 of SeededRandom(seed): (seed >>> 0) || 0x6d2b79f5, for an integral seed. */
static inline uint32_t mulberry32_start(int64_t seed) {
  uint32_t s = (uint32_t)(uint64_t)seed;   /* ToUint32: seed mod 2^32 */
  return s ? s : ORJ_MULBERRY_STEP;
}

/* The n-th value (0-based) returned by SeededRandom(seed).next(). */
static inline double mulberry32_draw(int64_t seed, uint64_t n) {
  uint32_t z = mulberry32_start(seed) + (uint32_t)((n + 1) * (uint64_t)ORJ_MULBERRY_STEP);
  z = (z ^ (z >> 15)) * (z | 1u);
  z ^= z + (z ^ (z >> 7)) * (z | 61u);
  return (double)(z ^ (z >> 14)) / 4294967296.0;
}

/* Largest draw index for which the JS double state is still exact. */
static inline uint64_t mulberry32_exact_limit(int64_t seed) {
  /* need s0 + (n+1)*C <= 2^53 */
  uint64_t s0 = mulberry32_start(seed);
  return ((1ull << 53) - s0) / ORJ_MULBERRY_STEP - 1;
}

/* The sampler's optional final-logit softcap: cap*tanh(x/cap) in binary64
 * from js_exp, rounded once to binary32. The reference declares a softcap
 * (final_logit_softcapping in its model config) but never applies it, so this
 * definition is the engine's own; it is pinned by closed-form tests. */
static inline float softcap_f32(float x, double cap) {
  double y = (double)x / cap;
  double a = y < 0 ? -y : y;
  double t;
  if (a > 40.0) {
    t = 1.0;
  } else if (a < 1.0e-4) {
    t = a - (a * a * a) / 3.0;
  } else {
    double e = js_exp(2.0 * a);
    t = (e - 1.0) / (e + 1.0);
  }
  if (y < 0) t = -t;
  if (y != y) t = y;
  return (float)(cap * t);
}

#endif
