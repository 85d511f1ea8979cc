// The binary64 table exponential of the chunk scan's rescales and of the
// finish kernel's normaliser recomputation: 2^(y/256) = 2^(j/256) * 2^k * e^r
// with y = 256 k + j + s, |s| <= 1/2, r = s ln2 / 256, a correctly rounded
// 256-entry table and the quadratic 1 + r + r^2/2: relative error below
// 4.2e-10 per evaluation (tests/test_scan_exp2.py pins it). exp2_256_tight
// takes the quartic instead, for the deep draw's masses: relative error
// below 1e-15 per evaluation.
#pragma once

#include <hip/hip_runtime.h>

#include "gs_exp2_table.h"

namespace gs {

// 2^(j/256), j = 0..255 (each translation unit holds its own copy)
static __constant__ double c_exp2_256[256] = {GS_EXP2_TABLE_256};

// Terms with (l - lmax)/T < -60 are not summed: each is below e^-60 of the
// maximum's term, so together they move the normaliser by less than
// V * e^-60 < 3e-21 relative. In units of y = 256 log2(e) (l - lmax)/T:
constexpr double kSkipY = -22160.0;

// tab: the table above, or a copy of it in LDS
__device__ __forceinline__ double exp2_256(double y, const double* tab) {
  const double n = __builtin_rint(y);
  const double s = y - n;  // |s| <= 1/2
  const double p = __builtin_fma(s, __builtin_fma(s, GS_EXP2_256_C2, GS_EXP2_256_C1), 1.0);
  const int ni = (int)n;
  return __builtin_ldexp(tab[ni & 255] * p, ni >> 8);
}

__device__ __forceinline__ double exp2_256_tight(double y, const double* tab) {
  const double n = __builtin_rint(y);
  const double s = y - n;  // |s| <= 1/2
  double p = __builtin_fma(s, GS_EXP2_256_C4, GS_EXP2_256_C3);
  p = __builtin_fma(s, p, GS_EXP2_256_C2);
  p = __builtin_fma(s, p, GS_EXP2_256_C1);
  p = __builtin_fma(s, p, 1.0);
  const int ni = (int)n;
  return __builtin_ldexp(tab[ni & 255] * p, ni >> 8);
}

}  // namespace gs
