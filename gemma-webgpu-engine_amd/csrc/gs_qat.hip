// int2 QAT LM head: the reference's logits producer
// (src/webgpu/decode-lm-head.ts:262-340, weights src/model/gemma-output-
// weights.ts:72-81), restated from its CPU definition cpuQatLinear
// (src/reference/qat-linear.ts:78-148):
//   logits[m][r] = srq(scale[r] * sum_k (code[r][k] - 2) * srq(x[m][k], in_scale), out_scale)
// with srq(v, s) = v for s = 0, else clamp(rint(v / s), -128, 127) * s
// rounded to float. Each lane owns one vocabulary row and sums its products
// in column order in binary64: a product of a small integer and a float is
// exact there, so the fused multiply-add rounds exactly where the reference's
// sequential binary64 sum does, and the logits equal cpuQatLinear's bit for
// bit. (The reference's WGSL kernel sums in binary32 in a subgroup order;
// its test allows 5e-4.)
//
// Weights: 2-bit codes, code k of a row at bits 2k..2k+1 of word k / 16
// (packInt2Rows). Row-major: word w of row r at r * (D / 16) + w, the
// checkpoint's order. Block-major: the 4-word block b of row r at
// (b * V + r) * 4, the reference's GPU order, where a wave's 64 lanes read
// 1 KiB in one coalesced load per block.
//
// HBM: V * D / 4 bytes of codes (96 MiB at V 262144, D 1536) + 4 V of scales
// + 4 M V of logits per call; the activations (M x D) are staged in LDS as
// binary64. Work: one bit-field extract, one conversion and one fused
// multiply-add per weight and row of x.
#include "gs_internal.h"

namespace gs {
namespace {

constexpr int kQatThreads = 256;
constexpr int kQatLdsDoubles = 4096;  // activations staged per pass: rows x width <= 32 KiB

struct QatArgs {
  const float* x;         // [M][D]
  const uint32_t* words;  // packed codes
  const float* scales;    // [V]
  float* out;             // [M][V]
  int32_t D, V, M;
  int32_t block_major;
  double in_scale, out_scale;
};

__device__ __forceinline__ double srq(double v, double s) {
  if (s == 0) return v;
  // + 0.0 turns a -0 from rint into +0, as the reference's floor-based
  // rounding returns for ratios in [-1/2, 0)
  double q = __builtin_rint(v / s) + 0.0;
  q = q < -128.0 ? -128.0 : (q > 127.0 ? 127.0 : q);
  return (double)(float)(q * s);
}

// kRows rows of x per pass (m0 .. m0 + kRows - 1, those below M)
template <int kRows>
__global__ __launch_bounds__(kQatThreads) void qat_lmhead_kernel(QatArgs a, int32_t m0) {
  __shared__ double act[kQatLdsDoubles];
  const int tid = threadIdx.x;
  const int D = a.D;
  const int rows = a.M - m0 < kRows ? a.M - m0 : kRows;
  for (int i = tid; i < kRows * D; i += kQatThreads) {
    const int m = i / D;
    act[i] = m < rows ? srq((double)a.x[(int64_t)(m0 + m) * D + (i - m * D)], a.in_scale) : 0.0;
  }
  __syncthreads();
  const int64_t r = (int64_t)blockIdx.x * kQatThreads + tid;
  if (r >= a.V) return;
  double acc[kRows];
#pragma unroll
  for (int m = 0; m < kRows; ++m) acc[m] = 0.0;
  const int blocks = D / 64;
  const uint4* w4 = (const uint4*)a.words;
  for (int b = 0; b < blocks; ++b) {
    const uint4 w = load_nt16(a.block_major ? w4 + (int64_t)b * a.V + r : w4 + r * blocks + b);
    const uint32_t q[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      // code ^ 2 read as a signed 2-bit field is code - 2
      const uint32_t flipped = q[j] ^ 0xAAAAAAAAu;
#pragma unroll
      for (int f = 0; f < 16; ++f) {
        const double wt = (double)(int)__builtin_amdgcn_sbfe((int)flipped, 2 * f, 2);
        const int k = b * 64 + j * 16 + f;
#pragma unroll
        for (int m = 0; m < kRows; ++m) acc[m] = __builtin_fma(wt, act[m * D + k], acc[m]);
      }
    }
  }
  const double scale = (double)a.scales[r];
#pragma unroll
  for (int m = 0; m < kRows; ++m) {
    if (m < rows) a.out[(int64_t)(m0 + m) * a.V + r] = (float)srq(acc[m] * scale, a.out_scale);
  }
}

}  // namespace

// rows of x per pass for width D (the LDS stage holds kQatLdsDoubles)
int qat_rows_per_pass(int32_t D) {
  const int r = kQatLdsDoubles / D;
  return r >= 4 ? 4 : (r >= 2 ? 2 : 1);
}

void launch_qat_lmhead(const float* x, int32_t M, int32_t D, const uint32_t* words, int32_t block_major,
                       const float* scales, int32_t V, double in_scale, double out_scale, float* out, hipStream_t s,
                       LaunchEvents ev) {
  QatArgs a{x, words, scales, out, D, V, M, block_major, in_scale, out_scale};
  const dim3 grid((unsigned)((V + kQatThreads - 1) / kQatThreads));
  const int most = qat_rows_per_pass(D);
  for (int32_t m0 = 0; m0 < M;) {
    // as many rows of x as the stage holds and remain, in a kernel made for that many
    const int left = M - m0;
    const int per = most >= 4 && left >= 4 ? 4 : (most >= 2 && left >= 2 ? 2 : 1);
    const bool first = m0 == 0, last = m0 + per >= M;
    hipEvent_t start = first ? ev.start : nullptr, stop = last ? ev.stop : nullptr;
    if (per == 4) hipExtLaunchKernelGGL(qat_lmhead_kernel<4>, grid, dim3(kQatThreads), 0, s, start, stop, 0, a, m0);
    else if (per == 2) hipExtLaunchKernelGGL(qat_lmhead_kernel<2>, grid, dim3(kQatThreads), 0, s, start, stop, 0, a, m0);
    else hipExtLaunchKernelGGL(qat_lmhead_kernel<1>, grid, dim3(kQatThreads), 0, s, start, stop, 0, a, m0);
    m0 += per;
  }
}

}  // namespace gs
