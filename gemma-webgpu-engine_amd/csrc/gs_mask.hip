// Constraint masker and raw-logit log-probability.
//
// build_masks_kernel: legalTokenIds (src/runtime/constraints.ts:56-92) for a
// byte-level DFA, as a 262144-bit mask per requested state. The reference
// walks a token-byte trie depth-first; here every token walks its own bytes
// (the vocab is a CSR of token byte strings), one token per lane, against a
// next-state table whose entries already fold in viability
// (src/runtime/constraints.ts:253-265, 300-322): next'[s][b] = -1 unless the
// edge exists and its target can still reach a final state. A token is legal
// from s iff it has at least one byte and no step yields -1 -- the set the
// trie DFS emits. Lanes of a wave64 cover 64 consecutive ids, so one ballot
// gives two mask words.
//
// logprob_kernel: tokenLogProbability (src/runtime/sampling.ts:67-80).
//
// mask_fill_kernel + mask_copy_kernel: maskConstraintLogits
// (src/runtime/constraints.ts:159-173): a row of -Infinity, then the raw
// logit copied back at every listed id inside [0, n). Listed ids may repeat
// (legal and termination lists overlap); repeats store the same value.
#include "gs_internal.h"

namespace gs {
namespace {

constexpr int kMaskThreads = 256;
constexpr int kLdsStates = 96;  // tables up to 96 x 256 x int16 (48 KiB) stay in LDS

__global__ __launch_bounds__(kMaskThreads) void build_masks_kernel(const int64_t* offsets, const uint8_t* bytes,
                                                                   int32_t vocab, const int16_t* next,
                                                                   int32_t n_states, const int32_t* states,
                                                                   int32_t n, uint32_t* masks, int32_t mask_words) {
  __shared__ int16_t s_next[kLdsStates * 256];
  const bool in_lds = n_states <= kLdsStates;
  if (in_lds) {
    for (int i = threadIdx.x; i < n_states * 256; i += kMaskThreads) s_next[i] = next[i];
  }
  __syncthreads();
  const int16_t* table = in_lds ? s_next : next;
  const int64_t t = (int64_t)blockIdx.x * kMaskThreads + threadIdx.x;
  const int lane = threadIdx.x & 63;
  int64_t b0 = 0, b1 = 0;
  if (t < vocab) { b0 = offsets[t]; b1 = offsets[t + 1]; }
  const int len = (int)(b1 - b0);
  // the first 16 bytes in registers, the rest read on demand
  uint32_t w[4] = {0, 0, 0, 0};
  for (int i = 0; i < len && i < 16; ++i) w[i >> 2] |= (uint32_t)bytes[b0 + i] << (8 * (i & 3));
  for (int q = 0; q < n; ++q) {
    int32_t s = states[q];
    bool legal = t < vocab && len > 0 && s >= 0 && s < n_states;
    for (int i = 0; legal && i < len; ++i) {
      const uint32_t b = i < 16 ? (w[i >> 2] >> (8 * (i & 3))) & 0xFFu : bytes[b0 + i];
      s = table[s * 256 + (int)b];
      legal = s >= 0;
    }
    const uint64_t bits = __ballot(legal);
    const int64_t word0 = ((int64_t)blockIdx.x * kMaskThreads + (threadIdx.x & ~63)) >> 5;
    if (lane < 2 && word0 + lane < mask_words) {
      masks[(int64_t)q * mask_words + word0 + lane] = (uint32_t)(bits >> (32 * lane));
    }
  }
}

constexpr int kLogThreads = 1024;

__global__ __launch_bounds__(kLogThreads) void logprob_kernel(const void* logits, int32_t dtype, int64_t stride,
                                                              int32_t vocab, const int32_t* tokens, double* out) {
  __shared__ double s_w[kLogThreads / 64];
  __shared__ double s_max;
  const int64_t row = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  auto value = [&](int64_t i) -> double {
    if (dtype == GS_BF16) {
      const uint16_t h = ((const uint16_t*)logits)[row * stride + i];
      return (double)__builtin_bit_cast(float, (uint32_t)h << 16);
    }
    return (double)((const float*)logits)[row * stride + i];
  };
  // Math.max over the raw logits (NaN propagates)
  double m = -__builtin_inf();
  for (int64_t i = threadIdx.x; i < vocab; i += kLogThreads) m = gsm::js_max(m, value(i));
  for (int k = 32; k > 0; k >>= 1) m = gsm::js_max(m, shfl_xor_f64(m, k));
  if (lane == 0) s_w[wave] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    double x = s_w[0];
    for (int w = 1; w < kLogThreads / 64; ++w) x = gsm::js_max(x, s_w[w]);
    s_max = x;
  }
  __syncthreads();
  const double mx = s_max;
  double d = 0.0;
  for (int64_t i = threadIdx.x; i < vocab; i += kLogThreads) d += gsm::js_exp(value(i) - mx);
  d = wave_sum_f64(d);
  __syncthreads();
  if (lane == 0) s_w[wave] = d;
  __syncthreads();
  if (threadIdx.x == 0) {
    double den = 0.0;
    for (int w = 0; w < kLogThreads / 64; ++w) den += s_w[w];
    const int32_t tok = tokens[row];
    out[row] = (tok >= 0 && tok < vocab) ? value(tok) - mx - gsm::js_log(den) : __builtin_nan("");
  }
}

constexpr int kFillThreads = 256;

__global__ __launch_bounds__(kFillThreads) void mask_fill_kernel(float* out, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * kFillThreads + threadIdx.x;
  if (i < n) out[i] = -__builtin_inff();
}

__global__ __launch_bounds__(kFillThreads) void mask_copy_kernel(const float* raw, int64_t n, const int32_t* ids,
                                                                 int64_t n_ids, float* out) {
  const int64_t k = (int64_t)blockIdx.x * kFillThreads + threadIdx.x;
  if (k >= n_ids) return;
  const int32_t id = ids[k];
  if (id >= 0 && id < n) out[id] = raw[id];
}

}  // namespace

void launch_mask_logits(const float* raw, int64_t n, const int32_t* ids, int64_t n_ids, float* out, hipStream_t s) {
  if (n > 0) {
    hipLaunchKernelGGL(mask_fill_kernel, dim3((unsigned)((n + kFillThreads - 1) / kFillThreads)), dim3(kFillThreads),
                       0, s, out, n);
  }
  if (n > 0 && n_ids > 0) {
    hipLaunchKernelGGL(mask_copy_kernel, dim3((unsigned)((n_ids + kFillThreads - 1) / kFillThreads)),
                       dim3(kFillThreads), 0, s, raw, n, ids, n_ids, out);
  }
}

void launch_masks(const int64_t* offsets, const uint8_t* bytes, int32_t vocab, const int16_t* next,
                  const int32_t* states, int32_t n, uint32_t* masks, int32_t mask_words, int32_t n_states,
                  hipStream_t s) {
  const int blocks = (vocab + kMaskThreads - 1) / kMaskThreads;
  hipLaunchKernelGGL(build_masks_kernel, dim3(blocks), dim3(kMaskThreads), 0, s, offsets, bytes, vocab, next,
                     n_states, states, n, masks, mask_words);
}

void launch_logprob(const void* logits, int32_t dtype, int32_t rows, int64_t stride, int32_t vocab,
                    const int32_t* tokens, double* out, hipStream_t s) {
  hipLaunchKernelGGL(logprob_kernel, dim3(rows), dim3(kLogThreads), 0, s, logits, dtype, stride, vocab, tokens, out);
}

}  // namespace gs
