/*
 * ORACLE -- test infrastructure only (tests/ and bench.py's cpu_baseline
 * leg). A C restatement of the reference's CPU int2 QAT linear layer, the
 * producer of its logits (src/reference/qat-linear.ts):
 *   or_pack_int2_rows   packInt2Rows (:45-71): code i of a row at bits 2i..2i+1
 *                       of word i / 16, rows of in / 16 words
 *   or_unpack_int2      unpackInt2 (:73-76)
 *   or_apply_srq        applySrq (:118-128, without the bfloat16 emulation):
 *                       scale 0 -> the value; else clamp(roundTiesToEven(v /
 *                       scale), -128, 127) * scale rounded to float
 *   or_qat_linear_int2  cpuQatLinear with bits 2 (:78-116): per output row,
 *                       dot = sum over columns in order of (code - 2) *
 *                       srq(input, inScale) in binary64, times the row scale,
 *                       srq(., outScale), stored as float
 *   or_repack_block_major  the block-major weight order of the reference's
 *                       GPU head (src/webgpu/decode-lm-head.ts:344-360):
 *                       block b of 4 words of every row, rows consecutive
 * Built into _build/liboracle.so beside sampler_ref.c.
 */
#include <math.h>
#include <stdint.h>

/* -1: a code above 3; -2: in not a multiple of 16 */
int or_pack_int2_rows(const uint8_t* codes, int64_t out_features, int64_t in_features, uint32_t* words) {
  if (in_features % 16 != 0) return -2;
  const int64_t n = out_features * in_features;
  for (int64_t w = 0; w < n / 16; ++w) {
    uint32_t packed = 0;
    for (int k = 0; k < 16; ++k) {
      const uint8_t c = codes[w * 16 + k];
      if (c > 3) return -1;
      packed |= (uint32_t)c << (2 * k);
    }
    words[w] = packed;
  }
  return 0;
}

int or_unpack_int2(const uint32_t* words, int64_t index) {
  return (int)((words[index / 16] >> ((index % 16) * 2)) & 3u);
}

static double round_ties_even(double v) {
  const double lower = floor(v);
  const double fraction = v - lower;
  if (fraction < 0.5) return lower;
  if (fraction > 0.5) return lower + 1;
  return fmod(lower, 2.0) == 0.0 ? lower : lower + 1;
}

double or_apply_srq(double value, double scale) {
  if (scale == 0) return value;
  double q = round_ties_even(value / scale);
  if (q < -128) q = -128;
  if (q > 127) q = 127;
  return (double)(float)(q * scale);
}

void or_qat_linear_int2(const float* input, const uint32_t* words, const float* row_scales, int64_t in_features,
                        int64_t out_features, double input_scale, double output_scale, float* out) {
  for (int64_t row = 0; row < out_features; ++row) {
    double dot = 0;
    const int64_t base = row * in_features;
    for (int64_t col = 0; col < in_features; ++col) {
      const double activation = or_apply_srq((double)input[col], input_scale);
      const int weight = or_unpack_int2(words, base + col) - 2;
      dot += weight * activation;
    }
    out[row] = (float)or_apply_srq(dot * (double)row_scales[row], output_scale);
  }
}

void or_repack_block_major(const uint32_t* row_major, int64_t out_features, int64_t in_features, uint32_t* block_major) {
  const int64_t words_per_row = in_features / 16;
  const int64_t blocks = words_per_row / 4;
  for (int64_t row = 0; row < out_features; ++row)
    for (int64_t b = 0; b < blocks; ++b)
      for (int j = 0; j < 4; ++j) block_major[(b * out_features + row) * 4 + j] = row_major[row * words_per_row + b * 4 + j];
}
