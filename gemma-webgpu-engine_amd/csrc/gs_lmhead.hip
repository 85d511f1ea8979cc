// lm_head logits producer: logits[m][v] = cap * tanh((H[m] . W[v]) / cap)
// (cap <= 0: no cap), bf16 inputs, f32 accumulate, on gfx950 MFMA.
//
// The reference's producer is an int2 QAT GEMV (src/webgpu/decode-lm-head.ts:
// 187-340); this is the bf16 tied-embedding variant the sampler consumes.
// At M = 64 rows the product is bound by streaming W (2*V*D bytes) from HBM,
// so the layout is built around W's reads:
//   * a workgroup = 4 wave64, each wave owns 32 vocab rows; the grid covers V
//     in slabs of 128 rows (and M in blocks of 64 rows);
//   * per 64-wide K block a lane loads 64 contiguous bytes of one weight row
//     (half the block: lanes 0-31 take k 0-31, lanes 32-63 take k 32-63), so
//     each row's 128-byte line is consumed whole and the next block is
//     prefetched into registers while the current one is multiplied;
//   * H's 64x64 block is staged in LDS (double-buffered, rows padded to 144 B)
//     and shared by the four waves;
//   * v_mfma_f32_32x32x16_bf16: a K block is 4 steps x 2 M tiles. The K order
//     inside a block is permuted identically for H and W (step s, lane half h
//     -> k = 32h + 8s + e), which leaves every dot product unchanged.
#include "gs_internal.h"

namespace gs {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kLmThreads = 256;
constexpr int kLmRows = 128;  // vocab rows per workgroup
constexpr int kLmM = 64;      // hidden rows per workgroup
constexpr int kKBlock = 64;
constexpr int kPad = 72;      // LDS row length in bf16 (64 + 8)

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

__global__ __launch_bounds__(kLmThreads) void lmhead_kernel(const uint16_t* __restrict__ H,
                                                            const uint16_t* __restrict__ W, int M, int D, int V,
                                                            float cap, float* __restrict__ out) {
  __shared__ __attribute__((aligned(16))) uint16_t sA[2][kLmM][kPad];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h = lane >> 5;
  const int n0 = blockIdx.x * kLmRows + wave * 32;
  const int m0 = blockIdx.y * kLmM;
  const int nrow = n0 + (lane & 31) < V ? n0 + (lane & 31) : V - 1;
  const uint16_t* wrow = W + (size_t)nrow * D + h * 32;

  const int ar = tid >> 2, ac = (tid & 3) * 16;
  auto load_a = [&](int buf, int kb) {
    uint4 v0 = make_uint4(0, 0, 0, 0), v1 = make_uint4(0, 0, 0, 0);
    if (m0 + ar < M) {
      const uint4* p = (const uint4*)(H + (size_t)(m0 + ar) * D + kb + ac);
      v0 = p[0];
      v1 = p[1];
    }
    *(uint4*)&sA[buf][ar][ac] = v0;
    *(uint4*)&sA[buf][ar][ac + 8] = v1;
  };

  f32x16 acc0, acc1;
#pragma unroll
  for (int i = 0; i < 16; ++i) { acc0[i] = 0.0f; acc1[i] = 0.0f; }
  uint4 b[4], bn[4];
  load_a(0, 0);
#pragma unroll
  for (int i = 0; i < 4; ++i) b[i] = ((const uint4*)wrow)[i];
  __syncthreads();

  const int nk = D / kKBlock;
  for (int kbi = 0; kbi < nk; ++kbi) {
    const int buf = kbi & 1;
    if (kbi + 1 < nk) {
      load_a(buf ^ 1, (kbi + 1) * kKBlock);
      const uint4* p = (const uint4*)(wrow + (size_t)(kbi + 1) * kKBlock);
#pragma unroll
      for (int i = 0; i < 4; ++i) bn[i] = p[i];
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const bf16x8 bf = as_bf16x8(b[s]);
      const bf16x8 a0 = as_bf16x8(*(const uint4*)&sA[buf][lane & 31][h * 32 + s * 8]);
      const bf16x8 a1 = as_bf16x8(*(const uint4*)&sA[buf][32 + (lane & 31)][h * 32 + s * 8]);
      acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, bf, acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, bf, acc1, 0, 0, 0);
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i) b[i] = bn[i];
  }

  // D layout of a 32x32 tile: lane l, register r -> column l % 32,
  // row 8*(r/4) + 4*(l/32) + r%4
  const int n = n0 + (lane & 31);
  if (n >= V) return;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int row = 8 * (r >> 2) + 4 * h + (r & 3);
    float x0 = acc0[r], x1 = acc1[r];
    if (cap > 0.0f) {
      x0 = cap * tanhf(x0 / cap);
      x1 = cap * tanhf(x1 / cap);
    }
    if (m0 + row < M) out[(size_t)(m0 + row) * V + n] = x0;
    if (m0 + 32 + row < M) out[(size_t)(m0 + 32 + row) * V + n] = x1;
  }
}

}  // namespace

void launch_lmhead(const uint16_t* hidden, const uint16_t* weight, int32_t m, int32_t width, int32_t vocab,
                   float softcap, float* out, hipStream_t s) {
  dim3 grid((vocab + kLmRows - 1) / kLmRows, (m + kLmM - 1) / kLmM);
  hipLaunchKernelGGL(lmhead_kernel, grid, dim3(kLmThreads), 0, s, hidden, weight, m, width, vocab, softcap, out);
}

}  // namespace gs
