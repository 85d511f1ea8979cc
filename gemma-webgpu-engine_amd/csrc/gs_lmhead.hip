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
//     each row's 128-byte line is consumed whole; weight and H loads run
//     three K blocks ahead of their use in a register ring, so no wait
//     covers a load issued less than two blocks earlier;
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

  // H: thread t stages 32 bytes of row t/4 of the 64x64 block (rows past M
  // read row M-1 and are stored as zeros)
  const int ar = tid >> 2, ac = (tid & 3) * 16;
  const bool a_live = m0 + ar < M;
  const uint16_t* hrow = H + (size_t)(a_live ? m0 + ar : M - 1) * D + ac;

  // A ring of kDepth K-blocks in flight per lane: the weight row slice this
  // lane multiplies (64 bytes) and this thread's share of the H block. The
  // main loop is unrolled by kDepth and branch-free, so every ring slot is a
  // fixed register set and each wait covers only loads issued kDepth - 1 or
  // kDepth blocks earlier (loads complete in issue order). Prefetches past
  // the last block re-read the last block (cache hits, never used).
  constexpr int kDepth = 3;
  const int nk = D / kKBlock;
  uint4 wr[kDepth][4], hr[kDepth][2];
  auto issue = [&](int slot, int kb) __attribute__((always_inline)) {
    kb = kb < nk ? kb : nk - 1;
    const uint4* pw = (const uint4*)(wrow + (size_t)kb * kKBlock);
    const uint4* ph = (const uint4*)(hrow + (size_t)kb * kKBlock);
#pragma unroll
    for (int i = 0; i < 4; ++i) wr[slot][i] = pw[i];
    hr[slot][0] = ph[0];
    hr[slot][1] = ph[1];
  };
  const uint32_t a_mask = a_live ? 0xFFFFFFFFu : 0u;  // rows past M stage zeros
  auto stage_h = [&](int buf, int slot) __attribute__((always_inline)) {
    const uint4 v0 = hr[slot][0], v1 = hr[slot][1];
    *(uint4*)&sA[buf][ar][ac] = make_uint4(v0.x & a_mask, v0.y & a_mask, v0.z & a_mask, v0.w & a_mask);
    *(uint4*)&sA[buf][ar][ac + 8] = make_uint4(v1.x & a_mask, v1.y & a_mask, v1.z & a_mask, v1.w & a_mask);
  };

  f32x16 acc0, acc1;
#pragma unroll
  for (int i = 0; i < 16; ++i) { acc0[i] = 0.0f; acc1[i] = 0.0f; }
  auto step = [&](int kbi, int p) __attribute__((always_inline)) {
    const int buf = kbi & 1;
    // the next block's H into the other buffer (its loads left kDepth-1 blocks ago)
    stage_h(buf ^ 1, (p + 1) % kDepth);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const bf16x8 bf = as_bf16x8(wr[p][s]);
      const bf16x8 a0 = as_bf16x8(*(const uint4*)&sA[buf][lane & 31][h * 32 + s * 8]);
      const bf16x8 a1 = as_bf16x8(*(const uint4*)&sA[buf][32 + (lane & 31)][h * 32 + s * 8]);
      acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, bf, acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, bf, acc1, 0, 0, 0);
    }
    issue(p, kbi + kDepth);  // refill this slot
    __syncthreads();
  };
#pragma unroll
  for (int p = 0; p < kDepth; ++p) issue(p, p);
  stage_h(0, 0);
  __syncthreads();
  const int n_main = nk - nk % kDepth;
  for (int kb0 = 0; kb0 < n_main; kb0 += kDepth) {
#pragma unroll
    for (int p = 0; p < kDepth; ++p) step(kb0 + p, p);
  }
  // the last nk % kDepth blocks sit in the first ring slots
#pragma unroll
  for (int p = 0; p < kDepth - 1; ++p) {
    if (n_main + p < nk) step(n_main + p, p);
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
    // non-temporal stores: the 64 x V logits stream past the caches (-11 us
    // of 261 at M 64, D 2048, V 262144, against write-back stores)
    if (m0 + row < M) __builtin_nontemporal_store(x0, &out[(size_t)(m0 + row) * V + n]);
    if (m0 + 32 + row < M) __builtin_nontemporal_store(x1, &out[(size_t)(m0 + 32 + row) * V + n]);
  }
}

}  // namespace

void launch_lmhead(const uint16_t* hidden, const uint16_t* weight, int32_t m, int32_t width, int32_t vocab,
                   float softcap, float* out, hipStream_t s, LaunchEvents ev) {
  dim3 grid((vocab + kLmRows - 1) / kLmRows, (m + kLmM - 1) / kLmM);
  hipExtLaunchKernelGGL(lmhead_kernel, grid, dim3(kLmThreads), 0, s, ev.start, ev.stop, 0, hidden, weight, m, width,
                        vocab, softcap, out);
}

}  // namespace gs
