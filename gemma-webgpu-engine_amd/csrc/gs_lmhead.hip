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

// Resident-H kernel for widths up to 2048: one workgroup per compute unit
// holds its 64-row block of H in registers for the whole launch and streams
// W in steps of 16 vocabulary rows, in runs of 16 steps (256 rows, 1 MB at
// D 2048) dealt round-robin to the workgroups, so the chip reads a window of
// adjacent runs at a time (199 us against 203 us for one contiguous range
// per workgroup).
//   * 8 waves split K: wave w owns the 32-wide K steps [w nS / 8, (w+1) nS / 8)
//     of the nS = D / 32, its H slice (64 rows) held as MFMA A operands
//     (v_mfma_f32_16x16x32_bf16: lane i + 16 g holds k = 32 s + 8 g .. + 7 of
//     row i of an M tile, 4 M tiles);
//   * per step a lane loads 16 bytes per K step of one vocabulary row (the
//     B operand), so the workgroup reads 16 whole rows of W (16 x 2D bytes,
//     contiguous) per step; two steps of loads are in flight per wave;
//   * the 8 waves' partial 64x16 tiles go through LDS (double-buffered), and
//     after one barrier each thread adds two outputs' partials in wave order
//     and applies the cap into an LDS stage of 16 steps, which then goes out
//     as 1 KB runs of each logits row in 16-byte stores. At M 64, D 2048,
//     V 262144 the logits cost 73 us of 258 stored per step (64-byte pieces
//     of 64 rows 4V bytes apart), 31 us of 216 staged over 8 steps, 19 us of
//     204 over 16 (185 us without stores); spreading a double-buffered stage's
//     stores over the next run's steps took 224 us, write-back stores 237 us.
// Every global access is a buffer access with no branch around it: rows past
// V or M, K steps a wave does not own, and the steps past a workgroup's run
// take an out-of-range offset (zeros, no memory request; stores dropped). The
// compiler's wait counts then cover exactly the loads a step consumes, as
// loads and stores share one in-order counter on this part.
constexpr int kResWaves = 8;
constexpr int kResThreads = 64 * kResWaves;
constexpr int kResN = 16;         // vocabulary rows per step
constexpr int kResStride = 68;    // LDS floats per vocabulary row of a partial (64 + 4)
constexpr int kResMaxWidth = 2048;
constexpr int32_t kResNT = 2;     // non-temporal cache policy of the streams
constexpr int kResStage = 16;     // steps of logits staged per flush
constexpr int kResStageStride = kResStage * kResN + 4;  // LDS floats per staged row

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int kS>  // K steps per wave, at most 8
__global__ __launch_bounds__(kResThreads) void lmhead_resident_kernel(const uint16_t* __restrict__ H,
                                                                      const uint16_t* __restrict__ W, int M, int D,
                                                                      int V, float cap, float* __restrict__ out) {
  __shared__ __attribute__((aligned(16))) float red[2][kResWaves][kResN * kResStride];
  __shared__ __attribute__((aligned(16))) float stage[64 * kResStageStride];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int j = lane & 15, g = lane >> 4;
  const int n_steps = D / 32;
  const int s_lo = wave * n_steps / kResWaves, s_hi = (wave + 1) * n_steps / kResWaves;
  const int my_steps = s_hi - s_lo;  // kS or kS - 1
  // this workgroup's steps k = 0 .. k_end - 1: run blockIdx.x + gridDim.x r
  // (r = k / kResStage), tile kResStage run + k % kResStage of 16 vocabulary
  // rows; steps on tiles past the last are empty
  const int n_tiles = (V + kResN - 1) / kResN;
  const int n_runs = (n_tiles + kResStage - 1) / kResStage;
  const int k_end = n_runs > (int)blockIdx.x ? ((n_runs - 1 - (int)blockIdx.x) / (int)gridDim.x + 1) * kResStage : 0;
  auto tile_of = [&](int k) __attribute__((always_inline)) {
    return ((int)blockIdx.x + (int)gridDim.x * (k / kResStage)) * kResStage + k % kResStage;
  };
  // byte offsets of this lane's K step s within a row of H or W
  uint32_t k_off[kS];
#pragma unroll
  for (int s = 0; s < kS; ++s) k_off[s] = s < my_steps ? (uint32_t)(64 * (s_lo + s) + 16 * g) : kBufferOutOfRange;

  // H slice: rows 16 mt + j of the M tiles (rows past M read zeros)
  const __amdgpu_buffer_rsrc_t hr =
      __builtin_amdgcn_make_buffer_rsrc((void*)H, (short)0, M * D * 2, kBufferWord3);
  bf16x8 hreg[4][kS];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
    for (int s = 0; s < kS; ++s) {
      const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(hr, k_off[s] + (uint32_t)((16 * mt + j) * D * 2), 0, 0);
      hreg[mt][s] = __builtin_bit_cast(bf16x8, v);
    }
  }
  u32x4 wbuf[2][kS];
  // step k's rows in a resource of their own (empty past the steps or the
  // tiles, short at V)
  auto issue = [&](int slot, int k) __attribute__((always_inline)) {
    const int t = tile_of(k);
    const bool live = k < k_end && t < n_tiles;
    const int rows = live ? (V - t * kResN < kResN ? V - t * kResN : kResN) : 0;
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(W + (size_t)(live ? t : 0) * kResN * D), (short)0, rows * D * 2, kBufferWord3);
    const uint32_t row_off = (uint32_t)(j * D * 2);
#pragma unroll
    for (int s = 0; s < kS; ++s) wbuf[slot][s] = __builtin_amdgcn_raw_buffer_load_b128(wr, row_off + k_off[s], 0, kResNT);
  };
  // the output block: rows past M fall outside the resource
  const __amdgpu_buffer_rsrc_t orc =
      __builtin_amdgcn_make_buffer_rsrc((void*)out, (short)0, M * V * 4, kBufferWord3);
  // reduction role: outputs (m, n) = (2 (tid >> 4) + e, tid & 15), e = 0, 1
  const int rn = tid & 15, rm = 2 * (tid >> 4);
  auto step = [&](int k, int u) __attribute__((always_inline)) {
    const int slot = u & 1;
    f32x4 acc[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) acc[mt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < kS; ++s) {
      const bf16x8 b = __builtin_bit_cast(bf16x8, wbuf[slot][s]);
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(hreg[mt][s], b, acc[mt], 0, 0, 0);
    }
    issue(slot, k + 2);
    // lane (j, g) holds rows 16 mt + 4 g + e of column j
    float* r = &red[slot][wave][j * kResStride + 4 * g];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) *(f32x4*)(r + 16 * mt) = acc[mt];
    __syncthreads();
    float x0 = 0.0f, x1 = 0.0f;
#pragma unroll
    for (int w = 0; w < kResWaves; ++w) {
      const float2 p = *(const float2*)&red[slot][w][rn * kResStride + rm];
      x0 += p.x;
      x1 += p.y;
    }
    if (cap > 0.0f) {
      x0 = cap * tanhf(x0 / cap);
      x1 = cap * tanhf(x1 / cap);
    }
    stage[rm * kResStageStride + kResN * u + rn] = x0;
    stage[(rm + 1) * kResStageStride + kResN * u + rn] = x1;
  };
  // a staged run: piece q = tid + 512 i is 16 bytes of row q / 64 at column
  // 4 (q % 64), so a wave writes one row's 1 KB. Columns of tiles past the
  // last, or past V, are dropped (V % 4 == 0: a piece lies within its row).
  constexpr int kRowPieces = kResStage * kResN / 4;  // 64
  auto flush = [&](int k0) __attribute__((always_inline)) {
    const int t0 = tile_of(k0);
#pragma unroll
    for (int i = 0; i < 64 * kRowPieces / kResThreads; ++i) {
      const int q = tid + kResThreads * i, row = q / kRowPieces, c = 4 * (q % kRowPieces);
      const f32x4 v = *(const f32x4*)&stage[row * kResStageStride + c];
      const int n = t0 * kResN + c;
      const uint32_t o = t0 + c / kResN < n_tiles && n < V ? (uint32_t)(row * V + n) * 4u : kBufferOutOfRange;
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), orc, o, 0, kResNT);
    }
  };
  // Straight-line runs of kResStage steps (even, so the two load slots
  // alternate in place); steps past the tiles read zeros and drop their
  // stores. The reduction buffer of step u is u & 1: the barrier of
  // step u + 1 orders step u's reads before step u + 2's writes; the barrier
  // before a flush orders the stage's writes before its reads, and the next
  // run's first barrier its reads before the next writes.
  auto run = [&](int k0) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < kResStage; ++u) step(k0 + u, u);
    __syncthreads();
    flush(k0);
  };
  issue(0, 0);
  // keep the first step's loads ahead of the second's (waits count in issue order)
  __builtin_amdgcn_sched_barrier(0);
  issue(1, 1);
  for (int k0 = 0; k0 < k_end; k0 += kResStage) run(k0);
}

}  // namespace

void launch_lmhead(const uint16_t* hidden, const uint16_t* weight, int32_t m, int32_t width, int32_t vocab,
                   float softcap, float* out, int32_t cu_count, hipStream_t s, LaunchEvents ev) {
  if (width <= kResMaxWidth && width % 32 == 0 && vocab % 4 == 0 && ((uintptr_t)out & 15) == 0 &&
      (int64_t)vocab * kLmM * 4 < ((int64_t)1 << 31)) {
    // one launch per 64-row block of H, one workgroup per compute unit
    const int k_steps = (width / 32 + kResWaves - 1) / kResWaves;
    const dim3 grid(cu_count > 0 ? cu_count : 256), block(kResThreads);
    for (int m0 = 0; m0 < m; m0 += kLmM) {
      const int mb = m - m0 < kLmM ? m - m0 : kLmM;
      const uint16_t* h = hidden + (size_t)m0 * width;
      float* o = out + (size_t)m0 * vocab;
      hipEvent_t start = m0 == 0 ? ev.start : nullptr, stop = m0 + kLmM >= m ? ev.stop : nullptr;
      switch (k_steps) {
#define GS_RES_CASE(k)                                                                                              \
  case k:                                                                                                           \
    hipExtLaunchKernelGGL(lmhead_resident_kernel<k>, grid, block, 0, s, start, stop, 0, h, weight, mb, width, vocab, \
                          softcap, o);                                                                              \
    break;
        GS_RES_CASE(1)
        GS_RES_CASE(2)
        GS_RES_CASE(3)
        GS_RES_CASE(4)
        GS_RES_CASE(5)
        GS_RES_CASE(6)
        GS_RES_CASE(7)
        GS_RES_CASE(8)
#undef GS_RES_CASE
      }
    }
    return;
  }
  dim3 grid((vocab + kLmRows - 1) / kLmRows, (m + kLmM - 1) / kLmM);
  hipExtLaunchKernelGGL(lmhead_kernel, grid, dim3(kLmThreads), 0, s, ev.start, ev.stop, 0, hidden, weight, m, width,
                        vocab, softcap, out);
}

}  // namespace gs
