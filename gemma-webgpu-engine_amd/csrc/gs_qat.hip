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
//
// Exact integer path (widths a multiple of 256 up to 2048, V a multiple of
// 16). Every activation a_k is a binary32 value, an integer multiple of its
// granule 2^g_k; with E the smallest granule of a row (nonzero a_k), every
// product (code - 2) a_k and every partial sum is an integer multiple of 2^E
// no larger than 2 sum |a_k|. When that bound is below 2^(E + 53), no partial
// sum rounds: the sequential binary64 sum is the exact sum, and so is
//   2^E (sum_k code_k A_k - 2 sum_k A_k),   A_k = a_k / 2^E (integers).
// qat_tile_kernel checks the bound per row of x, writes A_k as 7 balanced
// base-256 digits (int8 limbs), multiplies the codes (0..3, int8) by the
// limbs on v_mfma_i32_16x16x64_i8 (exact int32 sums), combines the limbs in
// wrapping 64-bit arithmetic (exact: the total fits in 53 bits) and applies
// the same epilogue, so the logits equal the binary64 path's bit for bit.
// Rows that fail the bound (a huge exponent range, subnormals, non-finite
// values) take the binary64 path in the same launch.
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
  // the reference's floor-based rounding (qat-linear.ts:142-148) returns +0
  // for ratios in [-1/2, 0), where rint gives -0, and keeps a ratio of -0
  // (floor(-0) is -0): a zero from rint becomes the ratio itself when that
  // is a zero, else +0
  const double r = v / s;
  double q = __builtin_rint(r);
  if (q == 0.0) q = r == 0.0 ? r : 0.0;
  q = q < -128.0 ? -128.0 : (q > 127.0 ? 127.0 : q);
  return (double)(float)(q * s);
}

// The activations of kRows rows of x from m0 (those below M) into act,
// after the input SRQ, in binary64 (the whole block calls it).
template <int kRows, int kThreads = kQatThreads>
__device__ __forceinline__ void qat_stage_act(const QatArgs& a, int32_t m0, double* act) {
  const int D = a.D;
  const int rows = a.M - m0 < kRows ? a.M - m0 : kRows;
  for (int i = threadIdx.x; i < kRows * D; i += kThreads) {
    const int m = i / D;
    act[i] = m < rows ? srq((double)a.x[(int64_t)(m0 + m) * D + (i - m * D)], a.in_scale) : 0.0;
  }
  __syncthreads();
}

// Logits of the staged rows (those below M and not skipped) at vocabulary
// row r < V.
template <int kRows>
__device__ __forceinline__ void qat_row_binary64(const QatArgs& a, int32_t m0, const bool (&skip)[kRows],
                                                 const double* act, int64_t r) {
  const int D = a.D;
  const int rows = a.M - m0 < kRows ? a.M - m0 : kRows;
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
    if (m < rows && !skip[m]) a.out[(int64_t)(m0 + m) * a.V + r] = (float)srq(acc[m] * scale, a.out_scale);
  }
}

// kRows rows of x per pass (m0 .. m0 + kRows - 1, those below M)
template <int kRows>
__global__ __launch_bounds__(kQatThreads) void qat_lmhead_kernel(QatArgs a, int32_t m0) {
  __shared__ double act[kQatLdsDoubles];
  bool skip[kRows];
#pragma unroll
  for (int m = 0; m < kRows; ++m) skip[m] = false;
  qat_stage_act<kRows>(a, m0, act);
  const int64_t r = (int64_t)blockIdx.x * kQatThreads + threadIdx.x;
  if (r < a.V) qat_row_binary64<kRows>(a, m0, skip, act, r);
}

// ---- the exact integer path
typedef int i32x4 __attribute__((ext_vector_type(4)));
constexpr int kQatLimbs = 7;                   // balanced base-256 digits of |A_k| < 2^52
constexpr uint64_t kQatSumBound = 1ull << 52;  // sum |A_k| below it: every partial sum exact

// Operand layout of the integer path: MFMA step s takes 64 codes of a row,
// lane row + 16 g of a 16-row tile holding 16 of them as 4 dwords, byte i of
// dword t being code 16 W + 4 i + t of word W = 16 q + 4 g + t' (s = 4 q + t').
// The tile kernel expands a code word into bytes in that order and writes
// the activations' limbs at the same positions; the dot product does not
// depend on the order of k.
// The activation's integer significand and granule exponent (the value is
// sig 2^g); false for a non-finite value.
__device__ __forceinline__ bool act_parts(float f, uint32_t* sig, int* g) {
  const uint32_t bits = __builtin_bit_cast(uint32_t, f);
  const uint32_t ex = (bits >> 23) & 0xFFu;
  if (ex == 0xFFu) return false;
  *sig = ex ? (bits & 0x7FFFFFu) | 0x800000u : bits & 0x7FFFFFu;
  *g = ex ? (int)ex - 150 : -149;
  return true;
}

// Per-row constants of a tile's two rows of x, reduced in LDS.
struct QatTileRows {
  int emin[2];                  // smallest granule exponent of the nonzero activations
  uint32_t bad[2];              // a non-finite activation, or a magnitude past the bound
  unsigned long long sabs[2];   // sum |A_k|
  unsigned long long ssum[2];   // sum A_k (wrapping; exact when the check passes)
};

constexpr int kQatMaxSteps = 2048 / 64;
constexpr int kQatTileThreads = 1024;
constexpr int kQatTileWaves = kQatTileThreads / 64;
constexpr int32_t kQatNT = 2;        // non-temporal cache policy of the code stream
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Rows 2 tile and 2 tile + 1 of x, one launch, one workgroup per compute unit
// over a contiguous run of 16-row vocabulary tiles. Each workgroup checks the
// two rows and writes their limbs into LDS as a 16-row operand tile (rows
// 8 r + limb, limb 7 zero; one thread per code word of 16 activations); its
// 16 waves then take the run's tiles in turn, the next tile's codes loading
// while the current one multiplies. A row the check refused takes the
// binary64 path over the same vocabulary rows afterwards. (Four 256-thread
// workgroups per compute unit, each repeating the check and the limbs, took
// 25.3 us instead of 24.4 at V 262144, D 1536; reducing the check's sums
// through an LDS array by one wave per row instead of LDS atomics, 24.9 us
// instead of 24.0.)
__global__ __launch_bounds__(kQatTileThreads) void qat_tile_kernel(QatArgs a, int32_t tile) {
  __shared__ union __attribute__((aligned(16))) {
    i32x4 op[kQatMaxSteps][64];   // the integer path's operand tile
    double act[2 * 2048];         // the binary64 path's activations
  } L;
  __shared__ QatTileRows R;
  const int tid = threadIdx.x;
  const int D = a.D, words = D / 16, quads = D / 256;
  const int m0 = 2 * tile;
  const int lane = tid & 63, wave = tid >> 6, j = lane & 15, g = lane >> 4;
  const int n_tiles = a.V / 16;
  const int t_lo = (int)((int64_t)blockIdx.x * n_tiles / gridDim.x);
  const int t_hi = (int)((int64_t)(blockIdx.x + 1) * n_tiles / gridDim.x);
  const int rows_here = a.M - m0 < 2 ? a.M - m0 : 2;
  // Every global access below is a buffer access with no branch around it:
  // codes of tiles past the run or of quads past the width, activations past
  // the rows and logits a lane does not own take an out-of-range offset (zeros, no memory request; stores
  // dropped). Loads and stores share one in-order wait counter, and a branch
  // around either made the compiler wait for every access in flight.
  const __amdgpu_buffer_rsrc_t cr =
      __builtin_amdgcn_make_buffer_rsrc((void*)a.words, (short)0, a.V * words * 4, kBufferWord3);
  const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc((void*)a.scales, (short)0, a.V * 4, kBufferWord3);
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc((void*)(a.x + (int64_t)m0 * D), (short)0,
                                                                      rows_here * D * 4, kBufferWord3);
  const __amdgpu_buffer_rsrc_t orr = __builtin_amdgcn_make_buffer_rsrc((void*)(a.out + (int64_t)m0 * a.V), (short)0,
                                                                       rows_here * a.V * 4, kBufferWord3);
  // words 16 q + 4 g .. + 3 of vocabulary row n (block 4 q + g in block-major
  // order) and the row's scale
  auto load = [&](int vt, u32x4 (&cw)[kQatMaxSteps / 4], float& sc) __attribute__((always_inline)) {
    const bool live = vt < t_hi;
    const uint32_t n = (uint32_t)vt * 16u + (uint32_t)j;
#pragma unroll
    for (int q = 0; q < kQatMaxSteps / 4; ++q) {
      const uint32_t off = a.block_major ? ((uint32_t)(4 * q + g) * (uint32_t)a.V + n) * 16u
                                         : (n * (uint32_t)words + (uint32_t)(16 * q + 4 * g)) * 4u;
      cw[q] = __builtin_amdgcn_raw_buffer_load_b128(cr, live && q < quads ? off : kBufferOutOfRange, 0, kQatNT);
    }
    sc = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(sr, live ? n * 4u : kBufferOutOfRange, 0, 0));
  };

  // the check: this thread's word W of row rr (activations 16 W .. 16 W + 15)
  const int rr = tid / words, W = tid - rr * words;
  const bool mine = tid < 2 * words;
  u32x4 xv[4];
#pragma unroll
  for (int v = 0; v < 4; ++v)
    xv[v] = __builtin_amdgcn_raw_buffer_load_b128(xr, mine ? (uint32_t)((rr * D + 16 * W) * 4 + 16 * v) : kBufferOutOfRange,
                                                  0, 0);
  if (tid < 2) { R.emin[tid] = 0x7FFFFFFF; R.bad[tid] = 0; R.sabs[tid] = 0; R.ssum[tid] = 0; }
  __syncthreads();
  // activations of rows past M, and of threads past the words, read zeros
  float f[16];
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    // the elements as scalars first: a bit cast of a vector element
    // subscript reads element 0 here
    const uint32_t xs[4] = {xv[v].x, xv[v].y, xv[v].z, xv[v].w};
#pragma unroll
    for (int e = 0; e < 4; ++e) f[4 * v + e] = (float)srq((double)__builtin_bit_cast(float, xs[e]), a.in_scale);
  }
  // An integer workgroup's first codes load while the rest of the check runs.
  // They go out once the activations are in: issued at the start, the whole
  // grid's first tiles (24 MB at D 1536) queued ahead of the activations' own
  // misses and tripled their latency.
  __builtin_amdgcn_sched_barrier(0);
  u32x4 b0[kQatMaxSteps / 4], b1[kQatMaxSteps / 4];
  float s0, s1;
  int vt = t_lo + wave;
  load(vt, b0, s0);
  __builtin_amdgcn_sched_barrier(0);
  int gmin = 0x7FFFFFFF;
  bool bad = false;
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    uint32_t sig;
    int g;
    if (!act_parts(f[e], &sig, &g)) bad = true;
    else if (sig) gmin = g < gmin ? g : gmin;
  }
  if (mine && gmin != 0x7FFFFFFF) atomicMin(&R.emin[rr], gmin);
  __syncthreads();
  const int E = mine && R.emin[rr] != 0x7FFFFFFF ? R.emin[rr] : 0;
  int64_t A[16];
  uint64_t sabs = 0, ssum = 0;
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    A[e] = 0;
    uint32_t sig = 0;
    int g = 0;
    if (!act_parts(f[e], &sig, &g) || !sig) continue;
    const int sh = g - E;
    if (sh > 62 - 24) { bad = true; continue; }
    const uint64_t mag = (uint64_t)sig << sh;
    if (mag >= kQatSumBound) { bad = true; continue; }
    A[e] = f[e] < 0.0f ? -(int64_t)mag : (int64_t)mag;
    sabs += mag;
    ssum += (uint64_t)A[e];
  }
  if (mine) {
    // (magnitudes below 2^52, at most 2048 of them: the sums do not wrap
    // unless the check fails anyway)
    atomicAdd(&R.sabs[rr], (unsigned long long)sabs);
    atomicAdd(&R.ssum[rr], (unsigned long long)ssum);
    if (bad) atomicOr(&R.bad[rr], 1u);
  }
  __syncthreads();
  bool ok[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) ok[q] = m0 + q < a.M && !R.bad[q] && R.sabs[q] < kQatSumBound;

  const bool any_ok = ok[0] || ok[1];
  // the limbs: tile row 8 rr + l, balanced base-256 digits of A (zeros for a
  // row the check refused), at the operand positions of word W. With
  // K = sum_l 128 256^l (l < 7) and |A| < 2^52, u = A + K has the base-256
  // digits c_l = d_l + 128 in [0, 255]; the int8 digit d_l = c_l - 128 is
  // byte l of u ^ K (byte 7 is zero).
  if (mine && any_ok) {
    const int q = W >> 4, gw = (W >> 2) & 3, tp = W & 3;
    const int step = 4 * q + tp;
    constexpr uint64_t kK = 0x0080808080808080ull;
    static_assert(kQatLimbs == 7, "K holds one 0x80 byte per limb");
    uint32_t* op_words = (uint32_t*)&L.op[step][0];
    // dword t of a limb's operand holds activations 4 i + t (byte i)
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      uint32_t lo[4], hi[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint64_t u = ((uint64_t)(ok[rr] ? A[4 * i + t] : 0) + kK) ^ kK;
        lo[i] = (uint32_t)u;
        hi[i] = (uint32_t)(u >> 32);
      }
#pragma unroll
      for (int l = 0; l < 8; ++l) {
        uint32_t dw = 0u;
#pragma unroll
        for (int i = 0; i < 4; ++i) dw |= (((l < 4 ? lo[i] : hi[i]) >> (8 * (l & 3))) & 0xFFu) << (8 * i);
        op_words[(8 * rr + l + 16 * gw) * 4 + t] = dw;
      }
    }
  }
  __syncthreads();

  auto multiply = [&](int vt, const u32x4 (&cw)[kQatMaxSteps / 4], float sc) __attribute__((always_inline)) {
    i32x4 acc = {0, 0, 0, 0};
#pragma unroll
    for (int q = 0; q < kQatMaxSteps / 4; ++q) {
      if (q < quads) {
        const uint32_t wq[4] = {cw[q].x, cw[q].y, cw[q].z, cw[q].w};
#pragma unroll
        for (int tp = 0; tp < 4; ++tp) {
          const uint32_t w = wq[tp];
          constexpr uint32_t kLow = 0x03030303u;
          const i32x4 b = {(int)(w & kLow), (int)((w >> 2) & kLow), (int)((w >> 4) & kLow), (int)((w >> 6) & kLow)};
          acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(L.op[4 * q + tp][lane], b, acc, 0, 0, 0);
        }
      }
    }
    // lane (j, g) holds tile rows 4 g .. 4 g + 3: row m0 + g / 2, limbs
    // 4 (g & 1) .. + 3; the limbs combine in wrapping 64-bit arithmetic (the
    // total is below 2^53 in magnitude, so the wrapped sum is exact)
    uint64_t p = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) p += (uint64_t)(int64_t)acc[e] << (8 * (4 * (g & 1) + e));
    p += shfl_xor_u64(p, 16);
    const int r = g >> 1;
    const uint32_t n = (uint32_t)vt * 16u + (uint32_t)j;
    const int64_t T = (int64_t)(p - 2 * (uint64_t)R.ssum[r]);
    const double dot = __builtin_ldexp((double)T, R.emin[r] != 0x7FFFFFFF ? R.emin[r] : 0);
    const float y = (float)srq(dot * (double)sc, a.out_scale);
    const bool st = (g & 1) == 0 && ok[r] && vt < t_hi;
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, y), orr,
                                          st ? ((uint32_t)r * (uint32_t)a.V + n) * 4u : kBufferOutOfRange, 0, 0);
  };
  // two register buffers with fixed roles: tile t multiplies from one while
  // tile t + 16 loads into the other (the first load went out with the
  // check); tiles past the run read zeros and store nothing
  if (any_ok) {
    for (; vt < t_hi; vt += 2 * kQatTileWaves) {
      load(vt + kQatTileWaves, b1, s1);
      multiply(vt, b0, s0);
      load(vt + 2 * kQatTileWaves, b0, s0);
      multiply(vt + kQatTileWaves, b1, s1);
    }
  }
  // rows the check refused: the binary64 path over this run's vocabulary
  // rows, the activations staged where the operand tile was
  const bool skip[2] = {ok[0], ok[1]};
  if (!(skip[0] && (skip[1] || m0 + 1 >= a.M))) {
    __syncthreads();
    qat_stage_act<2, kQatTileThreads>(a, m0, L.act);
    for (int64_t r = (int64_t)t_lo * 16 + tid; r < (int64_t)t_hi * 16; r += kQatTileThreads)
      qat_row_binary64<2>(a, m0, skip, L.act, r);
  }
}

}  // namespace

// rows of x per pass for width D (the LDS stage holds kQatLdsDoubles)
int qat_rows_per_pass(int32_t D) {
  const int r = kQatLdsDoubles / D;
  return r >= 4 ? 4 : (r >= 2 ? 2 : 1);
}


void launch_qat_lmhead(const float* x, int32_t M, int32_t D, const uint32_t* words, int32_t block_major,
                       const float* scales, int32_t V, double in_scale, double out_scale, float* out,
                       int32_t cu_count, hipStream_t s, LaunchEvents ev) {
  QatArgs a{x, words, scales, out, D, V, M, block_major, in_scale, out_scale};
  if (D % 256 == 0 && D <= 2048 && V % 16 == 0) {
    // one launch per pair of rows, one workgroup per compute unit
    const int tiles = (M + 1) / 2;
    for (int t = 0; t < tiles; ++t) {
      hipExtLaunchKernelGGL(qat_tile_kernel, dim3(cu_count > 0 ? cu_count : 256), dim3(kQatTileThreads), 0, s,
                            t == 0 ? ev.start : nullptr, t == tiles - 1 ? ev.stop : nullptr, 0, a, t);
    }
    return;
  }
  const dim3 grid((unsigned)((V + kQatThreads - 1) / kQatThreads));
  const int most = qat_rows_per_pass(D);
  for (int32_t m0 = 0; m0 < M;) {
    // as many rows of x as the stage holds and remain, in a kernel made for that many
    const int left = M - m0;
    const int per = most >= 4 && left >= 4 ? 4 : (most >= 2 && left >= 2 ? 2 : 1);
    const bool last = m0 + per >= M;
    hipEvent_t start = m0 == 0 ? ev.start : nullptr, stop = last ? ev.stop : nullptr;
    if (per == 4) hipExtLaunchKernelGGL(qat_lmhead_kernel<4>, grid, dim3(kQatThreads), 0, s, start, stop, 0, a, m0);
    else if (per == 2) hipExtLaunchKernelGGL(qat_lmhead_kernel<2>, grid, dim3(kQatThreads), 0, s, start, stop, 0, a, m0);
    else hipExtLaunchKernelGGL(qat_lmhead_kernel<1>, grid, dim3(kQatThreads), 0, s, start, stop, 0, a, m0);
    m0 += per;
  }
}

}  // namespace gs
