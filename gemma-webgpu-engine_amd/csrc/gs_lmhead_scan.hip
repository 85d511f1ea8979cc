// The lm_head fused with the sampler's streaming pass: the chunk scan's
// statistics and candidate lists come out of the GEMM's epilogue, so the
// logits are never read back (C5: logits = softcap(H W^T), then sampling;
// the reference's handoff this replaces is src/webgpu/decode-model.ts:127-150,
// its producer src/webgpu/decode-lm-head.ts:262-340).
//
// Three launches replace lmhead_kernel + scan_kernel:
//   * dead_bitmap_kernel, 16384 ids per workgroup: a row's excluded ids as a
//     bitmap [rows][V/32] -- the ids its constraint mask forbids, its penalty
//     window and its forced ids (the ids the scan leaves to the finish's exact
//     evaluation) -- and the row's threshold word cleared;
//   * lmhead_scan_kernel: the bf16 MFMA GEMM of lmhead_kernel over 256 vocab
//     rows per workgroup (eight waves of one 32-row tile each, every wave with
//     lmhead_kernel's register ring and per-lane K order, so the logits are
//     bit-identical), the same softcap epilogue and
//     non-temporal logits stores; then, per hidden row, the 256 logits of the
//     workgroup's "partial" go through LDS into one statistics record and one
//     candidate list, computed like a scan wave's: 16 lanes of 16 logits, the
//     lane maxima, the normaliser in binary32 terms against each lane's maximum
//     rescaled to the partial's, and every finite logit >= tau, tau the d-th
//     largest lane maximum (d = 4 for top-k rows, 8 otherwise);
//   * merge_parts_kernel, one workgroup per (chunk, row): the 32 partials of a
//     8192-id chunk become the scan's ChunkStat and lists -- wave entry w from
//     partials 8w .. 8w+7, the maximum, the normaliser rescaled once more, and
//     the sub-list of the listed entries at or above the row's threshold.
//
// Threshold. Each partial lists everything >= its own tau; the row's
// threshold is the largest tau of its truncated partials (an atomic maximum
// per row), so the entries >= it are exactly the row's logits >= it: the
// complete region the finish kernel works in. A partial of 256 ids guarantees
// only d entries at or above its tau, but over the 1024 partials of a
// 262144-id row the region holds far more (88 at least, 440 typically, over
// 300 rows of N(0, 3^2) logits with and without a 3%-legal mask, for d = 4);
// a region smaller than the cut the row needs takes the finish kernel's
// slower paths, which read the logits, as they do after the scan.
//
// The logits are still written: the finish evaluates its special ids and the
// exact and deep paths replay rows from them.
#include "gs_exp2.h"
#include "gs_internal.h"

namespace gs {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kFThreads = 512;  // eight waves, one 32-row vocab tile each
constexpr int kFM = 64;       // hidden rows per workgroup
constexpr int kFKBlock = 64;
constexpr int kFPad = 72;     // LDS row length of the H block in bf16 (64 + 8)
constexpr int kFDeadWords = kPartIds / 32;

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

// What a partial's statistics need of its row's configuration, read once per
// workgroup at its start (the reads then overlap the weight stream).
struct RowParam {
  double A;        // 256 log2(e) / T
  double softcap;  // the sampler's own cap (> 0: applied to the head's logits)
  float c32;       // A / 256 rounded to binary32
  int32_t route;   // Route; kRouteExact for rows past M (nothing written)
};

struct FusedShared {
  union __attribute__((aligned(16))) {
    uint16_t a[2][kFM][kFPad];  // the H block, double-buffered (K loop)
    float t[32][kPartIds];      // one 32-row M tile of capped logits, row-major (epilogue)
  } u;
  uint32_t dead[kFM][kFDeadWords];  // excluded ids of the partial, per hidden row
  RowParam rp[kFM];
  double tab[256];
};

// The d-th largest key of the 16 lanes of this lane's segment (segmask), as
// wave_kth_key: a lower bound at most 2^14 below it, found bit by bit with
// ballots from the first bit where the segment's smallest and largest keys
// differ. Segments leave the loop at different bits; a ballot counts the
// lanes still in it, and the mask keeps the count to the segment.
__device__ __forceinline__ uint32_t seg_kth_key(uint32_t key, uint32_t d, uint32_t lo, uint32_t hi,
                                                uint64_t segmask) {
  constexpr int kFloorBit = 14;
  const uint32_t diff = lo ^ hi;
  if (diff >> kFloorBit == 0) return lo & ~((1u << kFloorBit) - 1u);
  const int top = 31 - __builtin_clz(diff);
  uint32_t t = lo & ~((2u << top) - 1u);
  for (int b = top; b >= kFloorBit; --b) {
    const uint32_t c = t | (1u << b);
    if ((uint32_t)__popcll(__ballot(key >= c) & segmask) >= d) t = c;
  }
  return t;
}

// One hidden row's partial (this lane's 16 logits x of the row's 256, ids
// id0 .. id0 + 15): its statistics record and candidate list. The 16 lanes of
// a segment hold one row; every branch below is uniform over a segment, and
// each cross-lane step stays inside it (xor distances below 16).
__device__ __forceinline__ void partial_stats(float (&x)[16], const uint32_t dead_bits, const uint32_t id0,
                                              const RowParam rp, const uint64_t segmask, const double* s_tab,
                                              PartStat* ps, uint64_t* plist, uint32_t* row_thr) {
  const int lane = threadIdx.x & 63;
  const int j = lane & 15;
  const bool active = rp.route != kRouteExact;
  if (rp.softcap > 0) {
#pragma unroll
    for (int e = 0; e < 16; ++e) x[e] = gsm::softcap_f32(x[e], rp.softcap);
  }
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    if ((dead_bits >> e) & 1u) x[e] = -__builtin_inff();
  }
  float tmax = -__builtin_inff();
#pragma unroll
  for (int e = 0; e < 16; ++e) tmax = __builtin_elementwise_maximum(tmax, x[e]);
  const bool finite_max = tmax > -__builtin_inff() && tmax < __builtin_inff();
  const bool thread_bad = !(tmax < __builtin_inff());

  if (rp.route == kRouteGreedy) {
    // the partial's first maximum (the lowest id holding the largest value)
    uint32_t gid = 0xFFFFFFFFu;
#pragma unroll
    for (int e = 15; e >= 0; --e) {
      if (x[e] == tmax) gid = id0 + (uint32_t)e;
    }
    uint64_t best = gid != 0xFFFFFFFFu ? pack_entry(f32_key(tmax), gid) : 0ull;
    uint32_t bad = thread_bad ? 1u : 0u;
#pragma unroll
    for (int m = 8; m > 0; m >>= 1) {
      const uint64_t o = shfl_xor_u64(best, m);
      best = o > best ? o : best;
      bad |= shfl_xor_u32(bad, m);
    }
    if (j == 0 && active) {
      if (best) plist[0] = list_slot(__builtin_bit_cast(uint32_t, key_f32(entry_key(best))), entry_id(best));
      PartStat st{};
      st.max_key = entry_key(best);
      st.tau = entry_key(best);
      st.n = best ? 1u : 0u;
      st.flags = bad ? kChunkNonFinite : 0u;
      *ps = st;
    }
    return;
  }

  // the lane's sum of e^((l - tmax)/T) as in the chunk scan: binary32 terms
  // 2^(x c - B), one fma and one hardware exp2 each, added in pairs in
  // binary32 and the pairs in binary64; B's rounding divided out below
  const double A = rp.A;
  const float c32 = rp.c32;
  double sum = 0.0;
  float berr = 0.0f;
  bool scale_bad = false;
  if (finite_max) {
    const float B = tmax * c32;
    berr = __builtin_fmaf(tmax, c32, -B);
    scale_bad = !(__builtin_fabsf(B) < __builtin_inff()) || !(berr == berr);
#pragma unroll
    for (int e = 0; e < 16; e += 2) {
      const float t0 = __builtin_amdgcn_exp2f(__builtin_fmaf(x[e], c32, -B));
      const float t1 = __builtin_amdgcn_exp2f(__builtin_fmaf(x[e + 1], c32, -B));
      sum += (double)(t0 + t1);
    }
  }
  const uint32_t mykey = finite_max ? f32_key(tmax) : 0u;
  uint32_t wm = mykey, wlo = mykey, bad = (thread_bad || scale_bad) ? 1u : 0u;
#pragma unroll
  for (int m = 8; m > 0; m >>= 1) {
    const uint32_t a = shfl_xor_u32(wm, m), b = shfl_xor_u32(wlo, m);
    wm = a > wm ? a : wm;
    wlo = b < wlo ? b : wlo;
    bad |= shfl_xor_u32(bad, m);
  }
  if (bad) {
    // NaN or +inf among the live logits: outside the one-pass contract
    if (j == 0 && active) {
      PartStat st{};
      st.max_key = wm;
      st.flags = kChunkNonFinite;
      *ps = st;
    }
    return;
  }
  double part = 0.0;
  if (finite_max && sum > 0.0) {
    const double y = ((double)tmax - (double)key_f32(wm)) * A - 256.0 * (double)berr;
    part = y > kSkipY ? sum * exp2_256(y, s_tab) : 0.0;
  }
  // xor butterfly: each step adds the same two operands in every lane of a
  // pair, so every lane ends with the same sum
#pragma unroll
  for (int m = 1; m < 16; m <<= 1) part += shfl_xor_f64(part, m);

  const uint32_t d = rp.route == kRouteTopK ? 4u : 8u;
  const uint32_t lanes = (uint32_t)__popcll(__ballot(mykey != 0u) & segmask);
  const bool selected = lanes >= d;
  // (a tau at or below -inf's key lists every finite logit, as in the scan)
  uint32_t thr = kKeyNegInf + 1u;
  if (selected) {
    const uint32_t t = seg_kth_key(mykey, d, wlo, wm, segmask);
    thr = t > kKeyNegInf ? t : kKeyNegInf + 1u;
  }
  const float tf = key_f32(thr);

  // every finite logit >= tau, at positions taken from segment ballots
  const uint64_t below = (1ull << lane) - 1ull;
  uint32_t off = 0;
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const bool take = x[e] >= tf;
    const uint64_t m = __ballot(take) & segmask;
    if (m) {
      if (take && active) {
        const uint32_t pos = off + (uint32_t)__popcll(m & below);
        if (pos < (uint32_t)kPartCap) plist[pos] = list_slot(__builtin_bit_cast(uint32_t, x[e]), id0 + (uint32_t)e);
      }
      off += (uint32_t)__popcll(m);
    }
  }
  if (j == 0 && active) {
    PartStat st{};
    st.sum = part;
    st.max_key = wm;
    st.tau = thr;
    st.n = off;
    st.truncated = selected ? 1u : 0u;
    *ps = st;
    if (selected) atomicMax(row_thr, thr);
  }
}

template <int kDepth>
__global__ __launch_bounds__(kFThreads, 2) void lmhead_scan_kernel(const uint16_t* __restrict__ H,
                                                                   const uint16_t* __restrict__ W, int M, int D,
                                                                   int V, float cap, float* __restrict__ out,
                                                                   FusedArgs f) {
  __shared__ FusedShared S;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h = lane >> 5;
  const int slab = blockIdx.x;
  const int n0 = slab * kPartIds + wave * 32;  // the wave's tile: vocab rows n0 + (lane & 31)
  const int m0 = blockIdx.y * kFM;
  // the excluded-id words of the partial for the workgroup's 64 hidden rows
  // (thread t < 512: row t / 8, word t % 8), loaded first
  const int64_t vwords = V / 32;
  const int dr = tid >> 3;
  const uint32_t dw =
      m0 + dr < M ? f.dead[(int64_t)(m0 + dr) * vwords + (int64_t)slab * kFDeadWords + (tid & 7)] : 0xFFFFFFFFu;
  // the rows' configurations (thread t < 64: row m0 + t)
  gs_row_config cfg{};
  const bool cfg_row = tid < kFM && m0 + tid < M;
  if (cfg_row) cfg = f.configs[m0 + tid];
  const int nr = n0 + (lane & 31);
  const uint16_t* wrow = W + (size_t)(nr < V ? nr : V - 1) * D + h * 32;
  // H: thread t stages 16 bytes of row t/8 of the 64x64 block (rows past M
  // read row M-1 and are stored as zeros)
  const int ar = tid >> 3, ac = (tid & 7) * 8;
  const bool a_live = m0 + ar < M;
  const uint16_t* hrow = H + (size_t)(a_live ? m0 + ar : M - 1) * D + ac;

  // lmhead_kernel's register ring: kDepth K blocks in flight, the loop
  // unrolled by kDepth and branch-free (prefetches past the last block
  // re-read it)
  const int nk = D / kFKBlock;
  uint4 wr[kDepth][4], hr[kDepth];
  auto issue = [&](int slot, int kb) __attribute__((always_inline)) {
    kb = kb < nk ? kb : nk - 1;
    const uint4* pw = (const uint4*)(wrow + (size_t)kb * kFKBlock);
#pragma unroll
    for (int i = 0; i < 4; ++i) wr[slot][i] = pw[i];
    hr[slot] = *(const uint4*)(hrow + (size_t)kb * kFKBlock);
  };
  const uint32_t a_mask = a_live ? 0xFFFFFFFFu : 0u;
  auto stage_h = [&](int buf, int slot) __attribute__((always_inline)) {
    const uint4 v = hr[slot];
    *(uint4*)&S.u.a[buf][ar][ac] = make_uint4(v.x & a_mask, v.y & a_mask, v.z & a_mask, v.w & a_mask);
  };

  f32x16 acc0, acc1;  // M tiles 0 and 1
#pragma unroll
  for (int i = 0; i < 16; ++i) { acc0[i] = 0.0f; acc1[i] = 0.0f; }
  auto step = [&](int kbi, int p) __attribute__((always_inline)) {
    const int buf = kbi & 1;
    stage_h(buf ^ 1, (p + 1) % kDepth);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const bf16x8 bf = as_bf16x8(wr[p][s]);
      const bf16x8 a0 = as_bf16x8(*(const uint4*)&S.u.a[buf][lane & 31][h * 32 + s * 8]);
      const bf16x8 a1 = as_bf16x8(*(const uint4*)&S.u.a[buf][32 + (lane & 31)][h * 32 + s * 8]);
      acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, bf, acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, bf, acc1, 0, 0, 0);
    }
    issue(p, kbi + kDepth);
    __syncthreads();
  };
#pragma unroll
  for (int p = 0; p < kDepth; ++p) issue(p, p);
  S.dead[dr][tid & 7] = dw;
  if (tid < 256) S.tab[tid] = c_exp2_256[tid];
  if (tid < kFM) {
    RowParam rp{};
    rp.route = kRouteExact;
    if (cfg_row) {
      rp.route = plan_row_flat(cfg).route;
      rp.A = (1.0 / cfg.temperature) * GS_256_LOG2E;
      rp.c32 = (float)(rp.A * (1.0 / 256.0));
      rp.softcap = cfg.softcap;
    }
    S.rp[tid] = rp;
  }
  stage_h(0, 0);
  __syncthreads();
  const int n_main = nk - nk % kDepth;
  for (int kb0 = 0; kb0 < n_main; kb0 += kDepth) {
#pragma unroll
    for (int p = 0; p < kDepth; ++p) step(kb0 + p, p);
  }
#pragma unroll
  for (int p = 0; p < kDepth - 1; ++p) {
    if (n_main + p < nk) step(n_main + p, p);
  }
  // (the last step ended with a barrier: the H block is no longer read)

  // softcap and the logits stores, as lmhead_kernel. D layout of a 32x32
  // tile: lane l, register r -> column l % 32, row 8 (r / 4) + 4 (l / 32) + r % 4
  const int nl = lane & 31;
  const int n = n0 + nl;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int row = 8 * (r >> 2) + 4 * h + (r & 3);
    if (cap > 0.0f) {
      acc0[r] = cap * tanhf(acc0[r] / cap);
      acc1[r] = cap * tanhf(acc1[r] / cap);
    }
    if (m0 + row < M && n < V) __builtin_nontemporal_store(acc0[r], &out[(size_t)(m0 + row) * V + n]);
    if (m0 + 32 + row < M && n < V) __builtin_nontemporal_store(acc1[r], &out[(size_t)(m0 + 32 + row) * V + n]);
  }

  // the partials, one 32-row M tile at a time through LDS: segment s of wave
  // w takes row 4 w + s of the tile, lane j of the segment its logits
  // 16 j .. 16 j + 15
  const int seg = lane >> 4, j = lane & 15;
  const uint64_t segmask = 0xFFFFull << (16 * seg);
#pragma unroll
  for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
    for (int r = 0; r < 16; ++r) S.u.t[8 * (r >> 2) + 4 * h + (r & 3)][32 * wave + nl] = mt ? acc1[r] : acc0[r];
    lds_barrier();
    const int rl = 4 * wave + seg;  // row within the tile
    const int ml = 32 * mt + rl;    // row within the workgroup
    const int64_t grow = (int64_t)m0 + ml;
    const bool live = grow < M;
    float x[16];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float4 v = *(const float4*)&S.u.t[rl][16 * j + 4 * q];
      x[4 * q] = v.x; x[4 * q + 1] = v.y; x[4 * q + 2] = v.z; x[4 * q + 3] = v.w;
    }
    const uint32_t dead_bits = (S.dead[ml][j >> 1] >> (16 * (j & 1))) & 0xFFFFu;
    const int64_t pidx = (live ? grow : 0) * f.n_parts + slab;
    partial_stats(x, dead_bits, (uint32_t)(slab * kPartIds + 16 * j), S.rp[ml], segmask, S.tab, f.parts + pidx,
                  f.plists + pidx * kPartCap, f.row_thr + (live ? grow : 0));
    lds_barrier();
  }
}

// Row blockIdx.y's excluded ids, words [kDeadSpan x, kDeadSpan (x + 1)) of
// its bitmap (x = blockIdx.x): the ids the row's mask forbids (constrained
// rows), its penalty window and its forced ids (constrained rows) -- the sets
// the chunk scan leaves out -- assembled in LDS and stored once; the first
// workgroup of a row also clears its threshold word.
constexpr int kDeadSpan = 512;
__global__ __launch_bounds__(256) void dead_bitmap_kernel(SampleArgs a, FusedArgs f) {
  __shared__ uint32_t words[kDeadSpan];
  const int tid = threadIdx.x;
  const int64_t row = blockIdx.y;
  const int64_t w_base = (int64_t)blockIdx.x * kDeadSpan;
  const int64_t nw = a.mask_words;
  const gs_row_config cfg = a.configs[row];
  const bool constrained = cfg.mask_slot >= 0 && cfg.mask_slot < a.mask_slots;
  int64_t w0, w1;
  history_window(a, row, cfg, &w0, &w1);
  const bool forced = constrained && a.forced_offsets;
  const int64_t f0 = forced ? a.forced_offsets[row] : 0, f1 = forced ? a.forced_offsets[row + 1] : 0;
  const uint32_t* mk = constrained ? a.mask_table + (int64_t)cfg.mask_slot * a.mask_words : nullptr;
  for (int k = tid; k < kDeadSpan; k += 256) {
    const int64_t w = w_base + k;
    words[k] = constrained && w < nw ? ~mk[w] : 0u;
  }
  __syncthreads();
  const uint32_t id_lo = (uint32_t)(w_base * 32);
  auto mark = [&](int32_t id) {
    const uint32_t loc = (uint32_t)id - id_lo;
    if (id >= 0 && id < a.vocab && loc < (uint32_t)(kDeadSpan * 32)) atomicOr(&words[loc >> 5], 1u << (loc & 31));
  };
  for (int64_t i = w0 + tid; i < w1; i += 256) mark(a.history_ids[i]);
  for (int64_t i = f0 + tid; i < f1; i += 256) mark(a.forced_ids[i]);
  __syncthreads();
  for (int k = tid; k < kDeadSpan; k += 256) {
    const int64_t w = w_base + k;
    if (w < nw) f.dead[row * nw + w] = words[k];
  }
  if (blockIdx.x == 0 && tid == 0) f.row_thr[row] = 0u;
}

// The scan's ChunkStat and lists of chunk blockIdx.x of row blockIdx.y from
// its kPartsPerChunk partials (wave w: partials kPartsPerWave w ..).
__global__ __launch_bounds__(kScanThreads) void merge_parts_kernel(SampleArgs a, FusedArgs f) {
  constexpr int kPartsPerWave = kPartsPerChunk / kScanWaves;  // 8
  __shared__ double tab[256];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int chunk = blockIdx.x;
  const int64_t row = blockIdx.y;
  tab[tid] = c_exp2_256[tid];
  const gs_row_config cfg = a.configs[row];
  const Plan plan = plan_row(cfg);
  const uint32_t rthr = f.row_thr[row];
  __syncthreads();
  if (plan.route != kRouteExact) {
    // lane i < 32 of every wave holds partial i of the chunk
    const bool holds = lane < kPartsPerChunk;
    const int64_t p0 = row * f.n_parts + (int64_t)chunk * kPartsPerChunk;
    PartStat p{};
    if (holds) p = f.parts[p0 + lane];
    const uint64_t* pl = f.plists + p0 * kPartCap;
    ChunkStat* stat = a.stats + row * a.n_chunks + chunk;
    uint64_t* list = a.lists + (row * a.n_chunks + chunk) * kGatherCap;
    if (plan.route == kRouteGreedy) {
      uint64_t best = holds && p.n ? list_rank(pl[(int64_t)lane * kPartCap]) : 0ull;
      best = wave_max_u64(best);
      const uint32_t anybad = wave_or_u32(holds ? p.flags : 0u);
      if (tid == 0) {
        if (best) list[0] = list_slot(__builtin_bit_cast(uint32_t, key_f32(entry_key(best))), entry_id(best));
        ChunkStat st{};
        st.wmax[0] = entry_key(best);
        st.wflags[0] = (anybad & kChunkNonFinite) ? kChunkNonFinite : 0u;
        st.threshold = entry_key(best);
        st.n_sub[0] = best ? 1u : 0u;
        *stat = st;
      }
    } else {
      const bool cbad = (wave_or_u32(holds ? p.flags : 0u) & kChunkNonFinite) != 0u;
      const bool mine = holds && lane / kPartsPerWave == wave;
      const uint32_t wm = wave_max_u32(mine ? p.max_key : 0u);
      if (cbad) {
        if (lane == 0) {
          stat->wmax[wave] = wm;
          stat->wsum[wave] = 0.0;
          stat->wflags[wave] = kChunkNonFinite;
          stat->n_sub[wave] = 0;
          if (wave == 0) { stat->threshold = 0; stat->truncated = 0; }
        }
      } else {
        // the wave entry's normaliser: each partial's, rescaled from its
        // maximum to the entry's (binary64 sums in a fixed order)
        const double A = (1.0 / cfg.temperature) * GS_256_LOG2E;
        double part = 0.0;
        if (mine && p.sum > 0.0) {
          const double y = ((double)key_f32(p.max_key) - (double)key_f32(wm)) * A;
          part = y > kSkipY ? p.sum * exp2_256(y, tab) : 0.0;
        }
        part = wave_sum_f64_dpp(part);
        // the entry's sub-list: its partials' entries at or above the row's
        // threshold (every listed entry when no partial of the row truncated)
        const uint32_t thr = rthr ? rthr : kKeyNegInf + 1u;
        const uint32_t pn = holds ? p.n : 0u;
        const bool over = __ballot(mine && pn > (uint32_t)kPartCap) != 0;
        uint64_t* sub = list + wave * kSubCap;
        const uint64_t below = (1ull << lane) - 1ull;
        uint32_t off = 0;
#pragma unroll
        for (int q = 0; q < kPartsPerWave * kPartCap / 64; ++q) {
          const int s = lane + 64 * q;
          const int pp = kPartsPerWave * wave + s / kPartCap;  // partial within the chunk
          const int k = s % kPartCap;
          const uint32_t n_pp = (uint32_t)__shfl((int)pn, pp, 64);
          const uint32_t cnt = n_pp < (uint32_t)kPartCap ? n_pp : (uint32_t)kPartCap;
          uint64_t slot = 0;
          bool keep = false;
          if ((uint32_t)k < cnt) {
            slot = pl[(int64_t)pp * kPartCap + k];
            keep = entry_key(list_rank(slot)) >= thr;
          }
          const uint64_t m = __ballot(keep);
          if (keep) {
            const uint32_t pos = off + (uint32_t)__popcll(m & below);
            if (pos < (uint32_t)kSubCap) sub[pos] = slot;
          }
          off += (uint32_t)__popcll(m);
        }
        if (over && off <= (uint32_t)kSubCap) off = kSubCap + 1;  // a partial list was cut: incomplete
        if (lane == 0) {
          stat->wsum[wave] = part;
          stat->wmax[wave] = wm;
          stat->wflags[wave] = 0u;
          stat->n_sub[wave] = (uint16_t)(off < 0xFFFFu ? off : 0xFFFFu);
          if (wave == 0) {
            stat->threshold = thr;
            stat->truncated = rthr ? 1u : 0u;
          }
        }
      }
    }
  }
  // reset the queues the finish kernel fills for the exact and deep kernels,
  // as the chunk scan does (this kernel takes its place on the stream)
  if (row == 0 && chunk == 0 && tid == 0) {
    a.queue->count = 0;
    a.queue->next = 0;
    if (a.deep_queue) {
      a.deep_queue->count1 = 0;
      a.deep_queue->next1 = 0;
      a.deep_queue->count2 = 0;
      a.deep_queue->next2 = 0;
    }
  }
}

}  // namespace

void launch_lmhead_scan(const uint16_t* hidden, const uint16_t* weight, int32_t m, int32_t width, float softcap,
                        float* out, const SampleArgs& a, const FusedArgs& f, hipStream_t s, LaunchEvents ev) {
  const dim3 pre((a.mask_words + kDeadSpan - 1) / kDeadSpan, a.rows);
  hipExtLaunchKernelGGL(dead_bitmap_kernel, pre, dim3(256), 0, s, ev.start, nullptr, 0, a, f);
  dim3 grid(a.vocab / kPartIds, (m + kFM - 1) / kFM);
  hipExtLaunchKernelGGL(lmhead_scan_kernel<3>, grid, dim3(kFThreads), 0, s, nullptr, ev.stop, 0, hidden, weight, m,
                        width, a.vocab, softcap, out, f);
}

void launch_merge_parts(const SampleArgs& a, const FusedArgs& f, hipStream_t s, LaunchEvents ev) {
  hipExtLaunchKernelGGL(merge_parts_kernel, dim3(a.n_chunks, a.rows), dim3(kScanThreads), 0, s, ev.start, ev.stop, 0,
                        a, f);
}

}  // namespace gs
