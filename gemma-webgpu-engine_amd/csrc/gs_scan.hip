// One-pass chunk scan: the streaming half of the batched sampler.
//
// Grid (n_chunks, rows); one 256-thread workgroup reads one 8192-logit chunk
// of one row exactly once from HBM. Every 16-byte load of a thread is issued
// before any of them is used, so the whole chunk is in flight at once, and
// the history-window ids the chunk needs are read while it lands. Per chunk
// the workgroup emits:
//   * the chunk maximum and sum_i e^((l_i - lmax)/T) in binary64, the pieces
//     of the reference's softmax normaliser (src/runtime/sampling.ts:36-41).
//     Each thread sums against its own maximum, so no barrier precedes the
//     sum, and the 256 partial sums are rescaled to the chunk maximum after;
//   * a candidate list: every finite logit >= tau, where tau comes from a
//     radix select over the 256 per-thread maxima such that at least `depth`
//     of them are >= tau. The list therefore holds the chunk's top-`depth` in
//     the reference's (value desc, id asc) order (sampling.ts:33-35) and every
//     finite logit of the chunk >= tau. Each wave appends to a sub-list of
//     its own at positions taken from ballots, so no atomics are involved.
// Logits of "special" ids (the row's penalty window and forced ids) are left
// out here; the finish kernel evaluates them exactly. Masked ids (constraint
// bitmask) are -inf, as maskConstraintLogits makes them
// (src/runtime/constraints.ts:159-173).
//
// The normaliser's exponential is 2^(y/256) = 2^(j/256) * 2^k * e^r with a
// correctly rounded 256-entry table and a quadratic in r, |r| <= ln2/512:
// relative error below 4.2e-10 per term. Only the normaliser sees it, and only
// the top-p cut depends on the normaliser (its margin in the finish kernel
// covers this); every ordering and every probability the filters compare is
// recomputed exactly later.
#include "gs_exp2_table.h"
#include "gs_internal.h"

namespace gs {
namespace {

__constant__ double c_exp2_256[256] = {GS_EXP2_TABLE_256};

// Terms with (l - lmax)/T < -60 are not summed: each is below e^-60 of the
// maximum's term, so together they move the normaliser by less than
// V * e^-60 < 3e-21 relative. In units of y = 256 log2(e) (l - lmax)/T:
constexpr double kSkipY = -22160.0;

__device__ __forceinline__ double exp2_256(double y, const double* tab) {
  const double n = __builtin_rint(y);
  const double s = y - n;  // |s| <= 1/2
  const double p = __builtin_fma(s, __builtin_fma(s, GS_EXP2_256_C2, GS_EXP2_256_C1), 1.0);
  const int ni = (int)n;
  return __builtin_ldexp(tab[ni & 255] * p, ni >> 8);
}

template <typename In>
struct VecTraits;
template <>
struct VecTraits<float> {
  static constexpr int kVec = 4;  // logits per 16-byte load
  __device__ static uint32_t bits(const uint4& v, int j) {
    return j == 0 ? v.x : (j == 1 ? v.y : (j == 2 ? v.z : v.w));
  }
  __device__ static uint32_t one(const float* p) { return __builtin_bit_cast(uint32_t, *p); }
};
template <>
struct VecTraits<uint16_t> {
  static constexpr int kVec = 8;
  __device__ static uint32_t bits(const uint4& v, int j) {
    const uint32_t w = (j >> 1) == 0 ? v.x : ((j >> 1) == 1 ? v.y : ((j >> 1) == 2 ? v.z : v.w));
    return (j & 1) ? (w & 0xFFFF0000u) : (w << 16);
  }
  __device__ static uint32_t one(const uint16_t* p) { return (uint32_t)(*p) << 16; }
};

__device__ __noinline__ float capped(float x, double cap) { return gsm::softcap_f32(x, cap); }

// Threshold t over the u32 keys s_keys[0..kScanThreads): at least k keys are
// >= t (every key when fewer than k are non-zero) and, once an 8-bit digit
// narrows the count to k + slack or fewer, at most that many. MSB-first radix
// select with LDS histograms; every thread returns the same t.
__device__ uint32_t radix_floor(const uint32_t* s_keys, uint32_t* s_hist, uint32_t* s_sel, uint32_t k,
                                uint32_t slack) {
  const int tid = threadIdx.x;
  uint32_t prefix = 0, above = 0;
  for (int shift = 24; shift >= 0; shift -= 8) {
    s_hist[tid] = 0;
    __syncthreads();
    const uint32_t hi_mask = shift == 24 ? 0u : (0xFFFFFFFFu << (shift + 8));
    const uint32_t key = s_keys[tid];
    if ((key & hi_mask) == prefix) atomicAdd(&s_hist[(key >> shift) & 255u], 1u);
    __syncthreads();
    if (tid < 64) {
      // lane l holds bins 255-4l .. 252-4l, highest first
      uint32_t h[4], s = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q) { h[q] = s_hist[255 - 4 * tid - q]; s += h[q]; }
      const uint32_t incl = wave_scan_u32(s, tid);
      const uint64_t hit = __ballot(above + incl >= k);
      if (hit == 0) {
        // fewer than k keys share the prefix (first digit only): take them all
        if (tid == 63) { s_sel[0] = prefix; s_sel[1] = above; s_sel[2] = above + incl; s_sel[3] = 1; }
      } else if (tid == __ffsll((unsigned long long)hit) - 1) {
        uint32_t c = above + incl - s;
        int q = 0;
        while (q < 3 && c + h[q] < k) { c += h[q]; ++q; }
        s_sel[0] = prefix | ((uint32_t)(255 - 4 * tid - q) << shift);
        s_sel[1] = c;
        s_sel[2] = c + h[q];
        s_sel[3] = 0;
      }
    }
    __syncthreads();
    prefix = s_sel[0];
    above = s_sel[1];
    const uint32_t total = s_sel[2];
    const bool all = s_sel[3] != 0;
    if (all || total <= k + slack) return prefix;
  }
  return prefix;
}

struct ScanShared {
  uint32_t special[kChunk / 32];
  double tab[256];
  uint32_t keys[kScanThreads];
  uint32_t hist[256];
  uint32_t sel[4];
  double wsum[kScanWaves];
  uint32_t wmax[kScanWaves];
  uint32_t wbad[kScanWaves];
  uint32_t wlanes[kScanWaves];
  uint32_t wgather[kScanWaves];
  uint64_t wbest[kScanWaves];
};

// One chunk. kFull: all kChunk logits exist and rows are 16-byte aligned;
// kMasked: the row has a constraint mask. Each combination is straight-line
// code from the first load to the first barrier, so the only wait before the
// barrier is for the loads issued ahead of the chunk.
template <typename In, bool kFull, bool kMasked>
__device__ __forceinline__ void scan_chunk(const SampleArgs& a, const gs_row_config& cfg, const Plan plan,
                                           const int64_t row, const int chunk, const int n_valid, ScanShared& S) {
  using VT = VecTraits<In>;
  constexpr int kVec = VT::kVec;
  constexpr int kLoads = kElemsPerThread / kVec;
  constexpr uint32_t kLaneBits = (1u << kVec) - 1u;
  uint32_t* s_special = S.special;
  double* s_tab = S.tab;
  uint32_t* s_keys = S.keys;
  uint32_t* s_hist = S.hist;
  uint32_t* s_sel = S.sel;
  double* s_wsum = S.wsum;
  uint32_t* s_wmax = S.wmax;
  uint32_t* s_wbad = S.wbad;
  uint32_t* s_wlanes = S.wlanes;
  uint32_t* s_wgather = S.wgather;
  uint64_t* s_wbest = S.wbest;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bool greedy = plan.route == kRouteGreedy;
  const int64_t gbase = (int64_t)chunk * kChunk;
  const int32_t slot = cfg.mask_slot;
  ChunkStat* stat = a.stats + row * a.n_chunks + chunk;
  uint64_t* list = a.lists + (row * a.n_chunks + chunk) * kGatherCap;
  // any valid device address, read in place of absent inputs so that no load
  // sits under a branch
  const int32_t* dummy = (const int32_t*)a.configs;

  // -- loads the chunk does not wait for go first: the first window and
  //    forced ids and this thread's exp-table entry
  int64_t w0, w1;
  history_window(a, row, cfg, &w0, &w1);
  const int64_t wn = w1 - w0;
  const int32_t* hp = wn > 0 ? a.history_ids + w0 : dummy;
  const int32_t hid0 = hp[tid < wn ? tid : 0];
  const int32_t hid1 = hp[tid + kScanThreads < wn ? tid + kScanThreads : 0];
  int64_t f0 = 0, f1 = 0;
  if (kMasked && a.forced_offsets) { f0 = a.forced_offsets[row]; f1 = a.forced_offsets[row + 1]; }
  const int64_t fn = f1 - f0;
  const int32_t* fp = fn > 0 ? a.forced_ids + f0 : dummy;
  const int32_t fid0 = fp[tid < fn ? tid : 0];
  const double tabv = c_exp2_256[tid];

  // -- the chunk: all loads in flight before the first use
  const In* rowp = (const In*)a.logits + row * a.row_stride + gbase;
  uint4 raw[kLoads];
  if (kFull) {
#pragma unroll
    for (int v = 0; v < kLoads; ++v) raw[v] = *(const uint4*)(rowp + (v * kScanThreads + tid) * kVec);
  } else {
#pragma unroll
    for (int v = 0; v < kLoads; ++v) {
      const int loc = (v * kScanThreads + tid) * kVec;
      uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
      for (int j = 0; j < kVec; ++j) {
        const int i = loc + j < n_valid ? loc + j : n_valid - 1;  // bits past n_valid are cleared below
        const uint32_t b = VT::one(rowp + i);
        if (kVec == 4) w[j] = b;
        else w[j >> 1] |= (j & 1) ? (b & 0xFFFF0000u) : (b >> 16);
      }
      raw[v] = make_uint4(w[0], w[1], w[2], w[3]);
    }
  }
  uint32_t mword[kLoads];
  if (kMasked) {
    const uint32_t* maskp = a.mask_table + (int64_t)slot * a.mask_words + (gbase >> 5);
#pragma unroll
    for (int v = 0; v < kLoads; ++v) {
      const int loc = (v * kScanThreads + tid) * kVec;
      mword[v] = maskp[(loc < n_valid ? loc : n_valid - 1) >> 5];  // bits past n_valid are cleared below
    }
  }

  // -- special ids of this chunk as an LDS bitmap
  s_special[tid] = 0;  // kChunk / 32 == kScanThreads words
  s_tab[tid] = tabv;
  __syncthreads();
  // ids are below 2^31, so chunk offsets fit in 32 bits
  const int32_t base32 = (int32_t)gbase;
  auto mark = [&](int32_t id) {
    const uint32_t loc = (uint32_t)(id - base32);
    if (loc < (uint32_t)n_valid) atomicOr(&s_special[loc >> 5], 1u << (loc & 31));
  };
  if (tid < wn) mark(hid0);
  if (tid + kScanThreads < wn) mark(hid1);
  for (int64_t j = w0 + 2 * kScanThreads + tid; j < w1; j += kScanThreads) mark(a.history_ids[j]);
  if (tid < fn) mark(fid0);
  for (int64_t j = f0 + kScanThreads + tid; j < f1; j += kScanThreads) mark(a.forced_ids[j]);
  __syncthreads();

  // per-load bitmasks: valid = in range and not special; allowed = mask bit
  auto valid_bits = [&](int v) -> uint32_t {
    const int loc = (v * kScanThreads + tid) * kVec;
    uint32_t in_range = kLaneBits;
    if (!kFull) {
      const int left = n_valid - loc;
      in_range = left >= kVec ? kLaneBits : (left > 0 ? (1u << left) - 1u : 0u);
    }
    return in_range & ~(s_special[loc >> 5] >> (loc & 31)) & kLaneBits;
  };
  auto allowed_bits = [&](int v) -> uint32_t {
    const int loc = (v * kScanThreads + tid) * kVec;
    if (kMasked) return (mword[v] >> (loc & 31)) & kLaneBits;
    return kLaneBits;
  };
  const bool use_cap = cfg.softcap > 0;

  // values: excluded (special / out of range) and masked ids become -inf,
  // which neither the normaliser nor the candidate list admits. Most load
  // groups hold no such id: the per-element masking runs only for groups
  // where some lane of the wave has one.
  float x[kElemsPerThread];
#pragma unroll
  for (int v = 0; v < kLoads; ++v) {
    const uint32_t live = valid_bits(v) & allowed_bits(v);
#pragma unroll
    for (int j = 0; j < kVec; ++j) {
      float y = __builtin_bit_cast(float, VT::bits(raw[v], j));
      if (use_cap) y = capped(y, cfg.softcap);
      x[v * kVec + j] = y;
    }
    if (__ballot(live != kLaneBits)) {
#pragma unroll
      for (int j = 0; j < kVec; ++j) {
        if (!((live >> j) & 1u)) x[v * kVec + j] = -__builtin_inff();
      }
    }
  }

  // pass 1: the thread's maximum (NaN-propagating: NaN or +inf flags the row)
  float tmax = -__builtin_inff();
#pragma unroll
  for (int e = 0; e < kElemsPerThread; ++e) tmax = __builtin_elementwise_maximum(tmax, x[e]);
  const bool finite_max = tmax > -__builtin_inff() && tmax < __builtin_inff();
  // the normaliser below reads -inf as -FLT_MAX, which adds exactly 0 unless
  // the thread's maximum is -FLT_MAX itself: such rows take the exact path
  const bool thread_bad = !(tmax < __builtin_inff()) || tmax == -__FLT_MAX__;

  // ------------------------------------------------------------ greedy rows
  if (greedy) {
    // argmax keeps the first maximum (sampling.ts:92-96): the largest value,
    // then the lowest id holding it. Masked ids take part as -inf; a special
    // id's -inf here never outranks its exact value in the finish's merge.
    uint32_t gid = 0xFFFFFFFFu;
#pragma unroll
    for (int v = kLoads - 1; v >= 0; --v) {
#pragma unroll
      for (int j = kVec - 1; j >= 0; --j) {
        if (x[v * kVec + j] == tmax) gid = (uint32_t)(gbase + (v * kScanThreads + tid) * kVec + j);
      }
    }
    uint64_t best = gid != 0xFFFFFFFFu ? pack_entry(f32_key(tmax), gid) : 0ull;
    for (int m = 32; m > 0; m >>= 1) {
      const uint64_t o = shfl_xor_u64(best, m);
      best = o > best ? o : best;
    }
    const uint64_t wb = __ballot(thread_bad);
    if (lane == 0) { s_wbest[wave] = best; s_wbad[wave] = wb != 0; }
    __syncthreads();
    if (tid == 0) {
      uint64_t bst = 0;
      uint32_t anybad = 0;
      for (int w = 0; w < kScanWaves; ++w) { bst = s_wbest[w] > bst ? s_wbest[w] : bst; anybad |= s_wbad[w]; }
      if (bst) list[0] = list_slot(__builtin_bit_cast(uint32_t, key_f32(entry_key(bst))), entry_id(bst));
      ChunkStat st;
      st.sum = 0.0;
      st.max_key = entry_key(bst);
      st.n_list = bst ? 1u : 0u;
      st.n_finite = 0;
      st.threshold = entry_key(bst);
      st.truncated = 0;
      st.flags = anybad ? kChunkNonFinite : 0u;
      for (int w = 0; w < kScanWaves; ++w) st.n_sub[w] = 0;
      st.n_sub[0] = (uint16_t)st.n_list;
      *stat = st;
    }
    return;
  }

  // pass 2: sum of e^((l - tmax)/T) against the thread's own maximum, with
  // y = 256 log2(e) (l - tmax) / T formed by one fma; its rounding (of
  // tmax * A) is of the order of the reference's own rounding of l/T - M,
  // which the finish kernel's top-p margin already covers.
  const double A = (1.0 / cfg.temperature) * GS_256_LOG2E;
  double sum = 0.0;
  if (finite_max) {
    const double B = -(double)tmax * A;
    // logits below lim have (l - tmax)/T < -60 (lim is rounded down)
    const double lim64 = (double)tmax - 60.0 * cfg.temperature;
    // 1e-6 relative below lim64 before rounding to binary32 (half an ulp)
    const float lim = (float)(lim64 - (lim64 < 0 ? -lim64 : lim64) * 1.0e-6 - 1.0e-37);
    // groups of four terms, so the table reads of a group overlap; a group is
    // skipped when no lane of the wave has a term above e^-60. -inf enters as
    // -FLT_MAX (one med3; +inf rows are already flagged): its exponent is
    // finite and so negative that the term is 0.
#pragma unroll
    for (int g = 0; g < kElemsPerThread; g += 4) {
      const float gmax = __builtin_elementwise_maximum(__builtin_elementwise_maximum(x[g], x[g + 1]),
                                                       __builtin_elementwise_maximum(x[g + 2], x[g + 3]));
      if (__ballot(gmax >= lim)) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float xe = __builtin_amdgcn_fmed3f(x[g + q], -__FLT_MAX__, __FLT_MAX__);
          sum += exp2_256(__builtin_fma((double)xe, A, B), s_tab);
        }
      }
    }
  }

  // chunk maximum, flags and counts
  const uint32_t mykey = finite_max ? f32_key(tmax) : 0u;
  s_keys[tid] = mykey;
  {
    const uint32_t wm = wave_max_u32(mykey);
    const uint64_t wb = __ballot(thread_bad);
    const uint64_t wl = __ballot(mykey != 0u);
    if (lane == 0) {
      s_wmax[wave] = wm;
      s_wbad[wave] = wb != 0;
      s_wlanes[wave] = (uint32_t)__popcll(wl);
    }
  }
  __syncthreads();
  uint32_t cmax = 0, cbad = 0, lanes = 0;
#pragma unroll
  for (int w = 0; w < kScanWaves; ++w) {
    cmax = s_wmax[w] > cmax ? s_wmax[w] : cmax;
    cbad |= s_wbad[w];
    lanes += s_wlanes[w];
  }
  if (cbad) {
    // NaN or +inf among the live logits: outside the one-pass contract
    if (tid == 0) {
      ChunkStat st{};
      st.max_key = cmax;
      st.flags = kChunkNonFinite;
      *stat = st;
    }
    return;
  }

  // rescale the thread sums to the chunk maximum
  {
    double part = 0.0;
    if (finite_max && sum > 0.0) {
      const double y = ((double)tmax - (double)key_f32(cmax)) * A;
      part = y > kSkipY ? sum * exp2_256(y, s_tab) : 0.0;  // the chunk maximum's own factor is exactly 1
    }
    part = wave_sum_f64(part);
    if (lane == 0) s_wsum[wave] = part;
  }

  // tau: at least `depth` per-thread maxima are >= tau
  const uint32_t depth = (uint32_t)plan.depth;
  uint32_t tau = 0;
  const bool selected = lanes > depth + 32u;
  if (selected) tau = radix_floor(s_keys, s_hist, s_sel, depth, 32u);
  const uint32_t thr = tau > kKeyNegInf ? tau : kKeyNegInf + 1u;
  const float tf = key_f32(thr);

  // gather every finite logit >= tau into this wave's sub-list
  uint64_t* sub = list + wave * kSubCap;
  uint32_t off = 0;
#pragma unroll
  for (int v = 0; v < kLoads; ++v) {
#pragma unroll
    for (int j = 0; j < kVec; ++j) {
      const float y = x[v * kVec + j];
      const bool take = y >= tf;
      const uint64_t m = __ballot(take);
      if (m) {
        if (take) {
          const uint32_t pos =
              off + __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
          const uint32_t id = (uint32_t)(gbase + (v * kScanThreads + tid) * kVec + j);
          if (pos < (uint32_t)kSubCap) sub[pos] = list_slot(__builtin_bit_cast(uint32_t, y), id);
        }
        off += (uint32_t)__popcll(m);
      }
    }
  }
  if (lane == 0) s_wgather[wave] = off;
  __syncthreads();
  if (tid == 0) {
    ChunkStat st;
    double csum = 0.0;
    uint32_t listed = 0, overflow = 0;
    for (int w = 0; w < kScanWaves; ++w) {
      csum += s_wsum[w];
      const uint32_t g = s_wgather[w];
      const uint32_t n = g < (uint32_t)kSubCap ? g : (uint32_t)kSubCap;
      listed += n;
      overflow |= g > (uint32_t)kSubCap;
      st.n_sub[w] = (uint16_t)n;
    }
    st.sum = csum;
    st.max_key = cmax;
    st.n_list = listed;
    st.n_finite = 0;
    st.threshold = thr;
    // with a tau, lanes whose maximum lies below it left finite logits out
    st.truncated = selected ? 1u : 0u;
    st.flags = overflow ? kChunkOverflow : 0u;
    *stat = st;
  }
}


template <typename In>
__global__ __launch_bounds__(kScanThreads, 5) void scan_kernel(SampleArgs a) {
  __shared__ ScanShared S;
  const int64_t row = blockIdx.y;
  const int chunk = blockIdx.x;
  if (row == 0 && chunk == 0 && threadIdx.x == 0) {
    // reset the queue the finish kernel fills for the exact kernel; both run
    // after this kernel on the same stream
    a.queue->count = 0;
    a.queue->next = 0;
  }
  const gs_row_config cfg = a.configs[row];
  const Plan plan = plan_row(cfg);
  if (plan.route == kRouteExact) return;
  const int64_t gbase = (int64_t)chunk * kChunk;
  const int n_valid = (int)((int64_t)a.vocab - gbase < kChunk ? (int64_t)a.vocab - gbase : kChunk);
  const bool masked = cfg.mask_slot >= 0 && cfg.mask_slot < a.mask_slots;
  const bool full = n_valid == kChunk && a.vector_ok;
  if (full) {
    if (masked) scan_chunk<In, true, true>(a, cfg, plan, row, chunk, n_valid, S);
    else scan_chunk<In, true, false>(a, cfg, plan, row, chunk, n_valid, S);
  } else {
    if (masked) scan_chunk<In, false, true>(a, cfg, plan, row, chunk, n_valid, S);
    else scan_chunk<In, false, false>(a, cfg, plan, row, chunk, n_valid, S);
  }
}

}  // namespace

void launch_scan(const SampleArgs& a, hipStream_t s) {
  dim3 grid(a.n_chunks, a.rows);
  if (a.dtype == GS_BF16) hipLaunchKernelGGL(scan_kernel<uint16_t>, grid, dim3(kScanThreads), 0, s, a);
  else hipLaunchKernelGGL(scan_kernel<float>, grid, dim3(kScanThreads), 0, s, a);
}

}  // namespace gs
