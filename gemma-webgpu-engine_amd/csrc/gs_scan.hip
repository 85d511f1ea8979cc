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
//   * a candidate list: every finite logit >= tau, where tau is the smallest
//     of the four waves' d-th largest per-thread maxima (d = ceil(depth/4) + 2,
//     found with ballots inside each wave), so at least `depth` per-thread
//     maxima are >= tau. The list therefore holds the chunk's top-`depth` in
//     the reference's (value desc, id asc) order (sampling.ts:33-35) and every
//     finite logit of the chunk >= tau. Each wave appends to a sub-list of
//     its own at positions taken from ballots, so no atomics are involved.
// The chunk's loads are issued first, from kernel arguments alone; the row's
// options, window ids and mask words follow while they are in flight. After
// the special-id bitmap the workgroup meets at one barrier (chunk maximum,
// sums and tau); the statistics are written by thread 0 and each wave's
// lane 0 (its sub-list length), so no barrier follows the gather.
// Logits of "special" ids (the row's penalty window and forced ids) are left
// out here; the finish kernel evaluates them exactly. Masked ids (constraint
// bitmask) are -inf, as maskConstraintLogits makes them
// (src/runtime/constraints.ts:159-173).
//
// The normaliser's exponential is 2^(y/256) = 2^(j/256) * 2^k * e^r with a
// correctly rounded 256-entry table and a quadratic in r, |r| <= ln2/512:
// relative error below 4.2e-10 per evaluation; a term, its lane's rescale to
// the wave maximum and the wave's rescale to the chunk maximum make at most
// 1.3e-9. Only the normaliser sees it, and only
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

// The d-th largest of the wave's lane keys (d >= 1): the largest t with at
// least d keys >= t, found bit by bit from the top with ballots.
__device__ __forceinline__ uint32_t wave_kth_key(uint32_t key, uint32_t d) {
  uint32_t t = 0;
  for (int b = 31; b >= 0; --b) {
    const uint32_t c = t | (1u << b);
    if ((uint32_t)__popcll(__ballot(key >= c)) >= d) t = c;
  }
  return t;
}

struct ScanShared {
  uint32_t special[kChunk / 32];
  double tab[256];
  double wsum[kScanWaves];     // wave sum of e^((l - wave max)/T)
  uint32_t wmax[kScanWaves];   // wave maximum key
  uint32_t wbad[kScanWaves];
  uint32_t wlanes[kScanWaves]; // lanes with a finite maximum
  uint32_t wtau[kScanWaves];   // the wave's d-th largest lane maximum (0: fewer than d lanes)
  uint64_t wbest[kScanWaves];
};

// Loads of one chunk's logits (kFull: 16-byte vector loads).
template <typename In, bool kFull>
__device__ __forceinline__ void load_chunk(const SampleArgs& a, int64_t row, int64_t gbase, int n_valid,
                                           uint4 (&raw)[kElemsPerThread / VecTraits<In>::kVec]) {
  using VT = VecTraits<In>;
  constexpr int kVec = VT::kVec;
  constexpr int kLoads = kElemsPerThread / kVec;
  const int tid = threadIdx.x;
  const In* rowp = (const In*)a.logits + row * a.row_stride + gbase;
  if (kFull) {
#pragma unroll
    for (int v = 0; v < kLoads; ++v) raw[v] = *(const uint4*)(rowp + (v * kScanThreads + tid) * kVec);
  } else {
    // element loads at 32-bit byte offsets from the uniform row base
    const char* base = (const char*)rowp;
#pragma unroll
    for (int v = 0; v < kLoads; ++v) {
      const int loc = (v * kScanThreads + tid) * kVec;
      uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
      for (int j = 0; j < kVec; ++j) {
        const int i = loc + j < n_valid ? loc + j : n_valid - 1;  // bits past n_valid are cleared later
        const uint32_t b = VT::one((const In*)(base + (uint32_t)i * (uint32_t)sizeof(In)));
        if (kVec == 4) w[j] = b;
        else w[j >> 1] |= (j & 1) ? (b & 0xFFFF0000u) : (b >> 16);
      }
      raw[v] = make_uint4(w[0], w[1], w[2], w[3]);
    }
  }
}

// One chunk. kFull: all kChunk logits exist and rows are 16-byte aligned;
// kMasked: the row has a constraint mask. Each combination is straight-line
// code from the first load to the first barrier, so the only wait before the
// barrier is for the loads issued ahead of the chunk.
// The row's penalty window [w0, w1) and forced ids [f0, f1) as offsets into
// the history and forced id arrays.
struct RowRanges {
  int64_t w0, w1, f0, f1;
};

template <typename In, bool kFull, bool kMasked>
__device__ __forceinline__ void scan_chunk(const SampleArgs& a, const gs_row_config& cfg, const Plan plan,
                                           const RowRanges rr, const int64_t row, const int chunk,
                                           const int n_valid, ScanShared& S) {
  using VT = VecTraits<In>;
  constexpr int kVec = VT::kVec;
  constexpr int kLoads = kElemsPerThread / kVec;
  constexpr uint32_t kLaneBits = (1u << kVec) - 1u;
  uint32_t* s_special = S.special;
  double* s_tab = S.tab;
  double* s_wsum = S.wsum;
  uint32_t* s_wmax = S.wmax;
  uint32_t* s_wbad = S.wbad;
  uint32_t* s_wlanes = S.wlanes;
  uint32_t* s_wtau = S.wtau;
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

  // -- the window and forced ids and this thread's exp-table entry
  const int64_t w0 = rr.w0, w1 = rr.w1;
  const int64_t wn = w1 - w0;
  const int32_t* hp = wn > 0 ? a.history_ids + w0 : dummy;
  const int32_t hid0 = hp[tid < wn ? tid : 0];
  const int32_t hid1 = hp[tid + kScanThreads < wn ? tid + kScanThreads : 0];
  const int64_t f0 = kMasked ? rr.f0 : 0, f1 = kMasked ? rr.f1 : 0;
  const int64_t fn = f1 - f0;
  const int32_t* fp = fn > 0 ? a.forced_ids + f0 : dummy;
  const int32_t fid0 = fp[tid < fn ? tid : 0];
  const double tabv = c_exp2_256[tid];

  // -- the chunk: all loads in flight before the first use
  uint4 raw[kLoads];
  load_chunk<In, kFull>(a, row, gbase, n_valid, raw);
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

  // wave statistics: maximum, flags, finite lanes, the sum rescaled to the
  // wave maximum and the wave's d-th largest lane maximum
  const uint32_t mykey = finite_max ? f32_key(tmax) : 0u;
  const uint32_t depth = (uint32_t)plan.depth;
  const uint32_t dw = (depth + 3u) / 4u + 2u;
  {
    const uint32_t wm = wave_max_u32(mykey);
    const uint64_t wb = __ballot(thread_bad);
    const uint32_t wl = (uint32_t)__popcll(__ballot(mykey != 0u));
    double part = 0.0;
    if (finite_max && sum > 0.0) {
      const double y = ((double)tmax - (double)key_f32(wm)) * A;
      part = y > kSkipY ? sum * exp2_256(y, s_tab) : 0.0;  // the wave maximum's own factor is exactly 1
    }
    part = wave_sum_f64(part);
    const uint32_t wt = wl >= dw ? wave_kth_key(mykey, dw) : 0u;
    if (lane == 0) {
      s_wmax[wave] = wm;
      s_wbad[wave] = wb != 0;
      s_wlanes[wave] = wl;
      s_wsum[wave] = part;
      s_wtau[wave] = wt;
    }
  }
  __syncthreads();
  uint32_t cmax = 0, cbad = 0, lanes = 0, tau = 0xFFFFFFFFu, bound = 0;
#pragma unroll
  for (int w = 0; w < kScanWaves; ++w) {
    cmax = s_wmax[w] > cmax ? s_wmax[w] : cmax;
    cbad |= s_wbad[w];
    lanes += s_wlanes[w];
    if (s_wtau[w]) { tau = s_wtau[w] < tau ? s_wtau[w] : tau; bound += dw; }
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

  // tau: at least `depth` per-thread maxima are >= it (dw of each wave that
  // has dw finite lanes); nearly full chunks are listed whole
  const bool selected = lanes > depth + 32u && bound >= depth;
  const uint32_t thr = selected && tau > kKeyNegInf ? tau : kKeyNegInf + 1u;
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
  // the sub-list length; a count above kSubCap tells the finish it overflowed
  if (lane == 0) stat->n_sub[wave] = (uint16_t)(off < 0xFFFFu ? off : 0xFFFFu);
  if (tid == 0) {
    // the chunk sum: each wave's sum rescaled from its maximum to the chunk's
    double csum = 0.0;
#pragma unroll
    for (int w = 0; w < kScanWaves; ++w) {
      const double ws = s_wsum[w];
      if (ws > 0.0) {
        const double y = ((double)key_f32(s_wmax[w]) - (double)key_f32(cmax)) * A;
        csum += y > kSkipY ? ws * exp2_256(y, s_tab) : 0.0;
      }
    }
    stat->sum = csum;
    stat->max_key = cmax;
    stat->n_list = 0;
    stat->n_finite = 0;
    stat->threshold = thr;
    // with a tau, lanes whose maximum lies below it left finite logits out
    stat->truncated = selected ? 1u : 0u;
    stat->flags = 0u;
  }

}


// kMaskable: the batch has a mask table (otherwise no row is constrained and
// the masked variants, which need more registers, are left out).
template <typename In, bool kMaskable>
__global__ __launch_bounds__(kScanThreads, kMaskable ? 5 : 6) void scan_kernel(SampleArgs a) {
  __shared__ ScanShared S;
  const int64_t row = blockIdx.y;
  const int chunk = blockIdx.x;
  const gs_row_config cfg = a.configs[row];
  const Plan plan = plan_row(cfg);
  // row-uniform offsets read here, ahead of every branch and store, so they
  // come through the scalar cache and nothing waits on them behind the chunk
  RowRanges rr;
  history_window(a, row, cfg, &rr.w0, &rr.w1);
  rr.f0 = rr.f1 = 0;
  if (a.forced_offsets) { rr.f0 = a.forced_offsets[row]; rr.f1 = a.forced_offsets[row + 1]; }
  if (plan.route != kRouteExact) {
    const int64_t gbase = (int64_t)chunk * kChunk;
    const int n_valid = (int)((int64_t)a.vocab - gbase < kChunk ? (int64_t)a.vocab - gbase : kChunk);
    const bool masked = kMaskable && cfg.mask_slot >= 0 && cfg.mask_slot < a.mask_slots;
    const bool full = n_valid == kChunk && a.vector_ok;
    if (full) {
      if (masked) scan_chunk<In, true, kMaskable>(a, cfg, plan, rr, row, chunk, n_valid, S);
      else scan_chunk<In, true, false>(a, cfg, plan, rr, row, chunk, n_valid, S);
    } else {
      if (masked) scan_chunk<In, false, kMaskable>(a, cfg, plan, rr, row, chunk, n_valid, S);
      else scan_chunk<In, false, false>(a, cfg, plan, rr, row, chunk, n_valid, S);
    }
  }
  // reset the queue the finish kernel fills for the exact kernel (both run
  // after this kernel on the same stream). It is the kernel's last store, so
  // the loads above of the row's options and history offsets may use the
  // scalar cache.
  if (row == 0 && chunk == 0 && threadIdx.x == 0) {
    a.queue->count = 0;
    a.queue->next = 0;
  }
}

}  // namespace

void launch_scan(const SampleArgs& a, hipStream_t s) {
  dim3 grid(a.n_chunks, a.rows);
  const bool maskable = a.mask_slots > 0;
  if (a.dtype == GS_BF16) {
    if (maskable) hipLaunchKernelGGL((scan_kernel<uint16_t, true>), grid, dim3(kScanThreads), 0, s, a);
    else hipLaunchKernelGGL((scan_kernel<uint16_t, false>), grid, dim3(kScanThreads), 0, s, a);
  } else {
    if (maskable) hipLaunchKernelGGL((scan_kernel<float, true>), grid, dim3(kScanThreads), 0, s, a);
    else hipLaunchKernelGGL((scan_kernel<float, false>), grid, dim3(kScanThreads), 0, s, a);
  }
}

}  // namespace gs
