// Row finish: the per-row half of the batched sampler (one 1024-thread
// workgroup per row, after the chunk scan).
//
// It rebuilds, for one row, exactly the part of the reference's sorted
// candidate list that the filters can reach (src/runtime/sampling.ts:33-64):
//   1. evaluates the row's distinct special ids exactly: penalty-window ids
//      with their counts (sampling.ts:21-30) and, for constrained rows, the
//      termination / extra ids of selectConstrainedToken
//      (src/runtime/gemma-session.ts:1305-1329);
//   2. keeps the chunk-list entries whose key is at or above the highest
//      truncated chunk's threshold -- the region where the union of the
//      lists is complete -- and merges the chunk maxima and partial sums
//      with the specials into the softmax normaliser;
//   3. ranks the top 64 of that region (per-wave register sorts, then a
//      bitonic tree merge), merges in the specials of the region, and applies
//      top-k, min-p and top-p and the draw in one wave, with the reference's
//      comparisons on binary64 probabilities from the bit-exact js_exp;
//   4. when the filters reach past the top 64 (top-p or min-p cuts deep in
//      the list), sorts the whole region and repeats step 3 block-wide.
// The normaliser is summed in a different order from the reference's
// sequential loop, from the scan's binary32 terms, so every comparison that
// decides the outcome is checked against a margin that bounds the
// difference. A top-p cut within the scan normaliser's bound (3.9e-7
// relative) is settled again after the row's normaliser is recomputed in
// binary64 (4.2e-10 per term); rows that still fail a margin, need
// candidates outside the complete region, or hold non-finite logits are
// queued for the exact kernel, which replays the reference step by step.
//
// Global loads are issued in two batches (row inputs, then the list entries
// and special logits that LDS data locates), so the row's latency is a few
// memory round trips plus the rank work.
#include "gs_exact_row.h"
#include "gs_exp2.h"
#include "gs_internal.h"

namespace gs {
namespace {

// The checked build (-DGS_CHECKED): every index into the LDS candidate,
// region, special, hash, histogram and stage arrays, into a deep record's
// arrays and into the row's chunk lists goes through GS_CK(index, bound). An
// index out of range reads or writes element 0 instead and sets
// g_check_fail; the kernel then sends the row to the exact replay with
// GS_FLAG_INDEX_CHECK in place of any result it wrote, so a bad index shows
// as a flagged row, never as a fault or a silent wrong token. In the normal
// build GS_CK(i, n) is i.
#ifdef GS_CHECKED
__shared__ uint32_t g_check_fail;
template <typename I>
__device__ __forceinline__ I gs_ck(I i, int64_t n) {
  if ((uint64_t)(int64_t)i >= (uint64_t)n) {
    g_check_fail = 1u;
    return (I)0;
  }
  return i;
}
#define GS_CK(i, n) gs_ck((i), (int64_t)(n))
#define GS_CHECK_RESET()                          \
  do {                                            \
    if (threadIdx.x == 0) g_check_fail = 0u;      \
  } while (0)
#define GS_CHECK_FAILED() (g_check_fail != 0u)
#else
#define GS_CK(i, n) (i)
#define GS_CHECK_RESET() \
  do {                   \
  } while (0)
#define GS_CHECK_FAILED() false
#endif
#define GS_LEN(x) ((int64_t)(sizeof(x) / sizeof((x)[0])))

// The checked build also makes LDS races show. Much of this file is serial
// work by thread 0 or wave 0 (set-up words, reductions, the one-wave filters)
// whose results the other waves read after a barrier. A missing barrier there
// lets a wave read the word before wave 0 writes it, which happens only when
// wave 0 falls behind, and the read then sees whatever an earlier workgroup
// left in LDS. Here every workgroup barrier below is followed by a sleep of
// wave 0 (about 4000 cycles), so the other waves win such a race every time,
// and every workgroup of these kernels starts from cleared LDS, so the word
// they read is 0 every time. A missing barrier then changes the row's result
// on every run instead of once in many, and the comparison with the normal
// build shows it. Neither changes what a race-free kernel computes.
#ifdef GS_CHECKED
__device__ __forceinline__ void gs_checked_barrier() {
  __syncthreads();
  if (threadIdx.x < 64) __builtin_amdgcn_s_sleep(64);
}
__device__ __forceinline__ void gs_checked_clear(void* lds, size_t bytes) {
  uint32_t* p = (uint32_t*)lds;
  for (size_t i = threadIdx.x; i < bytes / 4; i += blockDim.x) p[i] = 0u;
  __syncthreads();
}
#define __syncthreads() gs_checked_barrier()
#define GS_CHECKED_CLEAR(u) gs_checked_clear(&(u), sizeof(u))
#else
#define GS_CHECKED_CLEAR(u) \
  do {                      \
  } while (0)
#endif

constexpr int kWaves = kFinishThreads / 64;
constexpr int kTopR = 64;                             // entries the fast path ranks exactly
constexpr int kSubThreads = 8;                        // threads that read one wave sub-list
constexpr int kSubPerThread = kSubCap / kSubThreads;  // slots each of them reads
constexpr int kSlotsPerThread = kHashSize / kFinishThreads;
constexpr int kIdsPerThread = 2;                      // window ids loaded ahead per thread
constexpr int kSpecQ = 4;  // list slots per thread read with the statistics (32 per sub-list)
constexpr uint32_t kDeepLists = 1u << 30;  // row flag: some sub-list holds more than 32 entries
constexpr uint32_t kSpecialOverflow = 1u << 29;  // row flag: an id found no hash slot (exact path)
constexpr uint32_t kExactRequest = 1u << 31;  // finish_row's answer: the row goes to the exact path
constexpr uint32_t kDeepRequest = 1u << 30;   // finish_row's answer: a full-vocabulary draw for deep_draw
constexpr double kDeepSpan = 40.0;             // natural-log span of those bins below the region floor
constexpr int kPrefixMin = 256;  // regions up to this size are sorted whole by the slow path
static_assert(kFinishMaxChunks * kScanWaves <= kFinishThreads, "one thread per chunk wave");

// e^x (x <= 0, binary32) in units of 2^-40, rounded down: the slow path's
// mass histogram
__device__ __forceinline__ unsigned long long mass_units(float x) {
  return (unsigned long long)(__builtin_amdgcn_exp2f(x * 1.44269504088896341f) * 0x1p40f);
}

__device__ __forceinline__ double block_scan_f64(double v, double* s_w, double* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const double incl = wave_scan_f64(v);
  if (lane == 63) s_w[wave] = incl;
  __syncthreads();
  double off = 0.0, tot = 0.0;
  for (int w = 0; w < kWaves; ++w) {
    const double x = s_w[w];
    if (w < wave) off += x;
    tot += x;
  }
  __syncthreads();
  *total = tot;
  return incl + off;
}

// The block-wide sum of one 64-bit integer per thread, in every thread
// (integer addition: the same sum in any order); s_w holds kWaves values.
__device__ __forceinline__ uint64_t block_sum_u64(uint64_t v, uint64_t* s_w) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  v = wave_sum_u64(v);
  __syncthreads();  // earlier readers of s_w are done
  if (lane == 0) s_w[wave] = v;
  __syncthreads();
  uint64_t t = 0ull;
  for (int w = 0; w < kWaves; ++w) t += s_w[w];
  __syncthreads();
  return t;
}
// the same for two values at once; s_w holds 2 kWaves values
__device__ __forceinline__ void block_sum2_u64(uint64_t x, uint64_t y, uint64_t* s_w, uint64_t* tx, uint64_t* ty) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  x = wave_sum_u64(x);
  y = wave_sum_u64(y);
  __syncthreads();  // earlier readers of s_w are done
  if (lane == 0) { s_w[wave] = x; s_w[kWaves + wave] = y; }
  __syncthreads();
  uint64_t a = 0ull, b = 0ull;
  for (int w = 0; w < kWaves; ++w) { a += s_w[w]; b += s_w[kWaves + w]; }
  __syncthreads();
  *tx = a;
  *ty = b;
}
// Sums of terms whose order in LDS depends on atomics (the deep draw's
// region and gathered candidates) go through 64-bit integers in units of
// 2^-50 of a reference scale, so that every run gives the same sum: a term
// up to the scale is at most 2^50 units, 4096 of them stay below 2^62, and
// each rounds by at most 2^-51 of the scale.
constexpr double kUnitScale = 0x1p50;
__device__ __forceinline__ uint64_t to_units(double x, double inv_scale) {
  return (uint64_t)__builtin_rint(x * inv_scale * kUnitScale);
}

// Block-wide sums, in every thread, of one binary64 value per thread in a
// fixed order (per wave, then the waves in order) and of one 64-bit integer
// per thread (the same sum in any order); s_w holds 2 * kWaves words and is
// used once per kernel, so no barrier follows the reads.
__device__ __forceinline__ void block_sum_f64_u64(double x, uint64_t y, double* s_w, double* tx, uint64_t* ty) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  uint64_t* s_u = (uint64_t*)(s_w + kWaves);
  x = wave_sum_f64_dpp(x);
  y = wave_sum_u64(y);
  if (lane == 0) { s_w[wave] = x; s_u[wave] = y; }
  __syncthreads();
  // lane l < kWaves holds wave l's totals; the same reductions then sum them
  *tx = wave_sum_f64_dpp(lane < kWaves ? s_w[lane] : 0.0);
  *ty = wave_sum_u64(lane < kWaves ? s_u[lane] : 0ull);
}

// (value key desc, id asc) on parallel arrays
__device__ __forceinline__ bool ranks_before(uint64_t ka, uint32_t ia, uint64_t kb, uint32_t ib) {
  return ka > kb || (ka == kb && ia < ib);
}

__device__ void block_sort_pairs_desc(uint64_t* key, uint32_t* id, int n) {
  for (int k = 2; k <= n; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < n; i += kFinishThreads) {
        const int p = i ^ j;
        if (p > i) {
          const bool desc = (i & k) == 0;
          const bool swap = desc ? ranks_before(key[p], id[p], key[i], id[i])
                                 : ranks_before(key[i], id[i], key[p], id[p]);
          if (swap) {
            const uint64_t tk = key[i]; key[i] = key[p]; key[p] = tk;
            const uint32_t ti = id[i]; id[i] = id[p]; id[p] = ti;
          }
        }
      }
      __syncthreads();
    }
  }
}

__device__ __forceinline__ uint64_t umax64(uint64_t a, uint64_t b) { return a > b ? a : b; }
__device__ __forceinline__ uint64_t umin64(uint64_t a, uint64_t b) { return a > b ? b : a; }

// One merge round: sorted (descending) runs of length L in src become runs
// of 2L in dst, each thread writing E consecutive outputs p .. p+E-1 of its
// merged run. A binary search finds how many of the first p outputs come from
// the first run (its entries first on ties); those outputs are then the E
// largest of the next E of each run (an exhausted run reads 0, no larger than
// any entry): the element-wise maximum of one and the other reversed is
// bitonic, and half-cleaners sort it.
template <int E>
__device__ __forceinline__ void merge_round(const uint64_t* src, uint64_t* dst, int L) {
  const int p0 = threadIdx.x * E;
  const int base = p0 & ~(2 * L - 1);
  const uint64_t* A = src + base;
  const uint64_t* B = src + base + L;
  const int p = p0 - base;
  int lo = p - L > 0 ? p - L : 0, hi = p < L ? p : L;
  while (lo < hi) {
    const int i = (lo + hi) >> 1;
    if (A[i] >= B[p - i - 1]) lo = i + 1; else hi = i;
  }
  const int i = lo, j = p - lo;
  uint64_t c[E];
#pragma unroll
  for (int q = 0; q < E; ++q) {
    const uint64_t x = i + q < L ? A[i + q] : 0ull;
    const uint64_t y = j + E - 1 - q < L ? B[j + E - 1 - q] : 0ull;
    c[q] = umax64(x, y);
  }
#pragma unroll
  for (int d = E >> 1; d > 0; d >>= 1) {
#pragma unroll
    for (int q = 0; q < E; ++q) {
      if ((q & d) == 0) {
        const uint64_t x = c[q], y = c[q + d];
        c[q] = umax64(x, y);
        c[q + d] = umin64(x, y);
      }
    }
  }
#pragma unroll
  for (int q = 0; q < E; ++q) dst[base + p + q] = c[q];
}

template <int E>
__device__ __forceinline__ void wave_sort_desc_regs(uint64_t (&v)[E]);

// Sorts src[0..n) descending into s[0..len), zero-padded: len is a power of
// two with n <= len and E <= len <= kFinishThreads * E; buf is len entries of
// scratch; src may be s or buf. Each wave sorts its 64 * E entries in
// registers and cross-lane steps, then merge rounds double the sorted runs (a
// bitonic network over the whole block costs about three times as much: its
// cross-wave stages need a barrier each). Threads past len / E only take the
// barriers. Ends with a barrier.
template <int E>
__device__ void sort_region(const uint64_t* src, int n, int len, uint64_t* s, uint64_t* buf) {
  const bool active = (int)threadIdx.x * E < len;
  uint64_t v[E];
#pragma unroll
  for (int q = 0; q < E; ++q) {
    const int i = threadIdx.x * E + q;
    v[q] = i < n ? src[i] : 0ull;
  }
  wave_sort_desc_regs<E>(v);
  __syncthreads();  // src and s may still be read by the caller's threads
  if (active) {
#pragma unroll
    for (int q = 0; q < E; ++q) s[threadIdx.x * E + q] = v[q];
  }
  __syncthreads();
  uint64_t* from = s;
  uint64_t* to = buf;
  for (int L = 64 * E; L < len; L <<= 1) {
    if (active) merge_round<E>(from, to, L);
    __syncthreads();
    uint64_t* t = from;
    from = to;
    to = t;
  }
  if (from != s) {
    if (active) {
#pragma unroll
      for (int q = 0; q < E; ++q) s[threadIdx.x * E + q] = from[threadIdx.x * E + q];
    }
    __syncthreads();
  }
}

// Descending bitonic sort of the 64*E entries one wave holds (lane l holds
// entries l*E .. l*E+E-1); every stage is a register or cross-lane step.
template <int E>
__device__ __forceinline__ void wave_sort_desc_regs(uint64_t (&v)[E]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int k = 2; k <= 64 * E; k <<= 1) {
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
      if (j < E) {
#pragma unroll
        for (int q = 0; q < E; ++q) {
          const int qp = q ^ j;
          if (qp > q) {
            const int i = lane * E + q;
            const uint64_t x = v[q], y = v[qp];
            const bool desc = (i & k) == 0;
            v[q] = desc ? umax64(x, y) : umin64(x, y);
            v[qp] = desc ? umin64(x, y) : umax64(x, y);
          }
        }
      } else {
#pragma unroll
        for (int q = 0; q < E; ++q) {
          const int i = lane * E + q;
          const uint64_t y = xlane_u64(v[q], j / E);
          const bool keep_max = ((i & j) == 0) == ((i & k) == 0);
          v[q] = keep_max ? umax64(v[q], y) : umin64(v[q], y);
        }
      }
    }
  }
}

// The kTopR largest entries of s[0..n) (n <= kWaves * 64 * E), descending,
// into top[0..kTopR) (zero-padded). Each wave sorts its 64*E entries in
// registers; the 16 wave lists then meet in a tree of bitonic merges (the
// element-wise maximum of a descending list and a reversed descending list
// holds the top half as a bitonic sequence, which six half-cleaner steps
// sort). tmp holds kWaves * 64 entries. Ends with a barrier.
template <int E>
__device__ void top_r(const uint64_t* s, int n, uint64_t* tmp, uint64_t* top) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint64_t v[E];
#pragma unroll
  for (int q = 0; q < E; ++q) {
    const int i = wave * 64 * E + lane * E + q;
    v[q] = i < n ? s[i] : 0ull;
  }
  wave_sort_desc_regs<E>(v);
#pragma unroll
  for (int q = 0; q < E; ++q) {
    const int i = lane * E + q;
    if (i < 64) tmp[GS_CK(wave * 64 + i, kFinishCap)] = v[q];
  }
  __syncthreads();
  for (int half = kWaves / 2; half >= 1; half >>= 1) {
    uint64_t x = 0;
    if (wave < half) {
      x = umax64(tmp[GS_CK(wave * 64 + lane, kFinishCap)], tmp[GS_CK((wave + half) * 64 + 63 - lane, kFinishCap)]);
#pragma unroll
      for (int j = 32; j > 0; j >>= 1) {
        const uint64_t y = xlane_u64(x, j);
        x = (lane & j) == 0 ? umax64(x, y) : umin64(x, y);
      }
    }
    __syncthreads();
    if (wave < half) tmp[GS_CK(wave * 64 + lane, kFinishCap)] = x;
    __syncthreads();
  }
  if (tid < kTopR) top[tid] = tmp[GS_CK(tid, kFinishCap)];
  __syncthreads();
}

// hist[bin] += 1 for every lane of the wave with `take`; the whole wave is
// active. When at least 8 such lanes share the first one's bin, they add
// together in one LDS atomic and the others one each: tied keys put most of a
// wave in one bin, and same-address LDS atomics from many lanes serialise
// (a row on a 1/8 logit grid spent 14.6 us in one such histogram). Otherwise
// every lane adds its own.
__device__ __forceinline__ void hist_add(uint32_t* hist, uint32_t bin, bool take) {
  const uint64_t m = __ballot(take);
  if (!m) return;
  const int lane = threadIdx.x & 63;
  const int leader = __ffsll((unsigned long long)m) - 1;
  const uint32_t lb = (uint32_t)__shfl((int)bin, leader, 64);
  const bool same = take && bin == lb;
  const uint64_t sm = __ballot(same);
  if (__popcll(sm) < 8) {
    if (take) atomicAdd(&hist[bin], 1u);
  } else if (lane == leader) {
    atomicAdd(&hist[lb], (uint32_t)__popcll(sm));
  } else if (take && !same) {
    atomicAdd(&hist[bin], 1u);
  }
}

// The kTopR largest entries of s[0..n) into top[0..kTopR), descending and
// zero-padded, found without sorting the region when possible. Keys lie in
// [lo, hi]. A 256-bin histogram of (key - lo) >> shift finds the bin holding
// the kTopR-th largest key: every entry of a higher bin outranks it, so the
// entries of that bin and above (the survivors) hold the top kTopR. A crowded
// boundary bin gets a second histogram inside it. The survivors (at most
// 128) are compacted and each finds its place by counting the survivors
// above it. Returns false, with top untouched, when more survive (massive
// ties); the caller then ranks the whole region. hist: 256 counters, zero on
// entry and on return; sel: 4 words; out: 128 entries of scratch (16-byte
// aligned, at least 129 entries). Ends with a barrier.
__device__ __forceinline__ int top_select_shift(uint32_t lo, uint32_t hi) {
  const uint32_t span = hi - lo;
  int shift = 0;
  while ((span >> shift) > 255u) ++shift;
  return shift;
}

// The slow path's ranking boundary (the comment at its call says why it is
// one): over the region s[0..n_ns) in LDS (keys in [sel_lo, sel_hi]) and the
// region's specials in_key[0..n_sp_in), the key above which either the first
// topK candidates (counting non-specials only) or a mass of want_mass
// (scaled down by 2^-10; infinite: no such bound) lies; 0 when none is met in
// the region or the boundary keeps all of it. Its non-specials are compacted
// into out[0..sel[3]). *region_mass: the region's mass e^(v - M) summed in
// binary32 terms (within 1e-5 relative), infinite when not summed. hist: 256
// counters, zero on entry and on return; bmass: 256 words of scratch. Called
// by the whole block; ends with a barrier.
__device__ __forceinline__ uint32_t prefix_floor(const uint64_t* region, int n_ns, const uint64_t* in_key, int n_sp_in,
                                              uint32_t sel_lo, uint32_t sel_hi, double T, double M, int top_k,
                                              double want_mass, uint32_t* hist, uint64_t* bmass, uint32_t* sel,
                                              uint64_t* out, double* region_mass) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bool by_rank = top_k > 0 && top_k < n_ns + n_sp_in;
  const bool by_mass = want_mass < __builtin_inf();
  if (!(by_rank || by_mass) || n_ns <= kPrefixMin) {
    if (tid == 0) *region_mass = __builtin_inf();
    // every thread reads *region_mass after the call: without this barrier a
    // wave could read the word before thread 0 writes it (whatever an earlier
    // workgroup left there) and take another branch than thread 0's wave
    __syncthreads();
    return 0;
  }
  const int shift = top_select_shift(sel_lo, sel_hi);
  // masses in units of 2^-40 e^0 (integer LDS atomics: binary32 ones
  // serialise badly)
  if (tid < 256) bmass[tid] = 0ull;
  __syncthreads();
  const double rT = 1.0 / T;
  for (int i = tid; i < n_ns; i += kFinishThreads) {
    const uint32_t key = entry_key(region[i]);
    if (key < sel_lo) continue;  // -inf (below every boundary, no mass)
    const uint32_t d = (key - sel_lo) >> shift;
    const uint32_t bin = d < 255u ? d : 255u;
    const float x = (float)((double)key_f32(key) * rT - M);
    atomicAdd(&hist[bin], 1u);
    atomicAdd((unsigned long long*)&bmass[bin], mass_units(x));
  }
  // the region's specials add mass (not count) to the bin of a key no
  // higher than their value times T (the lowest bin below sel_lo): a
  // boundary at or below that bin keeps them among the ranked candidates
  for (int j = tid; j < n_sp_in; j += kFinishThreads) {
    const double v = key_f64(in_key[GS_CK(j, kHashSize / 2)]);
    const double l = v * T;
    const double l_lo = l - (l < 0 ? -l : l) * 0x1p-40;
    const float lf = (float)l_lo;
    const uint32_t key = f32_key(lf) - ((double)lf > l_lo ? 1u : 0u);
    const uint32_t d = key < sel_lo ? 0u : (key - sel_lo) >> shift;
    const uint32_t bin = d < 255u ? d : 255u;
    atomicAdd((unsigned long long*)&bmass[bin], mass_units((float)(v - M)));
  }
  __syncthreads();
  if (wave == 0) {
    // lane l holds bins 255-4l .. 252-4l, highest first
    uint32_t h[4], c = 0;
    double m[4], ms = 0.0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      h[q] = hist[255 - 4 * lane - q];
      m[q] = (double)bmass[255 - 4 * lane - q] * 0x1p-40;
      c += h[q];
      ms += m[q];
    }
    const uint32_t incl = wave_scan_u32(c);
    const double mincl = wave_scan_f64(ms);
    if (lane == 63) *region_mass = mincl;
    const uint32_t want_n = by_rank ? (uint32_t)top_k : 0xFFFFFFFFu;
    const double want_m = want_mass;
    constexpr double kUnder = 1.0 - 0x1p-10;
    // the boundary bin of each bound (-1: not met in the region)
    int bn = -1, bm = -1;
    const uint64_t hit_n = __ballot(incl >= want_n);
    const uint64_t hit_m = __ballot(mincl * kUnder >= want_m);
    if (hit_n) {
      const int f = __ffsll((unsigned long long)hit_n) - 1;
      if (lane == f) {
        uint32_t cum = incl - c;
        int q = 0;
        while (q < 3 && cum + h[q] < want_n) { cum += h[q]; ++q; }
        bn = 255 - 4 * lane - q;
      }
      bn = __shfl(bn, f, 64);
    }
    if (hit_m) {
      const int f = __ffsll((unsigned long long)hit_m) - 1;
      if (lane == f) {
        double cum = mincl - ms;
        int q = 0;
        while (q < 3 && (cum + m[q]) * kUnder < want_m) { cum += m[q]; ++q; }
        bm = 255 - 4 * lane - q;
      }
      bm = __shfl(bm, f, 64);
    }
    const int b = bn > bm ? bn : bm;  // the higher boundary: fewer candidates
    if (lane == 0) {
      sel[0] = b > 0 ? (uint32_t)b : 0u;
      sel[3] = 0;
    }
  }
  __syncthreads();
  const uint32_t b = sel[0];
  if (tid < 256) hist[tid] = 0;  // zero again for the next use
  if (b == 0u) {
    __syncthreads();
    return 0;
  }
  // compact the non-specials at or above the boundary into out (one LDS
  // atomic per wave)
  const uint32_t floor_key = sel_lo + (b << shift);
  for (int i0 = 0; i0 < n_ns; i0 += kFinishThreads) {
    const int i = i0 + tid;
    const uint64_t e = i < n_ns ? region[i] : 0ull;
    const bool keep = i < n_ns && entry_key(e) >= floor_key;
    const uint64_t mk = __ballot(keep);
    uint32_t base = 0;
    if (lane == 0 && mk) base = atomicAdd(&sel[3], (uint32_t)__popcll(mk));
    base = readlane_u32(base, 0);
    if (keep) out[base + __builtin_amdgcn_mbcnt_hi((uint32_t)(mk >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mk, 0u))] = e;
  }
  __syncthreads();
  return floor_key;
}

// Appends thread-held entries (valid bits) with key >= floor_key to out[] at
// positions counted in sel[3] (one LDS atomic per wave); positions past 128
// are counted, not stored.
template <int kE>
__device__ __forceinline__ void compact_entries(const uint64_t (&e)[kE], uint32_t valid, uint32_t floor_key,
                                                uint32_t* sel, uint64_t* out) {
  const int lane = threadIdx.x & 63;
  constexpr int kOut = 128;
#pragma unroll
  for (int q = 0; q < kE; ++q) {
    const bool keep = ((valid >> q) & 1u) && entry_key(e[q]) >= floor_key;
    const uint64_t m = __ballot(keep);
    uint32_t base = 0;
    if (lane == 0 && m) base = atomicAdd(&sel[3], (uint32_t)__popcll(m));
    base = readlane_u32(base, 0);
    if (keep) {
      const uint32_t pos =
          base + __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
      if (pos < (uint32_t)kOut) out[pos] = e[q];
    }
  }
}

// The kTopR largest of the n_src (<= 128) distinct entries in src, descending
// into top[0..kTopR) and zero-padded. Ends with a barrier.
__device__ __forceinline__ void rank_survivors(const uint64_t* src, int n_src, uint64_t* top) {
  const int tid = threadIdx.x;
  // rank the survivors (at most 128) by counting: the entries are distinct,
  // so survivor i's place is the number of survivors above it. Eight threads
  // share survivor tid / 8, each counting over 16 of the survivors (out holds
  // at least 128 entries), and the eight counts meet by DPP; places past the
  // survivors stay zero.
  {
    const int i = tid >> 3, part = tid & 7;
    uint64_t ei = 0;
    uint32_t cnt = 0;
    if (i < n_src) {
      ei = src[i];
      const uint4* p = (const uint4*)(src + part * 16);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint4 w = p[j];
        const int k = part * 16 + 2 * j;
        const uint64_t x0 = ((uint64_t)w.y << 32) | w.x, x1 = ((uint64_t)w.w << 32) | w.z;
        cnt += (k < n_src && x0 > ei) ? 1u : 0u;
        cnt += (k + 1 < n_src && x1 > ei) ? 1u : 0u;
      }
    }
    cnt += dpp_u32<kDppQuad1032, 0xF>(0u, cnt);
    cnt += dpp_u32<kDppQuad2301, 0xF>(0u, cnt);
    cnt += dpp_u32<kDppRowHalfMirror, 0xF>(0u, cnt);  // lane l of 8 meets lane 7 - l: the other quad
    if (part == 0 && i < n_src && cnt < (uint32_t)kTopR) top[cnt] = ei;
    if (tid >= n_src && tid < kTopR) top[tid] = 0;
  }
  __syncthreads();
}

// The selection over entries the threads hold in registers, given a floor
// with at least kTopR valid entries at or above it (top_floor): those entries
// are compacted straight away and, when at most 128, ranked without a
// histogram; more run the histogram selection among themselves. *n_out
// counts every valid entry, as top_select_regs does with n = -1; sel[3] is
// zero on entry. Ends with a barrier.
template <int kE>
__device__ __forceinline__ bool top_select_regs_floor(const uint64_t (&e)[kE], uint32_t valid, uint32_t top_floor,
                                                      uint32_t hi, uint32_t* hist, uint32_t* sel, uint64_t* out,
                                                      uint64_t* top, uint32_t* n_out);

// The selection over entries the threads hold in registers: thread t's e[q]
// is an entry when bit q of `valid` is set. n (block-uniform) counts them, or
// is -1: then the first histogram pass also counts them into *n_out (zero on
// entry; one LDS atomic per wave). The histogram settles any count, so the
// pass runs whenever the count is unknown or above 128.
template <int kE>
__device__ __forceinline__ bool top_select_regs(const uint64_t (&e)[kE], uint32_t valid, int n, uint32_t lo,
                                                uint32_t hi, uint32_t* hist, uint32_t* sel, uint64_t* out,
                                                uint64_t* top, uint32_t* n_out) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  constexpr int kOut = 128;
  uint32_t floor_key = 0;  // survivors: valid entries with key >= floor_key
  if (n < 0) {
    const uint32_t w = wave_sum_u32((uint32_t)__popc(valid));
    if (lane == 0 && w) atomicAdd(n_out, w);
  }
  if (n > kOut || n < 0) {
    int shift = top_select_shift(lo, hi);
    uint32_t bin_lo = lo;    // start of the range being binned
    int width = 32;          // the range is [bin_lo, bin_lo + 2^width), 32: unbounded
    uint32_t above = 0;      // entries above the range (from the first round)
    floor_key = lo;
    bool ok = false;
    for (int round = 0; round < 2 && !ok; ++round) {
#pragma unroll
      for (int q = 0; q < kE; ++q) {
        if ((valid >> q) & 1u) {
          const uint32_t d = entry_key(e[q]) - bin_lo;  // entries below bin_lo wrap to large values
          const bool in_range = entry_key(e[q]) >= bin_lo && (width >= 32 || (d >> width) == 0u);
          const uint32_t bin = d >> shift;
          if (in_range) atomicAdd(&hist[bin < 255u ? bin : 255u], 1u);
        }
      }
      __syncthreads();
      if (wave == 0) {
        // lane l holds bins 255-4l .. 252-4l, highest first
        uint32_t h[4], c = 0;
#pragma unroll
        for (int q = 0; q < 4; ++q) { h[q] = hist[255 - 4 * lane - q]; c += h[q]; }
        const uint32_t incl = wave_scan_u32(c);
        const uint64_t hit = __ballot(above + incl >= (uint32_t)kTopR);
        const int first = hit ? __ffsll((unsigned long long)hit) - 1 : 63;
        if (lane == first) {
          uint32_t cum = above + incl - c;
          int q = 0;
          while (q < 3 && cum + h[q] < (uint32_t)kTopR) { cum += h[q]; ++q; }
          sel[0] = (uint32_t)(255 - 4 * lane - q);  // boundary bin
          sel[1] = cum;                              // entries above it
          sel[2] = cum + h[q];                       // survivors
        }
      }
      __syncthreads();
      const uint32_t b = sel[0];
      floor_key = bin_lo + (b << shift);
      ok = sel[2] <= (uint32_t)kOut;
      above = sel[1];
      if (tid < 256) hist[tid] = 0;  // zero again for the next round or the next use
      __syncthreads();
      if (!ok) {
        if (shift == 0) break;  // one key value holds too many entries
        bin_lo = floor_key;
        width = shift;
        shift = shift > 8 ? shift - 8 : 0;
      }
    }
    if (!ok) return false;
  }
  // compact the survivors into out[] (one LDS atomic per wave)
  if (tid == 0) sel[3] = 0;
  __syncthreads();
  compact_entries<kE>(e, valid, floor_key, sel, out);
  __syncthreads();
  rank_survivors(out, (int)(sel[3] < (uint32_t)kOut ? sel[3] : (uint32_t)kOut), top);
  return true;
}

template <int kE>
__device__ __forceinline__ bool top_select_regs_floor(const uint64_t (&e)[kE], uint32_t valid, uint32_t top_floor,
                                                      uint32_t hi, uint32_t* hist, uint32_t* sel, uint64_t* out,
                                                      uint64_t* top, uint32_t* n_out) {
  const int lane = threadIdx.x & 63;
  constexpr int kOut = 128;
  const uint32_t w = wave_sum_u32((uint32_t)__popc(valid));
  if (lane == 0 && w) atomicAdd(n_out, w);
  compact_entries<kE>(e, valid, top_floor, sel, out);
  __syncthreads();
  const uint32_t n_top = sel[3];
  if (n_top <= (uint32_t)kOut) {
    rank_survivors(out, (int)n_top, top);
    return true;
  }
  uint32_t vtop = 0;
#pragma unroll
  for (int q = 0; q < kE; ++q) {
    if (((valid >> q) & 1u) && entry_key(e[q]) >= top_floor) vtop |= 1u << q;
  }
  return top_select_regs<kE>(e, vtop, (int)n_top, top_floor, hi, hist, sel, out, top, nullptr);
}

// The selection over the region s[0..n) in LDS (n <= kFinishCap).
__device__ __forceinline__ bool top_select(const uint64_t* s, int n, uint32_t lo, uint32_t hi, uint32_t* hist,
                                           uint32_t* sel, uint64_t* out, uint64_t* top) {
  constexpr int kMaxE = kFinishCap / kFinishThreads;  // entries per thread
  uint64_t e[kMaxE];
  uint32_t valid = 0;
#pragma unroll
  for (int q = 0; q < kMaxE; ++q) {
    const int i = threadIdx.x + q * kFinishThreads;
    e[q] = i < n ? s[i] : 0ull;
    valid |= (i < n ? 1u : 0u) << q;
  }
  return top_select_regs<kMaxE>(e, valid, n, lo, hi, hist, sel, out, top, nullptr);
}

// special_insert that also reports the id's slot and whether this call put
// the id there (its "owner" evaluates it once the counts are complete)
__device__ __forceinline__ bool special_insert_owner(SpecialTable t, uint32_t id, uint32_t kind, int* slot) {
  uint32_t h = hash_id(id) & (kHashSize - 1);
  for (int probe = 0; probe < kMaxProbe; ++probe) {
    const uint32_t prev = atomicCAS(&t.ids[h], 0xFFFFFFFFu, id);
    if (prev == 0xFFFFFFFFu || prev == id) {
      if (kind == 0) atomicAdd(&t.counts[h], 1u);
      else atomicOr(&t.counts[h], kind << 24);
      *slot = (int)h;
      return prev == 0xFFFFFFFFu;
    }
    h = (h + 1) & (kHashSize - 1);
  }
  *slot = -1;
  return false;
}

__device__ __forceinline__ int pow2_at_least(int n) {
  int p = 1;
  while (p < n) p <<= 1;
  return p;
}

struct Shared {
  uint64_t sorted[kFinishCap];        // non-special entries of the complete region
  uint32_t hash_ids[kHashSize];       // after the specials are evaluated: the in-region
  uint32_t hash_counts[kHashSize];    // specials (keys in hash_ids, ids in hash_counts)
  uint64_t sp_key[kSpecialCap];       // specials: f64 key of their value
  uint32_t sp_id[kSpecialCap];
  double cand_p[kFinishCap];          // merged candidates: e^(value - M) (sort scratch before)
  uint32_t cand_id[kFinishCap];
  uint16_t c_nsub[kFinishMaxChunks * kScanWaves];  // sub-list lengths
  uint64_t top[kTopR];                // the fast path's ranked non-specials
  uint32_t hist[256];                 // top_select's histogram (zero between uses)
  double tab[256];                    // the table exponential's table (deep draw)
  double deep_m, deep_u, deep_margin; // a deep draw's inputs, left by finish_row
  uint64_t deep_floor;
  uint32_t deep_thr, deep_n, deep_count, deep_final;
  DeepPlan plan;                      // the deep draw's pass-2 plan
  uint32_t sel[4];
  double wsum[kWaves];
  double wtmp[kWaves];
  double wsum2[2 * kWaves];
  double total;
  double total_sp;                    // the specials' part of total
  uint64_t sp_max;
  uint32_t flags;
  uint32_t max_key;
  uint32_t thr_max;
  uint32_t any_truncated;
  // per wave holding chunk statistics: a key with at least kTopR / (those
  // waves) of its wave maxima at or above it (0: none)
  uint32_t top_floor[kFinishThreads / 64];
  uint32_t n_sorted;
  uint32_t n_special;
  uint32_t n_sp_in;
  uint32_t route_exact;
  uint32_t status_flags;
  uint32_t first_idx;
  uint32_t legal_bits;
  uint32_t special_legal;
  uint32_t fast_done;
  uint32_t exact_flags;
  uint64_t best_entry;
  uint32_t short_sum;  // the slow path's ranked candidates end short of the pool's end
  double pre_mass;     // the slow path's region mass estimate
};

__device__ void enqueue_exact(const SampleArgs& a, int64_t row, uint32_t flags) {
  const uint32_t q = atomicAdd(&a.queue->count, 1u);
  a.queue->rows[q] = (uint32_t)row;
  a.results[row].flags = flags;
}

// The finish's LDS and, for a row it replays in place, the exact path's
union FinishLds {
  Shared fin;
  exact::Lds ex;
};

// Sends the row to the exact path: replayed here by the whole workgroup when
// it has a scratch slot of its own (row < slots), else queued for the exact
// kernel. Every thread of the workgroup calls it.
__device__ __forceinline__ void to_exact(const SampleArgs& a, FinishLds& U, int64_t row, uint32_t flags) {
  if (row < a.exact_slots) {
    __syncthreads();  // every wave is done with the finish's LDS
    // the replay is a call of its own; it reads the arguments where the
    // kernel received them, so the kernel's copy never goes to the stack
    const SampleArgs& ka = *(const SampleArgs*)__builtin_amdgcn_kernarg_segment_ptr();
    exact::process_row(ka, U.ex, exact::scratch_at(a, row), row, flags);
  } else if (threadIdx.x == 0) {
    enqueue_exact(a, row, flags);
  }
}

__device__ void write_result(const SampleArgs& a, int64_t row, int32_t token, uint32_t flags, double p) {
  a.results[row].token = token;
  a.results[row].flags = flags;
  a.results[row].probability = p;
}

// value l / T of a non-special list entry, in binary64 as the reference
// computes it (sampling.ts:34)
__device__ __forceinline__ double nonspecial_value(uint64_t e, double T) { return (double)key_f32(entry_key(e)) / T; }

// The filters and the draw over the first n_avail (<= 128) candidates, whose
// exponentials e[] (probability = e / total, sampling.ts:39,42) and ids ids[]
// sit in LDS in list order, evaluated by the calling wave alone. Returns 0
// when the row is settled (result written), 1 when a cut or the draw lies past
// the candidates and the caller must widen them, 2 when a decision that
// depends on the normaliser (a top-p or typical-p cut, the typical set's
// order, a draw over the whole row's mass) lies within `margin` and
// `refinable` is set: the caller recomputes the normaliser and calls again
// with the tighter margin; 3 when the row needs the exact path, with its
// result flags in *exact_flags.
// `complete`: the candidates are the row's whole list. aux: 256 doubles of
// LDS scratch for typical-p. full_mass_rel: the bound on how far the
// reference's sum of all the row's probabilities lies from 1.
__device__ __forceinline__ int filters_and_draw_wave(const SampleArgs& a, int64_t row, const gs_row_config& cfg,
                                                     const double* e, double total, const uint32_t* ids, int n_avail,
                                                     bool complete, double margin, bool refinable, double full_mass_rel,
                                                     double* aux, uint32_t* exact_flags) {
  const int lane = threadIdx.x & 63;
  constexpr int kPerLane = 2;  // list index lane*2 + q
  double pl[kPerLane];
#pragma unroll
  for (int q = 0; q < kPerLane; ++q) {
    const int i = lane * kPerLane + q;
    pl[q] = i < n_avail ? e[i] / total : 0.0;
  }
  int n = n_avail;
  bool n_complete = complete;
  uint32_t exact_why = 0;
  bool near_normaliser = false;  // a decision within `margin` that only the normaliser's error can move
  // ---- top-k (sampling.ts:44): the candidates are the list's first
  // n_avail, so a cut inside them is the list's own
  if (cfg.top_k > 0 && cfg.top_k < n) {
    n = cfg.top_k;
    n_complete = true;
  }
  // ---- min-p (sampling.ts:45-48)
  if (cfg.min_p > 0) {
    const double floor_p = readlane_f64(pl[0], 0) * cfg.min_p;
    int first = 0x7FFFFFFF;
    bool bad = false;
#pragma unroll
    for (int q = kPerLane - 1; q >= 0; --q) {
      const int i = lane * kPerLane + q;
      if (i < n) {
        if (!(pl[q] >= floor_p)) first = i;
        const double d = pl[q] >= floor_p ? pl[q] - floor_p : floor_p - pl[q];
        if (d < kNearTie * floor_p) bad = true;
      }
    }
    // the list is sorted by value, so probabilities must not increase
    const double next = __shfl_down(pl[0], 1, 64);
    if (lane * kPerLane + 1 < n && pl[1] > pl[0]) bad = true;
    if (lane * kPerLane + 2 < n && next > pl[1]) bad = true;
    if (__ballot(bad)) exact_why |= 2u;
    first = (int)wave_min_u32((uint32_t)first);
    if (first != 0x7FFFFFFF) {
      n = first;
      n_complete = true;
    }
    if (n == 0) {
      if (lane == 0) write_result(a, row, -1, GS_FLAG_EMPTY_CANDIDATES, 0.0);
      return 0;
    }
  }
  // pool membership of list positions below n (typical-p drops some)
  bool kept[kPerLane];
#pragma unroll
  for (int q = 0; q < kPerLane; ++q) kept[q] = lane * kPerLane + q < n;
  // ---- typical-p (sampling.ts:49-55) over the whole pool: entropy in list
  // order, a stable ascending order of surprise |-ln p - H|, the leading
  // mass of that order up to typicalP, and the kept items back in list order
  // (sorted by probability desc, stable: the list's own order)
  if (cfg.typical_p < 1) {
    if (!n_complete) return 1;
    // The reference's pool is its list's first min(topK, V) entries
    // (sampling.ts:44). A row with fewer candidates (finite values: the rest
    // are -inf ids, masked or not) fills the pool with entries of probability
    // 0, whose p ln p turns the entropy NaN (sampling.ts:50), unless min-p
    // dropped them; the exact replay follows that arithmetic.
    if (complete && !(cfg.min_p > 0) && cfg.top_k > n_avail && a.vocab > n_avail) {
      *exact_flags = 0u;
      return 3;
    }
    double t = 0.0;
#pragma unroll
    for (int q = 0; q < kPerLane; ++q) t += kept[q] ? pl[q] * gsm::js_log(pl[q]) : 0.0;
    const double H = -wave_sum_f64_dpp(t);
    if (!(H == H)) {  // a probability of 0: the reference's arithmetic turns NaN
      *exact_flags = 0u;
      return 3;
    }
    // signed surprises a = -ln p - H (the surprise is |a|), kept in aux
    double sa[kPerLane], sp[kPerLane];
#pragma unroll
    for (int q = 0; q < kPerLane; ++q) {
      const int i = lane * kPerLane + q;
      sa[q] = kept[q] ? -gsm::js_log(pl[q]) - H : __builtin_inf();
      sp[q] = __builtin_fabs(sa[q]);
      if (i < 128) aux[i] = sa[q];
    }
    __builtin_amdgcn_wave_barrier();
    // The reference's signed surprises are ours shifted by one amount common
    // to every item: with its normaliser Z and ours Z (1 + e), every ln p
    // moves by -ln(1 + e) and H by about e (S - H), S the pool's mass, so
    // every a moves by about e (H + 1 - S): |shift| <= margin (H + 2). Each
    // item also carries its own rounding, rt. Two items on the same side of the entropy (a of one sign), both
    // clear of the shift, keep their order whatever the shift: only rounding
    // can swap them. Items on opposite sides, or near the entropy, can swap
    // when their surprises lie within twice the shift. Only equal signed
    // surprises are a tie in the reference too (equal probabilities: the same
    // exponential over one normaliser), kept in list order; equal surprises of
    // opposite sign move apart under any shift, so they count as ambiguous
    // like any other pair within twice the shift. rt needs to cover only items
    // of probability >= margin (|a| <= 20 + H, a few 1e-15 of rounding each):
    // a swap moves the kept set only across the cut, and a cut on an item of
    // smaller probability leaves the cumulative mass within margin of
    // typicalP, which the cut's own check below sends on.
    const double rt = 1e-13 * (H + 1.0);
    const double shift = margin * (H + 2.0) + rt;
    const double ms = 2.0 * margin * (H + 2.0) + rt;
    int rank[kPerLane];
    bool amb = false;
#pragma unroll
    for (int q = 0; q < kPerLane; ++q) {
      const int i = lane * kPerLane + q;
      int r = 0;
      for (int j = 0; j < n; ++j) {
        const double aj = aux[j];
        const double sj = __builtin_fabs(aj);
        r += (sj < sp[q] || (sj == sp[q] && j < i)) ? 1 : 0;
        const double d = sj >= sp[q] ? sj - sp[q] : sp[q] - sj;
        const bool same_side = (aj < 0.0) == (sa[q] < 0.0) && sj > shift && sp[q] > shift;
        if (kept[q] && j != i && aj != sa[q] && d <= (same_side ? 2.0 * rt : ms)) amb = true;
      }
      rank[q] = r;
    }
    __builtin_amdgcn_wave_barrier();
    // probabilities in surprise order; their leading mass up to typicalP
#pragma unroll
    for (int q = 0; q < kPerLane; ++q) {
      if (kept[q]) aux[128 + rank[q]] = pl[q];
    }
    __builtin_amdgcn_wave_barrier();
    double ps[kPerLane], cs[kPerLane];
    {
      double run = 0.0;
#pragma unroll
      for (int q = 0; q < kPerLane; ++q) {
        const int r = lane * kPerLane + q;
        ps[q] = r < n ? aux[128 + r] : 0.0;
        run += ps[q];
        cs[q] = run;
      }
      const double incl = wave_scan_f64(run);
#pragma unroll
      for (int q = 0; q < kPerLane; ++q) cs[q] += incl - run;
    }
    int cut = 0x7FFFFFFF;
    bool near = false;
#pragma unroll
    for (int q = kPerLane - 1; q >= 0; --q) {
      const int r = lane * kPerLane + q;
      if (r < n) {
        if (cs[q] >= cfg.typical_p) cut = r;
        const double d = cs[q] >= cfg.typical_p ? cs[q] - cfg.typical_p : cfg.typical_p - cs[q];
        if (d < margin) near = true;
      }
    }
    cut = (int)wave_min_u32((uint32_t)cut);
    if (cut == 0x7FFFFFFF) cut = n - 1;  // keepLeadingMass keeps the whole list
    if (__ballot(amb || near)) near_normaliser = true;
#pragma unroll
    for (int q = 0; q < kPerLane; ++q) kept[q] = kept[q] && rank[q] <= cut;
  }
  if (near_normaliser) {
    if (refinable && !exact_why) return 2;
    exact_why |= 4u;
  }
  // inclusive prefix sums of the pool's probabilities in list order
  double pre[kPerLane];
  {
    double s = 0.0;
#pragma unroll
    for (int q = 0; q < kPerLane; ++q) {
      s += kept[q] ? pl[q] : 0.0;
      pre[q] = s;
    }
    const double incl = wave_scan_f64(s);
#pragma unroll
    for (int q = 0; q < kPerLane; ++q) pre[q] += incl - s;
  }
  uint32_t tie = 0;
  bool full_mass = false;  // the pool is the whole row and reaches past the candidates
  // ---- top-p (sampling.ts:56,82-90)
  if (cfg.top_p < 1) {
    int cut = 0x7FFFFFFF;
    bool near = false;
#pragma unroll
    for (int q = kPerLane - 1; q >= 0; --q) {
      const int i = lane * kPerLane + q;
      if (kept[q]) {
        if (pre[q] >= cfg.top_p) cut = i;
        const double d = pre[q] >= cfg.top_p ? pre[q] - cfg.top_p : cfg.top_p - pre[q];
        if (d < margin) near = true;
      }
    }
    cut = (int)wave_min_u32((uint32_t)cut);
    if (__ballot(near)) {
      // only the normaliser's own error can have put the cut there: settle it
      // with the recomputed normaliser unless another check already failed
      if (refinable && !exact_why) return 2;
      exact_why |= 4u;
    }
    if (cut == 0x7FFFFFFF) {
      if (!n_complete) return 1;
      // the whole pool: its last member
      int last = -1;
#pragma unroll
      for (int q = 0; q < kPerLane; ++q) last = kept[q] ? lane * kPerLane + q : last;
      cut = (int)wave_max_u32((uint32_t)(last + 1)) - 1;
    } else {
      // 1e-6 boundary ties, as the reference comparison plan reports them
      const int cl = cut / kPerLane, cq = cut % kPerLane;
      const double cum = readlane_f64(cq == 0 ? pre[0] : pre[1], cl);
      const double pc = readlane_f64(cq == 0 ? pl[0] : pl[1], cl);
      const double prev = cum - pc;
      if (cum - cfg.top_p <= kTieReport * cfg.top_p || (cut > 0 && cfg.top_p - prev <= kTieReport * cfg.top_p)) {
        tie = GS_FLAG_TOPP_TIE;
      }
    }
    n = cut + 1;  // prefix sums below the cut are unchanged
  } else if (!n_complete) {
    // no cut inside the candidates: with no top-k bound and no min-p floor
    // the pool is the whole row (a full-vocabulary draw), whose candidate
    // total is the row's whole probability mass; otherwise its end lies past
    // the candidates
    if (!(cfg.top_k <= 0 && !(cfg.min_p > 0))) return 1;
    full_mass = true;
  }
  // ---- draw (sampling.ts:58-64): first pool member i with prefix_i >= u *
  // sum of the pool's probabilities
  int last = -1;
#pragma unroll
  for (int q = 0; q < kPerLane; ++q) {
    if (kept[q] && lane * kPerLane + q < n) last = lane * kPerLane + q;
  }
  last = (int)wave_max_u32((uint32_t)(last + 1)) - 1;
  double ctotal, dmargin;
  if (full_mass) {
    // the reference's sum of all V probabilities lies within full_mass_rel of
    // 1; the candidates' prefix sums carry the normaliser's error (margin)
    ctotal = 1.0;
    dmargin = margin + full_mass_rel + kNearTie;
  } else {
    ctotal = readlane_f64((last % kPerLane) == 0 ? pre[0] : pre[1], last / kPerLane);
    dmargin = kNearTie * ctotal;
  }
  const double u = cfg.rng_mode == GS_RNG_EXPLICIT ? cfg.uniform : gsm::mulberry32_draw(cfg.seed, cfg.draw_index);
  const double cursor = u * ctotal;
  int pick = 0x7FFFFFFF;
  bool near = false;
#pragma unroll
  for (int q = kPerLane - 1; q >= 0; --q) {
    const int i = lane * kPerLane + q;
    if (kept[q] && i < n) {
      if (pre[q] >= cursor) pick = i;
      const double d = pre[q] >= cursor ? pre[q] - cursor : cursor - pre[q];
      if (d < dmargin) near = true;
    }
  }
  pick = (int)wave_min_u32((uint32_t)pick);
  if (__ballot(near)) {
    // a full-vocabulary draw within the normaliser's margin: the block-wide
    // path hands it to the deep draw, which recomputes the normaliser
    if (full_mass && !exact_why) return 1;
    exact_why |= 8u;
  }
  if (exact_why) {
    *exact_flags = GS_FLAG_NEAR_TIE;
    return 3;
  }
  if (pick == 0x7FFFFFFF) {
    if (full_mass) return 1;  // the draw lies past the candidates
    *exact_flags = 0u;
    return 3;
  }
  if (lane == 0) write_result(a, row, (int32_t)ids[pick], tie, e[pick] / total);
  return 0;
}

// Calls visit(l, id) for every logit l of the row (soft-capped when cap > 0),
// the whole block over it: kB 16-byte loads per thread go out before any is
// used. Capped rows take a plain loop with the cap's call, so that the
// unrolled loop stays small.
// kRanged: only 16-byte pieces where some lane holds a logit in [lo, hi] are
// visited (one ballot per piece), for a visit that ignores every other logit.
template <int kB, bool kRanged = false, typename F>
__device__ __forceinline__ void visit_row(const SampleArgs& a, int64_t row, double cap, F&& visit, float lo = 0.0f,
                                          float hi = 0.0f) {
  const int tid = threadIdx.x;
  const int64_t V = a.vocab;
  int64_t from = 0;
  if (cap > 0) {
    from = V;
#pragma unroll 1
    for (int64_t i = tid; i < V; i += kFinishThreads) visit(softcap_call(load_logit(a, row, i), cap), (uint32_t)i);
  } else if (a.vector_ok) {
    const bool bf16 = a.dtype == GS_BF16;
    const int per = bf16 ? 8 : 4;
    const int64_t n_vec = V / per;
    const uint4* base = (const uint4*)((const char*)a.logits + row * a.row_stride * (bf16 ? 2 : 4));
    for (int64_t v0 = tid; v0 < n_vec; v0 += (int64_t)kB * kFinishThreads) {
      uint4 w[kB];
#pragma unroll
      for (int k = 0; k < kB; ++k) {
        const int64_t vi = v0 + (int64_t)k * kFinishThreads;
        w[k] = vi < n_vec ? load_nt16(base + vi) : make_uint4(0u, 0u, 0u, 0u);
      }
#pragma unroll
      for (int k = 0; k < kB; ++k) {
        const int64_t vi = v0 + (int64_t)k * kFinishThreads;
        if (vi >= n_vec) break;
        const uint32_t q[4] = {w[k].x, w[k].y, w[k].z, w[k].w};
        const uint32_t id0 = (uint32_t)(vi * per);
        if (kRanged) {
          bool hit = false;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float x0 = __builtin_bit_cast(float, bf16 ? q[j] << 16 : q[j]);
            const float x1 = __builtin_bit_cast(float, q[j] & 0xFFFF0000u);
            hit |= x0 >= lo && x0 <= hi;
            if (bf16) hit |= x1 >= lo && x1 <= hi;
          }
          if (!__ballot(hit)) continue;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (bf16) {
            visit(__builtin_bit_cast(float, q[j] << 16), id0 + 2 * j);
            visit(__builtin_bit_cast(float, q[j] & 0xFFFF0000u), id0 + 2 * j + 1);
          } else {
            visit(__builtin_bit_cast(float, q[j]), id0 + j);
          }
        }
      }
    }
    from = n_vec * per;
  }
  for (int64_t i = from + tid; i < V; i += kFinishThreads) visit(load_logit(a, row, i), (uint32_t)i);
}

// The normaliser's non-special part from scratch in binary64
// (sampling.ts:36-41): the sum over the row's allowed logits l (mask bit set,
// or every id of an unconstrained row) of e^(l/T - M) by the table
// exponential (4.2e-10 relative per term), minus the same terms of the
// allowed special ids, which the normaliser counts with their penalised
// values instead. Identical terms cancel exactly, so the difference keeps the
// sum's accuracy while the specials hold at most half of it; otherwise, or
// when a sum overflows, it returns -1. s_w: 2 kWaves words of LDS scratch;
// tab: the exponential's table in LDS. The whole block calls it.
__device__ double recompute_nonspecial_sum(const SampleArgs& a, int64_t row, const gs_row_config& cfg,
                                           bool constrained, double M, int n_sp, const uint32_t* sp_id,
                                           double* s_w, const double* tab) {
  const int tid = threadIdx.x;
  const double T = cfg.temperature;
  const uint32_t* mrow = constrained ? a.mask_table + (int64_t)cfg.mask_slot * a.mask_words : nullptr;
  // y = (l / T - M) 256 log2(e) in one fma: the quotient's and the products'
  // rounding move y by about 2^-52 |l| 256 log2(e) / T, 1e-14 relative on a
  // term, far inside the table exponential's error
  const double yA = (1.0 / T) * GS_256_LOG2E, yB = -M * GS_256_LOG2E;
  auto term_of_capped = [&](float l) -> double {
    const double y = __builtin_fma((double)l, yA, yB);
    // evaluated for every y (no branch), so that independent terms overlap;
    // exp2_256 reads its table at an index masked to 0..255 for any y
    const double e = exp2_256(y, tab);
    return y > kSkipY ? e : 0.0;
  };
  auto term = [&](float l) -> double {
    if (cfg.softcap > 0) l = softcap_call(l, cfg.softcap);
    return term_of_capped(l);
  };
  double all = 0.0;
  const int64_t V = a.vocab;
  if (mrow) {
    // constrained rows: only legal ids contribute (masked logits are -inf).
    // A thread holds kWords mask words and takes, per pass, the lowest set
    // bit of each: kWords independent loads per memory round trip, as many
    // passes as the wave's fullest word has bits, masked ids never evaluated
    constexpr int kWords = 4;
    const int32_t n_words = a.mask_words;
    for (int32_t w0 = tid; w0 < n_words; w0 += kWords * kFinishThreads) {
      uint32_t m[kWords];
#pragma unroll
      for (int k = 0; k < kWords; ++k) {
        const int32_t w = w0 + k * kFinishThreads;
        m[k] = w < n_words ? mrow[w] : 0u;
      }
      for (;;) {
        uint32_t any = 0;
#pragma unroll
        for (int k = 0; k < kWords; ++k) any |= m[k];
        if (!any) break;
        float l[kWords];
        bool ok[kWords];
#pragma unroll
        for (int k = 0; k < kWords; ++k) {
          const int64_t id = (int64_t)(w0 + k * kFinishThreads) * 32 + (m[k] ? __builtin_ctz(m[k]) : 0);
          ok[k] = m[k] != 0u && id < V;
          l[k] = load_logit(a, row, ok[k] ? id : 0);
          m[k] &= m[k] - 1u;
        }
        double t[kWords];
#pragma unroll
        for (int k = 0; k < kWords; ++k) t[k] = term(l[k]);
#pragma unroll
        for (int k = 0; k < kWords; ++k) all += ok[k] ? t[k] : 0.0;
      }
    }
  }
  // unconstrained rows: every id, four 16-byte loads per thread in flight
  // (visit_row); the sum keeps each thread's order
  if (!mrow) visit_row<4>(a, row, cfg.softcap, [&](float l, uint32_t) { all += term_of_capped(l); });
  // the allowed specials' raw terms (at most kSpecialCap of them, so kSpPer
  // per thread), loaded before the row's sum is reduced
  constexpr int kSpPer = kSpecialCap / kFinishThreads;
  static_assert(kSpecialCap % kFinishThreads == 0, "whole specials per thread");
  double tsp[kSpPer];
#pragma unroll
  for (int k = 0; k < kSpPer; ++k) {
    const int i = tid + k * kFinishThreads;
    tsp[k] = 0.0;
    if (i < n_sp) {
      const uint32_t id = sp_id[i];
      if (!mrow || ((mrow[id >> 5] >> (id & 31)) & 1u)) tsp[k] = term(load_logit(a, row, id));
    }
  }
  double t_all;
  block_scan_f64(all, s_w, &t_all);
  if (!(t_all < __builtin_inf() && t_all > 0.0)) return -1.0;
  // the specials' terms in units of 2^-50 t_all, summed as integers: the
  // specials sit in an order that atomics chose, so a binary64 sum could
  // differ in its last bits from run to run (at most 2048 2^-51 t_all off);
  // a term above t_all / 2 is counted apart
  const double inv = 1.0 / t_all;
  uint64_t su = 0ull, big = 0ull;
#pragma unroll
  for (int k = 0; k < kSpPer; ++k) {
    if (tsp[k] <= 0.5 * t_all) su += to_units(tsp[k], inv);
    else big = 1ull;
  }
  uint64_t su_all, big_all;
  block_sum2_u64(su, big, (uint64_t*)s_w, &su_all, &big_all);
  const double t_sp = (double)su_all / kUnitScale * t_all;
  return (big_all == 0ull && t_sp <= 0.5 * t_all) ? t_all - t_sp : -1.0;
}

constexpr int kCountRank = 512;    // candidates the bin walk ranks by counting
constexpr int kCountSmall = 128;  // gathered candidates ranked by counting without the bins
constexpr int kWalkMin = 2048;    // a full draw's prefix past this many entries is walked, not sorted
__device__ __noinline__ uint32_t walk_cursor_by_bins(const uint64_t* list, int n_list, double T, const uint64_t* keys,
                                                     const uint32_t* ids, int n, double M, double range_lo,
                                                     double p0, double target, double mrg, uint64_t* bmass,
                                                     uint32_t* sel, double* wtmp, uint64_t* kminmax,
                                                     uint32_t* cscratch, uint32_t* hit_id, double* hit_term);

// The finish of row blockIdx.x. Returns 0 when the row's result is written,
// else kExactRequest | the result flags the exact path keeps.
__device__ __forceinline__ uint32_t finish_row(const SampleArgs& a, FinishLds& U) {
  Shared& S = U.fin;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t row = blockIdx.x;
  // ---- first batch of global loads, all issued before the row's
  // configuration arrives: the per-wave chunk statistics (thread t holds
  // chunk t / kScanWaves, wave t % kScanWaves), the first kSpecQ slots of
  // every sub-list, the history and forced-id offsets. The list slots are
  // read before the sub-lists' lengths are known: they lie inside the row's
  // list buffer, and entries past a sub-list's length are dropped once it is.
  // Every load here is unconditional (threads past the last chunk wave or
  // sub-list read the first one and drop it where the value is used), so no
  // branch merge makes a thread wait for its load before the next is issued.
  const int n_wstats = a.n_chunks * kScanWaves;  // <= kFinishThreads
  const bool has_w = tid < n_wstats;
  const int tw = has_w ? tid : 0;
  const ChunkStat* wc = a.stats + row * a.n_chunks + tw / kScanWaves;
  const double w_sum = wc->wsum[tw % kScanWaves];
  const uint32_t w_max = wc->wmax[tw % kScanWaves];
  const uint32_t w_flags = wc->wflags[tw % kScanWaves];
  const uint32_t w_nsub = wc->n_sub[tw % kScanWaves];
  const uint32_t w_thr = wc->threshold;
  const uint32_t w_trunc = wc->truncated;
  const uint64_t* lists = a.lists + row * a.n_chunks * kGatherCap;
  const int n_subs = a.n_chunks * kScanWaves;
  // absent arrays are read at a valid address (the configs) and dropped
  const int64_t* hoff = a.history_offsets ? a.history_offsets : (const int64_t*)a.configs;
  const int64_t* foff = a.forced_offsets ? a.forced_offsets : (const int64_t*)a.configs;
  const int64_t h0r = hoff[row], h1r = hoff[row + 1], f0r = foff[row], f1r = foff[row + 1];

  const gs_row_config cfg = a.configs[row];
  // the list slots go out after the configuration: the first wait (for the
  // configuration) does not wait for them
  const int sl0 = tid / kSubThreads, k0 = tid % kSubThreads;
  uint64_t lv[kSubPerThread];
#pragma unroll
  for (int q = 0; q < kSpecQ; ++q) lv[q] = lists[GS_CK((int64_t)(sl0 < n_subs ? sl0 : 0) * kSubCap + k0 + q * kSubThreads, (int64_t)a.n_chunks * kGatherCap)];
  const Plan plan = plan_row_flat(cfg);
  if (cfg.mask_slot >= a.mask_slots) {
    // a constrained row whose mask is not in the table: never sampled unmasked
    if (tid == 0) write_result(a, row, -1, GS_FLAG_INVALID_SLOT, 0.0);
    return 0;
  }
  if (plan.route == kRouteExact) {
    return kExactRequest | 0u;
  }
  const bool greedy = plan.route == kRouteGreedy;
  const int32_t slot = cfg.mask_slot;
  const bool constrained = slot >= 0 && slot < a.mask_slots;
  const double T = cfg.temperature;
  const int64_t h0 = a.history_offsets ? h0r : 0, h1 = a.history_offsets ? h1r : 0;
  // forced ids belong to constrained rows only
  const int64_t f0 = constrained && a.forced_offsets ? f0r : 0, f1 = constrained && a.forced_offsets ? f1r : 0;

  // the penalty window (sampling.ts:22-24)
  int64_t w0 = 0, w1 = 0;
  if (a.history_offsets && cfg.repetition_window > 0) {
    const int64_t s0 = h1 - (int64_t)cfg.repetition_window;
    w0 = s0 > h0 ? s0 : h0;
    w1 = h1;
  }
  // The window and forced ids this thread owns, loaded unconditionally (a
  // position past the list reads its last entry, an empty list a valid dummy
  // address) and dropped where used: a load under a branch that may be
  // skipped would make every later wait for an earlier load a full wait.
  constexpr int kOwn = kIdsPerThread + 1;
  int32_t oraw_id[kOwn];
  bool oid_ok[kOwn];
  uint8_t fkind_raw;
  {
    const bool has_win = w1 > w0;
    const int32_t* wb = has_win ? a.history_ids : (const int32_t*)a.configs;
#pragma unroll
    for (int r = 0; r < kIdsPerThread; ++r) {
      const int64_t j = w0 + tid + (int64_t)r * kFinishThreads;
      oid_ok[r] = j < w1;
      oraw_id[r] = wb[has_win ? (j < w1 ? j : w1 - 1) : 0];
    }
    const bool has_forced = f1 > f0;
    const int64_t jf = has_forced ? (f0 + tid < f1 ? f0 + tid : f1 - 1) : 0;
    oid_ok[kIdsPerThread] = f0 + tid < f1;
    oraw_id[kIdsPerThread] = (has_forced ? a.forced_ids : (const int32_t*)a.configs)[jf];
    fkind_raw = (has_forced ? a.forced_kinds : (const uint8_t*)a.configs)[jf];
  }
  // specials this thread owns the loads of: its window positions and its
  // first forced id; rows with longer lists evaluate from the hash slots
  const bool own_path = w1 - w0 <= (int64_t)kIdsPerThread * kFinishThreads && f1 - f0 <= kFinishThreads;

  if (tid == 0) {
    S.flags = 0; S.max_key = 0; S.thr_max = 0; S.any_truncated = 0; S.n_sorted = 0; S.n_special = 0;
    S.sel[GS_CK(3, GS_LEN(S.sel))] = 0;
    S.n_sp_in = 0; S.route_exact = 0; S.status_flags = 0; S.first_idx = 0xFFFFFFFFu; S.legal_bits = 0;
    S.special_legal = 0; S.best_entry = 0; S.sp_max = 0; S.fast_done = 0; S.short_sum = 0;
  }
  for (int h = tid; h < kHashSize; h += kFinishThreads) { S.hash_ids[GS_CK(h, GS_LEN(S.hash_ids))] = 0xFFFFFFFFu; S.hash_counts[GS_CK(h, GS_LEN(S.hash_counts))] = 0; }
  if (tid < 256) S.hist[GS_CK(tid, GS_LEN(S.hist))] = 0;
  __syncthreads();

  // ---- 1. statistics: sub-list lengths into LDS; the flags, the maximum and
  // the truncation threshold reduced per wave (one LDS atomic each)
  if (has_w) S.c_nsub[GS_CK(tid, GS_LEN(S.c_nsub))] = (uint16_t)(w_nsub > (uint32_t)kSubCap ? (uint32_t)kSubCap : w_nsub);
  {
    // a sub-list length above kSubCap: the sub-list overflowed
    const uint32_t fl = wave_or_u32(has_w ? w_flags | (w_nsub > (uint32_t)kSubCap ? kChunkOverflow : 0u) |
                                                (w_nsub > (uint32_t)(kSpecQ * kSubThreads) ? kDeepLists : 0u)
                                          : 0u);
    const uint32_t mk = wave_max_u32(has_w ? w_max : 0u);
    const uint32_t th = wave_max_u32(has_w && w_trunc ? w_thr : 0u);
    const bool tr = __ballot(has_w && w_trunc != 0) != 0;
    if (lane == 0) {
      if (fl) atomicOr(&S.flags, fl);
      if (mk) atomicMax(&S.max_key, mk);
      if (tr) { atomicMax(&S.thr_max, th); atomicOr(&S.any_truncated, 1u); }
    }
    // A floor for the fast path's top kTopR: each wave holding statistics
    // takes the d-th largest of its wave maxima (d = kTopR / those waves,
    // rounded up), so the smallest of these floors has at least kTopR wave
    // maxima -- distinct non-special logits -- at or above it.
    const int n_sw = (n_wstats + 63) / 64;
    if (wave < n_sw) {
      const uint32_t d = (uint32_t)((kTopR + n_sw - 1) / n_sw);
      const uint32_t key = has_w && w_max > kKeyNegInf ? w_max : 0u;
      uint32_t khi, klo;
      wave_max_min_u32(key, &khi, &klo);
      const uint32_t live = (uint32_t)__popcll(__ballot(key != 0u));
      const uint32_t f = live >= d ? wave_kth_key(key, d, klo, khi) : 0u;
      if (lane == 0) S.top_floor[GS_CK(wave, GS_LEN(S.top_floor))] = f;
    }
  }
  // the owned specials' logits and mask words start loading now; they are
  // first used after the region is ranked
  int32_t oid[kOwn];
  uint32_t okind[kOwn];
#pragma unroll
  for (int r = 0; r < kOwn; ++r) {
    oid[r] = oid_ok[r] ? oraw_id[r] : -1;
    okind[r] = r == kIdsPerThread ? (uint32_t)fkind_raw & 3u : 0u;
  }
  uint32_t oraw[kOwn];  // logit bits as loaded (bf16: the 16 bits, widened at use)
  uint32_t omw[kOwn];
  int oslot[kOwn];
  bool ofirst[kOwn];
  // Every load issued so far has arrived by now (they went out before the
  // row's configuration came back); wait for them here, before the first
  // loads that only some rows issue. A later wait for one of them (or a reuse
  // of its register) would otherwise count those too and wait for the gathers.
  static_assert(kSpecQ == 4, "the list slots read with the statistics, waited for here");
  asm volatile("" ::"v"(lv[0]), "v"(lv[1]), "v"(lv[2]), "v"(lv[3]), "v"((uint32_t)fkind_raw));
  {
    // unconditional loads again: ids that are not owned read index 0
    int64_t gi[kOwn];
#pragma unroll
    for (int r = 0; r < kOwn; ++r) gi[r] = own_path && oid[r] >= 0 && oid[r] < a.vocab ? oid[r] : 0;
    if (a.dtype == GS_BF16) {
      const uint16_t* lp = (const uint16_t*)a.logits + row * a.row_stride;
#pragma unroll
      for (int r = 0; r < kOwn; ++r) oraw[r] = lp[gi[r]];
    } else {
      const uint32_t* lp = (const uint32_t*)a.logits + row * a.row_stride;
#pragma unroll
      for (int r = 0; r < kOwn; ++r) oraw[r] = lp[gi[r]];
    }
    // mask words for constrained rows only (a branch the whole workgroup takes)
#pragma unroll
    for (int r = 0; r < kOwn; ++r) omw[r] = 0u;
    if (constrained) {
      const uint32_t* mrow = a.mask_table + (int64_t)slot * a.mask_words;
#pragma unroll
      for (int r = 0; r < kOwn; ++r) omw[r] = mrow[gi[r] >> 5];
    }
  }
  // distinct special ids into the hash
  {
    SpecialTable tab{S.hash_ids, S.hash_counts};
    bool lost = false;  // an id that found no slot: the table is too crowded
#pragma unroll
    for (int r = 0; r < kOwn; ++r) {
      oslot[r] = -1;
      ofirst[r] = false;
      if (oid[r] >= 0 && oid[r] < a.vocab) {
        ofirst[r] = special_insert_owner(tab, (uint32_t)oid[r], okind[r], &oslot[r]);
        lost |= oslot[r] < 0;
      }
    }
    for (int64_t j = w0 + tid + (int64_t)kIdsPerThread * kFinishThreads; j < w1 && !lost; j += kFinishThreads) {
      const int32_t id = a.history_ids[j];
      if (id >= 0 && id < a.vocab) lost |= !special_insert(tab, (uint32_t)id, 0u);
    }
    for (int64_t j = f0 + tid + kFinishThreads; j < f1 && !lost; j += kFinishThreads) {
      const int32_t id = a.forced_ids[j];
      if (id >= 0 && id < a.vocab) lost |= !special_insert(tab, (uint32_t)id, (uint32_t)a.forced_kinds[j] & 3u);
    }
    if (__ballot(lost) && lane == 0) atomicOr(&S.flags, kSpecialOverflow);
  }
  __syncthreads();
  if (S.flags & kChunkNonFinite) {
    return kExactRequest | GS_FLAG_NONFINITE;
  }
  if (S.flags & kSpecialOverflow) {
    // more distinct window and forced ids than the table holds: the exact
    // path counts them per vocabulary id
    return kExactRequest | 0u;
  }
  if (!greedy && (S.flags & kChunkOverflow)) {
    return kExactRequest | 0u;
  }

  // ---- second batch of global loads: the hash-slot specials' logits and
  // mask words (rows whose specials are not owned) and the list slots past
  // the first kSpecQ
  uint32_t thr = S.thr_max;  // 0 when no chunk was truncated: every finite logit is listed
  // the specials to evaluate: each owner's (own_path), else every hash slot
  constexpr int kEval = kSlotsPerThread > kOwn ? kSlotsPerThread : kOwn;
  uint32_t hid[kEval], hpk[kEval], mw[kEval];
  float raw[kEval];
  if (own_path) {
#pragma unroll
    for (int r = 0; r < kEval; ++r) {
      const bool mine = r < kOwn && ofirst[r];
      hid[r] = mine ? (uint32_t)oid[r] : 0xFFFFFFFFu;
      hpk[r] = mine ? S.hash_counts[GS_CK(oslot[r], GS_LEN(S.hash_counts))] : 0u;
      raw[r] = 0.0f;  // the owned loads are read where the special is evaluated
      mw[r] = 0u;
    }
  } else {
#pragma unroll
    for (int r = 0; r < kEval; ++r) {
      hid[r] = r < kSlotsPerThread ? S.hash_ids[GS_CK(tid + r * kFinishThreads, GS_LEN(S.hash_ids))] : 0xFFFFFFFFu;
      hpk[r] = r < kSlotsPerThread ? S.hash_counts[GS_CK(tid + r * kFinishThreads, GS_LEN(S.hash_counts))] : 0u;
    }
#pragma unroll
    for (int r = 0; r < kEval; ++r) {
      const bool used = hid[r] != 0xFFFFFFFFu;
      raw[r] = used ? load_logit(a, row, hid[r]) : 0.0f;
      mw[r] = used && constrained ? a.mask_table[(int64_t)slot * a.mask_words + (hid[r] >> 5)] : 0u;
    }
  }

  // ---- the complete region: listed entries with key >= thr, appended with
  // one LDS atomic per wave
  const uint32_t sel_lo = thr > kKeyNegInf ? thr : kKeyNegInf + 1u;
  const uint32_t sel_hi = S.max_key > sel_lo ? S.max_key : sel_lo;
  // slots [lo, cnt) of the thread's sub-list slots k0 + q * kSubThreads
  auto append = [&](const uint64_t (&v)[kSubPerThread], int lo, int cnt) {
    uint64_t e[kSubPerThread];
    uint32_t keep = 0;
#pragma unroll
    for (int q = 0; q < kSubPerThread; ++q) {
      e[q] = 0;
      const int k = k0 + q * kSubThreads;
      if (k >= lo && k < cnt) {
        e[q] = list_rank(v[q]);
        if (entry_key(e[q]) >= thr) keep |= 1u << q;
      }
    }
    const uint32_t mine = (uint32_t)__popc(keep);
    const uint32_t incl = wave_scan_u32(mine);
    uint32_t base = 0;
    if (lane == 63) base = atomicAdd(&S.n_sorted, incl);
    base = readlane_u32(base, 63);
    uint32_t pos = base + incl - mine;
#pragma unroll
    for (int q = 0; q < kSubPerThread; ++q) {
      if ((keep >> q) & 1u) {
        if (pos < (uint32_t)kFinishCap) S.sorted[GS_CK(pos, GS_LEN(S.sorted))] = e[q];
        ++pos;
      }
    }
  };
  // The fast selection works on the list entries the threads already hold:
  // the first kSpecQ * kSubThreads slots of every sub-list came with the
  // statistics (rows with no longer sub-list and at most
  // kFinishThreads / kSubThreads sub-lists). Other rows, and the paths that
  // need the whole region, append it to LDS; deeper slots are read there in a
  // pass of their own, so that the common path never waits for loads issued
  // after the special gathers.
  constexpr int kHead = kSpecQ * kSubThreads;
  const int cnt0 = sl0 < n_subs ? (int)S.c_nsub[GS_CK(sl0, GS_LEN(S.c_nsub))] : 0;
  bool region_in_lds = false;
  int n_region = 0;
  auto fill_region = [&]() {  // block-wide, ends with a barrier
#pragma unroll
    for (int q = kSpecQ; q < kSubPerThread; ++q) lv[q] = 0;
    append(lv, 0, cnt0 < kHead ? cnt0 : kHead);
    if (S.flags & kDeepLists) {
      uint64_t v[kSubPerThread];
#pragma unroll
      for (int q = 0; q < kSubPerThread; ++q) {
        const int k = k0 + q * kSubThreads;
        v[q] = (k >= kHead && k < cnt0) ? lists[GS_CK((int64_t)sl0 * kSubCap + k, (int64_t)a.n_chunks * kGatherCap)] : 0ull;
      }
      append(v, kHead, cnt0);
    }
    // sub-lists past the first kFinishThreads / kSubThreads (more than 32 chunks)
    for (int s0 = kFinishThreads / kSubThreads; s0 < n_subs; s0 += kFinishThreads / kSubThreads) {
      const int sl = s0 + tid / kSubThreads;
      const int cnt = sl < n_subs ? (int)S.c_nsub[GS_CK(sl, GS_LEN(S.c_nsub))] : 0;
      uint64_t v[kSubPerThread];
#pragma unroll
      for (int q = 0; q < kSubPerThread; ++q) {
        const int k = k0 + q * kSubThreads;
        v[q] = k < cnt ? lists[GS_CK((int64_t)sl * kSubCap + k, (int64_t)a.n_chunks * kGatherCap)] : 0ull;
      }
      append(v, 0, cnt);
    }
    __syncthreads();
    n_region = (int)S.n_sorted;
    region_in_lds = true;
  };
  // the region's top kTopR non-specials, ranked while the specials' loads are
  // still in flight (false: too many ties, the fast path merges instead)
  bool top_ok = false;
  if (!greedy) {
    if (!(S.flags & kDeepLists) && n_subs <= kFinishThreads / kSubThreads) {
      uint64_t e[kSpecQ];
      uint32_t valid = 0;
#pragma unroll
      for (int q = 0; q < kSpecQ; ++q) {
        e[q] = 0;
        if (k0 + q * kSubThreads < cnt0) {
          e[q] = list_rank(lv[q]);
          if (entry_key(e[q]) >= thr) valid |= 1u << q;
        }
      }
      // the tightest floor the wave maxima give (every stats wave found one)
      uint32_t tfl = 0xFFFFFFFFu;
      for (int w = 0; w < (n_wstats + 63) / 64; ++w) tfl = S.top_floor[GS_CK(w, GS_LEN(S.top_floor))] < tfl ? S.top_floor[GS_CK(w, GS_LEN(S.top_floor))] : tfl;
      if (tfl > sel_lo && tfl != 0xFFFFFFFFu)
        top_ok = top_select_regs_floor<kSpecQ>(e, valid, tfl, sel_hi, S.hist, S.sel, (uint64_t*)S.cand_p, S.top,
                                               &S.n_sorted);
      else
        top_ok = top_select_regs<kSpecQ>(e, valid, -1, sel_lo, sel_hi, S.hist, S.sel, (uint64_t*)S.cand_p, S.top,
                                         &S.n_sorted);
      n_region = (int)S.n_sorted;
    } else {
      fill_region();
      if (n_region > kFinishCap) {
        // More entries than the LDS region holds. Any floor above the current
        // one leaves a complete region: a histogram of the listed keys (read
        // again from the lists) finds the lowest bin boundary with at most
        // kFinishCap entries above it, and the region is filled again above it.
        const int shift = top_select_shift(sel_lo, sel_hi);
        for (int s0 = 0; s0 < n_subs; s0 += kFinishThreads / kSubThreads) {
          const int sl = s0 + tid / kSubThreads;
          const int cnt = sl < n_subs ? (int)S.c_nsub[GS_CK(sl, GS_LEN(S.c_nsub))] : 0;
          // a trip count the whole wave shares (hist_add needs every lane)
#pragma unroll 1
          for (int k = k0; __ballot(k < cnt) != 0; k += kSubThreads) {
            const uint32_t key =
                k < cnt ? entry_key(list_rank(lists[GS_CK((int64_t)sl * kSubCap + k, (int64_t)a.n_chunks * kGatherCap)]))
                        : 0u;
            const uint32_t bin = (key - sel_lo) >> shift;
            hist_add(S.hist, GS_CK(bin < 255u ? bin : 255u, GS_LEN(S.hist)), k < cnt && key >= thr);
          }
        }
        __syncthreads();
        if (wave == 0) {
          // lane l holds bins 255-4l .. 252-4l, highest first
          uint32_t h[4], c = 0;
#pragma unroll
          for (int q = 0; q < 4; ++q) { h[q] = S.hist[GS_CK(255 - 4 * lane - q, GS_LEN(S.hist))]; c += h[q]; }
          const uint32_t incl = wave_scan_u32(c);
          const uint64_t hit = __ballot(incl > (uint32_t)kFinishCap);
          const int first = hit ? __ffsll((unsigned long long)hit) - 1 : 64;
          if (lane == first) {
            uint32_t cum = incl - c;
            int q = 0;
            while (cum + h[q] <= (uint32_t)kFinishCap) { cum += h[q]; ++q; }
            S.sel[GS_CK(0, GS_LEN(S.sel))] = (uint32_t)(255 - 4 * lane - q) + 1u;  // the lowest bin kept (256: none)
          }
          if (first == 64 && lane == 0) S.sel[GS_CK(0, GS_LEN(S.sel))] = 0u;
        }
        __syncthreads();
        const uint32_t b = S.sel[GS_CK(0, GS_LEN(S.sel))];
        if (tid < 256) S.hist[GS_CK(tid, GS_LEN(S.hist))] = 0;
        if (b == 0u || b > 255u) return kExactRequest | 0u;  // all of it fits, or no boundary fits
        thr = sel_lo + (b << shift);
        if (tid == 0) { S.n_sorted = 0; S.any_truncated = 1u; }
        __syncthreads();
        fill_region();
      }
      if (n_region <= kFinishCap)
        top_ok = top_select(S.sorted, n_region, thr > sel_lo ? thr : sel_lo, sel_hi, S.hist, S.sel,
                            (uint64_t*)S.cand_p, S.top);
    }
  }
  // the whole region in LDS, for the paths that rank or sort it
  auto need_region = [&]() {
    if (region_in_lds) return;
    __syncthreads();
    if (tid == 0) S.n_sorted = 0;
    __syncthreads();
    fill_region();
  };

  // evaluate every special exactly: mask / termination rules, then penalties.
  // Slots, flags and the maximum are gathered per wave, one LDS atomic each.
  {
    uint64_t my_max = 0;
    bool my_legal = false, my_nonfinite = false;
#pragma unroll
    for (int r = 0; r < kEval; ++r) {
      const uint32_t id = hid[r];
      const bool used = id != 0xFFFFFFFFu;
      const uint64_t m = __ballot(used);
      if (m == 0) continue;
      uint32_t base = 0;
      if (lane == 0) base = atomicAdd(&S.n_special, (uint32_t)__popcll(m));
      base = readlane_u32(base, 0);
      if (!used) continue;
      const uint32_t idx =
          base + __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
      if (idx >= (uint32_t)kSpecialCap) continue;
      const uint32_t count = hpk[r] & 0xFFFFFFu, kinds = hpk[r] >> 24;
      float x32 = raw[r];
      uint32_t mword = mw[r];
      if (own_path && r < kOwn) {
        const uint32_t b = oraw[r < kOwn ? r : 0];
        x32 = __builtin_bit_cast(float, a.dtype == GS_BF16 ? b << 16 : b);
        mword = omw[r < kOwn ? r : 0];
      }
      if (cfg.softcap > 0) x32 = softcap_call(x32, cfg.softcap);
      bool allowed = true;
      if (constrained) {
        const bool term = kinds & GS_FORCED_TERMINATION;
        const bool extra = kinds & GS_FORCED_EXTRA;
        allowed = term ? cfg.accepting != 0 : (extra || ((mword >> (id & 31)) & 1u));
      }
      my_legal |= allowed;
      my_nonfinite |= allowed && !(x32 < __builtin_inff());
      double x = allowed ? (double)x32 : -__builtin_inf();
      if (count > 0) {
        x = x < 0 ? x * cfg.repetition_penalty : x / cfg.repetition_penalty;
        x -= cfg.presence_penalty + (double)count * cfg.frequency_penalty;
      }
      const double v = greedy ? x : x / T;
      const uint64_t key = f64_key(v);
      S.sp_key[GS_CK(idx, GS_LEN(S.sp_key))] = key;
      S.sp_id[GS_CK(idx, GS_LEN(S.sp_id))] = id;
      my_max = key > my_max ? key : my_max;
    }
    const uint64_t legal_w = __ballot(my_legal), bad_w = __ballot(my_nonfinite);
    my_max = wave_max_u64(my_max);
    if (lane == 0) {
      if (legal_w) atomicOr(&S.special_legal, 1u);
      if (bad_w) atomicOr(&S.flags, kChunkNonFinite);
      if (my_max) atomicMax((unsigned long long*)&S.sp_max, (unsigned long long)my_max);
    }
  }
  __syncthreads();
  if (S.n_special > (uint32_t)kSpecialCap) {
    // more specials than the finish evaluates: the exact path takes any number
    return kExactRequest | 0u;
  }
  if (S.flags & kChunkNonFinite) {
    return kExactRequest | GS_FLAG_NONFINITE;
  }
  const int n_sp = (int)S.n_special;

  // ---- constrained dead end: no legal id at all (gemma-session.ts:1322-1326)
  if (constrained && S.max_key <= kKeyNegInf && !S.special_legal) {
    // a non-special id is legal iff its mask bit is set; count those bits
    const uint32_t* m = a.mask_table + (int64_t)slot * a.mask_words;
    uint32_t bits = 0;
    for (int w = tid; w < a.mask_words; w += kFinishThreads) bits |= m[w];
    if (bits) atomicOr(&S.legal_bits, 1u);
    __syncthreads();
    const uint32_t any_bits = S.legal_bits;
    __syncthreads();
    // specials' own mask bits may be the only set bits: those ids are not legal
    // (termination) or were evaluated above; count non-special legal bits exactly
    if (any_bits) {
      if (tid == 0) S.legal_bits = 0;
      __syncthreads();
      for (int w = tid; w < a.mask_words; w += kFinishThreads) {
        uint32_t word = m[w];
        for (int i = 0; i < n_sp; ++i) {
          const uint32_t id = S.sp_id[GS_CK(i, GS_LEN(S.sp_id))];
          if ((int)(id >> 5) == w) word &= ~(1u << (id & 31));
        }
        if (word) atomicOr(&S.legal_bits, 1u);
      }
      __syncthreads();
    }
    if (!S.legal_bits) {
      if (tid == 0) write_result(a, row, -1, GS_FLAG_DEAD_END, 0.0);
      return 0;
    }
  }

  // ---- greedy: first maximum of the penalised logits (sampling.ts:31,92-96)
  if (greedy) {
    for (int c = tid; c < a.n_chunks; c += kFinishThreads) {
      if (S.c_nsub[GS_CK(c * kScanWaves, GS_LEN(S.c_nsub))]) {
        atomicMax((unsigned long long*)&S.best_entry, (unsigned long long)list_rank(lists[GS_CK((int64_t)c * kGatherCap, (int64_t)a.n_chunks * kGatherCap)]));
      }
    }
    __syncthreads();
    if (tid == 0) {
      // best special by (value desc, id asc)
      int bs = -1;
      for (int i = 0; i < n_sp; ++i) {
        if (bs < 0 || ranks_before(S.sp_key[GS_CK(i, GS_LEN(S.sp_key))], S.sp_id[GS_CK(i, GS_LEN(S.sp_id))], S.sp_key[GS_CK(bs, GS_LEN(S.sp_key))], S.sp_id[GS_CK(bs, GS_LEN(S.sp_id))])) bs = i;
      }
      int32_t token;
      if (S.best_entry == 0) {
        token = bs >= 0 ? (int32_t)S.sp_id[GS_CK(bs, GS_LEN(S.sp_id))] : 0;
      } else {
        const uint32_t nid = entry_id(S.best_entry);
        const uint64_t nkey = f64_key((double)key_f32(entry_key(S.best_entry)));
        token = (bs >= 0 && ranks_before(S.sp_key[GS_CK(bs, GS_LEN(S.sp_key))], S.sp_id[GS_CK(bs, GS_LEN(S.sp_id))], nkey, nid)) ? (int32_t)S.sp_id[GS_CK(bs, GS_LEN(S.sp_id))]
                                                                                 : (int32_t)nid;
      }
      write_result(a, row, token, GS_FLAG_GREEDY, 1.0);
    }
    return 0;
  }

  if (n_region > kFinishCap) {
    return kExactRequest | 0u;
  }
  const int n_ns = n_region;

  // ---- the maximum value M = scaled[0].logit (sampling.ts:36): the best
  // finite non-special logit / T, or the best special value
  double M = -__builtin_inf();
  if (S.max_key > kKeyNegInf) M = (double)key_f32(S.max_key) / T;
  if (S.sp_max) {
    const double sm = key_f64(S.sp_max);
    if (sm > M) M = sm;
  }
  if (!(M > -__builtin_inf())) {
    // every logit is -inf: the reference's arithmetic turns NaN; replay it exactly
    return kExactRequest | 0u;
  }
  // Margins for the comparisons that depend on the normaliser (the top-p
  // cut). This total and the reference's differ by the scan's normaliser
  // error (kScanSumRel; kNormaliserRel once recomputed in binary64),
  // summation order (under V 2^-53 < 3e-11) and the reference's rounding of
  // l/T and of l/T - M in every term (2^-52 (2|M| + 60) for the terms that
  // matter) and of the rescale arguments (2^-53 |M|).
  const double ref_round = 0x1p-52 * (3.0 * (M < 0 ? -M : M) + 60.0);
  const double margin_fine = kNormaliserRel + ref_round;
  // how far the reference's sum of all V probabilities (each rounded, summed
  // in list order) lies from 1 at most
  const double full_mass_rel = (2.0 * (double)a.vocab + 2.0) * 0x1p-53;
  double margin = kScanSumRel + ref_round;
  bool refined = false;

  // ---- normaliser: the scan's per-wave partial sums rescaled from their wave
  // maximum to M (the rescale argument computed as the reference computes
  // l/T - M for that logit), plus every special (threads from the top down,
  // so that they are not the ones holding wave sums). The specials sit in
  // LDS in an order that atomics chose, so their terms (each at most 1: M is
  // at least every special's value) are summed as integers in units of
  // 2^-50 (at most 2048 2^-51 < 1e-12 off, against a normaliser of at least
  // 1): every run of a row gets the same normaliser, bit for bit.
  double t_chunks, t_sp;
  {
    double part = 0.0;
    uint64_t spart = 0ull;
    if (has_w && w_sum > 0.0 && w_max > kKeyNegInf) part = w_sum * gsm::js_exp((double)key_f32(w_max) / T - M);
    for (int i = kFinishThreads - 1 - tid; i < n_sp; i += kFinishThreads) spart += to_units(gsm::js_exp(key_f64(S.sp_key[GS_CK(i, GS_LEN(S.sp_key))]) - M), 1.0);
    uint64_t sp_units;
    block_sum_f64_u64(part, spart, S.wsum2, &t_chunks, &sp_units);
    t_sp = (double)sp_units / kUnitScale;
    if (tid == 0) { S.total = t_chunks + t_sp; S.total_sp = t_sp; }
  }
  if (!(t_chunks + t_sp < __builtin_inf())) {
    // an exponent argument beyond the double range (|l/T| near 1e18 or more)
    return kExactRequest | 0u;
  }

  // specials inside the complete region (value >= the threshold's value),
  // compacted into the dead hash table (one LDS atomic per wave) and ordered
  // there: up to 64 by one wave counting each one's rank, more by a
  // block-wide bitonic sort; usually there are none or a few
  uint64_t* in_key = (uint64_t*)S.hash_ids;
  uint32_t* in_id = S.hash_counts;
  const uint64_t region_floor = thr ? f64_key((double)key_f32(thr) / T) : 0;
  for (int i0 = 0; i0 < n_sp; i0 += kFinishThreads) {
    const int i = i0 + tid;
    const bool in = i < n_sp && S.sp_key[GS_CK(i, GS_LEN(S.sp_key))] >= region_floor;
    const uint64_t m = __ballot(in);
    uint32_t base = 0;
    if (lane == 0 && m) base = atomicAdd(&S.n_sp_in, (uint32_t)__popcll(m));
    base = readlane_u32(base, 0);
    if (in) {
      const uint32_t p = base + __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
      in_key[GS_CK(p, kHashSize / 2)] = S.sp_key[GS_CK(i, GS_LEN(S.sp_key))];
      in_id[GS_CK(p, kHashSize)] = S.sp_id[GS_CK(i, GS_LEN(S.sp_id))];
    }
  }
  __syncthreads();
  const int n_sp_in = (int)S.n_sp_in;
  if (n_sp_in <= 64) {
    if (n_sp_in > 1 && wave == 0) {
      const uint64_t k = lane < n_sp_in ? in_key[GS_CK(lane, kHashSize / 2)] : 0ull;
      const uint32_t id = lane < n_sp_in ? in_id[GS_CK(lane, kHashSize)] : 0xFFFFFFFFu;
      int rank = 0;  // the ids are distinct, so the ranks are too
      for (int j = 0; j < n_sp_in; ++j) rank += ranks_before(readlane_u64(k, j), readlane_u32(id, j), k, id) ? 1 : 0;
      if (lane < n_sp_in) {
        in_key[GS_CK(rank, kHashSize / 2)] = k;
        in_id[GS_CK(rank, kHashSize)] = id;
      }
    }
    __syncthreads();
  } else {
    const int m2 = pow2_at_least(n_sp_in);
    for (int i = n_sp_in + tid; i < m2; i += kFinishThreads) { in_key[GS_CK(i, kHashSize / 2)] = 0; in_id[GS_CK(i, kHashSize)] = 0xFFFFFFFFu; }
    __syncthreads();
    block_sort_pairs_desc(in_key, in_id, m2);
  }
  if (n_ns + n_sp_in == 0) {
    return kExactRequest | 0u;
  }
  double total = S.total;
  const bool region_complete = !S.any_truncated;
  // after a recomputed normaliser: the new total and the tight margin (the
  // whole block calls it; false when the row must take the exact path)
  auto refine = [&]() -> bool {
    // the table exponential's table into LDS (the deep draw's copy, if any, is the same)
    if (tid < 256) S.tab[GS_CK(tid, GS_LEN(S.tab))] = c_exp2_256[tid];
    __syncthreads();
    const double part = recompute_nonspecial_sum(a, row, cfg, constrained, M, n_sp, S.sp_id, S.wsum2, S.tab);
    if (!(part >= 0)) return false;
    total = part + S.total_sp;
    margin = margin_fine;
    refined = true;
    return true;
  };

  // ---- fast path: the top kTopR non-specials, merged with the region's
  // specials, settle every cut the filters make within them (when the
  // specials fit beside them in 2 * kTopR candidates)
  const int n_top_all = n_ns < kTopR ? n_ns : kTopR;
  if (n_sp_in <= 2 * kTopR - n_top_all) {
    uint64_t* tmp = (uint64_t*)S.cand_p;  // kWaves * 64 entries of merge scratch
    if (!top_ok) {
      need_region();
      if (n_ns <= kWaves * 64) top_r<1>(S.sorted, n_ns, tmp, S.top);
      else if (n_ns <= kWaves * 128) top_r<2>(S.sorted, n_ns, tmp, S.top);
      else top_r<4>(S.sorted, n_ns, tmp, S.top);
    }
    double* fp = S.cand_p + kWaves * 64;  // past the merge scratch
    uint32_t* fid = S.cand_id;
    int n_valid = 0;
    bool complete = false;
    if (wave == 0) {
      const int n_top = n_ns < kTopR ? n_ns : kTopR;
      const int n_sp_use = n_sp_in;
      for (int i = lane; i < n_top; i += 64) {
        const uint64_t e = S.top[GS_CK(i, GS_LEN(S.top))];
        const uint32_t id = entry_id(e);
        const uint64_t k = f64_key(nonspecial_value(e, T));
        int lo = 0, hi = n_sp_use;  // specials ranked before this entry
        while (lo < hi) {
          const int mid = (lo + hi) >> 1;
          if (ranks_before(in_key[GS_CK(mid, kHashSize / 2)], in_id[GS_CK(mid, kHashSize)], k, id)) lo = mid + 1; else hi = mid;
        }
        fp[GS_CK(i + lo, (kFinishCap - kWaves * 64))] = key_f64(k);
        fid[GS_CK(i + lo, kFinishCap)] = id;
      }
      for (int j = lane; j < n_sp_use; j += 64) {
        const uint64_t k = in_key[GS_CK(j, kHashSize / 2)];
        const uint32_t id = in_id[GS_CK(j, kHashSize)];
        int lo = 0, hi = n_top;  // ranked non-specials before this special
        while (lo < hi) {
          const int mid = (lo + hi) >> 1;
          const uint64_t e = S.top[GS_CK(mid, GS_LEN(S.top))];
          if (ranks_before(f64_key(nonspecial_value(e, T)), entry_id(e), k, id)) lo = mid + 1; else hi = mid;
        }
        fp[GS_CK(j + lo, (kFinishCap - kWaves * 64))] = key_f64(k);
        fid[GS_CK(j + lo, kFinishCap)] = id;
      }
      // the merged list equals the row's list up to the last ranked
      // non-special; specials below it may sit under unranked non-specials
      n_valid = n_top + n_sp_use;
      complete = region_complete && n_ns <= kTopR;
      if (n_ns > kTopR) {
        const uint64_t e = S.top[GS_CK(kTopR - 1, GS_LEN(S.top))];
        const uint64_t lk = f64_key(nonspecial_value(e, T));
        int after = 0;
        for (int j = lane; j < n_sp_use; j += 64) {
          if (!ranks_before(in_key[GS_CK(j, kHashSize / 2)], in_id[GS_CK(j, kHashSize)], lk, entry_id(e))) ++after;
        }
        after = (int)wave_sum_u32((uint32_t)after);
        n_valid -= after;
      }
      // a top-k cut inside the candidates is the list's own (sampling.ts:44):
      // only the first topK exponentials are needed
      if (cfg.top_k > 0 && cfg.top_k < n_valid) {
        n_valid = cfg.top_k;
        complete = true;
      }
      __builtin_amdgcn_wave_barrier();
      for (int i = lane; i < n_valid; i += 64) fp[GS_CK(i, (kFinishCap - kWaves * 64))] = gsm::js_exp(fp[GS_CK(i, (kFinishCap - kWaves * 64))] - M);
      __builtin_amdgcn_wave_barrier();
      uint32_t xf = 0;
      const int r = filters_and_draw_wave(a, row, cfg, fp, total, fid, n_valid, complete, margin, true, full_mass_rel,
                                          fp + 2 * kTopR, &xf);
      if (lane == 0) {
        S.fast_done = r == 0 ? 1u : (r == 2 ? 2u : (r == 3 ? 3u : 0u));
        S.exact_flags = xf;
      }
    }
    __syncthreads();
    if (S.fast_done == 2) {
      if (!refine()) {
        return kExactRequest | GS_FLAG_NEAR_TIE;
      }
      if (wave == 0) {
        uint32_t xf = 0;
        const int r = filters_and_draw_wave(a, row, cfg, fp, total, fid, n_valid, complete, margin, false,
                                            full_mass_rel, fp + 2 * kTopR, &xf);
        if (lane == 0) {
          S.fast_done = r == 0 ? 1u : (r == 3 ? 3u : 0u);
          S.exact_flags = xf;
        }
      }
      __syncthreads();
    }
    if (S.fast_done == 3) {
      return kExactRequest | S.exact_flags;
    }
    if (S.fast_done) return 0;
  }

  // ---- slow path: the candidates ranked block-wide, then the filters
  // (typical-p needs its whole pool among the fast path's candidates)
  if (cfg.typical_p < 1) {
    return kExactRequest | 0u;
  }
  // Only the candidates up to the pool's end are ranked: the first topK, or
  // those up to where the cumulative probability passes topP by twice the
  // margin of its comparisons (sampling.ts:44,56,82-90; min-p only shortens
  // the pool, and a cut inside the pool is the same whatever follows it). A
  // histogram of the region's keys, with each bin's mass e^(v - M) (binary32
  // exponentials summed as integers), finds the highest bin boundary above
  // which either bound is met.
  // Both undercount: the count takes non-specials only, the mass is scaled
  // down by 2^-10 (its binary32 terms err by under 1e-5 relative, and their
  // truncation to 2^-40 units only lowers it). The candidates whose
  // value is at or above the boundary's, specials included, are then the
  // candidate list's first n_pre + n_sp_pre: every other one ranks below
  // them all. The top-p pass checks the mass it sums over them.
  int n_pre = n_ns, n_sp_pre = n_sp_in;
  bool pre_cut = false;  // the ranked candidates end before the region does
  // a draw whose pool is the whole row (the draw's margin as below)
  const bool draw_pool = cfg.top_p >= 1 && cfg.top_k <= 0 && !(cfg.min_p > 0) && !constrained;
  const double u_draw = cfg.rng_mode == GS_RNG_EXPLICIT ? cfg.uniform : gsm::mulberry32_draw(cfg.seed, cfg.draw_index);
  const double draw_margin = margin + full_mass_rel + kNearTie;
  {
    uint64_t* scratch = (uint64_t*)S.cand_p;
    need_region();
    // a full-vocabulary draw ranks up to its cursor u, by twice the draw's margin
    const double want_m = cfg.top_p < 1 ? (cfg.top_p + 2.0 * margin) * total
                                        : (draw_pool ? (u_draw + 2.0 * draw_margin) * total : __builtin_inf());
    const uint32_t floor_key = prefix_floor(S.sorted, n_ns, in_key, n_sp_in, sel_lo, sel_hi, T, M, cfg.top_k, want_m,
                                            S.hist, (uint64_t*)S.tab, S.sel, scratch, &S.pre_mass);
    if (draw_pool && n_ns + n_sp_in <= kFinishCap &&
        S.pre_mass * (1.0 + 0x1p-10) + 1e-30 < (u_draw - 2.0 * draw_margin) * total) {
      // the cursor lies past the region, with room: the deep draw needs only
      // the candidates' exact terms, in any order
      for (int i = tid; i < n_ns; i += kFinishThreads) {
        const uint64_t e = S.sorted[GS_CK(i, GS_LEN(S.sorted))];
        S.cand_p[GS_CK(i, GS_LEN(S.cand_p))] = gsm::js_exp(nonspecial_value(e, T) - M);
        S.cand_id[GS_CK(i, GS_LEN(S.cand_id))] = entry_id(e);
      }
      for (int j = tid; j < n_sp_in; j += kFinishThreads) {
        S.cand_p[GS_CK(n_ns + j, GS_LEN(S.cand_p))] = gsm::js_exp(key_f64(in_key[GS_CK(j, kHashSize / 2)]) - M);
        S.cand_id[GS_CK(n_ns + j, GS_LEN(S.cand_id))] = in_id[GS_CK(j, kHashSize)];
      }
      if (tid == 0) {
        S.deep_m = M;
        S.deep_u = u_draw;
        S.deep_thr = thr;
        S.deep_floor = region_floor;
        S.deep_n = (uint32_t)(n_ns + n_sp_in);
        S.deep_margin = full_mass_rel + kNearTie;
      }
      __syncthreads();
      return kDeepRequest;
    }
    const int n_rank = floor_key ? (int)S.sel[GS_CK(3, GS_LEN(S.sel))] : n_ns;
    if (draw_pool && n_rank > kWalkMin && thr > kKeyNegInf && n_sp_in <= kHashSize - 5 * kCountRank) {
      // a full-vocabulary draw whose cursor falls deep in the complete
      // region: walk only the value bin it falls in (the region left
      // unsorted; every candidate's value lies in [floor value, M]);
      // cursors near a prefix, a wrong bin or a crowded one go the sorted
      // way below (the walk's scratch, the end of the in-region specials' id
      // array, lies past their n_sp_in entries)
      uint32_t hit_id = 0;
      double hit_term = 0.0;
      const uint32_t w = walk_cursor_by_bins(S.sorted, n_ns, T, in_key, in_id, n_ns + n_sp_in, M,
                                             (double)key_f32(thr) / T, 0.0, u_draw * total, draw_margin * total,
                                             (uint64_t*)S.tab, (uint32_t*)(S.top + 2), S.wsum2, S.top,
                                             S.hash_counts + (kHashSize - 5 * kCountRank), &hit_id, &hit_term);
      if (w == 0u) {
        if (tid == 0) write_result(a, row, (int32_t)hit_id, S.status_flags, hit_term / total);
        return 0;
      }
    }
    if (floor_key) {
      n_pre = (int)S.sel[GS_CK(3, GS_LEN(S.sel))];
      // specials at or above the boundary's value (in_key is descending)
      const uint64_t vfloor = f64_key((double)key_f32(floor_key) / T);
      int lo = 0, hi = n_sp_in;
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (in_key[GS_CK(mid, kHashSize / 2)] >= vfloor) lo = mid + 1; else hi = mid;
      }
      n_sp_pre = lo;
      pre_cut = true;
    }
    const uint64_t* src = pre_cut ? scratch : S.sorted;
    const int len = pow2_at_least(n_pre);
    if (n_pre <= kFinishThreads) sort_region<1>(src, n_pre, len > 1 ? len : 1, S.sorted, scratch);
    else if (n_pre <= 2 * kFinishThreads) sort_region<2>(src, n_pre, len, S.sorted, scratch);
    else sort_region<4>(src, n_pre, len, S.sorted, scratch);
  }
  const int n_cand = n_pre + n_sp_pre;
  if (n_cand > kFinishCap) {
    return kExactRequest | 0u;
  }
  // merge by rank into (value, id), then probabilities (sampling.ts:39,42)
  for (int i = tid; i < n_pre; i += kFinishThreads) {
    const uint64_t e = S.sorted[GS_CK(i, GS_LEN(S.sorted))];
    const uint32_t id = entry_id(e);
    const uint64_t k = f64_key(nonspecial_value(e, T));
    int lo = 0, hi = n_sp_pre;  // specials ranked before this entry
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (ranks_before(in_key[GS_CK(mid, kHashSize / 2)], in_id[GS_CK(mid, kHashSize)], k, id)) lo = mid + 1; else hi = mid;
    }
    S.cand_p[GS_CK(i + lo, GS_LEN(S.cand_p))] = key_f64(k);
    S.cand_id[GS_CK(i + lo, GS_LEN(S.cand_id))] = id;
  }
  for (int j = tid; j < n_sp_pre; j += kFinishThreads) {
    const uint64_t k = in_key[GS_CK(j, kHashSize / 2)];
    const uint32_t id = in_id[GS_CK(j, kHashSize)];
    int lo = 0, hi = n_pre;  // non-specials ranked before this special
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      const uint64_t e = S.sorted[GS_CK(mid, GS_LEN(S.sorted))];
      if (ranks_before(f64_key(nonspecial_value(e, T)), entry_id(e), k, id)) lo = mid + 1; else hi = mid;
    }
    S.cand_p[GS_CK(j + lo, GS_LEN(S.cand_p))] = key_f64(k);
    S.cand_id[GS_CK(j + lo, GS_LEN(S.cand_id))] = id;
  }
  __syncthreads();
  // exponentials; probability = e / total where the filters read them
  for (int i = tid; i < n_cand; i += kFinishThreads) S.cand_p[GS_CK(i, GS_LEN(S.cand_p))] = gsm::js_exp(S.cand_p[GS_CK(i, GS_LEN(S.cand_p))] - M);
  __syncthreads();

  // ---- top-k (sampling.ts:44)
  int n = n_cand;
  bool n_complete = region_complete && !pre_cut;
  if (cfg.top_k > 0 && (cfg.top_k < n || (pre_cut && cfg.top_k == n))) {
    n = cfg.top_k;
    n_complete = true;  // the first topK of the sorted list are all present
  }
  // ---- min-p (sampling.ts:45-48): p is non-increasing along the list
  if (cfg.min_p > 0) {
    const double floor_p = S.cand_p[GS_CK(0, GS_LEN(S.cand_p))] / total * cfg.min_p;
    uint32_t my_first = 0xFFFFFFFFu, my_route = 0;
    for (int i = tid; i < n; i += kFinishThreads) {
      const double p = S.cand_p[GS_CK(i, GS_LEN(S.cand_p))] / total;
      if (i + 1 < n && S.cand_p[GS_CK(i + 1, GS_LEN(S.cand_p))] / total > p) my_route |= 1u;  // not monotone: replay
      if (!(p >= floor_p) && (uint32_t)i < my_first) my_first = (uint32_t)i;
      const double d = p >= floor_p ? p - floor_p : floor_p - p;
      if (d < kNearTie * floor_p) my_route |= 2u;
    }
    // one LDS atomic per wave
    my_first = wave_min_u32(my_first);
    my_route = wave_or_u32(my_route);
    if (lane == 0) {
      if (my_first != 0xFFFFFFFFu) atomicMin(&S.first_idx, my_first);
      if (my_route) atomicOr(&S.route_exact, my_route);
    }
    __syncthreads();
    if (S.first_idx != 0xFFFFFFFFu) {
      n = (int)S.first_idx;
      n_complete = true;
    }
    __syncthreads();
    if (tid == 0) S.first_idx = 0xFFFFFFFFu;
    __syncthreads();
    if (n == 0) {
      if (tid == 0) write_result(a, row, -1, GS_FLAG_EMPTY_CANDIDATES, 0.0);
      return 0;
    }
  }
  // ---- top-p (sampling.ts:56,82-90) on inclusive prefix sums
  constexpr int kPer = kFinishCap / kFinishThreads;
  uint32_t tie_report = 0;
  if (cfg.top_p < 1) {
    double local[kPer];
    double base;
    for (;;) {
      double s = 0.0;
      for (int q = 0; q < kPer; ++q) {
        const int i = tid * kPer + q;
        s += i < n ? S.cand_p[GS_CK(i, GS_LEN(S.cand_p))] / total : 0.0;
        local[q] = s;
      }
      double tot;
      base = block_scan_f64(s, S.wtmp, &tot) - s;
      uint32_t my_first = 0xFFFFFFFFu;
      bool my_near = false;
      for (int q = kPer - 1; q >= 0; --q) {
        const int i = tid * kPer + q;
        if (i >= n) continue;
        const double cum = base + local[q];
        if (cum >= cfg.top_p) my_first = (uint32_t)i;
        const double d = cum >= cfg.top_p ? cum - cfg.top_p : cfg.top_p - cum;
        if (d < margin) my_near = true;
        // ranked candidates that end before the pool does settle the
        // comparisons past them only when their sum passes topP by twice the
        // margin (the last one's cumulative sum, set on every pass)
        if (i == n - 1 && pre_cut && !n_complete) S.short_sum = cum >= cfg.top_p + 2.0 * margin ? 0u : 1u;
      }
      // one LDS atomic per wave
      my_first = wave_min_u32(my_first);
      const bool wave_near = __ballot(my_near) != 0;
      if (lane == 0) {
        if (my_first != 0xFFFFFFFFu) atomicMin(&S.first_idx, my_first);
        if (wave_near) atomicOr(&S.route_exact, 4u);
      }
      __syncthreads();
      // a cut within the scan normaliser's margin alone: recompute it, redo
      if (refined || S.route_exact != 4u) break;
      __syncthreads();
      if (tid == 0) { S.route_exact = 0; S.first_idx = 0xFFFFFFFFu; }
      if (!refine()) {
        return kExactRequest | GS_FLAG_NEAR_TIE;
      }
      __syncthreads();
    }
    const uint32_t cut_idx = S.first_idx;
    int cut = (int)cut_idx;  // index of the item that reached topP
    if (cut_idx == 0xFFFFFFFFu || S.short_sum) {
      if (!n_complete) {
        return kExactRequest | 0u;
      }
      cut = n - 1;
    } else if (cut_idx >= (uint32_t)n) {
      return kExactRequest | GS_FLAG_INDEX_CHECK;
    } else if (tid == cut / kPer) {
      // 1e-6 boundary ties, as the reference comparison plan reports them
      const double cum = base + local[cut % kPer];
      const double prev = cum - S.cand_p[GS_CK(cut, GS_LEN(S.cand_p))] / total;
      if (cum - cfg.top_p <= kTieReport * cfg.top_p || (cut > 0 && cfg.top_p - prev <= kTieReport * cfg.top_p)) {
        atomicOr(&S.status_flags, GS_FLAG_TOPP_TIE);
      }
    }
    n = cut + 1;
    __syncthreads();
    if (tid == 0) S.first_idx = 0xFFFFFFFFu;
    __syncthreads();
  }
  // no cut reached past the region: the pool is the whole row (a
  // full-vocabulary draw), whose candidate total is the row's whole mass
  const bool full_mass = cfg.top_p >= 1 && !n_complete;
  if (full_mass && !(cfg.top_k <= 0 && !(cfg.min_p > 0))) {
    // a top-k or min-p pool that ends past the region
    return kExactRequest | 0u;
  }
  tie_report = S.status_flags;

  // ---- draw (sampling.ts:58-64): first i with prefix_i >= u * sum_{j<n} p_j
  // (with a full pool: u * 1, the prefix sums carrying the normaliser's error,
  // settled again with the recomputed normaliser when within that margin)
  const double u = u_draw;
  {
    double local[kPer];
    double s = 0.0;
    for (int q = 0; q < kPer; ++q) {
      const int i = tid * kPer + q;
      s += i < n ? S.cand_p[GS_CK(i, GS_LEN(S.cand_p))] / total : 0.0;
      local[q] = s;
    }
    double ctotal;
    const double base = block_scan_f64(s, S.wtmp, &ctotal) - s;
    double dmargin = kNearTie * ctotal;
    if (full_mass) {
      ctotal = 1.0;
      dmargin = margin + full_mass_rel + kNearTie;
    }
    const double cursor = u * ctotal;
    uint32_t my_first = 0xFFFFFFFFu;
    bool my_near = false;
    for (int q = kPer - 1; q >= 0; --q) {
      const int i = tid * kPer + q;
      if (i >= n) continue;
      const double pre = base + local[q];
      if (pre >= cursor) my_first = (uint32_t)i;
      const double d = pre >= cursor ? pre - cursor : cursor - pre;
      if (d < dmargin) my_near = true;
      // ranked candidates that end before the pool does settle the draw only
      // when their sum passes the cursor by twice the margin
      if (i == n - 1 && pre_cut && !(pre >= cursor + 2.0 * dmargin)) S.short_sum = 1u;
    }
    my_first = wave_min_u32(my_first);
    const bool wave_near = __ballot(my_near) != 0;
    if (lane == 0) {
      if (my_first != 0xFFFFFFFFu) atomicMin(&S.first_idx, my_first);
      if (wave_near) atomicOr(&S.route_exact, 8u);
    }
    __syncthreads();
    if (full_mass && !constrained && !pre_cut && (S.route_exact == 8u || S.first_idx == 0xFFFFFFFFu)) {
      // a full-vocabulary draw within the scan normaliser's margin or past
      // the region: the deep draw takes it from the region's candidates
      if (tid == 0) {
        S.deep_m = M;
        S.deep_u = u;
        S.deep_thr = thr;
        S.deep_floor = region_floor;
        S.deep_n = (uint32_t)n;
        S.deep_margin = full_mass_rel + kNearTie;
      }
      return kDeepRequest;
    }
    if (S.route_exact || S.first_idx == 0xFFFFFFFFu || S.short_sum) {
      // a near tie, or a full-vocabulary draw past the ranked candidates
      return kExactRequest | (S.route_exact ? GS_FLAG_NEAR_TIE : 0u);
    }
    const uint32_t i = S.first_idx;
    if (i >= (uint32_t)n) return kExactRequest | GS_FLAG_INDEX_CHECK;
    if (tid == 0) write_result(a, row, (int32_t)S.cand_id[GS_CK(i, GS_LEN(S.cand_id))], tie_report, S.cand_p[GS_CK(i, GS_LEN(S.cand_p))] / total);
    return 0;
  }
}

// Bin of a value v (l/T, or a special's penalised value) in the deep draw's
// tail histogram: kDeepBins bins of kDeepSpan / kDeepBins below vf, the
// region floor's value, bin 0 the highest, values further down in the last.
// A non-increasing function of v, so the bins are contiguous runs of the
// reference's sorted list.
// (vfc = vf kDeepBins / kDeepSpan: z = (vf - v) kDeepBins / kDeepSpan in one fma)
__device__ __forceinline__ double deep_z(double v, double vfc) {
  return __builtin_fma(v, -((double)kDeepBins / kDeepSpan), vfc);
}
__device__ __forceinline__ int deep_bin(double v, double vfc) {
  const double z = deep_z(v, vfc);
  return z < (double)(kDeepBins - 1) ? (int)z : kDeepBins - 1;
}
// A value's term relative to its bin's centre c_b = vf - (b + 1/2) w, w =
// kDeepSpan / kDeepBins: e^(v - c_b) = e^x with x = (b + 1/2 - z) w (b w and
// (b + 1/2) w are exact, so x is z w rounded once from there), |x| <=
// w / 2 (up to z's rounding, 1e-12 of a bin), by its degree-4 Taylor
// polynomial (remainder below 3e-14), in units of 2^-40 rounded to nearest
// (4.6e-13 relative): every term of a bin is about 2^40 units, and a bin of
// at most 2^21 + kSpecialCap of them sums below 2^62. The bin's mass is then
// its units times 2^-40 e^(c_b - M). For b < kDeepBins - 1 only.
__device__ __forceinline__ uint64_t deep_units(double z, int b) {
  constexpr double w = kDeepSpan / kDeepBins;
  const double x = __builtin_fma(-z, w, __builtin_fma((double)b, w, 0.5 * w));
  double p = __builtin_fma(x, 1.0 / 24.0, 1.0 / 6.0);
  p = __builtin_fma(x, p, 0.5);
  p = __builtin_fma(x, p, 1.0);
  p = __builtin_fma(x, p, 1.0);
  // p 2^40 < 2^52: adding 2^52 leaves the rounded integer in the mantissa field
  return __builtin_bit_cast(uint64_t, __builtin_fma(p, 0x1p40, 0x1p52)) & ((1ull << 52) - 1);
}
// a term of the last bin (values kDeepSpan or more below the floor): the
// quartic table exponential of v - M (1e-15 relative, the argument's rounding
// 2e-14), zero below e^-60 of the maximum
__device__ __forceinline__ double deep_term(double v, double M, const double* tab) {
  const double y = (v - M) * GS_256_LOG2E;
  return y > kSkipY ? exp2_256_tight(y, tab) : 0.0;
}
// adds value v's term to the histogram (mass) or to the last bin's sum
// (*tail); negate: subtracts it
__device__ __forceinline__ void deep_add(double v, double vfc, double M, const double* tab, uint64_t* mass,
                                         double* tail, bool negate) {
  const double z = deep_z(v, vfc);
  if (z < (double)(kDeepBins - 1)) {
    const int b = (int)z;
    const uint64_t n = deep_units(z, b);
    atomicAdd(&mass[GS_CK(b, kFinishCap)], negate ? 0ull - n : n);
  } else {
    const double t = deep_term(v, M, tab);
    *tail += negate ? -t : t;
  }
}

// Slot of id in the LDS hash set of the row's special ids (-1: absent).
__device__ __forceinline__ bool deep_is_special(const uint32_t* set, uint32_t id) {
  uint32_t h = hash_id(id) & (kHashSize - 1);
  for (int probe = 0; probe < kHashSize; ++probe) {
    const uint32_t x = set[h];
    if (x == id) return true;
    if (x == 0xFFFFFFFFu) return false;
    h = (h + 1) & (kHashSize - 1);
  }
  return false;
}

// The deep draw's tail histogram: every finite logit below the region floor
// (l <= l_below) adds its term to its bin (LDS atomics on integers, so the sums do not
// depend on their order), or to the returned per-thread sum of the last bin;
// specials are corrected by the caller. The whole block calls it.
__device__ __noinline__ double deep_histogram(const SampleArgs& a, int64_t row, double cap, double T, double rT,
                                              double M, float l_below, double vfc, uint64_t* mass,
                                              const double* tab) {
  double tail = 0.0;
  visit_row<4>(a, row, cap, [&](float l, uint32_t) {
    if (!(l > -__builtin_inff() && l <= l_below)) return;
    deep_add(div_by_temperature((double)l, T, rT), vfc, M, tab, mass, &tail, false);
  });
  return tail;
}

// The deep draw's gather, first step: every logit in [l_lo, l_hi] (a float
// range below the region floor that holds the wanted bins' logits with room
// to spare), as (float bits << 32 | id), appended to stage
// from *counter (at most kFinishCap kept; one LDS atomic per wave and
// logit position). The exact test runs on the few staged entries only. The
// whole block calls it.
__device__ __noinline__ void deep_stage(const SampleArgs& a, int64_t row, double cap, float l_lo, float l_hi,
                                        uint64_t* stage, uint32_t* counter) {
  const int lane = threadIdx.x & 63;
  visit_row<4, true>(a, row, cap, [&](float l, uint32_t id) {
    const bool pass = l >= l_lo && l <= l_hi;
    const uint64_t m = __ballot(pass);
    if (m == 0) return;
    const int leader = __builtin_ctzll(m);
    uint32_t base = 0;
    if (lane == leader) base = atomicAdd(counter, (uint32_t)__popcll(m));
    base = (uint32_t)__shfl((int)base, leader, 64);
    const uint32_t pos = base + (uint32_t)__popcll(m & ((1ull << lane) - 1ull));
    if (pass && pos < (uint32_t)kFinishCap) stage[GS_CK(pos, kFinishCap)] = ((uint64_t)__builtin_bit_cast(uint32_t, l) << 32) | id;
  }, l_lo, l_hi);
}

// Adds id to the LDS hash set of the row's special ids (kHashSize slots, at
// most kSpecialCap ids, so a free slot is always found).
__device__ __forceinline__ void deep_set_insert(uint32_t* set, uint32_t id) {
  uint32_t h = hash_id(id) & (kHashSize - 1);
  for (int probe = 0; probe < kHashSize; ++probe) {
    const uint32_t prev = atomicCAS(&set[h], 0xFFFFFFFFu, id);
    if (prev == 0xFFFFFFFFu || prev == id) return;
    h = (h + 1) & (kHashSize - 1);
  }
}

// The deep draw's LDS set-up, with the row's specials in sp_id[0..n_sp): the
// hash set of their ids (hash_counts), the exponential's table, the gather
// counters, and the mass histogram (sorted) zeroed unless it is loaded.
__device__ __noinline__ void deep_setup(Shared& S, int n_sp, bool zero_mass) {
  const int tid = threadIdx.x;
  for (int b = tid; b < kDeepBins; b += kFinishThreads) {
    if (zero_mass) S.sorted[GS_CK(b, GS_LEN(S.sorted))] = 0ull;
    S.hash_counts[GS_CK(b, GS_LEN(S.hash_counts))] = 0xFFFFFFFFu;
  }
  if (tid < 256) S.tab[GS_CK(tid, GS_LEN(S.tab))] = c_exp2_256[tid];
  if (tid == 0) {
    S.deep_count = 0;
    S.deep_final = 0;
  }
  __syncthreads();
  for (int i = tid; i < n_sp; i += kFinishThreads) deep_set_insert(S.hash_counts, S.sp_id[GS_CK(i, GS_LEN(S.sp_id))]);
  __syncthreads();
}

// The deep draw's inputs hold: the region floor at or below the row's
// largest value (every term below the floor at most 1, so the fixed-point
// sums stay below 2^22; a floor above it is left to the exact path) and a
// temperature div_by_temperature's range covers.
__device__ __forceinline__ bool deep_inputs_ok(const Shared& S, double T) {
  const double vf = (double)key_f32(S.deep_thr) / T;
  return vf <= S.deep_m && T >= 0x1p-20 && T <= 0x1p20;
}

// The deep draw's masses: the region's (over cand_p[0..n_reg)) into
// *r_total, and after[b] (over the histogram in sorted, in place) the mass of
// the region and of bins 0 .. b (a bin's mass: units x 2^-40 x e^(c_b - M),
// the last bin tail_mass). Returns the normaliser. The region's terms (in
// (0, 1], in an order atomics chose) are summed as integers in units of
// 2^-50 (under 4096 2^-51 < 2e-12 off, and the normaliser is at least 1);
// the bins, whose order is fixed, in binary64 (each thread's kPer
// consecutive bins in order, then block_scan_f64's waves in thread order),
// within 32 additions' rounding (under 4e-15 relative). Every run and both
// the single-workgroup and the many-workgroup draws get the same values,
// within the 2^-38 the walk's margin allows for the histogram. The whole
// block calls it.
__device__ __noinline__ double deep_prefix_masses(Shared& S, int n_reg, double tail_mass, double vf, double M,
                                                  double* r_total) {
  const int tid = threadIdx.x;
  constexpr int kPer = kFinishCap / kFinishThreads;  // region entries per thread (and bins)
  static_assert(kDeepBins == kFinishCap, "kPer bins per thread");
  const uint64_t* mass = S.sorted;
  uint64_t r = 0ull;
  for (int i = tid; i < n_reg; i += kFinishThreads) r += to_units(S.cand_p[GS_CK(i, GS_LEN(S.cand_p))], 1.0);
  const double r_tot = (double)block_sum_u64(r, (uint64_t*)S.wsum) / kUnitScale;
  *r_total = r_tot;
  double f[kPer];
  double sum = 0.0;
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    const int b = tid * kPer + q;
    double m = tail_mass;
    if (b < kDeepBins - 1) {
      // e^(c_b - M), c_b = vf - (b + 1/2) w
      const double y = __builtin_fma(-(b + 0.5), kDeepSpan / kDeepBins, vf - M) * GS_256_LOG2E;
      m = (double)mass[GS_CK(b, kFinishCap)] * 0x1p-40 * exp2_256_tight(y, S.tab);
    }
    sum += m;
    f[q] = sum;
  }
  double t;
  // (block_scan_f64's barriers also order every read of mass[] before after[] overwrites it)
  const double base = r_tot + (block_scan_f64(sum, S.wtmp, &t) - sum);
  double* after = (double*)S.sorted;
#pragma unroll
  for (int q = 0; q < kPer; ++q) after[GS_CK(tid * kPer + q, kFinishCap)] = base + f[q];
  return r_tot + t;
}

// What pass 1 leaves (the mass histogram in sorted, each thread's last-bin
// sum in `tail`) is completed and used: the specials go out of the
// histogram with their raw values and in with their penalised ones, the
// normaliser and every bin's prefix mass are summed in binary64 in a fixed
// order, and the region is walked with them. Returns 0 with the result written,
// kExactRequest | flags, or kDeepPass2 with S.plan holding the bins the
// cursor falls in and the logit range to gather.
constexpr uint32_t kDeepPass2 = 1u << 27;
__device__ __noinline__ uint32_t deep_mid(const SampleArgs& a, Shared& S, int64_t row, int n_sp, double tail) {
  const int tid = threadIdx.x, lane = tid & 63;
  const gs_row_config cfg = a.configs[row];
  const double T = cfg.temperature, rT = 1.0 / T;
  const double M = S.deep_m, u = S.deep_u;
  const uint32_t thr = S.deep_thr;
  const int n_reg = (int)S.deep_n;
  const double vf = (double)key_f32(thr) / T;  // the region floor's value
  const double vfc = vf * ((double)kDeepBins / kDeepSpan);
  // the largest float below the floor's logit: l <= l_below iff f32_key(l) < thr
  // (NaN aside; -0 and +0 share a key, and the float below both is -2^-149)
  const float l_below = key_f32(thr - 1u);
  uint64_t* mass = S.sorted;  // [kDeepBins - 1] terms in units of 2^-40 e^(c_b - M)
  // specials: out with their raw values (where pass 1 counted them; the
  // same units, so exactly), in with their penalised ones below the floor
  for (int i = tid; i < n_sp; i += kFinishThreads) {
    const uint32_t id = S.sp_id[GS_CK(i, GS_LEN(S.sp_id))];
    float l = load_logit(a, row, id);
    if (cfg.softcap > 0) l = softcap_call(l, cfg.softcap);
    if (l > -__builtin_inff() && f32_key(l) < thr) {
      deep_add(div_by_temperature((double)l, T, rT), vfc, M, S.tab, mass, &tail, true);
    }
    const double vs = key_f64(S.sp_key[GS_CK(i, GS_LEN(S.sp_key))]);
    if (S.sp_key[GS_CK(i, GS_LEN(S.sp_key))] < S.deep_floor && vs > -__builtin_inf()) deep_add(vs, vfc, M, S.tab, mass, &tail, false);
  }
  double tail_mass;
  block_scan_f64(tail, S.wtmp, &tail_mass);  // the last bin's mass (a fixed order)
  __syncthreads();
  // ---- the region's mass, and the bins' prefix masses
  constexpr int kPer = kFinishCap / kFinishThreads;  // region entries per thread (and bins)
  double r_total;
  const double total = deep_prefix_masses(S, n_reg, tail_mass, vf, M, &r_total);
  const double* after = (const double*)S.sorted;
  if (!(total < __builtin_inf()) || !(total > 0)) return kExactRequest | 0u;
  const double target = u * total;  // the cursor, in units of e
  // the decision margin: the reference's own rounding, the near-tie report
  // and the histogram (terms within 5e-13 relative, the bin masses' and
  // the binary64 sums' rounding)
  const double mrg = (S.deep_margin + 0x1p-38) * total;
  // ---- the region with the recomputed normaliser
  if (tid == 0) { S.first_idx = 0xFFFFFFFFu; S.route_exact = 0; }
  {
    double local[kPer];
    double sum = 0.0, r_mass;
#pragma unroll
    for (int q = 0; q < kPer; ++q) {
      const int i = tid * kPer + q;
      sum += i < n_reg ? S.cand_p[GS_CK(i, GS_LEN(S.cand_p))] : 0.0;
      local[q] = sum;
    }
    const double r_base = block_scan_f64(sum, S.wtmp, &r_mass) - sum;
    uint32_t first = 0xFFFFFFFFu;
    bool near = false;
#pragma unroll
    for (int q = kPer - 1; q >= 0; --q) {
      const int i = tid * kPer + q;
      if (i >= n_reg) continue;
      const double pre = r_base + local[q];
      if (pre >= target) first = (uint32_t)i;
      if ((pre >= target ? pre - target : target - pre) < mrg) near = true;
    }
    first = wave_min_u32(first);
    const bool wn = __ballot(near) != 0;
    if (lane == 0) {
      if (first != 0xFFFFFFFFu) atomicMin(&S.first_idx, first);
      if (wn) atomicOr(&S.route_exact, 1u);
    }
  }
  __syncthreads();
  // every wave reads the walk's outcome before any wave's bin search below
  // writes first_idx again (without this barrier a fast wave's bin index
  // could be read here as a region index)
  const bool walk_near = S.route_exact != 0;
  const uint32_t walk_first = S.first_idx;
  __syncthreads();
  if (walk_near) return kExactRequest | GS_FLAG_NEAR_TIE;
  if (walk_first != 0xFFFFFFFFu) {
    if (walk_first >= (uint32_t)n_reg) return kExactRequest | GS_FLAG_INDEX_CHECK;
    if (tid == 0) write_result(a, row, (int32_t)S.cand_id[GS_CK(walk_first, GS_LEN(S.cand_id))], 0u, S.cand_p[GS_CK(walk_first, GS_LEN(S.cand_p))] / total);
    return 0;
  }
  // ---- the bin the cursor falls in, and a neighbour where a boundary lies
  // within the margin (first_idx is still 0xFFFFFFFF: the walk found none)
  {
    uint32_t first = 0xFFFFFFFFu;
#pragma unroll
    for (int q = kPer - 1; q >= 0; --q) {
      if (after[GS_CK(tid * kPer + q, kFinishCap)] >= target) first = (uint32_t)(tid * kPer + q);
    }
    first = wave_min_u32(first);
    if (lane == 0 && first != 0xFFFFFFFFu) atomicMin(&S.first_idx, first);
  }
  __syncthreads();
  const int bc = (int)S.first_idx;
  if (bc < 0 || bc >= kDeepBins - 1) return kExactRequest | 0u;  // past the bins' span
  const int b_hi = after[GS_CK(bc, kFinishCap)] < target + mrg ? bc + 1 : bc;
  // bin bc - 1 taken in too when the mass before bc lies within the margin
  const bool take_prev = bc > 0 && after[GS_CK(bc - 1, kFinishCap)] >= target - mrg;
  const int b_lo = take_prev ? bc - 1 : bc;
  const double pre_before = b_lo > 0 ? after[GS_CK(b_lo - 1, kFinishCap)] : r_total;
  // the walk below starts after pre_before: the cursor must lie clearly past it
  if (pre_before >= target - mrg) return kExactRequest | GS_FLAG_NEAR_TIE;
  if (b_hi >= kDeepBins - 1) return kExactRequest | 0u;
  // the float range of (capped) logits whose values can fall in bins b_lo ..
  // b_hi: v in [vf - (b_hi + 1) w, vf - b_lo w] up to rounding, times T,
  // widened by 1e-6 relative (more than rounding the bounds to float moves them)
  double l_hi = (vf - b_lo * (kDeepSpan / kDeepBins)) * T;
  double l_lo = (vf - (b_hi + 1) * (kDeepSpan / kDeepBins)) * T;
  l_hi += 1e-6 * (1.0 + __builtin_fabs(l_hi));
  l_lo -= 1e-6 * (1.0 + __builtin_fabs(l_lo));
  __syncthreads();  // every read of after[] done before the gather reuses the array
  if (tid == 0) {
    S.plan.total = total;
    S.plan.target = target;
    S.plan.mrg = mrg;
    S.plan.pre_before = pre_before;
    S.plan.l_lo = (float)l_lo;
    S.plan.l_top = (float)l_hi < l_below ? (float)l_hi : l_below;
    S.plan.b_lo = b_lo;
    S.plan.b_hi = b_hi;
    S.deep_final = 0;
  }
  __syncthreads();
  return kDeepPass2;
}

// The walk of a cursor over n candidates left unsorted, without sorting
// them all. Candidate i < n_list is the non-special list entry list[i]
// (value l / T as the reference computes it), candidate n_list + j the
// special keys[j] (a value key) / ids[j]. The reference walks them in
// (value desc, id asc) order, adding their terms e^(v - M) to a prefix that
// starts at p0, and takes the first whose prefix reaches target
// (sampling.ts:58-64). Here a 256-bin histogram linear in the value below
// the largest (bin(v) = floor((v_hi - v) 256 / (v_hi - v_lo)), a
// non-increasing function of v, so each bin is a run of the sorted order),
// holding each bin's approximate mass (binary32 terms relative to the
// largest, in units of 2^-40, added as integers), names the bin the
// cursor falls in; the terms of the bins above it are summed as integers in
// units of 2^-50 of the largest term (n 2^-51 of it at most, inside mrg, and
// the same sum in every run: the candidates' order in LDS came from
// atomics); and only that bin's entries, when at most kCountRank, are ranked
// (by counting; the ids are distinct) and walked with the exact terms
// (js_exp, as the sorted walk computes them). Returns 0 with the
// candidate's id and term in *hit_id / *hit_term, 1 when a prefix lies
// within mrg of the target, 2 when the approximate masses named the wrong
// bin or the bin holds more than kCountRank entries: the caller then goes
// the sorted way. Scratch: bmass (256 words), sel (4), wtmp (2 kWaves),
// kminmax (2) and cscratch (5 kCountRank 32-bit words). The whole block
// calls it.
__device__ __noinline__ uint32_t walk_cursor_by_bins(const uint64_t* list, int n_list, double T, const uint64_t* keys,
                                                     const uint32_t* ids, int n, double M, double range_lo,
                                                     double p0, double target, double mrg, uint64_t* bmass,
                                                     uint32_t* sel, double* wtmp, uint64_t* kminmax,
                                                     uint32_t* cscratch, uint32_t* hit_id, double* hit_term) {
  const int tid = threadIdx.x, lane = tid & 63;
  // l / T as the reference rounds it, in three operations where the
  // quotient's conditions hold
  const bool fast_div = T >= 0x1p-20 && T <= 0x1p20;
  const double rT = 1.0 / T;
  auto get = [&](int i, uint64_t* k, uint32_t* id) {
    if (i < n_list) {
      const uint64_t e = list[GS_CK(i, kFinishCap)];
      const double l = (double)key_f32(entry_key(e));
      *k = f64_key(fast_div ? div_by_temperature(l, T, rT) : l / T);
      *id = entry_id(e);
    } else {
      *k = keys[GS_CK(i - n_list, kFinishCap)];
      *id = ids[GS_CK(i - n_list, kHashSize)];
    }
  };
  if (tid < 256) bmass[tid] = 0ull;
  if (tid == 0) { kminmax[0] = 0ull; kminmax[1] = 0ull; sel[1] = 0u; sel[2] = 0xFFFFFFFFu; sel[3] = 0u; }
  __syncthreads();
  // the value range: [range_lo, M] when the caller knows a bound (range_lo
  // < M), else the candidates' own (the minimum key as the maximum of the
  // complements)
  double v_hi = M, v_lo = range_lo;
  if (!(range_lo < M)) {
    uint64_t kmax = 0ull, kneg = 0ull;
    for (int i = tid; i < n; i += kFinishThreads) {
      uint64_t k;
      uint32_t id;
      get(i, &k, &id);
      kmax = k > kmax ? k : kmax;
      kneg = ~k > kneg ? ~k : kneg;
    }
    kmax = wave_max_u64(kmax);
    kneg = wave_max_u64(kneg);
    if (lane == 0) {
      atomicMax((unsigned long long*)&kminmax[0], (unsigned long long)kmax);
      atomicMax((unsigned long long*)&kminmax[1], (unsigned long long)kneg);
    }
    __syncthreads();
    v_hi = key_f64(kminmax[0]);
    v_lo = key_f64(~kminmax[1]);
  }
  const double bscale = v_hi > v_lo ? 256.0 / (v_hi - v_lo) : 0.0;
  auto bin_of = [&](double v) -> uint32_t {
    const double z = (v_hi - v) * bscale;
    return z < 255.0 ? (uint32_t)z : 255u;
  };
  const double e_top = gsm::js_exp(v_hi - M);  // the largest term
  // approximate masses: binary32 exponentials relative to the largest term
  // (within 1e-6 relative), in units of 2^-40 of it
  for (int i = tid; i < n; i += kFinishThreads) {
    uint64_t k;
    uint32_t id;
    get(i, &k, &id);
    const double v = key_f64(k);
    atomicAdd((unsigned long long*)&bmass[GS_CK(bin_of(v), 256)], mass_units((float)(v - v_hi)));
  }
  __syncthreads();
  if (tid < 64) {
    // lane l holds bins 4l .. 4l+3, highest values first
    double m[4], ms = 0.0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      m[q] = (double)bmass[4 * lane + q] * 0x1p-40 * e_top;
      ms += m[q];
    }
    const double incl = wave_scan_f64(ms);
    const uint64_t hit_m = __ballot(p0 + incl >= target);
    uint32_t b = 0xFFFFFFFFu;
    if (hit_m) {
      const int f = __ffsll((unsigned long long)hit_m) - 1;
      if (lane == f) {
        double cum = p0 + incl - ms;
        int q = 0;
        while (q < 3 && cum + m[q] < target) { cum += m[q]; ++q; }
        b = (uint32_t)(4 * lane + q);
      }
      b = readlane_u32(b, f);
    }
    if (lane == 0) sel[0] = b;
  }
  __syncthreads();
  const uint32_t bc = sel[0];
  if (bc == 0xFFFFFFFFu) return 2u;
  // the exact masses above the bin and in it, and the bin's entries compacted
  uint64_t* ck = (uint64_t*)cscratch;                 // [kCountRank]
  uint32_t* cid = cscratch + 2 * kCountRank;          // [kCountRank]
  double* ct = (double*)(cscratch + 3 * kCountRank);  // [kCountRank]
  const double inv_top = 1.0 / e_top;
  uint64_t above = 0ull, inbin = 0ull;
  for (int i = tid; i < n; i += kFinishThreads) {
    uint64_t k;
    uint32_t id;
    get(i, &k, &id);
    const double v = key_f64(k);
    const uint32_t b = bin_of(v);
    if (b > bc) continue;
    const double t = gsm::js_exp(v - M);
    if (b < bc) {
      above += to_units(t, inv_top);
    } else {
      inbin += to_units(t, inv_top);
      const uint32_t pos = atomicAdd(&sel[1], 1u);
      if (pos < (uint32_t)kCountRank) {
        ck[pos] = k;
        cid[pos] = id;
        ct[pos] = t;
      }
    }
  }
  uint64_t above_u, inbin_u;
  block_sum2_u64(above, inbin, (uint64_t*)wtmp, &above_u, &inbin_u);
  const double above_all = (double)above_u / kUnitScale * e_top;
  const double inbin_all = (double)inbin_u / kUnitScale * e_top;
  const int c = (int)sel[1];
  const double base = p0 + above_all;
  if ((base >= target ? base - target : target - base) < mrg) return 1u;
  if (base >= target || base + inbin_all < target || c > kCountRank) return 2u;
  // rank the bin's entries by counting, then walk them in order
  uint64_t k = 0ull;
  uint32_t id = 0u;
  double t = 0.0;
  int rank = 0;
  if (tid < c) {
    k = ck[tid];
    id = cid[tid];
    t = ct[tid];
#pragma unroll 8
    for (int j = 0; j < c; ++j) rank += ranks_before(ck[j], cid[j], k, id) ? 1 : 0;
  }
  __syncthreads();
  if (tid < c) {
    ck[rank] = k;
    cid[rank] = id;
    ct[rank] = t;
  }
  __syncthreads();
  const double tv = tid < c ? ct[tid] : 0.0;
  double tot;
  const double pre = base + block_scan_f64(tv, wtmp, &tot);
  const uint32_t mine = tid < c && pre >= target ? (uint32_t)tid : 0xFFFFFFFFu;
  const uint32_t wfirst = wave_min_u32(mine);
  const bool wnear = __ballot(tid < c && (pre >= target ? pre - target : target - pre) < mrg) != 0;
  if (lane == 0) {
    if (wfirst != 0xFFFFFFFFu) atomicMin(&sel[2], wfirst);
    if (wnear) atomicOr(&sel[3], 1u);
  }
  __syncthreads();
  const bool any_near = sel[3] != 0u;
  const uint32_t f = sel[2];
  if (!any_near && f < (uint32_t)c) {
    *hit_id = cid[f];
    *hit_term = ct[f];
  }
  __syncthreads();  // every thread has read sel[] and the compacted entries
  if (any_near) return 1u;
  if (f >= (uint32_t)c) return 2u;
  return 0u;
}

// Pass 2's staged logits (in cand_p as (float bits << 32 | id), deep_count of
// them) are tested against the plan's bins exactly, joined by the specials
// whose penalised values fall there, sorted (value desc, id asc) and walked
// with exact exponentials from the mass before the bins. Returns as deep_mid.
__device__ __noinline__ uint32_t deep_final(const SampleArgs& a, Shared& S, int64_t row, int n_sp) {
  const int tid = threadIdx.x, lane = tid & 63;
  const double T = a.configs[row].temperature, rT = 1.0 / T;
  const double M = S.deep_m;
  const double vfc = (double)key_f32(S.deep_thr) / T * ((double)kDeepBins / kDeepSpan);
  const DeepPlan plan = S.plan;
  constexpr int kPer = kFinishCap / kFinishThreads;
  if (S.deep_count > (uint32_t)kFinishCap) return kExactRequest | 0u;  // a crowd of equal values
  const uint64_t* stage = (const uint64_t*)S.cand_p;
  uint64_t* gkey = S.sorted;
  uint32_t* gid = S.hash_ids;
  const uint32_t* spset = S.hash_counts;
  const int n_s = (int)S.deep_count;
  auto gather = [&](double v, uint32_t id) {
    const int b = deep_bin(v, vfc);
    if (b < plan.b_lo || b > plan.b_hi) return;
    const uint32_t pos = atomicAdd(&S.deep_final, 1u);
    if (pos < (uint32_t)kFinishCap) { gkey[GS_CK(pos, kFinishCap)] = f64_key(v); gid[GS_CK(pos, kHashSize)] = id; }
  };
  for (int i = tid; i < n_s; i += kFinishThreads) {
    const uint64_t e = stage[GS_CK(i, kFinishCap)];
    const uint32_t id = (uint32_t)e;
    if (!deep_is_special(spset, id)) {
      gather(div_by_temperature((double)__builtin_bit_cast(float, (uint32_t)(e >> 32)), T, rT), id);
    }
  }
  for (int i = tid; i < n_sp; i += kFinishThreads) {
    const double vs = key_f64(S.sp_key[GS_CK(i, GS_LEN(S.sp_key))]);
    if (S.sp_key[GS_CK(i, GS_LEN(S.sp_key))] < S.deep_floor && vs > -__builtin_inf()) gather(vs, S.sp_id[GS_CK(i, GS_LEN(S.sp_id))]);
  }
  __syncthreads();
  const int n_g = (int)S.deep_final;
  if (n_g > kFinishCap || n_g == 0) return kExactRequest | 0u;
  // ---- sort them (value desc, id asc) and walk them with exact exponentials
  if (n_g <= kCountSmall) {
    // a few: each finds its place by counting the entries ranked before it
    // (the ids are distinct)
    uint64_t k = 0;
    uint32_t id = 0;
    int rank = 0;
    if (tid < n_g) {
      k = gkey[GS_CK(tid, kFinishCap)];
      id = gid[GS_CK(tid, kHashSize)];
#pragma unroll 8
      for (int j = 0; j < n_g; ++j) rank += ranks_before(gkey[GS_CK(j, kFinishCap)], gid[GS_CK(j, kHashSize)], k, id) ? 1 : 0;
    }
    __syncthreads();
    if (tid < n_g) {
      gkey[GS_CK(rank, kFinishCap)] = k;
      gid[GS_CK(rank, kHashSize)] = id;
    }
    __syncthreads();
  } else {
    // more: walk only the histogram bin the cursor falls in (the gathered
    // bins' entries are dense in value), else sort them all
    uint32_t hit_id = 0;
    double hit_term = 0.0;
    const uint32_t w = walk_cursor_by_bins(nullptr, 0, T, gkey, gid, n_g, M, M, plan.pre_before, plan.target,
                                           plan.mrg, (uint64_t*)S.tab, (uint32_t*)(S.top + 2), S.wsum2, S.top,
                                           S.hash_counts, &hit_id, &hit_term);
    if (w == 1u) return kExactRequest | GS_FLAG_NEAR_TIE;
    if (w == 0u) {
      if (tid == 0) write_result(a, row, (int32_t)hit_id, 0u, hit_term / plan.total);
      return 0;
    }
    const int m2 = pow2_at_least(n_g);
    for (int i = n_g + tid; i < m2; i += kFinishThreads) { gkey[GS_CK(i, kFinishCap)] = 0; gid[GS_CK(i, kHashSize)] = 0xFFFFFFFFu; }
    __syncthreads();
    block_sort_pairs_desc(gkey, gid, m2);
  }
  for (int i = tid; i < n_g; i += kFinishThreads) S.cand_p[GS_CK(i, GS_LEN(S.cand_p))] = gsm::js_exp(key_f64(gkey[GS_CK(i, kFinishCap)]) - M);
  if (tid == 0) { S.first_idx = 0xFFFFFFFFu; S.route_exact = 0; }
  __syncthreads();
  {
    double g_local[kPer];
    double sum = 0.0;
#pragma unroll
    for (int q = 0; q < kPer; ++q) {
      const int i = tid * kPer + q;
      sum += i < n_g ? S.cand_p[GS_CK(i, GS_LEN(S.cand_p))] : 0.0;
      g_local[q] = sum;
    }
    double g_total;
    const double g_base = block_scan_f64(sum, S.wtmp, &g_total) - sum;
    uint32_t first = 0xFFFFFFFFu;
    bool near = false;
#pragma unroll
    for (int q = kPer - 1; q >= 0; --q) {
      const int i = tid * kPer + q;
      if (i >= n_g) continue;
      const double pre = plan.pre_before + g_base + g_local[q];
      if (pre >= plan.target) first = (uint32_t)i;
      if ((pre >= plan.target ? pre - plan.target : plan.target - pre) < plan.mrg) near = true;
    }
    first = wave_min_u32(first);
    const bool wn = __ballot(near) != 0;
    if (lane == 0) {
      if (first != 0xFFFFFFFFu) atomicMin(&S.first_idx, first);
      if (wn) atomicOr(&S.route_exact, 1u);
    }
  }
  __syncthreads();
  if (S.route_exact) return kExactRequest | GS_FLAG_NEAR_TIE;
  const uint32_t first = S.first_idx;
  if (first == 0xFFFFFFFFu) return kExactRequest | 0u;
  if (first >= (uint32_t)n_g) return kExactRequest | GS_FLAG_INDEX_CHECK;
  if (tid == 0) write_result(a, row, (int32_t)gid[GS_CK(first, kHashSize)], 0u, S.cand_p[GS_CK(first, GS_LEN(S.cand_p))] / plan.total);
  return 0;
}

// A full-vocabulary draw (topK 0, topP 1, no min-p or typical-p) whose cursor
// lies past the complete region of the chunk lists, or within the scan
// normaliser's margin of one of its prefix sums (sampling.ts:58-64 over the
// whole sorted list), on the row's own workgroup. finish_row left the
// region's candidates in list order with their exact exponentials (cand_p /
// cand_id, deep_n of them), the row's specials (sp_key / sp_id) and M, u,
// the region floor and the reference's own rounding margin. One pass over the
// row's logits below the floor builds a fixed-point mass histogram over value
// bins (terms within 2^-40 relative), which gives the normaliser and every
// bin's prefix mass to that accuracy; the region is walked again with them;
// failing that, the bins the cursor falls in are gathered, sorted by (value
// desc, id asc), given their exact exponentials and walked. Returns 0 with
// the result written, or kExactRequest | flags. Unconstrained rows only; the
// whole block calls it.
__device__ __noinline__ uint32_t deep_draw(const SampleArgs& a, FinishLds& U) {
  Shared& S = U.fin;
  const int64_t row = blockIdx.x;
  const gs_row_config cfg = a.configs[row];
  const double T = cfg.temperature;
  if (!deep_inputs_ok(S, T)) return kExactRequest | 0u;
  if (S.deep_n > (uint32_t)kFinishCap) return kExactRequest | GS_FLAG_INDEX_CHECK;
  const int n_sp = (int)(S.n_special < (uint32_t)kSpecialCap ? S.n_special : (uint32_t)kSpecialCap);
  const double rT = 1.0 / T;
  const double vfc = (double)key_f32(S.deep_thr) / T * ((double)kDeepBins / kDeepSpan);
  const float l_below = key_f32(S.deep_thr - 1u);
  deep_setup(S, n_sp, true);
  // ---- pass 1: the tail's mass per bin
  const double tail = deep_histogram(a, row, cfg.softcap, T, rT, S.deep_m, l_below, vfc, S.sorted, S.tab);
  __syncthreads();
  const uint32_t r = deep_mid(a, S, row, n_sp, tail);
  if (r != kDeepPass2) return r;
  // ---- pass 2: stage the logits in the bins' float range (in cand_p)
  deep_stage(a, row, cfg.softcap, S.plan.l_lo, S.plan.l_top, (uint64_t*)S.cand_p, &S.deep_count);
  __syncthreads();
  return deep_final(a, S, row, n_sp);
}

// ---- the deep draw over many workgroups
// The finish leaves a deep row's inputs in its DeepRow (the region's
// candidates, the specials, M, u, the floor, the margin, a zeroed histogram)
// and queues it. Four launches follow, each one workgroup per compute unit
// taking items from the queues until they are drained (nothing waits for
// another workgroup; the launch boundaries order every write before the next
// launch's reads):
// - deep1_kernel: pass 1 over a part of a queued row (a run of chunks) into an
//   LDS histogram, added to the row's with 64-bit global atomics (integers:
//   the sums do not depend on the order), and the part's last-bin sum;
// - deep_mid_kernel: per queued row, the histogram and the walk (deep_mid);
//   a row that needs pass 2 is queued again;
// - deep2_kernel: pass 2 over a part of such a row, its logits in the plan's
//   range appended to the row's stage;
// - deep_final_kernel: per such row, deep_final.
// Parts are as many per row as there are compute units per queued row (at
// most one per chunk), so a lone row still spreads over many workgroups.

// The finish workgroup's hand-over of a deep row: 0, or kExactRequest when
// the inputs are out of the deep draw's range (the whole block calls it).
__device__ __noinline__ uint32_t deep_export(const SampleArgs& a, Shared& S) {
  const int tid = threadIdx.x;
  const int64_t row = blockIdx.x;
  if (!deep_inputs_ok(S, a.configs[row].temperature)) return kExactRequest | 0u;
  DeepRow& D = a.deep_rows[row];
  // the region count sizes the copy into the record: one past the record's
  // capacity is never copied (block-uniform: read after the caller's barrier)
  if (S.deep_n > (uint32_t)kFinishCap) return kExactRequest | GS_FLAG_INDEX_CHECK;
  const int n_reg = (int)S.deep_n;
  const int n_sp = (int)(S.n_special < (uint32_t)kSpecialCap ? S.n_special : (uint32_t)kSpecialCap);
  for (int i = tid; i < n_reg; i += kFinishThreads) { D.cand_p[GS_CK(i, GS_LEN(D.cand_p))] = S.cand_p[GS_CK(i, GS_LEN(S.cand_p))]; D.cand_id[GS_CK(i, GS_LEN(D.cand_id))] = S.cand_id[GS_CK(i, GS_LEN(S.cand_id))]; }
  for (int i = tid; i < n_sp; i += kFinishThreads) { D.sp_key[GS_CK(i, GS_LEN(D.sp_key))] = S.sp_key[GS_CK(i, GS_LEN(S.sp_key))]; D.sp_id[GS_CK(i, GS_LEN(D.sp_id))] = S.sp_id[GS_CK(i, GS_LEN(S.sp_id))]; }
  for (int b = tid; b < kDeepBins; b += kFinishThreads) D.hist[GS_CK(b, GS_LEN(D.hist))] = 0ull;
#ifdef GS_CHECKED
  __syncthreads();
  if (GS_CHECK_FAILED()) return kExactRequest | GS_FLAG_INDEX_CHECK;
#endif
  if (tid == 0) {
    D.M = S.deep_m;
    D.u = S.deep_u;
    D.margin = S.deep_margin;
    D.floor = S.deep_floor;
    D.thr = S.deep_thr;
    D.n_reg = (uint32_t)n_reg;
    D.n_sp = (uint32_t)n_sp;
    D.n_stage = 0;
    D.index_check = 0;
    D.index_check2 = 0;
    const uint32_t q = atomicAdd(&a.deep_queue->count1, 1u);
    a.deep_queue->rows[q] = (uint32_t)row;
  }
  return 0;
}

// The logits of ids [i0, i1) of a row (i0 a multiple of 8), softcapped when
// cap > 0, as visit(l, id), two 16-byte pieces per thread in flight; kRanged:
// pieces with no logit in [lo, hi] are skipped after one ballot.
template <bool kRanged, typename F>
__device__ __forceinline__ void visit_range(const SampleArgs& a, int64_t row, double cap, int64_t i0, int64_t i1,
                                            F&& visit, float lo = 0.0f, float hi = 0.0f) {
  const int tid = threadIdx.x;
  int64_t from = i0;
  if (cap > 0) {
    from = i1;
#pragma unroll 1
    for (int64_t i = i0 + tid; i < i1; i += kFinishThreads) visit(softcap_call(load_logit(a, row, i), cap), (uint32_t)i);
  } else if (a.vector_ok) {
    const bool bf16 = a.dtype == GS_BF16;
    const int per = bf16 ? 8 : 4;
    const int64_t v0 = i0 / per, v1 = i1 / per;
    const uint4* base = (const uint4*)((const char*)a.logits + row * a.row_stride * (bf16 ? 2 : 4));
    constexpr int kB = 2;
    for (int64_t vb = v0 + tid; vb < v1; vb += (int64_t)kB * kFinishThreads) {
      uint4 w[kB];
#pragma unroll
      for (int k = 0; k < kB; ++k) {
        const int64_t vi = vb + (int64_t)k * kFinishThreads;
        w[k] = vi < v1 ? load_nt16(base + vi) : make_uint4(0u, 0u, 0u, 0u);
      }
#pragma unroll
      for (int k = 0; k < kB; ++k) {
        const int64_t vi = vb + (int64_t)k * kFinishThreads;
        const uint32_t q[4] = {w[k].x, w[k].y, w[k].z, w[k].w};
        if (kRanged) {
          bool hit = false;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float x0 = __builtin_bit_cast(float, bf16 ? q[j] << 16 : q[j]);
            const float x1 = __builtin_bit_cast(float, q[j] & 0xFFFF0000u);
            hit |= vi < v1 && x0 >= lo && x0 <= hi;
            if (bf16) hit |= vi < v1 && x1 >= lo && x1 <= hi;
          }
          if (!__ballot(hit)) continue;
        }
        if (vi >= v1) continue;
        const uint32_t id0 = (uint32_t)(vi * per);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (bf16) {
            visit(__builtin_bit_cast(float, q[j] << 16), id0 + 2 * j);
            visit(__builtin_bit_cast(float, q[j] & 0xFFFF0000u), id0 + 2 * j + 1);
          } else {
            visit(__builtin_bit_cast(float, q[j]), id0 + j);
          }
        }
      }
    }
    from = v1 * per;
  }
  for (int64_t i = from + tid; i < i1; i += kFinishThreads) visit(load_logit(a, row, i), (uint32_t)i);
}

// Parts per queued row when `rows` rows are queued: about one compute unit
// each, at most one per chunk; chunks_per_part is set to cover the row.
__device__ __forceinline__ uint32_t deep_parts(const SampleArgs& a, uint32_t rows, uint32_t* chunks_per_part) {
  const uint32_t nc = (uint32_t)a.n_chunks;
  uint32_t p = rows ? (uint32_t)a.cu_count / rows : 1u;
  p = p < 1u ? 1u : (p > nc ? nc : p);
  const uint32_t cpp = (nc + p - 1u) / p;
  *chunks_per_part = cpp;
  return (nc + cpp - 1u) / cpp;
}

// Takes the next work item (every thread of the block gets it).
__device__ __forceinline__ uint32_t deep_take(Shared& S, uint32_t* next) {
  if (threadIdx.x == 0) S.sel[GS_CK(0, GS_LEN(S.sel))] = atomicAdd(next, 1u);
  __syncthreads();
  const uint32_t item = S.sel[GS_CK(0, GS_LEN(S.sel))];
  __syncthreads();
  return item;
}

// The record's counts lie within its arrays (deep_export writes them so);
// a record that says otherwise goes to the exact path, never into a copy.
__device__ __forceinline__ bool deep_counts_ok(const DeepRow& D) {
  return D.n_reg <= (uint32_t)kFinishCap && D.n_sp <= (uint32_t)kSpecialCap;
}

// The row's inputs back into LDS for deep_mid / deep_final (the whole block).
__device__ __noinline__ void deep_import(const DeepRow& D, Shared& S, bool with_region) {
  const int tid = threadIdx.x;
  const int n_sp = (int)D.n_sp;
  for (int i = tid; i < n_sp; i += kFinishThreads) { S.sp_key[GS_CK(i, GS_LEN(S.sp_key))] = D.sp_key[GS_CK(i, GS_LEN(D.sp_key))]; S.sp_id[GS_CK(i, GS_LEN(S.sp_id))] = D.sp_id[GS_CK(i, GS_LEN(D.sp_id))]; }
  if (with_region) {
    const int n_reg = (int)D.n_reg;
    for (int i = tid; i < n_reg; i += kFinishThreads) { S.cand_p[GS_CK(i, GS_LEN(S.cand_p))] = D.cand_p[GS_CK(i, GS_LEN(D.cand_p))]; S.cand_id[GS_CK(i, GS_LEN(S.cand_id))] = D.cand_id[GS_CK(i, GS_LEN(D.cand_id))]; }
  }
  if (tid == 0) {
    S.deep_m = D.M;
    S.deep_u = D.u;
    S.deep_margin = D.margin;
    S.deep_floor = D.floor;
    S.deep_thr = D.thr;
    S.deep_n = D.n_reg;
  }
  __syncthreads();
}

// Pass 1 over ids [i0, i1) of a queued row: its logits below the region
// floor into an LDS histogram, added to the row's global one, and the part's
// last-bin sum into tail[part] (the whole block calls it).
__device__ __noinline__ void deep1_part(const SampleArgs& a, Shared& S, int64_t row, int part, int64_t i0,
                                        int64_t i1) {
  const int tid = threadIdx.x;
  DeepRow& D = a.deep_rows[row];
  const gs_row_config cfg = a.configs[row];
  const double T = cfg.temperature, rT = 1.0 / T;
  const double M = D.M;
  const uint32_t thr = D.thr;
  const double vfc = (double)key_f32(thr) / T * ((double)kDeepBins / kDeepSpan);
  const float l_below = key_f32(thr - 1u);
  uint64_t* mass = S.sorted;
  GS_CHECK_RESET();
  for (int b = tid; b < kDeepBins; b += kFinishThreads) mass[GS_CK(b, kFinishCap)] = 0ull;
  if (tid < 256) S.tab[GS_CK(tid, GS_LEN(S.tab))] = c_exp2_256[tid];
  __syncthreads();
  double tail = 0.0;
  visit_range<false>(a, row, cfg.softcap, i0, i1, [&](float l, uint32_t) {
    if (!(l > -__builtin_inff() && l <= l_below)) return;
    deep_add(div_by_temperature((double)l, T, rT), vfc, M, S.tab, mass, &tail, false);
  });
  double t_all;
  block_scan_f64(tail, S.wtmp, &t_all);
  __syncthreads();
  for (int b = tid; b < kDeepBins; b += kFinishThreads) {
    const uint64_t m = mass[GS_CK(b, kFinishCap)];
    if (m) atomicAdd((unsigned long long*)&D.hist[GS_CK(b, GS_LEN(D.hist))], (unsigned long long)m);
  }
  if (tid == 0) D.tail[GS_CK(part, GS_LEN(D.tail))] = t_all;
#ifdef GS_CHECKED
  __syncthreads();
  if (GS_CHECK_FAILED() && tid == 0) D.index_check = 1u;
#endif
}

__global__ __launch_bounds__(kFinishThreads) void deep1_kernel(SampleArgs) {
  __shared__ FinishLds U;
  GS_CHECKED_CLEAR(U);
  Shared& S = U.fin;
  // the arguments read where the kernel received them (never copied to the stack)
  const SampleArgs& a = *(const SampleArgs*)__builtin_amdgcn_kernarg_segment_ptr();
  uint32_t cpp;
  const uint32_t parts = deep_parts(a, a.deep_queue->count1, &cpp);
  const uint32_t n_items = a.deep_queue->count1 * parts;
  for (;;) {
    const uint32_t item = deep_take(S, &a.deep_queue->next1);
    if (item >= n_items) break;
    const int64_t row = a.deep_queue->rows[item / parts];
    const int part = (int)(item % parts);
    const int64_t i0 = (int64_t)part * cpp * kChunk;
    const int64_t i1 = i0 + (int64_t)cpp * kChunk < (int64_t)a.vocab ? i0 + (int64_t)cpp * kChunk : (int64_t)a.vocab;
    deep1_part(a, S, row, part, i0, i1);
    __syncthreads();
  }
}

// Per queued row: the histogram and the walk; a row that needs pass 2 is
// queued for it (the whole block calls it).
__device__ __noinline__ uint32_t deep_mid_row(const SampleArgs& a, Shared& S, int64_t row, uint32_t parts) {
  const int tid = threadIdx.x;
  DeepRow& D = a.deep_rows[row];
#ifdef GS_CHECKED
  if (D.index_check) return kExactRequest | GS_FLAG_INDEX_CHECK;
#endif
  if (!deep_counts_ok(D)) return kExactRequest | GS_FLAG_INDEX_CHECK;
  GS_CHECK_RESET();
  deep_import(D, S, true);
  for (int b = tid; b < kDeepBins; b += kFinishThreads) S.sorted[GS_CK(b, GS_LEN(S.sorted))] = D.hist[GS_CK(b, GS_LEN(D.hist))];
  deep_setup(S, (int)D.n_sp, false);
  const double tail = tid < (int)parts ? D.tail[GS_CK(tid, GS_LEN(D.tail))] : 0.0;
  const uint32_t r = deep_mid(a, S, row, (int)D.n_sp, tail);
#ifdef GS_CHECKED
  __syncthreads();
  if (GS_CHECK_FAILED()) return kExactRequest | GS_FLAG_INDEX_CHECK;
#endif
  if (r != kDeepPass2) return r;
  if (tid == 0) {
    D.plan = S.plan;
    const uint32_t q = atomicAdd(&a.deep_queue->count2, 1u);
    a.deep_queue->rows[a.deep_max_rows + q] = (uint32_t)row;
  }
  return 0;
}

__global__ __launch_bounds__(kFinishThreads) void deep_mid_kernel(SampleArgs) {
  __shared__ FinishLds U;
  GS_CHECKED_CLEAR(U);
  Shared& S = U.fin;
  const SampleArgs& a = *(const SampleArgs*)__builtin_amdgcn_kernarg_segment_ptr();
  uint32_t cpp;
  const uint32_t parts = deep_parts(a, a.deep_queue->count1, &cpp);
  const uint32_t n_rows = a.deep_queue->count1;
  for (uint32_t i = blockIdx.x; i < n_rows; i += gridDim.x) {
    const int64_t row = a.deep_queue->rows[i];
    const uint32_t r = deep_mid_row(a, S, row, parts);
    if (r & kExactRequest) to_exact(a, U, row, r & ~kExactRequest);
    __syncthreads();
  }
}

// Pass 2 over ids [i0, i1) of a queued row: its logits in the plan's float
// range into the row's stage (one global atomic per wave and logit position;
// at most kFinishCap kept, all counted). The whole block calls it.
__device__ __noinline__ void deep2_part(const SampleArgs& a, int64_t row, int64_t i0, int64_t i1) {
  const int lane = threadIdx.x & 63;
  DeepRow& D = a.deep_rows[row];
  GS_CHECK_RESET();
#ifdef GS_CHECKED
  __syncthreads();
#endif
  const float l_lo = D.plan.l_lo, l_top = D.plan.l_top;
  visit_range<true>(a, row, a.configs[row].softcap, i0, i1, [&](float l, uint32_t id) {
    const bool pass = l >= l_lo && l <= l_top;
    const uint64_t m = __ballot(pass);
    if (m == 0) return;
    const int leader = __builtin_ctzll(m);
    uint32_t base = 0;
    if (lane == leader) base = atomicAdd(&D.n_stage, (uint32_t)__popcll(m));
    base = (uint32_t)__shfl((int)base, leader, 64);
    const uint32_t pos = base + (uint32_t)__popcll(m & ((1ull << lane) - 1ull));
    if (pass && pos < (uint32_t)kFinishCap) D.stage[GS_CK(pos, GS_LEN(D.stage))] = ((uint64_t)__builtin_bit_cast(uint32_t, l) << 32) | id;
  }, l_lo, l_top);
#ifdef GS_CHECKED
  __syncthreads();
  if (GS_CHECK_FAILED() && threadIdx.x == 0) D.index_check2 = 1u;
#endif
}

__global__ __launch_bounds__(kFinishThreads) void deep2_kernel(SampleArgs) {
  __shared__ FinishLds U;
  GS_CHECKED_CLEAR(U);
  Shared& S = U.fin;
  const SampleArgs& a = *(const SampleArgs*)__builtin_amdgcn_kernarg_segment_ptr();
  uint32_t cpp;
  const uint32_t parts = deep_parts(a, a.deep_queue->count2, &cpp);
  const uint32_t n_items = a.deep_queue->count2 * parts;
  for (;;) {
    const uint32_t item = deep_take(S, &a.deep_queue->next2);
    if (item >= n_items) break;
    const int64_t row = a.deep_queue->rows[a.deep_max_rows + item / parts];
    const int64_t i0 = (int64_t)(item % parts) * cpp * kChunk;
    const int64_t i1 = i0 + (int64_t)cpp * kChunk < (int64_t)a.vocab ? i0 + (int64_t)cpp * kChunk : (int64_t)a.vocab;
    deep2_part(a, row, i0, i1);
    __syncthreads();
  }
}

// Per row queued for pass 2: the exact test, the sort and the walk (the whole
// block calls it).
__device__ __noinline__ uint32_t deep_final_row(const SampleArgs& a, Shared& S, int64_t row) {
  const int tid = threadIdx.x;
  const DeepRow& D = a.deep_rows[row];
#ifdef GS_CHECKED
  if (D.index_check || D.index_check2) return kExactRequest | GS_FLAG_INDEX_CHECK;
#endif
  if (!deep_counts_ok(D)) return kExactRequest | GS_FLAG_INDEX_CHECK;
  GS_CHECK_RESET();
  deep_import(D, S, false);
  deep_setup(S, (int)D.n_sp, false);
  const uint32_t n_stage = D.n_stage;
  const int n_keep = (int)(n_stage < (uint32_t)kFinishCap ? n_stage : (uint32_t)kFinishCap);
  for (int i = tid; i < n_keep; i += kFinishThreads) ((uint64_t*)S.cand_p)[i] = D.stage[GS_CK(i, GS_LEN(D.stage))];
  if (tid == 0) {
    S.plan = D.plan;
    S.deep_count = n_stage;
  }
  __syncthreads();
  const uint32_t r = deep_final(a, S, row, (int)D.n_sp);
#ifdef GS_CHECKED
  __syncthreads();
  if (GS_CHECK_FAILED()) return kExactRequest | GS_FLAG_INDEX_CHECK;
#endif
  return r;
}

__global__ __launch_bounds__(kFinishThreads) void deep_final_kernel(SampleArgs) {
  __shared__ FinishLds U;
  GS_CHECKED_CLEAR(U);
  Shared& S = U.fin;
  const SampleArgs& a = *(const SampleArgs*)__builtin_amdgcn_kernarg_segment_ptr();
  const uint32_t n_rows = a.deep_queue->count2;
  for (uint32_t i = blockIdx.x; i < n_rows; i += gridDim.x) {
    const int64_t row = a.deep_queue->rows[a.deep_max_rows + i];
    const uint32_t r = deep_final_row(a, S, row);
    if (r & kExactRequest) to_exact(a, U, row, r & ~kExactRequest);
    __syncthreads();
  }
}

__global__ __launch_bounds__(kFinishThreads) void finish_kernel(SampleArgs a) {
  __shared__ FinishLds U;
  GS_CHECKED_CLEAR(U);
  GS_CHECK_RESET();
  uint32_t r = finish_row(a, U);
#ifdef GS_CHECKED
  __syncthreads();
  if (GS_CHECK_FAILED()) r = kExactRequest | GS_FLAG_INDEX_CHECK;
#endif
  if (r == kDeepRequest) {
    __syncthreads();
    // calls of their own that read the arguments where the kernel received
    // them, so the kernel's copy never goes to the stack; with deep records
    // the deep kernels take the row from here
    const SampleArgs& ka = *(const SampleArgs*)__builtin_amdgcn_kernarg_segment_ptr();
    r = a.deep_rows ? deep_export(ka, U.fin) : deep_draw(ka, U);
#ifdef GS_CHECKED
    __syncthreads();
    if (GS_CHECK_FAILED()) r = kExactRequest | GS_FLAG_INDEX_CHECK;
#endif
  }
  // the exact path is entered from here only, where nothing else is live
  if (r & kExactRequest) to_exact(a, U, blockIdx.x, r & ~kExactRequest);
}

}  // namespace

void launch_finish(const SampleArgs& a, hipStream_t s, LaunchEvents ev) {
  hipExtLaunchKernelGGL(finish_kernel, dim3(a.rows), dim3(kFinishThreads), 0, s, ev.start, ev.stop, 0, a);
}

void launch_deep(const SampleArgs& a, hipStream_t s, LaunchEvents ev) {
  // one workgroup per compute unit (each holds the finish's LDS), taking items
  // until the queues are drained
  const dim3 grid(a.cu_count), block(kFinishThreads);
  hipExtLaunchKernelGGL(deep1_kernel, grid, block, 0, s, ev.start, nullptr, 0, a);
  hipExtLaunchKernelGGL(deep_mid_kernel, grid, block, 0, s, nullptr, nullptr, 0, a);
  hipExtLaunchKernelGGL(deep2_kernel, grid, block, 0, s, nullptr, nullptr, 0, a);
  hipExtLaunchKernelGGL(deep_final_kernel, grid, block, 0, s, nullptr, ev.stop, 0, a);
}

}  // namespace gs
