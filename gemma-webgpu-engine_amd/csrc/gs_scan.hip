// One-pass chunk scan: the streaming half of the batched sampler.
//
// A chunk is 8192 consecutive logits of one row, read exactly once from HBM
// by one 256-thread workgroup (32 logits per thread, as 16-byte loads). Per
// chunk the workgroup emits:
//   * for each of its four waves, the wave maximum and sum_i e^((l_i -
//     wave max)/T) in binary64, the pieces of the reference's softmax
//     normaliser (src/runtime/sampling.ts:36-41); each thread sums against
//     its own maximum and the 64 partial sums are rescaled to the wave's;
//   * a candidate list: every finite logit >= tau, where tau is a threshold
//     with at least `depth` logits of the chunk at or above it. The list thus
//     holds the chunk's top-`depth` in the reference's (value desc, id asc)
//     order (sampling.ts:33-35) and every finite logit of the chunk >= tau.
//     Each wave appends to a sub-list of its own at positions taken from
//     ballots, staged in LDS and written out with one coalesced store.
// Logits of "special" ids (the row's penalty window and forced ids) are left
// out here; the finish kernel evaluates them exactly. Masked ids (constraint
// bitmask) are -inf, as maskConstraintLogits makes them
// (src/runtime/constraints.ts:159-173).
//
// Streaming. A group workgroup scans up to kMaxGroupChunks consecutive full
// chunks of one row as a two-stage software pipeline: the loads of chunk i+1
// are in flight while chunk i is reduced. Group loads are raw buffer loads
// whose extent is one chunk, so the prefetch past the group's last chunk
// returns zeros without a memory access and no load sits under a branch.
// The group's first chunk takes its tau from the lane maxima: the smallest of
// the four waves' d-th largest lane maxima (d = ceil(depth/4), plus 2 for
// top-p rows; found with ballots), exchanged at one LDS-only barrier. That tau serves every later
// chunk of the group as well -- the first chunk alone holds `depth` logits
// at or above it, so the group's top-`depth` are all >= it -- and the later
// chunks need no barrier and no exchange at all: each wave reduces, gathers
// and writes its own statistics. The launch is one generation of workgroups,
// each row's full chunks split evenly over its groups. The special ids of the
// group's whole extent are marked once, in an LDS bitmap, before the first
// chunk. A row's last, partial chunk (vocab not a multiple of 8192) and rows
// that are not 16-byte aligned are scanned one chunk per workgroup with
// bounded element loads.
//
// Normaliser error. A thread's terms are binary32: 2^(x c - B) by one fma
// and v_exp_f32 (relative error below 8.5e-8 over its whole binary32 domain
// [-150, 0], checked exhaustively by a GPU test against 1e-7), whose exponent
// carries the roundings of c and of the fma, 2u|y| for a term 2^y (u =
// 2^-24); weighted by the terms, with the thread's maximum among them at
// y = 0, these average at most 2.64 * 2u ln2 = 2.2e-7. The pair sums round
// once more (u). A thread's sum is thus within 3.8e-7 relative of the exact
// one; the lane rescale (2^(y/256) = 2^(j/256) * 2^k * e^r with a correctly
// rounded 256-entry table and a quadratic in r, 4.2e-10), the finish
// kernel's rescales (bit-exact exp) and binary64 sums add under 1e-9, so a
// chunk's sum is within 3.9e-7 relative (kScanSumRel). Only the normaliser sees it, and only the top-p cut depends
// on the normaliser: the finish kernel decides it with that margin and
// recomputes the normaliser in binary64 for rows inside it. Every ordering
// and every probability ratio the filters compare is recomputed exactly.
#include "gs_exp2.h"
#include "gs_internal.h"

namespace gs {
namespace {

constexpr int kChunkWords = kChunk / 32;  // special-bitmap words of one chunk
constexpr int kMaxGroupChunks = 16;       // chunks one group workgroup streams
// Resident scan workgroups per CU (the launch bound). A constrained row's
// mask is folded into the special-id bitmap before its chunks stream, so the
// constrained variants run the same loop as the others and share the bound
// (carrying mask words through the loop took them past 128 VGPRs: at 4 per
// CU they spilled, at 3 the masked scan of 256 x 262144 took 51 us).
template <typename In, bool kMaskable>
constexpr int scan_wg_per_cu() { return 4; }

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

// The calling wave's instruction-issue priority, 0..3 (s_setprio takes an
// immediate).
__device__ __forceinline__ void set_wave_priority(int p) {
  if (p >= 3) __builtin_amdgcn_s_setprio(3);
  else if (p == 2) __builtin_amdgcn_s_setprio(2);
  else if (p == 1) __builtin_amdgcn_s_setprio(1);
  else __builtin_amdgcn_s_setprio(0);
}

// Per-wave results of a group's first chunk, exchanged through LDS.
struct WaveSlots {
  uint32_t wbad[kScanWaves];
  uint32_t wlanes[kScanWaves]; // lanes with a finite maximum
  uint32_t wtau[kScanWaves];   // the wave's d-th largest lane maximum (0: fewer than d lanes)
  uint64_t wbest[kScanWaves];
};

struct ScanShared {
  uint32_t special[kMaxGroupChunks * kChunkWords];  // special ids of the workgroup's chunks (thread-major)
  double tab[256];
  WaveSlots slots[2];                // consecutive exchanges alternate between the two
  uint64_t stage[kScanWaves * kSubCap];  // each wave's list entries before they go out
};

// The row's penalty window [w0, w1) and forced ids [f0, f1) as offsets into
// the history and forced id arrays.
struct RowRanges {
  int64_t w0, w1, f0, f1;
};

// Loads of one chunk's logits for the single-chunk path (kFull: 16-byte
// vector loads; otherwise element loads bounded by n_valid).
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

// Cache policy of the logits loads: non-temporal (gfx950's NT bit, bit 1 of
// a buffer load's cache-policy operand). Every logit is read once, and
// marking the stream non-temporal keeps it from displacing what the caches
// hold for reuse: the penalties batch (256 x 262144 f32) scans in 46 us
// instead of 54.5 us.
constexpr int32_t kLoadNT = 2;

// Loads of chunk lc of a group (logits, and mask words for constrained rows).
// Each chunk gets a buffer resource of its own whose extent is the chunk
// (lc < nc) or empty (lc >= nc): loads of an empty one return zeros without
// a memory access. Lane offsets are tid * 16 and the load index goes into the
// scalar offset, so one VGPR addresses them all.
template <typename In>
__device__ __forceinline__ void load_group_logits(const char* lbase, int lc, int nc,
                                                  uint4 (&raw)[kElemsPerThread / VecTraits<In>::kVec]) {
  constexpr int kLoads = kElemsPerThread / VecTraits<In>::kVec;
  constexpr int32_t kChunkBytes = kChunk * (int32_t)sizeof(In);
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  const int tid = threadIdx.x;
  const __amdgpu_buffer_rsrc_t lg = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(lbase + (int64_t)lc * kChunkBytes), (short)0, lc < nc ? kChunkBytes : 0, kBufferWord3);
#pragma unroll
  for (int v = 0; v < kLoads; ++v) {
    const u32x4 w = __builtin_amdgcn_raw_buffer_load_b128(lg, tid * 16, v * kScanThreads * 16, kLoadNT);
    raw[v] = make_uint4(w.x, w.y, w.z, w.w);
  }
}
// A group chunk's mask words, one per lane: a wave's kLoads loads of kVec
// logits per thread cover 2 kVec consecutive mask words each, 64 in all, so
// lane l loads word j = l of its wave's share -- load v = l / (2 kVec),
// word v 8 kVec + 2 kVec wave + l % (2 kVec) of the chunk -- and a thread
// takes the word of its load v from lane v 2 kVec + (l kVec) / 32.
// Chunks lc >= nc read zeros (an empty buffer range).
template <typename In>
__device__ __forceinline__ uint32_t load_group_mask_lane(const char* mbase, int lc, int nc) {
  constexpr int kVec = VecTraits<In>::kVec;
  static_assert(kElemsPerThread / kVec * 2 * kVec == 64, "one mask word per lane");
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int word = (lane / (2 * kVec)) * 8 * kVec + 2 * kVec * wave + lane % (2 * kVec);
  const __amdgpu_buffer_rsrc_t mk = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(mbase + (int64_t)lc * (kChunkWords * 4)), (short)0, lc < nc ? kChunkWords * 4 : 0, kBufferWord3);
  return __builtin_amdgcn_raw_buffer_load_b32(mk, word * 4, 0, 0);
}
// Folds a constrained group's mask into its LDS special-id bitmap (thread-
// major: word i kChunkWords + tid, bit e = element e of thread tid in chunk
// i): an id the mask forbids is excluded from the scan like a special id.
// Writes every word of the group's nc chunks (the zero fill of an
// unconstrained group).
template <typename In>
__device__ __forceinline__ void fold_group_mask(const char* mk, int nc, uint32_t* s_special) {
  constexpr int kVec = VecTraits<In>::kVec;
  constexpr int kLoads = kElemsPerThread / kVec;
  constexpr uint32_t kLaneBits = (1u << kVec) - 1u;
  const int tid = threadIdx.x, lane = tid & 63;
  uint32_t w[kMaxGroupChunks];
#pragma unroll
  for (int i = 0; i < kMaxGroupChunks; ++i) w[i] = load_group_mask_lane<In>(mk, i, nc);
#pragma unroll
  for (int i = 0; i < kMaxGroupChunks; ++i) {
    if (i < nc) {
      uint32_t dead = 0;
#pragma unroll
      for (int v = 0; v < kLoads; ++v) {
        const int loc = (v * kScanThreads + tid) * kVec;
        const uint32_t mw = (uint32_t)__shfl((int)w[i], v * 2 * kVec + ((lane * kVec) >> 5), 64);
        dead |= (~(mw >> (loc & 31)) & kLaneBits) << (v * kVec);
      }
      s_special[i * kChunkWords + tid] = dead;
    }
  }
}
// The statistics and candidate list of one chunk from its loaded logits.
// kFull: all kChunk logits exist. special: the chunk's words of the LDS
// special-id bitmap, which also holds the ids a constraint mask forbids.
// thr_in > 0 is the group's tau (the stream path: no exchange); with
// thr_in == 0 the chunk takes its own tau and every path passes exactly one
// workgroup barrier. W: the LDS slots of an exchange. Returns the threshold the chunk applied
// when it truncated (0 otherwise).
template <typename In, bool kFull>
__device__ __forceinline__ uint32_t chunk_stats(const SampleArgs& a, const gs_row_config& cfg, const Plan plan,
                                                const int64_t row, const int chunk, const int n_valid,
                                                const uint4 (&raw)[kElemsPerThread / VecTraits<In>::kVec],
                                                const uint32_t* s_special, const double* s_tab, WaveSlots& W,
                                                uint64_t* s_stage, const uint32_t thr_in) {
  using VT = VecTraits<In>;
  constexpr int kVec = VT::kVec;
  constexpr int kLoads = kElemsPerThread / kVec;
  constexpr uint32_t kLaneBits = (1u << kVec) - 1u;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bool stream = thr_in != 0u;  // uniform over the workgroup
  const bool greedy = !stream && plan.route == kRouteGreedy;
  const int64_t gbase = (int64_t)chunk * kChunk;
  ChunkStat* stat = a.stats + row * a.n_chunks + chunk;
  uint64_t* list = a.lists + (row * a.n_chunks + chunk) * kGatherCap;

  // values: excluded (special / out of range) and masked ids become -inf,
  // which neither the normaliser nor the candidate list admits. The thread's
  // excluded elements are one bitmap word (bit e = element e of the thread);
  // the per-element masking runs only when some lane of the wave has one.
  float x[kElemsPerThread];
#pragma unroll
  for (int v = 0; v < kLoads; ++v) {
#pragma unroll
    for (int j = 0; j < kVec; ++j) x[v * kVec + j] = __builtin_bit_cast(float, VT::bits(raw[v], j));
  }
  if (cfg.softcap > 0) {
#pragma unroll
    for (int e = 0; e < kElemsPerThread; ++e) x[e] = capped(x[e], cfg.softcap);
  }
  uint32_t dead = s_special[tid];
  if (!kFull) {
#pragma unroll
    for (int v = 0; v < kLoads; ++v) {
      const int left = n_valid - (v * kScanThreads + tid) * kVec;
      const uint32_t in_range = left >= kVec ? kLaneBits : (left > 0 ? (1u << left) - 1u : 0u);
      dead |= (~in_range & kLaneBits) << (v * kVec);
    }
  }
  if (__ballot(dead != 0)) {
#pragma unroll
    for (int e = 0; e < kElemsPerThread; ++e) {
      if ((dead >> e) & 1u) x[e] = -__builtin_inff();
    }
  }

  // the thread's maximum (NaN-propagating: NaN or +inf flags the row)
  float tmax = -__builtin_inff();
#pragma unroll
  for (int e = 0; e < kElemsPerThread; ++e) tmax = __builtin_elementwise_maximum(tmax, x[e]);
  const bool finite_max = tmax > -__builtin_inff() && tmax < __builtin_inff();
  const bool thread_bad = !(tmax < __builtin_inff());

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
    if (lane == 0) { W.wbest[wave] = best; W.wbad[wave] = wb != 0; }
    lds_barrier();
    if (tid == 0) {
      uint64_t bst = 0;
      uint32_t anybad = 0;
      for (int w = 0; w < kScanWaves; ++w) { bst = W.wbest[w] > bst ? W.wbest[w] : bst; anybad |= W.wbad[w]; }
      if (bst) list[0] = list_slot(__builtin_bit_cast(uint32_t, key_f32(entry_key(bst))), entry_id(bst));
      ChunkStat st{};
      st.wmax[0] = entry_key(bst);
      st.wflags[0] = anybad ? kChunkNonFinite : 0u;
      st.threshold = entry_key(bst);
      st.n_sub[0] = bst ? 1u : 0u;
      *stat = st;
    }
    return 0u;
  }

  // the thread's sum of e^((l - tmax)/T) in binary32 terms 2^(x c - B),
  // c = log2(e)/T and B = tmax c rounded to binary32, each one fma and one
  // hardware exp2; terms are added in pairs in binary32 and the pairs in
  // binary64. The rounding of B (berr, exact by fma) is a factor 2^berr
  // common to the thread's terms, divided out in binary64 by the rescale
  // below. -inf (excluded, masked) enters as a term of exactly 0.
  const double A = (1.0 / cfg.temperature) * GS_256_LOG2E;  // 256 log2(e) / T
  const float c32 = (float)(A * (1.0 / 256.0));
  double sum = 0.0;
  float berr = 0.0f;
  bool scale_bad = false;
  if (finite_max) {
    const float B = tmax * c32;
    berr = __builtin_fmaf(tmax, c32, -B);
    // an infinite or NaN scale leaves the one-pass contract (exact path)
    scale_bad = !(__builtin_fabsf(B) < __builtin_inff()) || !(berr == berr);
#pragma unroll
    for (int e = 0; e < kElemsPerThread; e += 2) {
      const float t0 = __builtin_amdgcn_exp2f(__builtin_fmaf(x[e], c32, -B));
      const float t1 = __builtin_amdgcn_exp2f(__builtin_fmaf(x[e + 1], c32, -B));
      sum += (double)(t0 + t1);
    }
  }

  // wave statistics: the maximum, the flags and the sum rescaled to the wave
  // maximum (written below); the group's first chunk also takes its tau
  const uint32_t mykey = finite_max ? f32_key(tmax) : 0u;
  uint32_t wm, wlo;
  wave_max_min_u32(mykey, &wm, &wlo);
  const bool wave_bad = __ballot(thread_bad || scale_bad) != 0;
  double part = 0.0;
  if (finite_max && sum > 0.0) {
    // e^((tmax - wave max)/T) 2^-berr, in units of 2^(1/256)
    const double y = ((double)tmax - (double)key_f32(wm)) * A - 256.0 * (double)berr;
    part = y > kSkipY ? sum * exp2_256(y, s_tab) : 0.0;
  }
  part = wave_sum_f64_dpp(part);

  uint32_t thr = thr_in;
  bool selected = true;
  if (!stream) {
    const uint32_t depth = (uint32_t)plan.depth;
    // per wave: a quarter of the depth; top-p rows take two more each, which
    // lowers tau a little, so that the fast path's top 64 rarely lies below it
    const uint32_t dw = (depth + 3u) / 4u + (plan.route == kRouteTopK ? 0u : 2u);
    const uint32_t wl = (uint32_t)__popcll(__ballot(mykey != 0u));
    const uint32_t wt = wl >= dw ? wave_kth_key(mykey, dw, wlo, wm) : 0u;
    if (lane == 0) {
      W.wbad[wave] = wave_bad;
      W.wlanes[wave] = wl;
      W.wtau[wave] = wt;
    }
    lds_barrier();
    uint32_t cbad = 0, lanes = 0, tau = 0xFFFFFFFFu, bound = 0;
#pragma unroll
    for (int w = 0; w < kScanWaves; ++w) {
      cbad |= W.wbad[w];
      lanes += W.wlanes[w];
      if (W.wtau[w]) { tau = W.wtau[w] < tau ? W.wtau[w] : tau; bound += dw; }
    }
    if (cbad) {
      // NaN or +inf among the live logits: outside the one-pass contract
      if (lane == 0) {
        stat->wmax[wave] = wm;
        stat->wsum[wave] = 0.0;
        stat->wflags[wave] = kChunkNonFinite;
        stat->n_sub[wave] = 0;
        if (wave == 0) { stat->threshold = 0; stat->truncated = 0; }
      }
      return 0u;
    }
    // at least `depth` per-thread maxima are >= tau (dw of each wave that
    // has dw finite lanes); nearly full chunks are listed whole
    selected = lanes > depth + 32u && bound >= depth;
    thr = selected && tau > kKeyNegInf ? tau : kKeyNegInf + 1u;
  }
  const float tf = key_f32(thr);

  // gather every finite logit >= tau into this wave's sub-list, staged in LDS
  // at positions taken from ballots and written out with one coalesced store
  // per 64 entries (entries past kSubCap are counted, not kept)
  uint64_t* stage = s_stage + wave * kSubCap;
  uint64_t* sub = list + wave * kSubCap;
  const uint32_t id0 = (uint32_t)gbase + (uint32_t)(tid * kVec);
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
          const uint32_t id = id0 + (uint32_t)(v * kScanThreads * kVec + j);
          if (pos < (uint32_t)kSubCap) stage[pos] = list_slot(__builtin_bit_cast(uint32_t, y), id);
        }
        off += (uint32_t)__popcll(m);
      }
    }
  }
  {
    const uint32_t n = off < (uint32_t)kSubCap ? off : (uint32_t)kSubCap;
    if ((uint32_t)lane < n) sub[lane] = stage[lane];
    if ((uint32_t)lane + 64u < n) sub[lane + 64] = stage[lane + 64];
  }
  // the wave's statistics; a sub-list count above kSubCap tells the finish
  // that it overflowed
  if (lane == 0) {
    stat->wsum[wave] = part;
    stat->wmax[wave] = wm;
    stat->wflags[wave] = wave_bad ? kChunkNonFinite : 0u;
    stat->n_sub[wave] = (uint16_t)(off < 0xFFFFu ? off : 0xFFFFu);
    if (wave == 0) {
      stat->threshold = thr;
      // with a tau, lanes whose maximum lies below it left finite logits out
      stat->truncated = selected ? 1u : 0u;
    }
  }
  return selected ? thr : 0u;
}

// Marks the row's special ids that fall in [gbase, gbase + span) in the LDS
// bitmap, thread-major: chunk lc's word t holds thread t's elements, bit
// e = v * kVec + j for the logit at chunk offset (v * 256 + t) * kVec + j.
// The first window and forced ids were loaded by the caller ahead of the
// chunk loads.
template <typename In, bool kMasked>
__device__ __forceinline__ void mark_specials(const SampleArgs& a, const RowRanges rr, int64_t gbase, int span,
                                              int32_t hid0, int32_t hid1, int32_t fid0, uint32_t* s_special) {
  constexpr int kVec = VecTraits<In>::kVec;
  const int tid = threadIdx.x;
  const int64_t wn = rr.w1 - rr.w0;
  const int64_t f0 = kMasked ? rr.f0 : 0, f1 = kMasked ? rr.f1 : 0;
  const int64_t fn = f1 - f0;
  // ids are below 2^31, so offsets from the base fit in 32 bits
  const int32_t base32 = (int32_t)gbase;
  auto mark = [&](int32_t id) {
    const uint32_t loc = (uint32_t)(id - base32);
    if (loc < (uint32_t)span) {
      const uint32_t l = loc % (uint32_t)kChunk;
      const uint32_t t = (l / kVec) % kScanThreads;
      const uint32_t e = (l / (kVec * kScanThreads)) * kVec + l % kVec;
      atomicOr(&s_special[(loc / kChunk) * kChunkWords + t], 1u << e);
    }
  };
  if (tid < wn) mark(hid0);
  if (tid + kScanThreads < wn) mark(hid1);
  for (int64_t j = rr.w0 + 2 * kScanThreads + tid; j < rr.w1; j += kScanThreads) mark(a.history_ids[j]);
  if (tid < fn) mark(fid0);
  for (int64_t j = f0 + kScanThreads + tid; j < f1; j += kScanThreads) mark(a.forced_ids[j]);
}

// The first window and forced ids of the row (one or two per thread), read
// from valid addresses only, so that no load sits under a branch.
template <bool kMasked>
__device__ __forceinline__ void first_specials(const SampleArgs& a, const RowRanges rr, int32_t* hid0,
                                               int32_t* hid1, int32_t* fid0) {
  const int tid = threadIdx.x;
  const int32_t* dummy = (const int32_t*)a.configs;  // any valid device address
  const int64_t wn = rr.w1 - rr.w0;
  const int32_t* hp = wn > 0 ? a.history_ids + rr.w0 : dummy;
  *hid0 = hp[tid < wn ? tid : 0];
  *hid1 = hp[tid + kScanThreads < wn ? tid + kScanThreads : 0];
  const int64_t fn = kMasked ? rr.f1 - rr.f0 : 0;
  const int32_t* fp = fn > 0 ? a.forced_ids + rr.f0 : dummy;
  *fid0 = fp[tid < fn ? tid : 0];
}

// One chunk per workgroup: a row's partial last chunk, or any chunk of a row
// that is not 16-byte aligned (kFull false), or a full chunk otherwise.
template <typename In, bool kFull, bool kMasked>
__device__ __forceinline__ void scan_single(const SampleArgs& a, const gs_row_config& cfg, const Plan plan,
                                            const RowRanges rr, const int64_t row, const int chunk,
                                            const int n_valid, ScanShared& S, const bool row_masked) {
  using VT = VecTraits<In>;
  constexpr int kVec = VT::kVec;
  constexpr int kLoads = kElemsPerThread / kVec;
  const int tid = threadIdx.x;
  const int64_t gbase = (int64_t)chunk * kChunk;
  int32_t hid0, hid1, fid0;
  first_specials<kMasked>(a, rr, &hid0, &hid1, &fid0);
  const double tabv = c_exp2_256[tid];

  uint4 raw[kLoads];
  load_chunk<In, kFull>(a, row, gbase, n_valid, raw);
  // the ids the row's mask forbids start the thread's special-bitmap word
  // (kChunkWords == kScanThreads); bits past n_valid are excluded anyway
  uint32_t dead = 0;
  if (kMasked && row_masked) {
    constexpr uint32_t kLaneBits = (1u << kVec) - 1u;
    const uint32_t* maskp = a.mask_table + (int64_t)cfg.mask_slot * a.mask_words + (gbase >> 5);
#pragma unroll
    for (int v = 0; v < kLoads; ++v) {
      const int loc = (v * kScanThreads + tid) * kVec;
      const uint32_t mw = maskp[(loc < n_valid ? loc : n_valid - 1) >> 5];
      dead |= (~(mw >> (loc & 31)) & kLaneBits) << (v * kVec);
    }
  }

  S.special[tid] = dead;
  S.tab[tid] = tabv;
  lds_barrier();
  mark_specials<In, kMasked>(a, rr, gbase, n_valid, hid0, hid1, fid0, S.special);
  lds_barrier();
  chunk_stats<In, kFull>(a, cfg, plan, row, chunk, n_valid, raw, S.special, S.tab, S.slots[0], S.stage, 0u);
}

// Chunks [c0, c0 + nc) of one row, all full and 16-byte aligned, as a
// two-stage pipeline over two register buffers; the kernel has already
// issued the loads of the first chunk's logits into cur.
// kMasked: the kernel handles constrained rows; row_masked: this row is one
// (its mask is folded into the special-id bitmap first).
template <typename In, bool kMasked>
__device__ __forceinline__ void scan_group(const SampleArgs& a, const gs_row_config& cfg, const Plan plan,
                                           const RowRanges rr, const int64_t row, const int c0, const int nc,
                                           uint4 (&cur)[kElemsPerThread / VecTraits<In>::kVec], ScanShared& S,
                                           const bool row_masked) {
  constexpr int kLoads = kElemsPerThread / VecTraits<In>::kVec;
  const int tid = threadIdx.x;
  const int64_t gbase = (int64_t)c0 * kChunk;
  const char* lg = (const char*)((const In*)a.logits + row * a.row_stride + gbase);
  uint4 nxt[kLoads];
  load_group_logits<In>(lg, 1, nc, nxt);
  int32_t hid0, hid1, fid0;
  first_specials<kMasked>(a, rr, &hid0, &hid1, &fid0);
  const double tabv = c_exp2_256[tid];
  S.tab[tid] = tabv;
  if (kMasked && row_masked) {
    const char* mk = (const char*)(a.mask_table + (int64_t)cfg.mask_slot * a.mask_words + (gbase >> 5));
    fold_group_mask<In>(mk, nc, S.special);
  } else {
    for (int i = tid; i < nc * kChunkWords; i += kScanThreads) S.special[i] = 0;
  }
  lds_barrier();
  mark_specials<In, kMasked>(a, rr, gbase, nc * kChunk, hid0, hid1, fid0, S.special);
  lds_barrier();

  // Two buffers with fixed roles (the loop is unrolled by two, so no register
  // rotation copies wait on loads just issued): chunk i is reduced from cur
  // while chunk i+1 streams into nxt, then cur starts loading chunk i+2, and
  // chunk i+1 is reduced from nxt while chunk i+2 streams in.
  uint32_t thr = 0;
#pragma unroll 1
  for (int i = 0; i < nc; i += 2) {
    // Issue priority by the share of the group's chunks still to scan: a
    // CU's four workgroups start together, and by age alone the first
    // dispatched would run ahead and leave the last to finish with the CU
    // a quarter occupied; falling priority keeps them level, so the CU's
    // waves stay many until its last chunks (-3 us at 256 x 262144)
    set_wave_priority((4 * (nc - i) - 1) / nc);
    uint32_t t = chunk_stats<In, true>(a, cfg, plan, row, c0 + i, kChunk, cur, S.special + i * kChunkWords, S.tab,
                                       S.slots[0], S.stage, thr);
    thr = thr ? thr : t;
    load_group_logits<In>(lg, i + 2, nc, cur);
    if (i + 1 >= nc) break;
    t = chunk_stats<In, true>(a, cfg, plan, row, c0 + i + 1, kChunk, nxt, S.special + (i + 1) * kChunkWords, S.tab,
                              S.slots[1], S.stage, thr);
    thr = thr ? thr : t;
    load_group_logits<In>(lg, i + 3, nc, nxt);
  }
}

// Work split of one launch: blockIdx.x = g < n_groups scans the full chunks
// [g * n_grouped / n_groups, (g + 1) * n_grouped / n_groups) of row
// blockIdx.y; the workgroups after them scan the remaining chunks one each,
// from chunk n_grouped on.
struct ScanGrid {
  int32_t n_groups;
  int32_t n_grouped;
};

// kMaskable: the batch has a mask table (otherwise no row is constrained and
// the masked variants are left out).
template <typename In, bool kMaskable>
__global__ __launch_bounds__(kScanThreads, (scan_wg_per_cu<In, kMaskable>())) void scan_kernel(SampleArgs a, ScanGrid g) {
  __shared__ ScanShared S;
  constexpr int kLoads = kElemsPerThread / VecTraits<In>::kVec;
  const int64_t row = blockIdx.y;
  // a group's first chunk starts loading before anything else: its address
  // comes from the kernel arguments alone
  const bool group = (int)blockIdx.x < g.n_groups;
  const uint32_t gx = blockIdx.x, ng = (uint32_t)g.n_groups, nfull = (uint32_t)g.n_grouped;
  const int c0 = group ? (int)((gx * nfull) / ng) : 0;
  const int nc = group ? (int)(((gx + 1u) * nfull) / ng) - c0 : 0;
  uint4 cur[kLoads];
  if (group) {
    const char* lg = (const char*)((const In*)a.logits + row * a.row_stride + (int64_t)c0 * kChunk);
    load_group_logits<In>(lg, 0, nc, cur);
  }
  const gs_row_config cfg = a.configs[row];
  const Plan plan = plan_row(cfg);
  // row-uniform offsets read here, ahead of every branch and store, so they
  // come through the scalar cache
  RowRanges rr;
  history_window(a, row, cfg, &rr.w0, &rr.w1);
  rr.f0 = rr.f1 = 0;
  const bool masked = kMaskable && cfg.mask_slot >= 0 && cfg.mask_slot < a.mask_slots;
  // forced ids belong to constrained rows only
  if (a.forced_offsets && masked) { rr.f0 = a.forced_offsets[row]; rr.f1 = a.forced_offsets[row + 1]; }
  if (plan.route != kRouteExact) {
    // One path per kernel: with a mask table every row takes the masked
    // path, a row without a mask as if its mask were all ones (the two paths
    // inlined side by side cost the kernel 272 B of spills per lane at 4
    // workgroups per CU, the masked one alone 64 B).
    if (group) {
      scan_group<In, kMaskable>(a, cfg, plan, rr, row, c0, nc, cur, S, masked);
    } else {
      const int chunk = g.n_grouped + ((int)blockIdx.x - g.n_groups);
      const int64_t gbase = (int64_t)chunk * kChunk;
      const int n_valid = (int)((int64_t)a.vocab - gbase < kChunk ? (int64_t)a.vocab - gbase : kChunk);
      const bool full = n_valid == kChunk && a.vector_ok;
      if (full) scan_single<In, true, kMaskable>(a, cfg, plan, rr, row, chunk, n_valid, S, masked);
      else scan_single<In, false, kMaskable>(a, cfg, plan, rr, row, chunk, n_valid, S, masked);
    }
  }
  // reset the queues the finish kernel fills for the exact and deep kernels
  // (all run after this kernel on the same stream). It is the kernel's last
  // store, so the loads above of the row's options and history offsets may
  // use the scalar cache.
  if (row == 0 && blockIdx.x == 0 && threadIdx.x == 0) {
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

// Relative error of v_exp_f32 at the binary32 values with bit patterns
// first .. first + count - 1 (one sign), against binary64 exp2; the largest,
// as (error as binary32 bits) << 32 | y bits, by a 64-bit atomic maximum.
__global__ void exp2_check_kernel(uint32_t first, uint32_t count, unsigned long long* worst) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  unsigned long long mine = 0;
  if (i < count) {
    const uint32_t b = first + i;
    const float y = __builtin_bit_cast(float, b);
    const double r = exp2((double)y);
    if (r >= 0x1p-126 && r <= 0x1.fffffep127) {
      const double rel = __builtin_fabs((double)__builtin_amdgcn_exp2f(y) - r) / r;
      // rounded up to binary32, so the reported bound never understates
      float relf = (float)rel;
      if ((double)relf < rel) relf = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, relf) + 1u);
      mine = ((unsigned long long)__builtin_bit_cast(uint32_t, relf) << 32) | b;
    }
  }
  for (int m = 32; m > 0; m >>= 1) {
    const unsigned long long o = shfl_xor_u64(mine, m);
    mine = o > mine ? o : mine;
  }
  if ((threadIdx.x & 63) == 0 && mine) atomicMax(worst, mine);
}

}  // namespace

void launch_exp2_check(uint32_t first, uint32_t count, unsigned long long* worst, hipStream_t s) {
  if (count == 0) return;
  hipLaunchKernelGGL(exp2_check_kernel, dim3((count + 255) / 256), dim3(256), 0, s, first, count, worst);
}

namespace {

template <typename In, bool kMaskable>
void launch_scan_as(const SampleArgs& a, hipStream_t s, LaunchEvents ev) {
  // group workgroups over the full chunks of 16-byte aligned rows: as many
  // per row as fills every CU once (scan_wg_per_cu each), at least one per
  // kMaxGroupChunks chunks and at most one per chunk
  ScanGrid g;
  const int32_t n_full = a.vector_ok ? a.vocab / kChunk : 0;
  int64_t per_row = (int64_t)a.cu_count * scan_wg_per_cu<In, kMaskable>() / a.rows;
  const int64_t min_groups = (n_full + kMaxGroupChunks - 1) / kMaxGroupChunks;
  if (per_row < min_groups) per_row = min_groups;
  if (per_row > n_full) per_row = n_full;
  g.n_groups = (int32_t)per_row;
  g.n_grouped = n_full;
  dim3 grid(g.n_groups + (a.n_chunks - n_full), a.rows);
  hipExtLaunchKernelGGL((scan_kernel<In, kMaskable>), grid, dim3(kScanThreads), 0, s, ev.start, ev.stop, 0, a, g);
}

}  // namespace

void launch_scan(const SampleArgs& a, hipStream_t s, LaunchEvents ev) {
  const bool maskable = a.mask_slots > 0;
  if (a.dtype == GS_BF16) {
    if (maskable) launch_scan_as<uint16_t, true>(a, s, ev);
    else launch_scan_as<uint16_t, false>(a, s, ev);
  } else {
    if (maskable) launch_scan_as<float, true>(a, s, ev);
    else launch_scan_as<float, false>(a, s, ev);
  }
}

}  // namespace gs
