// Internal declarations shared by libgsample's kernels and host code.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/gsample.h"
#include "gs_math.h"

namespace gs {

// ---------------------------------------------------------------- layout
constexpr int kScanThreads = 256;                 // one workgroup = 4 wave64
constexpr int kScanWaves = kScanThreads / 64;
constexpr int kElemsPerThread = 32;
constexpr int kChunk = kScanThreads * kElemsPerThread;  // 8192 logits per chunk
constexpr int kSubCap = 128;                      // list entries each wave of a chunk may emit
constexpr int kGatherCap = kSubCap * kScanWaves;  // 512 list slots per chunk
constexpr int kMaxFastK = 64;                     // top-k handled by the one-pass path
constexpr int kTopPListL = 64;                    // rank depth per chunk in top-p mode
// Rank depth per chunk for top-k rows: min(topK, kTopKChunkDepth). The finish
// needs the row's top topK; a chunk holding more than 16 of them (about
// 1e-12 per chunk for topK 50 over 32 chunks of independent logits) leaves
// fewer than topK candidates above the lists' threshold, which the finish
// detects and replays exactly.
constexpr int kTopKChunkDepth = 16;
constexpr int kFinishThreads = 1024;
constexpr int kFinishCap = 4096;                  // sorted candidate region in the finish kernel
constexpr int kFinishMaxChunks = 256;             // chunk statistics the finish keeps in LDS
constexpr int64_t kMaxVocab = (int64_t)kFinishMaxChunks * kChunk;  // 2097152 ids
constexpr int kSpecialCap = 2048;                 // distinct (window + forced) ids the one-pass finish evaluates
constexpr int kHashSize = 4096;                   // open-addressing table for those ids
constexpr int kExactThreads = 1024;
constexpr int kExactTile = 4096;                  // LDS tile of the exact path's bitonic sort
// bytes of exact-path row scratch per context: one slot per row up to this
// (1024 rows at V = 262144 take 9 GiB, a small share of a 288 GB part), so a
// batch of that size replays its exact rows in place and never launches the
// exact kernel
constexpr int64_t kExactScratchBudget = 12ll << 30;

// relative margin under which a fast-path decision is re-resolved exactly;
// it bounds the reference's own sequential-sum error (V * 2^-53 ~ 3e-11)
constexpr double kNearTie = 1.0e-10;
// relative bound on the chunk scan's normaliser: binary32 terms from the
// hardware exp2, summed per thread (the derivation is in gs_scan.hip); the
// finish kernel decides normaliser-dependent cuts with this margin first
constexpr double kScanSumRel = 3.9e-7;
// relative margin of those decisions once the finish kernel has recomputed
// the normaliser in binary64 (4.2e-10 per term, summation order), with room
constexpr double kNormaliserRel = 4.0e-9;
// reporting tolerance for top-p boundary ties (1e-6 relative)
constexpr double kTieReport = 1.0e-6;

// ------------------------------------------------------- orderable keys
// 32-bit key of an f32 value, increasing with the value; -0 and +0 share a
// key (they are equal to the reference's comparator). 0 is never produced
// for a non-NaN value and marks "no element".
constexpr uint32_t kKeyNegInf = 0x007FFFFFu;    // key of -inf
constexpr uint32_t kKeyPosInf = 0xFF800000u;    // key of +inf

__host__ __device__ __forceinline__ uint32_t f32_key(float x) {
  uint32_t b = __builtin_bit_cast(uint32_t, x);
  if (b == 0x80000000u) b = 0;
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__host__ __device__ __forceinline__ float key_f32(uint32_t k) {
  const uint32_t b = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __builtin_bit_cast(float, b);
}
// 64-bit key of an f64 value (same conventions).
__host__ __device__ __forceinline__ uint64_t f64_key(double x) {
  uint64_t b = __builtin_bit_cast(uint64_t, x);
  if (b == 0x8000000000000000ull) b = 0;
  return (b >> 63) ? ~b : (b | 0x8000000000000000ull);
}
__host__ __device__ __forceinline__ double key_f64(uint64_t k) {
  const uint64_t b = (k >> 63) ? (k & 0x7fffffffffffffffull) : ~k;
  return __builtin_bit_cast(double, b);
}
// list entry: value key high, inverted id low -> descending order is
// (value desc, id asc), the reference's stable-sort order
__host__ __device__ __forceinline__ uint64_t pack_entry(uint32_t key, uint32_t id) {
  return ((uint64_t)key << 32) | (uint32_t)~id;
}
__host__ __device__ __forceinline__ uint32_t entry_key(uint64_t e) { return (uint32_t)(e >> 32); }
__host__ __device__ __forceinline__ uint32_t entry_id(uint64_t e) { return ~(uint32_t)e; }

// gsm::softcap_f32 as a call of its own: its binary64 divisions and
// exponential are some hundred instructions, which, expanded at every logit
// of an unrolled loop, would overflow the instruction cache for the rows that
// never use it
[[maybe_unused]] static __device__ __noinline__ float softcap_call(float x, double cap) { return gsm::softcap_f32(x, cap); }

// l / T rounded to nearest, from r = 1 / T rounded to nearest: q0 = l r
// lies within an ulp of l / T, the remainder l - q0 T is exact in one fma,
// and q0 + (l - q0 T) r rounded is l / T rounded (Markstein's theorem; it
// needs no overflow or underflow in the quotient and the remainder, which
// |l| < 2^128 with T in [2^-20, 2^20] guarantees). Three operations instead
// of the division's iteration. -0 gives +0, which the keys treat alike.
__device__ __forceinline__ double div_by_temperature(double l, double T, double r) {
  const double q0 = l * r;
  return __builtin_fma(__builtin_fma(-q0, T, l), r, q0);
}

// ---------------------------------------------------------- row routing
enum Route : int32_t {
  kRouteGreedy = 0,  // temperature 0: argmax, first maximum wins
  kRouteTopK = 1,    // 0 < topK <= kMaxFastK
  kRouteTopP = 2,    // topK 0 with a top-p or min-p cut
  kRouteExact = 3,   // sequential replay of the reference (everything else)
};

struct Plan {
  int32_t route;
  int32_t depth;  // per-chunk rank depth of the one-pass path
};

// Routes: greedy rows; top-k rows up to kMaxFastK (chunk lists min(topK, 16)
// deep, typical-p among them: its pool is the top-k); every other row keeps
// 64 entries per chunk (top-p and min-p cuts, top-k up to kFinishCap, draws
// over the whole vocabulary), and the finish resolves what falls inside the
// complete region; typical-p over a longer pool, extreme temperatures and
// forced rows take the exact replay.
__host__ __device__ __forceinline__ Plan plan_row(const gs_row_config& c) {
  if (c.temperature == 0) return Plan{kRouteGreedy, 1};
  if (c.options & GS_ROW_FORCE_EXACT) return Plan{kRouteExact, 0};
  // between these bounds l/T keeps the order and the ties of the f32 logits
  if (!(c.temperature >= 1.0e-200 && c.temperature <= 1.0e200)) return Plan{kRouteExact, 0};
  const bool topk_fast = c.top_k > 0 && c.top_k <= kMaxFastK;
  if (c.typical_p < 1 && !topk_fast) return Plan{kRouteExact, 0};
  if (topk_fast) return Plan{kRouteTopK, c.top_k < kTopKChunkDepth ? c.top_k : kTopKChunkDepth};
  if (c.top_k > kFinishCap) return Plan{kRouteExact, 0};
  return Plan{kRouteTopP, kTopPListL};
}
// plan_row with every field read whatever the route (selects, not branches),
// so that a kernel fetches the whole configuration at once instead of one
// field after another behind branches
__device__ __forceinline__ Plan plan_row_flat(const gs_row_config& c) {
  const bool greedy = c.temperature == 0;
  const bool forced = (c.options & GS_ROW_FORCE_EXACT) != 0;
  const bool t_out = !(c.temperature >= 1.0e-200 && c.temperature <= 1.0e200);
  const bool topk_fast = c.top_k > 0 && c.top_k <= kMaxFastK;
  const bool typical_long = c.typical_p < 1 && !topk_fast;
  const int depth_k = c.top_k < kTopKChunkDepth ? c.top_k : kTopKChunkDepth;
  const bool exact = forced || t_out || typical_long || c.top_k > kFinishCap;
  const int route = greedy ? kRouteGreedy : (exact ? kRouteExact : (topk_fast ? kRouteTopK : kRouteTopP));
  const int depth = greedy ? 1 : (exact ? 0 : (topk_fast ? depth_k : kTopPListL));
  return Plan{route, depth};
}

// ------------------------------------------------------- per-chunk state
struct ChunkStat {
  // wave w of the chunk's workgroup: sum of e^((l - wave max)/T) over its
  // finite non-special logits, the wave maximum's key (kKeyNegInf or below:
  // none) and kChunkNonFinite when NaN or +inf was among its live logits
  double wsum[kScanWaves];
  uint32_t wmax[kScanWaves];
  uint32_t wflags[kScanWaves];
  uint32_t threshold;  // the list holds every finite non-special logit with key >= threshold
  uint32_t truncated;  // some finite logit lies below the threshold
  // entries of wave w's sub-list, which starts at slot w * kSubCap; a count
  // above kSubCap means the wave had more and the sub-list is incomplete
  uint16_t n_sub[kScanWaves];
};

// A list slot holds the logit's f32 bits (after softcap) high and its id low;
// list_rank turns it into a pack_entry (value desc, id asc) ordering key.
__host__ __device__ __forceinline__ uint64_t list_slot(uint32_t bits, uint32_t id) {
  return ((uint64_t)bits << 32) | id;
}
__host__ __device__ __forceinline__ uint64_t list_rank(uint64_t slot) {
  return pack_entry(f32_key(__builtin_bit_cast(float, (uint32_t)(slot >> 32))), (uint32_t)slot);
}
constexpr uint32_t kChunkOverflow = 1u;
constexpr uint32_t kChunkNonFinite = 2u;

// The fused lm_head's epilogue summarises each hidden row's logits in
// partials of kPartIds consecutive ids (one per workgroup and row), which a
// merge kernel turns into the chunk scan's ChunkStat and lists.
constexpr int kPartIds = 256;
constexpr int kPartCap = 32;                          // list slots of one partial
constexpr int kPartsPerChunk = kChunk / kPartIds;     // 32
struct PartStat {
  double sum;         // sum of e^((l - max)/T) over the finite non-excluded logits
  uint32_t max_key;   // the maximum's key (0: none finite)
  uint32_t tau;       // the list holds every finite logit with key >= tau
  uint32_t n;         // entries at or above tau (more than kPartCap: the list is cut)
  uint16_t flags;     // kChunkNonFinite
  uint16_t truncated; // finite logits lie below tau
};

struct ExactQueue {
  uint32_t count;  // rows appended by the finish kernel
  uint32_t next;   // rows taken by the exact kernel
  uint32_t rows[1];
};

// The multi-workgroup deep draw (full-vocabulary draws whose cursor falls
// past the finish's region): the finish leaves each such row's inputs in a
// DeepRow and queues the row; the deep kernels then split its two passes
// over the row's logits into parts (runs of chunks) across workgroups, with
// a launch per row in between and after.
constexpr int kDeepBins = 4096;  // value bins of the deep draw's tail histogram
struct DeepPlan {
  double total, target, mrg, pre_before;  // the normaliser, the cursor, the margin, the mass before b_lo
  float l_lo, l_top;                      // the logit range pass 2 stages
  int32_t b_lo, b_hi;                     // the bins the cursor falls in
};
struct DeepRow {
  double M, u, margin;   // the row's maximum value, its uniform, the reference's rounding margin
  uint64_t floor;        // the region floor's value key
  uint32_t thr, n_reg, n_sp;  // the region floor's logit key, region candidates, specials
  uint32_t index_check;       // checked build: a pass-1 part failed an index check
  DeepPlan plan;
  uint32_t n_stage;           // pass-2 entries staged
  uint32_t index_check2;      // checked build: a pass-2 part failed an index check
  double tail[kFinishMaxChunks];         // pass 1: each part's last-bin sum
  uint64_t hist[kDeepBins];              // pass 1: bin sums in fixed point (global atomics)
  double cand_p[kFinishCap];             // the region's candidates: exact exponentials
  uint32_t cand_id[kFinishCap];
  uint64_t sp_key[kSpecialCap];          // the row's specials
  uint32_t sp_id[kSpecialCap];
  uint64_t stage[kFinishCap];            // pass 2: logits in the plan's range (value bits << 32 | id)
};
struct DeepQueue {
  uint32_t count1, next1;  // rows queued for pass 1, its work items taken
  uint32_t count2, next2;  // rows queued for pass 2, its work items taken
  uint32_t rows[1];        // [2 * max rows]: pass-1 rows, then pass-2 rows
};

// Arguments every sampling kernel reads.
struct SampleArgs {
  const void* logits;
  int64_t row_stride;
  int32_t dtype;
  int32_t rows;
  int32_t vocab;
  int32_t n_chunks;
  int32_t vector_ok;  // 16-byte aligned rows
  int32_t mask_words;
  const gs_row_config* configs;
  const int64_t* history_offsets;
  const int32_t* history_ids;
  const int64_t* forced_offsets;
  const int32_t* forced_ids;
  const uint8_t* forced_kinds;
  const uint32_t* mask_table;
  int32_t mask_slots;
  int32_t exact_slots;
  gs_row_result* results;
  ChunkStat* stats;     // [rows][n_chunks]
  uint64_t* lists;      // [rows][n_chunks][kGatherCap]
  ExactQueue* queue;
  uint8_t* exact_scratch;
  int64_t exact_slot_bytes;
  int64_t exact_capacity;  // entries per slot (power of two >= vocab)
  int32_t cu_count;        // compute units of the device
  DeepRow* deep_rows;      // [rows], or null: the finish's own workgroup takes its deep draws
  DeepQueue* deep_queue;
  int32_t deep_max_rows;   // pass-2 rows start at deep_queue->rows + deep_max_rows
};

// Buffers of the fused lm_head + statistics path.
struct FusedArgs {
  const gs_row_config* configs;
  uint32_t* dead;      // [rows][V/32] excluded ids (mask-forbidden, window, forced)
  PartStat* parts;     // [rows][n_parts]
  uint64_t* plists;    // [rows][n_parts][kPartCap] list slots
  uint32_t* row_thr;   // [rows] the largest tau of the row's truncated partials (0: none)
  int32_t n_parts;     // V / kPartIds
};

// A 16-byte load marked non-temporal, for rows streamed once: the stream
// does not displace what the caches hold for reuse.
// word 3 of a raw buffer resource on gfx9-family parts (gfx950 included)
constexpr int32_t kBufferWord3 = 0x00020000;
// a buffer offset past every resource's extent: the access returns zeros or
// is dropped, without a memory request
constexpr uint32_t kBufferOutOfRange = 0x80000000u;

__device__ __forceinline__ uint4 load_nt16(const uint4* p) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 v = __builtin_nontemporal_load((const u32x4*)p);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// --------------------------------------------------------- wave helpers
// Workgroup barrier for LDS traffic only: LDS stores before it are visible to
// every wave after it, and global loads in flight are not waited for.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Wave-wide reductions and scans with DPP row operations (quad_perm,
// row_shr, row_ror and the gfx9 row_bcast15/31), which stay in the VALU:
// their latency is a few cycles per step, where a cross-lane shuffle
// (ds_bpermute) costs an LDS round trip. Same-address LDS atomics from many
// lanes serialise (about 30 ns per lane), so values are reduced per wave first.
constexpr int kDppQuad1032 = 0xB1;  // quad_perm [1,0,3,2]
constexpr int kDppQuad2301 = 0x4E;  // quad_perm [2,3,0,1]
constexpr int kDppRowShr1 = 0x111;
constexpr int kDppRowShr2 = 0x112;
constexpr int kDppRowShr4 = 0x114;
constexpr int kDppRowShr8 = 0x118;
constexpr int kDppRowShl4 = 0x104;
constexpr int kDppRowRor4 = 0x124;
constexpr int kDppRowRor8 = 0x128;
constexpr int kDppRowHalfMirror = 0x141;  // lane l of each 8 to lane 7 - l
constexpr int kDppRowBcast15 = 0x142;  // lane 15 of a row to the next row (rows 1 and 3 written)
constexpr int kDppRowBcast31 = 0x143;  // lane 31 to rows 2 and 3

// v moved by the DPP control kCtrl; lanes without a source (or in rows that
// kRowMask disables) receive `identity`
template <int kCtrl, int kRowMask>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t identity, uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)identity, (int)v, kCtrl, kRowMask, 0xF, false);
}
template <int kCtrl, int kRowMask>
__device__ __forceinline__ uint64_t dpp_u64(uint64_t identity, uint64_t v) {
  const uint32_t lo = dpp_u32<kCtrl, kRowMask>((uint32_t)identity, (uint32_t)v);
  const uint32_t hi = dpp_u32<kCtrl, kRowMask>((uint32_t)(identity >> 32), (uint32_t)(v >> 32));
  return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint32_t readlane_u32(uint32_t v, int lane) {
  return (uint32_t)__builtin_amdgcn_readlane((int)v, lane);
}
__device__ __forceinline__ uint64_t readlane_u64(uint64_t v, int lane) {
  return ((uint64_t)readlane_u32((uint32_t)(v >> 32), lane) << 32) | readlane_u32((uint32_t)v, lane);
}
__device__ __forceinline__ double readlane_f64(double v, int lane) {
  return __builtin_bit_cast(double, readlane_u64(__builtin_bit_cast(uint64_t, v), lane));
}

// All-reduce of the wave: within rows by quad_perm and row_ror, across rows
// by the two broadcasts; lane 63 ends with the whole wave's result, which
// every lane then reads. OP(a, b) combines, ID is its identity.
#define GS_WAVE_REDUCE(T, DPP, v, ID, OP)                                          \
  do {                                                                             \
    v = OP(v, DPP<kDppQuad1032, 0xF>(ID, v));                                      \
    v = OP(v, DPP<kDppQuad2301, 0xF>(ID, v));                                      \
    v = OP(v, DPP<kDppRowRor4, 0xF>(ID, v));                                       \
    v = OP(v, DPP<kDppRowRor8, 0xF>(ID, v));                                       \
    v = OP(v, DPP<kDppRowBcast15, 0xA>(ID, v));                                    \
    v = OP(v, DPP<kDppRowBcast31, 0xC>(ID, v));                                    \
  } while (0)

__device__ __forceinline__ uint32_t op_max_u32(uint32_t a, uint32_t b) { return a > b ? a : b; }
__device__ __forceinline__ uint32_t op_min_u32(uint32_t a, uint32_t b) { return a < b ? a : b; }
__device__ __forceinline__ uint32_t op_or_u32(uint32_t a, uint32_t b) { return a | b; }
__device__ __forceinline__ uint32_t op_add_u32(uint32_t a, uint32_t b) { return a + b; }
__device__ __forceinline__ uint64_t op_max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  GS_WAVE_REDUCE(uint32_t, dpp_u32, v, 0u, op_max_u32);
  return readlane_u32(v, 63);
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
  GS_WAVE_REDUCE(uint32_t, dpp_u32, v, 0xFFFFFFFFu, op_min_u32);
  return readlane_u32(v, 63);
}
__device__ __forceinline__ uint32_t wave_or_u32(uint32_t v) {
  GS_WAVE_REDUCE(uint32_t, dpp_u32, v, 0u, op_or_u32);
  return readlane_u32(v, 63);
}
__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
  GS_WAVE_REDUCE(uint32_t, dpp_u32, v, 0u, op_add_u32);
  return readlane_u32(v, 63);
}
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
  GS_WAVE_REDUCE(uint64_t, dpp_u64, v, 0ull, op_max_u64);
  return readlane_u64(v, 63);
}
__device__ __forceinline__ uint64_t op_add_u64(uint64_t a, uint64_t b) { return a + b; }
__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) {
  GS_WAVE_REDUCE(uint64_t, dpp_u64, v, 0ull, op_add_u64);
  return readlane_u64(v, 63);
}
// the maximum and minimum of the wave's values, in every lane (the two
// chains interleaved step by step)
__device__ __forceinline__ void wave_max_min_u32(uint32_t v, uint32_t* vmax, uint32_t* vmin) {
  uint32_t a = v, b = v;
#define GS_MM_STEP(C, M)                                \
  { const uint32_t x = dpp_u32<C, M>(0u, a);            \
    const uint32_t y = dpp_u32<C, M>(0xFFFFFFFFu, b);   \
    a = x > a ? x : a; b = y < b ? y : b; }
  GS_MM_STEP(kDppQuad1032, 0xF) GS_MM_STEP(kDppQuad2301, 0xF) GS_MM_STEP(kDppRowRor4, 0xF)
  GS_MM_STEP(kDppRowRor8, 0xF) GS_MM_STEP(kDppRowBcast15, 0xA) GS_MM_STEP(kDppRowBcast31, 0xC)
#undef GS_MM_STEP
  *vmax = readlane_u32(a, 63);
  *vmin = readlane_u32(b, 63);
}
// the sum of the wave's binary64 values (a fixed order), in every lane
__device__ __forceinline__ double wave_sum_f64_dpp(double v) {
#define GS_SUM_STEP(C, M)                                                            \
  { const uint64_t u = __builtin_bit_cast(uint64_t, v);                              \
    const uint32_t lo = dpp_u32<C, M>(0u, (uint32_t)u);                              \
    const uint32_t hi = dpp_u32<C, M>(0u, (uint32_t)(u >> 32));                      \
    v += __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo); }
  GS_SUM_STEP(kDppQuad1032, 0xF) GS_SUM_STEP(kDppQuad2301, 0xF) GS_SUM_STEP(kDppRowRor4, 0xF)
  GS_SUM_STEP(kDppRowRor8, 0xF) GS_SUM_STEP(kDppRowBcast15, 0xA) GS_SUM_STEP(kDppRowBcast31, 0xC)
#undef GS_SUM_STEP
  return readlane_f64(v, 63);
}
// A lower bound t of the d-th largest of the wave's lane keys (d >= 1), at
// most 2^14 below it: the largest t whose low 14 bits are zero with at least
// d keys >= t, found bit by bit with ballots. Bits above the first one where
// the smallest and largest keys differ are common to every key and to the
// answer, so the search starts below them. (For binary32 keys 2^14 units are
// 2^-9 relative: a threshold that low admits a few more list entries.)
__device__ __forceinline__ uint32_t wave_kth_key(uint32_t key, uint32_t d, uint32_t lo, uint32_t hi) {
  constexpr int kFloorBit = 14;
  const uint32_t diff = lo ^ hi;
  if (diff >> kFloorBit == 0) return lo & ~((1u << kFloorBit) - 1u);
  const int top = 31 - __builtin_clz(diff);
  uint32_t t = lo & ~((2u << top) - 1u);  // the common prefix; every key is >= it
  for (int b = top; b >= kFloorBit; --b) {
    const uint32_t c = t | (1u << b);
    if ((uint32_t)__popcll(__ballot(key >= c)) >= d) t = c;
  }
  return t;
}

// Inclusive prefix sums across the wave: within each row of 16 lanes by
// row_shr 1, 2, 4, 8 (lanes without a source add zero), then the last lane
// of row 0 into rows 1 and 3 and the last lane of row 1 into rows 2 and 3.
__device__ __forceinline__ uint32_t wave_scan_u32(uint32_t v) {
  v += dpp_u32<kDppRowShr1, 0xF>(0u, v);
  v += dpp_u32<kDppRowShr2, 0xF>(0u, v);
  v += dpp_u32<kDppRowShr4, 0xF>(0u, v);
  v += dpp_u32<kDppRowShr8, 0xF>(0u, v);
  v += dpp_u32<kDppRowBcast15, 0xA>(0u, v);
  v += dpp_u32<kDppRowBcast31, 0xC>(0u, v);
  return v;
}
__device__ __forceinline__ double wave_scan_f64(double v) {
#define GS_SCAN_STEP(C, M) \
  v += __builtin_bit_cast(double, dpp_u64<C, M>(0ull, __builtin_bit_cast(uint64_t, v)));
  GS_SCAN_STEP(kDppRowShr1, 0xF) GS_SCAN_STEP(kDppRowShr2, 0xF) GS_SCAN_STEP(kDppRowShr4, 0xF)
  GS_SCAN_STEP(kDppRowShr8, 0xF) GS_SCAN_STEP(kDppRowBcast15, 0xA) GS_SCAN_STEP(kDppRowBcast31, 0xC)
#undef GS_SCAN_STEP
  return v;
}

// cross-lane shuffles for the bitonic networks (partner lane = lane ^ m)
__device__ __forceinline__ uint32_t shfl_xor_u32(uint32_t v, int m) { return (uint32_t)__shfl_xor((int)v, m, 64); }
__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m) {
  const uint32_t lo = shfl_xor_u32((uint32_t)v, m), hi = shfl_xor_u32((uint32_t)(v >> 32), m);
  return ((uint64_t)hi << 32) | lo;
}
// The value of lane (lane ^ m), m a power of two up to 32, moved in the
// VALU: quad_perm for 1 and 2, row_shl/row_shr 4 (each lane takes the one
// that stays in its row), row_ror 8, and gfx950's v_permlane16_swap /
// v_permlane32_swap for 16 and 32 (each lane takes the half it did not
// keep). For m known at compile time (unrolled loops) the switch folds away.
__device__ __forceinline__ uint32_t xlane_u32(uint32_t v, int m) {
  const int lane = threadIdx.x & 63;
  switch (m) {
    case 1:
      return dpp_u32<kDppQuad1032, 0xF>(0u, v);
    case 2:
      return dpp_u32<kDppQuad2301, 0xF>(0u, v);
    case 4: {
      const uint32_t up = dpp_u32<kDppRowShl4, 0xF>(0u, v), down = dpp_u32<kDppRowShr4, 0xF>(0u, v);
      return (lane & 4) ? down : up;
    }
    case 8:
      return dpp_u32<kDppRowRor8, 0xF>(0u, v);
    case 16: {
      const auto p = __builtin_amdgcn_permlane16_swap(v, v, false, false);
      return (lane & 16) ? p[0] : p[1];
    }
    default: {
      const auto p = __builtin_amdgcn_permlane32_swap(v, v, false, false);
      return (lane & 32) ? p[0] : p[1];
    }
  }
}
__device__ __forceinline__ uint64_t xlane_u64(uint64_t v, int m) {
  const uint32_t lo = xlane_u32((uint32_t)v, m), hi = xlane_u32((uint32_t)(v >> 32), m);
  return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ double shfl_xor_f64(double v, int m) {
  return __builtin_bit_cast(double, shfl_xor_u64(__builtin_bit_cast(uint64_t, v), m));
}
// butterfly sum of the wave's binary64 values, in every lane
__device__ __forceinline__ double wave_sum_f64(double v) {
  for (int m = 32; m > 0; m >>= 1) v += shfl_xor_f64(v, m);
  return v;
}
// bitonic sort of one u64 per lane, descending across the wave
__device__ __forceinline__ uint64_t wave_sort_desc(uint64_t x, int lane) {
  for (int k = 2; k <= 64; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      const uint64_t y = shfl_xor_u64(x, j);
      const uint64_t hi = x > y ? x : y, lo = x > y ? y : x;
      const bool lower = (lane & j) == 0;
      const bool desc_seg = (lane & k) == 0;
      x = (lower == desc_seg) ? hi : lo;
    }
  }
  return x;
}

// ----------------------------------------------------------- row inputs
__device__ __forceinline__ float load_logit(const SampleArgs& a, int64_t row, int64_t i) {
  if (a.dtype == GS_BF16) {
    const uint16_t* p = (const uint16_t*)a.logits + row * a.row_stride + i;
    return __builtin_bit_cast(float, (uint32_t)(*p) << 16);
  }
  return ((const float*)a.logits)[row * a.row_stride + i];
}

__device__ __forceinline__ bool mask_allows(const SampleArgs& a, int32_t slot, int64_t id) {
  return (a.mask_table[(int64_t)slot * a.mask_words + (id >> 5)] >> (id & 31)) & 1u;
}

// Window of the history that penalties read (sampling.ts:22-24).
__device__ __forceinline__ void history_window(const SampleArgs& a, int64_t row, const gs_row_config& c,
                                               int64_t* begin, int64_t* end) {
  *begin = *end = 0;
  if (!a.history_offsets || c.repetition_window <= 0) return;
  const int64_t h0 = a.history_offsets[row], h1 = a.history_offsets[row + 1];
  const int64_t s = h1 - (int64_t)c.repetition_window;
  *begin = s > h0 ? s : h0;
  *end = h1;
}

// -------------------------------------------- distinct ids of one row
// Hash of the row's distinct special ids (window ids with counts, forced
// ids with kinds), built in LDS by one workgroup.
struct SpecialTable {
  uint32_t* ids;     // kHashSize, 0xFFFFFFFF = empty
  uint32_t* counts;  // kHashSize: window count | kinds << 24
};

__device__ __forceinline__ uint32_t hash_id(uint32_t id) { return (id * 2654435761u) >> 20; }

// Probes an insert may take before the table counts as too crowded: a row
// with more than kSpecialCap distinct ids fills more than half the table,
// and a row that crowded (or whose ids cluster) is replayed on the exact
// path, which counts window ids per vocabulary id instead.
constexpr int kMaxProbe = 64;

// window ids add 1 to the low 24 bits; forced ids OR their kind into the top
// 8. Returns false when the id found no slot within kMaxProbe probes.
__device__ __forceinline__ bool special_insert(SpecialTable t, uint32_t id, uint32_t kind) {
  uint32_t h = hash_id(id) & (kHashSize - 1);
  for (int probe = 0; probe < kMaxProbe; ++probe) {
    const uint32_t prev = atomicCAS(&t.ids[h], 0xFFFFFFFFu, id);
    if (prev == 0xFFFFFFFFu || prev == id) {
      if (kind == 0) atomicAdd(&t.counts[h], 1u);
      else atomicOr(&t.counts[h], kind << 24);
      return true;
    }
    h = (h + 1) & (kHashSize - 1);
  }
  return false;
}

// ---------------------------------------------------- kernel launchers
// Optional timing events of one launch: hipExtLaunchKernel stamps `start`
// when the dispatch begins and `stop` when its last wave ends, so their
// elapsed time is the kernel alone (no event packets or launch gaps).
struct LaunchEvents {
  hipEvent_t start = nullptr;
  hipEvent_t stop = nullptr;
};

void launch_scan(const SampleArgs& a, hipStream_t s, LaunchEvents ev = {});
void launch_exp2_check(uint32_t first, uint32_t count, unsigned long long* worst, hipStream_t s);
void launch_finish(const SampleArgs& a, hipStream_t s, LaunchEvents ev = {});
void launch_exact(const SampleArgs& a, hipStream_t s, LaunchEvents ev = {});
void launch_deep(const SampleArgs& a, hipStream_t s, LaunchEvents ev = {});
void launch_logprob(const void* logits, int32_t dtype, int32_t rows, int64_t stride, int32_t vocab,
                    const int32_t* tokens, double* out, hipStream_t s);
void launch_mask_logits(const float* raw, int64_t n, const int32_t* ids, int64_t n_ids, float* out, hipStream_t s);
void launch_masks(const int64_t* offsets, const uint8_t* bytes, int32_t vocab, const int16_t* next,
                  const int32_t* states, int32_t n, uint32_t* masks, int32_t mask_words, int32_t n_states,
                  hipStream_t s);
void launch_qat_lmhead(const float* x, int32_t M, int32_t D, const uint32_t* words, int32_t block_major,
                       const float* scales, int32_t V, double in_scale, double out_scale, float* out,
                       int32_t cu_count, hipStream_t s, LaunchEvents ev = {});
void launch_lmhead(const uint16_t* hidden, const uint16_t* weight, int32_t m, int32_t width, int32_t vocab,
                   float softcap, float* out, int32_t cu_count, hipStream_t s, LaunchEvents ev = {});
// The fused path (vocab a multiple of kChunk): the excluded-id bitmaps, then
// the lm_head with the partial statistics; launch_merge_parts takes the chunk
// scan's place before the finish.
void launch_lmhead_scan(const uint16_t* hidden, const uint16_t* weight, int32_t m, int32_t width, float softcap,
                        float* out, const SampleArgs& a, const FusedArgs& f, hipStream_t s, LaunchEvents ev = {});
void launch_merge_parts(const SampleArgs& a, const FusedArgs& f, hipStream_t s, LaunchEvents ev = {});

}  // namespace gs
