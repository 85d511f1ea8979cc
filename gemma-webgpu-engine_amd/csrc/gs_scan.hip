// One-pass chunk scan: the streaming half of the batched sampler.
//
// Grid (n_chunks, rows); one 256-thread workgroup reads one 8192-logit chunk
// of one row exactly once from HBM (16-byte vector loads, 32 logits per
// thread held as order-preserving u32 keys in registers) and emits:
//   * the chunk maximum and sum_i e^((l_i - lmax)/T) in binary64, the pieces
//     of the reference's softmax normaliser (src/runtime/sampling.ts:36-41);
//   * a candidate list: every finite logit whose key is >= tau, where tau is
//     the depth-th largest per-lane maximum of the workgroup. At least
//     `depth` logits are >= tau, so the list holds the chunk's top-`depth`
//     in the reference's (value desc, id asc) order (sampling.ts:33-35), and
//     every finite logit of the chunk >= tau.
// Logits of "special" ids (the row's penalty window and forced ids) are left
// out here; the finish kernel evaluates them exactly. Masked ids (constraint
// bitmask) become -inf, as maskConstraintLogits does
// (src/runtime/constraints.ts:159-173).
#include "gs_internal.h"

namespace gs {
namespace {

constexpr int kWaves = kScanThreads / 64;

__constant__ double c_exp2_table[64] = {GSM_EXP2_TABLE_64};

template <typename In>
struct VecTraits;
template <>
struct VecTraits<float> {
  static constexpr int kVec = 4;  // logits per 16-byte load
  __device__ static void load(const float* p, float* out) {
    const float4 v = *(const float4*)p;
    out[0] = v.x; out[1] = v.y; out[2] = v.z; out[3] = v.w;
  }
  __device__ static float one(const float* p) { return *p; }
};
template <>
struct VecTraits<uint16_t> {
  static constexpr int kVec = 8;
  __device__ static void load(const uint16_t* p, float* out) {
    const uint4 v = *(const uint4*)p;
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[2 * i] = __builtin_bit_cast(float, w[i] << 16);
      out[2 * i + 1] = __builtin_bit_cast(float, w[i] & 0xFFFF0000u);
    }
  }
  __device__ static float one(const uint16_t* p) { return __builtin_bit_cast(float, (uint32_t)(*p) << 16); }
};

template <typename In>
__global__ __launch_bounds__(kScanThreads) void scan_kernel(SampleArgs a) {
  using VT = VecTraits<In>;
  constexpr int kVec = VT::kVec;
  constexpr int kLoads = kElemsPerThread / kVec;

  __shared__ uint32_t s_special[kChunk / 32];
  __shared__ uint64_t s_lanemax[kWaves][64];
  __shared__ uint64_t s_list[kGatherCap];
  __shared__ double s_wsum[kWaves];
  __shared__ uint32_t s_wmax[kWaves];
  __shared__ uint32_t s_wfinite[kWaves];
  __shared__ uint32_t s_wnonfinite[kWaves];
  __shared__ uint32_t s_wbest[kWaves];
  __shared__ uint32_t s_tau;
  __shared__ uint32_t s_count;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t row = blockIdx.y;
  const int chunk = blockIdx.x;
  const gs_row_config cfg = a.configs[row];
  const Plan plan = plan_row(cfg);
  if (plan.route == kRouteExact) return;
  const bool greedy = plan.route == kRouteGreedy;

  const int64_t gbase = (int64_t)chunk * kChunk;
  const int n_valid = (int)((int64_t)a.vocab - gbase < kChunk ? (int64_t)a.vocab - gbase : kChunk);
  const int32_t slot = cfg.mask_slot;
  const bool constrained = slot >= 0 && slot < a.mask_slots;

  // -- ids handled by the finish kernel: penalty window and forced ids
  for (int i = tid; i < kChunk / 32; i += kScanThreads) s_special[i] = 0;
  if (tid == 0) s_count = 0;
  __syncthreads();
  {
    int64_t w0, w1;
    history_window(a, row, cfg, &w0, &w1);
    for (int64_t j = w0 + tid; j < w1; j += kScanThreads) {
      const int64_t loc = (int64_t)a.history_ids[j] - gbase;
      if (loc >= 0 && loc < n_valid) atomicOr(&s_special[loc >> 5], 1u << (loc & 31));
    }
    if (constrained && a.forced_offsets) {
      const int64_t f0 = a.forced_offsets[row], f1 = a.forced_offsets[row + 1];
      for (int64_t j = f0 + tid; j < f1; j += kScanThreads) {
        const int64_t loc = (int64_t)a.forced_ids[j] - gbase;
        if (loc >= 0 && loc < n_valid) atomicOr(&s_special[loc >> 5], 1u << (loc & 31));
      }
    }
  }
  __syncthreads();

  // -- load the chunk once; keep order-preserving keys in registers
  const In* rowp = (const In*)a.logits + row * a.row_stride + gbase;
  const uint32_t* maskp = constrained ? a.mask_table + (int64_t)slot * a.mask_words + (gbase >> 5) : nullptr;
  const bool use_cap = cfg.softcap > 0;
  const bool full = n_valid == kChunk && a.vector_ok;
  uint32_t key[kElemsPerThread];
  uint32_t nonfinite = 0;
#pragma unroll
  for (int v = 0; v < kLoads; ++v) {
    const int loc = (v * kScanThreads + tid) * kVec;
    float x[kVec];
    if (full) {
      VT::load(rowp + loc, x);
    } else {
#pragma unroll
      for (int j = 0; j < kVec; ++j) x[j] = loc + j < n_valid ? VT::one(rowp + loc + j) : 0.0f;
    }
    const uint32_t lanebits = (1u << kVec) - 1u;
    const uint32_t special = (s_special[loc >> 5] >> (loc & 31)) & lanebits;
    const uint32_t allowed =
        constrained && loc < n_valid ? (maskp[loc >> 5] >> (loc & 31)) & lanebits : lanebits;
#pragma unroll
    for (int j = 0; j < kVec; ++j) {
      float y = x[j];
      if (use_cap) y = gsm::softcap_f32(y, cfg.softcap);
      const bool valid = loc + j < n_valid && !((special >> j) & 1u);
      uint32_t k = ((allowed >> j) & 1u) ? f32_key(y) : kKeyNegInf;
      const bool bad = valid && ((allowed >> j) & 1u) && !(y < __builtin_inff());  // NaN or +inf
      nonfinite |= bad ? 1u : 0u;
      key[v * kVec + j] = valid ? k : 0u;
    }
  }

  // -- chunk maximum
  uint32_t tmax = 0;
#pragma unroll
  for (int e = 0; e < kElemsPerThread; ++e) tmax = key[e] > tmax ? key[e] : tmax;
  {
    const uint32_t wm = wave_max_u32(tmax);
    const uint32_t wn = wave_max_u32(nonfinite);
    if (lane == 0) { s_wmax[wave] = wm; s_wnonfinite[wave] = wn; }
  }
  __syncthreads();
  uint32_t cmax = 0, cnonfinite = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    cmax = s_wmax[w] > cmax ? s_wmax[w] : cmax;
    cnonfinite |= s_wnonfinite[w];
  }

  // -- partial normaliser: sum e^((l - lmax)/T) over finite logits
  uint32_t nfin = 0;
  double sum = 0.0;
  const bool has_finite = cmax > kKeyNegInf && cmax < kKeyPosInf;
  if (!greedy && has_finite && !cnonfinite) {
    const double lmax = (double)key_f32(cmax);
    const double inv_t = 1.0 / cfg.temperature;
#pragma unroll
    for (int e = 0; e < kElemsPerThread; ++e) {
      if (key[e] > kKeyNegInf) {
        const double d = ((double)key_f32(key[e]) - lmax) * inv_t;
        if (d > -64.0) sum += gsm::exp_neg_fast(d, c_exp2_table);
      }
    }
  }
#pragma unroll
  for (int e = 0; e < kElemsPerThread; ++e) nfin += key[e] > kKeyNegInf ? 1u : 0u;

  if (greedy) {
    // argmax keeps the first maximum (sampling.ts:92-96): the lowest id whose key is cmax
    uint32_t best = 0xFFFFFFFFu;
#pragma unroll
    for (int e = 0; e < kElemsPerThread; ++e) {
      const int v = e / kVec, j = e % kVec;
      const uint32_t id = (uint32_t)(gbase + (v * kScanThreads + tid) * kVec + j);
      if (key[e] == cmax && cmax != 0u && id < best) best = id;
    }
    for (int m = 32; m > 0; m >>= 1) {
      const uint32_t o = shfl_xor_u32(best, m);
      best = o < best ? o : best;
    }
    if (lane == 0) s_wbest[wave] = best;
    __syncthreads();
    if (tid == 0) {
      uint32_t b = 0xFFFFFFFFu;
      for (int w = 0; w < kWaves; ++w) b = s_wbest[w] < b ? s_wbest[w] : b;
      const bool any = b != 0xFFFFFFFFu;
      if (any) a.lists[((int64_t)row * a.n_chunks + chunk) * kGatherCap] = pack_entry(cmax, b);
      ChunkStat st;
      st.sum = 0.0;
      st.max_key = cmax;
      st.n_list = any ? 1u : 0u;
      st.n_finite = 0;
      st.threshold = cmax;
      st.truncated = 0;
      st.flags = cnonfinite ? kChunkNonFinite : 0u;
      a.stats[row * a.n_chunks + chunk] = st;
    }
    return;
  }

  // -- tau: the depth-th largest lane maximum over the workgroup
  uint32_t lmaxk = 0;
#pragma unroll
  for (int e = 0; e < kElemsPerThread; ++e) {
    const uint32_t k = key[e] > kKeyNegInf ? key[e] : 0u;
    lmaxk = k > lmaxk ? k : lmaxk;
  }
  {
    const uint64_t mine = ((uint64_t)lmaxk << 32) | (uint32_t)(kScanThreads - tid);
    const uint64_t sorted = wave_sort_desc(mine, lane);
    s_lanemax[wave][lane] = sorted;
    const double ws = wave_sum_f64(sum);
    const uint32_t wf = wave_sum_u32(nfin);
    if (lane == 0) { s_wsum[wave] = ws; s_wfinite[wave] = wf; }
  }
  __syncthreads();
  {
    // rank of this workgroup entry among the 4 sorted wave lists
    const uint64_t c = s_lanemax[wave][lane];
    uint32_t rank = lane;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      if (w == wave) continue;
      int lo = 0, hi = 64;
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (s_lanemax[w][mid] > c) lo = mid + 1; else hi = mid;
      }
      rank += lo;
    }
    if (rank == (uint32_t)(plan.depth - 1)) s_tau = (uint32_t)(c >> 32);
  }
  __syncthreads();
  const uint32_t tau = s_tau;
  const uint32_t thr = tau > kKeyNegInf ? tau : kKeyNegInf + 1u;

  // -- gather every finite key >= thr (wave-aggregated LDS append)
  uint32_t mine = 0;
#pragma unroll
  for (int e = 0; e < kElemsPerThread; ++e) mine += key[e] >= thr ? 1u : 0u;
  const uint32_t incl = wave_scan_u32(mine, lane);
  uint32_t wbase = 0;
  if (lane == 63 && incl) wbase = atomicAdd(&s_count, incl);
  wbase = (uint32_t)__shfl((int)wbase, 63, 64);
  uint32_t pos = wbase + incl - mine;
  if (mine) {
#pragma unroll
    for (int e = 0; e < kElemsPerThread; ++e) {
      if (key[e] >= thr) {
        const int v = e / kVec, j = e % kVec;
        const uint32_t id = (uint32_t)(gbase + (v * kScanThreads + tid) * kVec + j);
        if (pos < (uint32_t)kGatherCap) s_list[pos] = pack_entry(key[e], id);
        ++pos;
      }
    }
  }
  __syncthreads();

  const uint32_t count = s_count;
  const uint32_t n_list = count < (uint32_t)kGatherCap ? count : (uint32_t)kGatherCap;
  uint64_t* out = a.lists + ((int64_t)row * a.n_chunks + chunk) * kGatherCap;
  for (uint32_t i = tid; i < n_list; i += kScanThreads) out[i] = s_list[i];
  if (tid == 0) {
    double csum = 0.0;
    uint32_t cfin = 0;
    for (int w = 0; w < kWaves; ++w) { csum += s_wsum[w]; cfin += s_wfinite[w]; }
    ChunkStat st;
    st.sum = csum;
    st.max_key = cmax;
    st.n_list = n_list;
    st.n_finite = cfin;
    st.threshold = thr;
    st.truncated = cfin > count ? 1u : 0u;
    st.flags = (count > (uint32_t)kGatherCap ? kChunkOverflow : 0u) | (cnonfinite ? kChunkNonFinite : 0u);
    a.stats[row * a.n_chunks + chunk] = st;
  }
}

}  // namespace

void launch_scan(const SampleArgs& a, hipStream_t s) {
  dim3 grid(a.n_chunks, a.rows);
  if (a.dtype == GS_BF16) hipLaunchKernelGGL(scan_kernel<uint16_t>, grid, dim3(kScanThreads), 0, s, a);
  else hipLaunchKernelGGL(scan_kernel<float>, grid, dim3(kScanThreads), 0, s, a);
}

}  // namespace gs
