// Row replay of the exact path: replays the reference sampler
// (src/runtime/sampling.ts:18-96) operation by operation for the rows the
// one-pass path could not settle -- rows needing candidates outside the
// complete region, decisions within the 1e-10 margin, typical-p, top-k above
// 64, pure multinomial draws, non-finite logits, or rows forced here.
//
// One 1024-thread workgroup replays one row with a scratch slot it holds
// alone: the finish kernel's own workgroup when the row has a slot (row <
// slots), else a workgroup of the exact kernel, which walks a device queue of
// the remaining rows. Per row it builds the binary64 values of all logits,
// sorts them by (value desc, id asc) with a bitonic sort (LDS tiles of 4096
// entries, global-memory stages above that), and then evaluates every sum,
// cut and the draw sequentially in list order on one lane, through LDS
// staging, so that each rounding is the reference's.
#pragma once
#include "gs_internal.h"

namespace gs {
namespace exact {
namespace {

constexpr int kWaves = kExactThreads / 64;

struct Scratch {
  uint64_t* key;   // [cap]
  uint32_t* id;    // [cap]
  double* prob;    // [cap]
  uint64_t* skey;  // [cap] sort keys of the candidate reorderings
  uint32_t* sidx;  // [cap]
  uint32_t* order; // [cap] candidate list as positions into key/id/prob
};

__device__ inline Scratch scratch_at(const SampleArgs& a, int64_t slot) {
  uint8_t* base = a.exact_scratch + slot * a.exact_slot_bytes;
  const int64_t cap = a.exact_capacity;
  Scratch s;
  s.key = (uint64_t*)base;
  s.prob = (double*)(base + 8 * cap);
  s.skey = (uint64_t*)(base + 16 * cap);
  s.id = (uint32_t*)(base + 24 * cap);
  s.sidx = (uint32_t*)(base + 28 * cap);
  s.order = (uint32_t*)(base + 32 * cap);
  return s;
}

struct Lds {  // the replay's LDS (a finish workgroup reuses its own for it)
  uint64_t tkey[kExactTile];
  uint32_t tid_[kExactTile];
  double stage[kExactTile];
  double wtmp[kWaves];
  uint32_t wtmp_u[kWaves];
  uint64_t wtmp_k[kWaves];
  uint32_t row;
  uint32_t flag;
  uint32_t count;
  int32_t legal;   // legal ids of a constrained row
  double result_p;
  int32_t result_token;
  uint32_t result_flags;
  double dtmp;
  double bcast_d[2];
  int64_t bcast_n;
};

__device__ __forceinline__ bool before(uint64_t ka, uint32_t ia, uint64_t kb, uint32_t ib) {
  return ka > kb || (ka == kb && ia < ib);
}

// Bitonic sort of (key desc, idx asc) pairs in global memory, n a power of two.
__device__ void sort_pairs(Lds& L, uint64_t* key, uint32_t* idx, int64_t n) {
  const int tid = threadIdx.x;
  const int64_t tile = n < kExactTile ? n : kExactTile;
  auto lds_stages = [&](int64_t t0, int64_t k_from, int64_t k_to, int64_t j_from) {
    // stages (k, j) with j < tile on the tile starting at t0
    for (int64_t i = tid; i < tile; i += kExactThreads) { L.tkey[i] = key[t0 + i]; L.tid_[i] = idx[t0 + i]; }
    __syncthreads();
    for (int64_t k = k_from; k <= k_to; k <<= 1) {
      for (int64_t j = (k == k_from ? j_from : k >> 1); j > 0; j >>= 1) {
        for (int64_t i = tid; i < tile; i += kExactThreads) {
          const int64_t p = i ^ j;
          if (p > i) {
            const bool desc = ((t0 + i) & k) == 0;
            const bool swap = desc ? before(L.tkey[p], L.tid_[p], L.tkey[i], L.tid_[i])
                                   : before(L.tkey[i], L.tid_[i], L.tkey[p], L.tid_[p]);
            if (swap) {
              const uint64_t tk = L.tkey[i]; L.tkey[i] = L.tkey[p]; L.tkey[p] = tk;
              const uint32_t ti = L.tid_[i]; L.tid_[i] = L.tid_[p]; L.tid_[p] = ti;
            }
          }
        }
        __syncthreads();
      }
    }
    for (int64_t i = tid; i < tile; i += kExactThreads) { key[t0 + i] = L.tkey[i]; idx[t0 + i] = L.tid_[i]; }
    __syncthreads();
  };
  for (int64_t t0 = 0; t0 < n; t0 += tile) lds_stages(t0, 2, tile, 1);
  for (int64_t k = tile << 1; k <= n; k <<= 1) {
    for (int64_t j = k >> 1; j >= tile; j >>= 1) {
      for (int64_t i = tid; i < n; i += kExactThreads) {
        const int64_t p = i ^ j;
        if (p > i) {
          const bool desc = (i & k) == 0;
          const uint64_t ki = key[i], kp = key[p];
          const uint32_t ii = idx[i], ip = idx[p];
          const bool swap = desc ? before(kp, ip, ki, ii) : before(ki, ii, kp, ip);
          if (swap) { key[i] = kp; key[p] = ki; idx[i] = ip; idx[p] = ii; }
        }
      }
      __syncthreads();
    }
    for (int64_t t0 = 0; t0 < n; t0 += tile) lds_stages(t0, k, k, tile >> 1);
  }
}

__device__ __forceinline__ int64_t pow2_ge(int64_t n) {
  int64_t p = 1;
  while (p < n) p <<= 1;
  return p;
}

// The one-lane walks below read their LDS values kSeqBatch at a time, ahead
// of the additions that consume them in order, so a walk runs at the
// latency of its binary64 additions instead of one LDS round trip per value.
constexpr int kSeqBatch = 32;

// acc + st[0] + ... + st[m-1], left to right, on the calling lane.
__device__ __forceinline__ double seq_sum_lds(const double* st, int64_t m, double acc) {
  int64_t i = 0;
  for (; i + kSeqBatch <= m; i += kSeqBatch) {
    double v[kSeqBatch];
#pragma unroll
    for (int k = 0; k < kSeqBatch; ++k) v[k] = st[i + k];
#pragma unroll
    for (int k = 0; k < kSeqBatch; ++k) acc = acc + v[k];
  }
  for (; i < m; ++i) acc = acc + st[i];
  return acc;
}

// Sequential left-to-right sum of prob[order[i]] for i < n, on one lane.
__device__ double sequential_sum(Lds& L, const double* prob, const uint32_t* order, int64_t n, bool identity) {
  double acc = 0.0;
  for (int64_t b = 0; b < n; b += kExactTile) {
    const int64_t m = n - b < kExactTile ? n - b : kExactTile;
    for (int64_t i = threadIdx.x; i < m; i += kExactThreads) L.stage[i] = prob[identity ? b + i : order[b + i]];
    __syncthreads();
    if (threadIdx.x == 0) {
      acc = seq_sum_lds(L.stage, m, acc);
      L.dtmp = acc;
    }
    __syncthreads();
    acc = L.dtmp;
    __syncthreads();
  }
  return acc;
}

// cumulativeCut (sampling.ts:82-90): number of items kept. Lane 0 of the
// workgroup walks the list; the running sum, the previous sum and the count
// are broadcast through LDS after every block so that all threads leave with
// the same values (every loop below with a barrier depends on them).
__device__ int64_t cumulative_cut(Lds& L, const double* prob, const uint32_t* order, int64_t n, double threshold,
                                  double* at_cut, double* before_cut) {
  double cum = 0.0, prev = 0.0;
  int64_t end = 0;
  bool done = false;
  for (int64_t b = 0; b < n && !done; b += kExactTile) {
    const int64_t m = n - b < kExactTile ? n - b : kExactTile;
    for (int64_t i = threadIdx.x; i < m; i += kExactThreads) L.stage[i] = prob[order[b + i]];
    __syncthreads();
    if (threadIdx.x == 0) {
      int64_t i = 0;
      bool stop = false;
      while (i < m && !stop) {
        // the next kSeqBatch values (reads past m stay inside the stage and
        // are not used)
        double v[kSeqBatch];
#pragma unroll
        for (int k = 0; k < kSeqBatch; ++k) v[k] = L.stage[(i + k) & (kExactTile - 1)];
        const int64_t cnt = m - i < kSeqBatch ? m - i : kSeqBatch;
#pragma unroll
        for (int k = 0; k < kSeqBatch; ++k) {
          if (k < cnt && !stop) {
            prev = cum;
            cum += v[k];
            ++end;
            if (!(end < n && cum < threshold)) stop = true;
          }
        }
        i += cnt;
      }
      L.flag = stop ? 1u : 0u;
      L.bcast_d[0] = cum;
      L.bcast_d[1] = prev;
      L.bcast_n = end;
    }
    __syncthreads();
    done = L.flag != 0;
    cum = L.bcast_d[0];
    prev = L.bcast_d[1];
    end = L.bcast_n;
    __syncthreads();
  }
  *at_cut = cum;
  *before_cut = prev;
  return end < 1 ? 1 : end;
}

// Replays row `row` on the calling workgroup (all kExactThreads threads),
// with the scratch S of a slot it holds alone; flags_in: the reasons the row
// came here (GS_FLAG_NEAR_TIE / GS_FLAG_NONFINITE), kept in its result flags.
__device__ __noinline__ void process_row(const SampleArgs& a, Lds& L, Scratch S, int64_t row, uint32_t flags_in) {
  const int tid = threadIdx.x;
  const gs_row_config cfg = a.configs[row];
  const bool greedy = cfg.temperature == 0;
  const int32_t slot = cfg.mask_slot;
  const bool constrained = slot >= 0 && slot < a.mask_slots;
  const int64_t V = a.vocab;
  const int64_t N = pow2_ge(V);
  const double T = cfg.temperature;

  // ---- values of every logit (masking, then penalties on the distinct window
  // ids). Window counts and forced kinds are kept per vocabulary id in the
  // slot's scratch (sidx and order are free until the candidate reorderings
  // below), so a window of any length and any number of distinct ids is
  // counted exactly (sampling.ts:22-30).
  uint32_t* counts = S.sidx;
  uint32_t* kinds = S.order;
  for (int64_t i = tid; i < V; i += kExactThreads) { counts[i] = 0; kinds[i] = 0; }
  if (tid == 0) L.legal = 0;
  __syncthreads();
  {
    int64_t w0, w1;
    history_window(a, row, cfg, &w0, &w1);
    for (int64_t j = w0 + tid; j < w1; j += kExactThreads) {
      const int32_t id = a.history_ids[j];
      if (id >= 0 && id < a.vocab) atomicAdd(&counts[id], 1u);
    }
    if (constrained && a.forced_offsets) {
      const int64_t f0 = a.forced_offsets[row], f1 = a.forced_offsets[row + 1];
      for (int64_t j = f0 + tid; j < f1; j += kExactThreads) {
        const int32_t id = a.forced_ids[j];
        if (id >= 0 && id < a.vocab) atomicOr(&kinds[id], (uint32_t)a.forced_kinds[j] & 3u);
      }
    }
  }
  __syncthreads();
  {
    int32_t legal = 0;  // legal ids this thread saw (constrained rows)
    for (int64_t i = tid; i < N; i += kExactThreads) {
      if (i < V) {
        float x = load_logit(a, row, i);
        if (cfg.softcap > 0) x = softcap_call(x, cfg.softcap);
        const uint32_t count = counts[i], kd = kinds[i];
        bool allowed = true;
        if (constrained) {
          // selectConstrainedToken's legal set (gemma-session.ts:1305-1329):
          // termination ids only when accepting, extra ids always, the rest by
          // the mask
          allowed = (kd & GS_FORCED_TERMINATION) ? cfg.accepting != 0
                                                  : ((kd & GS_FORCED_EXTRA) != 0 || mask_allows(a, slot, i));
          legal += allowed ? 1 : 0;
        }
        double l = allowed ? (double)x : -__builtin_inf();
        if (count > 0) {
          l = l < 0 ? l * cfg.repetition_penalty : l / cfg.repetition_penalty;
          l -= cfg.presence_penalty + (double)count * cfg.frequency_penalty;
        }
        S.key[i] = f64_key(greedy ? l : l / T);
        S.id[i] = (uint32_t)i;
      } else {
        S.key[i] = 0;
        S.id[i] = 0xFFFFFFFFu;
      }
    }
    if (constrained) {
      legal = (int32_t)wave_sum_u32((uint32_t)legal);
      if ((tid & 63) == 0 && legal) atomicAdd(&L.legal, legal);
    }
  }
  __syncthreads();
  if (constrained && L.legal <= 0) {
    // no legal id at all (gemma-session.ts:1322-1326)
    if (tid == 0) {
      a.results[row].token = -1;
      a.results[row].flags = flags_in | GS_FLAG_EXACT_PATH | GS_FLAG_DEAD_END;
      a.results[row].probability = 0.0;
    }
    __syncthreads();
    return;
  }

  if (greedy) {
    // argmax (sampling.ts:92-96): first index whose value beats every earlier
    // one under `>`; NaN never wins, and a NaN at index 0 is never replaced
    uint64_t kbest = 0;
    for (int64_t i = tid; i < V; i += kExactThreads) {
      const double v = key_f64(S.key[i]);
      if (v == v && S.key[i] > kbest) kbest = S.key[i];
    }
    for (int m = 32; m > 0; m >>= 1) { const uint64_t o = shfl_xor_u64(kbest, m); kbest = o > kbest ? o : kbest; }
    if ((tid & 63) == 0) L.wtmp_k[tid >> 6] = kbest;
    __syncthreads();
    kbest = 0;
    for (int w = 0; w < kWaves; ++w) kbest = L.wtmp_k[w] > kbest ? L.wtmp_k[w] : kbest;
    uint32_t ibest = 0xFFFFFFFFu;
    for (int64_t i = tid; i < V; i += kExactThreads) {
      if (S.key[i] == kbest && (uint32_t)i < ibest) ibest = (uint32_t)i;
    }
    for (int m = 32; m > 0; m >>= 1) { const uint32_t o = shfl_xor_u32(ibest, m); ibest = o < ibest ? o : ibest; }
    if ((tid & 63) == 0) L.wtmp_u[tid >> 6] = ibest;
    __syncthreads();
    if (tid == 0) {
      uint32_t b = 0xFFFFFFFFu;
      for (int w = 0; w < kWaves; ++w) b = L.wtmp_u[w] < b ? L.wtmp_u[w] : b;
      const double v0 = key_f64(S.key[0]);
      if (v0 != v0 || b == 0xFFFFFFFFu) b = 0;
      a.results[row].token = (int32_t)b;
      a.results[row].flags = flags_in | GS_FLAG_GREEDY | GS_FLAG_EXACT_PATH;
      a.results[row].probability = 1.0;
    }
    __syncthreads();
    return;
  }

  // ---- stable descending sort (sampling.ts:33-35)
  sort_pairs(L, S.key, S.id, N);

  // ---- probabilities (sampling.ts:36-42), the total summed in list order
  const double M = key_f64(S.key[0]);
  for (int64_t i = tid; i < V; i += kExactThreads) S.prob[i] = gsm::js_exp(key_f64(S.key[i]) - M);
  __syncthreads();
  const double total = sequential_sum(L, S.prob, nullptr, V, true);
  for (int64_t i = tid; i < V; i += kExactThreads) S.prob[i] = S.prob[i] / total;
  __syncthreads();

  // ---- top-k (sampling.ts:44)
  int64_t n = cfg.top_k > 0 ? (cfg.top_k < V ? cfg.top_k : V) : V;
  for (int64_t i = tid; i < n; i += kExactThreads) S.order[i] = (uint32_t)i;
  __syncthreads();

  // ---- min-p (sampling.ts:45-48): stable compaction of p >= p0 * minP
  if (cfg.min_p > 0) {
    const double floor_p = S.prob[S.order[0]] * cfg.min_p;
    // chunks of 1024 in order: wave/block prefix of keep flags
    uint32_t out = 0;
    for (int64_t b = 0; b < n; b += kExactThreads) {
      const int64_t i = b + tid;
      const uint32_t pos = i < n ? S.order[i] : 0;
      const uint32_t keep = (i < n && S.prob[pos] >= floor_p) ? 1u : 0u;
      const int lane = tid & 63, wave = tid >> 6;
      const uint32_t incl = wave_scan_u32(keep);
      if (lane == 63) L.wtmp_u[wave] = incl;
      __syncthreads();
      uint32_t off = 0, tot = 0;
      for (int w = 0; w < kWaves; ++w) { if (w < wave) off += L.wtmp_u[w]; tot += L.wtmp_u[w]; }
      __syncthreads();
      if (keep) S.sidx[out + off + incl - 1] = pos;
      out += tot;
    }
    __syncthreads();
    for (int64_t i = tid; i < out; i += kExactThreads) S.order[i] = S.sidx[i];
    __syncthreads();
    n = out;
    if (n == 0) {
      if (tid == 0) {
        a.results[row].token = -1;
        a.results[row].flags = flags_in | GS_FLAG_EXACT_PATH | GS_FLAG_EMPTY_CANDIDATES;
        a.results[row].probability = 0.0;
      }
      __syncthreads();
      return;
    }
  }

  // ---- typical-p (sampling.ts:49-55)
  if (cfg.typical_p < 1) {
    // entropy = sum - p * log(p), left to right
    double entropy = 0.0;
    for (int64_t b = 0; b < n; b += kExactTile) {
      const int64_t m = n - b < kExactTile ? n - b : kExactTile;
      // the terms p * log(p) in parallel (each rounded as the reference
      // rounds it), then subtracted left to right on one lane
      double* terms = (double*)L.tkey;
      for (int64_t i = tid; i < m; i += kExactThreads) {
        const double pi = S.prob[S.order[b + i]];
        terms[i] = pi * gsm::js_log(pi);
      }
      __syncthreads();
      if (tid == 0) {
        int64_t i = 0;
        for (; i + kSeqBatch <= m; i += kSeqBatch) {
          double v[kSeqBatch];
#pragma unroll
          for (int k = 0; k < kSeqBatch; ++k) v[k] = terms[i + k];
#pragma unroll
          for (int k = 0; k < kSeqBatch; ++k) entropy = entropy - v[k];
        }
        for (; i < m; ++i) entropy = entropy - terms[i];
        L.dtmp = entropy;
      }
      __syncthreads();
      entropy = L.dtmp;
      __syncthreads();
    }
    const int64_t n2 = pow2_ge(n);
    if (entropy == entropy) {
      // stable ascending sort by surprise = |-log(p) - entropy|
      for (int64_t i = tid; i < n2; i += kExactThreads) {
        if (i < n) {
          const double p = S.prob[S.order[i]];
          const double surprise = fabs(-gsm::js_log(p) - entropy);
          S.skey[i] = ~f64_key(surprise);
          S.sidx[i] = (uint32_t)i;
        } else {
          S.skey[i] = 0;
          S.sidx[i] = 0xFFFFFFFFu;
        }
      }
      __syncthreads();
      sort_pairs(L, S.skey, S.sidx, n2);
      // apply the permutation: order'[i] = order[sidx[i]] (through prob-free staging)
      for (int64_t i = tid; i < n; i += kExactThreads) S.skey[i] = S.order[S.sidx[i]];
      __syncthreads();
      for (int64_t i = tid; i < n; i += kExactThreads) S.order[i] = (uint32_t)S.skey[i];
      __syncthreads();
    }
    double at, before_cut;
    n = cumulative_cut(L, S.prob, S.order, n, cfg.typical_p, &at, &before_cut);
    // stable descending sort by probability
    bool any_nan = false;
    for (int64_t i = tid; i < n; i += kExactThreads) {
      const double p = S.prob[S.order[i]];
      if (p != p) any_nan = true;
    }
    if (tid == 0) L.flag = 0;
    __syncthreads();
    if (any_nan) atomicOr(&L.flag, 1u);
    __syncthreads();
    const bool nan_probs = L.flag != 0;
    __syncthreads();
    if (!nan_probs) {
      const int64_t m2 = pow2_ge(n);
      for (int64_t i = tid; i < m2; i += kExactThreads) {
        if (i < n) {
          S.skey[i] = f64_key(S.prob[S.order[i]]);
          S.sidx[i] = (uint32_t)i;
        } else {
          S.skey[i] = 0;
          S.sidx[i] = 0xFFFFFFFFu;
        }
      }
      __syncthreads();
      sort_pairs(L, S.skey, S.sidx, m2);
      for (int64_t i = tid; i < n; i += kExactThreads) S.skey[i] = S.order[S.sidx[i]];
      __syncthreads();
      for (int64_t i = tid; i < n; i += kExactThreads) S.order[i] = (uint32_t)S.skey[i];
      __syncthreads();
    }
  }

  // ---- top-p (sampling.ts:56)
  uint32_t tie = 0;
  if (cfg.top_p < 1) {
    double at, before_cut;
    const int64_t kept = cumulative_cut(L, S.prob, S.order, n, cfg.top_p, &at, &before_cut);
    if ((at >= cfg.top_p && at - cfg.top_p <= kTieReport * cfg.top_p) ||
        (kept > 1 && cfg.top_p - before_cut <= kTieReport * cfg.top_p)) {
      tie = GS_FLAG_TOPP_TIE;
    }
    n = kept;
  }

  // ---- draw (sampling.ts:58-64)
  const double ctotal = sequential_sum(L, S.prob, S.order, n, false);
  const double u = cfg.rng_mode == GS_RNG_EXPLICIT ? cfg.uniform : gsm::mulberry32_draw(cfg.seed, cfg.draw_index);
  double cursor = u * ctotal;
  if (tid == 0) L.result_token = -1;
  for (int64_t b = 0; b < n; b += kExactTile) {
    const int64_t m = n - b < kExactTile ? n - b : kExactTile;
    for (int64_t i = tid; i < m; i += kExactThreads) L.stage[i] = S.prob[S.order[b + i]];
    __syncthreads();
    if (tid == 0 && L.result_token < 0) {
      int64_t hit = -1;
      for (int64_t i = 0; i < m && hit < 0; i += kSeqBatch) {
        double v[kSeqBatch];
#pragma unroll
        for (int k = 0; k < kSeqBatch; ++k) v[k] = L.stage[(i + k) & (kExactTile - 1)];
        const int64_t cnt = m - i < kSeqBatch ? m - i : kSeqBatch;
#pragma unroll
        for (int k = 0; k < kSeqBatch; ++k) {
          if (k < cnt && hit < 0) {
            cursor -= v[k];
            if (cursor <= 0) hit = i + k;
          }
        }
      }
      if (hit >= 0) {
        L.result_token = (int32_t)S.id[S.order[b + hit]];
        L.result_p = L.stage[hit];
      }
      L.dtmp = cursor;
    }
    __syncthreads();
    cursor = L.dtmp;
    const bool found = L.result_token >= 0;
    __syncthreads();
    if (found) break;
  }
  if (tid == 0) {
    if (L.result_token < 0) {
      const uint32_t last = S.order[n - 1];
      L.result_token = (int32_t)S.id[last];
      L.result_p = S.prob[last];
    }
    a.results[row].token = L.result_token;
    a.results[row].flags = flags_in | GS_FLAG_EXACT_PATH | tie;
    a.results[row].probability = L.result_p;
  }
  __syncthreads();
}

}  // namespace
}  // namespace exact
}  // namespace gs
