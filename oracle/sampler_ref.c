/*
 * ORACLE — test infrastructure only (tests/, __graft_entry__.smoke(),
 * bench.py's cpu_baseline leg). Never part of the product path.
 *
 * CPU restatement of the reference's sampling stage, operation by operation,
 * so that every floating-point decision rounds exactly as the reference's
 * JavaScript does:
 *
 *   or_sample_token        src/runtime/sampling.ts:18-65 (sampleToken)
 *   or_token_log_prob      src/runtime/sampling.ts:67-80 (tokenLogProbability)
 *   or_draw                src/runtime/sampling.ts:3-16  (SeededRandom.next)
 *   or_dfa_legal_mask      src/runtime/constraints.ts:56-92 (legalTokenIds) for a
 *                          byte-level DFA: a token is legal iff every state
 *                          reached along its bytes exists and is viable
 *   or_viable_states       src/runtime/constraints.ts:300-322 (findViableStates)
 *   or_mask_logits         src/runtime/constraints.ts:159-173 (maskConstraintLogits)
 *   or_softcap_row         the engine's optional final-logit softcap
 *                          cap*tanh(x/cap) (jsmath.h softcap_f32); the
 *                          reference declares the cap but never applies it,
 *                          so it is pinned by closed-form tests only
 *
 * The steps kept alike (and why): the sampler's order of operations is the
 * reference's because the token ids must be bit-exact — widening to f64
 * (Array.from, :20), distinct-token counts in the window (:22-25), the penalty
 * formula (:28-29), greedy argmax with the first maximum winning (:31,92-96),
 * the stable descending sort (:33-35), sequential exp/sum/normalise in sorted
 * order (:36-42), the filter order top-k, min-p, typical-p, top-p (:44-56),
 * cumulativeCut's do-while (:82-90) and the cursor walk (:58-64).
 *
 * A stable sort on (value desc, id asc) is what V8's stable Array.sort gives
 * for any finite or infinite keys (the comparator's NaN for equal infinities
 * reads as "equal"). Inputs holding NaN are outside the contract.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "jsmath.h"

typedef struct or_config {
  double temperature;
  double top_p;
  double min_p;
  double typical_p;
  double repetition_penalty;
  double frequency_penalty;
  double presence_penalty;
  int32_t top_k;
  int32_t repetition_window;
} or_config;

/* Everything the sampler decided, for tie accounting in the tests. */
typedef struct or_trace {
  double maximum;        /* scaled[0].logit */
  double total;          /* sequential sum of exp(logit - maximum) */
  double probability;    /* item.probability of the chosen token (1 for greedy) */
  double cumulative_at_cut;   /* top-p: cumulative where the do-while stopped */
  double cumulative_before_cut;
  double cursor_start;   /* random() * candidateTotal */
  double candidate_total;
  int64_t candidates;    /* candidate count that entered the draw */
  int32_t greedy;        /* 1 when temperature == 0 */
  int32_t fallback_last; /* 1 when the walk ran off the end */
} or_trace;

typedef struct item {
  int32_t token;
  int32_t pad;
  double logit;
  double probability;
  double surprise;
} item;

/* ---- stable merge sort with a caller comparator (<0: a first) ---------- */
typedef int (*cmp_fn)(const item*, const item*);

static void merge_sort(item* a, item* tmp, int64_t n, cmp_fn cmp) {
  if (n < 2) return;
  if (n <= 16) {  /* insertion sort is stable */
    for (int64_t i = 1; i < n; ++i) {
      item x = a[i];
      int64_t j = i - 1;
      while (j >= 0 && cmp(&x, &a[j]) < 0) { a[j + 1] = a[j]; --j; }
      a[j + 1] = x;
    }
    return;
  }
  int64_t h = n / 2;
  merge_sort(a, tmp, h, cmp);
  merge_sort(a + h, tmp, n - h, cmp);
  int64_t i = 0, j = h, k = 0;
  while (i < h && j < n) {
    if (cmp(&a[j], &a[i]) < 0) tmp[k++] = a[j++];
    else tmp[k++] = a[i++];
  }
  while (i < h) tmp[k++] = a[i++];
  while (j < n) tmp[k++] = a[j++];
  memcpy(a, tmp, (size_t)n * sizeof(item));
}

/* (right.logit - left.logit) < 0  <=>  left.logit > right.logit */
static int by_logit_desc(const item* l, const item* r) {
  double d = r->logit - l->logit;
  return d < 0 ? -1 : (d > 0 ? 1 : 0);
}
static int by_surprise_asc(const item* l, const item* r) {
  double d = l->surprise - r->surprise;
  return d < 0 ? -1 : (d > 0 ? 1 : 0);
}
static int by_probability_desc(const item* l, const item* r) {
  double d = r->probability - l->probability;
  return d < 0 ? -1 : (d > 0 ? 1 : 0);
}

/* Fast path for the big sort: a total order on (logit desc, token asc) is
 * exactly the stable order, and qsort on it is much quicker than recursion. */
static int qsort_logit_desc(const void* a, const void* b) {
  const item* l = (const item*)a;
  const item* r = (const item*)b;
  if (l->logit > r->logit) return -1;
  if (l->logit < r->logit) return 1;
  return (l->token > r->token) - (l->token < r->token);
}

/* cumulativeCut: do { cum += p[end++] } while (end < n && cum < threshold) */
static int64_t cumulative_cut(const item* items, int64_t n, double threshold,
                              double* cum_at, double* cum_before) {
  double cumulative = 0.0, before = 0.0;
  int64_t end = 0;
  do {
    before = cumulative;
    cumulative += items[end].probability;
    end += 1;
  } while (end < n && cumulative < threshold);
  if (cum_at) *cum_at = cumulative;
  if (cum_before) *cum_before = before;
  return end < 1 ? 1 : end;
}

typedef struct count_entry { int32_t token; int32_t count; } count_entry;
static int by_token(const void* a, const void* b) {
  int32_t x = ((const count_entry*)a)->token, y = ((const count_entry*)b)->token;
  return (x > y) - (x < y);
}

/* Penalties (sampling.ts:21-30) applied in place to the f64 logits. */
static void apply_penalties(double* logits, int64_t V, const int32_t* history, int64_t hist_len,
                            const or_config* cfg) {
  if (cfg->repetition_window == 0 || hist_len == 0) return;
  int64_t start = hist_len - cfg->repetition_window;
  if (start < 0) start = 0;
  int64_t n = hist_len - start;
  count_entry* e = (count_entry*)malloc((size_t)n * sizeof(count_entry));
  for (int64_t i = 0; i < n; ++i) { e[i].token = history[start + i]; e[i].count = 1; }
  qsort(e, (size_t)n, sizeof(count_entry), by_token);
  int64_t i = 0;
  while (i < n) {
    int64_t j = i;
    while (j < n && e[j].token == e[i].token) ++j;
    int32_t token = e[i].token;
    double count = (double)(j - i);
    if (token >= 0 && token < V) {
      double l = logits[token];
      l = l < 0 ? l * cfg->repetition_penalty : l / cfg->repetition_penalty;
      l -= cfg->presence_penalty + count * cfg->frequency_penalty;
      logits[token] = l;
    }
    i = j;
  }
  free(e);
}

/* Returns the chosen token, or -1 where the reference would throw
 * (empty logits -> "Cannot sample empty logits"; an empty candidate list
 * after min-p, which the reference dereferences and fails on). */
int32_t or_sample_token(const double* raw, int64_t V, const int32_t* history, int64_t hist_len,
                        const or_config* cfg, double uniform, or_trace* trace) {
  or_trace local;
  if (!trace) trace = &local;
  memset(trace, 0, sizeof(*trace));
  if (V <= 0) return -1;
  double* logits = (double*)malloc((size_t)V * sizeof(double));
  memcpy(logits, raw, (size_t)V * sizeof(double));
  apply_penalties(logits, V, history, hist_len, cfg);

  if (cfg->temperature == 0) {
    int64_t best = 0;
    for (int64_t i = 1; i < V; ++i) if (logits[i] > logits[best]) best = i;
    trace->greedy = 1;
    trace->probability = 1.0;
    trace->candidates = 1;
    free(logits);
    return (int32_t)best;
  }

  item* scaled = (item*)malloc((size_t)V * sizeof(item));
  for (int64_t i = 0; i < V; ++i) {
    scaled[i].token = (int32_t)i;
    scaled[i].logit = logits[i] / cfg->temperature;
    scaled[i].probability = 0;
    scaled[i].surprise = 0;
  }
  free(logits);
  int has_nan = 0;
  for (int64_t i = 0; i < V; ++i) has_nan |= isnan(scaled[i].logit);
  if (!has_nan) {
    qsort(scaled, (size_t)V, sizeof(item), qsort_logit_desc);
  } else {
    item* tmp = (item*)malloc((size_t)V * sizeof(item));
    merge_sort(scaled, tmp, V, by_logit_desc);
    free(tmp);
  }

  double maximum = scaled[0].logit;
  double total = 0;
  for (int64_t i = 0; i < V; ++i) {
    scaled[i].probability = js_exp(scaled[i].logit - maximum);
    total += scaled[i].probability;
  }
  for (int64_t i = 0; i < V; ++i) scaled[i].probability /= total;
  trace->maximum = maximum;
  trace->total = total;

  item* cand = scaled;
  int64_t n = cfg->top_k > 0 ? (cfg->top_k < V ? cfg->top_k : V) : V;

  item* work = NULL;  /* owned copy once filters reorder or drop items */
  if (cfg->min_p > 0) {
    double threshold = cand[0].probability * cfg->min_p;
    work = (item*)malloc((size_t)n * sizeof(item));
    int64_t m = 0;
    for (int64_t i = 0; i < n; ++i) if (cand[i].probability >= threshold) work[m++] = cand[i];
    cand = work;
    n = m;
    if (n == 0) { free(scaled); free(work); return -1; }
  }
  if (cfg->typical_p < 1) {
    if (!work) {
      work = (item*)malloc((size_t)n * sizeof(item));
      memcpy(work, cand, (size_t)n * sizeof(item));
      cand = work;
    }
    double entropy = 0;
    for (int64_t i = 0; i < n; ++i) entropy = entropy - cand[i].probability * js_log(cand[i].probability);
    for (int64_t i = 0; i < n; ++i) cand[i].surprise = fabs(-js_log(cand[i].probability) - entropy);
    item* tmp = (item*)malloc((size_t)n * sizeof(item));
    merge_sort(cand, tmp, n, by_surprise_asc);
    n = cumulative_cut(cand, n, cfg->typical_p, NULL, NULL);
    merge_sort(cand, tmp, n, by_probability_desc);
    free(tmp);
  }
  trace->cumulative_at_cut = NAN;
  trace->cumulative_before_cut = NAN;
  if (cfg->top_p < 1) {
    n = cumulative_cut(cand, n, cfg->top_p, &trace->cumulative_at_cut, &trace->cumulative_before_cut);
  }

  double candidate_total = 0;
  for (int64_t i = 0; i < n; ++i) candidate_total = candidate_total + cand[i].probability;
  double cursor = uniform * candidate_total;
  trace->candidate_total = candidate_total;
  trace->cursor_start = cursor;
  trace->candidates = n;
  int32_t chosen = -1;
  for (int64_t i = 0; i < n; ++i) {
    cursor -= cand[i].probability;
    if (cursor <= 0) { chosen = cand[i].token; trace->probability = cand[i].probability; break; }
  }
  if (chosen < 0) {
    chosen = cand[n - 1].token;
    trace->probability = cand[n - 1].probability;
    trace->fallback_last = 1;
  }
  free(scaled);
  free(work);
  return chosen;
}

/* Same, for f32 logits widened exactly (Array.from over a Float32Array). */
int32_t or_sample_token_f32(const float* raw, int64_t V, const int32_t* history, int64_t hist_len,
                            const or_config* cfg, double uniform, or_trace* trace) {
  double* w = (double*)malloc((size_t)(V > 0 ? V : 1) * sizeof(double));
  for (int64_t i = 0; i < V; ++i) w[i] = (double)raw[i];
  int32_t t = or_sample_token(w, V, history, hist_len, cfg, uniform, trace);
  free(w);
  return t;
}

/* Math.max(a, b): NaN if either is NaN, and +0 wins over -0. */
static double js_max(double a, double b) {
  if (isnan(a) || isnan(b)) return NAN;
  if (a == b) return signbit(a) ? b : a;
  return a > b ? a : b;
}

/* tokenLogProbability: raw[t] - max - log(sum_i exp(raw[i] - max)), summed in id order. */
double or_token_log_prob(const double* raw, int64_t V, int64_t token) {
  if (token < 0 || token >= V) return NAN;
  double maximum = -INFINITY;
  for (int64_t i = 0; i < V; ++i) maximum = js_max(maximum, raw[i]);
  double denominator = 0;
  for (int64_t i = 0; i < V; ++i) denominator += js_exp(raw[i] - maximum);
  return raw[token] - maximum - js_log(denominator);
}

double or_exp(double x) { return js_exp(x); }
double or_log(double x) { return js_log(x); }

double or_draw(int64_t seed, uint64_t index) { return mulberry32_draw(seed, index); }

void or_softcap_row(const float* x, int64_t n, double cap, float* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = softcap_f32(x[i], cap);
}

void or_draws(int64_t seed, uint64_t first, int64_t count, double* out) {
  for (int64_t i = 0; i < count; ++i) out[i] = mulberry32_draw(seed, first + (uint64_t)i);
}

/* findViableStates: states from which some final state is reachable. */
void or_viable_states(const int32_t* next, int32_t n_states, const uint8_t* finals, uint8_t* viable) {
  memset(viable, 0, (size_t)n_states);
  for (int32_t s = 0; s < n_states; ++s) if (finals[s]) viable[s] = 1;
  int changed = 1;
  while (changed) {
    changed = 0;
    for (int32_t s = 0; s < n_states; ++s) {
      if (viable[s]) continue;
      for (int b = 0; b < 256; ++b) {
        int32_t t = next[(int64_t)s * 256 + b];
        if (t >= 0 && viable[t]) { viable[s] = 1; changed = 1; break; }
      }
    }
  }
}

/* Legal-token bitmask of one DFA state over a vocab CSR (offsets[V+1], bytes). */
void or_dfa_legal_mask(const int32_t* next, const uint8_t* viable, int32_t n_states,
                       const int64_t* offsets, const uint8_t* bytes, int64_t V,
                       int32_t state, uint32_t* mask) {
  int64_t words = (V + 31) / 32;
  memset(mask, 0, (size_t)words * 4);
  (void)n_states;
  for (int64_t t = 0; t < V; ++t) {
    int64_t a = offsets[t], b = offsets[t + 1];
    if (b <= a) continue;
    int32_t s = state;
    int ok = 1;
    for (int64_t i = a; i < b; ++i) {
      s = next[(int64_t)s * 256 + bytes[i]];
      if (s < 0 || !viable[s]) { ok = 0; break; }
    }
    if (ok) mask[t >> 5] |= 1u << (t & 31);
  }
}

/* maskConstraintLogits over f32: -inf except legal and termination ids. */
void or_mask_logits(const float* raw, int64_t V, const int32_t* legal, int64_t n_legal,
                    const int32_t* term, int64_t n_term, float* out) {
  for (int64_t i = 0; i < V; ++i) out[i] = -INFINITY;
  for (int64_t i = 0; i < n_legal; ++i) if (legal[i] >= 0 && legal[i] < V) out[legal[i]] = raw[legal[i]];
  for (int64_t i = 0; i < n_term; ++i) if (term[i] >= 0 && term[i] < V) out[term[i]] = raw[term[i]];
}
