/*
 * gsample — MI355X (gfx950) token sampling and constrained decoding.
 *
 * A C ABI over hand-written HIP kernels. Plain pointers and sizes only.
 * Every call returns a gs_status; gs_last_error() gives the message, which
 * for each reference error condition is the reference's own text.
 *
 * The reference's sampling stage is a set of synchronous TypeScript
 * functions called from the session decode loop; each entry point below
 * names the reference interface it replaces (path:line in the reference).
 *
 * Threading: a context owns one HIP stream and scratch memory; a context is
 * not thread-safe, distinct contexts are. Calls that take a `stream`
 * argument enqueue on that stream when it is non-NULL, else on the
 * context's stream. Caller memory is never freed by the library.
 */
#ifndef GSAMPLE_H
#define GSAMPLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GSAMPLE_ABI_VERSION 2

typedef enum gs_status {
  GS_OK = 0,
  GS_ERR_INVALID_ARGUMENT = 1,   /* bad pointer / size / dtype */
  GS_ERR_INVALID_CONFIG = 2,     /* "Invalid Gemma decoding config: ..." */
  GS_ERR_EMPTY_LOGITS = 3,       /* "Cannot sample empty logits" */
  GS_ERR_DEAD_END = 4,           /* "Generation constraint reached a tokenization dead end" */
  GS_ERR_CONSTRAINT_VIOLATION = 5, /* "Selected token violates the generation constraint" */
  GS_ERR_TOKEN_RANGE = 6,        /* "Token N is outside logits length V" */
  GS_ERR_STOP_TOKEN_RANGE = 7,   /* "Gemma stop token IDs must be below 262144" */
  GS_ERR_EMPTY_CANDIDATES = 8,   /* min-p left no candidate (the reference fails there) */
  GS_ERR_UNSUPPORTED = 9,        /* a size beyond a documented limit */
  GS_ERR_HIP = 10,               /* a HIP runtime error (message has the HIP text) */
  GS_ERR_NO_DEVICE = 11
} gs_status;

typedef enum gs_dtype { GS_F32 = 0, GS_BF16 = 1 } gs_dtype;

typedef enum gs_rng_mode {
  GS_RNG_SEEDED = 0,    /* random() is SeededRandom(seed).next(), draw number draw_index */
  GS_RNG_EXPLICIT = 1   /* random() returns `uniform` (a caller-supplied closure's value) */
} gs_rng_mode;

/* Per-row decoding options: every DecodingConfig field the sampler reads
 * (src/runtime/decoding.ts:1-14) plus what the session supplies around it. */
typedef struct gs_row_config {
  double temperature;         /* 0 => greedy argmax, no draw (sampling.ts:31) */
  double top_p;               /* 1 => off */
  double min_p;               /* 0 => off */
  double typical_p;           /* 1 => off */
  double repetition_penalty;
  double frequency_penalty;
  double presence_penalty;
  double softcap;             /* > 0: logit <- softcap*tanh(logit/softcap) first (Gemma final-logit cap) */
  double uniform;             /* GS_RNG_EXPLICIT: the value random() returns, in [0,1) */
  int64_t seed;               /* GS_RNG_SEEDED: SeededRandom(seed) (sampling.ts:3-8) */
  uint64_t draw_index;        /* GS_RNG_SEEDED: 0-based number of the draw */
  int32_t top_k;              /* 0 => off */
  int32_t repetition_window;  /* 0 => no penalties (sampling.ts:22-24) */
  int32_t rng_mode;           /* gs_rng_mode */
  int32_t mask_slot;          /* -1: unconstrained; else a row of the mask table */
  int32_t accepting;          /* constraint.accepting: termination ids are legal */
  int32_t options;            /* GS_ROW_* bits */
} gs_row_config;

#define GS_ROW_FORCE_EXACT 1u /* resolve this row on the sequential exact path */

/* kinds of per-row forced ids (gemma-session.ts:1305-1329) */
#define GS_FORCED_TERMINATION 1u /* EOS / stop id: legal only when accepting */
#define GS_FORCED_EXTRA 2u       /* additional legal id (e.g. the reasoning opener) */

/* result flags */
#define GS_FLAG_TOPP_TIE 1u       /* top-p boundary |cumulative - topP| <= 1e-6 * topP */
#define GS_FLAG_EXACT_PATH 2u     /* resolved on the sequential exact path */
#define GS_FLAG_NEAR_TIE 4u       /* a fast-path margin fell under 1e-10 (row re-resolved exactly) */
#define GS_FLAG_DEAD_END 8u       /* constrained row with no legal token */
#define GS_FLAG_NONFINITE 16u     /* NaN or +Inf logits: outside the reference's contract */
#define GS_FLAG_EMPTY_CANDIDATES 32u
#define GS_FLAG_GREEDY 64u
#define GS_FLAG_UNSUPPORTED 128u  /* beyond a documented size limit */
#define GS_FLAG_INVALID_SLOT 256u /* mask_slot >= 0 but not below the batch's mask_slots (row not sampled) */
#define GS_FLAG_INDEX_CHECK 512u  /* an index the finish read back from its workspace failed its range
                                     check; the row was re-resolved on the exact path (never expected) */

typedef struct gs_row_result {
  int32_t token;         /* sampled id; -1 when the row failed (see flags) */
  uint32_t flags;
  double probability;    /* the chosen item's probability in the reference's sorted softmax
                            (sampling.ts:42); 1 for greedy rows */
} gs_row_result;

typedef struct gs_context gs_context;

/* One batched sampling call. All pointers are DEVICE pointers on the
 * context's device unless noted. */
typedef struct gs_batch {
  const void* logits;                /* rows x row_stride elements of `dtype` */
  int64_t row_stride;                /* elements between rows (>= vocab size) */
  int32_t dtype;                     /* gs_dtype */
  int32_t rows;
  const gs_row_config* configs;      /* [rows] */
  const int64_t* history_offsets;    /* [rows+1] or NULL: history CSR (prompt + generated ids) */
  const int32_t* history_ids;
  const int64_t* forced_offsets;     /* [rows+1] or NULL: termination / extra ids of constrained rows */
  const int32_t* forced_ids;
  const uint8_t* forced_kinds;       /* GS_FORCED_* per forced id */
  const uint32_t* mask_table;        /* [slots][ceil(V/32)] legal-token bitmasks (gs_build_masks) */
  int32_t mask_slots;
  int32_t hints;                     /* GS_BATCH_* bits (0: none) */
  gs_row_result* results;            /* [rows] */
} gs_batch;

/* Batch hint: some row may take a full-vocabulary draw (temperature > 0,
 * topK 0, topP 1, no min-p or typical-p, no mask). Such a draw whose cursor
 * falls past the candidates the finish ranks is then spread over many
 * workgroups by four more launches (stage GS_STAGE_DEEP) instead of taking
 * the row's one workgroup; the results are identical either way. Without
 * the hint, and for batches of fewer than 4 rows (where the launches cost
 * more than they save on average), those launches are skipped.
 * gs_sample_host sets the hint itself from its host configs. */
#define GS_BATCH_FULL_DRAWS 1
/* Batch hint for gs_lmhead_sample (vocabularies that are a multiple of 8192
 * ids): the lm_head's epilogue computes the chunk scan's statistics and
 * candidate lists itself, so the logits are written but not read back (three
 * launches -- the rows' excluded-id bitmaps, the fused head, a merge of its
 * per-256-id partials into the scan's chunk records -- instead of the head and
 * the scan). Results equal the unfused path's tokens; probabilities agree
 * within the normaliser bound. Without the hint the head and the scan run
 * separately, which is faster at 64 x 2048 x 262144 on MI355X (220 against
 * 306 us for the head and the streaming stage). */
#define GS_BATCH_FUSED_HEAD 2

/* Library / device identity. */
int gs_abi_version(void);
int gs_device_count(int* out);

/* SeededRandom(seed).next() value number `index` (0 = first)
 * (src/runtime/sampling.ts:3-16), as the kernels compute it. */
double gs_seeded_random(int64_t seed, uint64_t index);

/* The engine's Math.exp / Math.log (bit-identical to the JS engine's, used by
 * sampling.ts:39,50,51,77,79) and its final-logit softcap, as the kernels
 * evaluate them. */
double gs_js_exp(double x);
double gs_js_log(double x);
float gs_softcap(float x, double cap);

/* validateDecodingConfig (src/runtime/decoding.ts:31-59) over HOST row
 * configs: GS_ERR_INVALID_CONFIG with "Invalid Gemma decoding config: ..."
 * (src/runtime/generation-config.ts:65) naming every failed field. ctx may
 * be NULL; gs_last_error(NULL) then holds the message. */
int gs_validate_configs(gs_context* ctx, const gs_row_config* configs, int32_t n);

/* Context: device ordinal, vocab size V (1 .. 2097152; larger returns
 * GS_ERR_UNSUPPORTED), the largest batch it will see. Calls on one context
 * share its scratch memory, so they must be ordered on one stream. Device
 * memory: per row about V / 2 bytes of chunk statistics and lists, plus
 * 36 * 2^ceil(log2 V) bytes of exact-path scratch for each of
 * min(max_rows, max(64, 12 GiB / that)) rows -- rows beyond those, in
 * larger batches, share the slots through a second kernel.
 * (no reference counterpart: the reference keeps its WebGPU device in a
 *  module singleton, src/webgpu/device.ts:4-40) */
int gs_create(int device, int32_t vocab_size, int32_t max_rows, gs_context** out);
int gs_destroy(gs_context* ctx);
const char* gs_last_error(const gs_context* ctx);
int gs_synchronize(gs_context* ctx);
void* gs_stream(gs_context* ctx);

/* Batched sampleToken: replaces sampleToken(rawLogits, history, config, random)
 * (src/runtime/sampling.ts:18-65) and, for constrained rows, the masking and
 * termination rules of selectConstrainedToken + maskConstraintLogits
 * (src/runtime/gemma-session.ts:1305-1329; src/runtime/constraints.ts:159-173).
 * Enqueues on `stream` (hipStream_t or NULL). Results are written to
 * batch->results; per-row failures are flagged there. */
int gs_sample(gs_context* ctx, const gs_batch* batch, void* stream);

/* gs_sample with no allocation at all, for callers that cannot allocate
 * device memory: code under HIP graph capture, tight serving loops, hosts
 * that forbid hipMalloc. No counterpart in the reference (its sampler
 * allocates a fresh JS array per call, src/runtime/sampling.ts:20,33-35).
 * The same kernels as gs_sample work in one fixed 27.4 MB device array that
 * each GPU holds from its first call until the process ends: no context,
 * no hipMalloc/hipFree. Limits: rows <= 64 and vocab_size <= 262144
 * (GS_ERR_UNSUPPORTED beyond them, nothing launched). Every pointer of
 * `batch` is device memory of the CURRENT device; `stream` is a hipStream_t
 * of that device (NULL: the null stream). Calls on one GPU share its array,
 * so calls whose kernels overlap on that GPU (concurrent streams or host
 * threads) race: order them on one stream. Failures set gs_last_error(NULL). */
int gs_sample_noalloc(const gs_batch* batch, int32_t vocab_size, void* stream);

/* As gs_sample, then waits and maps the first failing row to its reference
 * error (status + gs_last_error text). Host copy of the results in `host_out`
 * (may be NULL). */
int gs_sample_sync(gs_context* ctx, const gs_batch* batch, gs_row_result* host_out);

/* Batched sampleToken over HOST arrays, for hosts that hold the logits in
 * host memory as the reference does (its per-token readback copy,
 * src/webgpu/decode-model.ts:183-188, handed to sampleToken,
 * src/runtime/sampling.ts:18-65): every pointer of `batch` is a host pointer
 * except `logits` when logits_on_device != 0 (device memory, e.g. the output
 * of gs_lmhead) and `mask_table` (device memory filled by gs_build_masks);
 * batch->results is ignored. The arrays are staged into context-owned device
 * memory, the batch is sampled on the context's stream, and the call waits,
 * writes the rows' results to host_results[rows] and maps the first failing
 * row to its reference error as gs_sample_sync does. CSR offsets must start
 * at 0 and never decrease, and every mask_slot must lie in the mask table
 * (GS_ERR_INVALID_ARGUMENT otherwise). */
int gs_sample_host(gs_context* ctx, const gs_batch* batch, int32_t logits_on_device, gs_row_result* host_results);

/* Device memory for hosts without a GPU array library (the Node addon):
 * hipMalloc / hipFree on the context's device, and copies on the context's
 * stream that return when the bytes have arrived.
 * (no reference counterpart: the reference's buffers are WebGPU GPUBuffers,
 *  src/webgpu/decode-model.ts:127-188) */
int gs_device_alloc(gs_context* ctx, size_t bytes, void** out);
int gs_device_free(gs_context* ctx, void* ptr);
int gs_copy_to_device(gs_context* ctx, void* dst_device, const void* src_host, size_t bytes);
int gs_copy_to_host(gs_context* ctx, void* dst_host, const void* src_device, size_t bytes);

/* maskConstraintLogits (src/runtime/constraints.ts:159-173) on the device:
 * out[i] = raw[i] for every listed id i in [0, n) (ids outside are ignored),
 * -Infinity elsewhere. raw, ids and out are DEVICE pointers; enqueued on
 * `stream` (NULL: the context's). */
int gs_mask_logits(gs_context* ctx, const float* raw, int64_t n, const int32_t* ids, int64_t n_ids, float* out,
                   void* stream);
/* The same over HOST arrays with the reference's two id lists (legal ids,
 * termination ids); returns when out[n] holds the masked row. */
int gs_mask_logits_host(gs_context* ctx, const float* raw, int64_t n, const int32_t* legal, int64_t n_legal,
                        const int32_t* termination, int64_t n_termination, float* out);

/* tokenLogProbability (src/runtime/sampling.ts:67-80) per row:
 * out[r] = logits[r][token[r]] - max - log(sum exp(logits - max)), raw logits. */
int gs_token_log_prob(gs_context* ctx, const void* logits, int32_t dtype, int32_t rows, int64_t row_stride,
                      const int32_t* tokens, double* out, void* stream);

/* tokenLogProbability over HOST f32 rows [rows][V] and HOST tokens; throws the
 * reference's range error (sampling.ts:68-70) as GS_ERR_TOKEN_RANGE. */
int gs_token_log_prob_host(gs_context* ctx, const float* logits, int32_t rows, const int32_t* tokens, double* out);

/* Constraint tables. Replaces TokenByteTrie (src/runtime/token-byte-trie.ts:16-40)
 * with a token-bytes CSR: HOST arrays offsets[V+1] (int64) and bytes. Tokens
 * with no bytes (specials) are never legal. */
int gs_set_vocab(gs_context* ctx, const int64_t* offsets, const uint8_t* bytes, int64_t n_bytes);

/* A byte-level DFA (HOST arrays): next[n_states*256] (-1 = no edge) and
 * finals[n_states]. Viable states (co-reachable to a final state,
 * src/runtime/constraints.ts:300-322) are derived here. */
int gs_set_dfa(gs_context* ctx, int32_t n_states, const int32_t* next, const uint8_t* finals);

/* legalTokenIds (src/runtime/constraints.ts:56-92) for n DFA states at once,
 * as bitmasks: mask_table[i][ceil(V/32)] (DEVICE) gets state states[i] (HOST). */
int gs_build_masks(gs_context* ctx, const int32_t* states, int32_t n, uint32_t* mask_table, void* stream);

/* acceptToken (src/runtime/constraints.ts:94-103) per row, HOST arrays:
 * states_out[i] = the state after token tokens[i]'s bytes from states_in[i];
 * GS_ERR_CONSTRAINT_VIOLATION if any step has no edge or leaves the viable set. */
int gs_dfa_advance(gs_context* ctx, const int32_t* states_in, const int32_t* tokens, int32_t n,
                   int32_t* states_out);

/* acceptToken(tokenBytes) (src/runtime/constraints.ts:94-103) on one byte
 * string: *state_out = the state after bytes[0..n) from `state`;
 * GS_ERR_CONSTRAINT_VIOLATION ("Selected token violates the generation
 * constraint") if a byte has no edge or leads out of the viable set. An empty
 * string leaves the state unchanged. */
int gs_dfa_advance_bytes(gs_context* ctx, int32_t state, const uint8_t* bytes, int64_t n, int32_t* state_out);
/* legalTokenIds(trie) (src/runtime/constraints.ts:56-92) of one DFA state as
 * ascending HOST ids: the first min(cap, count) ids go to ids[], the count
 * to *n_out. Computed by the mask kernel of gs_build_masks. */
int gs_legal_token_ids(gs_context* ctx, int32_t state, int32_t* ids, int32_t cap, int32_t* n_out);
/* accepting (src/runtime/constraints.ts:52-54) of a byte-level DFA state. */
int gs_dfa_accepting(gs_context* ctx, int32_t state, int32_t* out);

/* lm_head logits producer (replaces the int2 QAT GEMV, src/webgpu/decode-lm-head.ts:187-340):
 * logits[m][v] = softcap*tanh((hidden[m] . weight[v]) / softcap)   (softcap <= 0: no cap)
 * hidden bf16 [m_rows][width], weight bf16 [V][width], logits f32 [m_rows][V]. */
int gs_lmhead(gs_context* ctx, const void* hidden, const void* weight, int32_t m_rows, int32_t width,
              float softcap, float* logits, void* stream);

/* lm_head followed by gs_sample on its f32 output (batch->logits is ignored and
 * replaced by `logits_scratch`, [m_rows][V] f32 device memory, 16-byte
 * aligned); with GS_BATCH_FUSED_HEAD in batch->hints the head computes the
 * sampler's per-chunk statistics itself (see the hint). */
int gs_lmhead_sample(gs_context* ctx, const void* hidden, const void* weight, int32_t width, float softcap,
                     float* logits_scratch, const gs_batch* batch, void* stream);

/* int2 QAT LM head, the reference's own logits producer
 * (src/webgpu/decode-lm-head.ts:262-340, weights src/model/gemma-output-weights.ts:72-81),
 * as its CPU definition cpuQatLinear states it (src/reference/qat-linear.ts:78-148):
 *   logits[m][v] = srq(row_scales[v] * sum_k (code[v][k] - 2) * srq(x[m][k], input_scale), output_scale)
 * with srq(y, s) = y for s = 0, else clamp(rint(y / s), -128, 127) * s rounded to float
 * (applySrq). x: f32 [m_rows][width]; packed_codes: 2-bit codes, code k of a row at bits
 * 2k..2k+1 of word k / 16 (packInt2Rows), as GS_QAT_ROW_MAJOR ([V][width / 16] words, the
 * checkpoint's lm_head.weight) or GS_QAT_BLOCK_MAJOR (4-word blocks [width / 64][V], the
 * reference's GPU order); row_scales: f32 [V]; logits: f32 [m_rows][V]; all device memory,
 * 16-byte aligned. width a multiple of 64, at most 4096. Each row's sum runs in column order in
 * binary64, so the logits equal cpuQatLinear's bit for bit. */
#define GS_QAT_ROW_MAJOR 0
#define GS_QAT_BLOCK_MAJOR 1
int gs_qat_lmhead(gs_context* ctx, const float* x, int32_t m_rows, int32_t width, const uint32_t* packed_codes,
                  int32_t layout, const float* row_scales, float input_scale, float output_scale, float* logits,
                  void* stream);

/* gs_qat_lmhead followed by gs_sample on its output (batch->logits is ignored and replaced by
 * `logits_scratch`, [batch->rows][V] f32 device memory; m_rows = batch->rows). */
int gs_qat_lmhead_sample(gs_context* ctx, const float* x, int32_t width, const uint32_t* packed_codes,
                         int32_t layout, const float* row_scales, float input_scale, float output_scale,
                         float* logits_scratch, const gs_batch* batch, void* stream);

/* Self-check of the bound the chunk scan's normaliser rests on; no
 * counterpart in the reference. Largest relative error of the hardware
 * binary32 exp2 (v_exp_f32, which the scan evaluates every term with) over
 * every binary32 y in [lo, hi] whose result is a normal number, against
 * binary64 exp2, on the context's device; *worst_y is where it occurs. The
 * scan's normaliser bound assumes at most 1e-7 over [-150, 2^-10].
 * Synchronous. */
int gs_check_exp2(gs_context* ctx, float lo, float hi, double* max_rel_err, float* worst_y);

/* Kernel timing with HIP events: replaces the WebGPU timestamp queries of
 * measureGpuDispatches (src/webgpu/gpu-timestamp.ts:1-56). After
 * gs_timing_begin(ctx, max_calls), the next max_calls gs_sample /
 * gs_lmhead_sample calls launch each of their kernels with a start and a stop
 * event (hipExtLaunchKernel), stamped when the dispatch begins and when its
 * last wave ends, so each figure is the kernel alone. gs_timing_end waits for
 * those events, writes per stage the summed milliseconds
 * (stage_ms[GS_STAGE_COUNT]) and the number of calls that ran that stage
 * (calls[GS_STAGE_COUNT]), and stops timing. */
#define GS_STAGE_LMHEAD 0 /* the lm_head kernel (bf16 or int2 QAT) */
#define GS_STAGE_SCAN 1   /* scan_kernel: the one HBM pass over the logits */
#define GS_STAGE_FINISH 2 /* finish_kernel: per-row merge, filters and draw */
#define GS_STAGE_EXACT 3  /* exact_kernel: replay of rows beyond the context's exact slots */
#define GS_STAGE_DEEP 4   /* deep1_kernel .. deep_final_kernel: full-vocabulary draws over many workgroups */
#define GS_STAGE_COUNT 5
int gs_timing_begin(gs_context* ctx, int32_t max_calls);
int gs_timing_end(gs_context* ctx, double* stage_ms, int32_t* calls);

#ifdef __cplusplus
}
#endif

#endif /* GSAMPLE_H */
