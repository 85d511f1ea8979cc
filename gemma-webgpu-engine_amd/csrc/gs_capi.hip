// libgsample C ABI: contexts, scratch, launches and error mapping.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "gs_internal.h"

using namespace gs;

struct gs_context {
  int device = 0;
  int32_t vocab = 0;
  int32_t max_rows = 0;
  int32_t n_chunks = 0;
  int32_t mask_words = 0;
  hipStream_t stream = nullptr;
  ChunkStat* d_stats = nullptr;
  uint64_t* d_lists = nullptr;
  ExactQueue* d_queue = nullptr;
  uint8_t* d_exact = nullptr;
  DeepRow* d_deep_rows = nullptr;   // [max_rows] records of the multi-workgroup deep draw
  DeepQueue* d_deep_queue = nullptr;
  int64_t exact_cap = 0;
  int64_t exact_slot_bytes = 0;
  int32_t exact_slots = 0;
  int32_t cu_count = 0;  // compute units of the device (the scan's work split)
  // constraint tables
  int64_t* d_vocab_offsets = nullptr;
  uint8_t* d_vocab_bytes = nullptr;
  std::vector<int64_t> vocab_offsets;
  std::vector<uint8_t> vocab_bytes;
  int32_t n_states = 0;
  int16_t* d_next = nullptr;
  std::vector<int32_t> next;      // viability folded in
  std::vector<uint8_t> finals;
  std::vector<uint8_t> viable;
  int32_t* d_states = nullptr;
  int32_t states_cap = 0;
  // device staging for the host-array entry points (grown on demand)
  uint8_t* d_stage = nullptr;
  size_t stage_cap = 0;
  // the fused lm_head path's per-row buffers (grown on demand)
  uint32_t* d_dead = nullptr;
  PartStat* d_parts = nullptr;
  uint64_t* d_plists = nullptr;
  uint32_t* d_row_thr = nullptr;
  int32_t fused_rows = 0;
  // kernel timing (gs_timing_begin / gs_timing_end): per timed call and stage,
  // the start and stop events of that stage's kernel launch
  std::vector<hipEvent_t> t_events;  // [max_calls][GS_STAGE_COUNT][2]
  std::vector<uint8_t> t_ran;        // [max_calls][GS_STAGE_COUNT]
  int32_t t_cap = 0;
  int32_t t_calls = 0;
  bool t_on = false;
  std::string error;
};

namespace {

// message of the last failure of a call made without a context, in a fixed
// buffer: a context-free call allocates nothing, not even for its message
thread_local char g_no_context_error[256] = "no context";

int fail_static(int status, const char* msg) {
  size_t n = strlen(msg);
  if (n > sizeof(g_no_context_error) - 1) n = sizeof(g_no_context_error) - 1;
  memcpy(g_no_context_error, msg, n);
  g_no_context_error[n] = 0;
  return status;
}

int fail(gs_context* ctx, int status, const std::string& msg) {
  if (ctx) ctx->error = msg;
  else fail_static(status, msg.c_str());
  return status;
}

#define GS_HIP(ctx, expr)                                                                  \
  do {                                                                                    \
    hipError_t e_ = (expr);                                                               \
    if (e_ != hipSuccess) return fail((ctx), GS_ERR_HIP, std::string(#expr ": ") + hipGetErrorString(e_)); \
  } while (0)

void free_dev(void* p) {
  if (p) (void)hipFree(p);
}

hipStream_t pick_stream(gs_context* ctx, void* stream) {
  return stream ? (hipStream_t)stream : ctx->stream;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Slot of the current call in the timing tables, or -1 when not timing.
int32_t timing_slot(gs_context* ctx) {
  if (!ctx->t_on || ctx->t_calls >= ctx->t_cap) return -1;
  return ctx->t_calls;
}

// The timing events of one stage's launch in timing slot `slot` (none when
// not timing).
LaunchEvents stage_events(gs_context* ctx, int32_t slot, int stage) {
  LaunchEvents ev;
  if (slot < 0) return ev;
  const size_t i = (size_t)slot * GS_STAGE_COUNT + stage;
  ev.start = ctx->t_events[i * 2];
  ev.stop = ctx->t_events[i * 2 + 1];
  ctx->t_ran[i] = 1;
  return ev;
}

// Grows the context's device staging buffer to at least `bytes`. Waits for
// the stream first: queued work may still read the old buffer.
int ensure_stage(gs_context* ctx, size_t bytes) {
  if (bytes <= ctx->stage_cap) return GS_OK;
  GS_HIP(ctx, hipStreamSynchronize(ctx->stream));
  free_dev(ctx->d_stage);
  ctx->d_stage = nullptr;
  ctx->stage_cap = 0;
  GS_HIP(ctx, hipMalloc(&ctx->d_stage, bytes));
  ctx->stage_cap = bytes;
  return GS_OK;
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Grows the fused lm_head path's buffers to at least `rows` rows (in steps
// of 64). Waits for the device first: queued work may still use the old ones.
int ensure_fused(gs_context* ctx, int32_t rows) {
  if (rows <= ctx->fused_rows) return GS_OK;
  GS_HIP(ctx, hipDeviceSynchronize());
  free_dev(ctx->d_dead);
  free_dev(ctx->d_parts);
  free_dev(ctx->d_plists);
  free_dev(ctx->d_row_thr);
  ctx->d_dead = nullptr;
  ctx->d_parts = nullptr;
  ctx->d_plists = nullptr;
  ctx->d_row_thr = nullptr;
  ctx->fused_rows = 0;
  const size_t r = (size_t)((rows + 63) / 64 * 64);
  const size_t n_parts = (size_t)ctx->vocab / kPartIds;
  if (hipMalloc(&ctx->d_dead, r * ctx->mask_words * sizeof(uint32_t)) != hipSuccess ||
      hipMalloc(&ctx->d_parts, r * n_parts * sizeof(PartStat)) != hipSuccess ||
      hipMalloc(&ctx->d_plists, r * n_parts * kPartCap * sizeof(uint64_t)) != hipSuccess ||
      hipMalloc(&ctx->d_row_thr, r * sizeof(uint32_t)) != hipSuccess) {
    (void)hipGetLastError();
    free_dev(ctx->d_dead);
    free_dev(ctx->d_parts);
    free_dev(ctx->d_plists);
    free_dev(ctx->d_row_thr);
    ctx->d_dead = nullptr;
    ctx->d_parts = nullptr;
    ctx->d_plists = nullptr;
    ctx->d_row_thr = nullptr;
    return fail(ctx, GS_ERR_HIP, "allocating the fused lm_head buffers failed");
  }
  ctx->fused_rows = (int32_t)r;
  return GS_OK;
}

// Per-row failures of a finished batch, mapped to the reference's errors
// (the first failing row decides).
int map_row_failures(gs_context* ctx, const gs_row_result* res, int32_t rows) {
  for (int32_t r = 0; r < rows; ++r) {
    const uint32_t f = res[r].flags;
    if (f & GS_FLAG_DEAD_END) return fail(ctx, GS_ERR_DEAD_END, "Generation constraint reached a tokenization dead end");
    if (f & GS_FLAG_EMPTY_CANDIDATES)
      return fail(ctx, GS_ERR_EMPTY_CANDIDATES, "min-p left no candidate token (row " + std::to_string(r) + ")");
    if (f & GS_FLAG_INVALID_SLOT)
      return fail(ctx, GS_ERR_INVALID_ARGUMENT, "row " + std::to_string(r) + ": mask_slot outside the mask table");
    if (f & GS_FLAG_UNSUPPORTED)
      return fail(ctx, GS_ERR_UNSUPPORTED, "row " + std::to_string(r) + ": beyond a documented size limit");
  }
  return GS_OK;
}

// A host CSR offsets array [rows+1]: starts at 0 and never decreases.
bool csr_ok(const int64_t* off, int32_t rows) {
  if (off[0] != 0) return false;
  for (int32_t r = 0; r < rows; ++r)
    if (off[r + 1] < off[r]) return false;
  return true;
}

// The first thing wrong with a batch's pointers and sizes (NULL: nothing).
const char* batch_error(const gs_batch* b, int32_t vocab) {
  if (!b->logits || !b->configs || !b->results) return "logits, configs and results are required";
  if (b->dtype != GS_F32 && b->dtype != GS_BF16) return "dtype must be f32 or bf16";
  if (b->row_stride < vocab) return "row_stride is smaller than the vocab";
  if (b->history_offsets && !b->history_ids) return "history_ids missing";
  if (b->forced_offsets && (!b->forced_ids || !b->forced_kinds)) return "forced ids missing";
  if (b->mask_slots > 0 && !b->mask_table) return "mask_table missing";
  return nullptr;
}

// Device memory one sampling launch works in: a context's, or the
// no-allocation entry point's fixed array.
struct Workspace {
  int32_t vocab = 0, n_chunks = 0, mask_words = 0, exact_slots = 0, cu_count = 0;
  ChunkStat* stats = nullptr;
  uint64_t* lists = nullptr;
  ExactQueue* queue = nullptr;
  uint8_t* exact = nullptr;
  int64_t exact_slot_bytes = 0, exact_cap = 0;
  DeepRow* deep_rows = nullptr;  // none: the finish's workgroups take their own deep draws
  DeepQueue* deep_queue = nullptr;
  int32_t deep_max_rows = 0;
};

// Batches of fewer rows keep their deep draws on the rows' own workgroups:
// the four deep launches cost about 17 us even when no row needs them, more
// than a lone row's expected saving (a deep draw takes one draw in ten or
// fewer, ~60 us faster over many workgroups).
constexpr int32_t kDeepMinRows = 4;

// true when the batch hints at full-vocabulary draws, has kDeepMinRows rows
// or more, and the workspace has the deep draw's records
bool deep_launch(const Workspace& w, const gs_batch* b) {
  return (b->hints & GS_BATCH_FULL_DRAWS) && b->rows >= kDeepMinRows && w.deep_rows && w.deep_queue &&
         b->rows <= w.deep_max_rows;
}

// The kernels' arguments for one checked batch in workspace w.
SampleArgs sample_args(const Workspace& w, const gs_batch* b) {
  const size_t esize = b->dtype == GS_BF16 ? 2 : 4;
  SampleArgs a{};
  a.logits = b->logits;
  a.row_stride = b->row_stride;
  a.dtype = b->dtype;
  a.rows = b->rows;
  a.vocab = w.vocab;
  a.n_chunks = w.n_chunks;
  a.vector_ok = aligned16(b->logits) && ((b->row_stride * esize) % 16 == 0);
  a.mask_words = w.mask_words;
  a.configs = b->configs;
  a.history_offsets = b->history_offsets;
  a.history_ids = b->history_ids;
  a.forced_offsets = b->forced_offsets;
  a.forced_ids = b->forced_ids;
  a.forced_kinds = b->forced_kinds;
  a.mask_table = b->mask_table;
  a.mask_slots = b->mask_table ? b->mask_slots : 0;
  a.exact_slots = w.exact_slots;
  a.results = b->results;
  a.stats = w.stats;
  a.lists = w.lists;
  a.queue = w.queue;
  a.exact_scratch = w.exact;
  a.exact_slot_bytes = w.exact_slot_bytes;
  a.exact_capacity = w.exact_cap;
  a.cu_count = w.cu_count;
  const bool deep = deep_launch(w, b);
  a.deep_rows = deep ? w.deep_rows : nullptr;
  a.deep_queue = deep ? w.deep_queue : nullptr;
  a.deep_max_rows = deep ? w.deep_max_rows : 0;
  return a;
}

// Enqueues the sampling kernels of one checked batch on stream s (ev: the
// timing events of each stage, none when not timing). The exact-path queue is
// reset by the chunk scan's first workgroup: no memset node, so the launch
// stays capturable and allocates nothing. fused: the lm_head's epilogue wrote
// the partial statistics, which the merge kernel turns into the chunk
// statistics in the scan's place (stage GS_STAGE_SCAN).
hipError_t launch_sample(const Workspace& w, const gs_batch* b, hipStream_t s, const LaunchEvents* ev,
                         const FusedArgs* fused = nullptr) {
  const SampleArgs a = sample_args(w, b);
  const bool deep = a.deep_rows != nullptr;
  if (fused) launch_merge_parts(a, *fused, s, ev[GS_STAGE_SCAN]);
  else launch_scan(a, s, ev[GS_STAGE_SCAN]);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  launch_finish(a, s, ev[GS_STAGE_FINISH]);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (deep) {
    // rows queued by the finish kernel for the multi-workgroup deep draw
    launch_deep(a, s, ev[GS_STAGE_DEEP]);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (b->rows > w.exact_slots) {
    // rows past the slots were queued by the finish kernel
    launch_exact(a, s, ev[GS_STAGE_EXACT]);
    e = hipGetLastError();
  }
  return e;
}

// A context's device memory as the sampling launches' workspace.
Workspace context_workspace(const gs_context* ctx) {
  Workspace w;
  w.vocab = ctx->vocab;
  w.n_chunks = ctx->n_chunks;
  w.mask_words = ctx->mask_words;
  w.exact_slots = ctx->exact_slots;
  w.cu_count = ctx->cu_count;
  w.stats = ctx->d_stats;
  w.lists = ctx->d_lists;
  w.queue = ctx->d_queue;
  w.exact = ctx->d_exact;
  w.exact_slot_bytes = ctx->exact_slot_bytes;
  w.exact_cap = ctx->exact_cap;
  w.deep_rows = ctx->d_deep_rows;
  w.deep_queue = ctx->d_deep_queue;
  w.deep_max_rows = ctx->max_rows;
  return w;
}

void destroy_timing(gs_context* ctx) {
  for (hipEvent_t e : ctx->t_events) (void)hipEventDestroy(e);
  ctx->t_events.clear();
  ctx->t_ran.clear();
  ctx->t_cap = ctx->t_calls = 0;
  ctx->t_on = false;
}

// ------------------------------------------------ no-allocation sampling
// gs_sample_noalloc works in one fixed device array instead of a context's
// memory: chunk statistics and lists for up to kNoAllocMaxRows rows of up to
// kNoAllocMaxVocab logits, the exact-path queue, and kNoAllocExactSlots
// exact-path row slots (rows past them are replayed by the exact kernel,
// which walks the queue with one workgroup per slot).
constexpr int32_t kNoAllocMaxRows = 64;
constexpr int32_t kNoAllocMaxVocab = 262144;
constexpr int32_t kNoAllocExactSlots = 2;
constexpr int kMaxDevices = 64;
constexpr size_t kNaChunks = (kNoAllocMaxVocab + kChunk - 1) / kChunk;
constexpr size_t align256c(size_t x) { return (x + 255) & ~(size_t)255; }
constexpr size_t kNaStatsBytes = align256c(kNoAllocMaxRows * kNaChunks * sizeof(ChunkStat));
constexpr size_t kNaListBytes = align256c(kNoAllocMaxRows * kNaChunks * kGatherCap * sizeof(uint64_t));
constexpr size_t kNaQueueBytes = align256c(sizeof(ExactQueue) + kNoAllocMaxRows * sizeof(uint32_t));
constexpr size_t kNaSlotBytes = 36 * (size_t)kNoAllocMaxVocab;  // 36 B per entry of a 2^18-entry slot
constexpr size_t kNoAllocScratchBytes =
    kNaStatsBytes + kNaListBytes + kNaQueueBytes + kNoAllocExactSlots * kNaSlotBytes;  // 27,427,328 B

}  // namespace

// The no-allocation entry point's device memory (27.4 MB): each GPU the
// library runs on holds its own copy until the process ends. Host code never
// passes this name to a kernel (on the host it is a stand-in, not a device
// address); it uses the per-device address hipGetSymbolAddress returns.
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {

struct NoAllocDevice {
  uint8_t* ptr = nullptr;  // device address of `scratch` on this device
  int32_t cu_count = 0;
};
NoAllocDevice g_noalloc[kMaxDevices];
std::mutex g_noalloc_mu;

// The array's address and the CU count of device `dev` (the current device),
// looked up once per device on its first call.
int noalloc_device(int dev, NoAllocDevice* out) {
  std::lock_guard<std::mutex> lock(g_noalloc_mu);
  NoAllocDevice& d = g_noalloc[dev];
  if (!d.ptr) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p)
      return fail_static(GS_ERR_HIP, "gs_sample_noalloc: hipGetSymbolAddress of the scratch array failed");
    int cu = 0;
    if (hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cu <= 0)
      return fail_static(GS_ERR_HIP, "gs_sample_noalloc: reading the device's compute-unit count failed");
    d.cu_count = cu;
    d.ptr = (uint8_t*)p;
  }
  *out = d;
  return GS_OK;
}

}  // namespace

extern "C" {

int gs_sample_noalloc(const gs_batch* b, int32_t vocab_size, void* stream) {
  if (!b) return fail_static(GS_ERR_INVALID_ARGUMENT, "null batch");
  if (vocab_size <= 0 || vocab_size > kNoAllocMaxVocab)
    return fail_static(GS_ERR_UNSUPPORTED,
                       "gs_sample_noalloc: vocab_size must be 1..262144 (the size of its fixed device scratch)");
  if (b->rows < 0 || b->rows > kNoAllocMaxRows)
    return fail_static(GS_ERR_UNSUPPORTED,
                       "gs_sample_noalloc: rows must be 0..64 (the size of its fixed device scratch)");
  if (b->rows == 0) return GS_OK;
  const char* bad = batch_error(b, vocab_size);
  if (bad) return fail_static(GS_ERR_INVALID_ARGUMENT, bad);
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail_static(GS_ERR_NO_DEVICE, "gs_sample_noalloc: no current HIP device");
  NoAllocDevice d;
  const int st = noalloc_device(dev, &d);
  if (st != GS_OK) return st;
  Workspace w;
  w.vocab = vocab_size;
  w.n_chunks = (vocab_size + kChunk - 1) / kChunk;
  w.mask_words = (vocab_size + 31) / 32;
  w.exact_slots = kNoAllocExactSlots;
  w.cu_count = d.cu_count;
  w.stats = (ChunkStat*)d.ptr;
  w.lists = (uint64_t*)(d.ptr + kNaStatsBytes);
  w.queue = (ExactQueue*)(d.ptr + kNaStatsBytes + kNaListBytes);
  w.exact = d.ptr + kNaStatsBytes + kNaListBytes + kNaQueueBytes;
  w.exact_cap = 1;
  while (w.exact_cap < vocab_size) w.exact_cap <<= 1;
  w.exact_slot_bytes = 36 * w.exact_cap;
  const LaunchEvents ev[GS_STAGE_COUNT] = {};
  const hipError_t e = launch_sample(w, b, (hipStream_t)stream, ev);
  if (e != hipSuccess) return fail_static(GS_ERR_HIP, hipGetErrorString(e));
  return GS_OK;
}

int gs_abi_version(void) { return GSAMPLE_ABI_VERSION; }

int gs_device_count(int* out) {
  if (!out) return GS_ERR_INVALID_ARGUMENT;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) n = 0;
  *out = n;
  return GS_OK;
}

double gs_seeded_random(int64_t seed, uint64_t index) { return gsm::mulberry32_draw(seed, index); }

double gs_js_exp(double x) { return gsm::js_exp(x); }
double gs_js_log(double x) { return gsm::js_log(x); }
float gs_softcap(float x, double cap) { return gsm::softcap_f32(x, cap); }

int gs_create(int device, int32_t vocab_size, int32_t max_rows, gs_context** out) {
  if (!out) return GS_ERR_INVALID_ARGUMENT;
  *out = nullptr;
  if (vocab_size <= 0 || max_rows <= 0) return GS_ERR_INVALID_ARGUMENT;
  if (vocab_size > kMaxVocab) return GS_ERR_UNSUPPORTED;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return GS_ERR_NO_DEVICE;
  if (device < 0 || device >= n) return GS_ERR_NO_DEVICE;
  gs_context* ctx = new gs_context();
  ctx->device = device;
  ctx->vocab = vocab_size;
  ctx->max_rows = max_rows;
  ctx->n_chunks = (vocab_size + kChunk - 1) / kChunk;
  ctx->mask_words = (vocab_size + 31) / 32;
  ctx->exact_cap = 1;
  while (ctx->exact_cap < vocab_size) ctx->exact_cap <<= 1;
  ctx->exact_slot_bytes = 36 * ctx->exact_cap;
  // exact-path scratch slots: one per row up to kExactScratchBudget bytes (at
  // least 64), so that a row of a batch within the slots is replayed by its
  // own finish workgroup and the exact kernel runs only for larger batches
  {
    const int64_t by_budget = std::max<int64_t>(64, kExactScratchBudget / ctx->exact_slot_bytes);
    ctx->exact_slots = (int32_t)std::min<int64_t>(max_rows, by_budget);
  }
  auto cleanup = [&](int status, const char* what) {
    gs_destroy(ctx);
    (void)what;
    return status;
  };
  if (hipSetDevice(device) != hipSuccess) return cleanup(GS_ERR_HIP, "hipSetDevice");
  if (hipDeviceGetAttribute(&ctx->cu_count, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess ||
      ctx->cu_count <= 0)
    return cleanup(GS_ERR_HIP, "device attributes");
  if (hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking) != hipSuccess) return cleanup(GS_ERR_HIP, "stream");
  const size_t stats_bytes = (size_t)max_rows * ctx->n_chunks * sizeof(ChunkStat);
  const size_t list_bytes = (size_t)max_rows * ctx->n_chunks * kGatherCap * sizeof(uint64_t);
  const size_t queue_bytes = sizeof(ExactQueue) + (size_t)max_rows * sizeof(uint32_t);
  if (hipMalloc(&ctx->d_stats, stats_bytes) != hipSuccess) return cleanup(GS_ERR_HIP, "stats");
  if (hipMalloc(&ctx->d_lists, list_bytes) != hipSuccess) return cleanup(GS_ERR_HIP, "lists");
  if (hipMalloc(&ctx->d_queue, queue_bytes) != hipSuccess) return cleanup(GS_ERR_HIP, "queue");
  if (hipMalloc(&ctx->d_exact, (size_t)ctx->exact_slot_bytes * ctx->exact_slots) != hipSuccess)
    return cleanup(GS_ERR_HIP, "exact scratch");
  if (hipMalloc(&ctx->d_deep_rows, sizeof(DeepRow) * (size_t)max_rows) != hipSuccess)
    return cleanup(GS_ERR_HIP, "deep draw records");
  if (hipMalloc(&ctx->d_deep_queue, sizeof(DeepQueue) + sizeof(uint32_t) * 2 * (size_t)max_rows) != hipSuccess)
    return cleanup(GS_ERR_HIP, "deep draw queue");
  *out = ctx;
  return GS_OK;
}

int gs_destroy(gs_context* ctx) {
  if (!ctx) return GS_OK;
  (void)hipSetDevice(ctx->device);
  if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
  free_dev(ctx->d_stats);
  free_dev(ctx->d_lists);
  free_dev(ctx->d_queue);
  free_dev(ctx->d_exact);
  free_dev(ctx->d_deep_rows);
  free_dev(ctx->d_deep_queue);
  free_dev(ctx->d_vocab_offsets);
  free_dev(ctx->d_vocab_bytes);
  free_dev(ctx->d_next);
  free_dev(ctx->d_states);
  free_dev(ctx->d_stage);
  free_dev(ctx->d_dead);
  free_dev(ctx->d_parts);
  free_dev(ctx->d_plists);
  free_dev(ctx->d_row_thr);
  destroy_timing(ctx);
  if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
  delete ctx;
  return GS_OK;
}

const char* gs_last_error(const gs_context* ctx) { return ctx ? ctx->error.c_str() : g_no_context_error; }

int gs_synchronize(gs_context* ctx) {
  if (!ctx) return GS_ERR_INVALID_ARGUMENT;
  GS_HIP(ctx, hipSetDevice(ctx->device));
  GS_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return GS_OK;
}

void* gs_stream(gs_context* ctx) { return ctx ? (void*)ctx->stream : nullptr; }

// validateDecodingConfig (src/runtime/decoding.ts:31-59) for the fields a row
// config carries, with the reference's messages joined as
// resolveGemmaGenerationConfig does (src/runtime/generation-config.ts:65).
int gs_validate_configs(gs_context* ctx, const gs_row_config* configs, int32_t n) {
  if (!configs || n < 0) return fail(ctx, GS_ERR_INVALID_ARGUMENT, "configs must be a host array");
  for (int32_t i = 0; i < n; ++i) {
    const gs_row_config& c = configs[i];
    std::vector<std::string> errors;
    if (!std::isfinite(c.temperature) || c.temperature < 0) errors.push_back("temperature must be >= 0");
    if (c.top_k < 0) errors.push_back("topK must be a non-negative integer");
    const double probs[3] = {c.top_p, c.min_p, c.typical_p};
    const char* names[3] = {"topP", "minP", "typicalP"};
    for (int k = 0; k < 3; ++k) {
      if (!std::isfinite(probs[k]) || probs[k] < 0 || probs[k] > 1) errors.push_back(std::string(names[k]) + " must be between 0 and 1");
    }
    if (!std::isfinite(c.repetition_penalty) || c.repetition_penalty <= 0) errors.push_back("repetitionPenalty must be > 0");
    if (c.repetition_window < 0) errors.push_back("repetitionWindow must be a non-negative integer");
    if (!std::isfinite(c.frequency_penalty) || c.frequency_penalty < 0) errors.push_back("frequencyPenalty must be finite and non-negative");
    if (!std::isfinite(c.presence_penalty) || c.presence_penalty < 0) errors.push_back("presencePenalty must be finite and non-negative");
    if (!errors.empty()) {
      std::string msg = "Invalid Gemma decoding config: ";
      for (size_t k = 0; k < errors.size(); ++k) msg += (k ? "; " : "") + errors[k];
      return fail(ctx, GS_ERR_INVALID_CONFIG, msg);
    }
    if (c.rng_mode == GS_RNG_SEEDED && c.draw_index > gsm::mulberry32_index_limit(c.seed)) {
      return fail(ctx, GS_ERR_UNSUPPORTED, "draw_index is beyond the exactly representable SeededRandom state");
    }
  }
  return GS_OK;
}


int gs_sample(gs_context* ctx, const gs_batch* b, void* stream) {
  if (!ctx || !b) return fail(ctx, GS_ERR_INVALID_ARGUMENT, "null context or batch");
  if (b->rows == 0) return GS_OK;
  if (b->rows < 0 || b->rows > ctx->max_rows) return fail(ctx, GS_ERR_INVALID_ARGUMENT, "rows outside [0, max_rows]");
  const char* bad = batch_error(b, ctx->vocab);
  if (bad) return fail(ctx, GS_ERR_INVALID_ARGUMENT, bad);
  GS_HIP(ctx, hipSetDevice(ctx->device));
  const Workspace w = context_workspace(ctx);
  const int32_t slot = timing_slot(ctx);
  LaunchEvents ev[GS_STAGE_COUNT];
  for (int k = GS_STAGE_SCAN; k <= GS_STAGE_FINISH; ++k) ev[k] = stage_events(ctx, slot, k);
  if (deep_launch(w, b)) ev[GS_STAGE_DEEP] = stage_events(ctx, slot, GS_STAGE_DEEP);
  if (b->rows > ctx->exact_slots) ev[GS_STAGE_EXACT] = stage_events(ctx, slot, GS_STAGE_EXACT);
  const hipError_t e = launch_sample(w, b, pick_stream(ctx, stream), ev);
  if (e != hipSuccess) return fail(ctx, GS_ERR_HIP, std::string("kernel launch: ") + hipGetErrorString(e));
  if (slot >= 0) ctx->t_calls++;
  return GS_OK;
}

int gs_sample_sync(gs_context* ctx, const gs_batch* b, gs_row_result* host_out) {
  int st = gs_sample(ctx, b, nullptr);
  if (st != GS_OK) return st;
  std::vector<gs_row_result> tmp;
  gs_row_result* dst = host_out;
  if (!dst) {
    tmp.resize(b->rows);
    dst = tmp.data();
  }
  GS_HIP(ctx, hipMemcpyAsync(dst, b->results, sizeof(gs_row_result) * b->rows, hipMemcpyDeviceToHost, ctx->stream));
  GS_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return map_row_failures(ctx, dst, b->rows);
}

int gs_sample_host(gs_context* ctx, const gs_batch* b, int32_t logits_on_device, gs_row_result* host_results) {
  if (!ctx || !b || !host_results) return fail(ctx, GS_ERR_INVALID_ARGUMENT, "null context, batch or results");
  if (b->rows == 0) return GS_OK;
  if (b->rows < 0 || b->rows > ctx->max_rows) return fail(ctx, GS_ERR_INVALID_ARGUMENT, "rows outside [0, max_rows]");
  if (!b->logits || !b->configs) return fail(ctx, GS_ERR_INVALID_ARGUMENT, "logits and configs are required");
  if (b->dtype != GS_F32 && b->dtype != GS_BF16) return fail(ctx, GS_ERR_INVALID_ARGUMENT, "dtype must be f32 or bf16");
  if (b->row_stride < ctx->vocab) return fail(ctx, GS_ERR_INVALID_ARGUMENT, "row_stride is smaller than the vocab");
  if (b->history_offsets && !b->history_ids) return fail(ctx, GS_ERR_INVALID_ARGUMENT, "history_ids missing");
  if (b->forced_offsets && (!b->forced_ids || !b->forced_kinds)) return fail(ctx, GS_ERR_INVALID_ARGUMENT, "forced ids missing");
  if (b->mask_slots > 0 && !b->mask_table) return fail(ctx, GS_ERR_INVALID_ARGUMENT, "mask_table missing");
  const int32_t R = b->rows;
  if (b->history_offsets && !csr_ok(b->history_offsets, R))
    return fail(ctx, GS_ERR_INVALID_ARGUMENT, "history_offsets must start at 0 and never decrease");
  if (b->forced_offsets && !csr_ok(b->forced_offsets, R))
    return fail(ctx, GS_ERR_INVALID_ARGUMENT, "forced_offsets must start at 0 and never decrease");
  for (int32_t r = 0; r < R; ++r) {
    const int32_t slot = b->configs[r].mask_slot;
    if (slot >= 0 && (b->mask_slots <= 0 || slot >= b->mask_slots))
      return fail(ctx, GS_ERR_INVALID_ARGUMENT, "row " + std::to_string(r) + ": mask_slot outside the mask table");
  }
  const size_t esize = b->dtype == GS_BF16 ? 2 : 4;
  const size_t logit_bytes = logits_on_device ? 0 : ((size_t)(R - 1) * b->row_stride + ctx->vocab) * esize;
  const int64_t n_hist = b->history_offsets ? b->history_offsets[R] : 0;
  const int64_t n_forced = b->forced_offsets ? b->forced_offsets[R] : 0;
  size_t off = 0;
  const size_t o_logits = off;
  off = align256(off + logit_bytes);
  const size_t o_cfg = off;
  off = align256(off + sizeof(gs_row_config) * R);
  const size_t o_hoff = off;
  off = align256(off + (b->history_offsets ? sizeof(int64_t) * (R + 1) : 0));
  const size_t o_hids = off;
  off = align256(off + sizeof(int32_t) * n_hist);
  const size_t o_foff = off;
  off = align256(off + (b->forced_offsets ? sizeof(int64_t) * (R + 1) : 0));
  const size_t o_fids = off;
  off = align256(off + sizeof(int32_t) * n_forced);
  const size_t o_fk = off;
  off = align256(off + n_forced);
  const size_t o_res = off;
  off = align256(off + sizeof(gs_row_result) * R);
  GS_HIP(ctx, hipSetDevice(ctx->device));
  int st = ensure_stage(ctx, off);
  if (st != GS_OK) return st;
  uint8_t* d = ctx->d_stage;
  hipStream_t s = ctx->stream;
  gs_batch db = *b;
  if (!logits_on_device) {
    GS_HIP(ctx, hipMemcpyAsync(d + o_logits, b->logits, logit_bytes, hipMemcpyHostToDevice, s));
    db.logits = d + o_logits;
  }
  GS_HIP(ctx, hipMemcpyAsync(d + o_cfg, b->configs, sizeof(gs_row_config) * R, hipMemcpyHostToDevice, s));
  db.configs = (const gs_row_config*)(d + o_cfg);
  if (b->history_offsets) {
    GS_HIP(ctx, hipMemcpyAsync(d + o_hoff, b->history_offsets, sizeof(int64_t) * (R + 1), hipMemcpyHostToDevice, s));
    if (n_hist) GS_HIP(ctx, hipMemcpyAsync(d + o_hids, b->history_ids, sizeof(int32_t) * n_hist, hipMemcpyHostToDevice, s));
    db.history_offsets = (const int64_t*)(d + o_hoff);
    db.history_ids = (const int32_t*)(d + o_hids);
  }
  if (b->forced_offsets) {
    GS_HIP(ctx, hipMemcpyAsync(d + o_foff, b->forced_offsets, sizeof(int64_t) * (R + 1), hipMemcpyHostToDevice, s));
    if (n_forced) {
      GS_HIP(ctx, hipMemcpyAsync(d + o_fids, b->forced_ids, sizeof(int32_t) * n_forced, hipMemcpyHostToDevice, s));
      GS_HIP(ctx, hipMemcpyAsync(d + o_fk, b->forced_kinds, n_forced, hipMemcpyHostToDevice, s));
    }
    db.forced_offsets = (const int64_t*)(d + o_foff);
    db.forced_ids = (const int32_t*)(d + o_fids);
    db.forced_kinds = d + o_fk;
  }
  db.results = (gs_row_result*)(d + o_res);
  for (int32_t r = 0; r < R; ++r) {
    const gs_row_config& c = b->configs[r];
    if (c.temperature > 0 && c.top_k <= 0 && c.top_p >= 1 && !(c.min_p > 0) && c.typical_p >= 1 && c.mask_slot < 0)
      db.hints |= GS_BATCH_FULL_DRAWS;
  }
  st = gs_sample(ctx, &db, s);
  if (st != GS_OK) return st;
  GS_HIP(ctx, hipMemcpyAsync(host_results, d + o_res, sizeof(gs_row_result) * R, hipMemcpyDeviceToHost, s));
  GS_HIP(ctx, hipStreamSynchronize(s));
  return map_row_failures(ctx, host_results, R);
}

int gs_device_alloc(gs_context* ctx, size_t bytes, void** out) {
  if (!ctx || !out) return fail(ctx, GS_ERR_INVALID_ARGUMENT, "null context or output");
  *out = nullptr;
  GS_HIP(ctx, hipSetDevice(ctx->device));
  GS_HIP(ctx, hipMalloc(out, bytes ? bytes : 1));
  return GS_OK;
}

int gs_device_free(gs_context* ctx, void* ptr) {
  if (!ctx) return fail(ctx, GS_ERR_INVALID_ARGUMENT, "null context");
  if (!ptr) return GS_OK;
  GS_HIP(ctx, hipSetDevice(ctx->device));
  GS_HIP(ctx, hipStreamSynchronize(ctx->stream));
  GS_HIP(ctx, hipFree(ptr));
  return GS_OK;
}

int gs_copy_to_device(gs_context* ctx, void* dst, const void* src, size_t bytes) {
  if (!ctx || (bytes && (!dst || !src))) return fail(ctx, GS_ERR_INVALID_ARGUMENT, "bad copy arguments");
  if (!bytes) return GS_OK;
  GS_HIP(ctx, hipSetDevice(ctx->device));
  GS_HIP(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
  GS_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return GS_OK;
}

int gs_copy_to_host(gs_context* ctx, void* dst, const void* src, size_t bytes) {
  if (!ctx || (bytes && (!dst || !src))) return fail(ctx, GS_ERR_INVALID_ARGUMENT, "bad copy arguments");
  if (!bytes) return GS_OK;
  GS_HIP(ctx, hipSetDevice(ctx->device));
  GS_HIP(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
  GS_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return GS_OK;
}

int gs_mask_logits(gs_context* ctx, const float* raw, int64_t n, const int32_t* ids, int64_t n_ids, float* out,
                   void* stream) {
  if (!ctx || n < 0 || n_ids < 0 || (n > 0 && (!raw || !out)) || (n_ids > 0 && !ids))
    return fail(ctx, GS_ERR_INVALID_ARGUMENT, "bad arguments");
  GS_HIP(ctx, hipSetDevice(ctx->device));
  launch_mask_logits(raw, n, ids, n_ids, out, pick_stream(ctx, stream));
  GS_HIP(ctx, hipGetLastError());
  return GS_OK;
}

int gs_mask_logits_host(gs_context* ctx, const float* raw, int64_t n, const int32_t* legal, int64_t n_legal,
                        const int32_t* termination, int64_t n_termination, float* out) {
  if (!ctx || n < 0 || n_legal < 0 || n_termination < 0 || (n > 0 && (!raw || !out)) || (n_legal > 0 && !legal) ||
      (n_termination > 0 && !termination))
    return fail(ctx, GS_ERR_INVALID_ARGUMENT, "bad arguments");
  if (n == 0) return GS_OK;
  const size_t o_raw = 0, o_out = align256(sizeof(float) * n), o_ids = o_out + align256(sizeof(float) * n);
  const size_t total = o_ids + sizeof(int32_t) * (n_legal + n_termination);
  GS_HIP(ctx, hipSetDevice(ctx->device));
  int st = ensure_stage(ctx, total);
  if (st != GS_OK) return st;
  uint8_t* d = ctx->d_stage;
  hipStream_t s = ctx->stream;
  GS_HIP(ctx, hipMemcpyAsync(d + o_raw, raw, sizeof(float) * n, hipMemcpyHostToDevice, s));
  if (n_legal) GS_HIP(ctx, hipMemcpyAsync(d + o_ids, legal, sizeof(int32_t) * n_legal, hipMemcpyHostToDevice, s));
  if (n_termination)
    GS_HIP(ctx, hipMemcpyAsync(d + o_ids + sizeof(int32_t) * n_legal, termination, sizeof(int32_t) * n_termination,
                               hipMemcpyHostToDevice, s));
  launch_mask_logits((const float*)(d + o_raw), n, (const int32_t*)(d + o_ids), n_legal + n_termination,
                     (float*)(d + o_out), s);
  GS_HIP(ctx, hipGetLastError());
  GS_HIP(ctx, hipMemcpyAsync(out, d + o_out, sizeof(float) * n, hipMemcpyDeviceToHost, s));
  GS_HIP(ctx, hipStreamSynchronize(s));
  return GS_OK;
}

int gs_token_log_prob(gs_context* ctx, const void* logits, int32_t dtype, int32_t rows, int64_t row_stride,
                      const int32_t* tokens, double* out, void* stream) {
  if (!ctx || !logits || !tokens || !out || rows < 0) return fail(ctx, GS_ERR_INVALID_ARGUMENT, "bad arguments");
  if (dtype != GS_F32 && dtype != GS_BF16) return fail(ctx, GS_ERR_INVALID_ARGUMENT, "dtype must be f32 or bf16");
  if (row_stride < ctx->vocab) return fail(ctx, GS_ERR_INVALID_ARGUMENT, "row_stride is smaller than the vocab");
  if (rows == 0) return GS_OK;
  GS_HIP(ctx, hipSetDevice(ctx->device));
  launch_logprob(logits, dtype, rows, row_stride, ctx->vocab, tokens, out, pick_stream(ctx, stream));
  GS_HIP(ctx, hipGetLastError());
  return GS_OK;
}

// Host convenience: tokenLogProbability with host buffers and the reference's range error.
int gs_token_log_prob_host(gs_context* ctx, const float* logits, int32_t rows, const int32_t* tokens, double* out) {
  if (!ctx || !logits || !tokens || !out || rows < 0) return fail(ctx, GS_ERR_INVALID_ARGUMENT, "bad arguments");
  for (int32_t r = 0; r < rows; ++r) {
    if (tokens[r] < 0 || tokens[r] >= ctx->vocab) {
      return fail(ctx, GS_ERR_TOKEN_RANGE,
                  "Token " + std::to_string(tokens[r]) + " is outside logits length " + std::to_string(ctx->vocab));
    }
  }
  if (rows == 0) return GS_OK;
  // staged in the context's reusable device buffer: logits, tokens, results
  const size_t logit_bytes = sizeof(float) * (size_t)rows * ctx->vocab;
  const size_t o_tok = align256(logit_bytes);
  const size_t o_out = o_tok + align256(sizeof(int32_t) * rows);
  GS_HIP(ctx, hipSetDevice(ctx->device));
  int st = ensure_stage(ctx, o_out + sizeof(double) * rows);
  if (st != GS_OK) return st;
  uint8_t* d = ctx->d_stage;
  hipStream_t s = ctx->stream;
  GS_HIP(ctx, hipMemcpyAsync(d, logits, logit_bytes, hipMemcpyHostToDevice, s));
  GS_HIP(ctx, hipMemcpyAsync(d + o_tok, tokens, sizeof(int32_t) * rows, hipMemcpyHostToDevice, s));
  launch_logprob(d, GS_F32, rows, ctx->vocab, ctx->vocab, (const int32_t*)(d + o_tok), (double*)(d + o_out), s);
  GS_HIP(ctx, hipGetLastError());
  GS_HIP(ctx, hipMemcpyAsync(out, d + o_out, sizeof(double) * rows, hipMemcpyDeviceToHost, s));
  GS_HIP(ctx, hipStreamSynchronize(s));
  return GS_OK;
}

int gs_check_exp2(gs_context* ctx, float lo, float hi, double* max_rel_err, float* worst_y) {
  if (!ctx || !max_rel_err || !worst_y || !(lo <= hi)) return fail(ctx, GS_ERR_INVALID_ARGUMENT, "bad arguments");
  GS_HIP(ctx, hipSetDevice(ctx->device));
  unsigned long long* d = nullptr;
  GS_HIP(ctx, hipMalloc(&d, sizeof(unsigned long long)));
  // every binary32 in [lo, hi]: the negative part by bit patterns from -0
  // up to lo's, the non-negative part from +0 up to hi's
  const uint32_t blo = __builtin_bit_cast(uint32_t, lo), bhi = __builtin_bit_cast(uint32_t, hi);
  int st = GS_OK;
  if (hipMemsetAsync(d, 0, sizeof(unsigned long long), ctx->stream) != hipSuccess) st = fail(ctx, GS_ERR_HIP, "memset failed");
  if (st == GS_OK && lo < 0) {
    const uint32_t neg_hi = hi < 0 ? bhi : 0x80000000u;  // the negative value nearest zero
    launch_exp2_check(neg_hi, blo - neg_hi + 1, d, ctx->stream);
  }
  if (st == GS_OK && hi >= 0) {
    const uint32_t pos_lo = lo >= 0 ? blo : 0u;
    launch_exp2_check(pos_lo, bhi - pos_lo + 1, d, ctx->stream);
  }
  unsigned long long h = 0;
  if (st == GS_OK && (hipGetLastError() != hipSuccess ||
                      hipMemcpyAsync(&h, d, sizeof(h), hipMemcpyDeviceToHost, ctx->stream) != hipSuccess ||
                      hipStreamSynchronize(ctx->stream) != hipSuccess)) {
    st = fail(ctx, GS_ERR_HIP, "exp2 check kernel failed");
  }
  (void)hipStreamSynchronize(ctx->stream);
  free_dev(d);
  if (st != GS_OK) return st;
  *max_rel_err = (double)__builtin_bit_cast(float, (uint32_t)(h >> 32));
  *worst_y = __builtin_bit_cast(float, (uint32_t)h);
  return GS_OK;
}

int gs_set_vocab(gs_context* ctx, const int64_t* offsets, const uint8_t* bytes, int64_t n_bytes) {
  if (!ctx || !offsets || (n_bytes > 0 && !bytes) || n_bytes < 0) return fail(ctx, GS_ERR_INVALID_ARGUMENT, "bad vocab");
  const int64_t V = ctx->vocab;
  if (offsets[0] != 0 || offsets[V] != n_bytes) return fail(ctx, GS_ERR_INVALID_ARGUMENT, "offsets must run 0..n_bytes");
  for (int64_t t = 0; t < V; ++t) {
    if (offsets[t + 1] < offsets[t]) return fail(ctx, GS_ERR_INVALID_ARGUMENT, "offsets must be non-decreasing");
  }
  GS_HIP(ctx, hipSetDevice(ctx->device));
  ctx->vocab_offsets.assign(offsets, offsets + V + 1);
  ctx->vocab_bytes.assign(bytes, bytes + n_bytes);
  free_dev(ctx->d_vocab_offsets);
  free_dev(ctx->d_vocab_bytes);
  ctx->d_vocab_offsets = nullptr;
  ctx->d_vocab_bytes = nullptr;
  GS_HIP(ctx, hipMalloc(&ctx->d_vocab_offsets, sizeof(int64_t) * (V + 1)));
  GS_HIP(ctx, hipMalloc(&ctx->d_vocab_bytes, std::max<int64_t>(n_bytes, 16)));
  GS_HIP(ctx, hipMemcpy(ctx->d_vocab_offsets, offsets, sizeof(int64_t) * (V + 1), hipMemcpyHostToDevice));
  if (n_bytes) GS_HIP(ctx, hipMemcpy(ctx->d_vocab_bytes, bytes, n_bytes, hipMemcpyHostToDevice));
  return GS_OK;
}

int gs_set_dfa(gs_context* ctx, int32_t n_states, const int32_t* next, const uint8_t* finals) {
  if (!ctx || n_states <= 0 || n_states > 32767 || !next || !finals)
    return fail(ctx, GS_ERR_INVALID_ARGUMENT, "DFA needs 1..32767 states, a next table and finals");
  for (int64_t i = 0; i < (int64_t)n_states * 256; ++i) {
    if (next[i] < -1 || next[i] >= n_states) return fail(ctx, GS_ERR_INVALID_ARGUMENT, "next-state out of range");
  }
  // findViableStates (constraints.ts:300-322): reverse reachability from finals
  std::vector<std::vector<int32_t>> preds(n_states);
  for (int32_t s = 0; s < n_states; ++s)
    for (int c = 0; c < 256; ++c)
      if (next[(int64_t)s * 256 + c] >= 0) preds[next[(int64_t)s * 256 + c]].push_back(s);
  std::vector<uint8_t> viable(n_states, 0);
  std::vector<int32_t> stack;
  for (int32_t s = 0; s < n_states; ++s)
    if (finals[s]) { viable[s] = 1; stack.push_back(s); }
  while (!stack.empty()) {
    const int32_t t = stack.back();
    stack.pop_back();
    for (int32_t p : preds[t])
      if (!viable[p]) { viable[p] = 1; stack.push_back(p); }
  }
  std::vector<int16_t> folded((size_t)n_states * 256);
  ctx->next.assign(next, next + (size_t)n_states * 256);
  for (size_t i = 0; i < folded.size(); ++i) {
    const int32_t t = next[i];
    folded[i] = (int16_t)((t >= 0 && viable[t]) ? t : -1);
  }
  GS_HIP(ctx, hipSetDevice(ctx->device));
  free_dev(ctx->d_next);
  ctx->d_next = nullptr;
  GS_HIP(ctx, hipMalloc(&ctx->d_next, folded.size() * sizeof(int16_t)));
  GS_HIP(ctx, hipMemcpy(ctx->d_next, folded.data(), folded.size() * sizeof(int16_t), hipMemcpyHostToDevice));
  ctx->n_states = n_states;
  ctx->finals.assign(finals, finals + n_states);
  ctx->viable = viable;
  return GS_OK;
}

int gs_build_masks(gs_context* ctx, const int32_t* states, int32_t n, uint32_t* mask_table, void* stream) {
  if (!ctx || (n > 0 && (!states || !mask_table)) || n < 0) return fail(ctx, GS_ERR_INVALID_ARGUMENT, "bad arguments");
  if (!ctx->d_next || !ctx->d_vocab_offsets) return fail(ctx, GS_ERR_INVALID_ARGUMENT, "set the vocab and the DFA first");
  for (int32_t i = 0; i < n; ++i) {
    if (states[i] < 0 || states[i] >= ctx->n_states) return fail(ctx, GS_ERR_INVALID_ARGUMENT, "state out of range");
  }
  if (n == 0) return GS_OK;
  GS_HIP(ctx, hipSetDevice(ctx->device));
  hipStream_t s = pick_stream(ctx, stream);
  if (n > ctx->states_cap) {
    GS_HIP(ctx, hipStreamSynchronize(s));
    free_dev(ctx->d_states);
    ctx->d_states = nullptr;
    GS_HIP(ctx, hipMalloc(&ctx->d_states, sizeof(int32_t) * n));
    ctx->states_cap = n;
  }
  GS_HIP(ctx, hipMemcpyAsync(ctx->d_states, states, sizeof(int32_t) * n, hipMemcpyHostToDevice, s));
  launch_masks(ctx->d_vocab_offsets, ctx->d_vocab_bytes, ctx->vocab, ctx->d_next, ctx->d_states, n, mask_table,
               ctx->mask_words, ctx->n_states, s);
  GS_HIP(ctx, hipGetLastError());
  GS_HIP(ctx, hipStreamSynchronize(s));  // the state list is reused by the next call
  return GS_OK;
}

int gs_dfa_advance(gs_context* ctx, const int32_t* states_in, const int32_t* tokens, int32_t n, int32_t* states_out) {
  if (!ctx || n < 0 || (n > 0 && (!states_in || !tokens || !states_out))) return fail(ctx, GS_ERR_INVALID_ARGUMENT, "bad arguments");
  if (ctx->next.empty() || ctx->vocab_offsets.empty()) return fail(ctx, GS_ERR_INVALID_ARGUMENT, "set the vocab and the DFA first");
  for (int32_t i = 0; i < n; ++i) {
    int32_t s = states_in[i];
    const int32_t t = tokens[i];
    if (s < 0 || s >= ctx->n_states || t < 0 || t >= ctx->vocab)
      return fail(ctx, GS_ERR_INVALID_ARGUMENT, "state or token out of range");
    for (int64_t k = ctx->vocab_offsets[t]; k < ctx->vocab_offsets[t + 1]; ++k) {
      s = ctx->next[(size_t)s * 256 + ctx->vocab_bytes[k]];
      if (s < 0 || !ctx->viable[s]) return fail(ctx, GS_ERR_CONSTRAINT_VIOLATION, "Selected token violates the generation constraint");
    }
    states_out[i] = s;
  }
  return GS_OK;
}

int gs_dfa_advance_bytes(gs_context* ctx, int32_t state, const uint8_t* bytes, int64_t n, int32_t* state_out) {
  if (!ctx || !state_out || n < 0 || (n > 0 && !bytes)) return fail(ctx, GS_ERR_INVALID_ARGUMENT, "bad arguments");
  if (ctx->next.empty()) return fail(ctx, GS_ERR_INVALID_ARGUMENT, "set the DFA first");
  if (state < 0 || state >= ctx->n_states) return fail(ctx, GS_ERR_INVALID_ARGUMENT, "state out of range");
  int32_t s = state;
  for (int64_t k = 0; k < n; ++k) {
    s = ctx->next[(size_t)s * 256 + bytes[k]];
    if (s < 0 || !ctx->viable[s]) return fail(ctx, GS_ERR_CONSTRAINT_VIOLATION, "Selected token violates the generation constraint");
  }
  *state_out = s;
  return GS_OK;
}

int gs_legal_token_ids(gs_context* ctx, int32_t state, int32_t* ids, int32_t cap, int32_t* n_out) {
  if (!ctx || !n_out || cap < 0 || (cap > 0 && !ids)) return fail(ctx, GS_ERR_INVALID_ARGUMENT, "bad arguments");
  if (!ctx->d_next || !ctx->d_vocab_offsets) return fail(ctx, GS_ERR_INVALID_ARGUMENT, "set the vocab and the DFA first");
  if (state < 0 || state >= ctx->n_states) return fail(ctx, GS_ERR_INVALID_ARGUMENT, "state out of range");
  GS_HIP(ctx, hipSetDevice(ctx->device));
  int st = ensure_stage(ctx, sizeof(uint32_t) * ctx->mask_words);
  if (st != GS_OK) return st;
  st = gs_build_masks(ctx, &state, 1, (uint32_t*)ctx->d_stage, ctx->stream);
  if (st != GS_OK) return st;
  std::vector<uint32_t> words(ctx->mask_words);
  GS_HIP(ctx, hipMemcpyAsync(words.data(), ctx->d_stage, sizeof(uint32_t) * words.size(), hipMemcpyDeviceToHost,
                             ctx->stream));
  GS_HIP(ctx, hipStreamSynchronize(ctx->stream));
  int32_t count = 0;
  for (int32_t w = 0; w < ctx->mask_words; ++w) {
    for (uint32_t bits = words[w]; bits; bits &= bits - 1) {
      const int32_t id = w * 32 + __builtin_ctz(bits);
      if (id >= ctx->vocab) break;
      if (count < cap) ids[count] = id;
      ++count;
    }
  }
  *n_out = count;
  return GS_OK;
}

int gs_dfa_accepting(gs_context* ctx, int32_t state, int32_t* out) {
  if (!ctx || !out || state < 0 || state >= ctx->n_states) return fail(ctx, GS_ERR_INVALID_ARGUMENT, "bad state");
  *out = ctx->finals[state] ? 1 : 0;
  return GS_OK;
}

int gs_lmhead(gs_context* ctx, const void* hidden, const void* weight, int32_t m_rows, int32_t width, float softcap,
              float* logits, void* stream) {
  if (!ctx || !hidden || !weight || !logits || m_rows <= 0 || width <= 0) return fail(ctx, GS_ERR_INVALID_ARGUMENT, "bad arguments");
  if (width % 64 != 0) return fail(ctx, GS_ERR_UNSUPPORTED, "lm_head width must be a multiple of 64");
  if (!aligned16(hidden) || !aligned16(weight)) return fail(ctx, GS_ERR_INVALID_ARGUMENT, "hidden and weight must be 16-byte aligned");
  GS_HIP(ctx, hipSetDevice(ctx->device));
  hipStream_t s = pick_stream(ctx, stream);
  const int32_t slot = timing_slot(ctx);
  launch_lmhead((const uint16_t*)hidden, (const uint16_t*)weight, m_rows, width, ctx->vocab, softcap, logits,
                ctx->cu_count, s, stage_events(ctx, slot, GS_STAGE_LMHEAD));
  GS_HIP(ctx, hipGetLastError());
  return GS_OK;
}

int gs_qat_lmhead(gs_context* ctx, const float* x, int32_t m_rows, int32_t width, const uint32_t* packed_codes,
                  int32_t layout, const float* row_scales, float input_scale, float output_scale, float* logits,
                  void* stream) {
  if (!ctx || !x || !packed_codes || !row_scales || !logits || m_rows <= 0 || width <= 0)
    return fail(ctx, GS_ERR_INVALID_ARGUMENT, "bad arguments");
  if (width % 64 != 0 || width > 4096) return fail(ctx, GS_ERR_UNSUPPORTED, "QAT lm_head width must be a multiple of 64, at most 4096");
  if (layout != GS_QAT_ROW_MAJOR && layout != GS_QAT_BLOCK_MAJOR) return fail(ctx, GS_ERR_INVALID_ARGUMENT, "unknown QAT weight layout");
  if (!aligned16(x) || !aligned16(packed_codes)) return fail(ctx, GS_ERR_INVALID_ARGUMENT, "x and the codes must be 16-byte aligned");
  if (!(input_scale >= 0) || !(output_scale >= 0)) return fail(ctx, GS_ERR_INVALID_ARGUMENT, "SRQ scales must be >= 0");
  GS_HIP(ctx, hipSetDevice(ctx->device));
  hipStream_t s = pick_stream(ctx, stream);
  const int32_t slot = timing_slot(ctx);
  launch_qat_lmhead(x, m_rows, width, packed_codes, layout == GS_QAT_BLOCK_MAJOR, row_scales, ctx->vocab, input_scale,
                    output_scale, logits, ctx->cu_count, s, stage_events(ctx, slot, GS_STAGE_LMHEAD));
  GS_HIP(ctx, hipGetLastError());
  return GS_OK;
}

int gs_qat_lmhead_sample(gs_context* ctx, const float* x, int32_t width, const uint32_t* packed_codes,
                         int32_t layout, const float* row_scales, float input_scale, float output_scale,
                         float* logits_scratch, const gs_batch* batch, void* stream) {
  if (!batch) return fail(ctx, GS_ERR_INVALID_ARGUMENT, "bad arguments");
  int st = gs_qat_lmhead(ctx, x, batch->rows, width, packed_codes, layout, row_scales, input_scale, output_scale,
                         logits_scratch, stream);
  if (st != GS_OK) return st;
  gs_batch b = *batch;
  b.logits = logits_scratch;
  b.dtype = GS_F32;
  b.row_stride = ctx->vocab;
  return gs_sample(ctx, &b, stream);
}

int gs_lmhead_sample(gs_context* ctx, const void* hidden, const void* weight, int32_t width, float softcap,
                     float* logits_scratch, const gs_batch* batch, void* stream) {
  if (!batch) return fail(ctx, GS_ERR_INVALID_ARGUMENT, "null batch");
  if (!ctx) return GS_ERR_INVALID_ARGUMENT;
  if (!(batch->hints & GS_BATCH_FUSED_HEAD) || ctx->vocab % kChunk != 0) {
    // the lm_head, then the chunk scan over its output (the faster of the two
    // at 64 x 2048 x 262144, and the path for vocabularies of partial chunks)
    int st = gs_lmhead(ctx, hidden, weight, batch->rows, width, softcap, logits_scratch, stream);
    if (st != GS_OK) return st;
    gs_batch b = *batch;
    b.logits = logits_scratch;
    b.dtype = GS_F32;
    b.row_stride = ctx->vocab;
    return gs_sample(ctx, &b, stream);
  }
  if (!hidden || !weight || !logits_scratch || width <= 0) return fail(ctx, GS_ERR_INVALID_ARGUMENT, "bad arguments");
  if (width % 64 != 0) return fail(ctx, GS_ERR_UNSUPPORTED, "lm_head width must be a multiple of 64");
  if (!aligned16(hidden) || !aligned16(weight) || !aligned16(logits_scratch))
    return fail(ctx, GS_ERR_INVALID_ARGUMENT, "hidden, weight and logits_scratch must be 16-byte aligned");
  gs_batch b = *batch;
  b.logits = logits_scratch;
  b.dtype = GS_F32;
  b.row_stride = ctx->vocab;
  if (b.rows == 0) return GS_OK;
  if (b.rows < 0 || b.rows > ctx->max_rows) return fail(ctx, GS_ERR_INVALID_ARGUMENT, "rows outside [0, max_rows]");
  const char* bad = batch_error(&b, ctx->vocab);
  if (bad) return fail(ctx, GS_ERR_INVALID_ARGUMENT, bad);
  GS_HIP(ctx, hipSetDevice(ctx->device));
  const int st = ensure_fused(ctx, b.rows);
  if (st != GS_OK) return st;
  const Workspace w = context_workspace(ctx);
  FusedArgs f{};
  f.configs = b.configs;
  f.dead = ctx->d_dead;
  f.parts = ctx->d_parts;
  f.plists = ctx->d_plists;
  f.row_thr = ctx->d_row_thr;
  f.n_parts = ctx->vocab / kPartIds;
  const int32_t slot = timing_slot(ctx);
  LaunchEvents ev[GS_STAGE_COUNT];
  for (int k = GS_STAGE_LMHEAD; k <= GS_STAGE_FINISH; ++k) ev[k] = stage_events(ctx, slot, k);
  if (deep_launch(w, &b)) ev[GS_STAGE_DEEP] = stage_events(ctx, slot, GS_STAGE_DEEP);
  if (b.rows > ctx->exact_slots) ev[GS_STAGE_EXACT] = stage_events(ctx, slot, GS_STAGE_EXACT);
  hipStream_t s = pick_stream(ctx, stream);
  launch_lmhead_scan((const uint16_t*)hidden, (const uint16_t*)weight, b.rows, width, softcap, logits_scratch,
                     sample_args(w, &b), f, s, ev[GS_STAGE_LMHEAD]);
  hipError_t e = hipGetLastError();
  if (e == hipSuccess) e = launch_sample(w, &b, s, ev, &f);
  if (e != hipSuccess) return fail(ctx, GS_ERR_HIP, std::string("kernel launch: ") + hipGetErrorString(e));
  if (slot >= 0) ctx->t_calls++;
  return GS_OK;
}

int gs_timing_begin(gs_context* ctx, int32_t max_calls) {
  if (!ctx || max_calls <= 0 || max_calls > 100000) return fail(ctx, GS_ERR_INVALID_ARGUMENT, "max_calls must be 1..100000");
  GS_HIP(ctx, hipSetDevice(ctx->device));
  destroy_timing(ctx);
  ctx->t_events.assign((size_t)max_calls * GS_STAGE_COUNT * 2, nullptr);
  ctx->t_ran.assign((size_t)max_calls * GS_STAGE_COUNT, 0);
  for (hipEvent_t& e : ctx->t_events) {
    if (hipEventCreate(&e) != hipSuccess) {
      destroy_timing(ctx);
      return fail(ctx, GS_ERR_HIP, "hipEventCreate failed");
    }
  }
  ctx->t_cap = max_calls;
  ctx->t_calls = 0;
  ctx->t_on = true;
  return GS_OK;
}

int gs_timing_end(gs_context* ctx, double* stage_ms, int32_t* calls) {
  if (!ctx || !stage_ms || !calls) return fail(ctx, GS_ERR_INVALID_ARGUMENT, "bad arguments");
  if (!ctx->t_on) return fail(ctx, GS_ERR_INVALID_ARGUMENT, "timing was not started");
  GS_HIP(ctx, hipSetDevice(ctx->device));
  for (int k = 0; k < GS_STAGE_COUNT; ++k) { stage_ms[k] = 0.0; calls[k] = 0; }
  int st = GS_OK;
  for (int32_t c = 0; c < ctx->t_calls && st == GS_OK; ++c) {
    for (int k = 0; k < GS_STAGE_COUNT; ++k) {
      if (!ctx->t_ran[(size_t)c * GS_STAGE_COUNT + k]) continue;
      hipEvent_t e0 = ctx->t_events[((size_t)c * GS_STAGE_COUNT + k) * 2];
      hipEvent_t e1 = ctx->t_events[((size_t)c * GS_STAGE_COUNT + k) * 2 + 1];
      float ms = 0.0f;
      if (hipEventSynchronize(e1) != hipSuccess || hipEventElapsedTime(&ms, e0, e1) != hipSuccess) {
        st = fail(ctx, GS_ERR_HIP, "reading a timing event failed");
        break;
      }
      stage_ms[k] += ms;
      calls[k] += 1;
    }
  }
  destroy_timing(ctx);
  return st;
}

}  // extern "C"
