/*
 * N-API addon over libgsample's C ABI (include/gsample.h): one JavaScript
 * function per entry point, no logic of its own beyond argument unpacking.
 * A non-zero gs_status becomes a thrown Error whose message is
 * gs_last_error()'s text -- for the reference's error conditions that is the
 * reference's own message (src/runtime/sampling.ts:19,69;
 * src/runtime/generation-config.ts:65,67; src/runtime/constraints.ts:99;
 * src/runtime/gemma-session.ts:1325) -- and whose `code` is the status name.
 *
 * Handles: a context is an External over a small box (so an explicit
 * destroy() and the garbage collector's finalizer cannot both free it);
 * device memory is an External over the raw device address, owned by the
 * JavaScript DeviceBuffer wrapper.
 */
#define NAPI_VERSION 8
#include <node_api.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "gsample.h"

typedef struct ctx_box {
  gs_context* ctx;
} ctx_box;

static const char* status_name(int st) {
  switch (st) {
    case GS_OK: return "GS_OK";
    case GS_ERR_INVALID_ARGUMENT: return "GS_ERR_INVALID_ARGUMENT";
    case GS_ERR_INVALID_CONFIG: return "GS_ERR_INVALID_CONFIG";
    case GS_ERR_EMPTY_LOGITS: return "GS_ERR_EMPTY_LOGITS";
    case GS_ERR_DEAD_END: return "GS_ERR_DEAD_END";
    case GS_ERR_CONSTRAINT_VIOLATION: return "GS_ERR_CONSTRAINT_VIOLATION";
    case GS_ERR_TOKEN_RANGE: return "GS_ERR_TOKEN_RANGE";
    case GS_ERR_STOP_TOKEN_RANGE: return "GS_ERR_STOP_TOKEN_RANGE";
    case GS_ERR_EMPTY_CANDIDATES: return "GS_ERR_EMPTY_CANDIDATES";
    case GS_ERR_UNSUPPORTED: return "GS_ERR_UNSUPPORTED";
    case GS_ERR_HIP: return "GS_ERR_HIP";
    case GS_ERR_NO_DEVICE: return "GS_ERR_NO_DEVICE";
    default: return "GS_ERR_UNKNOWN";
  }
}

/* Throws Error(message) with .code = code; returns NULL for the caller to return. */
static napi_value throw_error(napi_env env, const char* code, const char* message) {
  napi_value msg, err, code_v;
  napi_create_string_utf8(env, message, NAPI_AUTO_LENGTH, &msg);
  napi_create_error(env, NULL, msg, &err);
  napi_create_string_utf8(env, code, NAPI_AUTO_LENGTH, &code_v);
  napi_set_named_property(env, err, "code", code_v);
  napi_throw(env, err);
  return NULL;
}

static napi_value throw_status(napi_env env, gs_context* ctx, int st) {
  const char* m = gs_last_error(ctx);
  if (st == GS_ERR_NO_DEVICE && (!m || !*m || strcmp(m, "no context") == 0)) m = "no HIP device is available";
  return throw_error(env, status_name(st), m && *m ? m : status_name(st));
}

#define CHECK_NAPI(call)                                                     \
  do {                                                                       \
    if ((call) != napi_ok) return throw_error(env, "GS_NAPI", "N-API call failed: " #call); \
  } while (0)

#define GS_CALL(ctx, call)                                \
  do {                                                    \
    int st_ = (call);                                     \
    if (st_ != GS_OK) return throw_status(env, (ctx), st_); \
  } while (0)

#define ARGS(n)                                                          \
  size_t argc = (n);                                                     \
  napi_value argv[(n) > 0 ? (n) : 1];                                    \
  CHECK_NAPI(napi_get_cb_info(env, info, &argc, argv, NULL, NULL));

static int is_nullish(napi_env env, napi_value v) {
  napi_valuetype t;
  if (napi_typeof(env, v, &t) != napi_ok) return 1;
  return t == napi_null || t == napi_undefined;
}

static int get_f64(napi_env env, napi_value v, double* out) { return napi_get_value_double(env, v, out) == napi_ok; }

static int get_i32(napi_env env, napi_value v, int32_t* out) { return napi_get_value_int32(env, v, out) == napi_ok; }

static int get_i64(napi_env env, napi_value v, int64_t* out) { return napi_get_value_int64(env, v, out) == napi_ok; }

/* A typed array's data pointer and element count; `want` < 0 accepts any type. */
static int get_typed(napi_env env, napi_value v, int want, void** data, size_t* count) {
  bool is_ta = false;
  if (napi_is_typedarray(env, v, &is_ta) != napi_ok || !is_ta) return 0;
  napi_typedarray_type type;
  napi_value ab;
  size_t off;
  if (napi_get_typedarray_info(env, v, &type, count, data, &ab, &off) != napi_ok) return 0;
  return want < 0 || (int)type == want;
}

static gs_context* get_ctx(napi_env env, napi_value v) {
  ctx_box* box = NULL;
  if (napi_get_value_external(env, v, (void**)&box) != napi_ok || !box) return NULL;
  return box->ctx;
}

static void* get_ptr(napi_env env, napi_value v) {
  void* p = NULL;
  if (napi_get_value_external(env, v, &p) != napi_ok) return NULL;
  return p;
}

static napi_value make_f64(napi_env env, double x) {
  napi_value r;
  napi_create_double(env, x, &r);
  return r;
}

static napi_value make_i32(napi_env env, int32_t x) {
  napi_value r;
  napi_create_int32(env, x, &r);
  return r;
}

/* A new typed array of `count` elements; *data points at its storage. */
static napi_value new_typed(napi_env env, napi_typedarray_type type, size_t elem, size_t count, void** data) {
  napi_value ab, ta;
  if (napi_create_arraybuffer(env, elem * count, data, &ab) != napi_ok) return NULL;
  if (napi_create_typedarray(env, type, count, ab, 0, &ta) != napi_ok) return NULL;
  return ta;
}

/* Widens an Int32Array of CSR offsets to int64 (caller frees). */
static int64_t* widen_offsets(napi_env env, napi_value v, size_t want_count, int* ok) {
  void* data;
  size_t n;
  *ok = 0;
  if (!get_typed(env, v, napi_int32_array, &data, &n) || n != want_count) return NULL;
  int64_t* w = (int64_t*)malloc(sizeof(int64_t) * (n ? n : 1));
  if (!w) return NULL;
  for (size_t i = 0; i < n; ++i) w[i] = ((const int32_t*)data)[i];
  *ok = 1;
  return w;
}

/* ---- identity and host math ---------------------------------------- */

static napi_value js_abi_version(napi_env env, napi_callback_info info) {
  (void)info;
  return make_i32(env, gs_abi_version());
}

static napi_value js_device_count(napi_env env, napi_callback_info info) {
  (void)info;
  int n = 0;
  gs_device_count(&n);
  return make_i32(env, n);
}

static napi_value js_seeded_random(napi_env env, napi_callback_info info) {
  ARGS(2);
  int64_t seed, index;
  if (argc < 2 || !get_i64(env, argv[0], &seed) || !get_i64(env, argv[1], &index) || index < 0)
    return throw_error(env, "GS_ERR_INVALID_ARGUMENT", "seededRandom(seed, index) needs integers, index >= 0");
  return make_f64(env, gs_seeded_random(seed, (uint64_t)index));
}

static napi_value js_exp(napi_env env, napi_callback_info info) {
  ARGS(1);
  double x;
  if (argc < 1 || !get_f64(env, argv[0], &x)) return throw_error(env, "GS_ERR_INVALID_ARGUMENT", "jsExp(x)");
  return make_f64(env, gs_js_exp(x));
}

static napi_value js_log(napi_env env, napi_callback_info info) {
  ARGS(1);
  double x;
  if (argc < 1 || !get_f64(env, argv[0], &x)) return throw_error(env, "GS_ERR_INVALID_ARGUMENT", "jsLog(x)");
  return make_f64(env, gs_js_log(x));
}

static napi_value js_softcap(napi_env env, napi_callback_info info) {
  ARGS(2);
  double x, cap;
  if (argc < 2 || !get_f64(env, argv[0], &x) || !get_f64(env, argv[1], &cap))
    return throw_error(env, "GS_ERR_INVALID_ARGUMENT", "softcap(x, cap)");
  return make_f64(env, (double)gs_softcap((float)x, cap));
}

static void set_num(napi_env env, napi_value obj, const char* name, double v) {
  napi_set_named_property(env, obj, name, make_f64(env, v));
}

/* Byte layout of gs_row_config and gs_row_result, so the JavaScript side
 * packs exactly what this library was compiled with. */
static napi_value js_layouts(napi_env env, napi_callback_info info) {
  (void)info;
  napi_value out, cfg, res;
  napi_create_object(env, &out);
  napi_create_object(env, &cfg);
  napi_create_object(env, &res);
#define OFF(obj, T, f) set_num(env, obj, #f, (double)offsetof(T, f))
  set_num(env, cfg, "size", (double)sizeof(gs_row_config));
  OFF(cfg, gs_row_config, temperature);
  OFF(cfg, gs_row_config, top_p);
  OFF(cfg, gs_row_config, min_p);
  OFF(cfg, gs_row_config, typical_p);
  OFF(cfg, gs_row_config, repetition_penalty);
  OFF(cfg, gs_row_config, frequency_penalty);
  OFF(cfg, gs_row_config, presence_penalty);
  OFF(cfg, gs_row_config, softcap);
  OFF(cfg, gs_row_config, uniform);
  OFF(cfg, gs_row_config, seed);
  OFF(cfg, gs_row_config, draw_index);
  OFF(cfg, gs_row_config, top_k);
  OFF(cfg, gs_row_config, repetition_window);
  OFF(cfg, gs_row_config, rng_mode);
  OFF(cfg, gs_row_config, mask_slot);
  OFF(cfg, gs_row_config, accepting);
  OFF(cfg, gs_row_config, options);
  set_num(env, res, "size", (double)sizeof(gs_row_result));
  OFF(res, gs_row_result, token);
  OFF(res, gs_row_result, flags);
  OFF(res, gs_row_result, probability);
#undef OFF
  napi_set_named_property(env, out, "rowConfig", cfg);
  napi_set_named_property(env, out, "rowResult", res);
  return out;
}

/* validateConfigs(packedConfigs: Uint8Array): throws the joined reference
 * message on the first invalid row. */
static napi_value js_validate_configs(napi_env env, napi_callback_info info) {
  ARGS(1);
  void* data;
  size_t n;
  if (argc < 1 || !get_typed(env, argv[0], napi_uint8_array, &data, &n) || n % sizeof(gs_row_config))
    return throw_error(env, "GS_ERR_INVALID_ARGUMENT", "validateConfigs needs packed row configs (Uint8Array)");
  GS_CALL(NULL, gs_validate_configs(NULL, (const gs_row_config*)data, (int32_t)(n / sizeof(gs_row_config))));
  return NULL;
}

/* ---- contexts -------------------------------------------------------- */

static void ctx_finalize(napi_env env, void* data, void* hint) {
  (void)env;
  (void)hint;
  ctx_box* box = (ctx_box*)data;
  if (box->ctx) gs_destroy(box->ctx);
  free(box);
}

static napi_value js_create(napi_env env, napi_callback_info info) {
  ARGS(3);
  int32_t device, vocab, max_rows;
  if (argc < 3 || !get_i32(env, argv[0], &device) || !get_i32(env, argv[1], &vocab) || !get_i32(env, argv[2], &max_rows))
    return throw_error(env, "GS_ERR_INVALID_ARGUMENT", "create(device, vocabSize, maxRows)");
  gs_context* ctx = NULL;
  int st = gs_create(device, vocab, max_rows, &ctx);
  if (st != GS_OK) {
    if (st == GS_ERR_NO_DEVICE) return throw_error(env, status_name(st), "no HIP device is available");
    if (st == GS_ERR_UNSUPPORTED) return throw_error(env, status_name(st), "vocab size beyond 2097152 is not supported");
    return throw_error(env, status_name(st), "gs_create failed");
  }
  ctx_box* box = (ctx_box*)malloc(sizeof(ctx_box));
  if (!box) {
    gs_destroy(ctx);
    return throw_error(env, "GS_ERR_INVALID_ARGUMENT", "out of host memory");
  }
  box->ctx = ctx;
  napi_value ext;
  CHECK_NAPI(napi_create_external(env, box, ctx_finalize, NULL, &ext));
  return ext;
}

static napi_value js_destroy(napi_env env, napi_callback_info info) {
  ARGS(1);
  ctx_box* box = NULL;
  if (argc < 1 || napi_get_value_external(env, argv[0], (void**)&box) != napi_ok || !box)
    return throw_error(env, "GS_ERR_INVALID_ARGUMENT", "destroy(context)");
  if (box->ctx) gs_destroy(box->ctx);
  box->ctx = NULL;
  return NULL;
}

#define CTX_ARG(i)                                                                    \
  gs_context* ctx = (argc > (i)) ? get_ctx(env, argv[(i)]) : NULL;                    \
  if (!ctx) return throw_error(env, "GS_ERR_INVALID_ARGUMENT", "a live context is required");

static napi_value js_synchronize(napi_env env, napi_callback_info info) {
  ARGS(1);
  CTX_ARG(0);
  GS_CALL(ctx, gs_synchronize(ctx));
  return NULL;
}

/* ---- device memory ------------------------------------------------------ */

static napi_value js_device_alloc(napi_env env, napi_callback_info info) {
  ARGS(2);
  CTX_ARG(0);
  int64_t bytes;
  if (!get_i64(env, argv[1], &bytes) || bytes < 0) return throw_error(env, "GS_ERR_INVALID_ARGUMENT", "deviceAlloc(ctx, bytes)");
  void* p = NULL;
  GS_CALL(ctx, gs_device_alloc(ctx, (size_t)bytes, &p));
  napi_value ext;
  CHECK_NAPI(napi_create_external(env, p, NULL, NULL, &ext));
  return ext;
}

static napi_value js_device_free(napi_env env, napi_callback_info info) {
  ARGS(2);
  CTX_ARG(0);
  GS_CALL(ctx, gs_device_free(ctx, get_ptr(env, argv[1])));
  return NULL;
}

/* copyToDevice(ctx, deviceExt, byteOffset, typedArray) */
static napi_value js_copy_to_device(napi_env env, napi_callback_info info) {
  ARGS(4);
  CTX_ARG(0);
  void* dst = argc > 1 ? get_ptr(env, argv[1]) : NULL;
  int64_t off;
  void* src;
  size_t n;
  if (!dst || !get_i64(env, argv[2], &off) || off < 0 || !get_typed(env, argv[3], -1, &src, &n))
    return throw_error(env, "GS_ERR_INVALID_ARGUMENT", "copyToDevice(ctx, buffer, byteOffset, typedArray)");
  napi_typedarray_type t;
  napi_value ab;
  size_t o, len;
  void* d2;
  napi_get_typedarray_info(env, argv[3], &t, &len, &d2, &ab, &o);
  size_t esz = (t == napi_float64_array) ? 8 : (t == napi_float32_array || t == napi_int32_array || t == napi_uint32_array) ? 4
             : (t == napi_int16_array || t == napi_uint16_array) ? 2 : 1;
  GS_CALL(ctx, gs_copy_to_device(ctx, (uint8_t*)dst + off, src, n * esz));
  return NULL;
}

/* copyToHost(ctx, typedArray, deviceExt, byteOffset) */
static napi_value js_copy_to_host(napi_env env, napi_callback_info info) {
  ARGS(4);
  CTX_ARG(0);
  void* dst;
  size_t n;
  void* src = argc > 2 ? get_ptr(env, argv[2]) : NULL;
  int64_t off;
  if (!src || !get_typed(env, argv[1], -1, &dst, &n) || !get_i64(env, argv[3], &off) || off < 0)
    return throw_error(env, "GS_ERR_INVALID_ARGUMENT", "copyToHost(ctx, typedArray, buffer, byteOffset)");
  napi_typedarray_type t;
  napi_value ab;
  size_t o, len;
  void* d2;
  napi_get_typedarray_info(env, argv[1], &t, &len, &d2, &ab, &o);
  size_t esz = (t == napi_float64_array) ? 8 : (t == napi_float32_array || t == napi_int32_array || t == napi_uint32_array) ? 4
             : (t == napi_int16_array || t == napi_uint16_array) ? 2 : 1;
  GS_CALL(ctx, gs_copy_to_host(ctx, dst, (const uint8_t*)src + off, n * esz));
  return NULL;
}

/* ---- sampling ------------------------------------------------------------ */

/* sampleHost(ctx, logits, dtype, rows, rowStride, configs, histOffsets, histIds,
 *            forcedOffsets, forcedIds, forcedKinds, maskTable, maskSlots, results)
 * logits: Float32Array / Uint16Array (bf16 bits) on the host, or a device
 * External; offsets: Int32Array [rows+1] or null; maskTable: device External
 * or null; results: Uint8Array of rows * sizeof(gs_row_result). */
static napi_value js_sample_host(napi_env env, napi_callback_info info) {
  ARGS(14);
  CTX_ARG(0);
  if (argc < 14) return throw_error(env, "GS_ERR_INVALID_ARGUMENT", "sampleHost needs 14 arguments");
  gs_batch b;
  memset(&b, 0, sizeof(b));
  int32_t on_device = 0;
  void* data;
  size_t n;
  if (get_typed(env, argv[1], -1, &data, &n)) {
    b.logits = data;
  } else {
    b.logits = get_ptr(env, argv[1]);
    on_device = 1;
  }
  int64_t stride;
  if (!b.logits || !get_i32(env, argv[2], &b.dtype) || !get_i32(env, argv[3], &b.rows) || !get_i64(env, argv[4], &stride))
    return throw_error(env, "GS_ERR_INVALID_ARGUMENT", "sampleHost: logits, dtype, rows, rowStride");
  b.row_stride = stride;
  if (b.rows < 0) return throw_error(env, "GS_ERR_INVALID_ARGUMENT", "rows must be >= 0");
  if (!on_device) {
    const size_t esize = b.dtype == GS_BF16 ? 2 : 4;
    napi_typedarray_type t;
    napi_value ab;
    size_t o, len;
    napi_get_typedarray_info(env, argv[1], &t, &len, &data, &ab, &o);
    if ((b.dtype == GS_F32 && t != napi_float32_array) || (b.dtype == GS_BF16 && t != napi_uint16_array))
      return throw_error(env, "GS_ERR_INVALID_ARGUMENT", "logits must be a Float32Array (f32) or Uint16Array (bf16 bits)");
    (void)esize;
    /* the library stages rows x rowStride elements' worth (the last row's
       padding included), so the array must hold all of it */
    if (stride < 1 || (int64_t)len < (int64_t)b.rows * stride)
      return throw_error(env, "GS_ERR_INVALID_ARGUMENT", "logits array is shorter than rows x rowStride");
  }
  if (!get_typed(env, argv[5], napi_uint8_array, &data, &n) || n != (size_t)b.rows * sizeof(gs_row_config))
    return throw_error(env, "GS_ERR_INVALID_ARGUMENT", "configs must be rows packed gs_row_config (Uint8Array)");
  b.configs = (const gs_row_config*)data;
  int64_t* hoff = NULL;
  int64_t* foff = NULL;
  int ok = 1;
  napi_value result = NULL;
  if (!is_nullish(env, argv[6])) {
    hoff = widen_offsets(env, argv[6], (size_t)b.rows + 1, &ok);
    if (!ok) goto bad_args;
    if (!get_typed(env, argv[7], napi_int32_array, &data, &n) || (int64_t)n < hoff[b.rows]) goto bad_args;
    b.history_offsets = hoff;
    b.history_ids = (const int32_t*)data;
  }
  if (!is_nullish(env, argv[8])) {
    foff = widen_offsets(env, argv[8], (size_t)b.rows + 1, &ok);
    if (!ok) goto bad_args;
    if (!get_typed(env, argv[9], napi_int32_array, &data, &n) || (int64_t)n < foff[b.rows]) goto bad_args;
    b.forced_offsets = foff;
    b.forced_ids = (const int32_t*)data;
    if (!get_typed(env, argv[10], napi_uint8_array, &data, &n) || (int64_t)n < foff[b.rows]) goto bad_args;
    b.forced_kinds = (const uint8_t*)data;
  }
  if (!is_nullish(env, argv[11])) {
    b.mask_table = (const uint32_t*)get_ptr(env, argv[11]);
    if (!b.mask_table || !get_i32(env, argv[12], &b.mask_slots)) goto bad_args;
  }
  if (!get_typed(env, argv[13], napi_uint8_array, &data, &n) || n != (size_t)b.rows * sizeof(gs_row_result)) goto bad_args;
  {
    int st = gs_sample_host(ctx, &b, on_device, (gs_row_result*)data);
    free(hoff);
    free(foff);
    if (st != GS_OK) return throw_status(env, ctx, st);
    return result;
  }
bad_args:
  free(hoff);
  free(foff);
  return throw_error(env, "GS_ERR_INVALID_ARGUMENT",
                     "sampleHost: offsets must be Int32Array[rows+1] with matching id arrays, results Uint8Array");
}

/* tokenLogProbHost(ctx, logits Float32Array [rows*V], rows, tokens Int32Array) -> Float64Array */
static napi_value js_token_log_prob_host(napi_env env, napi_callback_info info) {
  ARGS(4);
  CTX_ARG(0);
  void *lg, *tk;
  size_t nl, nt;
  int32_t rows;
  if (!get_typed(env, argv[1], napi_float32_array, &lg, &nl) || !get_i32(env, argv[2], &rows) || rows < 0 ||
      !get_typed(env, argv[3], napi_int32_array, &tk, &nt) || nt < (size_t)rows)
    return throw_error(env, "GS_ERR_INVALID_ARGUMENT", "tokenLogProbHost(ctx, Float32Array, rows, Int32Array)");
  void* out;
  napi_value arr = new_typed(env, napi_float64_array, 8, (size_t)rows, &out);
  if (!arr) return throw_error(env, "GS_NAPI", "allocation failed");
  GS_CALL(ctx, gs_token_log_prob_host(ctx, (const float*)lg, rows, (const int32_t*)tk, (double*)out));
  return arr;
}

/* maskLogitsHost(ctx, raw Float32Array, legal Int32Array, termination Int32Array) -> Float32Array */
static napi_value js_mask_logits_host(napi_env env, napi_callback_info info) {
  ARGS(4);
  CTX_ARG(0);
  void *raw, *legal, *term;
  size_t n, nl, nt;
  if (!get_typed(env, argv[1], napi_float32_array, &raw, &n) || !get_typed(env, argv[2], napi_int32_array, &legal, &nl) ||
      !get_typed(env, argv[3], napi_int32_array, &term, &nt))
    return throw_error(env, "GS_ERR_INVALID_ARGUMENT", "maskLogitsHost(ctx, Float32Array, Int32Array, Int32Array)");
  void* out;
  napi_value arr = new_typed(env, napi_float32_array, 4, n, &out);
  if (!arr) return throw_error(env, "GS_NAPI", "allocation failed");
  GS_CALL(ctx, gs_mask_logits_host(ctx, (const float*)raw, (int64_t)n, (const int32_t*)legal, (int64_t)nl,
                                   (const int32_t*)term, (int64_t)nt, (float*)out));
  return arr;
}

/* ---- constraint tables ------------------------------------------------------ */

/* setVocab(ctx, offsets Int32Array [V+1], bytes Uint8Array) */
static napi_value js_set_vocab(napi_env env, napi_callback_info info) {
  ARGS(3);
  CTX_ARG(0);
  void *off, *bytes;
  size_t no, nb;
  if (!get_typed(env, argv[1], napi_int32_array, &off, &no) || !get_typed(env, argv[2], napi_uint8_array, &bytes, &nb))
    return throw_error(env, "GS_ERR_INVALID_ARGUMENT", "setVocab(ctx, Int32Array offsets, Uint8Array bytes)");
  int64_t* w = (int64_t*)malloc(sizeof(int64_t) * (no ? no : 1));
  if (!w) return throw_error(env, "GS_NAPI", "allocation failed");
  for (size_t i = 0; i < no; ++i) w[i] = ((const int32_t*)off)[i];
  int st = gs_set_vocab(ctx, w, (const uint8_t*)bytes, (int64_t)nb);
  free(w);
  if (st != GS_OK) return throw_status(env, ctx, st);
  return NULL;
}

/* setDfa(ctx, nStates, next Int32Array [nStates*256], finals Uint8Array [nStates]) */
static napi_value js_set_dfa(napi_env env, napi_callback_info info) {
  ARGS(4);
  CTX_ARG(0);
  int32_t ns;
  void *next, *fin;
  size_t nn, nf;
  if (!get_i32(env, argv[1], &ns) || ns <= 0 || !get_typed(env, argv[2], napi_int32_array, &next, &nn) ||
      nn != (size_t)ns * 256 || !get_typed(env, argv[3], napi_uint8_array, &fin, &nf) || nf != (size_t)ns)
    return throw_error(env, "GS_ERR_INVALID_ARGUMENT", "setDfa(ctx, nStates, Int32Array next, Uint8Array finals)");
  GS_CALL(ctx, gs_set_dfa(ctx, ns, (const int32_t*)next, (const uint8_t*)fin));
  return NULL;
}

/* buildMasks(ctx, states Int32Array, maskTable device External) */
static napi_value js_build_masks(napi_env env, napi_callback_info info) {
  ARGS(3);
  CTX_ARG(0);
  void* st_data;
  size_t n;
  void* table = argc > 2 ? get_ptr(env, argv[2]) : NULL;
  if (!get_typed(env, argv[1], napi_int32_array, &st_data, &n) || !table)
    return throw_error(env, "GS_ERR_INVALID_ARGUMENT", "buildMasks(ctx, Int32Array states, maskTable)");
  GS_CALL(ctx, gs_build_masks(ctx, (const int32_t*)st_data, (int32_t)n, (uint32_t*)table, NULL));
  GS_CALL(ctx, gs_synchronize(ctx));
  return NULL;
}

/* legalTokenIds(ctx, state) -> Int32Array (ascending) */
static napi_value js_legal_token_ids(napi_env env, napi_callback_info info) {
  ARGS(2);
  CTX_ARG(0);
  int32_t state, count = 0;
  if (!get_i32(env, argv[1], &state)) return throw_error(env, "GS_ERR_INVALID_ARGUMENT", "legalTokenIds(ctx, state)");
  GS_CALL(ctx, gs_legal_token_ids(ctx, state, NULL, 0, &count));
  void* out;
  napi_value arr = new_typed(env, napi_int32_array, 4, (size_t)count, &out);
  if (!arr) return throw_error(env, "GS_NAPI", "allocation failed");
  int32_t again = 0;
  GS_CALL(ctx, gs_legal_token_ids(ctx, state, (int32_t*)out, count, &again));
  return arr;
}

/* dfaAdvance(ctx, states Int32Array, tokens Int32Array) -> Int32Array */
static napi_value js_dfa_advance(napi_env env, napi_callback_info info) {
  ARGS(3);
  CTX_ARG(0);
  void *si, *tk;
  size_t ns, nt;
  if (!get_typed(env, argv[1], napi_int32_array, &si, &ns) || !get_typed(env, argv[2], napi_int32_array, &tk, &nt) ||
      ns != nt)
    return throw_error(env, "GS_ERR_INVALID_ARGUMENT", "dfaAdvance(ctx, Int32Array states, Int32Array tokens)");
  void* out;
  napi_value arr = new_typed(env, napi_int32_array, 4, ns, &out);
  if (!arr) return throw_error(env, "GS_NAPI", "allocation failed");
  GS_CALL(ctx, gs_dfa_advance(ctx, (const int32_t*)si, (const int32_t*)tk, (int32_t)ns, (int32_t*)out));
  return arr;
}

/* dfaAdvanceBytes(ctx, state, bytes Uint8Array) -> state */
static napi_value js_dfa_advance_bytes(napi_env env, napi_callback_info info) {
  ARGS(3);
  CTX_ARG(0);
  int32_t state, out = -1;
  void* bytes;
  size_t n;
  if (!get_i32(env, argv[1], &state) || !get_typed(env, argv[2], napi_uint8_array, &bytes, &n))
    return throw_error(env, "GS_ERR_INVALID_ARGUMENT", "dfaAdvanceBytes(ctx, state, Uint8Array)");
  GS_CALL(ctx, gs_dfa_advance_bytes(ctx, state, (const uint8_t*)bytes, (int64_t)n, &out));
  return make_i32(env, out);
}

static napi_value js_dfa_accepting(napi_env env, napi_callback_info info) {
  ARGS(2);
  CTX_ARG(0);
  int32_t state, out = 0;
  if (!get_i32(env, argv[1], &state)) return throw_error(env, "GS_ERR_INVALID_ARGUMENT", "dfaAccepting(ctx, state)");
  GS_CALL(ctx, gs_dfa_accepting(ctx, state, &out));
  napi_value r;
  napi_get_boolean(env, out != 0, &r);
  return r;
}

/* ---- lm_head ---------------------------------------------------------------- */

/* lmhead(ctx, hidden, weight, mRows, width, softcap, logits) -- device Externals */
static napi_value js_lmhead(napi_env env, napi_callback_info info) {
  ARGS(7);
  CTX_ARG(0);
  void* h = argc > 1 ? get_ptr(env, argv[1]) : NULL;
  void* w = argc > 2 ? get_ptr(env, argv[2]) : NULL;
  void* out = argc > 6 ? get_ptr(env, argv[6]) : NULL;
  int32_t m, width;
  double cap;
  if (!h || !w || !out || !get_i32(env, argv[3], &m) || !get_i32(env, argv[4], &width) || !get_f64(env, argv[5], &cap))
    return throw_error(env, "GS_ERR_INVALID_ARGUMENT", "lmhead(ctx, hidden, weight, mRows, width, softcap, logits)");
  GS_CALL(ctx, gs_lmhead(ctx, h, w, m, width, (float)cap, (float*)out, NULL));
  GS_CALL(ctx, gs_synchronize(ctx));
  return NULL;
}

/* qatLmhead(ctx, x, mRows, width, codes, layout, rowScales, inputScale, outputScale, logits) -- device
 * Externals: the int2 QAT head (gs_qat_lmhead) */
static napi_value js_qat_lmhead(napi_env env, napi_callback_info info) {
  ARGS(10);
  CTX_ARG(0);
  void* x = argc > 1 ? get_ptr(env, argv[1]) : NULL;
  void* codes = argc > 4 ? get_ptr(env, argv[4]) : NULL;
  void* scales = argc > 6 ? get_ptr(env, argv[6]) : NULL;
  void* out = argc > 9 ? get_ptr(env, argv[9]) : NULL;
  int32_t m, width, layout;
  double in_scale, out_scale;
  if (!x || !codes || !scales || !out || !get_i32(env, argv[2], &m) || !get_i32(env, argv[3], &width) ||
      !get_i32(env, argv[5], &layout) || !get_f64(env, argv[7], &in_scale) || !get_f64(env, argv[8], &out_scale))
    return throw_error(env, "GS_ERR_INVALID_ARGUMENT",
                       "qatLmhead(ctx, x, mRows, width, codes, layout, rowScales, inputScale, outputScale, logits)");
  GS_CALL(ctx, gs_qat_lmhead(ctx, (const float*)x, m, width, (const uint32_t*)codes, layout, (const float*)scales,
                             (float)in_scale, (float)out_scale, (float*)out, NULL));
  GS_CALL(ctx, gs_synchronize(ctx));
  return NULL;
}

/* ---- timing ---------------------------------------------------------------- */

static napi_value js_timing_begin(napi_env env, napi_callback_info info) {
  ARGS(2);
  CTX_ARG(0);
  int32_t n;
  if (!get_i32(env, argv[1], &n)) return throw_error(env, "GS_ERR_INVALID_ARGUMENT", "timingBegin(ctx, maxCalls)");
  GS_CALL(ctx, gs_timing_begin(ctx, n));
  return NULL;
}

static napi_value js_timing_end(napi_env env, napi_callback_info info) {
  ARGS(1);
  CTX_ARG(0);
  double ms[GS_STAGE_COUNT];
  int32_t calls[GS_STAGE_COUNT];
  GS_CALL(ctx, gs_timing_end(ctx, ms, calls));
  napi_value out, a, c;
  napi_create_object(env, &out);
  napi_create_array_with_length(env, GS_STAGE_COUNT, &a);
  napi_create_array_with_length(env, GS_STAGE_COUNT, &c);
  for (uint32_t k = 0; k < GS_STAGE_COUNT; ++k) {
    napi_set_element(env, a, k, make_f64(env, ms[k]));
    napi_set_element(env, c, k, make_i32(env, calls[k]));
  }
  napi_set_named_property(env, out, "stageMs", a);
  napi_set_named_property(env, out, "calls", c);
  return out;
}

static napi_value init(napi_env env, napi_value exports) {
  static const struct {
    const char* name;
    napi_callback cb;
  } fns[] = {
      {"abiVersion", js_abi_version},
      {"deviceCount", js_device_count},
      {"seededRandom", js_seeded_random},
      {"jsExp", js_exp},
      {"jsLog", js_log},
      {"softcap", js_softcap},
      {"layouts", js_layouts},
      {"validateConfigs", js_validate_configs},
      {"create", js_create},
      {"destroy", js_destroy},
      {"synchronize", js_synchronize},
      {"deviceAlloc", js_device_alloc},
      {"deviceFree", js_device_free},
      {"copyToDevice", js_copy_to_device},
      {"copyToHost", js_copy_to_host},
      {"sampleHost", js_sample_host},
      {"tokenLogProbHost", js_token_log_prob_host},
      {"maskLogitsHost", js_mask_logits_host},
      {"setVocab", js_set_vocab},
      {"setDfa", js_set_dfa},
      {"buildMasks", js_build_masks},
      {"legalTokenIds", js_legal_token_ids},
      {"dfaAdvance", js_dfa_advance},
      {"dfaAdvanceBytes", js_dfa_advance_bytes},
      {"dfaAccepting", js_dfa_accepting},
      {"lmhead", js_lmhead},
      {"qatLmhead", js_qat_lmhead},
      {"timingBegin", js_timing_begin},
      {"timingEnd", js_timing_end},
  };
  for (size_t i = 0; i < sizeof(fns) / sizeof(fns[0]); ++i) {
    napi_value f;
    if (napi_create_function(env, fns[i].name, NAPI_AUTO_LENGTH, fns[i].cb, NULL, &f) != napi_ok) return NULL;
    if (napi_set_named_property(env, exports, fns[i].name, f) != napi_ok) return NULL;
  }
  napi_value v;
  napi_create_int32(env, GS_STAGE_COUNT, &v);
  napi_set_named_property(env, exports, "STAGE_COUNT", v);
  return exports;
}

NAPI_MODULE(NODE_GYP_MODULE_NAME, init)
