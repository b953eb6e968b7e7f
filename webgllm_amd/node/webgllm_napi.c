/*
 * The Node N-API addon over libwebgllm_hip's C ABI: what the reference's
 * TypeScript engine would load in place of its WebGL2 backend (class Gpu,
 * src/gpu/gl.ts:47; the PacedGpu contract, src/gpu/paced.ts:11-22) and
 * beside it, as WebGpu.nativeProgram adds native kernels
 * (src/gpu/webgpu.ts:39-46). index.js wraps it in a HipGpu class with the
 * reference's method names.
 *
 * Handles (context, buffer, fence) are externals holding a tagged box, so a
 * handle of one kind passed where another is expected throws a TypeError
 * instead of reaching the library; a deleted, finished or destroyed handle
 * reaches it and comes back as WG_ERR_DISPOSED. Every failed call throws an
 * Error named "GpuError" (src/gpu/types.ts:14) whose `code` is the status's
 * name (WG_ERR_INVALID, WG_ERR_OOM, ...), `status` its number, and whose
 * message is the library's (wg_last_error).
 *
 * Paths cited are relative to packages/webgllm/ of the reference.
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <node_api.h>

#include "webgllm_hip.h"

/* ------------------------------------------------------------ plumbing */

enum { H_CTX = 0x63747821, H_BUF = 0x62756621, H_FENCE = 0x666e6321 };

typedef struct {
  uint32_t kind;
  void *p;
} box;

static void box_free(napi_env env, void *data, void *hint) {
  (void)env;
  (void)hint;
  free(data);
}

#define NAPI_OK(call)                                        \
  do {                                                       \
    if ((call) != napi_ok) {                                 \
      napi_throw_error(env, "EADDON", "N-API call failed: " #call); \
      return NULL;                                           \
    }                                                        \
  } while (0)

static const char *status_name(int rc) {
  switch (rc) {
    case WG_ERR_INVALID: return "WG_ERR_INVALID";
    case WG_ERR_OOM: return "WG_ERR_OOM";
    case WG_ERR_DEVICE: return "WG_ERR_DEVICE";
    case WG_ERR_ALIASED: return "WG_ERR_ALIASED";
    case WG_ERR_DISPOSED: return "WG_ERR_DISPOSED";
    case WG_ERR_UNSUPPORTED: return "WG_ERR_UNSUPPORTED";
    default: return "WG_ERR_UNKNOWN";
  }
}

/* Throws the library's failure as a GpuError; returns NULL for the caller. */
static napi_value throw_wg(napi_env env, int rc) {
  napi_value msg, code, err, name, status;
  const char *text = wg_last_error();
  napi_create_string_utf8(env, text ? text : "", NAPI_AUTO_LENGTH, &msg);
  napi_create_string_utf8(env, status_name(rc), NAPI_AUTO_LENGTH, &code);
  napi_create_error(env, code, msg, &err);
  napi_create_string_utf8(env, "GpuError", NAPI_AUTO_LENGTH, &name);
  napi_set_named_property(env, err, "name", name);
  napi_create_int32(env, rc, &status);
  napi_set_named_property(env, err, "status", status);
  napi_throw(env, err);
  return NULL;
}

static napi_value type_error(napi_env env, const char *what) {
  napi_throw_type_error(env, "EARG", what);
  return NULL;
}

static napi_value wrap(napi_env env, uint32_t kind, void *p) {
  box *b = (box *)malloc(sizeof(box));
  napi_value out;
  if (!b) {
    napi_throw_error(env, "EADDON", "out of host memory");
    return NULL;
  }
  b->kind = kind;
  b->p = p;
  if (napi_create_external(env, b, box_free, NULL, &out) != napi_ok) {
    free(b);
    napi_throw_error(env, "EADDON", "napi_create_external failed");
    return NULL;
  }
  return out;
}

/* The pointer of a handle of `kind`, or NULL after throwing a TypeError. */
static void *unwrap(napi_env env, napi_value v, uint32_t kind, const char *what) {
  napi_valuetype t;
  box *b = NULL;
  if (napi_typeof(env, v, &t) != napi_ok || t != napi_external ||
      napi_get_value_external(env, v, (void **)&b) != napi_ok || !b || b->kind != kind) {
    char msg[128];
    snprintf(msg, sizeof msg, "expected a %s handle", what);
    napi_throw_type_error(env, "EARG", msg);
    return NULL;
  }
  return b->p;
}

static int get_i64(napi_env env, napi_value v, int64_t *out) {
  napi_valuetype t;
  if (napi_typeof(env, v, &t) != napi_ok || t != napi_number) return 0;
  double d;
  if (napi_get_value_double(env, v, &d) != napi_ok) return 0;
  if (d != (double)(int64_t)d) return 0; /* integers only */
  *out = (int64_t)d;
  return 1;
}

static int get_i32(napi_env env, napi_value v, int32_t *out) {
  int64_t x;
  if (!get_i64(env, v, &x) || x < INT32_MIN || x > INT32_MAX) return 0;
  *out = (int32_t)x;
  return 1;
}

/* Bytes of an ArrayBuffer, a typed array, a DataView or a Buffer. */
static int get_bytes(napi_env env, napi_value v, void **data, size_t *len) {
  bool is;
  if (napi_is_arraybuffer(env, v, &is) == napi_ok && is)
    return napi_get_arraybuffer_info(env, v, data, len) == napi_ok;
  if (napi_is_typedarray(env, v, &is) == napi_ok && is) {
    napi_typedarray_type type;
    size_t n, off;
    napi_value ab;
    if (napi_get_typedarray_info(env, v, &type, &n, data, &ab, &off) != napi_ok) return 0;
    size_t el = 1;
    switch (type) {
      case napi_int16_array: case napi_uint16_array: el = 2; break;
      case napi_int32_array: case napi_uint32_array: case napi_float32_array: el = 4; break;
      case napi_float64_array: case napi_bigint64_array: case napi_biguint64_array: el = 8; break;
      default: el = 1;
    }
    *len = n * el;
    return 1;
  }
  if (napi_is_dataview(env, v, &is) == napi_ok && is) {
    napi_value ab;
    size_t off;
    return napi_get_dataview_info(env, v, len, data, &ab, &off) == napi_ok;
  }
  return 0;
}

static int is_nullish(napi_env env, napi_value v) {
  napi_valuetype t;
  return napi_typeof(env, v, &t) == napi_ok && (t == napi_undefined || t == napi_null);
}

static napi_value num(napi_env env, double d) {
  napi_value v;
  napi_create_double(env, d, &v);
  return v;
}

static napi_value str(napi_env env, const char *s, size_t n) {
  napi_value v;
  napi_create_string_utf8(env, s ? s : "", s ? n : 0, &v);
  return v;
}

static void set(napi_env env, napi_value obj, const char *key, napi_value v) {
  napi_set_named_property(env, obj, key, v);
}

#define ARGS(n)                                                       \
  size_t argc = (n);                                                  \
  napi_value argv[(n) > 0 ? (n) : 1];                                 \
  NAPI_OK(napi_get_cb_info(env, info, &argc, argv, NULL, NULL));      \
  for (size_t k_ = argc; k_ < (n); k_++) napi_get_undefined(env, &argv[k_])

#define INT32_ARG(i, var)                                                        \
  int32_t var;                                                                   \
  if (!get_i32(env, argv[i], &var)) return type_error(env, #var " must be an integer")

#define INT64_ARG(i, var)                                                        \
  int64_t var;                                                                   \
  if (!get_i64(env, argv[i], &var) || var < 0)                                  \
  return type_error(env, #var " must be a non-negative integer")

#define HANDLE_ARG(i, type, var, kind, what)                 \
  type *var = (type *)unwrap(env, argv[i], kind, what);      \
  if (!var) return NULL

/* ------------------------------------------------------------ library */

static napi_value js_version(napi_env env, napi_callback_info info) {
  (void)info;
  return str(env, wg_version(), strlen(wg_version()));
}

/* q4Sizes(N, K, layout, zero): the device arrays of a QuantMatrix
 * (src/weights.ts:153-178): {quants, scales, zeros} bytes. */
static napi_value js_q4_sizes(napi_env env, napi_callback_info info) {
  ARGS(4);
  INT32_ARG(0, N);
  INT32_ARG(1, K);
  INT32_ARG(2, layout);
  INT32_ARG(3, zero);
  size_t q = 0, s = 0, z = 0;
  int rc = wg_q4_sizes(N, K, layout, zero, &q, &s, &z);
  if (rc) return throw_wg(env, rc);
  napi_value o;
  NAPI_OK(napi_create_object(env, &o));
  set(env, o, "quants", num(env, (double)q));
  set(env, o, "scales", num(env, (double)s));
  set(env, o, "zeros", num(env, (double)z));
  return o;
}

/* ----------------------------------------------------- backend objects */

static napi_value js_ctx_create(napi_env env, napi_callback_info info) {
  ARGS(1);
  int32_t dev = 0;
  if (!is_nullish(env, argv[0]) && !get_i32(env, argv[0], &dev))
    return type_error(env, "device must be an integer");
  wg_ctx *c = NULL;
  int rc = wg_ctx_create(dev, &c);
  if (rc) return throw_wg(env, rc);
  return wrap(env, H_CTX, c);
}

static napi_value js_ctx_destroy(napi_env env, napi_callback_info info) {
  ARGS(1);
  HANDLE_ARG(0, wg_ctx, c, H_CTX, "context");
  int rc = wg_ctx_destroy(c);
  return rc ? throw_wg(env, rc) : NULL;
}

/* Gpu.limits (gl.ts:131-140), with the device's own figures. */
static napi_value js_ctx_limits(napi_env env, napi_callback_info info) {
  ARGS(1);
  HANDLE_ARG(0, wg_ctx, c, H_CTX, "context");
  wg_limits lim;
  int rc = wg_ctx_limits(c, &lim);
  if (rc) return throw_wg(env, rc);
  napi_value o;
  NAPI_OK(napi_create_object(env, &o));
  set(env, o, "device", num(env, lim.device));
  set(env, o, "computeUnits", num(env, lim.compute_units));
  set(env, o, "globalBytes", num(env, (double)lim.global_bytes));
  set(env, o, "maxAllocBytes", num(env, (double)lim.max_alloc_bytes));
  set(env, o, "ldsBytesPerBlock", num(env, lim.lds_bytes_per_block));
  set(env, o, "waveSize", num(env, lim.wave_size));
  set(env, o, "renderer", str(env, wg_version(), strlen(wg_version())));
  return o;
}

static napi_value js_bytes_live(napi_env env, napi_callback_info info) {
  ARGS(1);
  HANDLE_ARG(0, wg_ctx, c, H_CTX, "context");
  return num(env, (double)wg_bytes_live(c));
}

static napi_value js_staging(napi_env env, napi_callback_info info) {
  ARGS(1);
  HANDLE_ARG(0, wg_ctx, c, H_CTX, "context");
  int32_t slots = 0;
  size_t bytes = 0;
  int rc = wg_ctx_staging(c, &slots, &bytes);
  if (rc) return throw_wg(env, rc);
  napi_value o;
  NAPI_OK(napi_create_object(env, &o));
  set(env, o, "slots", num(env, slots));
  set(env, o, "bytes", num(env, (double)bytes));
  return o;
}

/* bufCreate(ctx, bytes, init?): Gpu.texture (gl.ts:263-305). */
static napi_value js_buf_create(napi_env env, napi_callback_info info) {
  ARGS(3);
  HANDLE_ARG(0, wg_ctx, c, H_CTX, "context");
  INT64_ARG(1, bytes);
  void *init = NULL;
  size_t len = 0;
  if (!is_nullish(env, argv[2])) {
    if (!get_bytes(env, argv[2], &init, &len)) return type_error(env, "init must be bytes");
    if ((int64_t)len != bytes) return type_error(env, "init must hold exactly `bytes` bytes");
  }
  wg_buf *b = NULL;
  int rc = wg_buf_create(c, (size_t)bytes, init, &b);
  if (rc) return throw_wg(env, rc);
  return wrap(env, H_BUF, b);
}

/* bufWrite(ctx, buf, offset, data): Gpu.write (gl.ts:354-374). */
static napi_value js_buf_write(napi_env env, napi_callback_info info) {
  ARGS(4);
  HANDLE_ARG(0, wg_ctx, c, H_CTX, "context");
  HANDLE_ARG(1, wg_buf, b, H_BUF, "buffer");
  INT64_ARG(2, offset);
  void *data = NULL;
  size_t len = 0;
  if (!get_bytes(env, argv[3], &data, &len)) return type_error(env, "data must be bytes");
  int rc = wg_buf_write(c, b, (size_t)offset, data, len);
  return rc ? throw_wg(env, rc) : NULL;
}

static napi_value js_buf_zero(napi_env env, napi_callback_info info) {
  ARGS(2);
  HANDLE_ARG(0, wg_ctx, c, H_CTX, "context");
  HANDLE_ARG(1, wg_buf, b, H_BUF, "buffer");
  int rc = wg_buf_zero(c, b);
  return rc ? throw_wg(env, rc) : NULL;
}

static napi_value js_buf_delete(napi_env env, napi_callback_info info) {
  ARGS(2);
  HANDLE_ARG(0, wg_ctx, c, H_CTX, "context");
  HANDLE_ARG(1, wg_buf, b, H_BUF, "buffer");
  int rc = wg_buf_delete(c, b);
  return rc ? throw_wg(env, rc) : NULL;
}

static napi_value js_buf_size(napi_env env, napi_callback_info info) {
  ARGS(1);
  HANDLE_ARG(0, wg_buf, b, H_BUF, "buffer");
  return num(env, (double)wg_buf_size(b));
}

/* readStart(ctx, buf, offset, bytes): a fence (PendingRead, gl.ts:740-782). */
static napi_value js_read_start(napi_env env, napi_callback_info info) {
  ARGS(4);
  HANDLE_ARG(0, wg_ctx, c, H_CTX, "context");
  HANDLE_ARG(1, wg_buf, b, H_BUF, "buffer");
  INT64_ARG(2, offset);
  INT64_ARG(3, bytes);
  wg_fence *f = NULL;
  int rc = wg_read_start(c, b, (size_t)offset, (size_t)bytes, &f);
  if (rc) return throw_wg(env, rc);
  return wrap(env, H_FENCE, f);
}

static napi_value js_fence_ready(napi_env env, napi_callback_info info) {
  ARGS(1);
  HANDLE_ARG(0, wg_fence, f, H_FENCE, "fence");
  int rc = wg_fence_ready(f);
  if (rc < 0) return throw_wg(env, rc);
  napi_value v;
  napi_get_boolean(env, rc == 1, &v);
  return v;
}

/* readFinish(fence, bytes): waits, returns an ArrayBuffer of `bytes`. */
static napi_value js_read_finish(napi_env env, napi_callback_info info) {
  ARGS(2);
  HANDLE_ARG(0, wg_fence, f, H_FENCE, "fence");
  INT64_ARG(1, bytes);
  void *data = NULL;
  napi_value ab;
  NAPI_OK(napi_create_arraybuffer(env, (size_t)bytes, &data, &ab));
  int rc = wg_read_finish(f, data);
  return rc ? throw_wg(env, rc) : ab;
}

static napi_value js_read_cancel(napi_env env, napi_callback_info info) {
  ARGS(1);
  HANDLE_ARG(0, wg_fence, f, H_FENCE, "fence");
  int rc = wg_read_cancel(f);
  return rc ? throw_wg(env, rc) : NULL;
}

/* readNow(ctx, buf, offset, bytes): Gpu.readNow (gl.ts:658-700). */
static napi_value js_read_now(napi_env env, napi_callback_info info) {
  ARGS(4);
  HANDLE_ARG(0, wg_ctx, c, H_CTX, "context");
  HANDLE_ARG(1, wg_buf, b, H_BUF, "buffer");
  INT64_ARG(2, offset);
  INT64_ARG(3, bytes);
  void *data = NULL;
  napi_value ab;
  NAPI_OK(napi_create_arraybuffer(env, (size_t)bytes, &data, &ab));
  int rc = wg_read_now(c, b, (size_t)offset, (size_t)bytes, data);
  return rc ? throw_wg(env, rc) : ab;
}

static napi_value js_flush(napi_env env, napi_callback_info info) {
  ARGS(1);
  HANDLE_ARG(0, wg_ctx, c, H_CTX, "context");
  int rc = wg_flush(c);
  return rc ? throw_wg(env, rc) : NULL;
}

static napi_value js_finish(napi_env env, napi_callback_info info) {
  ARGS(1);
  HANDLE_ARG(0, wg_ctx, c, H_CTX, "context");
  int rc = wg_finish(c);
  return rc ? throw_wg(env, rc) : NULL;
}

/* ------------------------------------------------------------ typed ops */

/* A matrix object {N, K, layout, zero, quants: buf, scales?: buf,
 * zeros?: buf} as the C descriptor. */
static int read_matrix(napi_env env, napi_value o, wg_q4_matrix *m) {
  napi_value v;
  memset(m, 0, sizeof *m);
  int32_t *ints[4] = {&m->N, &m->K, &m->layout, &m->zero};
  const char *names[4] = {"N", "K", "layout", "zero"};
  for (int k = 0; k < 4; k++) {
    if (napi_get_named_property(env, o, names[k], &v) != napi_ok || !get_i32(env, v, ints[k])) {
      char msg[96];
      snprintf(msg, sizeof msg, "matrix.%s must be an integer", names[k]);
      napi_throw_type_error(env, "EARG", msg);
      return 0;
    }
  }
  const char *arrays[3] = {"quants", "scales", "zeros"};
  void **ptrs[3] = {(void **)&m->quants, (void **)&m->scales, (void **)&m->zeros};
  for (int k = 0; k < 3; k++) {
    if (napi_get_named_property(env, o, arrays[k], &v) != napi_ok) return 0;
    if (is_nullish(env, v)) continue;
    wg_buf *b = (wg_buf *)unwrap(env, v, H_BUF, "buffer");
    if (!b) return 0;
    *ptrs[k] = wg_buf_ptr(b);
    if (!*ptrs[k]) {
      napi_throw_error(env, "WG_ERR_DISPOSED", "a matrix buffer was deleted");
      return 0;
    }
  }
  return 1;
}

static void *buf_ptr_arg(napi_env env, napi_value v, int optional, int *ok) {
  *ok = 1;
  if (optional && is_nullish(env, v)) return NULL;
  wg_buf *b = (wg_buf *)unwrap(env, v, H_BUF, "buffer");
  if (!b) {
    *ok = 0;
    return NULL;
  }
  void *p = wg_buf_ptr(b);
  if (!p) {
    *ok = 0;
    napi_throw_error(env, "WG_ERR_DISPOSED", "the buffer was deleted");
  }
  return p;
}

/* repack(ctx, kind, matrix, row0, rows, src, srcRows?): the loaders'
 * packers on the GPU (packQ4_0, packQ4_K, repack.ts:60-168); kind
 * "q4_0" | "q4_k" | "q4_k_native" | "q8_0" | "q6_k". */
static napi_value js_repack(napi_env env, napi_callback_info info) {
  ARGS(7);
  HANDLE_ARG(0, wg_ctx, c, H_CTX, "context");
  char kind[16];
  size_t n = 0;
  if (napi_get_value_string_utf8(env, argv[1], kind, sizeof kind, &n) != napi_ok)
    return type_error(env, "kind must be a string");
  wg_q4_matrix m;
  if (!read_matrix(env, argv[2], &m)) return NULL;
  INT32_ARG(3, row0);
  INT32_ARG(4, rows);
  int ok;
  const void *src = buf_ptr_arg(env, argv[5], 0, &ok);
  if (!ok) return NULL;
  const int32_t *src_rows = (const int32_t *)buf_ptr_arg(env, argv[6], 1, &ok);
  if (!ok) return NULL;
  void *s = wg_ctx_stream(c);
  int rc;
  if (!strcmp(kind, "q4_0")) rc = wg_repack_q4_0(&m, row0, rows, src, src_rows, s);
  else if (!strcmp(kind, "q4_k")) rc = wg_repack_q4_k(&m, row0, rows, src, src_rows, s);
  else if (!strcmp(kind, "q4_k_native")) rc = wg_repack_q4_k_native(&m, row0, rows, src, src_rows, s);
  else if (!strcmp(kind, "q8_0")) rc = wg_repack_q8_0(&m, row0, rows, src, src_rows, s);
  else if (!strcmp(kind, "q6_k")) rc = wg_repack_q6_k(&m, row0, rows, src, src_rows, s);
  else return type_error(env, "kind must be q4_0, q4_k, q4_k_native, q8_0 or q6_k");
  return rc ? throw_wg(env, rc) : NULL;
}

/* dequant(ctx, matrix, row0, rows, out): matrixRow (repack.ts:865-891). */
static napi_value js_dequant(napi_env env, napi_callback_info info) {
  ARGS(5);
  HANDLE_ARG(0, wg_ctx, c, H_CTX, "context");
  wg_q4_matrix m;
  if (!read_matrix(env, argv[1], &m)) return NULL;
  INT32_ARG(2, row0);
  INT32_ARG(3, rows);
  int ok;
  float *out = (float *)buf_ptr_arg(env, argv[4], 0, &ok);
  if (!ok) return NULL;
  int rc = wg_q4_dequant(&m, row0, rows, out, wg_ctx_stream(c));
  return rc ? throw_wg(env, rc) : NULL;
}

/* gemv(ctx, matrix, x, M, y): splitPartials + pf (engine.ts:5241-5377;
 * kernels.ts:744-895, :69-79): y [M][N] f32 = x [M][K] halves times W^T. */
static napi_value js_gemv(napi_env env, napi_callback_info info) {
  ARGS(5);
  HANDLE_ARG(0, wg_ctx, c, H_CTX, "context");
  wg_q4_matrix m;
  if (!read_matrix(env, argv[1], &m)) return NULL;
  int ok;
  const uint16_t *x = (const uint16_t *)buf_ptr_arg(env, argv[2], 0, &ok);
  if (!ok) return NULL;
  INT32_ARG(3, M);
  float *y = (float *)buf_ptr_arg(env, argv[4], 0, &ok);
  if (!ok) return NULL;
  int rc = wg_q4_gemv(&m, x, M, m.K, y, m.N, NULL, wg_ctx_stream(c));
  return rc ? throw_wg(env, rc) : NULL;
}

static napi_value js_argmax_scratch_bytes(napi_env env, napi_callback_info info) {
  ARGS(2);
  INT32_ARG(0, M);
  INT32_ARG(1, V);
  return num(env, (double)wg_argmax_scratch_bytes(M, V));
}

/* argmax(ctx, logits, M, V, ids, scratch): Engine.argmax (engine.ts:8271-8336). */
static napi_value js_argmax(napi_env env, napi_callback_info info) {
  ARGS(6);
  HANDLE_ARG(0, wg_ctx, c, H_CTX, "context");
  int ok;
  const float *logits = (const float *)buf_ptr_arg(env, argv[1], 0, &ok);
  if (!ok) return NULL;
  INT32_ARG(2, M);
  INT32_ARG(3, V);
  int32_t *ids = (int32_t *)buf_ptr_arg(env, argv[4], 0, &ok);
  if (!ok) return NULL;
  HANDLE_ARG(5, wg_buf, scratch, H_BUF, "buffer");
  void *sp = wg_buf_ptr(scratch);
  int rc = wg_argmax_rows(logits, M, V, V, ids, NULL, sp, wg_buf_size(scratch), wg_ctx_stream(c));
  return rc ? throw_wg(env, rc) : NULL;
}

/* ---------------------------------------------------------- file readers */

static napi_value dims_array(napi_env env, const int64_t *dims, int n) {
  napi_value a;
  napi_create_array_with_length(env, (size_t)n, &a);
  for (int k = 0; k < n; k++) napi_set_element(env, a, (uint32_t)k, num(env, (double)dims[k]));
  return a;
}

/* ggufHeader(path): readGgufHeader (src/gguf.ts:276-328): {version,
 * dataOffset, tensors: [{name, dims, type, offset, bytes}], meta: {key:
 * value}} (arrays as {type, length}). */
static napi_value js_gguf_header(napi_env env, napi_callback_info info) {
  ARGS(1);
  char path[4096];
  size_t n = 0;
  if (napi_get_value_string_utf8(env, argv[0], path, sizeof path, &n) != napi_ok)
    return type_error(env, "path must be a string");
  wg_gguf *g = NULL;
  int rc = wg_gguf_open(path, &g);
  if (rc) return throw_wg(env, rc);
  napi_value o, tensors, meta;
  napi_create_object(env, &o);
  set(env, o, "version", num(env, wg_gguf_version(g)));
  set(env, o, "dataOffset", num(env, (double)wg_gguf_data_offset(g)));
  int64_t nt = wg_gguf_tensor_count(g), nm = wg_gguf_meta_count(g);
  napi_create_array_with_length(env, (size_t)nt, &tensors);
  for (int64_t i = 0; i < nt; i++) {
    wg_gguf_tensor_info t;
    if ((rc = wg_gguf_tensor(g, i, &t))) break;
    napi_value e;
    napi_create_object(env, &e);
    set(env, e, "name", str(env, t.name, strlen(t.name)));
    set(env, e, "dims", dims_array(env, t.dims, t.n_dims));
    set(env, e, "type", num(env, t.type));
    set(env, e, "offset", num(env, (double)t.offset));
    set(env, e, "bytes", num(env, (double)t.bytes));
    napi_set_element(env, tensors, (uint32_t)i, e);
  }
  napi_create_object(env, &meta);
  for (int64_t i = 0; !rc && i < nm; i++) {
    wg_gguf_value v;
    if ((rc = wg_gguf_meta(g, i, &v))) break;
    napi_value val;
    if (v.type == 8) {
      val = str(env, v.s, (size_t)v.length);
    } else if (v.type == 9) {
      napi_create_object(env, &val);
      set(env, val, "type", num(env, v.elem_type));
      set(env, val, "length", num(env, (double)v.length));
    } else if (v.type == 6 || v.type == 12) {
      val = num(env, v.f);
    } else if (v.type == 7) {
      napi_get_boolean(env, v.i != 0, &val);
    } else {
      val = num(env, (double)v.i);
    }
    set(env, meta, v.key, val);
  }
  set(env, o, "tensors", tensors);
  set(env, o, "meta", meta);
  if (rc) {
    napi_value err;
    (void)err;
    wg_gguf_close(g);
    return throw_wg(env, rc);
  }
  wg_gguf_close(g);
  return o;
}

/* onnxGraph(path): parseOnnxModel (src/onnx.ts:71-282): {name, nodes:
 * [{name, opType, domain, inputs, outputs, attributes: {name: {type, i,
 * f, s, ints}}}], initializers: [{name, dims, dataType, rawBytes, location,
 * offset, length}]}. */
static napi_value js_onnx_graph(napi_env env, napi_callback_info info) {
  ARGS(1);
  char path[4096];
  size_t n = 0;
  if (napi_get_value_string_utf8(env, argv[0], path, sizeof path, &n) != napi_ok)
    return type_error(env, "path must be a string");
  wg_onnx *f = NULL;
  int rc = wg_onnx_open(path, &f);
  if (rc) return throw_wg(env, rc);
  napi_value o, nodes, inits;
  napi_create_object(env, &o);
  const char *gname = wg_onnx_graph_name(f);
  set(env, o, "name", str(env, gname, gname ? strlen(gname) : 0));
  int64_t nn = wg_onnx_node_count(f), ni = wg_onnx_init_count(f);
  napi_create_array_with_length(env, (size_t)nn, &nodes);
  for (int64_t i = 0; !rc && i < nn; i++) {
    wg_onnx_node_info ni_;
    if ((rc = wg_onnx_node(f, i, &ni_))) break;
    napi_value e, ins, outs, attrs;
    napi_create_object(env, &e);
    set(env, e, "name", str(env, ni_.name, strlen(ni_.name)));
    set(env, e, "opType", str(env, ni_.op_type, strlen(ni_.op_type)));
    set(env, e, "domain", str(env, ni_.domain, strlen(ni_.domain)));
    napi_create_array_with_length(env, (size_t)ni_.n_inputs, &ins);
    for (int32_t j = 0; j < ni_.n_inputs; j++) {
      const char *s = wg_onnx_node_input(f, i, j);
      napi_set_element(env, ins, (uint32_t)j, str(env, s, s ? strlen(s) : 0));
    }
    napi_create_array_with_length(env, (size_t)ni_.n_outputs, &outs);
    for (int32_t j = 0; j < ni_.n_outputs; j++) {
      const char *s = wg_onnx_node_output(f, i, j);
      napi_set_element(env, outs, (uint32_t)j, str(env, s, s ? strlen(s) : 0));
    }
    napi_create_object(env, &attrs);
    for (int32_t j = 0; j < ni_.n_attrs; j++) {
      wg_onnx_attr a;
      if ((rc = wg_onnx_node_attr(f, i, j, &a))) break;
      napi_value av;
      napi_create_object(env, &av);
      set(env, av, "type", num(env, a.type));
      if (a.type == 1) set(env, av, "f", num(env, a.f));
      if (a.type == 2) set(env, av, "i", num(env, (double)a.i));
      if (a.type == 3) set(env, av, "s", str(env, a.s, (size_t)a.s_len));
      if (a.type == 7) set(env, av, "ints", dims_array(env, a.ints, (int)a.n_ints));
      if (a.type == 4) set(env, av, "tensor", num(env, (double)a.tensor));
      set(env, attrs, a.name, av);
    }
    set(env, e, "inputs", ins);
    set(env, e, "outputs", outs);
    set(env, e, "attributes", attrs);
    napi_set_element(env, nodes, (uint32_t)i, e);
  }
  napi_create_array_with_length(env, (size_t)ni, &inits);
  for (int64_t i = 0; !rc && i < ni; i++) {
    wg_onnx_tensor_info t;
    if ((rc = wg_onnx_tensor(f, i, &t))) break;
    napi_value e;
    napi_create_object(env, &e);
    set(env, e, "name", str(env, t.name, strlen(t.name)));
    set(env, e, "dims", dims_array(env, t.dims, t.n_dims));
    set(env, e, "dataType", num(env, t.data_type));
    set(env, e, "rawBytes", num(env, (double)t.raw_bytes));
    if (t.location) {
      set(env, e, "location", str(env, t.location, strlen(t.location)));
      set(env, e, "offset", num(env, (double)t.offset));
      set(env, e, "length", num(env, (double)t.length));
    }
    napi_set_element(env, inits, (uint32_t)i, e);
  }
  set(env, o, "nodes", nodes);
  set(env, o, "initializers", inits);
  wg_onnx_close(f);
  if (rc) return throw_wg(env, rc);
  return o;
}

/* ------------------------------------------------------------- module */

static napi_value init(napi_env env, napi_value exports) {
  static const struct {
    const char *name;
    napi_callback fn;
  } fns[] = {
      {"version", js_version},
      {"q4Sizes", js_q4_sizes},
      {"ctxCreate", js_ctx_create},
      {"ctxDestroy", js_ctx_destroy},
      {"ctxLimits", js_ctx_limits},
      {"bytesLive", js_bytes_live},
      {"staging", js_staging},
      {"bufCreate", js_buf_create},
      {"bufWrite", js_buf_write},
      {"bufZero", js_buf_zero},
      {"bufDelete", js_buf_delete},
      {"bufSize", js_buf_size},
      {"readStart", js_read_start},
      {"fenceReady", js_fence_ready},
      {"readFinish", js_read_finish},
      {"readCancel", js_read_cancel},
      {"readNow", js_read_now},
      {"flush", js_flush},
      {"finish", js_finish},
      {"repack", js_repack},
      {"dequant", js_dequant},
      {"gemv", js_gemv},
      {"argmaxScratchBytes", js_argmax_scratch_bytes},
      {"argmax", js_argmax},
      {"ggufHeader", js_gguf_header},
      {"onnxGraph", js_onnx_graph},
  };
  for (size_t i = 0; i < sizeof fns / sizeof fns[0]; i++) {
    napi_value f;
    if (napi_create_function(env, fns[i].name, NAPI_AUTO_LENGTH, fns[i].fn, NULL, &f) != napi_ok ||
        napi_set_named_property(env, exports, fns[i].name, f) != napi_ok) {
      napi_throw_error(env, "EADDON", "cannot export the addon's functions");
      return NULL;
    }
  }
  napi_value consts;
  napi_create_object(env, &consts);
  set(env, consts, "LAYOUT_ROWGROUP", num(env, WG_LAYOUT_ROWGROUP));
  set(env, consts, "LAYOUT_Q4K", num(env, WG_LAYOUT_Q4K));
  set(env, consts, "LAYOUT_Q8", num(env, WG_LAYOUT_Q8));
  set(env, consts, "LAYOUT_Q6K", num(env, WG_LAYOUT_Q6K));
  set(env, consts, "ZERO_8", num(env, WG_ZERO_8));
  set(env, consts, "ZERO_U8", num(env, WG_ZERO_U8));
  set(env, consts, "ZERO_F16", num(env, WG_ZERO_F16));
  set(env, exports, "constants", consts);
  return exports;
}

NAPI_MODULE(webgllm_hip, init)
