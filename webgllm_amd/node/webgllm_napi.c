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
#include <stdarg.h>
#include <stddef.h>
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

/* readFinish(fence, bytes?): waits, returns an ArrayBuffer of the fence's
 * bytes (a `bytes` other than the read's is refused before anything is
 * copied); a plain fence returns an empty one. */
static napi_value js_read_finish(napi_env env, napi_callback_info info) {
  ARGS(2);
  HANDLE_ARG(0, wg_fence, f, H_FENCE, "fence");
  const size_t have = wg_fence_bytes(f);
  if (!is_nullish(env, argv[1])) {
    INT64_ARG(1, bytes);
    if ((uint64_t)bytes != (uint64_t)have) {
      char text[128];
      snprintf(text, sizeof text, "readFinish: the read holds %zu bytes, not %lld", have,
               (long long)bytes);
      napi_value msg, code, err, name;
      napi_create_string_utf8(env, text, NAPI_AUTO_LENGTH, &msg);
      napi_create_string_utf8(env, "WG_ERR_INVALID", NAPI_AUTO_LENGTH, &code);
      napi_create_error(env, code, msg, &err);
      napi_create_string_utf8(env, "GpuError", NAPI_AUTO_LENGTH, &name);
      napi_set_named_property(env, err, "name", name);
      napi_throw(env, err);
      return NULL;
    }
  }
  void *data = NULL;
  napi_value ab;
  NAPI_OK(napi_create_arraybuffer(env, have, &data, &ab));
  int rc = wg_read_finish(f, have ? data : NULL);
  return rc ? throw_wg(env, rc) : ab;
}

/* fence(ctx): PacedGpu.fence (src/gpu/paced.ts:11-22), a fence behind the
 * work queued so far; fenceReady polls it, readCancel deletes it
 * (deleteFence), readFinish waits for it. */
static napi_value js_fence_record(napi_env env, napi_callback_info info) {
  ARGS(1);
  HANDLE_ARG(0, wg_ctx, c, H_CTX, "context");
  wg_fence *f = NULL;
  int rc = wg_fence_record(c, &f);
  if (rc) return throw_wg(env, rc);
  return wrap(env, H_FENCE, f);
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

/* ------------------------------------------------------------ typed ops
 *
 * Every device operand is a buffer handle, or [handle, byteOffset] for a
 * view into one. Before any launch the addon checks that each operand
 * holds what the shapes imply from its offset on (rows of a [M][ld] array:
 * (M - 1) ld + width elements), and throws a GpuError WG_ERR_INVALID
 * otherwise, as the reference's backend throws for a texture over its
 * limits (src/gpu/gl.ts:271-275); the library then checks the shapes
 * themselves. */

static napi_value throw_limits(napi_env env, const char *fmt, ...) {
  char text[256];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(text, sizeof text, fmt, ap);
  va_end(ap);
  napi_value msg, code, err, name, status;
  napi_create_string_utf8(env, text, NAPI_AUTO_LENGTH, &msg);
  napi_create_string_utf8(env, "WG_ERR_INVALID", NAPI_AUTO_LENGTH, &code);
  napi_create_error(env, code, msg, &err);
  napi_create_string_utf8(env, "GpuError", NAPI_AUTO_LENGTH, &name);
  napi_set_named_property(env, err, "name", name);
  napi_create_int32(env, WG_ERR_INVALID, &status);
  napi_set_named_property(env, err, "status", status);
  napi_throw(env, err);
  return NULL;
}

/* Elements a [rows][ld] array of rows `width` wide spans (0 for no rows). */
static uint64_t span(int64_t rows, int64_t ld, int64_t width) {
  if (rows <= 0 || width <= 0) return 0;
  return (uint64_t)(rows - 1) * (uint64_t)(ld > width ? ld : width) + (uint64_t)width;
}

/* A device operand: the pointer `need` bytes of which must lie in its
 * buffer from its offset on. Optional operands may be null or undefined
 * (NULL out). Returns 0 after throwing. */
static int operand(napi_env env, napi_value v, uint64_t need, int optional, const char *what,
                   void **out) {
  *out = NULL;
  if (is_nullish(env, v)) {
    if (optional) return 1;
    char msg[96];
    snprintf(msg, sizeof msg, "%s: a buffer is required", what);
    napi_throw_type_error(env, "EARG", msg);
    return 0;
  }
  napi_value h = v;
  int64_t offset = 0;
  bool is_array = false;
  if (napi_is_array(env, v, &is_array) == napi_ok && is_array) {
    uint32_t n = 0;
    napi_value off;
    if (napi_get_array_length(env, v, &n) != napi_ok || n != 2 ||
        napi_get_element(env, v, 0, &h) != napi_ok || napi_get_element(env, v, 1, &off) != napi_ok ||
        !get_i64(env, off, &offset) || offset < 0) {
      char msg[96];
      snprintf(msg, sizeof msg, "%s: a view is [buffer, byteOffset >= 0]", what);
      napi_throw_type_error(env, "EARG", msg);
      return 0;
    }
  }
  char kind[96];
  snprintf(kind, sizeof kind, "buffer for %s", what);
  wg_buf *b = (wg_buf *)unwrap(env, h, H_BUF, kind);
  if (!b) return 0;
  char *p = (char *)wg_buf_ptr(b);
  if (!p) {
    char msg[96];
    snprintf(msg, sizeof msg, "%s: the buffer was deleted", what);
    napi_value m, c, err;
    napi_create_string_utf8(env, msg, NAPI_AUTO_LENGTH, &m);
    napi_create_string_utf8(env, "WG_ERR_DISPOSED", NAPI_AUTO_LENGTH, &c);
    napi_create_error(env, c, m, &err);
    napi_value name;
    napi_create_string_utf8(env, "GpuError", NAPI_AUTO_LENGTH, &name);
    napi_set_named_property(env, err, "name", name);
    napi_throw(env, err);
    return 0;
  }
  const uint64_t size = wg_buf_size(b);
  if ((uint64_t)offset > size || need > size - (uint64_t)offset) {
    throw_limits(env, "%s: %llu bytes needed at offset %lld of a %llu-byte buffer", what,
                 (unsigned long long)need, (long long)offset, (unsigned long long)size);
    return 0;
  }
  *out = p + offset;
  return 1;
}

#define OPERAND(i, type, var, need, optional, what)                              \
  type *var;                                                                      \
  do {                                                                            \
    void *p_;                                                                     \
    if (!operand(env, argv[i], (uint64_t)(need), optional, what, &p_)) return NULL; \
    var = (type *)p_;                                                             \
  } while (0)

static int get_f64(napi_env env, napi_value v, double *out) {
  napi_valuetype t;
  return napi_typeof(env, v, &t) == napi_ok && t == napi_number &&
         napi_get_value_double(env, v, out) == napi_ok;
}

#define FLOAT_ARG(i, var)                                                        \
  float var;                                                                     \
  do {                                                                           \
    double d_;                                                                   \
    if (!get_f64(env, argv[i], &d_)) return type_error(env, #var " must be a number"); \
    var = (float)d_;                                                             \
  } while (0)

static int prop(napi_env env, napi_value o, const char *key, napi_value *v) {
  bool has = false;
  if (napi_has_named_property(env, o, key, &has) != napi_ok || !has) {
    napi_get_undefined(env, v);
    return 1;
  }
  return napi_get_named_property(env, o, key, v) == napi_ok;
}

/* An integer property (0 when absent). */
static int prop_i32(napi_env env, napi_value o, const char *key, int32_t *out) {
  napi_value v;
  *out = 0;
  if (!prop(env, o, key, &v)) return 0;
  if (is_nullish(env, v)) return 1;
  if (!get_i32(env, v, out)) {
    char msg[96];
    snprintf(msg, sizeof msg, "%s must be an integer", key);
    napi_throw_type_error(env, "EARG", msg);
    return 0;
  }
  return 1;
}

static int prop_f32(napi_env env, napi_value o, const char *key, float *out) {
  napi_value v;
  double d = 0;
  *out = 0.0f;
  if (!prop(env, o, key, &v)) return 0;
  if (is_nullish(env, v)) return 1;
  if (!get_f64(env, v, &d)) {
    char msg[96];
    snprintf(msg, sizeof msg, "%s must be a number", key);
    napi_throw_type_error(env, "EARG", msg);
    return 0;
  }
  *out = (float)d;
  return 1;
}

static int prop_operand(napi_env env, napi_value o, const char *key, uint64_t need, int optional,
                        void **out) {
  napi_value v;
  if (!prop(env, o, key, &v)) return 0;
  return operand(env, v, need, optional, key, out);
}

/* A matrix object {N, K, layout, zero, quants, scales?, zeros?} (the
 * QuantMatrix arrays, src/weights.ts:1-31) as the C descriptor, each array
 * holding what wg_q4_sizes says its shape needs. */
static int read_matrix(napi_env env, napi_value o, wg_q4_matrix *m) {
  memset(m, 0, sizeof *m);
  napi_valuetype t;
  if (napi_typeof(env, o, &t) != napi_ok || t != napi_object) {
    napi_throw_type_error(env, "EARG", "matrix must be an object");
    return 0;
  }
  if (!prop_i32(env, o, "N", &m->N) || !prop_i32(env, o, "K", &m->K) ||
      !prop_i32(env, o, "layout", &m->layout) || !prop_i32(env, o, "zero", &m->zero))
    return 0;
  size_t q = 0, s = 0, z = 0;
  int rc = wg_q4_sizes(m->N, m->K, m->layout, m->zero, &q, &s, &z);
  if (rc) {
    throw_wg(env, rc);
    return 0;
  }
  void *p;
  if (!prop_operand(env, o, "quants", q, 0, &p)) return 0;
  m->quants = p;
  if (!prop_operand(env, o, "scales", s, s == 0, &p)) return 0;
  m->scales = p;
  if (!prop_operand(env, o, "zeros", z, z == 0, &p)) return 0;
  m->zeros = p;
  return 1;
}

#define MATRIX_ARG(i, var) \
  wg_q4_matrix var;        \
  if (!read_matrix(env, argv[i], &var)) return NULL

/* An attention shape {heads, kvHeads, headDim, rotatedDims?, eps?, useNorm?}. */
static int read_attn_shape(napi_env env, napi_value o, wg_attn_shape *sh) {
  memset(sh, 0, sizeof *sh);
  napi_valuetype t;
  if (napi_typeof(env, o, &t) != napi_ok || t != napi_object) {
    napi_throw_type_error(env, "EARG", "shape must be an object");
    return 0;
  }
  if (!prop_i32(env, o, "heads", &sh->heads) || !prop_i32(env, o, "kvHeads", &sh->kv_heads) ||
      !prop_i32(env, o, "headDim", &sh->head_dim) ||
      !prop_i32(env, o, "rotatedDims", &sh->rotated_dims) || !prop_f32(env, o, "eps", &sh->eps) ||
      !prop_i32(env, o, "useNorm", &sh->use_norm))
    return 0;
  if (!sh->rotated_dims) sh->rotated_dims = sh->head_dim;
  if (sh->heads <= 0 || sh->kv_heads <= 0 || sh->head_dim <= 0) {
    throw_limits(env, "attention shape: %d heads over %d KV heads of %d", sh->heads, sh->kv_heads,
                 sh->head_dim);
    return 0;
  }
  return 1;
}

#define SHAPE_ARG(i, var) \
  wg_attn_shape var;      \
  if (!read_attn_shape(env, argv[i], &var)) return NULL

/* An epilogue object (wg_epilogue with camelCase names) for M rows of an
 * N-row matrix; absent fields are zero or null. */
static int read_epilogue(napi_env env, napi_value o, int32_t M, int32_t N, wg_epilogue *e) {
  memset(e, 0, sizeof *e);
  napi_valuetype t;
  if (napi_typeof(env, o, &t) != napi_ok || t != napi_object) {
    napi_throw_type_error(env, "EARG", "epilogue must be an object");
    return 0;
  }
  static const struct {
    const char *key;
    size_t at;
  } ints[] = {
      {"mode", offsetof(wg_epilogue, mode)},
      {"nParts", offsetof(wg_epilogue, n_parts)},
      {"ldPartsIn", offsetof(wg_epilogue, ld_parts_in)},
      {"normCount", offsetof(wg_epilogue, norm_count)},
      {"ldResidual", offsetof(wg_epilogue, ld_residual)},
      {"ldOut16", offsetof(wg_epilogue, ld_out16)},
      {"ldPartsOut", offsetof(wg_epilogue, ld_parts_out)},
      {"heads", offsetof(wg_epilogue, heads)},
      {"kvHeads", offsetof(wg_epilogue, kv_heads)},
      {"headDim", offsetof(wg_epilogue, head_dim)},
      {"ctx", offsetof(wg_epilogue, ctx)},
      {"ropeRows", offsetof(wg_epilogue, rope_rows)},
      {"ldQOut", offsetof(wg_epilogue, ld_q_out)},
      {"convWidth", offsetof(wg_epilogue, conv_width)},
  };
  for (size_t k = 0; k < sizeof ints / sizeof ints[0]; k++)
    if (!prop_i32(env, o, ints[k].key, (int32_t *)((char *)e + ints[k].at))) return 0;
  if (!prop_f32(env, o, "eps", &e->eps) || !prop_f32(env, o, "normMult", &e->norm_mult) ||
      !prop_f32(env, o, "normMultOut", &e->norm_mult_out))
    return 0;
  const int64_t hd = e->head_dim;
  const uint64_t out16_width = e->mode == WG_EPI_SWIGLU      ? (uint64_t)N / 2
                               : e->mode == WG_EPI_SHORT_CONV ? (uint64_t)N / 3
                                                              : (uint64_t)N;
  /* (short conv) channels and width */
  const uint64_t cd = (uint64_t)N / 3, cw = (uint64_t)(e->conv_width > 1 ? e->conv_width : 1);
  const uint64_t cache = (uint64_t)(e->ctx > 0 ? e->ctx : 0) * (uint64_t)(e->kv_heads > 0 ? e->kv_heads : 0) *
                         (uint64_t)(hd > 0 ? hd : 0) * 2;
  const struct {
    const char *key;
    void **at;
    uint64_t need;
  } ptrs[] = {
      {"normParts", (void **)&e->norm_parts, span(M, e->ld_parts_in, e->n_parts) * 4},
      {"rowScale", (void **)&e->row_scale, (uint64_t)M * 4},
      {"residual", (void **)&e->residual, span(M, e->ld_residual, N) * 4},
      {"out16", (void **)&e->out16, span(M, e->ld_out16, (int64_t)out16_width) * 2},
      {"out16W", (void **)&e->out16_w, (uint64_t)N * 4},
      {"partsOut", (void **)&e->parts_out, span(M, e->ld_parts_out, N / 4) * 4},
      {"rope", (void **)&e->rope, (uint64_t)(e->rope_rows > 0 ? e->rope_rows : 0) * (uint64_t)(hd > 0 ? hd : 0) * 4},
      {"pos0", (void **)&e->pos0, 4},
      {"qOut", (void **)&e->q_out, span(M, e->ld_q_out, (int64_t)e->heads * hd) * 4},
      {"kCache", (void **)&e->k_cache, cache},
      {"vCache", (void **)&e->v_cache, cache},
      {"convTaps", (void **)&e->conv_taps, cd * cw * 4},
      {"convState", (void **)&e->conv_state, cd * (cw - 1) * 4},
      {"convStateOut", (void **)&e->conv_state_out, cd * (cw - 1) * 4},
      {"convPrefixes", (void **)&e->conv_prefixes, (uint64_t)M * (cw - 1) * cd * 4},
      {"pickParts", &e->pick_parts, (uint64_t)wg_pick_parts_bytes(M)},
  };
  for (size_t k = 0; k < sizeof ptrs / sizeof ptrs[0]; k++)
    if (!prop_operand(env, o, ptrs[k].key, ptrs[k].need, 1, ptrs[k].at)) return 0;
  return 1;
}

static void *ctx_stream(wg_ctx *c) { return wg_ctx_stream(c); }

#define DONE(rc) return (rc) ? throw_wg(env, (rc)) : NULL

/* repack(ctx, kind, matrix, row0, rows, src, srcRows?): the loaders'
 * packers on the GPU (packQ4_0, packQ4_K, repack.ts:60-168); kind "q4_0" |
 * "q4_k" | "q4_k_native" | "q8_0" | "q6_k"; src holds `rows` rows of the
 * file's blocks, srcRows (or null) the logical row of each stored row. */
static napi_value js_repack(napi_env env, napi_callback_info info) {
  ARGS(7);
  HANDLE_ARG(0, wg_ctx, c, H_CTX, "context");
  char kind[16];
  size_t n = 0;
  if (napi_get_value_string_utf8(env, argv[1], kind, sizeof kind, &n) != napi_ok)
    return type_error(env, "kind must be a string");
  MATRIX_ARG(2, m);
  INT32_ARG(3, row0);
  INT32_ARG(4, rows);
  if (row0 < 0 || rows < 1 || row0 > m.N - rows)
    return throw_limits(env, "repack: rows [%d, %d) of a %d-row matrix", row0, row0 + rows, m.N);
  uint64_t per_row = 0; /* a row's bytes in the file */
  if (!strcmp(kind, "q4_0")) per_row = (uint64_t)(m.K / 32) * 18;
  else if (!strcmp(kind, "q4_k") || !strcmp(kind, "q4_k_native")) per_row = (uint64_t)(m.K / 256) * 144;
  else if (!strcmp(kind, "q8_0")) per_row = (uint64_t)(m.K / 32) * 34;
  else if (!strcmp(kind, "q6_k")) per_row = (uint64_t)(m.K / 256) * 210;
  else return type_error(env, "kind must be q4_0, q4_k, q4_k_native, q8_0 or q6_k");
  /* srcRows: host int32 of `rows` source rows, each checked against the
   * rows src holds, then copied to the device for the launch */
  wg_buf *rows_buf = NULL;
  const int32_t *src_rows = NULL;
  void *src_v;
  if (is_nullish(env, argv[6])) {
    if (!operand(env, argv[5], per_row * (uint64_t)rows, 0, "src", &src_v)) return NULL;
  } else {
    napi_typedarray_type type;
    size_t n_rows = 0, off = 0;
    void *data = NULL;
    napi_value ab;
    bool is = false;
    if (napi_is_typedarray(env, argv[6], &is) != napi_ok || !is ||
        napi_get_typedarray_info(env, argv[6], &type, &n_rows, &data, &ab, &off) != napi_ok ||
        type != napi_int32_array)
      return type_error(env, "srcRows must be an Int32Array");
    if (n_rows != (size_t)rows) return throw_limits(env, "repack: %zu srcRows for %d rows", n_rows, rows);
    if (!operand(env, argv[5], per_row, 0, "src", &src_v)) return NULL;
    /* the rows src holds from its offset on */
    napi_value h = argv[5];
    int64_t src_off = 0;
    bool arr = false;
    if (napi_is_array(env, h, &arr) == napi_ok && arr) {
      napi_value o;
      napi_get_element(env, argv[5], 1, &o);
      get_i64(env, o, &src_off);
      napi_get_element(env, argv[5], 0, &h);
    }
    const uint64_t have = (wg_buf_size((wg_buf *)unwrap(env, h, H_BUF, "buffer")) - (uint64_t)src_off) / per_row;
    const int32_t *r = (const int32_t *)data;
    for (int32_t i = 0; i < rows; i++)
      if (r[i] < 0 || (uint64_t)r[i] >= have)
        return throw_limits(env, "repack: srcRows[%d] = %d; src holds %llu rows", i, r[i],
                            (unsigned long long)have);
    int rc = wg_buf_create(c, (size_t)rows * 4, data, &rows_buf);
    if (rc) return throw_wg(env, rc);
    src_rows = (const int32_t *)wg_buf_ptr(rows_buf);
  }
  const void *src = src_v;
  void *s = ctx_stream(c);
  int rc;
  if (!strcmp(kind, "q4_0")) rc = wg_repack_q4_0(&m, row0, rows, src, src_rows, s);
  else if (!strcmp(kind, "q4_k")) rc = wg_repack_q4_k(&m, row0, rows, src, src_rows, s);
  else if (!strcmp(kind, "q4_k_native")) rc = wg_repack_q4_k_native(&m, row0, rows, src, src_rows, s);
  else if (!strcmp(kind, "q8_0")) rc = wg_repack_q8_0(&m, row0, rows, src, src_rows, s);
  else rc = wg_repack_q6_k(&m, row0, rows, src, src_rows, s);
  if (rows_buf) (void)wg_buf_delete(c, rows_buf); /* freed once the launch is done */
  DONE(rc);
}

/* dequant(ctx, matrix, row0, rows, out): matrixRow (repack.ts:865-891),
 * rows x K floats. */
static napi_value js_dequant(napi_env env, napi_callback_info info) {
  ARGS(5);
  HANDLE_ARG(0, wg_ctx, c, H_CTX, "context");
  MATRIX_ARG(1, m);
  INT32_ARG(2, row0);
  INT32_ARG(3, rows);
  if (rows < 1) return throw_limits(env, "dequant: %d rows", rows);
  OPERAND(4, float, out, (uint64_t)rows * (uint64_t)m.K * 4, 0, "out");
  DONE(wg_q4_dequant(&m, row0, rows, out, ctx_stream(c)));
}

/* q4kRecordHalves(ctx, matrix, scales, zeros): packQ4_K's half scales and
 * zero points of a Q4_K-records matrix (N K / 32 halves each), kept for
 * the prompt GEMMs (no reference counterpart; packQ4_K's own arrays). */
static napi_value js_q4k_record_halves(napi_env env, napi_callback_info info) {
  ARGS(4);
  HANDLE_ARG(0, wg_ctx, c, H_CTX, "context");
  MATRIX_ARG(1, m);
  const uint64_t n = (uint64_t)m.N * (uint64_t)(m.K / 32) * 2;
  OPERAND(2, uint16_t, scales, n, 0, "scales");
  OPERAND(3, uint16_t, zeros, n, 0, "zeros");
  DONE(wg_q4k_record_halves(&m, scales, zeros, ctx_stream(c)));
}

/* gemv(ctx, matrix, x, M, y, epilogue?, ldx?, ldy?): splitPartials + pf and
 * the passes folded into it (engine.ts:5241-5377; kernels.ts:744-895,
 * :1169-1361): y [M][ldy] f32 = x [M][ldx] halves times W^T, with the
 * epilogue's norm, residual, SwiGLU or RoPE + KV write. */
static napi_value js_gemv(napi_env env, napi_callback_info info) {
  ARGS(8);
  HANDLE_ARG(0, wg_ctx, c, H_CTX, "context");
  MATRIX_ARG(1, m);
  INT32_ARG(3, M);
  int32_t ldx = m.K, ldy = m.N;
  if (!is_nullish(env, argv[6]) && !get_i32(env, argv[6], &ldx)) return type_error(env, "ldx must be an integer");
  if (!is_nullish(env, argv[7]) && !get_i32(env, argv[7], &ldy)) return type_error(env, "ldy must be an integer");
  if (M < 1 || M > 8) return throw_limits(env, "gemv: %d rows (1 to 8)", M);
  OPERAND(2, const uint16_t, x, span(M, ldx, m.K) * 2, 0, "x");
  wg_epilogue ep;
  const int has_ep = !is_nullish(env, argv[5]);
  if (has_ep && !read_epilogue(env, argv[5], M, m.N, &ep)) return NULL;
  const int needs_y = !has_ep || ep.mode == WG_EPI_STORE;
  OPERAND(4, float, y, needs_y ? span(M, ldy, m.N) * 4 : 0, !needs_y, "y");
  DONE(wg_q4_gemv(&m, x, M, ldx, y, ldy, has_ep ? &ep : NULL, ctx_stream(c)));
}

/* gemm(ctx, matrix, A, M, C, {lda?, ldc?, residual?, ldr?, rowScale?,
 * colOf?}): Engine.matmul for a prompt batch (engine.ts:4969-5234) on
 * MFMA: C [M][ldc] f32 = (residual) + row_scale * A [M][lda] halves W^T. */
static napi_value js_gemm(napi_env env, napi_callback_info info) {
  ARGS(6);
  HANDLE_ARG(0, wg_ctx, c, H_CTX, "context");
  MATRIX_ARG(1, m);
  INT32_ARG(3, M);
  if (M < 1) return throw_limits(env, "gemm: %d rows", M);
  int32_t lda = m.K, ldc = m.N, ldr = m.N;
  void *residual = NULL, *row_scale = NULL, *col_of = NULL;
  if (!is_nullish(env, argv[5])) {
    napi_value o = argv[5];
    int32_t v;
    if (!prop_i32(env, o, "lda", &v)) return NULL;
    if (v) lda = v;
    if (!prop_i32(env, o, "ldc", &v)) return NULL;
    if (v) ldc = v;
    if (!prop_i32(env, o, "ldr", &v)) return NULL;
    if (v) ldr = v;
    if (!prop_operand(env, o, "residual", span(M, ldr, m.N) * 4, 1, &residual) ||
        !prop_operand(env, o, "rowScale", (uint64_t)M * 4, 1, &row_scale) ||
        !prop_operand(env, o, "colOf", (uint64_t)m.N * 4, 1, &col_of))
      return NULL;
  }
  OPERAND(2, const uint16_t, A, span(M, lda, m.K) * 2, 0, "A");
  OPERAND(4, float, C, span(M, ldc, m.N) * 4, 0, "C");
  DONE(wg_q4_gemm(&m, A, M, lda, C, ldc, (const float *)residual, ldr, (const float *)row_scale,
                  (const int32_t *)col_of, ctx_stream(c)));
}

/* gemmSwiglu(ctx, matrix, A, M, out16, rowScale?, lda?, ldo?): the gate|up
 * GEMM with SwiGLU folded in (src/gpu/native.ts:33; kernels.ts:1066-1077):
 * out16 [M][ldo] halves, N / 2 columns. */
static napi_value js_gemm_swiglu(napi_env env, napi_callback_info info) {
  ARGS(8);
  HANDLE_ARG(0, wg_ctx, c, H_CTX, "context");
  MATRIX_ARG(1, m);
  INT32_ARG(3, M);
  if (M < 1) return throw_limits(env, "gemmSwiglu: %d rows", M);
  int32_t lda = m.K, ldo = m.N / 2;
  if (!is_nullish(env, argv[6]) && !get_i32(env, argv[6], &lda)) return type_error(env, "lda must be an integer");
  if (!is_nullish(env, argv[7]) && !get_i32(env, argv[7], &ldo)) return type_error(env, "ldo must be an integer");
  OPERAND(2, const uint16_t, A, span(M, lda, m.K) * 2, 0, "A");
  OPERAND(4, uint16_t, out16, span(M, ldo, m.N / 2) * 2, 0, "out16");
  OPERAND(5, const float, row_scale, (uint64_t)M * 4, 1, "rowScale");
  DONE(wg_q4_gemm_swiglu(&m, A, M, lda, out16, ldo, row_scale, ctx_stream(c)));
}

/* embed(ctx, matrix, ids, M, h, epilogue?, ldh?): embed / embedFold
 * (kernels.ts:1092-1149, :985-1041): h [M][ldh] = the ids' dequantized
 * rows, with the epilogue's prescaled half input and sums of squares. */
static napi_value js_embed(napi_env env, napi_callback_info info) {
  ARGS(7);
  HANDLE_ARG(0, wg_ctx, c, H_CTX, "context");
  MATRIX_ARG(1, m);
  INT32_ARG(3, M);
  if (M < 1) return throw_limits(env, "embed: %d rows", M);
  int32_t ldh = m.K;
  if (!is_nullish(env, argv[6]) && !get_i32(env, argv[6], &ldh)) return type_error(env, "ldh must be an integer");
  OPERAND(2, const int32_t, ids, (uint64_t)M * 4, 0, "ids");
  OPERAND(4, float, h, span(M, ldh, m.K) * 4, 0, "h");
  wg_epilogue ep;
  const int has_ep = !is_nullish(env, argv[5]);
  if (has_ep && !read_epilogue(env, argv[5], M, m.K, &ep)) return NULL;
  DONE(wg_embed(&m, ids, M, h, ldh, has_ep ? &ep : NULL, ctx_stream(c)));
}

/* embedDrafts(ctx, matrix, ids, rows, table, nSteps, cursor, h, epilogue?,
 * ldh?): verifyDrafts and embed in one launch (row 0 embeds ids[0], rows
 * 1 .. rows - 1 the table's row *cursor, also written to ids). */
static napi_value js_embed_drafts(napi_env env, napi_callback_info info) {
  ARGS(10);
  HANDLE_ARG(0, wg_ctx, c, H_CTX, "context");
  MATRIX_ARG(1, m);
  INT32_ARG(3, rows);
  INT32_ARG(5, n_steps);
  if (rows < 2 || n_steps < 1) return throw_limits(env, "embedDrafts: %d rows, %d table rows", rows, n_steps);
  int32_t ldh = m.K;
  if (!is_nullish(env, argv[9]) && !get_i32(env, argv[9], &ldh)) return type_error(env, "ldh must be an integer");
  OPERAND(2, int32_t, ids, (uint64_t)rows * 4, 0, "ids");
  OPERAND(4, const int32_t, table, (uint64_t)n_steps * (uint64_t)(rows - 1) * 4, 0, "table");
  OPERAND(6, const int32_t, cursor, 4, 0, "cursor");
  OPERAND(7, float, h, span(rows, ldh, m.K) * 4, 0, "h");
  wg_epilogue ep;
  const int has_ep = !is_nullish(env, argv[8]);
  if (has_ep && !read_epilogue(env, argv[8], rows, m.K, &ep)) return NULL;
  DONE(wg_embed_drafts(&m, ids, rows, table, n_steps, cursor, h, ldh, has_ep ? &ep : NULL, ctx_stream(c)));
}

/* normToH2(ctx, x, M, D, w, eps, out, rowScale, ldx?, ldo?): NORM_TO_H2
 * with PRESCALE 32 (kernels.ts:89, :1195-1242). */
static napi_value js_norm_to_h2(napi_env env, napi_callback_info info) {
  ARGS(10);
  HANDLE_ARG(0, wg_ctx, c, H_CTX, "context");
  INT32_ARG(2, M);
  INT32_ARG(3, D);
  FLOAT_ARG(5, eps);
  if (M < 1 || D < 1) return throw_limits(env, "normToH2: %d rows of %d", M, D);
  int32_t ldx = D, ldo = D;
  if (!is_nullish(env, argv[8]) && !get_i32(env, argv[8], &ldx)) return type_error(env, "ldx must be an integer");
  if (!is_nullish(env, argv[9]) && !get_i32(env, argv[9], &ldo)) return type_error(env, "ldo must be an integer");
  OPERAND(1, const float, x, span(M, ldx, D) * 4, 0, "x");
  OPERAND(4, const float, w, (uint64_t)D * 4, 0, "w");
  OPERAND(6, uint16_t, out, span(M, ldo, D) * 2, 0, "out");
  OPERAND(7, float, row_scale, (uint64_t)M * 4, 0, "rowScale");
  DONE(wg_norm_to_h2(x, M, D, ldx, w, eps, out, ldo, row_scale, ctx_stream(c)));
}

/* headPrep(ctx, qkv, M, shape, qNorm?, kNorm?, rope, ropeRows, pos0, qOut,
 * kCache, vCache, ctxRows, ldq?, ldqo?): headPrep + values
 * (kernels.ts:2196-2322, :3030-3045). */
static napi_value js_head_prep(napi_env env, napi_callback_info info) {
  ARGS(15);
  HANDLE_ARG(0, wg_ctx, c, H_CTX, "context");
  INT32_ARG(2, M);
  SHAPE_ARG(3, sh);
  INT32_ARG(7, rope_rows);
  INT32_ARG(12, ctx_rows);
  const int64_t hd = sh.head_dim, qd = (int64_t)sh.heads * hd, kvd = (int64_t)sh.kv_heads * hd;
  int32_t ldq = (int32_t)(qd + 2 * kvd), ldqo = (int32_t)qd;
  if (!is_nullish(env, argv[13]) && !get_i32(env, argv[13], &ldq)) return type_error(env, "ldq must be an integer");
  if (!is_nullish(env, argv[14]) && !get_i32(env, argv[14], &ldqo)) return type_error(env, "ldqo must be an integer");
  if (M < 1 || rope_rows < 1 || ctx_rows < 1)
    return throw_limits(env, "headPrep: %d rows, %d rope rows, %d cache rows", M, rope_rows, ctx_rows);
  OPERAND(1, const float, qkv, span(M, ldq, qd + 2 * kvd) * 4, 0, "qkv");
  OPERAND(4, const float, q_norm, (uint64_t)hd * 4, 1, "qNorm");
  OPERAND(5, const float, k_norm, (uint64_t)hd * 4, 1, "kNorm");
  OPERAND(6, const float, rope, (uint64_t)rope_rows * (uint64_t)hd * 4, 0, "rope");
  OPERAND(8, const int32_t, pos0, 4, 0, "pos0");
  OPERAND(9, float, q_out, span(M, ldqo, qd) * 4, 0, "qOut");
  OPERAND(10, uint16_t, k_cache, (uint64_t)ctx_rows * (uint64_t)kvd * 2, 0, "kCache");
  OPERAND(11, uint16_t, v_cache, (uint64_t)ctx_rows * (uint64_t)kvd * 2, 0, "vCache");
  DONE(wg_head_prep(qkv, M, ldq, &sh, q_norm, k_norm, rope, rope_rows, pos0, q_out, ldqo, k_cache,
                    v_cache, ctx_rows, ctx_stream(c)));
}

static napi_value js_attn_scratch_bytes(napi_env env, napi_callback_info info) {
  ARGS(4);
  INT32_ARG(0, M);
  INT32_ARG(1, heads);
  INT32_ARG(2, head_dim);
  INT32_ARG(3, max_keys);
  return num(env, (double)wg_attn_scratch_bytes(M, heads, head_dim, max_keys));
}

/* attnDecode(ctx, q, M, shape, kCache, vCache, pos0, maxKeys, out, scratch,
 * ldq?, ldo?): scores, attend, attendPanel + attendPanelCombine
 * (kernels.ts:2386-2579, :2803-3027) for up to a few query rows.
 * attnPrefill(ctx, q, M, shape, kCache, vCache, pos0, maxKeys, out, ldq?,
 * ldo?): the prompt plan (engine.ts:6359-6630). */
static napi_value attn_common(napi_env env, napi_callback_info info, int prefill) {
  ARGS(12);
  HANDLE_ARG(0, wg_ctx, c, H_CTX, "context");
  INT32_ARG(2, M);
  SHAPE_ARG(3, sh);
  INT32_ARG(7, max_keys);
  const int extra = prefill ? 9 : 10;
  const int64_t qd = (int64_t)sh.heads * sh.head_dim, kvd = (int64_t)sh.kv_heads * sh.head_dim;
  int32_t ldq = (int32_t)qd, ldo = (int32_t)qd;
  if (!is_nullish(env, argv[extra]) && !get_i32(env, argv[extra], &ldq)) return type_error(env, "ldq must be an integer");
  if (!is_nullish(env, argv[extra + 1]) && !get_i32(env, argv[extra + 1], &ldo)) return type_error(env, "ldo must be an integer");
  if (M < 1 || max_keys < 1) return throw_limits(env, "attention: %d rows over %d keys", M, max_keys);
  OPERAND(1, const float, q, span(M, ldq, qd) * 4, 0, "q");
  OPERAND(4, const uint16_t, k_cache, (uint64_t)max_keys * (uint64_t)kvd * 2, 0, "kCache");
  OPERAND(5, const uint16_t, v_cache, (uint64_t)max_keys * (uint64_t)kvd * 2, 0, "vCache");
  OPERAND(6, const int32_t, pos0, 4, 0, "pos0");
  OPERAND(8, uint16_t, out, span(M, ldo, qd) * 2, 0, "out");
  if (prefill)
    DONE(wg_attn_prefill(q, M, ldq, &sh, k_cache, v_cache, pos0, max_keys, out, ldo, ctx_stream(c)));
  const size_t need = wg_attn_scratch_bytes(M, sh.heads, sh.head_dim, max_keys);
  OPERAND(9, void, scratch, need, 0, "scratch");
  DONE(wg_attn_decode(q, M, ldq, &sh, k_cache, v_cache, pos0, max_keys, out, ldo, scratch, need,
                      ctx_stream(c)));
}

static napi_value js_attn_decode(napi_env env, napi_callback_info info) {
  return attn_common(env, info, 0);
}

static napi_value js_attn_prefill(napi_env env, napi_callback_info info) {
  return attn_common(env, info, 1);
}

/* attnDecodePrep(ctx, qkv, M, shape, qNorm?, kNorm?, rope, ropeRows, pos0,
 * kCache, vCache, ctxRows, out, scratch, qOut?, ldqkv?, ldo?): headPrep +
 * values and the decode attention in one launch (kernels.ts:2196-2322,
 * :2803-3027); throws WG_ERR_UNSUPPORTED for a shape the kernel does not
 * take (then headPrep and attnDecode). */
static napi_value js_attn_decode_prep(napi_env env, napi_callback_info info) {
  ARGS(17);
  HANDLE_ARG(0, wg_ctx, c, H_CTX, "context");
  INT32_ARG(2, M);
  SHAPE_ARG(3, sh);
  INT32_ARG(7, rope_rows);
  INT32_ARG(11, ctx_rows);
  const int64_t hd = sh.head_dim, qd = (int64_t)sh.heads * hd, kvd = (int64_t)sh.kv_heads * hd;
  int32_t ldqkv = (int32_t)(qd + 2 * kvd), ldo = (int32_t)qd;
  if (!is_nullish(env, argv[15]) && !get_i32(env, argv[15], &ldqkv)) return type_error(env, "ldqkv must be an integer");
  if (!is_nullish(env, argv[16]) && !get_i32(env, argv[16], &ldo)) return type_error(env, "ldo must be an integer");
  if (M < 1 || ctx_rows < 1 || rope_rows < 1)
    return throw_limits(env, "attnDecodePrep: %d rows, a cache of %d", M, ctx_rows);
  OPERAND(1, const float, qkv, span(M, ldqkv, qd + 2 * kvd) * 4, 0, "qkv");
  OPERAND(4, const float, q_norm, (uint64_t)hd * 4, 1, "qNorm");
  OPERAND(5, const float, k_norm, (uint64_t)hd * 4, 1, "kNorm");
  OPERAND(6, const float, rope, (uint64_t)rope_rows * (uint64_t)hd * 4, 0, "rope");
  OPERAND(8, const int32_t, pos0, 4, 0, "pos0");
  OPERAND(9, uint16_t, k_cache, (uint64_t)ctx_rows * (uint64_t)kvd * 2, 0, "kCache");
  OPERAND(10, uint16_t, v_cache, (uint64_t)ctx_rows * (uint64_t)kvd * 2, 0, "vCache");
  OPERAND(12, uint16_t, out, span(M, ldo, qd) * 2, 0, "out");
  const size_t need = wg_attn_scratch_bytes(M, sh.heads, sh.head_dim, ctx_rows);
  OPERAND(13, void, scratch, need, 0, "scratch");
  OPERAND(14, float, q_out, span(M, (int32_t)qd, qd) * 4, 1, "qOut");
  DONE(wg_attn_decode_prep(qkv, M, ldqkv, &sh, q_norm, k_norm, rope, rope_rows, ctx_rows, k_cache,
                           v_cache, pos0, ctx_rows, q_out, (int32_t)qd, out, ldo, scratch, need,
                           ctx_stream(c)));
}

/* shortConv(ctx, bcx, M, D, W, taps, state, stateOut, prefixes?, out, ldb?,
 * ldo?): convFused + convPrefixes (kernels.ts:1447-1523; Engine.convolve,
 * engine.ts:5806-5899). */
static napi_value js_short_conv(napi_env env, napi_callback_info info) {
  ARGS(12);
  HANDLE_ARG(0, wg_ctx, c, H_CTX, "context");
  INT32_ARG(2, M);
  INT32_ARG(3, D);
  INT32_ARG(4, W);
  if (M < 1 || D < 1 || W < 2) return throw_limits(env, "shortConv: %d rows of %d, width %d", M, D, W);
  int32_t ldb = 3 * D, ldo = D;
  if (!is_nullish(env, argv[10]) && !get_i32(env, argv[10], &ldb)) return type_error(env, "ldb must be an integer");
  if (!is_nullish(env, argv[11]) && !get_i32(env, argv[11], &ldo)) return type_error(env, "ldo must be an integer");
  const uint64_t st = (uint64_t)(W - 1) * (uint64_t)D * 4;
  OPERAND(1, const float, bcx, span(M, ldb, 3 * (int64_t)D) * 4, 0, "bcx");
  OPERAND(5, const float, taps, (uint64_t)D * (uint64_t)W * 4, 0, "taps");
  OPERAND(6, const float, state, st, 0, "state");
  OPERAND(7, float, state_out, st, 0, "stateOut");
  OPERAND(8, float, prefixes, (uint64_t)M * st, 1, "prefixes");
  OPERAND(9, uint16_t, out, span(M, ldo, D) * 2, 0, "out");
  DONE(wg_short_conv(bcx, M, D, ldb, W, taps, state, state_out, prefixes, out, ldo, ctx_stream(c)));
}

/* convAccept(ctx, prefixes, kept, rows, D, W, state): Engine.accept's
 * rollback (engine.ts:8063-8086, COPY_ROWS kernels.ts:2177-2183). */
static napi_value js_conv_accept(napi_env env, napi_callback_info info) {
  ARGS(7);
  HANDLE_ARG(0, wg_ctx, c, H_CTX, "context");
  INT32_ARG(2, kept);
  INT32_ARG(3, rows);
  INT32_ARG(4, D);
  INT32_ARG(5, W);
  if (rows < 1 || D < 1 || W < 2) return throw_limits(env, "convAccept: %d rows of %d, width %d", rows, D, W);
  const uint64_t st = (uint64_t)(W - 1) * (uint64_t)D * 4;
  OPERAND(1, const float, prefixes, (uint64_t)rows * st, 0, "prefixes");
  OPERAND(6, float, state, st, 0, "state");
  DONE(wg_conv_accept(prefixes, kept, rows, D, W, state, ctx_stream(c)));
}

/* convStates(ctx, [{prefixes, state, dim, width}]): a device array of
 * wg_conv_state for verifyAccept, in a new buffer (its size checked
 * against each layer's, `rows` prefixes each). */
static napi_value js_conv_states(napi_env env, napi_callback_info info) {
  ARGS(3);
  HANDLE_ARG(0, wg_ctx, c, H_CTX, "context");
  INT32_ARG(2, rows);
  bool is = false;
  uint32_t n = 0;
  if (napi_is_array(env, argv[1], &is) != napi_ok || !is ||
      napi_get_array_length(env, argv[1], &n) != napi_ok || n == 0 || n > 4096)
    return type_error(env, "convStates takes a non-empty array of layers");
  if (rows < 1 || rows > 64) return throw_limits(env, "convStates: %d rows", rows);
  wg_conv_state *arr = (wg_conv_state *)calloc(n, sizeof *arr);
  if (!arr) {
    napi_throw_error(env, "EADDON", "out of host memory");
    return NULL;
  }
  for (uint32_t i = 0; i < n; i++) {
    napi_value o;
    void *p;
    if (napi_get_element(env, argv[1], i, &o) != napi_ok || !prop_i32(env, o, "dim", &arr[i].dim) ||
        !prop_i32(env, o, "width", &arr[i].width)) {
      free(arr);
      return NULL;
    }
    if (arr[i].dim < 1 || arr[i].width < 2) {
      free(arr);
      return throw_limits(env, "convStates: layer %u is %d wide with %d taps", i, arr[i].dim, arr[i].width);
    }
    const uint64_t st = (uint64_t)(arr[i].width - 1) * (uint64_t)arr[i].dim * 4;
    if (!prop_operand(env, o, "prefixes", (uint64_t)rows * st, 0, &p)) {
      free(arr);
      return NULL;
    }
    arr[i].prefixes = (float *)p;
    if (!prop_operand(env, o, "state", st, 0, &p)) {
      free(arr);
      return NULL;
    }
    arr[i].state = (float *)p;
  }
  wg_buf *b = NULL;
  int rc = wg_buf_create(c, (size_t)n * sizeof *arr, arr, &b);
  free(arr);
  if (rc) return throw_wg(env, rc);
  return wrap(env, H_BUF, b);
}

/* verifyAccept(ctx, picks, rows, convs, nConv, maxState, pos, ids, hist,
 * histLen, keptLog, logLen, cursor): Engine.accept after a verify batch with
 * the handler's keep rule (engine.ts:8063-8086, handler.ts:1811-1887), on
 * the device. */
static napi_value js_verify_accept(napi_env env, napi_callback_info info) {
  ARGS(13);
  HANDLE_ARG(0, wg_ctx, c, H_CTX, "context");
  INT32_ARG(2, rows);
  INT32_ARG(4, n_conv);
  INT32_ARG(5, max_state);
  INT32_ARG(9, hist_len);
  INT32_ARG(11, log_len);
  if (rows < 1 || n_conv < 0 || hist_len < 0 || log_len < 0)
    return throw_limits(env, "verifyAccept: %d rows, %d conv layers", rows, n_conv);
  OPERAND(1, const int32_t, picks, (uint64_t)rows * 4, 0, "picks");
  OPERAND(3, const wg_conv_state, convs, (uint64_t)n_conv * sizeof(wg_conv_state), n_conv == 0, "convs");
  OPERAND(6, int32_t, pos, 4, 0, "pos");
  OPERAND(7, int32_t, ids, (uint64_t)rows * 4, 0, "ids");
  OPERAND(8, int32_t, hist, (uint64_t)hist_len * 4, hist_len == 0, "hist");
  OPERAND(10, int32_t, kept_log, (uint64_t)log_len * 4, log_len == 0, "keptLog");
  OPERAND(12, int32_t, cursor, 4, 0, "cursor");
  DONE(wg_verify_accept(picks, rows, convs, n_conv, max_state, pos, ids, hist, hist_len, kept_log,
                        log_len, cursor, ctx_stream(c)));
}

/* verifyAcceptParts(ctx, parts, picksOut, rows, convs, nConv, maxState, pos,
 * ids, hist, histLen, keptLog, logLen, cursor): argmaxParts and
 * verifyAccept in one launch (the picks also to picksOut). */
static napi_value js_verify_accept_parts(napi_env env, napi_callback_info info) {
  ARGS(14);
  HANDLE_ARG(0, wg_ctx, c, H_CTX, "context");
  INT32_ARG(3, rows);
  INT32_ARG(5, n_conv);
  INT32_ARG(6, max_state);
  INT32_ARG(10, hist_len);
  INT32_ARG(12, log_len);
  if (rows < 1 || rows > 8 || n_conv < 0 || hist_len < 0 || log_len < 0)
    return throw_limits(env, "verifyAcceptParts: %d rows, %d conv layers", rows, n_conv);
  OPERAND(1, const void, parts, (uint64_t)wg_pick_parts_bytes(rows), 0, "parts");
  OPERAND(2, int32_t, picks_out, (uint64_t)rows * 4, 0, "picksOut");
  OPERAND(4, const wg_conv_state, convs, (uint64_t)n_conv * sizeof(wg_conv_state), n_conv == 0, "convs");
  OPERAND(7, int32_t, pos, 4, 0, "pos");
  OPERAND(8, int32_t, ids, (uint64_t)rows * 4, 0, "ids");
  OPERAND(9, int32_t, hist, (uint64_t)hist_len * 4, hist_len == 0, "hist");
  OPERAND(11, int32_t, kept_log, (uint64_t)log_len * 4, log_len == 0, "keptLog");
  OPERAND(13, int32_t, cursor, 4, 0, "cursor");
  DONE(wg_verify_accept_parts(parts, picks_out, rows, convs, n_conv, max_state, pos, ids, hist,
                              hist_len, kept_log, log_len, cursor, ctx_stream(c)));
}

/* verifyDrafts(ctx, ids, rows, table, nSteps, cursor): a verify step's
 * drafts from a device table (the reference's lookupDraft runs on the
 * host, src/draft.ts:15-45). */
static napi_value js_verify_drafts(napi_env env, napi_callback_info info) {
  ARGS(6);
  HANDLE_ARG(0, wg_ctx, c, H_CTX, "context");
  INT32_ARG(2, rows);
  INT32_ARG(4, n_steps);
  if (rows < 2 || n_steps < 1) return throw_limits(env, "verifyDrafts: %d rows, %d steps", rows, n_steps);
  OPERAND(1, int32_t, ids, (uint64_t)rows * 4, 0, "ids");
  OPERAND(3, const int32_t, table, (uint64_t)n_steps * (uint64_t)(rows - 1) * 4, 0, "table");
  OPERAND(5, const int32_t, cursor, 4, 0, "cursor");
  DONE(wg_verify_drafts(ids, rows, table, n_steps, cursor, ctx_stream(c)));
}

static napi_value js_argmax_scratch_bytes(napi_env env, napi_callback_info info) {
  ARGS(2);
  INT32_ARG(0, M);
  INT32_ARG(1, V);
  return num(env, (double)wg_argmax_scratch_bytes(M, V));
}

/* argmax(ctx, logits, M, V, ids, scratch, tops?, ld?): Engine.argmax
 * (engine.ts:8271-8336; CHUNK_MAX_AT + CHUNK_ARGMAX_ROWS,
 * kernels.ts:3169-3246). */
static napi_value js_argmax(napi_env env, napi_callback_info info) {
  ARGS(8);
  HANDLE_ARG(0, wg_ctx, c, H_CTX, "context");
  INT32_ARG(2, M);
  INT32_ARG(3, V);
  int32_t ld = V;
  if (!is_nullish(env, argv[7]) && !get_i32(env, argv[7], &ld)) return type_error(env, "ld must be an integer");
  if (M < 1 || V < 1) return throw_limits(env, "argmax: %d rows of %d", M, V);
  const size_t need = wg_argmax_scratch_bytes(M, V);
  OPERAND(1, const float, logits, span(M, ld, V) * 4, 0, "logits");
  OPERAND(4, int32_t, ids, (uint64_t)M * 4, 0, "ids");
  OPERAND(5, void, scratch, need, 0, "scratch");
  OPERAND(6, float, tops, (uint64_t)M * 4, 1, "tops");
  DONE(wg_argmax_rows(logits, M, V, ld, ids, tops, scratch, need, ctx_stream(c)));
}

/* argmaxAdvance(ctx, logits, V, ids, pos, hist?, histLen, scratch, tops?):
 * one greedy decode step's pick and advance on the device (the guessed
 * forward's pick, engine.ts:8095-8110, :8318-8336). */
static napi_value js_argmax_advance(napi_env env, napi_callback_info info) {
  ARGS(9);
  HANDLE_ARG(0, wg_ctx, c, H_CTX, "context");
  INT32_ARG(2, V);
  INT32_ARG(6, hist_len);
  if (V < 1 || hist_len < 0) return throw_limits(env, "argmaxAdvance: %d logits", V);
  const size_t need = wg_argmax_scratch_bytes(1, V);
  OPERAND(1, const float, logits, (uint64_t)V * 4, 0, "logits");
  OPERAND(3, int32_t, ids, 4, 0, "ids");
  OPERAND(4, int32_t, pos, 4, 0, "pos");
  OPERAND(5, int32_t, hist, (uint64_t)hist_len * 4, hist_len == 0, "hist");
  OPERAND(7, void, scratch, need, 0, "scratch");
  OPERAND(8, float, tops, 4, 1, "tops");
  DONE(wg_argmax_advance(logits, V, ids, pos, hist, hist_len, tops, scratch, need, ctx_stream(c)));
}

static napi_value js_pick_parts_bytes(napi_env env, napi_callback_info info) {
  ARGS(1);
  INT32_ARG(0, M);
  return num(env, (double)wg_pick_parts_bytes(M));
}

/* argmaxParts(ctx, parts, M, ids, tops?, pos?, hist?, histLen): the greedy
 * picks from a head GEMV's pickParts (the epilogue's first stage of
 * CHUNK_ARGMAX_ROWS, kernels.ts:3169-3246); with pos (M = 1) the decode
 * step's advance as argmaxAdvance. */
static napi_value js_argmax_parts(napi_env env, napi_callback_info info) {
  ARGS(8);
  HANDLE_ARG(0, wg_ctx, c, H_CTX, "context");
  INT32_ARG(2, M);
  INT32_ARG(7, hist_len);
  if (M < 1 || M > 8 || hist_len < 0) return throw_limits(env, "argmaxParts: %d rows", M);
  OPERAND(1, const void, parts, (uint64_t)wg_pick_parts_bytes(M), 0, "parts");
  OPERAND(3, int32_t, ids, (uint64_t)M * 4, 0, "ids");
  OPERAND(4, float, tops, (uint64_t)M * 4, 1, "tops");
  OPERAND(5, int32_t, pos, 4, 1, "pos");
  OPERAND(6, int32_t, hist, (uint64_t)hist_len * 4, 1, "hist");
  DONE(wg_argmax_parts(parts, M, ids, tops, pos, hist, hist_len, ctx_stream(c)));
}

static napi_value js_pick_scratch_bytes(napi_env env, napi_callback_info info) {
  ARGS(2);
  INT32_ARG(0, M);
  INT32_ARG(1, V);
  return num(env, (double)wg_pick_scratch_bytes(M, V));
}

/* pickCandidates(ctx, logits, M, V, count, chunksOut, candidates, scratch,
 * {ld?, mask?, seenRows?, nSeen?, row0?, penalty?, presencePenalty?,
 * allowed?, allowedRows?, ldAllowed?}): Engine.pick's penalized chunk
 * candidates (engine.ts:8352-8473; kernels.ts:3085-3163, :3265-3323). */
static napi_value js_pick_candidates(napi_env env, napi_callback_info info) {
  ARGS(9);
  HANDLE_ARG(0, wg_ctx, c, H_CTX, "context");
  INT32_ARG(2, M);
  INT32_ARG(3, V);
  INT32_ARG(4, count);
  if (M < 1 || V < 1 || count < 1 || count > 64)
    return throw_limits(env, "pickCandidates: %d rows of %d, %d chunks", M, V, count);
  int32_t ld = V, n_seen = 0, row0 = 0, allowed_rows = 0, ld_allowed = 0;
  float penalty = 1.0f, presence = 0.0f;
  void *mask = NULL, *seen = NULL, *allowed = NULL;
  if (!is_nullish(env, argv[8])) {
    napi_value o = argv[8];
    int32_t v;
    if (!prop_i32(env, o, "ld", &v)) return NULL;
    if (v) ld = v;
    if (!prop_i32(env, o, "nSeen", &n_seen) || !prop_i32(env, o, "row0", &row0) ||
        !prop_i32(env, o, "allowedRows", &allowed_rows) || !prop_i32(env, o, "ldAllowed", &ld_allowed))
      return NULL;
    napi_value pv;
    if (!prop(env, o, "penalty", &pv)) return NULL;
    if (!is_nullish(env, pv) && !prop_f32(env, o, "penalty", &penalty)) return NULL;
    if (!prop_f32(env, o, "presencePenalty", &presence)) return NULL;
    if (n_seen < 0 || allowed_rows < 0 || ld_allowed < 0)
      return throw_limits(env, "pickCandidates: negative counts");
    if (!prop_operand(env, o, "mask", (uint64_t)V, 1, &mask) ||
        !prop_operand(env, o, "seenRows", (uint64_t)n_seen * 16, n_seen == 0, &seen) ||
        !prop_operand(env, o, "allowed", span(allowed_rows, ld_allowed, ld_allowed) * 4, 1, &allowed))
      return NULL;
  }
  const size_t need = wg_pick_scratch_bytes(M, V);
  OPERAND(1, const float, logits, span(M, ld, V) * 4, 0, "logits");
  OPERAND(5, int32_t, chunks_out, (uint64_t)M * (uint64_t)count * 4, 0, "chunksOut");
  OPERAND(6, float, candidates, (uint64_t)M * (uint64_t)count * 256 * 4, 0, "candidates");
  OPERAND(7, void, scratch, need, 0, "scratch");
  DONE(wg_pick_candidates(logits, M, V, ld, (const uint8_t *)mask, (const int32_t *)seen, n_seen,
                          row0, penalty, presence, (const uint32_t *)allowed, allowed_rows,
                          ld_allowed, count, chunks_out, candidates, scratch, need, ctx_stream(c)));
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
      {"fence", js_fence_record},
      {"repack", js_repack},
      {"dequant", js_dequant},
      {"q4kRecordHalves", js_q4k_record_halves},
      {"gemv", js_gemv},
      {"gemm", js_gemm},
      {"gemmSwiglu", js_gemm_swiglu},
      {"embed", js_embed},
      {"normToH2", js_norm_to_h2},
      {"headPrep", js_head_prep},
      {"attnScratchBytes", js_attn_scratch_bytes},
      {"attnDecode", js_attn_decode},
      {"attnPrefill", js_attn_prefill},
      {"attnDecodePrep", js_attn_decode_prep},
      {"shortConv", js_short_conv},
      {"convAccept", js_conv_accept},
      {"convStates", js_conv_states},
      {"verifyAccept", js_verify_accept},
      {"verifyDrafts", js_verify_drafts},
      {"verifyAcceptParts", js_verify_accept_parts},
      {"embedDrafts", js_embed_drafts},
      {"argmaxScratchBytes", js_argmax_scratch_bytes},
      {"argmax", js_argmax},
      {"argmaxAdvance", js_argmax_advance},
      {"argmaxParts", js_argmax_parts},
      {"pickPartsBytes", js_pick_parts_bytes},
      {"pickScratchBytes", js_pick_scratch_bytes},
      {"pickCandidates", js_pick_candidates},
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
  set(env, consts, "ZERO_Q4K", num(env, WG_ZERO_Q4K));
  set(env, consts, "EPI_STORE", num(env, WG_EPI_STORE));
  set(env, consts, "EPI_SWIGLU", num(env, WG_EPI_SWIGLU));
  set(env, consts, "EPI_ROPE_KV", num(env, WG_EPI_ROPE_KV));
  set(env, consts, "EPI_SHORT_CONV", num(env, WG_EPI_SHORT_CONV));
  set(env, consts, "CONV_STATE_BYTES", num(env, (double)sizeof(wg_conv_state)));
  set(env, exports, "constants", consts);
  return exports;
}

NAPI_MODULE(webgllm_hip, init)
