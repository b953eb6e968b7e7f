// The backend object (reference: class Gpu, src/gpu/gl.ts:47, and the
// PacedGpu contract, src/gpu/paced.ts:11-22), on HIP: a context owns a
// device and one stream, buffers stand in for textures, readbacks complete
// behind events.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>
#include <string>
#include <unordered_set>

#include "common.h"
#include "dot.h"

namespace wg {

static thread_local char g_error[512] = "";

int fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof g_error, fmt, ap);
  va_end(ap);
  return code;
}

int launched(const char *what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(WG_ERR_DEVICE, "%s launch: %s", what, hipGetErrorString(e));
  return WG_OK;
}

int check_matrix(const wg_q4_matrix *m, const char *who) {
  WG_REQUIRE(m, "%s: no matrix", who);
  WG_REQUIRE(m->N > 0 && m->N % 4 == 0, "%s: matrix rows (%d) must be a positive multiple of 4",
             who, m->N);
  WG_REQUIRE(m->quants, "%s: matrix has no quants", who);
  if (m->layout == WG_LAYOUT_ROWGROUP) {
    WG_REQUIRE(m->K > 0 && m->K % 32 == 0,
               "%s: matrix columns (%d) must be a positive multiple of 32", who, m->K);
    WG_REQUIRE(m->scales, "%s: matrix has no scales", who);
    WG_REQUIRE(m->zero == WG_ZERO_8 || m->zero == WG_ZERO_U8 || m->zero == WG_ZERO_F16,
               "%s: unknown zero-point kind %d", who, m->zero);
    WG_REQUIRE(m->zero == WG_ZERO_8 || m->zeros, "%s: matrix has no zero points", who);
  } else if (m->layout == WG_LAYOUT_Q4K) {
    WG_REQUIRE(m->K > 0 && m->K % 256 == 0,
               "%s: Q4_K matrix columns (%d) must be a positive multiple of 256", who, m->K);
  } else if (m->layout == WG_LAYOUT_Q8 || m->layout == WG_LAYOUT_Q6K) {
    const int unit = m->layout == WG_LAYOUT_Q8 ? 32 : 256;
    WG_REQUIRE(m->K > 0 && m->K % unit == 0,
               "%s: %d-bit matrix columns (%d) must be a positive multiple of %d", who,
               m->layout == WG_LAYOUT_Q8 ? 8 : 6, m->K, unit);
    WG_REQUIRE(m->scales, "%s: matrix has no scales", who);
  } else {
    return fail(WG_ERR_UNSUPPORTED, "%s: unknown matrix layout %d", who, m->layout);
  }
  return WG_OK;
}

// Launch-shape knobs (the reference keeps its own in a TUNING table,
// src/engine.ts:147-625): read by the launchers, set through wg_tuning_set.
struct Knob {
  const char *name;
  int value, lo, hi;
};
static Knob g_knobs[] = {
    {"gemv_wg_per_cu", 2, 1, 16},        // persistent row-group GEMV workgroups per CU
    {"gemv_wg_per_cu_wide", 8, 1, 16},   // the same for matrices of 16384+ row groups
    {"q4k_wg_per_cu", 2, 1, 16},         // persistent Q4_K GEMV workgroups per CU
    {"wide_wg_per_cu", 2, 1, 16},        // the same for 8-bit and Q6_K GEMVs
    {"gemv_min_waves", 8192, 0, 1 << 20},  // split K within a workgroup below this
    {"gemv_few_stream", 1, 0, 1},        // 3 to 8 tokens on the streaming kernel (0: row groups)
    {"gemv_few_wg_per_cu", 1, 1, 16},    // its persistent workgroups per CU
    {"decode_wg_per_cu", 1, 1, 4},       // persistent decode workgroups (8 waves) per CU
    {"attn_prefill_mfma", 4, 0, 4},      // prompt attention: MFMA waves a workgroup (1, 2, 4), 0 VALU
    {"gemm_tile", 0, 0, 3},              // prefill GEMM tile: 0 chooses; 1 64x128, 2 128x128, 3 128x256
    {"delta_narrow_rows", 16, 0, 1 << 20},  // Gated DeltaNet batches up to this: 16-column workgroups
};

int tuning(const char *name) {
  for (auto &k : g_knobs)
    if (!strcmp(k.name, name)) return k.value;
  return 0;
}

// Kernels whose dynamic LDS limit was raised, per device (the attribute
// is a property of the kernel on the current device).
int raise_lds(const void *kernel, int bytes) {
  static std::mutex mu;
  static std::unordered_set<std::string> done;
  int dev = 0;
  WG_HIP(hipGetDevice(&dev));
  char key[64];
  snprintf(key, sizeof key, "%p/%d/%d", kernel, dev, bytes);
  std::lock_guard<std::mutex> lock(mu);
  if (done.count(key)) return WG_OK;
  WG_HIP(hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes));
  done.insert(key);
  return WG_OK;
}

int persistent_grid(int work_groups, int per_cu) {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  if (!cus[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cus[dev] = n;
  }
  int cap = cus[dev] * per_cu;
  return work_groups < cap ? work_groups : cap;
}

}  // namespace wg

using namespace wg;

struct wg_buf {
  wg_ctx *ctx;
  void *ptr;
  size_t bytes;
};

struct wg_ctx {
  int device;
  hipStream_t stream;
  std::mutex lock;
  std::unordered_set<wg_buf *> live;
  size_t bytes = 0;
};

struct wg_fence {
  wg_ctx *ctx;
  hipEvent_t done;
  void *host;  // pinned staging
  size_t bytes;
};

extern "C" {

int wg_tuning_set(const char *name, int32_t value) {
  WG_REQUIRE(name, "wg_tuning_set: no name");
  for (auto &k : g_knobs)
    if (!strcmp(k.name, name)) {
      WG_REQUIRE(value >= k.lo && value <= k.hi, "wg_tuning_set: %s = %d is outside [%d, %d]",
                 name, value, k.lo, k.hi);
      k.value = value;
      return WG_OK;
    }
  return fail(WG_ERR_INVALID, "wg_tuning_set: no knob named %s", name);
}

int wg_tuning_get(const char *name, int32_t *value) {
  WG_REQUIRE(name && value, "wg_tuning_get: null argument");
  for (auto &k : g_knobs)
    if (!strcmp(k.name, name)) {
      *value = k.value;
      return WG_OK;
    }
  return fail(WG_ERR_INVALID, "wg_tuning_get: no knob named %s", name);
}

const char *wg_last_error(void) { return g_error; }
const char *wg_version(void) { return "webgllm_hip 0.1 gfx950"; }

int wg_ctx_create(int device, wg_ctx **out) {
  WG_REQUIRE(out, "wg_ctx_create: no output");
  int n = 0;
  WG_HIP(hipGetDeviceCount(&n));
  WG_REQUIRE(device >= 0 && device < n, "wg_ctx_create: device %d of %d", device, n);
  WG_HIP(hipSetDevice(device));
  hipStream_t s;
  WG_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  wg_ctx *c = new wg_ctx();
  c->device = device;
  c->stream = s;
  *out = c;
  return WG_OK;
}

int wg_ctx_destroy(wg_ctx *c) {
  WG_REQUIRE(c, "wg_ctx_destroy: no context");
  WG_HIP(hipSetDevice(c->device));
  WG_HIP(hipStreamSynchronize(c->stream));
  for (wg_buf *b : c->live) {
    (void)hipFree(b->ptr);
    delete b;
  }
  c->live.clear();
  (void)hipStreamDestroy(c->stream);
  delete c;
  return WG_OK;
}

int wg_ctx_limits(wg_ctx *c, wg_limits *out) {
  WG_REQUIRE(c && out, "wg_ctx_limits: null argument");
  hipDeviceProp_t p;
  WG_HIP(hipGetDeviceProperties(&p, c->device));
  out->device = c->device;
  out->compute_units = p.multiProcessorCount;
  out->global_bytes = (int64_t)p.totalGlobalMem;
  out->max_alloc_bytes = (int64_t)p.totalGlobalMem;
  out->lds_bytes_per_block = (int32_t)p.sharedMemPerBlock;
  out->wave_size = p.warpSize;
  return WG_OK;
}

void *wg_ctx_stream(wg_ctx *c) { return c ? (void *)c->stream : nullptr; }

int wg_buf_create(wg_ctx *c, size_t bytes, const void *init, wg_buf **out) {
  WG_REQUIRE(c && out, "wg_buf_create: null argument");
  WG_REQUIRE(bytes > 0, "wg_buf_create: empty buffer");
  WG_HIP(hipSetDevice(c->device));
  void *p = nullptr;
  hipError_t e = hipMalloc(&p, bytes);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return fail(WG_ERR_OOM, "wg_buf_create: %zu bytes: %s", bytes, hipGetErrorString(e));
  }
  if (init) {
    e = hipMemcpyAsync(p, init, bytes, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) {
      (void)hipFree(p);
      return fail(WG_ERR_DEVICE, "wg_buf_create: upload: %s", hipGetErrorString(e));
    }
  }
  wg_buf *b = new wg_buf{c, p, bytes};
  std::lock_guard<std::mutex> g(c->lock);
  c->live.insert(b);
  c->bytes += bytes;
  *out = b;
  return WG_OK;
}

static int owned(wg_ctx *c, wg_buf *b, const char *who) {
  WG_REQUIRE(c && b, "%s: null argument", who);
  std::lock_guard<std::mutex> g(c->lock);
  if (!c->live.count(b)) return fail(WG_ERR_DISPOSED, "%s: buffer was deleted", who);
  return WG_OK;
}

int wg_buf_write(wg_ctx *c, wg_buf *b, size_t offset, const void *src, size_t bytes) {
  int rc = owned(c, b, "wg_buf_write");
  if (rc) return rc;
  WG_REQUIRE(src || !bytes, "wg_buf_write: no data");
  WG_REQUIRE(offset <= b->bytes && bytes <= b->bytes - offset,
             "wg_buf_write: [%zu, %zu) is outside the %zu-byte buffer", offset, offset + bytes,
             b->bytes);
  WG_HIP(hipMemcpyAsync((char *)b->ptr + offset, src, bytes, hipMemcpyHostToDevice, c->stream));
  WG_HIP(hipStreamSynchronize(c->stream));
  return WG_OK;
}

int wg_buf_zero(wg_ctx *c, wg_buf *b) {
  int rc = owned(c, b, "wg_buf_zero");
  if (rc) return rc;
  WG_HIP(hipMemsetAsync(b->ptr, 0, b->bytes, c->stream));
  return WG_OK;
}

int wg_buf_delete(wg_ctx *c, wg_buf *b) {
  int rc = owned(c, b, "wg_buf_delete");
  if (rc) return rc;
  // The stream may still read it.
  WG_HIP(hipStreamSynchronize(c->stream));
  {
    std::lock_guard<std::mutex> g(c->lock);
    c->live.erase(b);
    c->bytes -= b->bytes;
  }
  WG_HIP(hipFree(b->ptr));
  delete b;
  return WG_OK;
}

void *wg_buf_ptr(wg_buf *b) { return b ? b->ptr : nullptr; }
size_t wg_buf_size(wg_buf *b) { return b ? b->bytes : 0; }

size_t wg_bytes_live(wg_ctx *c) {
  if (!c) return 0;
  std::lock_guard<std::mutex> g(c->lock);
  return c->bytes;
}

int wg_read_start(wg_ctx *c, wg_buf *b, size_t offset, size_t bytes, wg_fence **out) {
  int rc = owned(c, b, "wg_read_start");
  if (rc) return rc;
  WG_REQUIRE(out, "wg_read_start: no output");
  WG_REQUIRE(offset <= b->bytes && bytes <= b->bytes - offset && bytes > 0,
             "wg_read_start: [%zu, %zu) is outside the %zu-byte buffer", offset, offset + bytes,
             b->bytes);
  void *host = nullptr;
  WG_HIP(hipHostMalloc(&host, bytes, hipHostMallocDefault));
  hipEvent_t ev;
  hipError_t e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
  if (e == hipSuccess)
    e = hipMemcpyAsync(host, (char *)b->ptr + offset, bytes, hipMemcpyDeviceToHost, c->stream);
  if (e == hipSuccess) e = hipEventRecord(ev, c->stream);
  if (e != hipSuccess) {
    (void)hipHostFree(host);
    return fail(WG_ERR_DEVICE, "wg_read_start: %s", hipGetErrorString(e));
  }
  *out = new wg_fence{c, ev, host, bytes};
  return WG_OK;
}

int wg_fence_ready(wg_fence *f) {
  WG_REQUIRE(f, "wg_fence_ready: no fence");
  hipError_t e = hipEventQuery(f->done);
  if (e == hipSuccess) return 1;
  if (e == hipErrorNotReady) return 0;
  return fail(WG_ERR_DEVICE, "wg_fence_ready: %s", hipGetErrorString(e));
}

static void fence_free(wg_fence *f) {
  (void)hipEventDestroy(f->done);
  (void)hipHostFree(f->host);
  delete f;
}

int wg_read_finish(wg_fence *f, void *dst) {
  WG_REQUIRE(f, "wg_read_finish: no fence");
  hipError_t e = hipEventSynchronize(f->done);
  if (e != hipSuccess) {
    fence_free(f);
    return fail(WG_ERR_DEVICE, "wg_read_finish: %s", hipGetErrorString(e));
  }
  if (dst) memcpy(dst, f->host, f->bytes);
  fence_free(f);
  return WG_OK;
}

int wg_read_cancel(wg_fence *f) {
  WG_REQUIRE(f, "wg_read_cancel: no fence");
  (void)hipEventSynchronize(f->done);
  fence_free(f);
  return WG_OK;
}

int wg_read_now(wg_ctx *c, wg_buf *b, size_t offset, size_t bytes, void *dst) {
  wg_fence *f = nullptr;
  int rc = wg_read_start(c, b, offset, bytes, &f);
  if (rc) return rc;
  return wg_read_finish(f, dst);
}

int wg_flush(wg_ctx *c) {
  WG_REQUIRE(c, "wg_flush: no context");
  return WG_OK;  // HIP submits as it goes; nothing is held back.
}

int wg_finish(wg_ctx *c) {
  WG_REQUIRE(c, "wg_finish: no context");
  WG_HIP(hipStreamSynchronize(c->stream));
  return WG_OK;
}

int wg_q4_sizes(int32_t N, int32_t K, int32_t layout, int32_t zero, size_t *qb, size_t *sb,
                size_t *zb) {
  WG_REQUIRE(N > 0 && N % 4 == 0, "wg_q4_sizes: rows (%d) must be a positive multiple of 4", N);
  size_t q = 0, s = 0, z = 0;
  if (layout == WG_LAYOUT_ROWGROUP) {
    WG_REQUIRE(K > 0 && K % 32 == 0, "wg_q4_sizes: columns (%d) must be a multiple of 32", K);
    size_t blocks = (size_t)N * (K / 32);
    q = blocks * 16;
    s = blocks * 2;
    z = zero == WG_ZERO_U8 ? blocks : zero == WG_ZERO_F16 ? blocks * 2 : 0;
  } else if (layout == WG_LAYOUT_Q4K) {
    WG_REQUIRE(K > 0 && K % 256 == 0, "wg_q4_sizes: Q4_K columns (%d) must be a multiple of 256",
               K);
    q = (size_t)N * (K / 256) * 144;
  } else if (layout == WG_LAYOUT_Q8) {
    WG_REQUIRE(K > 0 && K % 32 == 0, "wg_q4_sizes: 8-bit columns (%d) must be a multiple of 32", K);
    q = (size_t)N * K;
    s = (size_t)N * (K / 32) * 2;
  } else if (layout == WG_LAYOUT_Q6K) {
    WG_REQUIRE(K > 0 && K % 256 == 0, "wg_q4_sizes: Q6_K columns (%d) must be a multiple of 256",
               K);
    q = (size_t)N * (K / 256) * 208;
    s = (size_t)N * (K / 256) * 2;
  } else {
    return fail(WG_ERR_UNSUPPORTED, "wg_q4_sizes: unknown layout %d", layout);
  }
  if (qb) *qb = q;
  if (sb) *sb = s;
  if (zb) *zb = z;
  return WG_OK;
}

}  // extern "C"
