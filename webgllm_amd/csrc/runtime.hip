// The backend object (reference: class Gpu, src/gpu/gl.ts:47, and the
// PacedGpu contract, src/gpu/paced.ts:11-22), on HIP: a context owns a
// device and one stream, buffers stand in for textures, readbacks complete
// behind events.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <mutex>
#include <string>
#include <unordered_set>
#include <utility>
#include <vector>

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
    WG_REQUIRE(m->zero == WG_ZERO_8 || m->zero == WG_ZERO_U8 || m->zero == WG_ZERO_F16 ||
                   m->zero == WG_ZERO_Q4K,
               "%s: unknown zero-point kind %d", who, m->zero);
    WG_REQUIRE(m->zero == WG_ZERO_8 || m->zero == WG_ZERO_Q4K || m->zeros,
               "%s: matrix has no zero points", who);
    WG_REQUIRE(m->zero != WG_ZERO_Q4K || m->K % 256 == 0,
               "%s: Q4_K row-group columns (%d) must be a multiple of 256", who, m->K);
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
  std::atomic<int> value;
  int lo, hi;
};
static Knob g_knobs[] = {
    {"gemv_wg_per_cu", 2, 1, 16},        // persistent row-group GEMV workgroups per CU
    {"gemv_wg_per_cu_small", 1, 1, 16},  // the same for matrices of 1024 row groups or fewer
    {"gemv_wg_per_cu_deep", 3, 1, 16},   // the same for 4096 to 16383 row groups
    {"gemv_wg_per_cu_wide", 8, 1, 16},   // the same for matrices of 16384+ row groups
    {"q4k_wg_per_cu", 3, 1, 16},         // persistent Q4_K GEMV workgroups per CU
    {"q4k_rows", 1, 0, 1},               // Q4_K GEMV: every lane on a row group's 4 rows (0: 2 rows)
    {"wide_wg_per_cu", 2, 1, 16},        // the same for 8-bit and Q6_K GEMVs
    {"gemv_min_waves", 8192, 0, 1 << 20},  // split K within a workgroup below this
    {"gemv_few_stream", 1, 0, 1},        // 3 to 8 tokens on the streaming kernel (0: row groups)
    {"gemv_few_wg_per_cu", 1, 1, 16},    // its persistent workgroups per CU
    {"gemv_mfma", 1, 0, 2},              // row-group GEMV on MFMA: 1 for 3 to 8 tokens, 2 also 1 and 2, 0 never
    {"gemv_mfma_wg_per_cu", 0, 0, 16},   // its persistent workgroups per CU (0: by shape)
    {"gemv_mfma_pairs", 4, 2, 8},        // its block pairs a wave (2, 4, 8)
    {"attn_prefill_mfma", 4, 0, 4},      // prompt attention: MFMA waves a workgroup (1, 2, 4), 0 VALU
    {"attn_mfma", 1, 0, 2},              // decode attention in one launch on MFMA: 1 where it is faster (past 8 queries a KV head, from 16384 keys, outside the XCD-grouped split form's range with KV heads a multiple of 8, else up to 2048 keys), 2 always, 0 never
    {"attn_fused", 1, 0, 2},             // decode attention in one launch: 1 where it is faster, 2 always, 0 never
    {"attn_xcd", 1, 0, 2},               // decode attention with each XCD combining its own KV heads (a multiple of 8): 1 the split form up to 4 queries a KV head below 4096 keys and the MFMA form grouped, 2 the split form always, 0 never
    {"attn_split_chunks", 0, 0, 4},      // its 64-key chunks a workgroup (1, 2, 4; 0 chooses)
    {"attn_split_waves", 1, 0, 1},       // its chunks spread over up to 16 waves (1), or a wave a query (0)
    {"gemm_tile", 0, 0, 3},              // prefill GEMM tile: 0 chooses; 1 64x128, 2 128x128, 3 128x256
    {"gemm_pingpong", 0, 0, 1},          // 128 x 256 tiles: 1 two wave groups half a step apart, 0 in lock-step
    {"gemm_splits", 0, 0, 8},            // prefill GEMM K splits (1, 2, 4, 8): 0 chooses
    {"delta_narrow_rows", 16, 0, 1 << 20},  // Gated DeltaNet batches up to this: 16-column workgroups
};

int tuning(const char *name) {
  for (auto &k : g_knobs)
    if (!strcmp(k.name, name)) return k.value.load(std::memory_order_relaxed);
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

// ------------------------------------------------------------ backend objects
//
// Pinned host staging: each context keeps a pool of page-locked slots, each
// with its own event. A write copies the caller's bytes into a slot and
// queues the upload from it (the caller's buffer is free at once, as after
// gl.texSubImage2D, and nothing waits); a read queues the download into a
// slot that its fence holds until finished or cancelled. A slot whose copy
// may still be in flight is reused only after its event has completed.
namespace {

enum SlotState { SLOT_FREE, SLOT_INFLIGHT, SLOT_FENCED };

struct Slot {
  void *host = nullptr;
  size_t cap = 0;
  hipEvent_t done = nullptr;
  SlotState state = SLOT_FREE;
};

constexpr size_t SLOT_MIN = 64 << 10;  // smallest slot: 64 KiB
constexpr int INFLIGHT_MAX = 16;       // uploads in flight before a write waits for the oldest

// Live handles, so that a call on a deleted buffer, a finished fence or a
// destroyed context reports WG_ERR_DISPOSED instead of touching freed memory.
struct Registry {
  std::mutex mu;
  std::unordered_set<const void *> live;
};
Registry &registry() {
  static Registry *r = new Registry();  // never destroyed: handles may outlive static teardown
  return *r;
}
void reg_add(const void *h) {
  std::lock_guard<std::mutex> g(registry().mu);
  registry().live.insert(h);
}
void reg_del(const void *h) {
  std::lock_guard<std::mutex> g(registry().mu);
  registry().live.erase(h);
}
bool reg_has(const void *h) {
  std::lock_guard<std::mutex> g(registry().mu);
  return h && registry().live.count(h);
}

}  // namespace

// Zeroes `bytes` bytes at p (256-byte aligned): 16 bytes a lane, the tail
// by the first lanes.
__global__ void zero_bytes_kernel(uint8_t *p, size_t bytes) {
  const size_t n16 = bytes / 16;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n16;
       i += (size_t)gridDim.x * blockDim.x)
    reinterpret_cast<uint4 *>(p)[i] = make_uint4(0, 0, 0, 0);
  const size_t tail = n16 * 16 + blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (blockIdx.x == 0 && tail < bytes) p[tail] = 0;
}

struct wg_buf {
  wg_ctx *ctx;
  void *ptr;
  size_t bytes;
};

// A fence: a read's (its staging slot's event) or a plain one (its own
// event, no slot, no bytes).
struct wg_fence {
  wg_ctx *ctx;
  Slot *slot;
  size_t bytes;
  hipEvent_t ev;
};

struct wg_ctx {
  int device;
  hipStream_t stream;
  std::mutex lock;
  std::unordered_set<wg_buf *> live;
  std::unordered_set<wg_fence *> fences;
  std::vector<Slot *> pool;
  // deleted buffers' memory, freed once the work queued before the delete is done
  std::vector<std::pair<void *, hipEvent_t>> graveyard;
  size_t bytes = 0;
};

namespace {

// Frees the graveyard entries whose events have completed (all with `wait`).
// Caller holds c->lock.
void reap(wg_ctx *c, bool wait) {
  auto &gy = c->graveyard;
  for (size_t k = 0; k < gy.size();) {
    hipError_t e = wait ? hipEventSynchronize(gy[k].second) : hipEventQuery(gy[k].second);
    if (e == hipErrorNotReady) {
      k++;
      continue;
    }
    (void)hipFree(gy[k].first);
    (void)hipEventDestroy(gy[k].second);
    gy[k] = gy.back();
    gy.pop_back();
  }
}

// A slot of at least `bytes` for the caller (marked `state`). Caller holds c->lock.
int take_slot(wg_ctx *c, size_t bytes, SlotState state, Slot **out, const char *who) {
  Slot *best = nullptr;
  int inflight = 0;
  for (Slot *s : c->pool) {
    if (s->state == SLOT_INFLIGHT) {
      if (hipEventQuery(s->done) == hipErrorNotReady) {
        inflight++;
        continue;
      }
      s->state = SLOT_FREE;
    }
    if (s->state != SLOT_FREE) continue;
    if (s->cap >= bytes && (!best || best->cap < bytes || s->cap < best->cap)) best = s;
    else if (!best) best = s;  // a free slot to grow if none is large enough
  }
  if (!best && inflight >= INFLIGHT_MAX) {  // bounded pool: wait for an upload to land
    for (Slot *s : c->pool)
      if (s->state == SLOT_INFLIGHT) {
        WG_HIP(hipEventSynchronize(s->done));
        s->state = SLOT_FREE;
        best = s;
        break;
      }
  }
  if (!best) {
    best = new Slot();
    hipError_t e = hipEventCreateWithFlags(&best->done, hipEventDisableTiming);
    if (e != hipSuccess) {
      delete best;
      return fail(WG_ERR_DEVICE, "%s: event: %s", who, hipGetErrorString(e));
    }
    c->pool.push_back(best);
  }
  if (best->cap < bytes) {
    size_t cap = bytes > SLOT_MIN ? bytes : SLOT_MIN;
    void *h = nullptr;
    hipError_t e = hipHostMalloc(&h, cap, hipHostMallocDefault);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      return fail(WG_ERR_OOM, "%s: %zu bytes of pinned staging: %s", who, cap,
                  hipGetErrorString(e));
    }
    if (best->host) (void)hipHostFree(best->host);
    best->host = h;
    best->cap = cap;
  }
  best->state = state;
  *out = best;
  return WG_OK;
}

// The context and buffer are live and the buffer belongs to the context.
int owned(wg_ctx *c, wg_buf *b, const char *who) {
  WG_REQUIRE(c && b, "%s: null argument", who);
  if (!reg_has(c)) return fail(WG_ERR_DISPOSED, "%s: the context was destroyed", who);
  if (!reg_has(b)) return fail(WG_ERR_DISPOSED, "%s: buffer was deleted", who);
  WG_REQUIRE(b->ctx == c, "%s: the buffer belongs to another context", who);
  return WG_OK;
}

hipEvent_t fence_event(const wg_fence *f) { return f->slot ? f->slot->done : f->ev; }

void fence_release(wg_fence *f, bool copied) {
  // a fence's copy that was never waited for may still be landing: its slot
  // is reused only after its event
  if (f->slot) f->slot->state = copied ? SLOT_FREE : SLOT_INFLIGHT;
  if (f->ev) (void)hipEventDestroy(f->ev);
  f->ctx->fences.erase(f);
  reg_del(f);
  delete f;
}

}  // namespace

extern "C" {

int wg_tuning_set(const char *name, int32_t value) {
  WG_REQUIRE(name, "wg_tuning_set: no name");
  for (auto &k : g_knobs)
    if (!strcmp(k.name, name)) {
      WG_REQUIRE(value >= k.lo && value <= k.hi, "wg_tuning_set: %s = %d is outside [%d, %d]",
                 name, value, k.lo, k.hi);
      k.value.store(value, std::memory_order_relaxed);
      return WG_OK;
    }
  return fail(WG_ERR_INVALID, "wg_tuning_set: no knob named %s", name);
}

int wg_tuning_get(const char *name, int32_t *value) {
  WG_REQUIRE(name && value, "wg_tuning_get: null argument");
  for (auto &k : g_knobs)
    if (!strcmp(k.name, name)) {
      *value = k.value.load(std::memory_order_relaxed);
      return WG_OK;
    }
  return fail(WG_ERR_INVALID, "wg_tuning_get: no knob named %s", name);
}

const char *wg_last_error(void) { return g_error; }
const char *wg_version(void) { return "webgllm_hip 0.2 gfx950"; }

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
  reg_add(c);
  *out = c;
  return WG_OK;
}

int wg_ctx_destroy(wg_ctx *c) {
  WG_REQUIRE(c, "wg_ctx_destroy: no context");
  if (!reg_has(c)) return fail(WG_ERR_DISPOSED, "wg_ctx_destroy: the context was destroyed");
  reg_del(c);
  WG_HIP(hipSetDevice(c->device));
  hipError_t sync = hipStreamSynchronize(c->stream);
  {
    std::lock_guard<std::mutex> g(c->lock);
    // outstanding reads are cancelled: their handles report WG_ERR_DISPOSED
    for (wg_fence *f : c->fences) {
      reg_del(f);
      if (f->ev) (void)hipEventDestroy(f->ev);
      delete f;
    }
    c->fences.clear();
    for (wg_buf *b : c->live) {
      reg_del(b);
      (void)hipFree(b->ptr);
      delete b;
    }
    c->live.clear();
    reap(c, true);
    for (Slot *s : c->pool) {
      (void)hipEventDestroy(s->done);
      if (s->host) (void)hipHostFree(s->host);
      delete s;
    }
    c->pool.clear();
  }
  (void)hipStreamDestroy(c->stream);
  delete c;
  if (sync != hipSuccess)
    return fail(WG_ERR_DEVICE, "wg_ctx_destroy: %s", hipGetErrorString(sync));
  return WG_OK;
}

int wg_ctx_limits(wg_ctx *c, wg_limits *out) {
  WG_REQUIRE(c && out, "wg_ctx_limits: null argument");
  if (!reg_has(c)) return fail(WG_ERR_DISPOSED, "wg_ctx_limits: the context was destroyed");
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

void *wg_ctx_stream(wg_ctx *c) { return reg_has(c) ? (void *)c->stream : nullptr; }

int wg_buf_create(wg_ctx *c, size_t bytes, const void *init, wg_buf **out) {
  WG_REQUIRE(c && out, "wg_buf_create: null argument");
  if (!reg_has(c)) return fail(WG_ERR_DISPOSED, "wg_buf_create: the context was destroyed");
  WG_REQUIRE(bytes > 0, "wg_buf_create: empty buffer");
  WG_HIP(hipSetDevice(c->device));
  {
    std::lock_guard<std::mutex> g(c->lock);
    reap(c, false);
  }
  void *p = nullptr;
  hipError_t e = hipMalloc(&p, bytes);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return fail(WG_ERR_OOM, "wg_buf_create: %zu bytes: %s", bytes, hipGetErrorString(e));
  }
  wg_buf *b = new wg_buf{c, p, bytes};
  {
    std::lock_guard<std::mutex> g(c->lock);
    c->live.insert(b);
    c->bytes += bytes;
  }
  reg_add(b);
  if (init) {
    int rc = wg_buf_write(c, b, 0, init, bytes);
    if (rc) {
      char msg[512];
      snprintf(msg, sizeof msg, "%s", wg_last_error());
      (void)wg_buf_delete(c, b);
      return fail(rc, "wg_buf_create: %s", msg);
    }
  }
  *out = b;
  return WG_OK;
}

int wg_buf_write(wg_ctx *c, wg_buf *b, size_t offset, const void *src, size_t bytes) {
  int rc = owned(c, b, "wg_buf_write");
  if (rc) return rc;
  WG_REQUIRE(src || !bytes, "wg_buf_write: no data");
  WG_REQUIRE(offset <= b->bytes && bytes <= b->bytes - offset,
             "wg_buf_write: [%zu, %zu) is outside the %zu-byte buffer", offset, offset + bytes,
             b->bytes);
  if (!bytes) return WG_OK;
  WG_HIP(hipSetDevice(c->device));
  std::lock_guard<std::mutex> g(c->lock);
  Slot *s = nullptr;
  rc = take_slot(c, bytes, SLOT_INFLIGHT, &s, "wg_buf_write");
  if (rc) return rc;
  memcpy(s->host, src, bytes);
  hipError_t e =
      hipMemcpyAsync((char *)b->ptr + offset, s->host, bytes, hipMemcpyHostToDevice, c->stream);
  if (e == hipSuccess) e = hipEventRecord(s->done, c->stream);
  if (e != hipSuccess) {
    // the copy may or may not have been queued: wait for the stream before the slot is reused
    (void)hipStreamSynchronize(c->stream);
    s->state = SLOT_FREE;
    return fail(WG_ERR_DEVICE, "wg_buf_write: %s", hipGetErrorString(e));
  }
  return WG_OK;
}

int wg_buf_zero(wg_ctx *c, wg_buf *b) {
  int rc = owned(c, b, "wg_buf_zero");
  if (rc) return rc;
  WG_HIP(hipSetDevice(c->device));
  // a kernel, not a memset node: a caller may capture the context's stream
  const size_t n16 = b->bytes / 16;
  const size_t blocks = (n16 + 255) / 256;
  zero_bytes_kernel<<<(unsigned)(blocks < 1024 ? (blocks ? blocks : 1) : 1024), 256, 0,
                      c->stream>>>((uint8_t *)b->ptr, b->bytes);
  return launched("wg_buf_zero");
}

int wg_buf_delete(wg_ctx *c, wg_buf *b) {
  int rc = owned(c, b, "wg_buf_delete");
  if (rc) return rc;
  WG_HIP(hipSetDevice(c->device));
  reg_del(b);
  std::lock_guard<std::mutex> g(c->lock);
  c->live.erase(b);
  c->bytes -= b->bytes;
  // the stream may still read it: freed once the work queued so far is done
  hipEvent_t ev = nullptr;
  hipError_t e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
  if (e == hipSuccess) e = hipEventRecord(ev, c->stream);
  if (e == hipSuccess) {
    c->graveyard.emplace_back(b->ptr, ev);
  } else {
    if (ev) (void)hipEventDestroy(ev);
    (void)hipStreamSynchronize(c->stream);
    (void)hipFree(b->ptr);
  }
  delete b;
  reap(c, false);
  return WG_OK;
}

void *wg_buf_ptr(wg_buf *b) { return reg_has(b) ? b->ptr : nullptr; }
size_t wg_buf_size(wg_buf *b) { return reg_has(b) ? b->bytes : 0; }

size_t wg_bytes_live(wg_ctx *c) {
  if (!reg_has(c)) return 0;
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
  WG_HIP(hipSetDevice(c->device));
  std::lock_guard<std::mutex> g(c->lock);
  Slot *s = nullptr;
  rc = take_slot(c, bytes, SLOT_FENCED, &s, "wg_read_start");
  if (rc) return rc;
  hipError_t e =
      hipMemcpyAsync(s->host, (char *)b->ptr + offset, bytes, hipMemcpyDeviceToHost, c->stream);
  if (e == hipSuccess) e = hipEventRecord(s->done, c->stream);
  if (e != hipSuccess) {
    (void)hipStreamSynchronize(c->stream);
    s->state = SLOT_FREE;
    return fail(WG_ERR_DEVICE, "wg_read_start: %s", hipGetErrorString(e));
  }
  wg_fence *f = new wg_fence{c, s, bytes, nullptr};
  c->fences.insert(f);
  reg_add(f);
  *out = f;
  return WG_OK;
}

int wg_fence_record(wg_ctx *c, wg_fence **out) {
  WG_REQUIRE(c && out, "wg_fence_record: null argument");
  if (!reg_has(c)) return fail(WG_ERR_DISPOSED, "wg_fence_record: the context was destroyed");
  WG_HIP(hipSetDevice(c->device));
  hipEvent_t ev = nullptr;
  hipError_t e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
  if (e == hipSuccess) e = hipEventRecord(ev, c->stream);
  if (e != hipSuccess) {
    if (ev) (void)hipEventDestroy(ev);
    return fail(WG_ERR_DEVICE, "wg_fence_record: %s", hipGetErrorString(e));
  }
  wg_fence *f = new wg_fence{c, nullptr, 0, ev};
  {
    std::lock_guard<std::mutex> g(c->lock);
    c->fences.insert(f);
  }
  reg_add(f);
  *out = f;
  return WG_OK;
}

size_t wg_fence_bytes(wg_fence *f) { return reg_has(f) ? f->bytes : 0; }

int wg_fence_ready(wg_fence *f) {
  WG_REQUIRE(f, "wg_fence_ready: no fence");
  if (!reg_has(f)) return fail(WG_ERR_DISPOSED, "wg_fence_ready: the read was finished or cancelled");
  hipError_t e = hipEventQuery(fence_event(f));
  if (e == hipSuccess) return 1;
  if (e == hipErrorNotReady) return 0;
  return fail(WG_ERR_DEVICE, "wg_fence_ready: %s", hipGetErrorString(e));
}

int wg_read_finish(wg_fence *f, void *dst) {
  WG_REQUIRE(f, "wg_read_finish: no fence");
  if (!reg_has(f))
    return fail(WG_ERR_DISPOSED, "wg_read_finish: the read was finished or cancelled");
  wg_ctx *c = f->ctx;
  hipError_t e = hipEventSynchronize(fence_event(f));
  std::lock_guard<std::mutex> g(c->lock);
  if (e == hipSuccess && dst && f->slot) memcpy(dst, f->slot->host, f->bytes);
  fence_release(f, e == hipSuccess);
  if (e != hipSuccess) return fail(WG_ERR_DEVICE, "wg_read_finish: %s", hipGetErrorString(e));
  return WG_OK;
}

int wg_read_cancel(wg_fence *f) {
  WG_REQUIRE(f, "wg_read_cancel: no fence");
  if (!reg_has(f))
    return fail(WG_ERR_DISPOSED, "wg_read_cancel: the read was finished or cancelled");
  std::lock_guard<std::mutex> g(f->ctx->lock);
  fence_release(f, false);  // no wait: the slot is reused after its copy lands
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
  if (!reg_has(c)) return fail(WG_ERR_DISPOSED, "wg_flush: the context was destroyed");
  return WG_OK;  // HIP submits as it goes; nothing is held back.
}

int wg_finish(wg_ctx *c) {
  WG_REQUIRE(c, "wg_finish: no context");
  if (!reg_has(c)) return fail(WG_ERR_DISPOSED, "wg_finish: the context was destroyed");
  WG_HIP(hipSetDevice(c->device));
  WG_HIP(hipStreamSynchronize(c->stream));
  std::lock_guard<std::mutex> g(c->lock);
  reap(c, false);
  return WG_OK;
}

int wg_ctx_staging(wg_ctx *c, int32_t *slots, size_t *bytes) {
  WG_REQUIRE(c, "wg_ctx_staging: no context");
  if (!reg_has(c)) return fail(WG_ERR_DISPOSED, "wg_ctx_staging: the context was destroyed");
  std::lock_guard<std::mutex> g(c->lock);
  size_t total = 0;
  for (Slot *s : c->pool) total += s->cap;
  if (slots) *slots = (int32_t)c->pool.size();
  if (bytes) *bytes = total;
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
    if (zero == WG_ZERO_Q4K) {
      WG_REQUIRE(K % 256 == 0, "wg_q4_sizes: Q4_K row-group columns (%d) must be a multiple of 256",
                 K);
      s = (size_t)N * (K / 256) * 16;  // a 64-byte record a row group and super-block
    }
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
