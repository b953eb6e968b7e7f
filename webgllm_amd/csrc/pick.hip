// Greedy pick (the reference's CHUNK_MAX_AT + CHUNK_ARGMAX_ROWS,
// src/gpu/kernels.ts:3169-3246): the lowest token id holding the largest
// logit. Comparisons are strict > starting from -3e38 at id 0, so NaN never
// wins and an all -inf row picks id 0, as the reference's scan does.
// Stage 1: each workgroup reduces 1024 logits of a row to (max, first id),
// every load issued before the first comparison; stage 2: one wave per row
// reduces the workgroups' results in id order. wg_argmax_advance's stage 2
// also moves a decode step on (the token to ids[0] and the history, the
// position up by one) so that a captured step replays at the next position
// without the host, as the reference's guessed forward reads its pick from
// the ids texture (src/engine.ts:8095-8110, :8318-8336).
#include "common.h"
#include "pick_core.h"

namespace wg {
namespace {

constexpr int SPAN = 1024;
constexpr int PER = SPAN / 256;  // logits a thread loads

using Best = PickBest;
__device__ inline Best better(Best a, Best b) { return pick_better(a, b); }
__device__ inline Best wave_best(Best b) { return pick_wave_best(b); }

// A row's pick from its candidates' best: nothing above -3e38 (or only NaN)
// keeps id 0, as the reference's scan does; with `pos` (one row) the
// decode step's advance: ids[0] = the pick, hist[*pos + 1] = the pick when
// *pos + 1 < hist_len, *pos += 1.
__device__ inline void pick_store(Best b, int m, int32_t *ids, float *tops, int32_t *pos,
                                  int32_t *hist, int hist_len) {
  if (b.id == PICK_NONE) b = {PICK_FLOOR, 0};
  ids[m] = b.id;
  if (tops) tops[m] = b.v;
  if (pos) {
    const int p = *pos;
    if (hist && p + 1 >= 0 && p + 1 < hist_len) hist[p + 1] = b.id;
    *pos = p + 1;
  }
}

__global__ __launch_bounds__(256) void argmax_stage1(const float *logits, int V, int ld,
                                                     float *part_v, int *part_id, int parts) {
  __shared__ float sv[4];
  __shared__ int si[4];
  const int m = blockIdx.y, p = blockIdx.x;
  const float *row = logits + (int64_t)m * ld;
  Best b{-3e38f, 0x7fffffff};
  const int i0 = p * SPAN + threadIdx.x;
  float v[PER];
#pragma unroll
  for (int u = 0; u < PER; u++) v[u] = i0 + 256 * u < V ? row[i0 + 256 * u] : -INFINITY;
#pragma unroll
  for (int u = 0; u < PER; u++)  // ids rise within a thread: strict > keeps the first
    if (v[u] > b.v) b = {v[u], i0 + 256 * u};
  b = wave_best(b);
  if ((threadIdx.x & 63) == 0) {
    sv[threadIdx.x >> 6] = b.v;
    si[threadIdx.x >> 6] = b.id;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    Best t{sv[0], si[0]};
    for (int w = 1; w < 4; w++) t = better(t, Best{sv[w], si[w]});
    part_v[m * parts + p] = t.v;
    part_id[m * parts + p] = t.id;
  }
}

// With `pos` (one row): ids[0] = the pick, hist[*pos + 1] = the pick when
// *pos + 1 < hist_len, *pos += 1.
__global__ __launch_bounds__(64) void argmax_stage2(const float *part_v, const int *part_id,
                                                    int parts, int32_t *ids, float *tops,
                                                    int32_t *pos, int32_t *hist, int hist_len) {
  const int m = blockIdx.x;
  Best b{-3e38f, 0x7fffffff};
  for (int p = threadIdx.x; p < parts; p += 64) b = better(b, Best{part_v[m * parts + p],
                                                                   part_id[m * parts + p]});
  b = wave_best(b);
  if (threadIdx.x == 0) pick_store(b, m, ids, tops, pos, hist, hist_len);
}

// The pick from a head GEMV's parts (row m = blockIdx.x): the count of
// workgroups that wrote, then their (value, id) in slots m WG_PICK_SLOTS + p.
// 256 threads a row, each loading its up to 16 parts at once (one memory
// round trip after the count's).
constexpr int PARTS_PER = WG_PICK_SLOTS / 256;
__global__ __launch_bounds__(256) void argmax_parts_kernel(const char *pick_parts, int32_t *ids,
                                                           float *tops, int32_t *pos,
                                                           int32_t *hist, int hist_len) {
  __shared__ Best lds[4];
  const int m = blockIdx.x;
  const int parts = min(*reinterpret_cast<const int *>(pick_parts), WG_PICK_SLOTS);
  const uint2 *row =
      reinterpret_cast<const uint2 *>(pick_parts + PICK_HEADER) + (int64_t)m * WG_PICK_SLOTS;
  uint2 raw[PARTS_PER];
#pragma unroll
  for (int k = 0; k < PARTS_PER; k++) {
    const int p = (int)threadIdx.x + 256 * k;
    raw[k] = p < parts ? row[p] : make_uint2(__float_as_uint(PICK_FLOOR), (uint32_t)PICK_NONE);
  }
  Best b{PICK_FLOOR, PICK_NONE};
#pragma unroll
  for (int k = 0; k < PARTS_PER; k++)
    b = better(b, Best{__uint_as_float(raw[k].x), (int)raw[k].y});
  b = wave_best(b);
  if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = b;
  __syncthreads();
  if (threadIdx.x == 0) {
    Best t = lds[0];
    for (int w = 1; w < 4; w++) t = better(t, lds[w]);
    pick_store(t, m, ids, tops, pos, hist, hist_len);
  }
}

}  // namespace
}  // namespace wg

using namespace wg;

extern "C" {

size_t wg_argmax_scratch_bytes(int32_t M, int32_t V) {
  size_t parts = (size_t)(V + SPAN - 1) / SPAN;
  return (size_t)M * parts * 8;
}

int wg_argmax_rows(const float *logits, int32_t M, int32_t V, int32_t ld, int32_t *ids,
                   float *tops, void *scratch, size_t scratch_bytes, void *stream) {
  WG_REQUIRE(logits && ids && scratch, "wg_argmax_rows: null argument");
  WG_REQUIRE(M >= 1 && V >= 1 && ld >= V, "wg_argmax_rows: %d rows of %d (stride %d)", M, V, ld);
  WG_REQUIRE(scratch_bytes >= wg_argmax_scratch_bytes(M, V),
             "wg_argmax_rows: scratch of %zu bytes, %zu needed", scratch_bytes,
             wg_argmax_scratch_bytes(M, V));
  int parts = (V + SPAN - 1) / SPAN;
  float *pv = (float *)scratch;
  int *pi = (int *)((char *)scratch + (size_t)M * parts * 4);
  hipStream_t s = as_stream(stream);
  argmax_stage1<<<dim3(parts, M), 256, 0, s>>>(logits, V, ld, pv, pi, parts);
  int rc = launched("wg_argmax_rows");
  if (rc) return rc;
  argmax_stage2<<<M, 64, 0, s>>>(pv, pi, parts, ids, tops, nullptr, nullptr, 0);
  return launched("wg_argmax_rows (stage 2)");
}

int wg_argmax_advance(const float *logits, int32_t V, int32_t *ids, int32_t *pos, int32_t *hist,
                      int32_t hist_len, float *tops, void *scratch, size_t scratch_bytes,
                      void *stream) {
  WG_REQUIRE(logits && ids && pos && scratch, "wg_argmax_advance: null argument");
  WG_REQUIRE(V >= 1, "wg_argmax_advance: %d logits", V);
  WG_REQUIRE(hist_len >= 0 && (hist || hist_len == 0),
             "wg_argmax_advance: history of %d entries at %p", hist_len, (void *)hist);
  WG_REQUIRE(scratch_bytes >= wg_argmax_scratch_bytes(1, V),
             "wg_argmax_advance: scratch of %zu bytes, %zu needed", scratch_bytes,
             wg_argmax_scratch_bytes(1, V));
  int parts = (V + SPAN - 1) / SPAN;
  float *pv = (float *)scratch;
  int *pi = (int *)((char *)scratch + (size_t)parts * 4);
  hipStream_t s = as_stream(stream);
  argmax_stage1<<<dim3(parts, 1), 256, 0, s>>>(logits, V, V, pv, pi, parts);
  int rc = launched("wg_argmax_advance");
  if (rc) return rc;
  argmax_stage2<<<1, 64, 0, s>>>(pv, pi, parts, ids, tops, pos, hist, hist_len);
  return launched("wg_argmax_advance (stage 2)");
}

size_t wg_pick_parts_bytes(int32_t M) {
  return M < 1 ? 0 : (size_t)PICK_HEADER + (size_t)M * WG_PICK_SLOTS * sizeof(PickBest);
}

int wg_argmax_parts(const void *pick_parts, int32_t M, int32_t *ids, float *tops, int32_t *pos,
                    int32_t *hist, int32_t hist_len, void *stream) {
  WG_REQUIRE(pick_parts && ids, "wg_argmax_parts: null argument");
  WG_REQUIRE(M >= 1 && M <= 8, "wg_argmax_parts: %d rows (1 to 8)", M);
  WG_REQUIRE(!pos || M == 1, "wg_argmax_parts: the advance takes one row, not %d", M);
  WG_REQUIRE(hist_len >= 0 && (hist || hist_len == 0),
             "wg_argmax_parts: history of %d entries at %p", hist_len, (void *)hist);
  WG_REQUIRE(((uintptr_t)pick_parts & 15) == 0, "wg_argmax_parts: parts not 16-byte aligned");
  argmax_parts_kernel<<<M, 256, 0, as_stream(stream)>>>((const char *)pick_parts, ids, tops, pos,
                                                       hist, hist_len);
  return launched("wg_argmax_parts");
}

}  // extern "C"
