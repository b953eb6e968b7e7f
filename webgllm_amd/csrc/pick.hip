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

namespace wg {
namespace {

constexpr int SPAN = 1024;
constexpr int PER = SPAN / 256;  // logits a thread loads

struct Best {
  float v;
  int id;
};

// The better of two candidates: larger value, ties to the lower id.
__device__ inline Best better(Best a, Best b) {
  if (b.v > a.v || (b.v == a.v && b.id < a.id)) return b;
  return a;
}

__device__ inline Best wave_best(Best b) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    Best o{__shfl_xor(b.v, off, 64), __shfl_xor(b.id, off, 64)};
    b = better(b, o);
  }
  return b;
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
  if (threadIdx.x == 0) {
    // Nothing above -3e38 (or only NaN): the reference's scan keeps id 0.
    if (b.id == 0x7fffffff) b = {-3e38f, 0};
    ids[m] = b.id;
    if (tops) tops[m] = b.v;
    if (pos) {
      const int p = *pos;
      if (hist && p + 1 >= 0 && p + 1 < hist_len) hist[p + 1] = b.id;
      *pos = p + 1;
    }
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

}  // extern "C"
