// Greedy pick (the reference's CHUNK_MAX_AT + CHUNK_ARGMAX_ROWS,
// src/gpu/kernels.ts:3169-3246): the lowest token id holding the largest
// logit. Comparisons are strict > starting from -3e38 at id 0, so NaN never
// wins and an all -inf row picks id 0, as the reference's scan does.
// Stage 1: each workgroup reduces 4096 logits of a row to (max, first id);
// stage 2: one wave per row reduces the workgroups' results in id order.
#include "common.h"

namespace wg {
namespace {

constexpr int SPAN = 4096;

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
  int i0 = p * SPAN;
  int i1 = min(V, i0 + SPAN);
  for (int i = i0 + threadIdx.x; i < i1; i += 256) {
    float v = row[i];
    if (v > b.v) b = {v, i};  // ids rise within a thread: strict > keeps the first
  }
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

__global__ __launch_bounds__(64) void argmax_stage2(const float *part_v, const int *part_id,
                                                    int parts, int32_t *ids, float *tops) {
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
  argmax_stage2<<<M, 64, 0, s>>>(pv, pi, parts, ids, tops);
  return launched("wg_argmax_rows (stage 2)");
}

}  // extern "C"
