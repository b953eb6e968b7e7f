// The greedy pick's candidate and its merge (the reference's CHUNK_MAX_AT
// scan, src/gpu/kernels.ts:3169-3205), shared by the pick kernels and the
// head GEMV's epilogue that runs the pick's first stage.
#pragma once

#include "common.h"

namespace wg {

// The pick's parts: a count (the workgroups that wrote, int32 at byte 0),
// then (value, id) per row and workgroup at byte 16 + 8 (m WG_PICK_SLOTS + p).
constexpr int PICK_HEADER = 16;
constexpr float PICK_FLOOR = -3e38f;  // the scan's start: only larger values enter
constexpr int PICK_NONE = 0x7fffffff;

struct PickBest {
  float v;
  int id;
};

// The better of two candidates: larger value, ties to the lower id. (With
// values that entered through a strict > from PICK_FLOOR, never NaN, the
// merge is associative and commutative: any order gives the same pick.)
__device__ inline PickBest pick_better(PickBest a, PickBest b) {
  if (b.v > a.v || (b.v == a.v && b.id < a.id)) return b;
  return a;
}

__device__ inline PickBest pick_xor(PickBest b, int off) {
  return pick_better(b, PickBest{__shfl_xor(b.v, off, 64), __shfl_xor(b.id, off, 64)});
}

__device__ inline PickBest pick_wave_best(PickBest b) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) b = pick_xor(b, off);
  return b;
}

}  // namespace wg
