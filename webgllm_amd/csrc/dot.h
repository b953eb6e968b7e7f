// Nibble dot products on gfx950 without MFMA: two 4-bit weights become two
// fp16 subnormals (q * 2^-24, or 16 q * 2^-24 for a high nibble) in one
// dword, and v_dot2_f32_f16 multiplies them by two half activations with
// float32 accumulation. Every product is exact; the 2^-24 (and 1/16) is
// taken out again once per block.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace wg {

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

__device__ inline half2v as_h2(uint32_t u) { return __builtin_bit_cast(half2v, u); }

__device__ inline float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(as_h2(a), as_h2(b), c, false);
}

// v_perm_b32 selectors: bytes 0 and 1 of a dword into the low byte of each
// half (the other bytes zero); bytes 2 and 3 likewise.
constexpr uint32_t SEL01 = 0x0c010c00u;
constexpr uint32_t SEL23 = 0x0c030c02u;
constexpr uint32_t LO4 = 0x000f000fu;
constexpr uint32_t HI4 = 0x00f000f0u;
constexpr uint32_t ONES = 0x3c003c00u;  // (1.0h, 1.0h)

// One dword of nibble bytes (weights k..k+3 low, and their partners high)
// as 4 subnormal pairs: lo0 = (q_k, q_k+1), lo1 = (q_k+2, q_k+3) and the
// high nibbles' pairs hi0, hi1 (times 16).
struct NibblePairs {
  uint32_t lo0, lo1, hi0, hi1;
};

__device__ inline NibblePairs split_nibbles(uint32_t w) {
  uint32_t p0 = __builtin_amdgcn_perm(0u, w, SEL01);
  uint32_t p1 = __builtin_amdgcn_perm(0u, w, SEL23);
  return {p0 & LO4, p1 & LO4, p0 & HI4, p1 & HI4};
}

// Sum of 8 halves held as 4 dwords.
__device__ inline float sum8(const uint4 &a, float acc) {
  acc = dot2(a.x, ONES, acc);
  acc = dot2(a.y, ONES, acc);
  acc = dot2(a.z, ONES, acc);
  return dot2(a.w, ONES, acc);
}

__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Wave64 reductions through DPP (no LDS round trip): within quads, half
// rows and rows, then rows into lane 63 by the row broadcasts; the result is
// read back from lane 63, so it is wave-uniform. `id` is the operation's
// identity, taken by lanes a step does not write.
template <int CTRL, int ROW_MASK>
__device__ inline float dpp_f(float x, float id) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, id),
                                                               __builtin_bit_cast(int, x), CTRL,
                                                               ROW_MASK, 0xf, false));
}
template <typename Op>
__device__ inline float wave_reduce_dpp(float v, float id, Op op) {
  v = op(v, dpp_f<0xb1, 0xf>(v, id));   // quad_perm [1, 0, 3, 2]
  v = op(v, dpp_f<0x4e, 0xf>(v, id));   // quad_perm [2, 3, 0, 1]
  v = op(v, dpp_f<0x141, 0xf>(v, id));  // row_half_mirror
  v = op(v, dpp_f<0x140, 0xf>(v, id));  // row_mirror: every lane holds its row's result
  v = op(v, dpp_f<0x142, 0xa>(v, id));  // row_bcast:15 into rows 1 and 3
  v = op(v, dpp_f<0x143, 0xc>(v, id));  // row_bcast:31 into rows 2 and 3
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}
__device__ inline float wave_max_u(float v) {
  return wave_reduce_dpp(v, -INFINITY, [](float a, float b) { return fmaxf(a, b); });
}
__device__ inline float wave_sum_u(float v) {
  return wave_reduce_dpp(v, 0.0f, [](float a, float b) { return a + b; });
}

// Reduce-scatter of 4 per-lane values over the 64 lanes in 7 shuffles:
// afterwards lanes 16 r .. 16 r + 15 all hold the wave's sum of v[r].
__device__ inline float wave_sum4(float v0, float v1, float v2, float v3) {
  const int lane = threadIdx.x & 63;
  const bool hi = lane & 32;
  float s0 = hi ? v0 : v2, s1 = hi ? v1 : v3;
  float k0 = hi ? v2 : v0, k1 = hi ? v3 : v1;
  k0 += __shfl_xor(s0, 32, 64);
  k1 += __shfl_xor(s1, 32, 64);
  const bool hi2 = lane & 16;
  float k = hi2 ? k1 : k0;
  k += __shfl_xor(hi2 ? k0 : k1, 16, 64);
  k += __shfl_xor(k, 8, 64);
  k += __shfl_xor(k, 4, 64);
  k += __shfl_xor(k, 2, 64);
  k += __shfl_xor(k, 1, 64);
  return k;
}

// The row a lane holds after wave_sum4.
__device__ inline int wave_sum4_row() { return (threadIdx.x >> 4) & 3; }

// Workgroups a persistent kernel launches per compute unit.
int persistent_grid(int work_groups, int per_cu);
// Allows `kernel` `bytes` of dynamic LDS on the current device (once a device).
int raise_lds(const void *kernel, int bytes);
// A launch-shape knob's value (see wg_tuning_set).
int tuning(const char *name);

}  // namespace wg
