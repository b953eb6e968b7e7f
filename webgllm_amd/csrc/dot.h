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

// Cross-lane moves without an LDS round trip (a shuffle is a ds_bpermute,
// whose latency a chain of reductions pays at every step): the value of
// lane l ^ 32 (v_permlane32_swap: the wave's halves trade places), of lane
// l ^ 16 (v_permlane16_swap: rows 0 and 1, 2 and 3 trade), and DPP
// rotations within 16-lane rows.
__device__ inline float xor32(float v) {
  const unsigned u = __builtin_bit_cast(unsigned, v);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __builtin_bit_cast(float, (threadIdx.x & 32) ? r[0] : r[1]);
}
__device__ inline float xor16(float v) {
  const unsigned u = __builtin_bit_cast(unsigned, v);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return __builtin_bit_cast(float, (threadIdx.x & 16) ? r[0] : r[1]);
}
// lane (l - N) mod 16 of the same row (row_ror:N)
template <int N>
__device__ inline float row_ror(float v) {
  static_assert(N >= 1 && N < 16, "rotation");
  return __builtin_bit_cast(
      float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x120 + N, 0xf, 0xf, false));
}

// op over the lanes of the wave that share lane % P (P a power of two,
// 1 to 32), on every one of them. Each step combines a lane with the lane
// P 2^k away in the same group (a rotation within 16-lane rows, then the
// row and half swaps); both lanes of a pair combine the same two values,
// so with a commutative op every lane of a group ends with the same bits.
template <int P, typename Op>
__device__ inline float group_reduce(float v, Op op) {
  static_assert(P >= 1 && P <= 32 && (P & (P - 1)) == 0, "group stride");
  if constexpr (P <= 1) v = op(v, row_ror<1>(v));
  if constexpr (P <= 2) v = op(v, row_ror<2>(v));
  if constexpr (P <= 4) v = op(v, row_ror<4>(v));
  if constexpr (P <= 8) v = op(v, row_ror<8>(v));
  if constexpr (P <= 16) v = op(v, xor16(v));
  return op(v, xor32(v));
}
struct Plus {
  __device__ float operator()(float a, float b) const { return a + b; }
};
struct Max {
  __device__ float operator()(float a, float b) const { return fmaxf(a, b); }
};
// The sum over each group of 4 consecutive lanes, on each of them (DPP
// quad permutes [1 0 3 2], then [2 3 0 1]).
__device__ inline float quad_sum(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xb1, 0xf, 0xf, false));
  return v + __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4e, 0xf, 0xf, false));
}
// Reduce-scatter of 8 per-lane values: afterwards lanes 8 t .. 8 t + 7 all
// hold the wave's sum of v[t] (halves, rows and 8-lane halves of rows
// trade the values they keep, then each 8 lanes add up by quad permutes
// and a half-row mirror).
__device__ inline float wave_sum8(const float (&v)[8]) {
  const int lane = threadIdx.x & 63;
  const bool h32 = lane & 32, h16 = lane & 16, h8 = lane & 8;
  float a[4], b[2];
#pragma unroll
  for (int t = 0; t < 4; t++) a[t] = (h32 ? v[t + 4] : v[t]) + xor32(h32 ? v[t] : v[t + 4]);
#pragma unroll
  for (int u = 0; u < 2; u++) b[u] = (h16 ? a[u + 2] : a[u]) + xor16(h16 ? a[u] : a[u + 2]);
  float c = (h8 ? b[1] : b[0]) + row_ror<8>(h8 ? b[0] : b[1]);
  c += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, c), 0xb1, 0xf, 0xf, false));
  c += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, c), 0x4e, 0xf, 0xf, false));
  return c + __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, c), 0x141, 0xf, 0xf, false));
}
// The wave's sum / max on every lane.
__device__ inline float wave_sum(float v) { return group_reduce<1>(v, Plus()); }
__device__ inline float wave_max(float v) { return group_reduce<1>(v, Max()); }

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

// Reduce-scatter of 4 per-lane values over the 64 lanes (two lane swaps,
// then a sum within 16-lane rows): afterwards lanes 16 r .. 16 r + 15 all
// hold the wave's sum of v[r].
__device__ inline float wave_sum4(float v0, float v1, float v2, float v3) {
  const int lane = threadIdx.x & 63;
  const bool hi = lane & 32;
  float s0 = hi ? v0 : v2, s1 = hi ? v1 : v3;
  float k0 = hi ? v2 : v0, k1 = hi ? v3 : v1;
  k0 += xor32(s0);
  k1 += xor32(s1);
  const bool hi2 = lane & 16;
  float k = hi2 ? k1 : k0;
  k += xor16(hi2 ? k0 : k1);
  k += row_ror<8>(k);
  k += row_ror<4>(k);
  k += row_ror<2>(k);
  return k + row_ror<1>(k);
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
