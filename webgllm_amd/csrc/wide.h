// 8-bit and Q6_K matrices (WG_LAYOUT_Q8, WG_LAYOUT_Q6K): where a row's
// weights sit, and the exact dequant of 32 consecutive weights, shared by
// the dequant and embedding kernels.
#pragma once

#include "common.h"

namespace wg {

// Row n, block b of an 8-bit matrix (src/weights.ts:14-20): the index of
// its half scale; its 32 codes are bytes 32 si .. 32 si + 31.
__host__ __device__ inline int64_t q8_index(int n, int b, int blocks) {
  return ((int64_t)(n >> 2) * blocks + b) * 4 + (n & 3);
}

// Weights 32 b .. 32 b + 31 of row n as matrixRow reads an 8-bit matrix
// (src/repack.ts:873-876): fp32(d * q), exact (an 11-bit significand times
// an 8-bit integer).
__device__ inline void dequant32_q8(const int8_t *quants, const uint16_t *scales, int n, int b,
                                    int blocks, float *out) {
  const int64_t si = q8_index(n, b, blocks);
  const float d = half_to_float(scales[si]);
  const int8_t *q = quants + si * 32;
#pragma unroll 8
  for (int j = 0; j < 32; j++) out[j] = d * (float)q[j];
}

// Row n, super-block s of a Q6_K matrix (src/weights.ts:23-30): the index
// of its record (208 bytes at 208 x) and of its half d.
__host__ __device__ inline int64_t q6k_index(int n, int s, int supers) {
  return ((int64_t)(n >> 2) * supers + s) * 4 + (n & 3);
}

// Weights 256 s + 32 j .. + 31 (j = 0..7) of a Q6_K record, as
// dequantize_row_q6_K (src/repack.ts:405-440): in half h = j / 4, for l =
// 0..31 and group i = j % 4,
//   q = (ql[64 h + l + 32 (i & 1)] >> 4 (i >> 1) & 15) | (qh[32 h + l] >> 2 i & 3) << 4
//   w = fp32(d sc[8 h + l / 16 + 2 i] (q - 32)),
// d sc exact, the product with q - 32 rounded once (in doubles, then to
// float, as the reference's Float32Array store).
__device__ inline void dequant32_q6k(const uint8_t *rec, float d, int j, float *out) {
  const int h = j >> 2, i = j & 3;
  const uint8_t *ql = rec + 64 * h + 32 * (i & 1);
  const uint8_t *qh = rec + 128 + 32 * h;
  const int8_t *sc = reinterpret_cast<const int8_t *>(rec + 192 + 8 * h + 2 * i);
  const int lshift = 4 * (i >> 1), hshift = 2 * i;
  const double ds0 = (double)d * sc[0], ds1 = (double)d * sc[1];
  for (int l = 0; l < 32; l++) {
    const int q = ((ql[l] >> lshift) & 15) | (((qh[l] >> hshift) & 3) << 4);
    out[l] = (float)((l < 16 ? ds0 : ds1) * (double)(q - 32));
  }
}

}  // namespace wg
