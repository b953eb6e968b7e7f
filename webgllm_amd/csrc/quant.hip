// Load-time repacking of quantized weights on the GPU, and the bit-exact
// dequant (the reference's matrixRow). The reference repacks on the CPU
// while loading (src/repack.ts); here the file's bytes are copied to the
// device once and rearranged there, one thread per row block.
#include "common.h"
#include "wide.h"
#include "kernels.h"

namespace wg {
namespace {

__device__ inline uint32_t ld32_unaligned(const uint8_t *p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}
__device__ inline uint16_t ld16_unaligned(const uint8_t *p) {
  return (uint16_t)(p[0] | (p[1] << 8));
}

// packQ4_0 (src/repack.ts:60-88): thread = (row i, block b).
__global__ void repack_q4_0_kernel(uint32_t *quants, uint16_t *scales, const uint8_t *src,
                                   const int32_t *src_rows, int row0, int rows, int blocks) {
  int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (int64_t)rows * blocks) return;
  int i = (int)(t / blocks), b = (int)(t % blocks);
  int n = row0 + i;
  int s = src_rows ? src_rows[i] : i;
  const uint8_t *p = src + ((int64_t)s * blocks + b) * 18;
  int64_t si = ((int64_t)(n >> 2) * blocks + b) * 4 + (n & 3);
  scales[si] = ld16_unaligned(p);
  uint4 q;
  q.x = ld32_unaligned(p + 2);
  q.y = ld32_unaligned(p + 6);
  q.z = ld32_unaligned(p + 10);
  q.w = ld32_unaligned(p + 14);
  reinterpret_cast<uint4 *>(quants)[si] = q;
}

// packMatMulNBits (src/repack.ts:342-390): output byte j = weight j (low
// nibble of source byte j/2 ... ) re-interleaved to Q4_0 order; thread =
// (row i, block b).
__global__ void repack_nbits_kernel(uint32_t *quants, uint16_t *scales, uint8_t *zeros,
                                    const uint8_t *quant, const uint8_t *scale_bytes,
                                    const uint8_t *zp, const int32_t *src_rows, int row0,
                                    int rows, int blocks) {
  int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (int64_t)rows * blocks) return;
  int i = (int)(t / blocks), b = (int)(t % blocks);
  int n = row0 + i;
  int s = src_rows ? src_rows[i] : i;
  const uint8_t *p = quant + ((int64_t)s * blocks + b) * 16;
  int64_t si = ((int64_t)(n >> 2) * blocks + b) * 4 + (n & 3);
  uint8_t out[16];
#pragma unroll
  for (int k = 0; k < 8; k++) {
    uint8_t lo = p[k], hi = p[8 + k];
    out[2 * k] = (uint8_t)((lo & 0x0f) | ((hi & 0x0f) << 4));
    out[2 * k + 1] = (uint8_t)((lo >> 4) | (hi & 0xf0));
  }
  uint4 q;
  q.x = ld32_unaligned(out);
  q.y = ld32_unaligned(out + 4);
  q.z = ld32_unaligned(out + 8);
  q.w = ld32_unaligned(out + 12);
  reinterpret_cast<uint4 *>(quants)[si] = q;
  scales[si] = ld16_unaligned(scale_bytes + ((int64_t)s * blocks + b) * 2);
  if (zeros) {
    int zp_stride = (blocks + 1) / 2;
    zeros[si] = zp ? (zp[(int64_t)s * zp_stride + (b >> 1)] >> ((b & 1) << 2)) & 15 : 8;
  }
}

// packQ4_K (src/repack.ts:100-168): thread = (row i, super-block s,
// sub-block pair is/2). Same (d', z') chain: d' = half(d * sc); z' =
// half(dmin * m / d') with the quotient in doubles; d' == 0 -> q = 15,
// d' = half(-dmin * m / 15), z' = 0.
__global__ void repack_q4_k_kernel(uint32_t *quants, uint16_t *scales, uint16_t *zero_halves,
                                   const uint8_t *src, const int32_t *src_rows, int row0,
                                   int rows, int supers) {
  int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (int64_t)rows * supers * 4) return;
  int pair = (int)(t & 3);
  int64_t rs = t >> 2;
  int i = (int)(rs / supers), s = (int)(rs % supers);
  int n = row0 + i;
  int sr = src_rows ? src_rows[i] : i;
  int blocks = supers * 8;
  const uint8_t *p = src + ((int64_t)sr * supers + s) * 144;
  double d = half_to_float(ld16_unaligned(p));
  double dmin = half_to_float(ld16_unaligned(p + 2));
  int is = 2 * pair;
  int64_t si = ((int64_t)(n >> 2) * blocks + s * 8 + is) * 4 + (n & 3);
  const uint8_t *at = p + 16 + is * 16;
  const uint32_t LOW = 0x0f0f0f0fu;
  uint4 q0, q1;
  uint32_t lo[4], hi[4];
#pragma unroll
  for (int w = 0; w < 4; w++) {
    uint32_t a = ld32_unaligned(at + 4 * w), b = ld32_unaligned(at + 16 + 4 * w);
    lo[w] = (a & LOW) | ((b & LOW) << 4);
    hi[w] = ((a >> 4) & LOW) | (b & ~LOW);
  }
  q0 = make_uint4(lo[0], lo[1], lo[2], lo[3]);
  q1 = make_uint4(hi[0], hi[1], hi[2], hi[3]);
  uint4 *qv = reinterpret_cast<uint4 *>(quants);
  for (int j = 0; j < 2; j++) {
    int sc, mn;
    q4k_scale_min(p + 4, is + j, &sc, &mn);
    double scale = d * sc, mins = dmin * mn;
    int64_t a2 = si + 4 * j;
    uint16_t h = double_to_half_ref(scale);
    float hv = half_to_float(h);
    if (hv != 0.0f) {
      scales[a2] = h;
      zero_halves[a2] = double_to_half_ref(mins / (double)hv);
      qv[a2] = j ? q1 : q0;
    } else {
      scales[a2] = double_to_half_ref(-mins / 15.0);
      zero_halves[a2] = 0;
      qv[a2] = make_uint4(0xffffffffu, 0xffffffffu, 0xffffffffu, 0xffffffffu);
    }
  }
}

// packQ4_K's quants with Q4_K's own scales kept (WG_ZERO_Q4K): thread =
// (row group gi of the range, super-block s). The group's 4 rows' nibbles go
// out as repack_q4_k_kernel writes them (15s for a constant block), and its
// record gets the rows' d and dmin and the 8 blocks' 6-bit scales and mins.
__global__ void repack_q4_k_rec_kernel(uint32_t *quants, uint8_t *recs, const uint8_t *src,
                                       const int32_t *src_rows, int row0, int rows, int supers) {
  int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (int64_t)(rows / 4) * supers) return;
  const int gi = (int)(t / supers), s = (int)(t % supers);
  const int g = row0 / 4 + gi, blocks = supers * 8;
  uint8_t rec[Q4K_REC];
  for (int k = 0; k < Q4K_REC; k++) rec[k] = 0;
  uint4 *qv = reinterpret_cast<uint4 *>(quants);
  const uint32_t LOW = 0x0f0f0f0fu;
  for (int r = 0; r < 4; r++) {
    const int i = 4 * gi + r;
    const int sr = src_rows ? src_rows[i] : i;
    const uint8_t *p = src + ((int64_t)sr * supers + s) * 144;
    for (int k = 0; k < 4; k++) rec[4 * r + k] = p[k];
    const double d = half_to_float(ld16_unaligned(p));
    const double dmin = half_to_float(ld16_unaligned(p + 2));
    for (int pair = 0; pair < 4; pair++) {
      const uint8_t *at = p + 16 + pair * 32;
      uint32_t lo[4], hi[4];
      for (int w = 0; w < 4; w++) {
        uint32_t a = ld32_unaligned(at + 4 * w), b = ld32_unaligned(at + 16 + 4 * w);
        lo[w] = (a & LOW) | ((b & LOW) << 4);
        hi[w] = ((a >> 4) & LOW) | (b & ~LOW);
      }
      for (int j2 = 0; j2 < 2; j2++) {
        const int j = 2 * pair + j2;
        int sc, mn;
        q4k_scale_min(p + 4, j, &sc, &mn);
        q4k_rec_put(rec, j, r, sc, mn);
        uint16_t dq, zq;
        const bool constant = q4k_block_dz(d, dmin, sc, mn, &dq, &zq);
        const uint32_t *w = j2 ? hi : lo;
        qv[((int64_t)g * blocks + s * 8 + j) * 4 + r] =
            constant ? make_uint4(0xffffffffu, 0xffffffffu, 0xffffffffu, 0xffffffffu)
                     : make_uint4(w[0], w[1], w[2], w[3]);
      }
    }
  }
  uint4 *o = reinterpret_cast<uint4 *>(recs + ((int64_t)g * supers + s) * Q4K_REC);
  for (int k = 0; k < Q4K_REC / 16; k++) {
    uint32_t v[4];
    for (int w = 0; w < 4; w++) v[w] = ld32_unaligned(rec + 16 * k + 4 * w);
    o[k] = make_uint4(v[0], v[1], v[2], v[3]);
  }
}

// WG_ZERO_Q4K records -> packQ4_K's per-block (d', z') halves at the
// WG_ZERO_F16 indices (the prefill GEMM's operands): thread = (row n, block b).
__global__ void q4k_rec_expand_kernel(const uint8_t *recs, uint16_t *scales, uint16_t *zeros,
                                      int N, int blocks) {
  int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (int64_t)N * blocks) return;
  const int n = (int)(t / blocks), b = (int)(t % blocks);
  const uint8_t *rec = recs + ((int64_t)(n >> 2) * (blocks / 8) + b / 8) * Q4K_REC;
  uint16_t dq, zq;
  q4k_rec_dz(rec, b & 7, n & 3, &dq, &zq);
  const int64_t si = ((int64_t)(n >> 2) * blocks + b) * 4 + (n & 3);
  scales[si] = dq;
  zeros[si] = zq;
}

// Q4_K super-blocks regrouped by rows of 4 (record (g * supers + s) * 4 + r):
// thread = one 16-byte piece of one record.
__global__ void repack_q4_k_native_kernel(uint8_t *dst, const uint8_t *src,
                                          const int32_t *src_rows, int row0, int rows,
                                          int supers) {
  int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (int64_t)rows * supers * 9) return;
  int piece = (int)(t % 9);
  int64_t rs = t / 9;
  int i = (int)(rs / supers), s = (int)(rs % supers);
  int n = row0 + i;
  int sr = src_rows ? src_rows[i] : i;
  const uint8_t *p = src + ((int64_t)sr * supers + s) * 144 + piece * 16;
  uint8_t *o = dst + (((int64_t)(n >> 2) * supers + s) * 4 + (n & 3)) * 144 + piece * 16;
#pragma unroll
  for (int k = 0; k < 16; k++) o[k] = p[k];
}

// matrixRow (src/repack.ts:865-891), ROWGROUP: thread = (row, block): 32
// weights fp32(d * (q - z)) with the product and difference in doubles, as
// the reference computes them.
__global__ void dequant_rowgroup_kernel(const uint32_t *quants, const uint16_t *scales,
                                        const void *zeros, int zero_kind, int row0, int rows,
                                        int blocks, float *out) {
  int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (int64_t)rows * blocks) return;
  int i = (int)(t / blocks), b = (int)(t % blocks);
  int n = row0 + i;
  int64_t si = ((int64_t)(n >> 2) * blocks + b) * 4 + (n & 3);
  double d, z;
  if (zero_kind == WG_ZERO_Q4K) {  // packQ4_K's halves rebuilt from the record
    uint16_t dq, zq;
    q4k_rec_dz((const uint8_t *)scales + ((int64_t)(n >> 2) * (blocks / 8) + b / 8) * Q4K_REC,
               b & 7, n & 3, &dq, &zq);
    d = half_to_float(dq);
    z = half_to_float(zq);
  } else {
    d = half_to_float(scales[si]);
    z = zero_kind == WG_ZERO_U8    ? (double)((const uint8_t *)zeros)[si]
        : zero_kind == WG_ZERO_F16 ? (double)half_to_float(((const uint16_t *)zeros)[si])
                                   : 8.0;
  }
  uint4 q = reinterpret_cast<const uint4 *>(quants)[si];
  uint32_t w[4] = {q.x, q.y, q.z, q.w};
  float *o = out + (int64_t)i * blocks * 32 + b * 32;
#pragma unroll
  for (int j = 0; j < 16; j++) {
    uint32_t byte = (w[j >> 2] >> (8 * (j & 3))) & 0xffu;
    o[j] = (float)(d * ((double)(byte & 15u) - z));
    o[j + 16] = (float)(d * ((double)(byte >> 4) - z));
  }
}

// The same for WG_LAYOUT_Q4K: thread = (row, super-block, sub-block);
// (d', z') rebuilt with packQ4_K's chain, weights in the file's order.
__global__ void dequant_q4k_kernel(const uint8_t *quants, int row0, int rows, int supers,
                                   float *out) {
  int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (int64_t)rows * supers * 8) return;
  int j = (int)(t & 7);
  int64_t rs = t >> 3;
  int i = (int)(rs / supers), s = (int)(rs % supers);
  int n = row0 + i;
  const uint8_t *p = quants + (((int64_t)(n >> 2) * supers + s) * 4 + (n & 3)) * 144;
  double d = half_to_float(ld16_unaligned(p));
  double dmin = half_to_float(ld16_unaligned(p + 2));
  int sc, mn;
  q4k_scale_min(p + 4, j, &sc, &mn);
  uint16_t h = double_to_half_ref(d * sc);
  double mins = dmin * mn;
  double scale, zero;
  bool constant = half_to_float(h) == 0.0f;
  if (!constant) {
    scale = half_to_float(h);
    zero = half_to_float(double_to_half_ref(mins / scale));
  } else {
    scale = half_to_float(double_to_half_ref(-mins / 15.0));
    zero = 0.0;
  }
  const uint8_t *q = p + 16 + (j >> 1) * 32;
  float *o = out + (int64_t)i * supers * 256 + s * 256 + j * 32;
  for (int l = 0; l < 32; l++) {
    int nib = constant ? 15 : (j & 1) ? q[l] >> 4 : q[l] & 15;
    o[l] = (float)(scale * ((double)nib - zero));
  }
}

// packQ8_0 (src/repack.ts:174-200): thread = (row i, block b); the 34-byte
// block's half scale and 32 codes as they are.
__global__ void repack_q8_0_kernel(uint8_t *quants, uint16_t *scales, const uint8_t *src,
                                   const int32_t *src_rows, int row0, int rows, int blocks) {
  int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (int64_t)rows * blocks) return;
  int i = (int)(t / blocks), b = (int)(t % blocks);
  int n = row0 + i;
  int s = src_rows ? src_rows[i] : i;
  const uint8_t *p = src + ((int64_t)s * blocks + b) * 34;
  int64_t si = q8_index(n, b, blocks);
  scales[si] = ld16_unaligned(p);
  uint4 *q = reinterpret_cast<uint4 *>(quants + si * 32);
  q[0] = make_uint4(ld32_unaligned(p + 2), ld32_unaligned(p + 6), ld32_unaligned(p + 10),
                    ld32_unaligned(p + 14));
  q[1] = make_uint4(ld32_unaligned(p + 18), ld32_unaligned(p + 22), ld32_unaligned(p + 26),
                    ld32_unaligned(p + 30));
}

// quantizeQ8 (src/repack.ts:634-704): thread = (row i, block b). max is
// the largest |v| (NaN if any v is, as Math.max); scale = toHalf(max / 127);
// a block whose scale is not > 0 (zero or NaN) gets q = 0; otherwise q =
// ToInt32(v / scale + 128.5) - 128 clamped to +-127, the quotient and sum
// in doubles (ToInt32 truncates toward zero and maps NaN and infinities to
// 0; |v / scale| stays below 2^9, so it never wraps).
__global__ void quantize_q8_kernel(uint8_t *quants, uint16_t *scales, const float *src, int K,
                                   int row0, int rows, int blocks) {
  int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (int64_t)rows * blocks) return;
  int i = (int)(t / blocks), b = (int)(t % blocks);
  int n = row0 + i;
  const float *v = src + (int64_t)i * K + b * 32;
  float mx = 0.0f;
  for (int j = 0; j < 32; j++) {
    float a = fabsf(v[j]);
    if (a > mx || a != a) mx = a;
    if (mx != mx) break;
  }
  int64_t si = q8_index(n, b, blocks);
  uint16_t h = double_to_half_ref((double)mx / 127.0);
  double scale = half_to_float(h);
  scales[si] = h;
  int8_t *q = reinterpret_cast<int8_t *>(quants + si * 32);
  if (!(scale > 0.0)) {
    for (int j = 0; j < 32; j++) q[j] = 0;
    return;
  }
  for (int j = 0; j < 32; j++) {
    double x = (double)v[j] / scale + 128.5;
    int iv = (x == x && x > -2147483648.0 && x < 2147483648.0) ? (int)x : 0;  // trunc
    iv -= 128;
    q[j] = (int8_t)(iv > 127 ? 127 : iv < -127 ? -127 : iv);
  }
}

// packQ6_K (src/repack.ts:706-728): thread = (row i, super-block s, 16-byte
// piece p of the 208 kept bytes); piece 0 also moves the half d.
__global__ void repack_q6_k_kernel(uint8_t *quants, uint16_t *scales, const uint8_t *src,
                                   const int32_t *src_rows, int row0, int rows, int supers) {
  int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (int64_t)rows * supers * 13) return;
  int piece = (int)(t % 13);
  int64_t rs = t / 13;
  int i = (int)(rs / supers), s = (int)(rs % supers);
  int n = row0 + i;
  int sr = src_rows ? src_rows[i] : i;
  const uint8_t *p = src + ((int64_t)sr * supers + s) * 210;
  int64_t at = q6k_index(n, s, supers);
  const uint8_t *from = p + piece * 16;
  reinterpret_cast<uint4 *>(quants + at * 208)[piece] =
      make_uint4(ld32_unaligned(from), ld32_unaligned(from + 4), ld32_unaligned(from + 8),
                 ld32_unaligned(from + 12));
  if (piece == 0) scales[at] = ld16_unaligned(p + 208);
}

// matrixRow of an 8-bit matrix: thread = (row, block).
__global__ void dequant_q8_kernel(const int8_t *quants, const uint16_t *scales, int row0, int rows,
                                  int blocks, float *out) {
  int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (int64_t)rows * blocks) return;
  int i = (int)(t / blocks), b = (int)(t % blocks);
  dequant32_q8(quants, scales, row0 + i, b, blocks, out + (int64_t)i * blocks * 32 + b * 32);
}

// A Q6_K matrix's rows as dequantizeQ6_K: thread = (row, super-block, 32-piece).
__global__ void dequant_q6k_kernel(const uint8_t *quants, const uint16_t *scales, int row0,
                                   int rows, int supers, float *out) {
  int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (int64_t)rows * supers * 8) return;
  int j = (int)(t & 7);
  int64_t rs = t >> 3;
  int i = (int)(rs / supers), s = (int)(rs % supers);
  int64_t at = q6k_index(row0 + i, s, supers);
  dequant32_q6k(quants + at * 208, half_to_float(scales[at]), j,
                out + (int64_t)i * supers * 256 + s * 256 + j * 32);
}

// rowsToFloats (src/load-gguf.ts:557-580): thread = one 32-weight piece of
// one row (`pieces` a row). Each format as the reference's dequantizer
// computes it: the arithmetic in doubles, each weight rounded once to float.
constexpr int GGML_F32 = 0, GGML_F16 = 1, GGML_Q4_1 = 3, GGML_Q8_0 = 8, GGML_Q4_K = 12,
              GGML_Q5_K = 13, GGML_Q6_K = 14;

__global__ void rows_to_floats_kernel(int type, const uint8_t *src, int64_t pieces_total,
                                      float *out) {
  int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= pieces_total) return;
  float *o = out + t * 32;
  if (type == GGML_F32) {  // thread = one value
    out[t] = __builtin_bit_cast(float, ld32_unaligned(src + t * 4));
  } else if (type == GGML_F16) {
    out[t] = half_to_float(ld16_unaligned(src + t * 2));
  } else if (type == GGML_Q8_0) {  // dequantizeQ8_0 (src/repack.ts:514-528)
    const uint8_t *p = src + t * 34;
    double d = half_to_float(ld16_unaligned(p));
    for (int j = 0; j < 32; j++) o[j] = (float)(d * (int8_t)p[2 + j]);
  } else if (type == GGML_Q4_1) {  // dequantizeQ4_1 (src/repack.ts:447-466)
    const uint8_t *p = src + t * 20;
    double d = half_to_float(ld16_unaligned(p)), m = half_to_float(ld16_unaligned(p + 2));
    for (int j = 0; j < 16; j++) {
      o[j] = (float)((p[4 + j] & 15) * d + m);
      o[j + 16] = (float)((p[4 + j] >> 4) * d + m);
    }
  } else if (type == GGML_Q4_K || type == GGML_Q5_K) {
    // dequantizeQ4_K / dequantizeQ5_K (src/repack.ts:474-511, :535-572):
    // sub-block j = 2 is + hi of a super-block, d * sc * q - dmin * m.
    const int64_t s = t >> 3;
    const int j = (int)(t & 7);
    const bool five = type == GGML_Q5_K;
    const uint8_t *p = src + s * (five ? 176 : 144);
    double d = half_to_float(ld16_unaligned(p)), dmin = half_to_float(ld16_unaligned(p + 2));
    int sc, mn;
    q4k_scale_min(p + 4, j, &sc, &mn);
    const double d1 = d * sc, min1 = dmin * mn;
    const uint8_t *q = p + (five ? 48 : 16) + (j >> 1) * 32;
    const int shift = (j & 1) * 4;
    for (int l = 0; l < 32; l++) {
      int v = (q[l] >> shift) & 15;
      if (five && (p[16 + l] & (1 << j))) v += 16;
      o[l] = (float)(d1 * v - min1);
    }
  } else {  // GGML_Q6_K (src/repack.ts:405-440)
    const int64_t s = t >> 3;
    const uint8_t *p = src + s * 210;
    dequant32_q6k(p, half_to_float(ld16_unaligned(p + 208)), (int)(t & 7), o);
  }
}

inline unsigned grid_for(int64_t threads, int per) { return (unsigned)((threads + per - 1) / per); }

}  // namespace

int launch_q4k_expand(const wg_q4_matrix *w, uint16_t *scales, uint16_t *zeros, hipStream_t s) {
  const int blocks = w->K / 32;
  q4k_rec_expand_kernel<<<grid_for((int64_t)w->N * blocks, 256), 256, 0, s>>>(
      (const uint8_t *)w->scales, scales, zeros, w->N, blocks);
  return launched("Q4_K record expansion");
}

}  // namespace wg

using namespace wg;

extern "C" {

static int check_rows(const wg_q4_matrix *m, int row0, int rows, const char *who) {
  WG_REQUIRE(row0 >= 0 && rows >= 0 && row0 + rows <= m->N,
             "%s: rows %d..%d are outside the matrix", who, row0, row0 + rows);
  return WG_OK;
}

int wg_repack_q4_0(const wg_q4_matrix *m, int32_t row0, int32_t rows, const void *src,
                   const int32_t *src_rows, void *stream) {
  int rc = check_matrix(m, "wg_repack_q4_0");
  if (rc) return rc;
  if ((rc = check_rows(m, row0, rows, "wg_repack_q4_0"))) return rc;
  WG_REQUIRE(m->layout == WG_LAYOUT_ROWGROUP && m->zero == WG_ZERO_8,
             "wg_repack_q4_0: Q4_0 rows go into a row-group matrix without zero points");
  WG_REQUIRE(src, "wg_repack_q4_0: no source");
  if (!rows) return WG_OK;
  int blocks = m->K / 32;
  int64_t n = (int64_t)rows * blocks;
  repack_q4_0_kernel<<<grid_for(n, 256), 256, 0, as_stream(stream)>>>(
      (uint32_t *)m->quants, (uint16_t *)m->scales, (const uint8_t *)src, src_rows, row0, rows,
      blocks);
  return launched("wg_repack_q4_0");
}

int wg_repack_nbits(const wg_q4_matrix *m, int32_t row0, int32_t rows, const void *quant,
                    const void *scales, const void *zp, const int32_t *src_rows, void *stream) {
  int rc = check_matrix(m, "wg_repack_nbits");
  if (rc) return rc;
  if ((rc = check_rows(m, row0, rows, "wg_repack_nbits"))) return rc;
  WG_REQUIRE(m->layout == WG_LAYOUT_ROWGROUP && m->zero != WG_ZERO_F16,
             "wg_repack_nbits: MatMulNBits rows go into a row-group matrix with u8 or no zeros");
  WG_REQUIRE(!zp || m->zero == WG_ZERO_U8,
             "wg_repack_nbits: zero points given for a matrix without them");
  WG_REQUIRE(quant && scales, "wg_repack_nbits: no source");
  if (!rows) return WG_OK;
  int blocks = m->K / 32;
  int64_t n = (int64_t)rows * blocks;
  repack_nbits_kernel<<<grid_for(n, 256), 256, 0, as_stream(stream)>>>(
      (uint32_t *)m->quants, (uint16_t *)m->scales,
      m->zero == WG_ZERO_U8 ? (uint8_t *)m->zeros : nullptr, (const uint8_t *)quant,
      (const uint8_t *)scales, (const uint8_t *)zp, src_rows, row0, rows, blocks);
  return launched("wg_repack_nbits");
}

int wg_repack_q4_k(const wg_q4_matrix *m, int32_t row0, int32_t rows, const void *src,
                   const int32_t *src_rows, void *stream) {
  int rc = check_matrix(m, "wg_repack_q4_k");
  if (rc) return rc;
  if ((rc = check_rows(m, row0, rows, "wg_repack_q4_k"))) return rc;
  WG_REQUIRE(m->layout == WG_LAYOUT_ROWGROUP && (m->zero == WG_ZERO_F16 || m->zero == WG_ZERO_Q4K),
             "wg_repack_q4_k: Q4_K rows go into a row-group matrix with half zero points or "
             "Q4_K records");
  WG_REQUIRE(m->K % 256 == 0, "wg_repack_q4_k: columns (%d) must be a multiple of 256", m->K);
  WG_REQUIRE(src, "wg_repack_q4_k: no source");
  if (!rows) return WG_OK;
  int supers = m->K / 256;
  if (m->zero == WG_ZERO_Q4K) {
    WG_REQUIRE(row0 % 4 == 0 && rows % 4 == 0,
               "wg_repack_q4_k: rows must start and end on a row group");
    const int64_t n = (int64_t)(rows / 4) * supers;
    repack_q4_k_rec_kernel<<<grid_for(n, 64), 64, 0, as_stream(stream)>>>(
        (uint32_t *)m->quants, (uint8_t *)m->scales, (const uint8_t *)src, src_rows, row0, rows,
        supers);
    return launched("wg_repack_q4_k");
  }
  int64_t n = (int64_t)rows * supers * 4;
  repack_q4_k_kernel<<<grid_for(n, 256), 256, 0, as_stream(stream)>>>(
      (uint32_t *)m->quants, (uint16_t *)m->scales, (uint16_t *)m->zeros, (const uint8_t *)src,
      src_rows, row0, rows, supers);
  return launched("wg_repack_q4_k");
}

int wg_q4k_record_halves(const wg_q4_matrix *m, uint16_t *scales, uint16_t *zeros,
                         void *stream) {
  int rc = check_matrix(m, "wg_q4k_record_halves");
  if (rc) return rc;
  WG_REQUIRE(m->layout == WG_LAYOUT_ROWGROUP && m->zero == WG_ZERO_Q4K,
             "wg_q4k_record_halves: the matrix holds no Q4_K records");
  WG_REQUIRE(scales && zeros, "wg_q4k_record_halves: null output");
  // (bytes: N K / 32 halves each; the records are N K / 16 bytes too)
  const size_t n = (size_t)m->N * (m->K / 32) * 2;
  WG_REQUIRE(!overlaps(scales, n, zeros, n) && !overlaps(scales, n, m->scales, n) &&
                 !overlaps(zeros, n, m->scales, n),
             "wg_q4k_record_halves: outputs overlap each other or the records");
  return launch_q4k_expand(m, scales, zeros, as_stream(stream));
}

int wg_repack_q4_k_native(const wg_q4_matrix *m, int32_t row0, int32_t rows, const void *src,
                          const int32_t *src_rows, void *stream) {
  int rc = check_matrix(m, "wg_repack_q4_k_native");
  if (rc) return rc;
  if ((rc = check_rows(m, row0, rows, "wg_repack_q4_k_native"))) return rc;
  WG_REQUIRE(m->layout == WG_LAYOUT_Q4K, "wg_repack_q4_k_native: destination is not Q4_K");
  WG_REQUIRE(row0 % 4 == 0 && rows % 4 == 0,
             "wg_repack_q4_k_native: rows must start and end on a row group");
  WG_REQUIRE(src, "wg_repack_q4_k_native: no source");
  if (!rows) return WG_OK;
  int supers = m->K / 256;
  int64_t n = (int64_t)rows * supers * 9;
  repack_q4_k_native_kernel<<<grid_for(n, 256), 256, 0, as_stream(stream)>>>(
      (uint8_t *)m->quants, (const uint8_t *)src, src_rows, row0, rows, supers);
  return launched("wg_repack_q4_k_native");
}

int wg_repack_q8_0(const wg_q4_matrix *m, int32_t row0, int32_t rows, const void *src,
                   const int32_t *src_rows, void *stream) {
  int rc = check_matrix(m, "wg_repack_q8_0");
  if (rc) return rc;
  if ((rc = check_rows(m, row0, rows, "wg_repack_q8_0"))) return rc;
  WG_REQUIRE(m->layout == WG_LAYOUT_Q8, "wg_repack_q8_0: Q8_0 rows go into an 8-bit matrix");
  WG_REQUIRE(src, "wg_repack_q8_0: no source");
  if (!rows) return WG_OK;
  int blocks = m->K / 32;
  repack_q8_0_kernel<<<grid_for((int64_t)rows * blocks, 256), 256, 0, as_stream(stream)>>>(
      (uint8_t *)m->quants, (uint16_t *)m->scales, (const uint8_t *)src, src_rows, row0, rows,
      blocks);
  return launched("wg_repack_q8_0");
}

int wg_quantize_q8(const wg_q4_matrix *m, int32_t row0, int32_t rows, const float *src,
                   void *stream) {
  int rc = check_matrix(m, "wg_quantize_q8");
  if (rc) return rc;
  if ((rc = check_rows(m, row0, rows, "wg_quantize_q8"))) return rc;
  WG_REQUIRE(m->layout == WG_LAYOUT_Q8, "wg_quantize_q8: the destination is not an 8-bit matrix");
  WG_REQUIRE(src, "wg_quantize_q8: no source");
  if (!rows) return WG_OK;
  int blocks = m->K / 32;
  quantize_q8_kernel<<<grid_for((int64_t)rows * blocks, 256), 256, 0, as_stream(stream)>>>(
      (uint8_t *)m->quants, (uint16_t *)m->scales, src, m->K, row0, rows, blocks);
  return launched("wg_quantize_q8");
}

int wg_repack_q6_k(const wg_q4_matrix *m, int32_t row0, int32_t rows, const void *src,
                   const int32_t *src_rows, void *stream) {
  int rc = check_matrix(m, "wg_repack_q6_k");
  if (rc) return rc;
  if ((rc = check_rows(m, row0, rows, "wg_repack_q6_k"))) return rc;
  WG_REQUIRE(m->layout == WG_LAYOUT_Q6K, "wg_repack_q6_k: Q6_K rows go into a Q6_K matrix");
  WG_REQUIRE(src, "wg_repack_q6_k: no source");
  if (!rows) return WG_OK;
  int supers = m->K / 256;
  repack_q6_k_kernel<<<grid_for((int64_t)rows * supers * 13, 256), 256, 0, as_stream(stream)>>>(
      (uint8_t *)m->quants, (uint16_t *)m->scales, (const uint8_t *)src, src_rows, row0, rows,
      supers);
  return launched("wg_repack_q6_k");
}

int wg_rows_to_floats(int32_t type, const void *src, int32_t rows, int32_t K, float *out,
                      void *stream) {
  WG_REQUIRE(src && out && rows >= 0 && K > 0, "wg_rows_to_floats: bad arguments");
  int unit;
  switch (type) {
    case GGML_F32: case GGML_F16: unit = 1; break;
    case GGML_Q4_1: case GGML_Q8_0: unit = 32; break;
    case GGML_Q4_K: case GGML_Q5_K: case GGML_Q6_K: unit = 256; break;
    default:
      return fail(WG_ERR_UNSUPPORTED,
                  "wg_rows_to_floats: ggml type %d (F32, F16, Q4_1, Q4_K, Q5_K, Q6_K and Q8_0 "
                  "convert)", type);
  }
  WG_REQUIRE(K % unit == 0, "wg_rows_to_floats: a row of %d weights is not whole blocks of %d",
             K, unit);
  if (!rows) return WG_OK;
  // a thread per value (F32, F16) or per 32-weight piece
  const int64_t total = (int64_t)rows * (unit == 1 ? K : K / 32);
  rows_to_floats_kernel<<<grid_for(total, 256), 256, 0, as_stream(stream)>>>(
      type, (const uint8_t *)src, total, out);
  return launched("wg_rows_to_floats");
}

int wg_q4_dequant(const wg_q4_matrix *m, int32_t row0, int32_t rows, float *out, void *stream) {
  int rc = check_matrix(m, "wg_q4_dequant");
  if (rc) return rc;
  if ((rc = check_rows(m, row0, rows, "wg_q4_dequant"))) return rc;
  WG_REQUIRE(out, "wg_q4_dequant: no output");
  if (!rows) return WG_OK;
  if (m->layout == WG_LAYOUT_ROWGROUP) {
    int blocks = m->K / 32;
    int64_t n = (int64_t)rows * blocks;
    dequant_rowgroup_kernel<<<grid_for(n, 256), 256, 0, as_stream(stream)>>>(
        (const uint32_t *)m->quants, (const uint16_t *)m->scales, m->zeros, m->zero, row0, rows,
        blocks, out);
  } else if (m->layout == WG_LAYOUT_Q8) {
    int blocks = m->K / 32;
    dequant_q8_kernel<<<grid_for((int64_t)rows * blocks, 256), 256, 0, as_stream(stream)>>>(
        (const int8_t *)m->quants, (const uint16_t *)m->scales, row0, rows, blocks, out);
  } else if (m->layout == WG_LAYOUT_Q6K) {
    int supers = m->K / 256;
    dequant_q6k_kernel<<<grid_for((int64_t)rows * supers * 8, 256), 256, 0, as_stream(stream)>>>(
        (const uint8_t *)m->quants, (const uint16_t *)m->scales, row0, rows, supers, out);
  } else {
    int supers = m->K / 256;
    int64_t n = (int64_t)rows * supers * 8;
    dequant_q4k_kernel<<<grid_for(n, 256), 256, 0, as_stream(stream)>>>(
        (const uint8_t *)m->quants, row0, rows, supers, out);
  }
  return launched("wg_q4_dequant");
}

}  // extern "C"
