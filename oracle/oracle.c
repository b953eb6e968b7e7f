/*
 * CPU oracle for webgllm's Q4 decode/prefill hot path (test infrastructure;
 * see oracle.h). Paths cited are relative to packages/webgllm/ of the
 * reference.
 */
#define _POSIX_C_SOURCE 199309L
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ fp16 */

/* src/half.ts:7-32. The value is first stored as a float32 (round to
 * nearest), then rounded to nearest-even half; subnormals, overflow to
 * infinity, NaN to a quiet NaN with the sign kept. */
uint16_t orc_to_half(double value) {
  float f = (float)value;
  uint32_t x;
  memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  int exp = (int)((x >> 23) & 0xffu);
  uint32_t mant = x & 0x7fffffu;
  if (exp == 0xff) return (uint16_t)(sign | 0x7c00u | (mant ? 0x200u : 0u));
  int e = exp - 127 + 15;
  if (e >= 31) return (uint16_t)(sign | 0x7c00u);
  if (e <= 0) {
    if (e < -10) return (uint16_t)sign;
    mant |= 0x800000u;
    int shift = 14 - e;
    uint32_t half = 1u << (shift - 1);
    uint32_t rest = mant & ((1u << shift) - 1u);
    uint32_t h = mant >> shift;
    if (rest > half || (rest == half && (h & 1u))) h++;
    return (uint16_t)(sign | h);
  }
  uint32_t h = ((uint32_t)e << 10) | (mant >> 13);
  uint32_t rest = mant & 0x1fffu;
  if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h++;
  return (uint16_t)(sign | h);
}

/* src/half.ts:37-55: every half's value. */
float orc_from_half(uint16_t h) {
  int sign = (h & 0x8000u) ? -1 : 1;
  int exp = (h >> 10) & 0x1f;
  int mant = h & 0x3ff;
  if (exp == 0) return (float)(sign * (double)mant * ldexp(1.0, -24));
  if (exp == 31) return mant ? NAN : (sign > 0 ? INFINITY : -INFINITY);
  return (float)(sign * (1.0 + mant / 1024.0) * ldexp(1.0, exp - 15));
}

static float half_table[65536];
static int half_table_ready = 0;
static const float *htab(void) {
  if (!half_table_ready) {
    for (int h = 0; h < 65536; h++) half_table[h] = orc_from_half((uint16_t)h);
    half_table_ready = 1;
  }
  return half_table;
}

static inline uint32_t rd32(const uint8_t *p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}
static inline uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* ------------------------------------------------------------ packers */

/* src/repack.ts:60-88: GGUF Q4_0 blocks (fp16 d, 16 nibble bytes) copied as
 * words into the row-group layout; src_rows picks each row's source row. */
int orc_pack_q4_0(orc_qm *m, int row0, const uint8_t *src, size_t src_len, int rows,
                  const int32_t *src_rows) {
  int blocks = m->K / 32;
  if (row0 < 0 || row0 + rows > m->N) return -1;
  if (src_len < (size_t)rows * blocks * 18) return -2;
  for (int i = 0; i < rows; i++) {
    int n = row0 + i;
    size_t p = (size_t)(src_rows ? src_rows[i] : i) * blocks * 18;
    size_t si = orc_si(m->N, blocks, n, 0);
    for (int b = 0; b < blocks; b++, p += 18, si += 4) {
      m->scales[si] = rd16(src + p);
      for (int w = 0; w < 4; w++) m->quants[si * 4 + w] = rd32(src + p + 2 + 4 * w);
    }
  }
  return 0;
}

/* get_scale_min_k4 as src/repack.ts:127-140 decodes it: sub-blocks is and
 * is + 1 of a super-block's 12 scale bytes. */
static void scale_min_pair(const uint8_t *sc, int is, int *s1, int *m1, int *s2, int *m2) {
  if (is < 4) {
    *s1 = sc[is] & 63;
    *m1 = sc[is + 4] & 63;
    *s2 = sc[is + 1] & 63;
    *m2 = sc[is + 5] & 63;
  } else {
    *s1 = (sc[is + 4] & 15) | ((sc[is - 4] >> 6) << 4);
    *m1 = (sc[is + 4] >> 4) | ((sc[is] >> 6) << 4);
    *s2 = (sc[is + 5] & 15) | ((sc[is - 3] >> 6) << 4);
    *m2 = (sc[is + 5] >> 4) | ((sc[is + 1] >> 6) << 4);
  }
}

/* src/repack.ts:100-168: Q4_K super-blocks (144 B) into 4-bit blocks of 32
 * with fractional zero points. Sub-block scale d' = half(d * sc) and zero
 * z' = half(dmin * m / d') (the quotient in doubles, stored through a
 * float32 by toHalf); a sub-block whose d' is 0 becomes q = 15 everywhere,
 * d' = half(-dmin * m / 15), z' = 0. Nibbles re-interleaved to Q4_0 order. */
int orc_pack_q4_k(orc_qm *m, int row0, const uint8_t *src, size_t src_len, int rows,
                  const int32_t *src_rows) {
  if (!m->zero_halves) return -3;
  if (row0 < 0 || row0 + rows > m->N) return -1;
  const float *half = htab();
  int blocks = m->K / 32, supers = m->K / 256;
  if (src_len < (size_t)rows * supers * 144) return -2;
  const uint32_t LOW = 0x0f0f0f0fu;
  for (int i = 0; i < rows; i++) {
    int n = row0 + i;
    size_t p = (size_t)(src_rows ? src_rows[i] : i) * supers * 144;
    size_t si = orc_si(m->N, blocks, n, 0);
    for (int s = 0; s < supers; s++, p += 144) {
      double d = half[rd16(src + p)];
      double dmin = half[rd16(src + p + 2)];
      const uint8_t *sc = src + p + 4;
      for (int is = 0; is < 8; is += 2, si += 8) {
        int s1, m1, s2, m2;
        scale_min_pair(sc, is, &s1, &m1, &s2, &m2);
        const uint8_t *at = src + p + 16 + is * 16;
        size_t qi = si * 4;
        for (int w = 0; w < 4; w++) {
          uint32_t a = rd32(at + 4 * w), b = rd32(at + 16 + 4 * w);
          m->quants[qi + w] = (a & LOW) | ((b & LOW) << 4);
          m->quants[qi + 16 + w] = ((a >> 4) & LOW) | (b & ~LOW);
        }
        for (int j = 0; j < 2; j++) {
          double scale = d * (j ? s2 : s1);
          double mn = dmin * (j ? m2 : m1);
          size_t a2 = si + 4 * j;
          uint16_t h = orc_to_half(scale);
          if (half[h] != 0.0f) {
            m->scales[a2] = h;
            m->zero_halves[a2] = orc_to_half(mn / (double)half[h]);
          } else {
            for (int w = 0; w < 4; w++) m->quants[a2 * 4 + w] = 0xffffffffu;
            m->scales[a2] = orc_to_half(-mn / 15.0);
            m->zero_halves[a2] = 0;
          }
        }
      }
    }
  }
  return 0;
}

/* src/repack.ts:342-390: MatMulNBits rows (element 2i in byte i's low
 * nibble) into Q4_0 nibble order: output byte j holds weight j low and
 * weight j + 16 high; scales as given, zero points two blocks a byte. */
int orc_pack_nbits(orc_qm *m, int row0, const uint8_t *quant, const uint8_t *scale_bytes,
                   const uint8_t *zp, int rows, const int32_t *src_rows) {
  int blocks = m->K / 32, zp_stride = (blocks + 1) / 2;
  if (row0 < 0 || row0 + rows > m->N) return -1;
  if (zp && !m->zeros) return -4;
  uint8_t *q = (uint8_t *)m->quants;
  for (int i = 0; i < rows; i++) {
    int n = row0 + i;
    int s = src_rows ? src_rows[i] : i;
    size_t p = (size_t)s * blocks * 16, sp = (size_t)s * blocks * 2, zr = (size_t)s * zp_stride;
    size_t si = orc_si(m->N, blocks, n, 0);
    for (int b = 0; b < blocks; b++, p += 16, sp += 2, si += 4) {
      size_t qi = si * 16;
      for (int k = 0; k < 8; k++) {
        uint8_t lo = quant[p + k], hi = quant[p + 8 + k];
        q[qi + 2 * k] = (uint8_t)((lo & 0x0f) | ((hi & 0x0f) << 4));
        q[qi + 2 * k + 1] = (uint8_t)((lo >> 4) | (hi & 0xf0));
      }
      m->scales[si] = rd16(scale_bytes + sp);
      if (zp && m->zeros) m->zeros[si] = (zp[zr + (b >> 1)] >> ((b & 1) << 2)) & 15;
    }
  }
  return 0;
}

/* src/repack.ts:312-337: the scales and zero points only (raw quants). */
int orc_pack_nbits_scales(orc_qm *m, int row0, const uint8_t *scale_bytes, const uint8_t *zp,
                          int rows) {
  int blocks = m->K / 32, zp_stride = (blocks + 1) / 2;
  if (row0 < 0 || row0 + rows > m->N) return -1;
  for (int i = 0; i < rows; i++) {
    int n = row0 + i;
    size_t sp = (size_t)i * blocks * 2, zr = (size_t)i * zp_stride;
    size_t si = orc_si(m->N, blocks, n, 0);
    for (int b = 0; b < blocks; b++, sp += 2, si += 4) {
      m->scales[si] = rd16(scale_bytes + sp);
      if (zp && m->zeros) m->zeros[si] = (zp[zr + (b >> 1)] >> ((b & 1) << 2)) & 15;
    }
  }
  return 0;
}

/* src/repack.ts:216-245: the same nibble rearrangement as orc_pack_nbits,
 * on 32-bit words (its own restatement, so each pins the other). */
void orc_quants_from_raw(const uint8_t *raw, int N, int K, uint32_t *quants) {
  int blocks = K / 32;
  for (int n = 0; n < N; n++) {
    size_t s = (size_t)n * blocks * 4;
    size_t o = orc_si(N, blocks, n, 0) * 4;
    for (int b = 0; b < blocks; b++, s += 4, o += 16) {
      for (int h = 0; h < 2; h++) {
        uint32_t lo = rd32(raw + 4 * (s + h)), hi = rd32(raw + 4 * (s + 2 + h));
        uint32_t even = (lo & 0x0f0f0f0fu) | ((hi & 0x0f0f0f0fu) << 4);
        uint32_t odd = ((lo >> 4) & 0x0f0f0f0fu) | (hi & 0xf0f0f0f0u);
        uint32_t e0 = even & 0xffffu, o0 = odd & 0xffffu, e1 = even >> 16, o1 = odd >> 16;
        quants[o + 2 * h] = ((e0 | (e0 << 8)) & 0x00ff00ffu) | (((o0 | (o0 << 8)) & 0x00ff00ffu) << 8);
        quants[o + 2 * h + 1] =
            ((e1 | (e1 << 8)) & 0x00ff00ffu) | (((o1 | (o1 << 8)) & 0x00ff00ffu) << 8);
      }
    }
  }
}

/* src/repack.ts:865-891: row n as the GPU dequantizes it, scale * (q - z)
 * in doubles, stored as float32. z = 8, a u8 zero point or a half. */
void orc_matrix_row(const orc_qm *m, int n, float *out) {
  const float *half = htab();
  int blocks = m->K / 32;
  const uint8_t *q = (const uint8_t *)m->quants;
  for (int b = 0; b < blocks; b++) {
    size_t si = orc_si(m->N, blocks, n, b);
    double scale = half[m->scales[si]];
    double zero = m->zero_halves ? (double)half[m->zero_halves[si]]
                  : m->zeros     ? (double)m->zeros[si]
                                 : 8.0;
    for (int j = 0; j < 32; j++) {
      int nib;
      if (m->raw)
        nib = (m->raw[((size_t)n * blocks + b) * 16 + (j >> 1)] >> ((j & 1) << 2)) & 15;
      else if (j < 16)
        nib = q[(si - 4 * (size_t)b) * 16 + (size_t)b * 64 + j] & 15;
      else
        nib = q[(si - 4 * (size_t)b) * 16 + (size_t)b * 64 + j - 16] >> 4;
      out[b * 32 + j] = (float)(scale * ((double)nib - zero));
    }
  }
}

/* Every row of a matrix as orc_matrix_row gives it (rows in parallel). */
void orc_matrix_dense(const orc_qm *m, float *out, int threads) {
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(static)
#endif
  for (int n = 0; n < m->N; n++) orc_matrix_row(m, n, out + (size_t)n * m->K);
  (void)threads;
}

/* src/repack.ts:474-511 (ggml's dequantize_row_q4_K as the reference
 * states it): w = d * sc * q - dmin * m, in doubles, stored as float32. */
void orc_dequantize_q4_k(const uint8_t *src, int rows, int K, float *out) {
  const float *half = htab();
  size_t supers = (size_t)rows * K / 256;
  for (size_t s = 0; s < supers; s++) {
    const uint8_t *p = src + s * 144;
    double d = half[rd16(p)], dmin = half[rd16(p + 2)];
    size_t y = s * 256;
    for (int is = 0; is < 8; is += 2) {
      const uint8_t *q = p + 16 + is * 16;
      int s1, m1, s2, m2;
      scale_min_pair(p + 4, is, &s1, &m1, &s2, &m2);
      double d1 = d * s1, min1 = dmin * m1, d2 = d * s2, min2 = dmin * m2;
      for (int l = 0; l < 32; l++) out[y++] = (float)(d1 * (q[l] & 15) - min1);
      for (int l = 0; l < 32; l++) out[y++] = (float)(d2 * (q[l] >> 4) - min2);
    }
  }
}

/* src/load-onnx.ts:471-501, 4-bit: scale * (nibble - zero) per block. */
void orc_dequantize_nbits_row(int K, const uint8_t *quant, const uint8_t *scales,
                              const uint8_t *zp, int n, float *out) {
  const float *half = htab();
  int blocks = K / 32, zp_stride = (blocks + 1) / 2;
  for (int b = 0; b < blocks; b++) {
    size_t sp = ((size_t)n * blocks + b) * 2;
    double scale = half[rd16(scales + sp)];
    int zero = zp ? (zp[(size_t)n * zp_stride + (b >> 1)] >> ((b & 1) << 2)) & 15 : 8;
    size_t q = ((size_t)n * blocks + b) * 16;
    for (int j = 0; j < 16; j++) {
      uint8_t byte = quant[q + j];
      out[b * 32 + 2 * j] = (float)(scale * ((byte & 15) - zero));
      out[b * 32 + 2 * j + 1] = (float)(scale * ((byte >> 4) - zero));
    }
  }
}

/* src/load-onnx.ts:450-462: float32 scales of a q4 export rounded to halves. */
void orc_half_bytes_f32(const float *src, size_t n, uint16_t *out) {
  for (size_t i = 0; i < n; i++) out[i] = orc_to_half(src[i]);
}

/* ------------------------------------------------ synthetic quantizers */

/* ggml's reference Q4_0 quantizer (quantize_row_q4_0_ref, ggml-quants.c,
 * MIT; not vendored in the reference, whose GGUF files come from it):
 * m = the signed weight of largest magnitude, d = m / -8, id = 1 / d,
 * stored d = half(d), q = min(15, (int8)(w * id + 8.5)). */
void orc_quantize_q4_0(const float *w, int rows, int K, uint8_t *out) {
  size_t blocks = (size_t)rows * K / 32;
  for (size_t b = 0; b < blocks; b++) {
    const float *x = w + b * 32;
    float amax = 0.0f, mx = 0.0f;
    for (int j = 0; j < 32; j++) {
      float v = x[j];
      if (amax < fabsf(v)) {
        amax = fabsf(v);
        mx = v;
      }
    }
    float d = mx / -8.0f;
    float id = d ? 1.0f / d : 0.0f;
    uint16_t dh = orc_to_half(d);
    uint8_t *o = out + b * 18;
    o[0] = dh & 255;
    o[1] = dh >> 8;
    for (int j = 0; j < 16; j++) {
      float x0 = x[j] * id, x1 = x[16 + j] * id;
      int q0 = (int)(signed char)(x0 + 8.5f), q1 = (int)(signed char)(x1 + 8.5f);
      if (q0 > 15) q0 = 15;
      if (q1 > 15) q1 = 15;
      o[2 + j] = (uint8_t)(q0 | (q1 << 4));
    }
  }
}

/* The MatMulNBits workload's quantizer (an asymmetric 4-bit scheme with a
 * given zero point per block): scale = half(absmax / max(zp, 15 - zp)),
 * q = clamp(round(w / scale) + zp, 0, 15); quant bytes [rows][K/32][16]
 * with element 2i in byte i's low nibble, zero points two blocks a byte,
 * low nibble first (src/load-onnx.ts:471-501 reads them back). */
void orc_quantize_nbits(const float *w, int rows, int K, const uint8_t *zpb, uint8_t *quant,
                        uint16_t *scales, uint8_t *zp_packed) {
  const float *half = htab();
  int blocks = K / 32, zp_stride = (blocks + 1) / 2;
  memset(zp_packed, 0, (size_t)rows * zp_stride);
  for (int n = 0; n < rows; n++)
    for (int b = 0; b < blocks; b++) {
      const float *x = w + (size_t)n * K + b * 32;
      int zp = zpb[(size_t)n * blocks + b] & 15;
      float amax = 0.0f;
      for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(x[j]));
      int span = zp > 15 - zp ? zp : 15 - zp;
      uint16_t sh = orc_to_half(amax / (float)span);
      float s = half[sh];
      scales[(size_t)n * blocks + b] = sh;
      uint8_t *q = quant + ((size_t)n * blocks + b) * 16;
      for (int j = 0; j < 16; j++) {
        int v[2];
        for (int t = 0; t < 2; t++) {
          float r = s > 0.0f ? rintf(x[2 * j + t] / s) : 0.0f;
          int qq = (int)r + zp;
          v[t] = qq < 0 ? 0 : qq > 15 ? 15 : qq;
        }
        q[j] = (uint8_t)(v[0] | (v[1] << 4));
      }
      zp_packed[(size_t)n * zp_stride + (b >> 1)] |= (uint8_t)(zp << ((b & 1) << 2));
    }
}

/* ---------------------------------------------------------------- matmul */

void orc_gemv_f64(const orc_qm *m, const float *x, int M, double *y, int threads) {
  int N = m->N, K = m->K;
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel
#endif
  {
    float *row = (float *)malloc(sizeof(float) * K);
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
    for (int n = 0; n < N; n++) {
      orc_matrix_row(m, n, row);
      for (int t = 0; t < M; t++) {
        double s = 0.0;
        const float *xt = x + (size_t)t * K;
        for (int k = 0; k < K; k++) s += (double)row[k] * (double)xt[k];
        y[(size_t)t * N + n] = s;
      }
    }
    free(row);
  }
  (void)threads;
}

/* The split rule of src/engine.ts:5316-5327: slices per token =
 * max(1, min(maxSplit, ceil(splitFragments / groups), blocks / 4)). */
static void split_rule(int groups, int blocks, int split_fragments, int max_split, int *kb_slice,
                       int *slices) {
  int a = (split_fragments + groups - 1) / groups;
  int split = max_split < a ? max_split : a;
  if (blocks / 4 < split) split = blocks / 4;
  if (split < 1) split = 1;
  *kb_slice = (blocks + split - 1) / split;
  *slices = (blocks + *kb_slice - 1) / *kb_slice;
}

/* src/gpu/kernels.ts:163-296 (word texels, split) and :744-895: a fragment
 * is a row group x token x K-slice; per block it forms the 8 activation
 * vec4s from halves (h2lo/h2hi), sa = dot(A0 + ... + A7, 1), per row
 * b = sum of dot(lo nibbles, A_w) + dot(hi nibbles, A_w+4), and
 * acc += d * (b - z * sa), all in float32; pf (kernels.ts:69-79) adds the
 * slices' partial sums in slice order. */
void orc_matmul_split(const orc_qm *m, const uint16_t *x16, int M, float *y, int threads,
                      int split_fragments, int max_split) {
  const float *half = htab();
  int N = m->N, K = m->K, blocks = K / 32, groups = N / 4;
  int kb_slice, slices;
  split_rule(groups, blocks, split_fragments, max_split, &kb_slice, &slices);
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(static) collapse(2)
#endif
  for (int g = 0; g < groups; g++)
    for (int t = 0; t < M; t++) {
      float total[4] = {0, 0, 0, 0};
      const uint16_t *xa = x16 + (size_t)t * K;
      for (int s = 0; s < slices; s++) {
        int kb0 = s * kb_slice, kb1 = kb0 + kb_slice < blocks ? kb0 + kb_slice : blocks;
        float acc[4] = {0, 0, 0, 0};
        for (int kb = kb0; kb < kb1; kb++) {
          float A[8][4];
          for (int j = 0; j < 4; j++)
            for (int c = 0; c < 4; c++) {
              A[2 * j][c] = half[xa[kb * 32 + 8 * j + c]];
              A[2 * j + 1][c] = half[xa[kb * 32 + 8 * j + 4 + c]];
            }
          /* Activation vec4 A_w holds elements 4w..4w+3 of the block
           * (h2lo/h2hi of texel w/2): weights 4w..4w+3 are word w's low
           * nibbles, 16+4w.. its high ones. */
          float sv[4] = {0, 0, 0, 0};
          for (int j = 0; j < 8; j++)
            for (int c = 0; c < 4; c++) sv[c] += A[j][c];
          float sa = sv[0] + sv[1] + sv[2] + sv[3];
          for (int r = 0; r < 4; r++) {
            size_t si = ((size_t)g * blocks + kb) * 4 + r;
            float d = half[m->scales[si]];
            float z = m->zero_halves ? half[m->zero_halves[si]]
                      : m->zeros     ? (float)m->zeros[si]
                                     : 8.0f;
            float b = 0.0f;
            for (int w = 0; w < 4; w++) {
              uint32_t word = m->quants[si * 4 + w];
              float dl = 0.0f, dh = 0.0f;
              for (int c = 0; c < 4; c++) {
                dl += (float)((word >> (8 * c)) & 15u) * A[w][c];
                dh += (float)((word >> (8 * c + 4)) & 15u) * A[w + 4][c];
              }
              b += dl + dh;
            }
            acc[r] += d * (b - z * sa);
          }
        }
        for (int r = 0; r < 4; r++) total[r] += acc[r];
      }
      for (int r = 0; r < 4; r++) y[(size_t)t * N + 4 * g + r] = total[r];
    }
  (void)threads;
}

/* -------------------------------------------- 8-bit and Q6_K matrices */

/* src/repack.ts:174-200: GGUF Q8_0 blocks (fp16 d, 32 int8) into an 8-bit
 * matrix: scale index si = (n >> 2) * blocks * 4 + (n & 3) + 4 b, the 32
 * codes at bytes 32 si.. as they are. */
int orc_pack_q8_0(uint8_t *quants, uint16_t *scales, int N, int K, int row0, const uint8_t *src,
                  size_t src_len, int rows, const int32_t *src_rows) {
  int blocks = K / 32;
  if (row0 < 0 || row0 + rows > N) return -1;
  for (int i = 0; i < rows; i++) {
    int n = row0 + i;
    int from = src_rows ? src_rows[i] : i;
    if ((size_t)(from + 1) * blocks * 34 > src_len) return -1;
    const uint8_t *p = src + (size_t)from * blocks * 34;
    size_t si = (size_t)(n >> 2) * blocks * 4 + (n & 3);
    for (int b = 0; b < blocks; b++, p += 34, si += 4) {
      scales[si] = rd16(p);
      memcpy(quants + si * 32, p + 2, 32);
    }
  }
  return 0;
}

/* src/repack.ts:634-704 (quantizeQ8): per block of 32, max = the largest
 * |v| (NaN if any is: Math.max), h = toHalf(max / 127); a scale that is not
 * > 0 gives q = 0; otherwise q = ((v / scale + 128.5) | 0) - 128 clamped to
 * +-127, the quotient and sum in doubles and `| 0` JavaScript's ToInt32
 * (truncation toward zero; NaN and infinities give 0). */
static int32_t to_int32(double x) {
  if (!(x == x) || isinf(x)) return 0;
  double t = trunc(x);
  double m = fmod(t, 4294967296.0);
  if (m < 0) m += 4294967296.0;
  return (int32_t)(uint32_t)m;
}

int orc_quantize_q8(uint8_t *quants, uint16_t *scales, int N, int K, int row0,
                    const float *values, int rows) {
  const float *half = htab();
  int blocks = K / 32;
  if (row0 < 0 || row0 + rows > N) return -1;
  for (int i = 0; i < rows; i++) {
    int n = row0 + i;
    const float *v = values + (size_t)i * K;
    size_t si = (size_t)(n >> 2) * blocks * 4 + (n & 3);
    for (int b = 0; b < blocks; b++, v += 32, si += 4) {
      double max = 0;
      for (int j = 0; j < 32; j++) {
        double a = fabs((double)v[j]);
        max = (a != a || max != max) ? NAN : (a > max ? a : max);
      }
      uint16_t h = orc_to_half(max / 127);
      double scale = half[h];
      scales[si] = h;
      int8_t *q = (int8_t *)(quants + si * 32);
      if (!(scale > 0)) {
        memset(q, 0, 32);
        continue;
      }
      for (int j = 0; j < 32; j++) {
        int32_t x = to_int32((double)v[j] / scale + 128.5) - 128;
        q[j] = (int8_t)(x > 127 ? 127 : x < -127 ? -127 : x);
      }
    }
  }
  return 0;
}

/* src/repack.ts:706-728 (packQ6_K): a row's super-block (210 bytes: ql[128],
 * qh[64], int8 scales[16], fp16 d) kept as its first 208 bytes at record
 * (g * supers + s) * 4 + r, its d in the scales there. (src_rows, which the
 * reference's packer does not take, picks each row's source row.) */
int orc_pack_q6_k(uint8_t *quants, uint16_t *scales, int N, int K, int row0, const uint8_t *src,
                  size_t src_len, int rows, const int32_t *src_rows) {
  int supers = K / 256;
  if (row0 < 0 || row0 + rows > N) return -1;
  for (int i = 0; i < rows; i++) {
    int n = row0 + i, g = n >> 2, r = n & 3;
    int from = src_rows ? src_rows[i] : i;
    if ((size_t)(from + 1) * supers * 210 > src_len) return -1;
    for (int s = 0; s < supers; s++) {
      const uint8_t *p = src + ((size_t)from * supers + s) * 210;
      size_t at = ((size_t)g * supers + s) * 4 + r;
      memcpy(quants + at * 208, p, 208);
      scales[at] = rd16(p + 208);
    }
  }
  return 0;
}

/* src/repack.ts:447-466 (dequantize_row_q4_1 as the reference states it):
 * blocks of 32 (fp16 d, fp16 m, 16 nibble bytes: weight j low, j + 16
 * high), w = q d + m in doubles, stored as float32. */
void orc_dequantize_q4_1(const uint8_t *src, int rows, int K, float *out) {
  const float *half = htab();
  size_t blocks = (size_t)rows * K / 32;
  for (size_t b = 0; b < blocks; b++) {
    const uint8_t *p = src + b * 20;
    double d = half[rd16(p)], m = half[rd16(p + 2)];
    for (int j = 0; j < 16; j++) {
      out[b * 32 + j] = (float)((p[4 + j] & 15) * d + m);
      out[b * 32 + j + 16] = (float)((p[4 + j] >> 4) * d + m);
    }
  }
}

/* src/repack.ts:535-572 (dequantize_row_q5_K as the reference states it):
 * super-blocks of 256 (fp16 d, fp16 dmin, 12 scale/min bytes, qh[32],
 * qs[128]); sub-block j: w = d sc (q + 16 (qh bit j)) - dmin m. */
void orc_dequantize_q5_k(const uint8_t *src, int rows, int K, float *out) {
  const float *half = htab();
  size_t supers = (size_t)rows * K / 256;
  for (size_t s = 0; s < supers; s++) {
    const uint8_t *p = src + s * 176;
    double d = half[rd16(p)], dmin = half[rd16(p + 2)];
    const uint8_t *qh = p + 16;
    float *y = out + s * 256;
    for (int is = 0; is < 8; is += 2) {
      const uint8_t *ql = p + 48 + is * 16;
      int s1, m1, s2, m2;
      scale_min_pair(p + 4, is, &s1, &m1, &s2, &m2);
      double d1 = d * s1, min1 = dmin * m1, d2 = d * s2, min2 = dmin * m2;
      for (int l = 0; l < 32; l++)
        *y++ = (float)(d1 * ((ql[l] & 15) + ((qh[l] >> is) & 1 ? 16 : 0)) - min1);
      for (int l = 0; l < 32; l++)
        *y++ = (float)(d2 * ((ql[l] >> 4) + ((qh[l] >> (is + 1)) & 1 ? 16 : 0)) - min2);
    }
  }
}

/* src/repack.ts:514-528: out = d * int8, per 34-byte block. */
void orc_dequantize_q8_0(const uint8_t *src, int rows, int K, float *out) {
  const float *half = htab();
  size_t blocks = (size_t)rows * K / 32;
  for (size_t b = 0; b < blocks; b++) {
    const uint8_t *p = src + b * 34;
    double d = half[rd16(p)];
    for (int j = 0; j < 32; j++) out[b * 32 + j] = (float)(d * (int8_t)p[2 + j]);
  }
}

/* src/repack.ts:405-440 (ggml's dequantize_row_q6_K as the reference states
 * it): in half n of a super-block, for l = 0..31 and is = l / 16,
 *   y[128n + l]      = d sc[8n + is]     (ql[64n + l] & 15       | (qh[32n + l] & 3) << 4      - 32)
 *   y[128n + l + 32] = d sc[8n + is + 2] (ql[64n + l + 32] & 15  | (qh[32n + l] >> 2 & 3) << 4 - 32)
 *   y[128n + l + 64] = d sc[8n + is + 4] (ql[64n + l] >> 4       | (qh[32n + l] >> 4 & 3) << 4 - 32)
 *   y[128n + l + 96] = d sc[8n + is + 6] (ql[64n + l + 32] >> 4  | (qh[32n + l] >> 6) << 4     - 32)
 * d sc exact in doubles, each product rounded once to float32. */
static void q6k_super(const uint8_t *p, double d, float *y) {
  for (int n = 0; n < 2; n++, y += 128) {
    const uint8_t *ql = p + n * 64, *qh = p + 128 + n * 32;
    const int8_t *sc = (const int8_t *)(p + 192 + n * 8);
    for (int l = 0; l < 32; l++) {
      int is = l / 16;
      int h = qh[l];
      y[l] = (float)(d * sc[is] * (((ql[l] & 15) | ((h & 3) << 4)) - 32));
      y[l + 32] = (float)(d * sc[is + 2] * (((ql[l + 32] & 15) | (((h >> 2) & 3) << 4)) - 32));
      y[l + 64] = (float)(d * sc[is + 4] * (((ql[l] >> 4) | (((h >> 4) & 3) << 4)) - 32));
      y[l + 96] = (float)(d * sc[is + 6] * (((ql[l + 32] >> 4) | (((h >> 6) & 3) << 4)) - 32));
    }
  }
}

void orc_dequantize_q6_k(const uint8_t *src, int rows, int K, float *out) {
  const float *half = htab();
  size_t supers = (size_t)rows * K / 256;
  for (size_t s = 0; s < supers; s++) {
    const uint8_t *p = src + s * 210;
    q6k_super(p, half[rd16(p + 208)], out + s * 256);
  }
}

/* matrixRow of an 8-bit matrix (src/repack.ts:873-876): scale * signed byte. */
void orc_q8_row(const uint8_t *quants, const uint16_t *scales, int K, int n, float *out) {
  const float *half = htab();
  int blocks = K / 32;
  for (int b = 0; b < blocks; b++) {
    size_t si = (size_t)(n >> 2) * blocks * 4 + (n & 3) + 4 * (size_t)b;
    double d = half[scales[si]];
    for (int j = 0; j < 32; j++) out[b * 32 + j] = (float)(d * (int8_t)quants[si * 32 + j]);
  }
}

/* Row n of a 6-bit matrix: each record's bytes as dequantize_row_q6_K reads
 * them (src/weights.ts:23-30; the Q6_K head's formula, src/gpu/kernels.ts:
 * 3376-3390). */
void orc_q6k_row(const uint8_t *quants, const uint16_t *scales, int K, int n, float *out) {
  const float *half = htab();
  int supers = K / 256;
  for (int s = 0; s < supers; s++) {
    size_t at = ((size_t)(n >> 2) * supers + s) * 4 + (n & 3);
    q6k_super(quants + at * 208, half[scales[at]], out + s * 256);
  }
}

/* The 8-bit matmul (src/gpu/kernels.ts:219-246; split as orc_matmul_split):
 * per block and row, b = sum over the 8 words of dot(q, A_w) with q the
 * signed bytes as floats, then acc += d * b, float32; slices summed in
 * order. */
void orc_matmul_q8(const uint8_t *quants, const uint16_t *scales, int N, int K,
                   const uint16_t *x16, int M, float *y, int threads, int split_fragments,
                   int max_split) {
  const float *half = htab();
  int blocks = K / 32, groups = N / 4;
  int kb_slice, slices;
  split_rule(groups, blocks, split_fragments, max_split, &kb_slice, &slices);
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(static) collapse(2)
#endif
  for (int g = 0; g < groups; g++)
    for (int t = 0; t < M; t++) {
      float total[4] = {0, 0, 0, 0};
      const uint16_t *xa = x16 + (size_t)t * K;
      for (int s = 0; s < slices; s++) {
        int kb0 = s * kb_slice, kb1 = kb0 + kb_slice < blocks ? kb0 + kb_slice : blocks;
        float acc[4] = {0, 0, 0, 0};
        for (int kb = kb0; kb < kb1; kb++)
          for (int r = 0; r < 4; r++) {
            size_t si = ((size_t)g * blocks + kb) * 4 + r;
            const int8_t *q = (const int8_t *)(quants + si * 32);
            float b = 0.0f;
            for (int w = 0; w < 8; w++) {
              float dw = 0.0f;
              for (int c = 0; c < 4; c++)
                dw += (float)q[4 * w + c] * half[xa[kb * 32 + 4 * w + c]];
              b += dw;
            }
            acc[r] += half[scales[si]] * b;
          }
        for (int r = 0; r < 4; r++) total[r] += acc[r];
      }
      for (int r = 0; r < 4; r++) y[(size_t)t * N + 4 * g + r] = total[r];
    }
  (void)threads;
}

/* The Q6_K head (src/gpu/kernels.ts:3593-3686): per row and super-block, P
 * = sum over the 16 sub-blocks of sc * sum (q - 32) a (float32), then acc
 * += d * P. */
void orc_matmul_q6k(const uint8_t *quants, const uint16_t *scales, int N, int K,
                    const uint16_t *x16, int M, float *y, int threads) {
  const float *half = htab();
  int supers = K / 256;
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(static) collapse(2)
#endif
  for (int n = 0; n < N; n++)
    for (int t = 0; t < M; t++) {
      const uint16_t *xa = x16 + (size_t)t * K;
      float acc = 0.0f;
      for (int s = 0; s < supers; s++) {
        size_t at = ((size_t)(n >> 2) * supers + s) * 4 + (n & 3);
        const uint8_t *p = quants + at * 208;
        float P = 0.0f;
        for (int sub = 0; sub < 16; sub++) {
          /* sub-block sub covers weights 16 sub .. 16 sub + 15: half n = sub / 8,
           * group i = sub % 8 / 2, l = 16 (sub % 2) + 0..15 */
          int hn = sub / 8, i = (sub % 8) / 2, l0 = 16 * (sub % 2);
          const uint8_t *ql = p + 64 * hn + 32 * (i & 1), *qh = p + 128 + 32 * hn;
          float dot = 0.0f;
          for (int l = l0; l < l0 + 16; l++) {
            int q = ((ql[l] >> (4 * (i >> 1))) & 15) | (((qh[l] >> (2 * i)) & 3) << 4);
            dot += (float)(q - 32) * half[xa[256 * s + 128 * hn + 32 * i + l]];
          }
          P += (float)((const int8_t *)(p + 192))[8 * hn + 2 * i + l0 / 16] * dot;
        }
        acc += half[scales[at]] * P;
      }
      y[(size_t)t * N + n] = acc;
    }
  (void)threads;
}

/* ---------------------------------------------------- sampling candidates */

/* PENALIZED (src/gpu/kernels.ts:3102-3122) for token id of batch row r:
 * -1e30 where it may not be drawn (allowed bit clear, mask 2, past V),
 * else a seen token's logit divided (positive) or multiplied (negative) by
 * the penalty and less the presence penalty. */
static float orc_penalized(float v, int id, int r, int V, const uint8_t *mask,
                           const int32_t *seen, int n_seen, float penalty, float presence,
                           const uint32_t *allowed, int allowed_rows, int ld_allowed) {
  if (id >= V) return -1e30f;
  if (allowed) {
    int row = allowed_rows == 1 ? 0 : r;
    if (row >= allowed_rows) return -1e30f;
    if (!((allowed[(size_t)row * ld_allowed + (id >> 5)] >> (id & 31)) & 1u)) return -1e30f;
  }
  int m = mask ? mask[id] : 0;
  if (m == 2) return -1e30f;
  int state = m;
  for (int k = 0; k < n_seen; k++)
    if (seen[4 * k] == id && r >= seen[4 * k + 2] && r < seen[4 * k + 3]) state = seen[4 * k + 1];
  if (state == 1 || state == 3) {
    v = v < 0.0f ? v * penalty : v / penalty;
    v -= presence;
  }
  return v;
}

/* CHUNK_MAX + CHUNK_RANK + CHUNK_BY_RANK + CHUNK_GATHER (src/gpu/kernels.ts:
 * 3147-3163, :3265-3323; Engine.pick, src/engine.ts:8352-8473): per row,
 * each 256-token chunk's largest penalized logit, the chunks ranked (larger
 * first, ties to the lower index), the first `count` chunks' indices and
 * penalized logits. */
void orc_pick_candidates(const float *logits, int M, int V, const uint8_t *mask,
                         const int32_t *seen, int n_seen, int row0, float penalty,
                         float presence, const uint32_t *allowed, int allowed_rows,
                         int ld_allowed, int count, int32_t *chunks_out, float *cand_out) {
  int total = (V + 255) / 256;
  float *mx = malloc(sizeof(float) * total);
  for (int m = 0; m < M; m++) {
    const float *row = logits + (size_t)m * V;
    int r = row0 + m;
    for (int c = 0; c < total; c++) {
      float best = -1e30f;
      for (int t = 0; t < 256; t++) {
        int id = c * 256 + t;
        float v = orc_penalized(id < V ? row[id] : 0.0f, id, r, V, mask, seen, n_seen, penalty,
                                presence, allowed, allowed_rows, ld_allowed);
        if (v > best) best = v;
      }
      mx[c] = best;
    }
    for (int c = 0; c < total; c++) {
      int rank = 0;
      for (int i = 0; i < total; i++) rank += mx[i] > mx[c] || (mx[i] == mx[c] && i < c);
      if (rank < count) chunks_out[(size_t)m * count + rank] = c;
    }
    for (int k = 0; k < count; k++) {
      int c = chunks_out[(size_t)m * count + k];
      for (int t = 0; t < 256; t++) {
        int id = c * 256 + t;
        cand_out[((size_t)m * count + k) * 256 + t] =
            orc_penalized(id < V ? row[id] : 0.0f, id, r, V, mask, seen, n_seen, penalty,
                          presence, allowed, allowed_rows, ld_allowed);
      }
    }
  }
  free(mx);
}

/* ------------------------------------------------------------ elementwise */

/* packH2 (src/gpu/kernels.ts:32-36): clamped to +-65504, then to halves. */
void orc_f32_to_h2(const float *x, size_t n, uint16_t *out) {
  for (size_t i = 0; i < n; i++) {
    float v = x[i];
    if (v > 65504.0f) v = 65504.0f;
    if (v < -65504.0f) v = -65504.0f;
    out[i] = orc_to_half(v);
  }
}

/* RMS_SCALE + NORM_TO_H2 (src/gpu/kernels.ts:1195-1242): x * w / sqrt(mean
 * of squares + eps), computed here in doubles. */
void orc_rms_norm(const float *x, const float *w, int M, int D, float eps, float *out) {
  for (int m = 0; m < M; m++) {
    double s = 0.0;
    for (int i = 0; i < D; i++) s += (double)x[(size_t)m * D + i] * x[(size_t)m * D + i];
    double r = 1.0 / sqrt(s / D + (double)eps);
    for (int i = 0; i < D; i++) out[(size_t)m * D + i] = (float)(x[(size_t)m * D + i] * r * w[i]);
  }
}

/* REDUCE_SWIGLU (src/gpu/kernels.ts:1066-1077): silu(gate) * up, gate rows
 * first then up rows in each token's row of 2F. */
void orc_swiglu(const float *gu, int M, int F, float *out) {
  for (int m = 0; m < M; m++)
    for (int i = 0; i < F; i++) {
      double g = gu[(size_t)m * 2 * F + i], u = gu[(size_t)m * 2 * F + F + i];
      out[(size_t)m * F + i] = (float)(g / (1.0 + exp(-g)) * u);
    }
}

/* ------------------------------------------------------------- attention */

int orc_rope_rows(int context) { return 1024 + (context + 1023) / 1024; }

/* src/engine.ts:1292-1312: cos and sin of pos * theta^(-2i/freqDims) in
 * doubles, stored as float32; rows 0..1023 are positions, row 1024 + h the
 * position 1024 h. Row r: head_dim/2 cosines, then head_dim/2 sines. */
void orc_rope_table(double theta, int head_dim, int rotated_dims, int freq_dims, int context,
                    float *table) {
  int half = head_dim / 2, rows = orc_rope_rows(context);
  for (int r = 0; r < rows; r++) {
    double pos = r < 1024 ? r : (double)(r - 1024) * 1024.0;
    for (int i = 0; i < half; i++) {
      double freq = i < rotated_dims / 2 ? pow(theta, (-2.0 * i) / freq_dims) : 0.0;
      double angle = pos * freq;
      table[(size_t)r * head_dim + i] = (float)cos(angle);
      table[(size_t)r * head_dim + half + i] = (float)sin(angle);
    }
  }
}

/* headPrep (src/gpu/kernels.ts:2196-2322) for one head of head_dim values:
 * optional RMS norm over the head (inverse sqrt of the mean square + eps,
 * times norm_w), RoPE on the rotated dims (dim j pairs with j + R/2 at
 * frequency j, angle of pos = lo + 1024 hi added from the table's two
 * rows), times scale. float32 like the shader. */
void orc_head_prep(const float *x, const float *norm_w, const float *rope, int head_dim,
                   int rotated_dims, int pos, float eps, float scale, int use_norm, float *out) {
  float inv = 1.0f;
  if (use_norm) {
    float s = 0.0f;
    for (int i = 0; i < head_dim; i++) s += x[i] * x[i];
    inv = 1.0f / sqrtf(s / (float)head_dim + eps);
  }
  int P = rotated_dims / 2;
  int lo = pos & 1023, hi = 1024 + (pos >> 10);
  for (int t = 0; t < head_dim; t++) {
    float v = x[t] * (use_norm ? inv * norm_w[t] : 1.0f);
    float r = v;
    if (t < 2 * P) {
      int first = t < P;
      int tp = first ? t + P : t - P;
      int f = first ? t : tp;
      float p = x[tp] * (use_norm ? inv * norm_w[tp] : 1.0f);
      float c1 = rope[(size_t)lo * head_dim + f], s1 = rope[(size_t)lo * head_dim + head_dim / 2 + f];
      float c2 = rope[(size_t)hi * head_dim + f], s2 = rope[(size_t)hi * head_dim + head_dim / 2 + f];
      float cs = c1 * c2 - s1 * s2, sn = s1 * c2 + c1 * s2;
      r = first ? v * cs - p * sn : v * cs + p * sn;
    }
    out[t] = r * scale;
  }
}

/* src/attention-check.ts:48-92 in doubles: per query head h (KV head
 * h / group), scores q . k_j over keys 0..keys-1, softmax with the max
 * subtracted, weighted sum of values. kc/vc rows hold kv_stride halves a
 * position (KV head kh at kh * head_dim). */
void orc_attention_f64(const float *q, const uint16_t *kc, const uint16_t *vc, int heads,
                       int kv_heads, int head_dim, int keys, int kv_stride, double *out) {
  const float *half = htab();
  int group = heads / kv_heads;
  double *scores = (double *)malloc(sizeof(double) * (keys > 0 ? keys : 1));
  for (int h = 0; h < heads; h++) {
    int kh = h / group;
    double mx = -INFINITY;
    for (int j = 0; j < keys; j++) {
      double s = 0.0;
      for (int d = 0; d < head_dim; d++)
        s += (double)q[h * head_dim + d] * half[kc[(size_t)j * kv_stride + kh * head_dim + d]];
      scores[j] = s;
      if (s > mx) mx = s;
    }
    double l = 0.0;
    for (int d = 0; d < head_dim; d++) out[h * head_dim + d] = 0.0;
    for (int j = 0; j < keys; j++) {
      double e = exp(scores[j] - mx);
      l += e;
      for (int d = 0; d < head_dim; d++)
        out[h * head_dim + d] += e * half[vc[(size_t)j * kv_stride + kh * head_dim + d]];
    }
    for (int d = 0; d < head_dim; d++) out[h * head_dim + d] /= l;
  }
  free(scores);
}

/* The shaders' float32 form of the same attention (scores, attend:
 * src/gpu/kernels.ts:2386-2579): scores q.k summed in float32, the max
 * subtracted, exp and the weighted values summed in float32, divided by the
 * total. Heads in parallel (OpenMP) with threads > 0: the CPU baseline's
 * attention. out: float32 [heads * head_dim]. */
void orc_attention_f32(const float *q, const uint16_t *kc, const uint16_t *vc, int heads,
                       int kv_heads, int head_dim, int keys, int kv_stride, float *out,
                       int threads) {
  const float *half = htab();
  int group = heads / kv_heads;
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(static)
#endif
  for (int h = 0; h < heads; h++) {
    int kh = h / group;
    float *scores = (float *)malloc(sizeof(float) * (keys > 0 ? keys : 1));
    float mx = -INFINITY;
    for (int j = 0; j < keys; j++) {
      float s = 0.0f;
      for (int d = 0; d < head_dim; d++)
        s += q[h * head_dim + d] * half[kc[(size_t)j * kv_stride + kh * head_dim + d]];
      scores[j] = s;
      if (s > mx) mx = s;
    }
    float l = 0.0f;
    float *o = out + (size_t)h * head_dim;
    for (int d = 0; d < head_dim; d++) o[d] = 0.0f;
    for (int j = 0; j < keys; j++) {
      float e = expf(scores[j] - mx);
      l += e;
      for (int d = 0; d < head_dim; d++) o[d] += e * half[vc[(size_t)j * kv_stride + kh * head_dim + d]];
    }
    for (int d = 0; d < head_dim; d++) o[d] = l > 0.0f ? o[d] / l : 0.0f;
    free(scores);
  }
  (void)threads;
}

/* ------------------------------------------------------- short conv */

/* convFused / convPrefixes (src/gpu/kernels.ts:1447-1523) for M tokens of
 * in_proj output bcx ([M][3D]: B | C | x, src/weights.ts:180-190):
 * y_t = B_t * x_t; out_t = C_t * sum_k taps[c*W + k] * y[t - (W-1) + k]
 * (earlier tokens' y from state, W-1 rows oldest first); new_state = the
 * last W-1 y rows; prefixes (if not NULL) block p-1 = the state after the
 * first p tokens. float32 like the shader. */
void orc_short_conv(const float *bcx, int M, int D, int W, const float *taps, const float *state,
                    float *out, float *new_state, float *prefixes) {
  int w1 = W - 1;
#define YV(t, c) ((t) >= 0 ? bcx[(size_t)(t) * 3 * D + (c)] * bcx[(size_t)(t) * 3 * D + 2 * D + (c)] \
                           : state[(size_t)(w1 + (t)) * D + (c)])
  for (int m = 0; m < M; m++)
    for (int c = 0; c < D; c++) {
      float a = 0.0f;
      for (int k = 0; k < W; k++) a += taps[(size_t)c * W + k] * YV(m - w1 + k, c);
      out[(size_t)m * D + c] = bcx[(size_t)m * 3 * D + D + c] * a;
    }
  for (int i = 0; i < w1; i++)
    for (int c = 0; c < D; c++) new_state[(size_t)i * D + c] = YV(M - w1 + i, c);
  if (prefixes)
    for (int p = 1; p <= M; p++)
      for (int i = 0; i < w1; i++)
        for (int c = 0; c < D; c++)
          prefixes[((size_t)(p - 1) * w1 + i) * D + c] = YV(p - w1 + i, c);
#undef YV
}

/* --------------------------------------------------------------- pick */

/* CHUNK_MAX_AT + CHUNK_ARGMAX_ROWS (src/gpu/kernels.ts:3169-3246): the
 * first position of the largest logit in each 256-logit chunk (strict >,
 * so NaN never wins), then the first chunk with the largest maximum: the
 * lowest id holding the maximum. Starts from -3e38 at id 0. */
int orc_argmax(const float *logits, int V, float *top) {
  float best = -3e38f;
  int at = 0;
  for (int c = 0; c * 256 < V; c++) {
    float mx = -3e38f;
    int pos = 0;
    for (int t = 0; t < 256 && c * 256 + t < V; t++)
      if (logits[c * 256 + t] > mx) {
        mx = logits[c * 256 + t];
        pos = t;
      }
    if (mx > best) {
      best = mx;
      at = c * 256 + pos;
    }
  }
  if (top) *top = best;
  return at;
}

/* ------------------------------------------------------ Gated DeltaNet */

/* deltaSequential (src/delta-rule.ts:38-62): one head, token by token, in
 * doubles. q, k [T][dk] (q already over sqrt(dk)), v [T][dv], beta and g
 * (the log-decay) [T]; S [dk][dv] in and out; o [T][dv]. Per token, with
 * a = exp(g): d = beta (v - a S^T k), S <- a S + k d^T, o = S^T q, the last
 * taken as a S^T q + (q.k) d. */
void orc_delta_sequential(int dk, int dv, int T, const double *q, const double *k,
                          const double *v, const double *beta, const double *g, double *S,
                          double *o) {
  double *d = malloc(sizeof(double) * dv);
  for (int t = 0; t < T; t++) {
    const double *qt = q + (size_t)t * dk, *kt = k + (size_t)t * dk;
    double a = exp(g[t]), qk = 0.0;
    for (int i = 0; i < dk; i++) qk += qt[i] * kt[i];
    for (int j = 0; j < dv; j++) {
      double kv = 0.0, qs = 0.0;
      for (int i = 0; i < dk; i++) {
        kv += S[(size_t)i * dv + j] * kt[i];
        qs += S[(size_t)i * dv + j] * qt[i];
      }
      d[j] = beta[t] * (v[(size_t)t * dv + j] - a * kv);
      o[(size_t)t * dv + j] = a * qs + qk * d[j];
    }
    for (int i = 0; i < dk; i++)
      for (int j = 0; j < dv; j++) S[(size_t)i * dv + j] = a * S[(size_t)i * dv + j] + kt[i] * d[j];
  }
  free(d);
}

/* deltaChunked (src/delta-rule.ts:73-166): the same recurrence in chunks of
 * `chunk` tokens after a first chunk of `first` (0: chunk). Within a chunk
 * of n tokens, G the running sum of g from its start:
 *   A[r][s] = beta_r e^{G_r - G_s} k_r.k_s (s < r), T = (I + A)^-1,
 *   U = T diag(beta) V, W = T diag(beta e^G) K, P[r][s] = e^{G_r - G_s} q_r.k_s
 *   (s <= r), Oi = P U, Q' = e^G Q - P W;
 * then from the chunk's starting state S0: D = U - W S0, O = Oi + Q' S0,
 * S = e^{G_last} S0 + sum_s e^{G_last - G_s} k_s d_s^T. With save_at > 0 the
 * state after token save_at (a chunk end) is copied to snap. This code is
 * arranged chunk by chunk; the reference computes the state-free tensors
 * for all chunks first, which changes no value. */
void orc_delta_chunked(int dk, int dv, int T, const double *q, const double *k,
                       const double *v, const double *beta, const double *g, double *S,
                       double *o, int chunk, int first, int save_at, double *snap) {
  if (first <= 0 || first > chunk) first = chunk;
  const int C = chunk;
  double *G = malloc(sizeof(double) * C), *A = calloc((size_t)C * C, sizeof(double));
  double *Ti = calloc((size_t)C * C, sizeof(double)), *P = calloc((size_t)C * C, sizeof(double));
  double *U = malloc(sizeof(double) * C * dv), *W = malloc(sizeof(double) * C * dk);
  double *Oi = malloc(sizeof(double) * C * dv), *Qp = malloc(sizeof(double) * C * dk);
  double *D = malloc(sizeof(double) * C * dv), *next = malloc(sizeof(double) * dk * dv);
  for (int c0 = 0; c0 < T;) {
    const int n = (c0 == 0 ? first : C) < T - c0 ? (c0 == 0 ? first : C) : T - c0;
    const double *qc = q + (size_t)c0 * dk, *kc = k + (size_t)c0 * dk, *vc = v + (size_t)c0 * dv;
    for (int r = 0; r < n; r++) G[r] = (r ? G[r - 1] : 0.0) + g[c0 + r];
    for (int r = 0; r < n; r++)
      for (int s = 0; s <= r; s++) {
        double kk = 0.0, qk = 0.0;
        for (int i = 0; i < dk; i++) {
          kk += kc[(size_t)r * dk + i] * kc[(size_t)s * dk + i];
          qk += qc[(size_t)r * dk + i] * kc[(size_t)s * dk + i];
        }
        const double e = exp(G[r] - G[s]);
        A[r * C + s] = s < r ? beta[c0 + r] * e * kk : 0.0;
        P[r * C + s] = e * qk;
      }
    /* forward substitution: row r of (I + A)^-1 from the rows above it */
    for (int r = 0; r < n; r++)
      for (int j = 0; j <= r; j++) {
        double acc = j == r ? 1.0 : 0.0;
        for (int s = j; s < r; s++) acc -= A[r * C + s] * Ti[s * C + j];
        Ti[r * C + j] = acc;
      }
    for (int r = 0; r < n; r++) {
      for (int j = 0; j < dv; j++) U[(size_t)r * dv + j] = 0.0;
      for (int i = 0; i < dk; i++) W[(size_t)r * dk + i] = 0.0;
      for (int s = 0; s <= r; s++) {
        const double tb = Ti[r * C + s] * beta[c0 + s], eg = exp(G[s]);
        for (int j = 0; j < dv; j++) U[(size_t)r * dv + j] += tb * vc[(size_t)s * dv + j];
        for (int i = 0; i < dk; i++) W[(size_t)r * dk + i] += tb * eg * kc[(size_t)s * dk + i];
      }
    }
    for (int r = 0; r < n; r++) {
      const double eg = exp(G[r]);
      for (int j = 0; j < dv; j++) Oi[(size_t)r * dv + j] = 0.0;
      for (int i = 0; i < dk; i++) Qp[(size_t)r * dk + i] = eg * qc[(size_t)r * dk + i];
      for (int s = 0; s <= r; s++) {
        const double p = P[r * C + s];
        for (int j = 0; j < dv; j++) Oi[(size_t)r * dv + j] += p * U[(size_t)s * dv + j];
        for (int i = 0; i < dk; i++) Qp[(size_t)r * dk + i] -= p * W[(size_t)s * dk + i];
      }
    }
    for (int r = 0; r < n; r++)
      for (int j = 0; j < dv; j++) {
        double ws = 0.0, qs = 0.0;
        for (int i = 0; i < dk; i++) {
          ws += W[(size_t)r * dk + i] * S[(size_t)i * dv + j];
          qs += Qp[(size_t)r * dk + i] * S[(size_t)i * dv + j];
        }
        D[(size_t)r * dv + j] = U[(size_t)r * dv + j] - ws;
        o[(size_t)(c0 + r) * dv + j] = Oi[(size_t)r * dv + j] + qs;
      }
    const double last = G[n - 1];
    for (int i = 0; i < dk; i++)
      for (int j = 0; j < dv; j++) {
        double acc = exp(last) * S[(size_t)i * dv + j];
        for (int s = 0; s < n; s++)
          acc += exp(last - G[s]) * kc[(size_t)s * dk + i] * D[(size_t)s * dv + j];
        next[(size_t)i * dv + j] = acc;
      }
    memcpy(S, next, sizeof(double) * dk * dv);
    c0 += n;
    if (snap && c0 == save_at) memcpy(snap, S, sizeof(double) * dk * dv);
  }
  free(G); free(A); free(Ti); free(P); free(U); free(W); free(Oi); free(Qp); free(D); free(next);
}

/* LIN_GATES (src/gpu/kernels.ts:1544-1562): from one row of the b|a
 * projection (b of the H heads, then a), beta = sigmoid(b) and the
 * log-decay A * softplus(a + dt_bias) (A = -exp(A_log), negative). */
void orc_delta_gates(const float *ba, int ldba, int H, const float *A, const float *dt,
                     double *beta, double *log_decay) {
  (void)ldba;
  for (int h = 0; h < H; h++) {
    beta[h] = 1.0 / (1.0 + exp(-(double)ba[h]));
    const double t = (double)ba[H + h] + dt[h];
    const double softplus = (t > 0.0 ? t : 0.0) + log1p(exp(-fabs(t)));
    log_decay[h] = (double)A[h] * softplus;
  }
}

/* LIN_PREP (src/gpu/kernels.ts:1646-1665): one head's q or k over
 * sqrt(sum of squares + 1e-6), q also over sqrt(dk). */
void orc_delta_prep(const float *x, int dk, int is_q, double *out) {
  double ss = 0.0;
  for (int i = 0; i < dk; i++) ss += (double)x[i] * x[i];
  const double inv = 1.0 / sqrt(ss + 1e-6) * (is_q ? 1.0 / sqrt((double)dk) : 1.0);
  for (int i = 0; i < dk; i++) out[i] = x[i] * inv;
}

/* linearAttend's recurrence for M rows (src/engine.ts:6697-6815): each
 * row's gates and q/k prep, then the delta rule per head, in doubles.
 * qkv rows hold q (H dk) | k (H dk) | v (H dv), ba rows b (H) | a (H);
 * state [H][dk][dv] in and out; snap (if save_at in 1..M) the state after
 * row save_at; out [M][H dv]. */
void orc_delta_rule(const float *qkv, int ldq, const float *ba, int ldba, const float *A,
                    const float *dt, int H, int dk, int dv, int M, double *state, int save_at,
                    double *snap, double *out) {
  const int K = H * dk;
  double *q = malloc(sizeof(double) * dk), *k = malloc(sizeof(double) * dk);
  double *v = malloc(sizeof(double) * dv), *o = malloc(sizeof(double) * dv);
  double *beta = malloc(sizeof(double) * H), *lg = malloc(sizeof(double) * H);
  for (int m = 0; m < M; m++) {
    const float *row = qkv + (size_t)m * ldq;
    orc_delta_gates(ba + (size_t)m * ldba, ldba, H, A, dt, beta, lg);
    for (int h = 0; h < H; h++) {
      orc_delta_prep(row + (size_t)h * dk, dk, 1, q);
      orc_delta_prep(row + K + (size_t)h * dk, dk, 0, k);
      for (int j = 0; j < dv; j++) v[j] = row[2 * K + (size_t)h * dv + j];
      orc_delta_sequential(dk, dv, 1, q, k, v, beta + h, lg + h,
                           state + (size_t)h * dk * dv, o);
      for (int j = 0; j < dv; j++) out[(size_t)m * H * dv + (size_t)h * dv + j] = o[j];
    }
    if (snap && m + 1 == save_at) memcpy(snap, state, sizeof(double) * H * dk * dv);
  }
  free(q); free(k); free(v); free(o); free(beta); free(lg);
}

/* LIN_CONV + LIN_CONV_STATE (src/gpu/kernels.ts:1564-1641): silu of the
 * depthwise causal convolution over the first C channels of each input
 * row (w [C][W], tap W-1 the current token), earlier tokens from state
 * [W-1][C] (oldest first); state_out = the last W-1 raw input rows. */
void orc_delta_conv(const float *in, int ldi, int M, int C, int W, const float *w,
                    const float *state, double *out, float *state_out) {
  for (int m = 0; m < M; m++)
    for (int c = 0; c < C; c++) {
      double acc = 0.0;
      for (int k = 0; k < W; k++) {
        const int t = m - (W - 1) + k;
        const double x = t >= 0 ? in[(size_t)t * ldi + c] : state[(size_t)(W - 1 + t) * C + c];
        acc += (double)w[(size_t)c * W + k] * x;
      }
      out[(size_t)m * C + c] = acc / (1.0 + exp(-acc));
    }
  for (int i = 0; i < W - 1; i++)
    for (int c = 0; c < C; c++) {
      const int t = M - (W - 1) + i;
      state_out[(size_t)i * C + c] =
          t >= 0 ? in[(size_t)t * ldi + c] : state[(size_t)(M + i) * C + c];
    }
}

/* LIN_NORM (src/gpu/kernels.ts:1836-1860): each head's output over its
 * RMS (eps inside), times the shared weights w [dv] and silu(z). */
void orc_delta_norm(const float *o, int ldo, int M, int H, int dv, const float *z, int ldz,
                    const float *w, float eps, double *out) {
  for (int m = 0; m < M; m++)
    for (int h = 0; h < H; h++) {
      const float *oh = o + (size_t)m * ldo + (size_t)h * dv;
      const float *zh = z + (size_t)m * ldz + (size_t)h * dv;
      double ss = 0.0;
      for (int j = 0; j < dv; j++) ss += (double)oh[j] * oh[j];
      const double inv = 1.0 / sqrt(ss / dv + (double)eps);
      for (int j = 0; j < dv; j++)
        out[(size_t)m * H * dv + (size_t)h * dv + j] =
            oh[j] * inv * w[j] * (zh[j] / (1.0 + exp(-(double)zh[j])));
    }
}

double orc_now(void) {
  struct timespec ts;
  clock_gettime(CLOCK_MONOTONIC, &ts);
  return ts.tv_sec + ts.tv_nsec * 1e-9;
}
