// Residual-stream glue between the matmuls: RMS norm into half activations,
// SwiGLU, and the embedding lookup (the reference's RMS_SCALE / NORM_TO_H2,
// REDUCE_SWIGLU and embed kernels, src/gpu/kernels.ts:1195-1264,
// :1066-1077, :1092-1149). Half outputs are clamped to +-65504 as packH2
// does (kernels.ts:32-36).
#include "common.h"
#include "dot.h"
#include "epilogue.h"
#include "wide.h"

namespace wg {
namespace {

__device__ inline uint16_t to_h(float v) {
  v = fminf(fmaxf(v, -65504.0f), 65504.0f);
  return __builtin_bit_cast(uint16_t, (_Float16)v);
}

// Block-wide sum over 256 threads (4 waves).
__device__ inline float block_sum256(float v, float *lds) {
  v = wave_sum(v);
  int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) lds[w] = v;
  __syncthreads();
  float t = lds[0] + lds[1] + lds[2] + lds[3];
  __syncthreads();
  return t;
}

// One workgroup per row: 1 / sqrt(mean x^2 + eps), then half(x * w * r).
__global__ __launch_bounds__(256) void rms_norm_kernel(const float *x, int D, int ldx,
                                                       const float *w, float eps, uint16_t *out,
                                                       int ldo, float *rs_out) {
  __shared__ float lds[4];
  const float *xr = x + (int64_t)blockIdx.x * ldx;
  float s = 0.0f;
  for (int i = threadIdx.x * 4; i < D; i += 1024) {
    float4 v = *reinterpret_cast<const float4 *>(xr + i);
    s += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
  }
  float r = 1.0f / sqrtf(block_sum256(s, lds) / (float)D + eps);
  if (rs_out && threadIdx.x == 0) rs_out[blockIdx.x] = r;
  uint16_t *o = out + (int64_t)blockIdx.x * ldo;
  for (int i = threadIdx.x * 4; i < D; i += 1024) {
    float4 v = *reinterpret_cast<const float4 *>(xr + i);
    float4 g = *reinterpret_cast<const float4 *>(w + i);
    ushort4 h;
    h.x = to_h(v.x * r * g.x);
    h.y = to_h(v.y * r * g.y);
    h.z = to_h(v.z * r * g.z);
    h.w = to_h(v.w * r * g.w);
    *reinterpret_cast<ushort4 *>(o + i) = h;
  }
}

// The reference's prescaled form (NORM_TO_H2 with PRESCALE): out =
// half(x * w / mult), rs_out[m] = mult / sqrt(mean x^2 + eps), the factor a
// product over out takes afterwards.
__global__ __launch_bounds__(256) void norm_to_h2_kernel(const float *x, int D, int ldx,
                                                         const float *w, float eps, float mult,
                                                         uint16_t *out, int ldo, float *rs_out) {
  __shared__ float lds[4];
  const float *xr = x + (int64_t)blockIdx.x * ldx;
  float s = 0.0f;
  for (int i = threadIdx.x * 4; i < D; i += 1024) {
    float4 v = *reinterpret_cast<const float4 *>(xr + i);
    s += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
  }
  const float ms = block_sum256(s, lds) / (float)D;
  if (threadIdx.x == 0) rs_out[blockIdx.x] = mult / sqrtf(ms + eps);
  uint16_t *o = out + (int64_t)blockIdx.x * ldo;
  for (int i = threadIdx.x * 4; i < D; i += 1024) {
    float4 v = *reinterpret_cast<const float4 *>(xr + i);
    float4 g = *reinterpret_cast<const float4 *>(w + i);
    ushort4 h;
    h.x = to_h(v.x * g.x / mult);
    h.y = to_h(v.y * g.y / mult);
    h.z = to_h(v.z * g.z / mult);
    h.w = to_h(v.w * g.w / mult);
    *reinterpret_cast<ushort4 *>(o + i) = h;
  }
}

// out[m][i] = half(silu(gu[m][i]) * gu[m][F + i]).
__global__ void swiglu_kernel(const float *gu, int M, int F, int ldg, uint16_t *out, int ldo) {
  int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (int64_t)M * F) return;
  int m = (int)(t / F), i = (int)(t % F);
  float g = gu[(int64_t)m * ldg + i], u = gu[(int64_t)m * ldg + F + i];
  out[(int64_t)m * ldo + i] = to_h(g / (1.0f + __expf(-g)) * u);
}

// The rows' token ids: ids[m], or (a verify step's drafts from a device
// table) ids[0] and, for rows m >= 1, entry m - 1 of table row *cursor
// (the last row once the cursor is past it), which the row's first thread
// also writes to ids[m] for the accept that follows.
struct EmbedIds {
  int32_t *ids;
  const int32_t *table;  // (or null)
  int n_steps;
  const int32_t *cursor;
};

__device__ inline int embed_id(const EmbedIds &s, int M, int m, bool first) {
  if (!s.table || m == 0) return s.ids[m];
  int step = *s.cursor;
  step = step < 0 ? 0 : (step >= s.n_steps ? s.n_steps - 1 : step);
  const int n = s.table[(int64_t)step * (M - 1) + m - 1];
  if (first) s.ids[m] = n;
  return n;
}

// The embedding's extras (a GEMV epilogue's STORE outputs): the next
// norm's prescaled half input and the sums of squares of each 4 values.
__device__ inline void embed_extras(const wg_epilogue &e, int m, int c0, const float *v) {
  if (e.out16) {
    uint16_t *o16 = e.out16 + (int64_t)m * e.ld_out16 + c0;
    for (int j = 0; j < 32; j++) o16[j] = half_bits(v[j] * e.out16_w[c0 + j] / e.norm_mult_out);
  }
  if (e.parts_out) {
    float *pp = e.parts_out + (int64_t)m * e.ld_parts_out + c0 / 4;
    for (int k = 0; k < 8; k++)
      pp[k] = v[4 * k] * v[4 * k] + v[4 * k + 1] * v[4 * k + 1] + v[4 * k + 2] * v[4 * k + 2] +
              v[4 * k + 3] * v[4 * k + 3];
  }
}

// Embedding rows of a ROWGROUP matrix: thread = (token m, 4 values of a
// block), 256 threads a workgroup (a constant: the workgroup size is not
// read from the dispatch's arguments before the first load). Values 4j ..
// 4j + 3 of a block are the low (j < 4) or high nibbles of its bytes
// 4 (j % 4) .. + 3: one 32-bit load a thread; its 4 outputs, prescaled
// halves and one sum of squares are the thread's own. The next norm's
// weights load ahead of the token id they do not depend on.
__global__ __launch_bounds__(256) void embed_rowgroup_kernel(
    const uint32_t *quants, const uint16_t *scales, const void *zeros, int zero_kind,
    const EmbedIds ids, int M, int blocks, int N, float *h, int ldh, const wg_epilogue e) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int quads = blocks * 8;
  if (t >= (int64_t)M * quads) return;
  const int m = (int)(t / quads), qd = (int)(t % quads);
  const int b = qd >> 3, j = qd & 7;
  const int c0 = b * 32 + 4 * j;  // the thread's first value
  float w16[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (e.out16)
#pragma unroll
    for (int i = 0; i < 4; i++) w16[i] = e.out16_w[c0 + i];
  const int n = embed_id(ids, M, m, qd == 0);
  float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (n >= 0 && n < N) {  // an id outside the vocabulary embeds as zeros
    const int64_t si = ((int64_t)(n >> 2) * blocks + b) * 4 + (n & 3);
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
    const uint32_t word = quants[si * 4 + (j & 3)];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t byte = (word >> (8 * i)) & 0xffu;
      const uint32_t nib = j < 4 ? (byte & 15u) : (byte >> 4);
      v[i] = (float)(d * ((double)nib - z));
    }
  }
  float *o = h + (int64_t)m * ldh + c0;
#pragma unroll
  for (int i = 0; i < 4; i++) o[i] = v[i];
  if (e.out16) {
    uint16_t *o16 = e.out16 + (int64_t)m * e.ld_out16 + c0;
#pragma unroll
    for (int i = 0; i < 4; i++) o16[i] = half_bits(v[i] * w16[i] / e.norm_mult_out);
  }
  if (e.parts_out)
    e.parts_out[(int64_t)m * e.ld_parts_out + c0 / 4] =
        v[0] * v[0] + v[1] * v[1] + v[2] * v[2] + v[3] * v[3];
}

// Embedding rows of a Q4_K matrix: thread = (token m, super-block s,
// sub-block j), with packQ4_K's (d', z') chain (src/repack.ts:100-168).
__global__ __launch_bounds__(256) void embed_q4k_kernel(const uint8_t *quants,
                                                        const EmbedIds ids, int M, int supers,
                                                        int N, float *h, int ldh,
                                                        const wg_epilogue e) {
  int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= (int64_t)M * supers * 8) return;
  int j = (int)(t & 7);
  int64_t ms = t >> 3;
  int m = (int)(ms / supers), s = (int)(ms % supers);
  int n = embed_id(ids, M, m, s == 0 && j == 0);
  float *o = h + (int64_t)m * ldh + s * 256 + j * 32;
  if (n < 0 || n >= N) {
    float zr[32] = {};
    for (int l = 0; l < 32; l++) o[l] = 0.0f;
    embed_extras(e, m, s * 256 + j * 32, zr);
    return;
  }
  const uint8_t *p = quants + (((int64_t)(n >> 2) * supers + s) * 4 + (n & 3)) * 144;
  double d = half_to_float((uint16_t)(p[0] | (p[1] << 8)));
  double dmin = half_to_float((uint16_t)(p[2] | (p[3] << 8)));
  int sc, mn;
  q4k_scale_min(p + 4, j, &sc, &mn);
  uint16_t hq = double_to_half_ref(d * sc);
  double mins = dmin * mn;
  bool constant = half_to_float(hq) == 0.0f;
  double scale = constant ? half_to_float(double_to_half_ref(-mins / 15.0)) : half_to_float(hq);
  double zero = constant ? 0.0 : half_to_float(double_to_half_ref(mins / scale));
  const uint8_t *q = p + 16 + (j >> 1) * 32;
  float v[32];
  for (int l = 0; l < 32; l++) {
    int nib = constant ? 15 : (j & 1) ? q[l] >> 4 : q[l] & 15;
    v[l] = (float)(scale * ((double)nib - zero));
    o[l] = v[l];
  }
  embed_extras(e, m, s * 256 + j * 32, v);
}

// Embedding rows of an 8-bit or Q6_K matrix: thread = (token m, 32-weight
// piece c), each piece dequantized as wg_q4_dequant does.
template <int LAYOUT>
__global__ void embed_wide_kernel(const uint8_t *quants, const uint16_t *scales,
                                  const EmbedIds ids, int M, int K, int N, float *h, int ldh,
                                  const wg_epilogue e) {
  const int pieces = K / 32;
  int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (int64_t)M * pieces) return;
  int m = (int)(t / pieces), c = (int)(t % pieces);
  int n = embed_id(ids, M, m, c == 0);
  float v[32];
  if (n < 0 || n >= N) {
    for (int j = 0; j < 32; j++) v[j] = 0.0f;
  } else if constexpr (LAYOUT == WG_LAYOUT_Q8) {
    dequant32_q8(reinterpret_cast<const int8_t *>(quants), scales, n, c, pieces, v);
  } else {
    const int supers = K / 256;
    const int64_t at = q6k_index(n, c >> 3, supers);
    dequant32_q6k(quants + at * 208, half_to_float(scales[at]), c & 7, v);
  }
  float *o = h + (int64_t)m * ldh + c * 32;
  for (int j = 0; j < 32; j++) o[j] = v[j];
  embed_extras(e, m, c * 32, v);
}

}  // namespace
}  // namespace wg

using namespace wg;

static int embed_rows(const wg_q4_matrix *emb, const EmbedIds &ids, int32_t M, float *h,
                      int32_t ldh, const wg_epilogue *ep, void *stream) {
  int rc = check_matrix(emb, "wg_embed");
  if (rc) return rc;
  WG_REQUIRE(ids.ids && h && M >= 1 && ldh >= emb->K, "wg_embed: bad arguments");
  wg_epilogue e = {};
  if (ep) e = *ep;
  if (e.out16)
    WG_REQUIRE(e.out16_w && e.ld_out16 >= emb->K && e.norm_mult_out != 0.0f,
               "wg_embed: the prescaled half output needs weights, a stride and a prescale");
  if (e.parts_out)
    WG_REQUIRE(e.ld_parts_out >= emb->K / 4, "wg_embed: parts stride too small");
  hipStream_t s = as_stream(stream);
  if (emb->layout == WG_LAYOUT_ROWGROUP) {
    int blocks = emb->K / 32;
    int64_t n = (int64_t)M * blocks * 8;
    embed_rowgroup_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(
        (const uint32_t *)emb->quants, (const uint16_t *)emb->scales, emb->zeros, emb->zero, ids,
        M, blocks, emb->N, h, ldh, e);
  } else if (emb->layout == WG_LAYOUT_Q8 || emb->layout == WG_LAYOUT_Q6K) {
    int64_t n = (int64_t)M * (emb->K / 32);
    auto kernel = emb->layout == WG_LAYOUT_Q8 ? embed_wide_kernel<WG_LAYOUT_Q8>
                                              : embed_wide_kernel<WG_LAYOUT_Q6K>;
    kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>((const uint8_t *)emb->quants,
                                                       (const uint16_t *)emb->scales, ids, M,
                                                       emb->K, emb->N, h, ldh, e);
  } else {
    int supers = emb->K / 256;
    int64_t n = (int64_t)M * supers * 8;
    embed_q4k_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(
        (const uint8_t *)emb->quants, ids, M, supers, emb->N, h, ldh, e);
  }
  return launched("wg_embed");
}

extern "C" {

int wg_rms_norm(const float *x, int32_t M, int32_t D, int32_t ldx, const float *w, float eps,
                uint16_t *out, int32_t ldo, float *rs_out, void *stream) {
  WG_REQUIRE(x && w && out, "wg_rms_norm: null argument");
  WG_REQUIRE(M >= 1 && D >= 4 && D % 4 == 0, "wg_rms_norm: %d rows of %d (a multiple of 4)", M,
             D);
  WG_REQUIRE(ldx >= D && ldx % 4 == 0 && ldo >= D && ldo % 4 == 0,
             "wg_rms_norm: strides %d, %d for rows of %d", ldx, ldo, D);
  WG_REQUIRE(((uintptr_t)x & 15) == 0 && ((uintptr_t)w & 15) == 0 && ((uintptr_t)out & 7) == 0,
             "wg_rms_norm: misaligned buffers");
  rms_norm_kernel<<<M, 256, 0, as_stream(stream)>>>(x, D, ldx, w, eps, out, ldo, rs_out);
  return launched("wg_rms_norm");
}

int wg_norm_to_h2(const float *x, int32_t M, int32_t D, int32_t ldx, const float *w, float eps,
                  uint16_t *out, int32_t ldo, float *row_scale, void *stream) {
  WG_REQUIRE(x && w && out && row_scale, "wg_norm_to_h2: null argument");
  WG_REQUIRE(M >= 1 && D >= 4 && D % 4 == 0 && ldx >= D && ldo >= D && ldx % 4 == 0 &&
                 ldo % 4 == 0,
             "wg_norm_to_h2: strides %d, %d for rows of %d", ldx, ldo, D);
  WG_REQUIRE(((uintptr_t)x & 15) == 0 && ((uintptr_t)w & 15) == 0 && ((uintptr_t)out & 7) == 0,
             "wg_norm_to_h2: misaligned buffers");
  norm_to_h2_kernel<<<M, 256, 0, as_stream(stream)>>>(x, D, ldx, w, eps, 32.0f, out, ldo,
                                                      row_scale);
  return launched("wg_norm_to_h2");
}

int wg_swiglu(const float *gu, int32_t M, int32_t F, int32_t ldg, uint16_t *out, int32_t ldo,
              void *stream) {
  WG_REQUIRE(gu && out, "wg_swiglu: null argument");
  WG_REQUIRE(M >= 1 && F >= 1 && ldg >= 2 * F && ldo >= F, "wg_swiglu: bad shape");
  int64_t n = (int64_t)M * F;
  swiglu_kernel<<<(unsigned)((n + 255) / 256), 256, 0, as_stream(stream)>>>(gu, M, F, ldg, out,
                                                                            ldo);
  return launched("wg_swiglu");
}


int wg_embed(const wg_q4_matrix *emb, const int32_t *ids, int32_t M, float *h, int32_t ldh,
             const wg_epilogue *ep, void *stream) {
  // (ids are only read without a table)
  return embed_rows(emb, EmbedIds{const_cast<int32_t *>(ids), nullptr, 0, nullptr}, M, h, ldh,
                    ep, stream);
}

int wg_embed_drafts(const wg_q4_matrix *emb, int32_t *ids, int32_t rows, const int32_t *table,
                    int32_t n_steps, const int32_t *cursor, float *h, int32_t ldh,
                    const wg_epilogue *ep, void *stream) {
  WG_REQUIRE(ids && table && cursor, "wg_embed_drafts: null argument");
  WG_REQUIRE(rows >= 2 && n_steps >= 1, "wg_embed_drafts: %d rows, %d table rows", rows, n_steps);
  return embed_rows(emb, EmbedIds{ids, table, n_steps, cursor}, rows, h, ldh, ep, stream);
}

}  // extern "C"
