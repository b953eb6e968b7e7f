// Decode attention pieces shared by the attention kernels and the
// persistent decode kernel: one (KV head, key chunk) item of split-K flash
// decoding, and the combine of a KV head's query heads over its chunks
// (the online softmax of the reference's attendPanel / attendPanelCombine,
// src/gpu/kernels.ts:2803-3027).
#pragma once

#include "common.h"
#include "dot.h"
#include "epilogue.h"

namespace wg {

constexpr int CHUNK = 64;  // keys an item takes

// Head preparation's arithmetic (the reference's headPrep,
// src/gpu/kernels.ts:2196-2322), shared by head_prep_kernel and the decode
// attention that prepares its own heads, so that both give the same bits.
// The norm's sum of squares runs in one fixed order: per c = 0..3 the
// dims 32 t + 8 c + e (e = 0..7 fastest, then t), as fmas from zero, then
// (S0 + S1) + (S2 + S3).
__device__ inline float head_norm_inv(float total, int hd, float eps) {
  return 1.0f / sqrtf(total / (float)hd + eps);
}
// The rotation of v by its partner p: cos and sin of the position's low
// (c1, s1) and high (c2, s2) table rows combined by angle addition.
__device__ inline float rope_rotate(float v, float p, bool first, float c1, float s1, float c2,
                                    float s2) {
  const float cs = __builtin_fmaf(c1, c2, -(s1 * s2)), sn = __builtin_fmaf(s1, c2, c1 * s2);
  return first ? __builtin_fmaf(v, cs, -(p * sn)) : __builtin_fmaf(v, cs, p * sn);
}

// LDS bytes attn_chunk_item needs for GM queries of head_dim hd.
__host__ __device__ constexpr size_t attn_lds_bytes(int GM, int hd) {
  return (size_t)2 * CHUNK * (hd + 2) * 2 + (size_t)GM * hd * 4 + (size_t)GM * CHUNK * 4 +
         (size_t)GM * 8;
}

// Partial results of one (query row, query head, chunk): the chunk's max
// score, its sum of exp(score - max), and the weighted values.
struct PartialLayout {
  int hd, chunks;
  __device__ int64_t base(int qh_row, int chunk) const {
    return ((int64_t)qh_row * chunks + chunk) * (hd + 2);
  }
};

// One (KV head kh, chunk c) item for a workgroup of NT threads: queries are rows
// m < M of heads kh * G .. kh * G + G - 1, GM = G * M of them; n_keys (> c *
// CHUNK) keys are visible to the last row. smem holds attn_lds_bytes(GM,
// HD): K and V tiles, the queries, the chunk's scores, and per query its
// max and sum of weights. Every thread of the workgroup calls it.
template <int HD, int NT = 256>
__device__ inline void attn_chunk_item(const float *q, int ldq, int M, int H, int KV,
                                       const uint16_t *k_cache, const uint16_t *v_cache,
                                       int pos0, int n_keys, int kh, int c, float *partial,
                                       int chunks, unsigned char *smem) {
  constexpr int KSTR = HD + 2;  // LDS row stride in halves (breaks bank conflicts)
  const int GMq = (H / KV) * M;
  uint16_t *ks = reinterpret_cast<uint16_t *>(smem);
  uint16_t *vs = ks + CHUNK * KSTR;
  float *qs = reinterpret_cast<float *>(vs + CHUNK * KSTR);
  float *sc = qs + GMq * HD;
  float *mx = sc + GMq * CHUNK;
  float *lsum = mx + GMq;
  const int tid = threadIdx.x;
  const int j0 = c * CHUNK;
  const int G = H / KV, GM = G * M;
  const int kvd = KV * HD;
  const int nk = min(CHUNK, n_keys - j0);
  // Stage K and V rows j0 .. j0 + nk - 1 of head kh: 16-byte pieces.
  constexpr int PIECES = HD / 8;
  for (int i = tid; i < nk * PIECES; i += NT) {
    int r = i / PIECES, p = i % PIECES;
    const uint4 *kp = reinterpret_cast<const uint4 *>(k_cache + (int64_t)(j0 + r) * kvd + kh * HD);
    const uint4 *vp = reinterpret_cast<const uint4 *>(v_cache + (int64_t)(j0 + r) * kvd + kh * HD);
    uint4 kv = kp[p], vv = vp[p];
    uint32_t *kd = reinterpret_cast<uint32_t *>(ks + r * KSTR + p * 8);
    uint32_t *vd = reinterpret_cast<uint32_t *>(vs + r * KSTR + p * 8);
    kd[0] = kv.x; kd[1] = kv.y; kd[2] = kv.z; kd[3] = kv.w;
    vd[0] = vv.x; vd[1] = vv.y; vd[2] = vv.z; vd[3] = vv.w;
  }
  for (int i = tid; i < GM * HD; i += NT) {
    int qi = i / HD, d = i % HD;
    int g = qi % G, m = qi / G;
    qs[i] = q[(int64_t)m * ldq + (int64_t)(kh * G + g) * HD + d];
  }
  __syncthreads();
  // Scores, causal: row m sees keys j <= pos0 + m.
  for (int i = tid; i < GM * CHUNK; i += NT) {
    int qi = i / CHUNK, r = i % CHUNK;
    int m = qi / G;
    float s = -INFINITY;
    if (r < nk && j0 + r <= pos0 + m) {
      const float *qv = qs + qi * HD;
      const uint16_t *kr = ks + r * KSTR;
      float a = 0.0f;
#pragma unroll 8
      for (int d = 0; d < HD; d += 2) {
        uint32_t k2 = *reinterpret_cast<const uint32_t *>(kr + d);
        half2v kk = as_h2(k2);
        a = __builtin_fmaf(qv[d], (float)kk.x, a);
        a = __builtin_fmaf(qv[d + 1], (float)kk.y, a);
      }
      s = a;
    }
    sc[i] = s;
  }
  __syncthreads();
  // Per query: the chunk's max and sum of weights (one wave per query).
  const int wave = tid >> 6, lane = tid & 63;
  for (int qi = wave; qi < GM; qi += NT / 64) {
    float v = lane < CHUNK ? sc[qi * CHUNK + lane] : -INFINITY;
    float m_ = v;
    m_ = wave_max(m_);
    float e = (m_ == -INFINITY || v == -INFINITY) ? 0.0f : __expf(v - m_);
    if (lane < CHUNK) sc[qi * CHUNK + lane] = e;
    float l = wave_sum(e);
    if (lane == 0) {
      mx[qi] = m_;
      lsum[qi] = l;
    }
  }
  __syncthreads();
  // Weighted values.
  PartialLayout pl{HD, chunks};
  for (int i = tid; i < GM * HD; i += NT) {
    int qi = i / HD, d = i % HD;
    const float *e = sc + qi * CHUNK;
    float a = 0.0f;
    for (int r = 0; r < nk; r++) {
      half2v vv = as_h2(*reinterpret_cast<const uint32_t *>(vs + r * KSTR + (d & ~1)));
      a = __builtin_fmaf(e[r], (float)((d & 1) ? vv.y : vv.x), a);
    }
    int g = qi % G, m = qi / G;
    int row = m * H + kh * G + g;
    float *out = partial + pl.base(row, c);
    out[2 + d] = a;
    if (d == 0) {
      out[0] = mx[qi];
      out[1] = lsum[qi];
    }
  }
}


// The combine of every query head of KV head kh (rows m < M) over the
// chunks of ck keys into half outputs: running max over the
// chunks, weights exp(m_c - max), sum of weights times the chunks' sums,
// then each output dim as the weighted sum of the chunks' values (a
// workgroup of NT threads). lds holds
// 2 GM used + GM floats, used = the chunks of the last row's keys.
template <int HD, int NT = 256>
__device__ inline void attn_combine_group(const float *partial, int chunks, int M, int H, int KV,
                                          int kh, int pos0, int max_keys, uint16_t *out,
                                          int ldo, float *lds, int ck = CHUNK) {
  const int G = H / KV, GM = G * M, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int n_all = min(pos0 + M, max_keys);
  const int used_all = n_all > 0 ? (n_all + ck - 1) / ck : 0;
  float *wts = lds, *ls = lds + GM * used_all, *inv = ls + GM * used_all;
  PartialLayout pl{HD, chunks};
  for (int i = tid; i < GM * used_all; i += NT) {
    int qi = i / used_all, c = i % used_all;
    int g = qi % G, m = qi / G;
    const float *pp = partial + pl.base(m * H + kh * G + g, c);
    wts[i] = pp[0];
    ls[i] = pp[1];
  }
  __syncthreads();
  for (int qi = wave; qi < GM; qi += NT / 64) {
    const int m = qi / G;
    const int nk = min(pos0 + m + 1, max_keys);  // keys row m sees
    const int used = nk > 0 ? (nk + ck - 1) / ck : 0;
    float *w = wts + qi * used_all;
    float mx = -INFINITY;
    for (int c = lane; c < used; c += 64) mx = fmaxf(mx, w[c]);
    mx = wave_max(mx);
    float l = 0.0f;
    for (int c = lane; c < used_all; c += 64) {
      float v = w[c];
      float e = (c >= used || v == -INFINITY) ? 0.0f : __expf(v - mx);
      w[c] = e;
      l += e * ls[qi * used_all + c];
    }
    l = wave_sum(l);
    if (lane == 0) inv[qi] = l > 0.0f ? 1.0f / l : 0.0f;
  }
  __syncthreads();
  for (int i = tid; i < GM * HD; i += NT) {
    const int qi = i / HD, d = i % HD;
    const int g = qi % G, m = qi / G;
    const float *pp = partial + pl.base(m * H + kh * G + g, 0) + 2 + d;
    const float *w = wts + qi * used_all;
    float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
    int c = 0;
    for (; c + 4 <= used_all; c += 4) {
      a0 = __builtin_fmaf(w[c], pp[(int64_t)c * (HD + 2)], a0);
      a1 = __builtin_fmaf(w[c + 1], pp[(int64_t)(c + 1) * (HD + 2)], a1);
      a2 = __builtin_fmaf(w[c + 2], pp[(int64_t)(c + 2) * (HD + 2)], a2);
      a3 = __builtin_fmaf(w[c + 3], pp[(int64_t)(c + 3) * (HD + 2)], a3);
    }
    for (; c < used_all; c++) a0 = __builtin_fmaf(w[c], pp[(int64_t)c * (HD + 2)], a0);
    out[(int64_t)m * ldo + (int64_t)(kh * G + g) * HD + d] =
        half_bits(((a0 + a1) + (a2 + a3)) * inv[qi]);
  }
}

}  // namespace wg
