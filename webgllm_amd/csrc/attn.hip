// Attention over the fp16 KV cache for decode and speculative verify.
//
// head_prep: the reference's headPrep + values (src/gpu/kernels.ts:2196-2322,
// :3030-3045): per head, optional RMS norm over head_dim, RoPE on the
// rotated dims (dim j pairs with j + R/2 at frequency j; the angle of
// pos = lo + 1024 hi is added from two rows of the table, as
// Engine.ropeTable builds it, src/engine.ts:1292-1312), times 1/sqrt(hd)
// for queries; keys and values go into the cache as halves.
//
// attn_decode: scores / attend / attendPanel (kernels.ts:2386-2579,
// :2803-3027) as split-K flash decoding: a workgroup takes one KV head and a
// chunk of 64 keys for every query row and every query head sharing that KV
// head (GQA: each key and value is read once for all of them), stages the
// K and V tiles in LDS, and writes the chunk's (max, sum of weights,
// weighted sum of values); a combine pass rescales the chunks by their
// running max (attendPanelCombine's online softmax) into half outputs.
// The position comes from device memory so a captured graph replays at any
// position; chunks past the last key leave at once.
#include "attn_core.h"
#include "common.h"
#include "dot.h"

namespace wg {
namespace {

constexpr int MAX_HD = 256;

__device__ inline uint16_t to_h(float v) {
  v = fminf(fmaxf(v, -65504.0f), 65504.0f);
  return __builtin_bit_cast(uint16_t, (_Float16)v);
}

// One wave per (row m, head slot): slots [0, H) queries, [H, H + KV) keys,
// [H + KV, H + 2 KV) values.
__global__ __launch_bounds__(64) void head_prep_kernel(
    const float *qkv, int ldq, int H, int KV, int hd, int R, float eps, int use_norm,
    const float *q_norm, const float *k_norm, const float *rope, int rope_rows,
    const int32_t *pos0_dev, float *q_out, int ldqo, uint16_t *k_cache, uint16_t *v_cache,
    int ctx) {
  const int slot = blockIdx.x, m = blockIdx.y, lane = threadIdx.x;
  const int pos = *pos0_dev + m;
  const float *x = qkv + (int64_t)m * ldq + (int64_t)slot * hd;
  const int kvd = KV * hd;
  if (pos < 0 || pos >= ctx || 1024 + (pos >> 10) >= rope_rows) {
    // A row past the cache has no position: its query is zero, nothing is stored.
    if (slot < H)
      for (int t = lane; t < hd; t += 64) q_out[(int64_t)m * ldqo + (int64_t)slot * hd + t] = 0.0f;
    return;
  }
  if (slot >= H + KV) {  // values: into the cache as they are
    uint16_t *vo = v_cache + (int64_t)pos * kvd + (int64_t)(slot - H - KV) * hd;
    for (int t = lane; t < hd; t += 64) vo[t] = to_h(x[t]);
    return;
  }
  const bool is_q = slot < H;
  const float *nw = is_q ? q_norm : k_norm;
  float inv = 1.0f;
  if (use_norm) {
    float s = 0.0f;
    for (int t = lane; t < hd; t += 64) s += x[t] * x[t];
    s = wave_sum(s);
    inv = 1.0f / sqrtf(s / (float)hd + eps);
  }
  const int P = R / 2;
  const int lo = pos & 1023, hi = 1024 + (pos >> 10);
  const float *r_lo = rope + (int64_t)lo * hd, *r_hi = rope + (int64_t)hi * hd;
  const float scale = is_q ? 1.0f / sqrtf((float)hd) : 1.0f;
  for (int t = lane; t < hd; t += 64) {
    float v = x[t] * (use_norm ? inv * nw[t] : 1.0f);
    float r = v;
    if (t < 2 * P) {
      bool first = t < P;
      int tp = first ? t + P : t - P;
      int f = first ? t : tp;
      float p = x[tp] * (use_norm ? inv * nw[tp] : 1.0f);
      float c1 = r_lo[f], s1 = r_lo[hd / 2 + f], c2 = r_hi[f], s2 = r_hi[hd / 2 + f];
      float cs = c1 * c2 - s1 * s2, sn = s1 * c2 + c1 * s2;
      r = first ? v * cs - p * sn : v * cs + p * sn;
    }
    if (is_q) {
      q_out[(int64_t)m * ldqo + (int64_t)slot * hd + t] = r * scale;
    } else {
      k_cache[(int64_t)pos * kvd + (int64_t)(slot - H) * hd + t] = to_h(r);
    }
  }
}

// Workgroup = (KV head kh, chunk c); chunks past the last key leave at once.
template <int HD>
__global__ __launch_bounds__(256) void attn_chunk_kernel(
    const float *q, int ldq, int M, int H, int KV, const uint16_t *k_cache,
    const uint16_t *v_cache, const int32_t *pos0_dev, int max_keys, float *partial, int chunks) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int pos0 = *pos0_dev;
  // The last row sees keys 0 .. pos0 + M - 1; never more than the cache holds.
  const int n_keys = min(pos0 + M, max_keys);
  if ((int)blockIdx.y * CHUNK >= n_keys) return;
  attn_chunk_item<HD>(q, ldq, M, H, KV, k_cache, v_cache, pos0, n_keys, blockIdx.x, blockIdx.y,
                      partial, chunks, smem);
}

// One workgroup of 256 per (query head h, row m): the chunks' online-softmax
// combine. Lanes take chunks for the running max and the weights
// exp(m_c - max); then each thread sums one dim over the chunks, whose loads
// are independent (no chain through the chunk loop).
__global__ __launch_bounds__(256) void attn_combine_kernel(const float *partial, int M, int H,
                                                           int hd, int chunks,
                                                           const int32_t *pos0_dev,
                                                           int max_keys, uint16_t *out, int ldo) {
  __shared__ float wts[4096 / CHUNK * 16];
  __shared__ float red[8];
  const int h = blockIdx.x, m = blockIdx.y, tid = threadIdx.x;
  const int n_keys = min(*pos0_dev + m + 1, max_keys);  // keys row m sees
  uint16_t *o = out + (int64_t)m * ldo + (int64_t)h * hd;
  if (n_keys <= 0) {
    for (int d = tid; d < hd; d += 256) o[d] = 0;
    return;
  }
  const int used = (n_keys + CHUNK - 1) / CHUNK;
  const int row = m * H + h;
  PartialLayout pl{hd, chunks};
  float mx = -INFINITY;
  for (int c = tid; c < used; c += 256) mx = fmaxf(mx, partial[pl.base(row, c)]);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  if ((tid & 63) == 0) red[tid >> 6] = mx;
  __syncthreads();
  const float gmax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  float l = 0.0f;
  for (int c = tid; c < used; c += 256) {
    const float *p = partial + pl.base(row, c);
    float w = p[0] == -INFINITY ? 0.0f : __expf(p[0] - gmax);
    if (c < (int)(sizeof(wts) / sizeof(float))) wts[c] = w;
    l += w * p[1];
  }
  l = wave_sum(l);
  __syncthreads();
  if ((tid & 63) == 0) red[4 + (tid >> 6)] = l;
  __syncthreads();
  const float inv = 1.0f / (red[4] + red[5] + red[6] + red[7]);
  const int cap = (int)(sizeof(wts) / sizeof(float));
  for (int d = tid; d < hd; d += 256) {
    float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
    int c = 0;
    for (; c + 4 <= used; c += 4) {
      float w0, w1, w2, w3;
      if (c + 3 < cap) {
        w0 = wts[c]; w1 = wts[c + 1]; w2 = wts[c + 2]; w3 = wts[c + 3];
      } else {
        const float *q = partial + pl.base(row, c);
        w0 = q[0] == -INFINITY ? 0.0f : __expf(q[0] - gmax);
        q += hd + 2;
        w1 = q[0] == -INFINITY ? 0.0f : __expf(q[0] - gmax);
        q += hd + 2;
        w2 = q[0] == -INFINITY ? 0.0f : __expf(q[0] - gmax);
        q += hd + 2;
        w3 = q[0] == -INFINITY ? 0.0f : __expf(q[0] - gmax);
      }
      a0 += w0 * partial[pl.base(row, c) + 2 + d];
      a1 += w1 * partial[pl.base(row, c + 1) + 2 + d];
      a2 += w2 * partial[pl.base(row, c + 2) + 2 + d];
      a3 += w3 * partial[pl.base(row, c + 3) + 2 + d];
    }
    for (; c < used; c++) {
      const float *q = partial + pl.base(row, c);
      float w = c < cap ? wts[c] : (q[0] == -INFINITY ? 0.0f : __expf(q[0] - gmax));
      a0 += w * q[2 + d];
    }
    o[d] = to_h((a0 + a1 + a2 + a3) * inv);
  }
}

}  // namespace
}  // namespace wg

using namespace wg;

extern "C" {

int wg_head_prep(const float *qkv, int32_t M, int32_t ldq, const wg_attn_shape *sh,
                 const float *q_norm, const float *k_norm, const float *rope, int32_t rope_rows,
                 const int32_t *pos0, float *q_out, int32_t ldqo, uint16_t *k_cache,
                 uint16_t *v_cache, int32_t ctx, void *stream) {
  WG_REQUIRE(sh && qkv && rope && pos0 && q_out && k_cache && v_cache,
             "wg_head_prep: null argument");
  WG_REQUIRE(M >= 1 && M <= 65535, "wg_head_prep: %d rows", M);
  WG_REQUIRE(sh->kv_heads > 0 && sh->heads % sh->kv_heads == 0,
             "wg_head_prep: %d query heads over %d KV heads", sh->heads, sh->kv_heads);
  WG_REQUIRE(sh->head_dim >= 2 && sh->head_dim <= MAX_HD && sh->head_dim % 2 == 0,
             "wg_head_prep: head_dim %d", sh->head_dim);
  WG_REQUIRE(sh->rotated_dims >= 0 && sh->rotated_dims <= sh->head_dim &&
                 sh->rotated_dims % 2 == 0,
             "wg_head_prep: rotated dims %d", sh->rotated_dims);
  WG_REQUIRE(!sh->use_norm || (q_norm && k_norm), "wg_head_prep: norm weights missing");
  WG_REQUIRE(ctx >= 1 && rope_rows >= 1024 + (ctx + 1023) / 1024,
             "wg_head_prep: a rope table of %d rows for a %d-position cache (needs %d)",
             rope_rows, ctx, 1024 + (ctx + 1023) / 1024);
  int slots = sh->heads + 2 * sh->kv_heads;
  WG_REQUIRE(ldq >= slots * sh->head_dim && ldqo >= sh->heads * sh->head_dim,
             "wg_head_prep: strides too small");
  head_prep_kernel<<<dim3(slots, M), 64, 0, as_stream(stream)>>>(
      qkv, ldq, sh->heads, sh->kv_heads, sh->head_dim, sh->rotated_dims, sh->eps, sh->use_norm,
      q_norm, k_norm, rope, rope_rows, pos0, q_out, ldqo, k_cache, v_cache, ctx);
  return launched("wg_head_prep");
}

size_t wg_attn_scratch_bytes(int32_t M, int32_t heads, int32_t head_dim, int32_t max_keys) {
  int64_t chunks = (max_keys + CHUNK - 1) / CHUNK;
  return (size_t)M * heads * chunks * (head_dim + 2) * sizeof(float);
}

int wg_attn_decode(const float *q, int32_t M, int32_t ldq, const wg_attn_shape *sh,
                   const uint16_t *k_cache, const uint16_t *v_cache, const int32_t *pos0,
                   int32_t max_keys, uint16_t *out, int32_t ldo, void *scratch,
                   size_t scratch_bytes, void *stream) {
  WG_REQUIRE(sh && q && k_cache && v_cache && pos0 && out && scratch,
             "wg_attn_decode: null argument");
  int H = sh->heads, KV = sh->kv_heads, hd = sh->head_dim;
  WG_REQUIRE(KV > 0 && H % KV == 0, "wg_attn_decode: %d query heads over %d KV heads", H, KV);
  WG_REQUIRE(M >= 1 && (H / KV) * M <= 64,
             "wg_attn_decode: %d rows x %d heads per KV head (at most 64)", M, H / KV);
  WG_REQUIRE(hd == 64 || hd == 128, "wg_attn_decode: head_dim %d (64 or 128)", hd);
  WG_REQUIRE(max_keys >= M, "wg_attn_decode: max_keys %d < rows %d", max_keys, M);
  WG_REQUIRE(ldq >= H * hd && ldo >= H * hd, "wg_attn_decode: strides too small");
  WG_REQUIRE(scratch_bytes >= wg_attn_scratch_bytes(M, H, hd, max_keys),
             "wg_attn_decode: scratch of %zu bytes, %zu needed", scratch_bytes,
             wg_attn_scratch_bytes(M, H, hd, max_keys));
  int chunks = (max_keys + CHUNK - 1) / CHUNK;
  hipStream_t s = as_stream(stream);
  size_t lds = attn_lds_bytes((H / KV) * M, hd);
  static bool raised = false;  // allow more than 64 KiB of dynamic LDS, once
  if (!raised) {
    WG_HIP(hipFuncSetAttribute((const void *)attn_chunk_kernel<64>,
                               hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
    WG_HIP(hipFuncSetAttribute((const void *)attn_chunk_kernel<128>,
                               hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
    raised = true;
  }
  if (hd == 64)
    attn_chunk_kernel<64><<<dim3(KV, chunks), 256, lds, s>>>(
        q, ldq, M, H, KV, k_cache, v_cache, pos0, max_keys, (float *)scratch, chunks);
  else
    attn_chunk_kernel<128><<<dim3(KV, chunks), 256, lds, s>>>(
        q, ldq, M, H, KV, k_cache, v_cache, pos0, max_keys, (float *)scratch, chunks);
  int rc = launched("wg_attn_decode");
  if (rc) return rc;
  attn_combine_kernel<<<dim3(H, M), 256, 0, s>>>((const float *)scratch, M, H, hd, chunks, pos0,
                                                 max_keys, out, ldo);
  return launched("wg_attn_decode (combine)");
}

}  // extern "C"
