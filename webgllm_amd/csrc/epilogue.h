// The GEMV epilogues (see wg_epilogue in include/webgllm_hip.h). The sums
// arrive in the wave_sum4 layout: lanes 16 r .. 16 r + 15 hold row 4g + r of
// every token (tot[m], in units of 2^-24); lane 16 r + m writes token m.
#pragma once

#include "common.h"
#include "dot.h"
#include "pick_core.h"

namespace wg {

__device__ inline uint16_t half_bits(float v) {
  v = fminf(fmaxf(v, -65504.0f), 65504.0f);
  return __builtin_bit_cast(uint16_t, (_Float16)v);
}

// The per-token factor: the input's 1 / RMS (times the producer's prescale)
// and row_scale. Every lane of the wave takes part; all get the result.
template <int M>
__device__ inline void input_scales(const wg_epilogue &e, float s[M]) {
  const int lane = threadIdx.x & 63;
  float a[M];
#pragma unroll
  for (int m = 0; m < M; m++) a[m] = 0.0f;
  if (e.norm_parts) {  // the M tokens' loads together, each token's sums in order
    const float *p = e.norm_parts;
    // 16-byte loads where the parts are 16-byte aligned (the usual case).
    if ((((uintptr_t)p) & 15) == 0 && (e.n_parts & 3) == 0 && (e.ld_parts_in & 3) == 0) {
      for (int i = lane; i < (e.n_parts >> 2); i += 64) {
        float4 t[M];
#pragma unroll
        for (int m = 0; m < M; m++)
          t[m] = reinterpret_cast<const float4 *>(p + (int64_t)m * e.ld_parts_in)[i];
#pragma unroll
        for (int m = 0; m < M; m++) a[m] += (t[m].x + t[m].y) + (t[m].z + t[m].w);
      }
    } else {
      for (int i = lane; i < e.n_parts; i += 64) {
        float t[M];
#pragma unroll
        for (int m = 0; m < M; m++) t[m] = p[(int64_t)m * e.ld_parts_in + i];
#pragma unroll
        for (int m = 0; m < M; m++) a[m] += t[m];
      }
    }
  }
#pragma unroll
  for (int m = 0; m < M; m++) {
    float v = 1.0f;
    if (e.norm_parts) {
      const float sum = wave_sum(a[m]);
      v = e.norm_mult / sqrtf(sum / (float)e.norm_count + e.eps);
    }
    if (e.row_scale) v *= e.row_scale[m];
    s[m] = v;
  }
}

// input_scales computed by a workgroup of NW waves together: wave w sums
// the 16-byte pieces w, w + NW, ... of the parts, and the waves' sums meet
// in LDS (`lds`: NW * M floats), so a workgroup reads the parts once rather
// than once a wave (every wave of every workgroup reads the same lines at
// the kernel's start). Every thread of the workgroup calls it: it holds a
// barrier.
template <int M, int NW>
__device__ inline void input_scales_wg(const wg_epilogue &e, float s[M], float *lds, int mr = M) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (e.norm_parts) {
    // The M tokens' loads go out together (a token at a time, each waited
    // for its loads and wave sum before the next began); each token's sums
    // keep their order, so the results are unchanged.
    float a[M];
#pragma unroll
    for (int m = 0; m < M; m++) a[m] = 0.0f;
    const float *p = e.norm_parts;
    if ((((uintptr_t)p) & 15) == 0 && (e.n_parts & 3) == 0 && (e.ld_parts_in & 3) == 0) {
      for (int i = wave * 64 + lane; i < (e.n_parts >> 2); i += NW * 64) {
        float4 t[M];
#pragma unroll
        for (int m = 0; m < M; m++)
          t[m] = m < mr ? reinterpret_cast<const float4 *>(p + (int64_t)m * e.ld_parts_in)[i]
                        : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
        for (int m = 0; m < M; m++) a[m] += (t[m].x + t[m].y) + (t[m].z + t[m].w);
      }
    } else {
      for (int i = wave * 64 + lane; i < e.n_parts; i += NW * 64) {
        float t[M];
#pragma unroll
        for (int m = 0; m < M; m++) t[m] = m < mr ? p[(int64_t)m * e.ld_parts_in + i] : 0.0f;
#pragma unroll
        for (int m = 0; m < M; m++) a[m] += t[m];
      }
    }
#pragma unroll
    for (int m = 0; m < M; m++) {
      const float sum = wave_sum(a[m]);
      if (lane == 0) lds[wave * M + m] = sum;
    }
    __syncthreads();
  }
#pragma unroll
  for (int m = 0; m < M; m++) {
    float v = 1.0f;
    if (e.norm_parts) {
      float a = 0.0f;
#pragma unroll
      for (int w = 0; w < NW; w++) a += lds[w * M + m];
      v = e.norm_mult / sqrtf(a / (float)e.norm_count + e.eps);
    }
    if (e.row_scale) v *= e.row_scale[m < mr ? m : 0];
    s[m] = v;
  }
}

// The epilogue's operands of one row group that do not depend on its sums,
// loaded ahead (with the row group's weights) so the epilogue does not wait
// for memory: the residual and the next norm's weight (STORE), the rope
// table entries of the lane's dim at its position (ROPE_KV), the lane's
// channel's taps and state (SHORT_CONV).
constexpr int CONV_MAX_W = 4;
struct EpiPre {
  float res, w16;
  float c1, s1, c2, s2;
  float tp[CONV_MAX_W], st[CONV_MAX_W - 1];
};

// (SHORT_CONV) channel c's taps and state, for the lane's row r of a row
// group of x rows.
__device__ inline void conv_prefetch(const wg_epilogue &e, int c, int D, bool live, EpiPre &p) {
  const int W = e.conv_width;
#pragma unroll
  for (int k = 0; k < CONV_MAX_W; k++) p.tp[k] = live && k < W ? e.conv_taps[(int64_t)c * W + k] : 0.0f;
#pragma unroll
  for (int i = 0; i < CONV_MAX_W - 1; i++)
    p.st[i] = live && i < W - 1 ? e.conv_state[(int64_t)i * D + c] : 0.0f;
}

// (SHORT_CONV) channel c's outputs for the lane's token m = lane % 16, from
// its B, C and x sums (bv, cv, xv, final): y = B x, the window of the last W
// y's from the lanes of the earlier tokens (lane - d) and the state, then
// what short_conv_kernel computes, in its order. Every lane of the wave
// takes part (the window's shuffles); `live`: the channel and token exist.
__device__ inline void conv_finish(const wg_epilogue &e, int c, int D, int M, float bv, float cv,
                                   float xv, bool live, const EpiPre &p) {
  const int lane = threadIdx.x & 63, m = lane & 15;
  const int W = e.conv_width;
  const float y = bv * xv;
  // y of token m - d, d < CONV_MAX_W, from the lane d lanes down (its own
  // 16-lane group when m >= d)
  float sh[CONV_MAX_W];
  sh[0] = y;
#pragma unroll
  for (int d = 1; d < CONV_MAX_W; d++) sh[d] = __shfl(y, (lane - d) & 63, 64);
  // the window: yw[k] = y of token t = m - (W - 1) + k; before the batch
  // (t < 0) state row W - 1 + t = m + k, oldest first
  float yw[CONV_MAX_W];
#pragma unroll
  for (int k = 0; k < CONV_MAX_W; k++) {
    const int d = W - 1 - k;
    float v = 0.0f;
#pragma unroll
    for (int dd = 0; dd < CONV_MAX_W; dd++)
      if (dd == d) v = sh[dd];
    if (m < d) {
#pragma unroll
      for (int i = 0; i < CONV_MAX_W - 1; i++)
        if (i == m + k) v = p.st[i];
    }
    yw[k] = v;
  }
  float a = 0.0f;
#pragma unroll
  for (int k = 0; k < CONV_MAX_W; k++)
    if (k < W) a += p.tp[k] * yw[k];
  if (!live) return;
  e.out16[(int64_t)m * e.ld_out16 + c] = half_bits(cv * a);
  if (e.conv_prefixes)  // the state after the first m + 1 tokens
#pragma unroll
    for (int i = 0; i < CONV_MAX_W - 1; i++)
      if (i < W - 1) e.conv_prefixes[((int64_t)m * (W - 1) + i) * D + c] = yw[i + 1];
  if (m == M - 1)
#pragma unroll
    for (int i = 0; i < CONV_MAX_W - 1; i++)
      if (i < W - 1) e.conv_state_out[(int64_t)i * D + c] = yw[i + 1];
}

// The position the epilogue uses (ROPE_KV), read once per kernel.
template <int MODE>
__device__ inline int epi_pos0(const wg_epilogue &e) {
  if constexpr (MODE == WG_EPI_ROPE_KV) return *e.pos0;
  return 0;
}

// Row (4 g + r, r = lane / 16 % 4) for token m = lane % 16 (m < M): the
// operands finish<M, MODE> needs. g >= G loads nothing.
template <int M, int MODE>
__device__ inline void epi_prefetch(const wg_epilogue &e, int g, int G, int pos0, EpiPre &p,
                                    int mr = M) {
  const int lane = threadIdx.x & 63;
  const int r = (lane >> 4) & 3, m = lane & 15;
  const bool live = g < G && m < mr;
  const int n = 4 * g + r;
  p.res = p.w16 = p.c1 = p.s1 = p.c2 = p.s2 = 0.0f;
  if constexpr (MODE == WG_EPI_STORE) {
    if (live && e.residual) p.res = e.residual[(int64_t)m * e.ld_residual + n];
    if (live && e.out16) p.w16 = e.out16_w[n];
  } else if constexpr (MODE == WG_EPI_ROPE_KV) {
    const int hd = e.head_dim, P = hd / 2;
    const int qd = e.heads * hd, kd = e.kv_heads * hd;
    const int row = 4 * g;
    const int pos = live ? pos0 + m : -1;
    const bool in_cache = pos >= 0 && pos < e.ctx && 1024 + (pos >> 10) < e.rope_rows;
    if (in_cache && row < qd + kd) {
      const int base = row < qd ? 0 : qd;
      const int i = ((row - base) % hd) / 4;
      const int f = (2 * i + (r >> 1) + ((r & 1) ? P : 0)) % P;
      const float *r_lo = e.rope + (int64_t)(pos & 1023) * hd;
      const float *r_hi = e.rope + (int64_t)(1024 + (pos >> 10)) * hd;
      p.c1 = r_lo[f];
      p.s1 = r_lo[P + f];
      p.c2 = r_hi[f];
      p.s2 = r_hi[P + f];
    }
  }
}

// Picks tot[m] for this lane's token without dynamic register indexing:
// a chain of selects on constant indices, written as a compile-time
// recursion (a loop over i, not yet unrolled when the compiler looks for
// dynamically indexed arrays, moved the M floats into LDS from M = 3 on).
template <int M, int I = 0>
__device__ inline float pick(const float (&tot)[M], int m) {
  if constexpr (I + 1 >= M) {
    return tot[I];
  } else {
    return m == I ? tot[I] : pick<M, I + 1>(tot, m);
  }
}

// Row group g's four rows for tokens 0..M-1, with the operands
// epi_prefetch<M, MODE> loaded for g. Called by every lane of the wave (the
// shuffles need all of them), with g >= G for idle waves.
template <int MODE>
__device__ inline void finish_value(const wg_epilogue &e, int g, float v, bool live, float *y,
                                    int ldy, const EpiPre &pre, int pos0);

template <int M, int MODE>
__device__ inline void finish(const wg_epilogue &e, int g, int G, const float (&tot)[M],
                              const float (&scale)[M], float *y, int ldy, const EpiPre &pre,
                              int pos0) {
  const int m = threadIdx.x & 15;
  const int mm = m < M ? m : 0;
  const float v = pick<M>(tot, mm) * 0x1p24f * pick<M>(scale, mm);  // (an index would put scale in LDS)
  finish_value<MODE>(e, g, v, g < G && m < M, y, ldy, pre, pos0);
}

// Row 4 g + r (r = lane / 16 % 4) of token m = lane % 16 is v (final, before
// the epilogue's own operation); `live`: the row and token exist. Called by
// every lane of the wave.
template <int MODE>
__device__ inline void finish_value(const wg_epilogue &e, int g, float v, bool live, float *y,
                                    int ldy, const EpiPre &pre, int pos0) {
  const int lane = threadIdx.x & 63;
  const int r = (lane >> 4) & 3, m = lane & 15;
  const int n = 4 * g + r;
  if constexpr (MODE == WG_EPI_STORE) {
    if (live && e.residual) v += pre.res;
    if (live && y) y[(int64_t)m * ldy + n] = v;
    if (live && e.out16)
      e.out16[(int64_t)m * e.ld_out16 + n] = half_bits(v * pre.w16 / e.norm_mult_out);
    if (e.parts_out) {
      float sq = live ? v * v : 0.0f;
      sq += xor16(sq);
      sq += xor32(sq);
      if (live && r == 0) e.parts_out[(int64_t)m * e.ld_parts_out + g] = sq;
    }
  } else if constexpr (MODE == WG_EPI_SWIGLU) {
    // rows (gate 2i, gate 2i + 1, up 2i, up 2i + 1): row r < 2 meets row r + 2
    float up = xor32(v);
    if (live && r < 2) {
      float gate = v;
      float o = gate / (1.0f + __expf(-gate)) * up;
      e.out16[(int64_t)m * e.ld_out16 + 2 * g + r] = half_bits(o);
    }
  } else {  // WG_EPI_ROPE_KV
    const int hd = e.head_dim, P = hd / 2;
    const int qd = e.heads * hd, kd = e.kv_heads * hd;
    float partner = xor16(v);  // rows 0 <-> 1 and 2 <-> 3
    const int row = 4 * g;
    int pos = live ? pos0 + m : -1;
    bool in_cache = pos >= 0 && pos < e.ctx && 1024 + (pos >> 10) < e.rope_rows;
    if (row < qd + kd) {
      const bool is_q = row < qd;
      const int base = is_q ? 0 : qd;
      const int head = (row - base) / hd;
      const int i = ((row - base) % hd) / 4;
      // dims of rows r = 0..3: 2i, 2i + P, 2i + 1, 2i + 1 + P
      const int d = 2 * i + (r >> 1) + ((r & 1) ? P : 0);
      const bool first = (r & 1) == 0;
      float o = 0.0f;
      if (in_cache) {
        float cs = pre.c1 * pre.c2 - pre.s1 * pre.s2, sn = pre.s1 * pre.c2 + pre.c1 * pre.s2;
        o = first ? v * cs - partner * sn : v * cs + partner * sn;
      }
      if (live) {
        if (is_q)
          e.q_out[(int64_t)m * e.ld_q_out + (int64_t)head * hd + d] =
              in_cache ? o * (1.0f / sqrtf((float)hd)) : 0.0f;
        else if (in_cache)
          e.k_cache[(int64_t)pos * kd + (int64_t)head * hd + d] = half_bits(o);
      }
    } else if (live && in_cache) {
      const int dv = row - qd - kd + r;
      e.v_cache[(int64_t)pos * kd + dv] = half_bits(v);
    }
  }
}

// (pick_parts) Row n's stored value v of the lane's token into the lane's
// running best: only values above the scan's floor enter (NaN never does).
__device__ inline void pick_take(PickBest &b, float v, int n, bool live) {
  if (live && v > PICK_FLOOR) b = pick_better(b, PickBest{v, n});
}

// (pick_parts) The workgroup's best of every token into its slot: the lanes
// of a token (lane % 16, rows lane / 16 % 4) merged by swaps, then the W
// waves through LDS. Every thread of the workgroup calls it.
template <int W>
__device__ inline void pick_flush(const wg_epilogue &e, PickBest b, int M,
                                  PickBest (&lds)[W][16]) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  b = pick_xor(b, 16);
  b = pick_xor(b, 32);
  if (lane < 16) lds[wave][lane] = b;
  __syncthreads();
  if (wave == 0 && lane < M) {
    PickBest t = lds[0][lane];
#pragma unroll
    for (int w = 1; w < W; w++) t = pick_better(t, lds[w][lane]);
    auto *parts = reinterpret_cast<PickBest *>(static_cast<char *>(e.pick_parts) + PICK_HEADER);
    parts[(int64_t)lane * WG_PICK_SLOTS + blockIdx.x] = t;
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) *static_cast<int *>(e.pick_parts) = (int)gridDim.x;
}

}  // namespace wg
