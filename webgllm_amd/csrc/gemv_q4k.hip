// Decode / few-token GEMV straight from GGUF Q4_K super-blocks
// (WG_LAYOUT_Q4K: 144-byte records regrouped by rows of 4), 0.5625 bytes a
// weight. The reference repacks Q4_K into 32-blocks with half scale d' and
// half zero point z' (packQ4_K, src/repack.ts:100-168) and its shaders then
// compute d' (sum q a - z' sum a) per block (src/gpu/kernels.ts:744-895).
// Here (d', z') are rebuilt in registers from the super-block header:
//   d' = half(d * sc);  d' z' with z' = half(dmin * m / d');
//   a sub-block whose d' is 0 is the constant -dmin * m, which packQ4_K
//   writes as q = 15 with scale half(-dmin * m / 15) and z' = 0.
// (The quotient uses v_rcp_f32: z' can differ from the reference's
// correctly rounded one by one half-ulp when min / d' lies within 2 float
// ulps of a half rounding boundary. The bit-exact dequant is wg_q4_dequant.)
//
// Mapping (wave64): one wave per row group; lane = (super-block sb of 8,
// row pair rp, 32-byte chunk c of the 128 nibble bytes). Chunk c holds
// sub-block 2c in its low nibbles and 2c + 1 in its high nibbles (byte l:
// weight l of each), so one dword gives (q_l, q_l+1) pairs of both, which
// meet natural-order activation pairs in v_dot2_f32_f16 (see dot.h).
#include "common.h"
#include "dot.h"
#include "kernels.h"
#include "epilogue.h"

namespace wg {
namespace {

struct SubScales {
  float d0, dz0, d1, dz1;  // d' and d' z' of sub-blocks 2c and 2c + 1
};

// d' and d' z' of one sub-block from its 6-bit scale and min.
__device__ inline void sub_scale(float d, float dmin, uint32_t sc, uint32_t mn, float &dq,
                                 float &dz) {
  float ds = d * (float)sc;  // exact: 11-bit half times a 6-bit integer
  dq = (float)(_Float16)ds;  // half(d * sc), round to nearest even
  float mins = dmin * (float)mn;  // exact
  if (dq != 0.0f) {
    float zq = (float)(_Float16)(mins * __builtin_amdgcn_rcpf(dq));
    dz = dq * zq;
  } else {
    // Constant sub-block: 15 * half(-mins / 15) for every weight.
    dz = -15.0f * (float)(_Float16)(-mins * (1.0f / 15.0f));
  }
}

// The 6-bit scales and mins of sub-blocks 2c and 2c + 1
// (get_scale_min_k4, as src/repack.ts:127-140 decodes it). h.y, h.z, h.w are
// the 12 scale bytes sc[0..11].
__device__ inline SubScales decode(const uint4 &h, int c) {
  float d = (float)as_h2(h.x).x, dmin = (float)as_h2(h.x).y;
  int sh = (c & 1) * 16;
  uint32_t y2 = h.y >> sh, z2 = h.z >> sh, w2 = h.w >> sh;
  uint32_t s0, s1, m0, m1;
  if (c < 2) {
    s0 = y2 & 63u;
    s1 = (y2 >> 8) & 63u;
    m0 = z2 & 63u;
    m1 = (z2 >> 8) & 63u;
  } else {
    s0 = (w2 & 15u) | ((y2 & 0xc0u) >> 2);
    s1 = ((w2 >> 8) & 15u) | (((y2 >> 8) & 0xc0u) >> 2);
    m0 = ((w2 >> 4) & 15u) | ((z2 & 0xc0u) >> 2);
    m1 = ((w2 >> 12) & 15u) | (((z2 >> 8) & 0xc0u) >> 2);
  }
  SubScales s;
  sub_scale(d, dmin, s0, m0, s.d0, s.dz0);
  sub_scale(d, dmin, s1, m1, s.d1, s.dz1);
  return s;
}

template <int M, int MODE>
__global__ __launch_bounds__(256) void gemv_q4k_kernel(const uint8_t *__restrict__ quants,
                                                       const uint16_t *__restrict__ x, int ldx,
                                                       float *__restrict__ y, int ldy,
                                                       const wg_epilogue e, int G, int S) {
  const int lane = threadIdx.x & 63;
  const int g = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (g >= G) return;
  const int pos0 = epi_pos0<MODE>(e);
  EpiPre pre;
  epi_prefetch<M, MODE>(e, g, G, pos0, pre);
  const int c = lane & 3, rp = (lane >> 2) & 1, sb = lane >> 3;
  float acc[2][M];
#pragma unroll
  for (int r = 0; r < 2; r++)
#pragma unroll
    for (int m = 0; m < M; m++) acc[r][m] = 0.0f;

  for (int s = sb; s < S; s += 8) {
    const uint8_t *rec = quants + (((int64_t)g * S + s) * 4 + 2 * rp) * 144;
    uint4 h[2], q[2][2];
#pragma unroll
    for (int r = 0; r < 2; r++) {
      const uint8_t *p = rec + r * 144;
      h[r] = *reinterpret_cast<const uint4 *>(p);
      q[r][0] = *reinterpret_cast<const uint4 *>(p + 16 + 32 * c);
      q[r][1] = *reinterpret_cast<const uint4 *>(p + 32 + 32 * c);
    }
    // Activations of sub-blocks 2c (a[m][0..3]) and 2c + 1 (a[m][4..7]).
    uint4 a[M][8];
#pragma unroll
    for (int m = 0; m < M; m++) {
      const uint4 *xp = reinterpret_cast<const uint4 *>(x + (int64_t)m * ldx + s * 256 + 64 * c);
#pragma unroll
      for (int i = 0; i < 8; i++) a[m][i] = xp[i];
    }
    float sa0[M], sa1[M];
#pragma unroll
    for (int m = 0; m < M; m++) {
      float t0 = sum8(a[m][0], 0.0f), t1 = sum8(a[m][4], 0.0f);
      t0 = sum8(a[m][1], t0);
      t1 = sum8(a[m][5], t1);
      t0 = sum8(a[m][2], t0);
      t1 = sum8(a[m][6], t1);
      t0 = sum8(a[m][3], t0);
      t1 = sum8(a[m][7], t1);
      sa0[m] = t0 * 0x1p-24f;
      sa1[m] = t1 * 0x1p-24f;
    }
#pragma unroll
    for (int r = 0; r < 2; r++) {
      SubScales sc = decode(h[r], c);
      NibblePairs np[8];
      const uint32_t w[8] = {q[r][0].x, q[r][0].y, q[r][0].z, q[r][0].w,
                             q[r][1].x, q[r][1].y, q[r][1].z, q[r][1].w};
#pragma unroll
      for (int i = 0; i < 8; i++) np[i] = split_nibbles(w[i]);
#pragma unroll
      for (int m = 0; m < M; m++) {
        // Dword i of the chunk is bytes 4i..4i+3: activation dwords 2i and
        // 2i + 1 of each sub-block.
        const uint32_t A0[16] = {a[m][0].x, a[m][0].y, a[m][0].z, a[m][0].w,
                                 a[m][1].x, a[m][1].y, a[m][1].z, a[m][1].w,
                                 a[m][2].x, a[m][2].y, a[m][2].z, a[m][2].w,
                                 a[m][3].x, a[m][3].y, a[m][3].z, a[m][3].w};
        const uint32_t A1[16] = {a[m][4].x, a[m][4].y, a[m][4].z, a[m][4].w,
                                 a[m][5].x, a[m][5].y, a[m][5].z, a[m][5].w,
                                 a[m][6].x, a[m][6].y, a[m][6].z, a[m][6].w,
                                 a[m][7].x, a[m][7].y, a[m][7].z, a[m][7].w};
        float lo = 0.0f, hi = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
          lo = dot2(np[i].lo0, A0[2 * i], lo);
          hi = dot2(np[i].hi0, A1[2 * i], hi);
          lo = dot2(np[i].lo1, A0[2 * i + 1], lo);
          hi = dot2(np[i].hi1, A1[2 * i + 1], hi);
        }
        float v = acc[r][m];
        v = __builtin_fmaf(sc.d0, lo, v);
        v = __builtin_fmaf(-sc.dz0, sa0[m], v);
        v = __builtin_fmaf(sc.d1 * 0.0625f, hi, v);
        v = __builtin_fmaf(-sc.dz1, sa1[m], v);
        acc[r][m] = v;
      }
    }
  }
  float scale[M], tot[M];
  input_scales<M>(e, scale);
  // Rows 2 rp and 2 rp + 1 of each lane; one reduction for every lane (the
  // shuffles must not run under a lane-dependent branch).
#pragma unroll
  for (int m = 0; m < M; m++) {
    float a0 = acc[0][m], a1 = acc[1][m];
    tot[m] = wave_sum4(rp ? 0.0f : a0, rp ? 0.0f : a1, rp ? a0 : 0.0f, rp ? a1 : 0.0f);
  }
  finish<M, MODE>(e, g, G, tot, scale, y, ldy, pre, pos0);
}

// ---------------------------------------------------------------------------
// Streaming variant for 1 or 2 tokens: persistent workgroups of 4 waves; K
// split into KS parts (a wave each, reduced through LDS); a lane keeps the
// activations (and their sub-block sums) of its NS super-blocks' chunk c
// in registers for every row group, and streams row groups with the next
// one's records loaded before the current one is computed.
template <int NS>
struct KUnit {
  uint4 h[NS][2];
  uint4 q[NS][2][2];
};

template <int NS>
__device__ inline void load_kunit(KUnit<NS> &u, const uint8_t *__restrict__ quants, int g, int S,
                                  int s0, int s_end, int rp, int c, bool live) {
#pragma unroll
  for (int j = 0; j < NS; j++) {
    int s = s0 + 8 * j;
    if (live && s < s_end) {
      const uint8_t *rec = quants + (((int64_t)g * S + s) * 4 + 2 * rp) * 144;
#pragma unroll
      for (int r = 0; r < 2; r++) {
        const uint8_t *p = rec + r * 144;
        u.h[j][r] = *reinterpret_cast<const uint4 *>(p);
        u.q[j][r][0] = *reinterpret_cast<const uint4 *>(p + 16 + 32 * c);
        u.q[j][r][1] = *reinterpret_cast<const uint4 *>(p + 32 + 32 * c);
      }
    } else {
#pragma unroll
      for (int r = 0; r < 2; r++) {
        u.h[j][r] = make_uint4(0u, 0u, 0u, 0u);  // d = dmin = 0: contributes nothing
        u.q[j][r][0] = u.q[j][r][1] = make_uint4(0u, 0u, 0u, 0u);
      }
    }
  }
}

template <int M, int NS, int KS, int MODE>
__global__ __launch_bounds__(256) void gemv_q4k_stream_kernel(
    const uint8_t *__restrict__ quants, const uint16_t *__restrict__ x, int ldx,
    float *__restrict__ y, int ldy, const wg_epilogue e, int G, int S) {
  constexpr int RGW = 4 / KS;
  __shared__ float red[2][4][4 * M];
  __shared__ float nred[4 * M];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int part = wave % KS, slot = wave / KS;
  const int c = lane & 3, rp = (lane >> 2) & 1, sb = lane >> 3;
  const int SP = (S + KS - 1) / KS;
  const int s0 = part * SP + sb;
  const int s_end = min(S, (part + 1) * SP);

  // The first row group's records go out before the activations (see the
  // row-group kernel).
  const int stride = gridDim.x * RGW;
  int g = blockIdx.x * RGW + slot;
  KUnit<NS> next;
  load_kunit<NS>(next, quants, g, S, s0, s_end, rp, c, g < G);
  const int pos0 = epi_pos0<MODE>(e);
  EpiPre pnext = {};
  if (part == 0) epi_prefetch<M, MODE>(e, g, G, pos0, pnext);

  uint4 a[M][NS][8];
  float sa0[M][NS], sa1[M][NS];
#pragma unroll
  for (int m = 0; m < M; m++)
#pragma unroll
    for (int j = 0; j < NS; j++) {
      int s = s0 + 8 * j;
      if (s < s_end) {
        const uint4 *xp =
            reinterpret_cast<const uint4 *>(x + (int64_t)m * ldx + s * 256 + 64 * c);
#pragma unroll
        for (int i = 0; i < 8; i++) a[m][j][i] = xp[i];
      } else {
#pragma unroll
        for (int i = 0; i < 8; i++) a[m][j][i] = make_uint4(0u, 0u, 0u, 0u);
      }
    }
  float scale[M];
  input_scales_wg<M, 4>(e, scale, nred);
#pragma unroll
  for (int m = 0; m < M; m++)
#pragma unroll
    for (int j = 0; j < NS; j++) {
      float t0 = sum8(a[m][j][0], 0.0f), t1 = sum8(a[m][j][4], 0.0f);
      t0 = sum8(a[m][j][1], t0);
      t1 = sum8(a[m][j][5], t1);
      t0 = sum8(a[m][j][2], t0);
      t1 = sum8(a[m][j][6], t1);
      t0 = sum8(a[m][j][3], t0);
      t1 = sum8(a[m][j][7], t1);
      sa0[m][j] = t0 * 0x1p-24f;
      sa1[m][j] = t1 * 0x1p-24f;
    }

  int it = 0;
  for (int g0 = blockIdx.x * RGW; g0 < G; g0 += stride, g += stride, it ^= 1) {
    KUnit<NS> u = next;
    load_kunit<NS>(next, quants, g + stride, S, s0, s_end, rp, c, g + stride < G);
    const EpiPre pe = pnext;
    if (part == 0) epi_prefetch<M, MODE>(e, g + stride, G, pos0, pnext);
    float acc[2][M];
#pragma unroll
    for (int r = 0; r < 2; r++)
#pragma unroll
      for (int m = 0; m < M; m++) acc[r][m] = 0.0f;
#pragma unroll
    for (int j = 0; j < NS; j++)
#pragma unroll
      for (int r = 0; r < 2; r++) {
        SubScales sc = decode(u.h[j][r], c);
        const uint32_t w[8] = {u.q[j][r][0].x, u.q[j][r][0].y, u.q[j][r][0].z, u.q[j][r][0].w,
                               u.q[j][r][1].x, u.q[j][r][1].y, u.q[j][r][1].z, u.q[j][r][1].w};
        NibblePairs np[8];
#pragma unroll
        for (int i = 0; i < 8; i++) np[i] = split_nibbles(w[i]);
#pragma unroll
        for (int m = 0; m < M; m++) {
          const uint4 *A0 = a[m][j], *A1 = a[m][j] + 4;
          float lo = 0.0f, hi = 0.0f;
#pragma unroll
          for (int i = 0; i < 8; i++) {
            const uint4 &p0 = A0[i >> 1], &p1 = A1[i >> 1];
            uint32_t x0 = (i & 1) ? p0.z : p0.x, x1 = (i & 1) ? p0.w : p0.y;
            uint32_t y0 = (i & 1) ? p1.z : p1.x, y1 = (i & 1) ? p1.w : p1.y;
            lo = dot2(np[i].lo0, x0, lo);
            hi = dot2(np[i].hi0, y0, hi);
            lo = dot2(np[i].lo1, x1, lo);
            hi = dot2(np[i].hi1, y1, hi);
          }
          float v = acc[r][m];
          v = __builtin_fmaf(sc.d0, lo, v);
          v = __builtin_fmaf(-sc.dz0, sa0[m][j], v);
          v = __builtin_fmaf(sc.d1 * 0.0625f, hi, v);
          v = __builtin_fmaf(-sc.dz1, sa1[m][j], v);
          acc[r][m] = v;
        }
      }
    // Rows 2 rp and 2 rp + 1 of each lane, reduced into the wave_sum4 layout.
    const int row = wave_sum4_row();
    float tot[M];
#pragma unroll
    for (int m = 0; m < M; m++) {
      float a0 = acc[0][m], a1 = acc[1][m];
      tot[m] = wave_sum4(rp ? 0.0f : a0, rp ? 0.0f : a1, rp ? a0 : 0.0f, rp ? a1 : 0.0f);
    }
    if constexpr (KS > 1) {
      if ((lane & 15) == 0 && part > 0)
#pragma unroll
        for (int m = 0; m < M; m++) red[it][wave][row * M + m] = tot[m];
      __syncthreads();
      if (part == 0)
#pragma unroll
        for (int m = 0; m < M; m++)
#pragma unroll
          for (int p = 1; p < KS; p++) tot[m] += red[it][wave + p][row * M + m];
    }
    if (part == 0) finish<M, MODE>(e, g, G, tot, scale, y, ldy, pe, pos0);
  }
}

template <int M, int NS, int KS>
int launch_kstream(const wg_q4_matrix *w, const uint16_t *x, int ldx, float *y, int ldy,
                   const wg_epilogue &e, hipStream_t s) {
  int G = w->N / 4, S = w->K / 256;
  constexpr int RGW = 4 / KS;
  int grid = persistent_grid((G + RGW - 1) / RGW, tuning("q4k_wg_per_cu"));
  auto q = (const uint8_t *)w->quants;
  if (e.mode == WG_EPI_SWIGLU)
    gemv_q4k_stream_kernel<M, NS, KS, WG_EPI_SWIGLU><<<grid, 256, 0, s>>>(q, x, ldx, y, ldy, e,
                                                                         G, S);
  else if (e.mode == WG_EPI_ROPE_KV)
    gemv_q4k_stream_kernel<M, NS, KS, WG_EPI_ROPE_KV><<<grid, 256, 0, s>>>(q, x, ldx, y, ldy, e,
                                                                          G, S);
  else
    gemv_q4k_stream_kernel<M, NS, KS, WG_EPI_STORE><<<grid, 256, 0, s>>>(q, x, ldx, y, ldy, e,
                                                                        G, S);
  return launched("wg_q4_gemv (Q4_K)");
}

template <int M>
int launch_kstream_m(const wg_q4_matrix *w, const uint16_t *x, int ldx, float *y, int ldy,
                     const wg_epilogue &ep, hipStream_t s) {
  // As the row-group GEMV: at most 2 super-blocks a lane, and a further K
  // split (while every part keeps 8 super-blocks) for small matrices.
  int S = w->K / 256, G = w->N / 4;
  int ks = S <= 16 ? 1 : S <= 32 ? 2 : S <= 64 ? 4 : 0;
  if (!ks) return -1;
  while (ks < 4 && G * ks < tuning("gemv_min_waves") && S / (2 * ks) >= 8) ks *= 2;
  int ns = (S + ks - 1) / ks > 8 ? 2 : 1;
  if (ks == 1) return ns == 1 ? launch_kstream<M, 1, 1>(w, x, ldx, y, ldy, ep, s)
                              : launch_kstream<M, 2, 1>(w, x, ldx, y, ldy, ep, s);
  if (ks == 2) return ns == 1 ? launch_kstream<M, 1, 2>(w, x, ldx, y, ldy, ep, s)
                              : launch_kstream<M, 2, 2>(w, x, ldx, y, ldy, ep, s);
  return ns == 1 ? launch_kstream<M, 1, 4>(w, x, ldx, y, ldy, ep, s)
                 : launch_kstream<M, 2, 4>(w, x, ldx, y, ldy, ep, s);
}

// ---------------------------------------------------------------------------
// Streaming kernel with every lane on all 4 rows of a row group, for 1 or 2
// tokens and K of 16 to 64 super-blocks (K split into KS parts of at most
// 16): lane = (super-block sl of 16, 32-byte chunk c of 4), so a lane takes
// chunk c (the low nibbles of sub-block 2c, the high nibbles of 2c + 1) of
// one super-block of the part for the group's 4 rows. Its activations and
// their sums are loaded once; row groups are streamed through two register
// sets (the loop unrolled by 2, so the prefetched records are never
// copied). Scales are rebuilt per row and sub-block without branches, and a
// dword of nibble bytes becomes its 4 pairs in 5 instructions: pairs
// (w_l, w_l+2) with one mask, (w_l+1, w_l+3) with one permute and a mask,
// the lane's activations paired to match once.
struct Q4kRows {
  uint4 h[4];     // the 4 rows' headers: d | dmin, 12 bytes of 6-bit scales and mins
  uint4 q[4][2];  // the 4 rows' 32 nibble bytes of chunk c
};

__device__ inline void load_q4k_rows(Q4kRows &u, const uint8_t *__restrict__ quants, int g,
                                     int S, int s, int c) {
  const uint8_t *rec = quants + ((int64_t)g * S + s) * 4 * 144;
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const uint8_t *p = rec + r * 144;
    u.h[r] = *reinterpret_cast<const uint4 *>(p);
    u.q[r][0] = *reinterpret_cast<const uint4 *>(p + 16 + 32 * c);
    u.q[r][1] = *reinterpret_cast<const uint4 *>(p + 32 + 32 * c);
  }
}

// d' and d' z' of sub-blocks 2c and 2c + 1 of one row (packQ4_K's rounding,
// src/repack.ts:127-163; z' through v_rcp_f32 as sub_scale above), without
// branches: the 6-bit fields are picked by selects, the constant sub-block
// (d' = 0) by a select.
__device__ inline SubScales decode_rows(const uint4 &h, int c) {
  const float d = (float)as_h2(h.x).x, dmin = (float)as_h2(h.x).y;
  const int sh = (c & 1) * 16;
  const uint32_t y2 = h.y >> sh, z2 = h.z >> sh, w2 = h.w >> sh;
  const bool hi = c >= 2;
  // sub-blocks 0..3: scale = sc[j] & 63, min = sc[j + 4] & 63; 4..7: the low
  // (scale) or high (min) nibble of sc[j + 4] under the top 2 bits of sc[j - 4]
  // (scale) or sc[j] (min)
  const uint32_t slo = hi ? w2 : y2, mlo = hi ? (w2 >> 4) : z2;
  const uint32_t top = hi ? 0xfu : 0x3fu;
  const uint32_t s0 = (slo & top) | (hi ? ((y2 >> 2) & 0x30u) : 0u);
  const uint32_t s1 = ((slo >> 8) & top) | (hi ? ((y2 >> 10) & 0x30u) : 0u);
  const uint32_t m0 = (mlo & top) | (hi ? ((z2 >> 2) & 0x30u) : 0u);
  const uint32_t m1 = ((mlo >> 8) & top) | (hi ? ((z2 >> 10) & 0x30u) : 0u);
  SubScales o;
  const float sc[2] = {(float)s0, (float)s1}, mn[2] = {(float)m0, (float)m1};
  float dq[2], dz[2];
#pragma unroll
  for (int k = 0; k < 2; k++) {
    dq[k] = (float)(_Float16)(d * sc[k]);  // exact product, rounded once
    const float mins = dmin * mn[k];       // exact
    const float z = (float)(_Float16)(mins * __builtin_amdgcn_rcpf(dq[k]));
    const float cz = -15.0f * (float)(_Float16)(-mins * (1.0f / 15.0f));
    dz[k] = dq[k] != 0.0f ? dq[k] * z : cz;
  }
  o.d0 = dq[0];
  o.dz0 = dz[0];
  o.d1 = dq[1];
  o.dz1 = dz[1];
  return o;
}

// v_perm_b32 selector: bytes 1 and 3 into the low byte of each half.
constexpr uint32_t SEL13 = 0x0c030c01u;

template <int M, int KS, int MODE>
__global__ __launch_bounds__(256) void gemv_q4k_rows_kernel(
    const uint8_t *__restrict__ quants, const uint16_t *__restrict__ x, int ldx,
    float *__restrict__ y, int ldy, const wg_epilogue e, int G, int S) {
  constexpr int RGW = 4 / KS;  // row groups a workgroup takes at a time
  __shared__ float red[2][4][4 * M];
  __shared__ float nred[4 * M];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int part = wave % KS, slot = wave / KS;
  const int c = lane & 3, sl = lane >> 2;
  const int SP = (S + KS - 1) / KS;
  const int s_raw = part * SP + sl;
  const bool s_live = sl < SP && s_raw < S;
  const int s = s_live ? s_raw : 0;  // idle lanes read super-block 0 and add zeros
  const int stride = gridDim.x * RGW;
  const int g_first = blockIdx.x * RGW + slot;

  Q4kRows A, B;
  load_q4k_rows(A, quants, min(g_first, G - 1), S, s, c);
  const int pos0 = epi_pos0<MODE>(e);
  EpiPre pnext = {};
  if (part == 0) epi_prefetch<M, MODE>(e, g_first, G, pos0, pnext);

  // This lane's 64 activations (sub-block 2c, then 2c + 1) paired as the
  // nibbles come: even (a_4i, a_4i+2) and odd (a_4i+1, a_4i+3); their sums.
  uint32_t ae[M][2][8], ao[M][2][8];
  float sa[M][2];
#pragma unroll
  for (int m = 0; m < M; m++) {
    const uint4 *xp = reinterpret_cast<const uint4 *>(x + (int64_t)m * ldx + s * 256 + 64 * c);
#pragma unroll
    for (int k = 0; k < 2; k++) {
      uint4 a4[4];
#pragma unroll
      for (int i = 0; i < 4; i++)
        a4[i] = s_live ? xp[4 * k + i] : make_uint4(0u, 0u, 0u, 0u);
      const uint32_t dw[16] = {a4[0].x, a4[0].y, a4[0].z, a4[0].w, a4[1].x, a4[1].y,
                               a4[1].z, a4[1].w, a4[2].x, a4[2].y, a4[2].z, a4[2].w,
                               a4[3].x, a4[3].y, a4[3].z, a4[3].w};
      float t = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; i++) {
        ae[m][k][i] = __builtin_amdgcn_perm(dw[2 * i + 1], dw[2 * i], 0x05040100u);
        ao[m][k][i] = __builtin_amdgcn_perm(dw[2 * i + 1], dw[2 * i], 0x07060302u);
        t = dot2(dw[2 * i], ONES, t);
        t = dot2(dw[2 * i + 1], ONES, t);
      }
      sa[m][k] = t * 0x1p-24f;
    }
  }
  float scale[M];
  input_scales_wg<M, 4>(e, scale, nred);

  // one row group: the 4 rows' sums for each token, then the epilogue
  auto step = [&](const Q4kRows &u, int g, int it, const EpiPre &pe) {
    float acc[4][M];
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const SubScales sc = decode_rows(u.h[r], c);
      const uint32_t w[8] = {u.q[r][0].x, u.q[r][0].y, u.q[r][0].z, u.q[r][0].w,
                             u.q[r][1].x, u.q[r][1].y, u.q[r][1].z, u.q[r][1].w};
      uint32_t le[8], lo[8], he[8], ho[8];
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const uint32_t p = __builtin_amdgcn_perm(0u, w[i], SEL13);
        le[i] = w[i] & LO4;
        he[i] = w[i] & HI4;
        lo[i] = p & LO4;
        ho[i] = p & HI4;
      }
#pragma unroll
      for (int m = 0; m < M; m++) {
        float l = 0.0f, h = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
          l = dot2(le[i], ae[m][0][i], l);
          h = dot2(he[i], ae[m][1][i], h);
          l = dot2(lo[i], ao[m][0][i], l);
          h = dot2(ho[i], ao[m][1][i], h);
        }
        float v = sc.d0 * l;
        v = __builtin_fmaf(-sc.dz0, sa[m][0], v);
        v = __builtin_fmaf(sc.d1 * 0.0625f, h, v);
        v = __builtin_fmaf(-sc.dz1, sa[m][1], v);
        acc[r][m] = v;
      }
    }
    const int row = wave_sum4_row();
    float tot[M];
#pragma unroll
    for (int m = 0; m < M; m++) tot[m] = wave_sum4(acc[0][m], acc[1][m], acc[2][m], acc[3][m]);
    if constexpr (KS > 1) {
      if ((lane & 15) == 0 && part > 0)
#pragma unroll
        for (int m = 0; m < M; m++) red[it][wave][row * M + m] = tot[m];
      __syncthreads();
      if (part == 0)
#pragma unroll
        for (int m = 0; m < M; m++)
#pragma unroll
          for (int p = 1; p < KS; p++) tot[m] += red[it][wave + p][row * M + m];
    }
    if (part == 0) finish<M, MODE>(e, g, G, tot, scale, y, ldy, pe, pos0);
  };

  // g0 is the same for every wave of the workgroup, so all of them run the
  // same iterations (the reductions' barriers); g >= G is an idle slot
  for (int g0 = blockIdx.x * RGW, g = g_first; g0 < G; g0 += 2 * stride, g += 2 * stride) {
    load_q4k_rows(B, quants, min(g + stride, G - 1), S, s, c);
    EpiPre pe = pnext;
    if (part == 0) epi_prefetch<M, MODE>(e, g + stride, G, pos0, pnext);
    step(A, g, 0, pe);
    if (g0 + stride >= G) break;
    load_q4k_rows(A, quants, min(g + 2 * stride, G - 1), S, s, c);
    pe = pnext;
    if (part == 0) epi_prefetch<M, MODE>(e, g + 2 * stride, G, pos0, pnext);
    step(B, g + stride, 1, pe);
  }
}

template <int M, int KS>
int launch_rows(const wg_q4_matrix *w, const uint16_t *x, int ldx, float *y, int ldy,
                const wg_epilogue &e, hipStream_t s) {
  const int G = w->N / 4, S = w->K / 256;
  constexpr int RGW = 4 / KS;
  const int grid = persistent_grid((G + RGW - 1) / RGW, tuning("q4k_wg_per_cu"));
  auto q = (const uint8_t *)w->quants;
  if (e.mode == WG_EPI_SWIGLU)
    gemv_q4k_rows_kernel<M, KS, WG_EPI_SWIGLU><<<grid, 256, 0, s>>>(q, x, ldx, y, ldy, e, G, S);
  else if (e.mode == WG_EPI_ROPE_KV)
    gemv_q4k_rows_kernel<M, KS, WG_EPI_ROPE_KV><<<grid, 256, 0, s>>>(q, x, ldx, y, ldy, e, G, S);
  else
    gemv_q4k_rows_kernel<M, KS, WG_EPI_STORE><<<grid, 256, 0, s>>>(q, x, ldx, y, ldy, e, G, S);
  return launched("wg_q4_gemv (Q4_K)");
}

// K of 16 to 64 super-blocks in parts of at most 16; -1 for other shapes.
template <int M>
int launch_rows_m(const wg_q4_matrix *w, const uint16_t *x, int ldx, float *y, int ldy,
                  const wg_epilogue &ep, hipStream_t s) {
  const int S = w->K / 256;
  if (S < 16 || S > 64) return -1;
  const int ks = S <= 16 ? 1 : S <= 32 ? 2 : 4;
  if (ks == 1) return launch_rows<M, 1>(w, x, ldx, y, ldy, ep, s);
  if (ks == 2) return launch_rows<M, 2>(w, x, ldx, y, ldy, ep, s);
  return launch_rows<M, 4>(w, x, ldx, y, ldy, ep, s);
}

template <int M>
int launch_m(const wg_q4_matrix *w, const uint16_t *x, int ldx, float *y, int ldy,
             const wg_epilogue &e, hipStream_t s) {
  int G = w->N / 4, S = w->K / 256;
  auto q = (const uint8_t *)w->quants;
  if (e.mode == WG_EPI_SWIGLU)
    gemv_q4k_kernel<M, WG_EPI_SWIGLU><<<(G + 3) / 4, 256, 0, s>>>(q, x, ldx, y, ldy, e, G, S);
  else if (e.mode == WG_EPI_ROPE_KV)
    gemv_q4k_kernel<M, WG_EPI_ROPE_KV><<<(G + 3) / 4, 256, 0, s>>>(q, x, ldx, y, ldy, e, G, S);
  else
    gemv_q4k_kernel<M, WG_EPI_STORE><<<(G + 3) / 4, 256, 0, s>>>(q, x, ldx, y, ldy, e, G, S);
  return launched("wg_q4_gemv (Q4_K)");
}

}  // namespace

int launch_gemv_q4k(const wg_q4_matrix *w, const uint16_t *x, int M, int ldx, float *y, int ldy,
                    const wg_epilogue &ep, hipStream_t s) {
  if (M <= 2 && tuning("q4k_rows")) {
    int rc = M == 1 ? launch_rows_m<1>(w, x, ldx, y, ldy, ep, s)
                    : launch_rows_m<2>(w, x, ldx, y, ldy, ep, s);
    if (rc != -1) return rc;
  }
  if (M <= 2) {
    int rc = M == 1 ? launch_kstream_m<1>(w, x, ldx, y, ldy, ep, s)
                    : launch_kstream_m<2>(w, x, ldx, y, ldy, ep, s);
    if (rc != -1) return rc;
  }
  switch (M) {
    case 1: return launch_m<1>(w, x, ldx, y, ldy, ep, s);
    case 2: return launch_m<2>(w, x, ldx, y, ldy, ep, s);
    case 3: return launch_m<3>(w, x, ldx, y, ldy, ep, s);
    case 4: return launch_m<4>(w, x, ldx, y, ldy, ep, s);
    case 5: return launch_m<5>(w, x, ldx, y, ldy, ep, s);
    case 6: return launch_m<6>(w, x, ldx, y, ldy, ep, s);
    case 7: return launch_m<7>(w, x, ldx, y, ldy, ep, s);
    default: return launch_m<8>(w, x, ldx, y, ldy, ep, s);
  }
}

}  // namespace wg
