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
