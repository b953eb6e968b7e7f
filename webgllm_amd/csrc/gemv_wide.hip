// Decode / few-token GEMV for 8-bit and Q6_K matrices (WG_LAYOUT_Q8,
// WG_LAYOUT_Q6K): the reference's 8-bit split matmul (src/gpu/kernels.ts:
// 219-246: per block acc += d * sum q a) and its Q6_K output head
// (kernels.ts:3593-3686: per super-block acc += d * sum_sub sc * sum (q -
// 32) a), which real GGUF files need: their embeddings (the tied output
// head) are Q6_K, and every tensor the loader does not keep in 4 bits is
// requantized to 8 (src/load-gguf.ts:428-442, :486-555).
//
// The same shape as the 4-bit GEMV (gemv.hip): a wave per row group, lanes
// over "chunks" along K, a chunk's 4 rows loaded with 128-bit loads,
// dequant in registers, v_dot2_f32_f16 with float32 accumulation, a
// butterfly over the lanes and the shared epilogues.
//  - 8-bit: a chunk is a block of 32 (the group's 4 block rows are 128
//    contiguous bytes). A code byte q becomes q + 128 with one xor a dword,
//    a byte permute puts two of them in the low bytes of two halves (fp16
//    subnormals (q + 128) 2^-24, exact), and sum q a = sum (q + 128) a -
//    128 sum a, the activation sum loaded once per lane.
//  - Q6_K: a chunk is 64 weights of one row's super-block s: half h, and
//    l = 16 c .. 16 c + 15 of its 32 positions, in the four groups i of
//    dequantize_row_q6_K (weights 128 h + 32 i + l, sub-blocks 8 h + 2 i +
//    c). Its bytes are ql[64 h + l], ql[64 h + 32 + l] and qh[32 h + l]:
//    three 16-byte loads a row, and the 8 scale bytes of the half. Four
//    6-bit codes of one group are rebuilt in a dword with two masks and an
//    or, then taken as subnormals as above; sum (q - 32) a = sum q a - 32
//    sum a per sub-block.
#include "common.h"
#include "dot.h"
#include "kernels.h"
#include "epilogue.h"

namespace wg {
namespace {

struct Mat {
  const uint8_t *quants;
  const uint16_t *scales;
  int C;  // chunks per row
  int S;  // 8-bit: blocks per row; Q6_K: super-blocks per row
};

// Dword k (0..7) of 8 half pairs held as two uint4.
__device__ inline uint32_t dw(const uint4 &a, const uint4 &b, int k) {
  const uint4 &v = k < 4 ? a : b;
  const int c = k & 3;
  return c == 0 ? v.x : c == 1 ? v.y : c == 2 ? v.z : v.w;
}
__device__ inline uint32_t comp(const uint4 &v, int c) {
  return c == 0 ? v.x : c == 1 ? v.y : c == 2 ? v.z : v.w;
}

struct Q8 {
  static constexpr int AV = 4;    // uint4 activation loads a chunk takes per token
  static constexpr int NSUM = 1;  // activation sums a chunk needs per token
  template <int NB>
  struct Unit {
    uint4 q[NB][4][2];
    uint2 sc[NB];
  };

  template <int NB>
  __device__ static void load(Unit<NB> &u, const Mat &m, int g, int c, int j, bool live) {
    if (live) {
      const int64_t si = ((int64_t)g * m.S + c) * 4;
      const uint4 *qp = reinterpret_cast<const uint4 *>(m.quants + si * 32);
#pragma unroll
      for (int r = 0; r < 4; r++) {
        u.q[j][r][0] = qp[2 * r];
        u.q[j][r][1] = qp[2 * r + 1];
      }
      u.sc[j] = *reinterpret_cast<const uint2 *>(m.scales + si);
    } else {
#pragma unroll
      for (int r = 0; r < 4; r++) u.q[j][r][0] = u.q[j][r][1] = make_uint4(0u, 0u, 0u, 0u);
      u.sc[j] = make_uint2(0u, 0u);  // scale 0: contributes nothing
    }
  }

  // Chunk c's activations of one token and their sum (times 2^-24).
  __device__ static void acts(const uint16_t *xr, int c, bool live, uint4 (&a)[AV],
                              float (&sa)[NSUM]) {
    if (live) {
      const uint4 *xp = reinterpret_cast<const uint4 *>(xr + (int64_t)c * 32);
#pragma unroll
      for (int i = 0; i < 4; i++) a[i] = xp[i];
    } else {
#pragma unroll
      for (int i = 0; i < 4; i++) a[i] = make_uint4(0u, 0u, 0u, 0u);
    }
    float s0 = sum8(a[0], 0.0f), s1 = sum8(a[1], 0.0f);
    s0 = sum8(a[2], s0);
    s1 = sum8(a[3], s1);
    sa[0] = (s0 + s1) * 0x1p-24f;
  }

  // acc[r][m] += row 4g + r of the unit's chunks times token m (units of 2^-24).
  template <int M, int NB>
  __device__ static void accumulate(const Unit<NB> &u, const uint4 (&a)[M][NB][AV],
                                    const float (&sa)[M][NB][NSUM], float (&acc)[4][M]) {
#pragma unroll
    for (int j = 0; j < NB; j++) {
      const float d[4] = {(float)as_h2(u.sc[j].x).x, (float)as_h2(u.sc[j].x).y,
                          (float)as_h2(u.sc[j].y).x, (float)as_h2(u.sc[j].y).y};
#pragma unroll
      for (int r = 0; r < 4; r++) {
        uint32_t p[16];
#pragma unroll
        for (int w = 0; w < 8; w++) {
          const uint32_t v = (w < 4 ? comp(u.q[j][r][0], w) : comp(u.q[j][r][1], w - 4)) ^
                             0x80808080u;
          p[2 * w] = __builtin_amdgcn_perm(0u, v, SEL01);
          p[2 * w + 1] = __builtin_amdgcn_perm(0u, v, SEL23);
        }
#pragma unroll
        for (int mm = 0; mm < M; mm++) {
          float b0 = 0.0f, b1 = 0.0f;
#pragma unroll
          for (int k = 0; k < 16; k += 2) {
            b0 = dot2(p[k], comp(a[mm][j][k >> 2], k & 3), b0);
            b1 = dot2(p[k + 1], comp(a[mm][j][k >> 2], (k & 3) + 1), b1);
          }
          const float v = __builtin_fmaf(-128.0f, sa[mm][j][0], b0 + b1);
          acc[r][mm] = __builtin_fmaf(d[r], v, acc[r][mm]);
        }
      }
    }
  }
};

struct Q6K {
  static constexpr int AV = 8;
  static constexpr int NSUM = 4;
  template <int NB>
  struct Unit {
    uint4 qa[NB][4], qb[NB][4], qh[NB][4];
    uint2 sc[NB][4];
    uint2 d[NB];
  };

  template <int NB>
  __device__ static void load(Unit<NB> &u, const Mat &m, int g, int c, int j, bool live) {
    if (live) {
      const int s = c >> 2, h = (c >> 1) & 1, cc = c & 1;
      const int64_t at = ((int64_t)g * m.S + s) * 4;
      const uint8_t *rec = m.quants + at * 208;
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const uint8_t *p = rec + r * 208;
        u.qa[j][r] = *reinterpret_cast<const uint4 *>(p + 64 * h + 16 * cc);
        u.qb[j][r] = *reinterpret_cast<const uint4 *>(p + 64 * h + 32 + 16 * cc);
        u.qh[j][r] = *reinterpret_cast<const uint4 *>(p + 128 + 32 * h + 16 * cc);
        u.sc[j][r] = *reinterpret_cast<const uint2 *>(p + 192 + 8 * h);
      }
      u.d[j] = *reinterpret_cast<const uint2 *>(m.scales + at);
    } else {
#pragma unroll
      for (int r = 0; r < 4; r++) {
        u.qa[j][r] = u.qb[j][r] = u.qh[j][r] = make_uint4(0u, 0u, 0u, 0u);
        u.sc[j][r] = make_uint2(0u, 0u);
      }
      u.d[j] = make_uint2(0u, 0u);  // d = 0: contributes nothing
    }
  }

  // Chunk c's activations of one token: group i's 16 at 256 s + 128 h + 32 i
  // + 16 c in a[2 i], a[2 i + 1]; their sums (times 2^-24) in sa[i].
  __device__ static void acts(const uint16_t *xr, int c, bool live, uint4 (&a)[AV],
                              float (&sa)[NSUM]) {
    const int k0 = (c >> 2) * 256 + ((c >> 1) & 1) * 128 + (c & 1) * 16;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      if (live) {
        const uint4 *xp = reinterpret_cast<const uint4 *>(xr + k0 + 32 * i);
        a[2 * i] = xp[0];
        a[2 * i + 1] = xp[1];
      } else {
        a[2 * i] = a[2 * i + 1] = make_uint4(0u, 0u, 0u, 0u);
      }
      sa[i] = sum8(a[2 * i + 1], sum8(a[2 * i], 0.0f)) * 0x1p-24f;
    }
  }

  template <int M, int NB>
  __device__ static void accumulate(const Unit<NB> &u, const uint4 (&a)[M][NB][AV],
                                    const float (&sa)[M][NB][NSUM], float (&acc)[4][M]) {
    const int cc = threadIdx.x & 1;  // a lane's chunks all have c % 2 = lane % 2
#pragma unroll
    for (int j = 0; j < NB; j++) {
      const float d[4] = {(float)as_h2(u.d[j].x).x, (float)as_h2(u.d[j].x).y,
                          (float)as_h2(u.d[j].y).x, (float)as_h2(u.d[j].y).y};
#pragma unroll
      for (int r = 0; r < 4; r++) {
        // The 6-bit codes of groups 0..3 for positions 4 w .. 4 w + 3, as
        // subnormal half pairs: p[i][2 w], p[i][2 w + 1].
        uint32_t p[4][8];
#pragma unroll
        for (int w = 0; w < 4; w++) {
          const uint32_t A = comp(u.qa[j][r], w), B = comp(u.qb[j][r], w),
                         H = comp(u.qh[j][r], w);
          const uint32_t g[4] = {(A & 0x0f0f0f0fu) | ((H << 4) & 0x30303030u),
                                 (B & 0x0f0f0f0fu) | ((H << 2) & 0x30303030u),
                                 ((A >> 4) & 0x0f0f0f0fu) | (H & 0x30303030u),
                                 ((B >> 4) & 0x0f0f0f0fu) | ((H >> 2) & 0x30303030u)};
#pragma unroll
          for (int i = 0; i < 4; i++) {
            p[i][2 * w] = __builtin_amdgcn_perm(0u, g[i], SEL01);
            p[i][2 * w + 1] = __builtin_amdgcn_perm(0u, g[i], SEL23);
          }
        }
        // Sub-block scales 8 h + 2 i + c: bytes c, c + 2 of sc.x (i = 0, 1)
        // and of sc.y (i = 2, 3), sign-extended (v_bfe_i32; the builtin's
        // result type is unsigned, so it is read back as a signed int).
        float sc[4];
#pragma unroll
        for (int i = 0; i < 4; i++)
          sc[i] = (float)(int32_t)__builtin_amdgcn_sbfe(i < 2 ? u.sc[j][r].x : u.sc[j][r].y,
                                                       8 * (cc + 2 * (i & 1)), 8);
#pragma unroll
        for (int mm = 0; mm < M; mm++) {
          float v = 0.0f;
#pragma unroll
          for (int i = 0; i < 4; i++) {
            float b0 = 0.0f, b1 = 0.0f;
#pragma unroll
            for (int k = 0; k < 8; k += 2) {
              b0 = dot2(p[i][k], dw(a[mm][j][2 * i], a[mm][j][2 * i + 1], k), b0);
              b1 = dot2(p[i][k + 1], dw(a[mm][j][2 * i], a[mm][j][2 * i + 1], k + 1), b1);
            }
            v = __builtin_fmaf(sc[i], __builtin_fmaf(-32.0f, sa[mm][j][i], b0 + b1), v);
          }
          acc[r][mm] = __builtin_fmaf(d[r], v, acc[r][mm]);
        }
      }
    }
  }
};

// Streaming form for 1 or 2 tokens (see gemv_stream_kernel): persistent
// workgroups of 4 waves, K split into KS parts (a wave each, reduced
// through LDS), each lane's activations (chunks c0 and c0 + 64) held in
// registers for every row group, the next row group's unit loaded before
// the current one is computed.
template <class F, int M, int NB, int KS, int MODE>
__global__ __launch_bounds__(256) void gemv_wide_stream_kernel(const Mat mat,
                                                               const uint16_t *__restrict__ x,
                                                               int ldx, float *__restrict__ y,
                                                               int ldy, const wg_epilogue e,
                                                               int G) {
  constexpr int RGW = 4 / KS;
  __shared__ float red[2][4][4 * M];
  __shared__ float nred[4 * M];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int part = wave % KS, slot = wave / KS;
  // Parts of an even number of chunks, so a chunk's parity is its lane's
  // (the Q6_K scales depend on it).
  const int CP = ((mat.C + KS - 1) / KS + 1) & ~1;
  const int c0 = part * CP + lane;
  const int c_end = min(mat.C, (part + 1) * CP);

  const int stride = gridDim.x * RGW;
  int g = blockIdx.x * RGW + slot;
  typename F::template Unit<NB> next;
#pragma unroll
  for (int j = 0; j < NB; j++) F::load(next, mat, g, c0 + 64 * j, j, g < G && c0 + 64 * j < c_end);
  const int pos0 = epi_pos0<MODE>(e);
  EpiPre pnext = {};
  if (part == 0) epi_prefetch<M, MODE>(e, g, G, pos0, pnext);

  uint4 a[M][NB][F::AV];
  float sa[M][NB][F::NSUM];
#pragma unroll
  for (int m = 0; m < M; m++)
#pragma unroll
    for (int j = 0; j < NB; j++)
      F::acts(x + (int64_t)m * ldx, c0 + 64 * j, c0 + 64 * j < c_end, a[m][j], sa[m][j]);
  float scale[M];
  input_scales_wg<M, 4>(e, scale, nred);

  int it = 0;
  for (int g0 = blockIdx.x * RGW; g0 < G; g0 += stride, g += stride, it ^= 1) {
    const typename F::template Unit<NB> u = next;
    const int gn = g + stride;
#pragma unroll
    for (int j = 0; j < NB; j++)
      F::load(next, mat, gn, c0 + 64 * j, j, gn < G && c0 + 64 * j < c_end);
    const EpiPre pe = pnext;
    if (part == 0) epi_prefetch<M, MODE>(e, gn, G, pos0, pnext);
    float acc[4][M];
#pragma unroll
    for (int r = 0; r < 4; r++)
#pragma unroll
      for (int m = 0; m < M; m++) acc[r][m] = 0.0f;
    F::template accumulate<M, NB>(u, a, sa, acc);
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
  }
}

// Any M <= 8: a wave per row group, lanes over the chunks; tokens taken in
// pairs, each pair's activations loaded per chunk.
template <class F, int M, int MODE>
__global__ __launch_bounds__(256) void gemv_wide_rowgroup_kernel(const Mat mat,
                                                                 const uint16_t *__restrict__ x,
                                                                 int ldx, float *__restrict__ y,
                                                                 int ldy, const wg_epilogue e,
                                                                 int G) {
  const int lane = threadIdx.x & 63;
  const int g = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (g >= G) return;  // whole waves leave together
  const int pos0 = epi_pos0<MODE>(e);
  EpiPre pre;
  epi_prefetch<M, MODE>(e, g, G, pos0, pre);
  float acc[4][M];
#pragma unroll
  for (int r = 0; r < 4; r++)
#pragma unroll
    for (int m = 0; m < M; m++) acc[r][m] = 0.0f;
  for (int c = lane; c < mat.C; c += 64) {
    typename F::template Unit<1> u;
    F::load(u, mat, g, c, 0, true);
#pragma unroll
    for (int m0 = 0; m0 < M; m0 += 2) {
      constexpr int P = 2;
      uint4 a[P][1][F::AV];
      float sa[P][1][F::NSUM];
      float t[4][P];
#pragma unroll
      for (int q = 0; q < P; q++) {
        const bool has = m0 + q < M;
        F::acts(x + (int64_t)(has ? m0 + q : m0) * ldx, c, has, a[q][0], sa[q][0]);
#pragma unroll
        for (int r = 0; r < 4; r++) t[r][q] = has ? acc[r][m0 + q] : 0.0f;
      }
      F::template accumulate<P, 1>(u, a, sa, t);
#pragma unroll
      for (int q = 0; q < P; q++)
        if (m0 + q < M)
#pragma unroll
          for (int r = 0; r < 4; r++) acc[r][m0 + q] = t[r][q];
    }
  }
  float scale[M], tot[M];
  input_scales<M>(e, scale);
#pragma unroll
  for (int m = 0; m < M; m++) tot[m] = wave_sum4(acc[0][m], acc[1][m], acc[2][m], acc[3][m]);
  finish<M, MODE>(e, g, G, tot, scale, y, ldy, pre, pos0);
}

template <class F, int M, int NB, int KS>
int launch_stream(const Mat &mat, int G, const uint16_t *x, int ldx, float *y, int ldy,
                  const wg_epilogue &e, hipStream_t s) {
  constexpr int RGW = 4 / KS;
  int grid = persistent_grid((G + RGW - 1) / RGW, tuning("wide_wg_per_cu"));
  if (e.mode == WG_EPI_SWIGLU)
    gemv_wide_stream_kernel<F, M, NB, KS, WG_EPI_SWIGLU><<<grid, 256, 0, s>>>(mat, x, ldx, y, ldy,
                                                                             e, G);
  else if (e.mode == WG_EPI_ROPE_KV)
    gemv_wide_stream_kernel<F, M, NB, KS, WG_EPI_ROPE_KV><<<grid, 256, 0, s>>>(mat, x, ldx, y,
                                                                              ldy, e, G);
  else
    gemv_wide_stream_kernel<F, M, NB, KS, WG_EPI_STORE><<<grid, 256, 0, s>>>(mat, x, ldx, y, ldy,
                                                                            e, G);
  return launched("wg_q4_gemv (8/6-bit)");
}

// K split so a lane holds at most 2 chunks' activations, and further (while
// every part keeps 64 chunks) when the row groups alone would give fewer
// than gemv_min_waves waves; -1 where the chunks do not fit (K too long).
template <class F, int M>
int launch_stream_k(const Mat &mat, int G, const uint16_t *x, int ldx, float *y, int ldy,
                    const wg_epilogue &ep, hipStream_t s) {
  const int C = mat.C;
  int ks = C <= 64 ? 1 : C <= 128 ? 2 : C <= 512 ? 4 : 0;
  if (!ks) return -1;
  while (ks < 4 && G * ks < tuning("gemv_min_waves") && C / (2 * ks) >= 64) ks *= 2;
  const int nb = (C + ks - 1) / ks > 64 ? 2 : 1;
  if (ks == 1) return launch_stream<F, M, 1, 1>(mat, G, x, ldx, y, ldy, ep, s);
  if (ks == 2) return nb == 1 ? launch_stream<F, M, 1, 2>(mat, G, x, ldx, y, ldy, ep, s)
                              : launch_stream<F, M, 2, 2>(mat, G, x, ldx, y, ldy, ep, s);
  return nb == 1 ? launch_stream<F, M, 1, 4>(mat, G, x, ldx, y, ldy, ep, s)
                 : launch_stream<F, M, 2, 4>(mat, G, x, ldx, y, ldy, ep, s);
}

template <class F, int M>
int launch_rowgroup(const Mat &mat, int G, const uint16_t *x, int ldx, float *y, int ldy,
                    const wg_epilogue &e, hipStream_t s) {
  const unsigned grid = (unsigned)((G + 3) / 4);
  if (e.mode == WG_EPI_SWIGLU)
    gemv_wide_rowgroup_kernel<F, M, WG_EPI_SWIGLU><<<grid, 256, 0, s>>>(mat, x, ldx, y, ldy, e, G);
  else if (e.mode == WG_EPI_ROPE_KV)
    gemv_wide_rowgroup_kernel<F, M, WG_EPI_ROPE_KV><<<grid, 256, 0, s>>>(mat, x, ldx, y, ldy, e,
                                                                        G);
  else
    gemv_wide_rowgroup_kernel<F, M, WG_EPI_STORE><<<grid, 256, 0, s>>>(mat, x, ldx, y, ldy, e, G);
  return launched("wg_q4_gemv (8/6-bit)");
}

template <class F>
int launch_fmt(const Mat &mat, int G, const uint16_t *x, int M, int ldx, float *y, int ldy,
               const wg_epilogue &e, hipStream_t s) {
  if (M <= 2) {
    int rc = M == 1 ? launch_stream_k<F, 1>(mat, G, x, ldx, y, ldy, e, s)
                    : launch_stream_k<F, 2>(mat, G, x, ldx, y, ldy, e, s);
    if (rc != -1) return rc;
  }
  switch (M) {
    case 1: return launch_rowgroup<F, 1>(mat, G, x, ldx, y, ldy, e, s);
    case 2: return launch_rowgroup<F, 2>(mat, G, x, ldx, y, ldy, e, s);
    case 3: return launch_rowgroup<F, 3>(mat, G, x, ldx, y, ldy, e, s);
    case 4: return launch_rowgroup<F, 4>(mat, G, x, ldx, y, ldy, e, s);
    case 5: return launch_rowgroup<F, 5>(mat, G, x, ldx, y, ldy, e, s);
    case 6: return launch_rowgroup<F, 6>(mat, G, x, ldx, y, ldy, e, s);
    case 7: return launch_rowgroup<F, 7>(mat, G, x, ldx, y, ldy, e, s);
    default: return launch_rowgroup<F, 8>(mat, G, x, ldx, y, ldy, e, s);
  }
}

}  // namespace

int launch_gemv_wide(const wg_q4_matrix *w, const uint16_t *x, int M, int ldx, float *y, int ldy,
                     const wg_epilogue &e, hipStream_t s) {
  Mat mat;
  mat.quants = (const uint8_t *)w->quants;
  mat.scales = (const uint16_t *)w->scales;
  const int G = w->N / 4;
  if (w->layout == WG_LAYOUT_Q8) {
    mat.S = w->K / 32;
    mat.C = mat.S;
    return launch_fmt<Q8>(mat, G, x, M, ldx, y, ldy, e, s);
  }
  mat.S = w->K / 256;
  mat.C = mat.S * 4;
  return launch_fmt<Q6K>(mat, G, x, M, ldx, y, ldy, e, s);
}

}  // namespace wg
