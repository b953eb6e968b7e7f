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

template <int M>
__global__ __launch_bounds__(256) void gemv_q4k_kernel(const uint8_t *__restrict__ quants,
                                                       const uint16_t *__restrict__ x, int ldx,
                                                       float *__restrict__ y, int ldy,
                                                       const float *residual, int ldr,
                                                       const float *__restrict__ row_scale,
                                                       int G, int S) {
  const int lane = threadIdx.x & 63;
  const int g = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (g >= G) return;
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
  // Reduce over c (lane bits 0-1) and sb (bits 3-5); rp (bit 2) keeps rows apart.
#pragma unroll
  for (int r = 0; r < 2; r++)
#pragma unroll
    for (int m = 0; m < M; m++) {
      float v = acc[r][m];
      v += __shfl_xor(v, 1, 64);
      v += __shfl_xor(v, 2, 64);
      v += __shfl_xor(v, 8, 64);
      v += __shfl_xor(v, 16, 64);
      v += __shfl_xor(v, 32, 64);
      if ((lane & ~4) == 0) {  // lanes 0 (rows 0, 1) and 4 (rows 2, 3)
        int n = 4 * g + 2 * rp + r;
        v *= 0x1p24f;
        if (row_scale) v *= row_scale[m];
        if (residual) v += residual[(int64_t)m * ldr + n];
        y[(int64_t)m * ldy + n] = v;
      }
    }
}

template <int M>
int launch_m(const wg_q4_matrix *w, const uint16_t *x, int ldx, float *y, int ldy,
             const wg_epilogue *ep, hipStream_t s) {
  int G = w->N / 4, S = w->K / 256;
  gemv_q4k_kernel<M><<<(G + 3) / 4, 256, 0, s>>>(
      (const uint8_t *)w->quants, x, ldx, y, ldy, ep ? ep->residual : nullptr,
      ep ? ep->ld_residual : 0, ep ? ep->row_scale : nullptr, G, S);
  return launched("wg_q4_gemv (Q4_K)");
}

}  // namespace

int launch_gemv_q4k(const wg_q4_matrix *w, const uint16_t *x, int M, int ldx, float *y, int ldy,
                    const wg_epilogue *ep, hipStream_t s) {
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
