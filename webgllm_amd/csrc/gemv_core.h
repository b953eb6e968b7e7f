// Shared pieces of the 4-bit GEMVs: nibble unpacking to fp16 subnormals,
// block dot products, zero points, and the streamed unit of one row group
// (a lane's blocks of the group's 4 rows with their scales and zeros).
#pragma once

#include "common.h"
#include "dot.h"

namespace wg {

// The 16 fp16-subnormal nibble pairs of one 16-byte block row, in the
// order the activation pairs come: for word w, (q[4w], q[4w+1]) and
// (q[4w+2], q[4w+3]) (low nibbles, factor 1), then (q[16+4w], q[17+4w]) and
// (q[18+4w], q[19+4w]) (high nibbles, factor 16).
struct Nibbles {
  uint32_t lo[8], hi[8];
};

__device__ inline void unpack(const uint4 &q, Nibbles &n) {
  uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
  for (int i = 0; i < 4; i++) {
    uint32_t p0 = __builtin_amdgcn_perm(0u, w[i], SEL01);
    uint32_t p1 = __builtin_amdgcn_perm(0u, w[i], SEL23);
    n.lo[2 * i] = p0 & LO4;
    n.lo[2 * i + 1] = p1 & LO4;
    n.hi[2 * i] = p0 & HI4;
    n.hi[2 * i + 1] = p1 & HI4;
  }
}

// sum q a over a block, times 2^-24: a[0..3] are the 32 activations as 16
// half pairs, a[0], a[1] elements 0..15, a[2], a[3] 16..31.
__device__ inline float block_dot(const Nibbles &n, const uint4 *a) {
  const uint32_t lo_a[8] = {a[0].x, a[0].y, a[0].z, a[0].w, a[1].x, a[1].y, a[1].z, a[1].w};
  const uint32_t hi_a[8] = {a[2].x, a[2].y, a[2].z, a[2].w, a[3].x, a[3].y, a[3].z, a[3].w};
  float lo = 0.0f, hi = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    lo = dot2(n.lo[i], lo_a[i], lo);
    hi = dot2(n.hi[i], hi_a[i], hi);
  }
  return __builtin_fmaf(hi, 0.0625f, lo);
}

__device__ inline float block_sum(const uint4 *a) {
  float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    s0 = dot2(a[i].x, ONES, s0);
    s1 = dot2(a[i].y, ONES, s1);
    s0 = dot2(a[i].z, ONES, s0);
    s1 = dot2(a[i].w, ONES, s1);
  }
  return s0 + s1;
}

template <int ZK>
__device__ inline void load_zeros(const void *zeros, int64_t si, float z[4]) {
  if constexpr (ZK == WG_ZERO_8) {
    z[0] = z[1] = z[2] = z[3] = 8.0f;
  } else if constexpr (ZK == WG_ZERO_U8) {
    uint32_t v = *reinterpret_cast<const uint32_t *>((const uint8_t *)zeros + si);
    z[0] = (float)(v & 0xffu);
    z[1] = (float)((v >> 8) & 0xffu);
    z[2] = (float)((v >> 16) & 0xffu);
    z[3] = (float)(v >> 24);
  } else {
    uint2 v = *reinterpret_cast<const uint2 *>((const uint16_t *)zeros + si);
    z[0] = (float)as_h2(v.x).x;
    z[1] = (float)as_h2(v.x).y;
    z[2] = (float)as_h2(v.y).x;
    z[3] = (float)as_h2(v.y).y;
  }
}


// WG_ZERO_Q4K: the record's (d, dmin) words of row group g's super-block
// holding block b (every lane of the super-block loads the same 16 bytes),
// and the block's 48 bits of 6-bit scales and mins (block 2i at dword 3i,
// 2i + 1 at dword 3i + 1, 16 bits in) as lo (bits 0-31) and hi (32-47).
__device__ inline void q4k_load(const void *scales, int64_t g, int B, int b, uint4 &dd,
                                uint2 &bits) {
  const uint8_t *rec =
      reinterpret_cast<const uint8_t *>(scales) + (g * (B / 8) + (b >> 3)) * Q4K_REC;
  const int jb = b & 7;
  dd = *reinterpret_cast<const uint4 *>(rec);
  const uint2 w2 = *reinterpret_cast<const uint2 *>(rec + 16 + 4 * (3 * (jb >> 1) + (jb & 1)));
  const uint32_t sh = (uint32_t)(jb & 1) * 16u;
  bits.x = __builtin_amdgcn_alignbit(w2.y, w2.x, sh);
  bits.y = w2.y >> sh;
}
// The 4 rows' d' = half(d sc), exactly as packQ4_K rounds it, and zero terms
// c = dmin m (their products exact in float32), from q4k_load's words: a
// block weighs d' q - c, where packQ4_K's d' half(dmin m / d') rounds c to
// a half's precision.
__device__ inline void q4k_dc(const uint4 &dd, const uint2 &bits, float (&d)[4], float (&c)[4]) {
  const uint32_t lo = bits.x, hi = bits.y;
  const uint32_t sc[4] = {lo & 63u, (lo >> 12) & 63u, (lo >> 24) & 63u, (hi >> 4) & 63u};
  const uint32_t mn[4] = {(lo >> 6) & 63u, (lo >> 18) & 63u,
                          __builtin_amdgcn_alignbit(hi, lo, 30) & 63u, (hi >> 10) & 63u};
  const uint32_t dw[4] = {dd.x, dd.y, dd.z, dd.w};
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const float dr = (float)as_h2(dw[r]).x, mr = (float)as_h2(dw[r]).y;
    d[r] = (float)(_Float16)(dr * (float)sc[r]);
    c[r] = mr * (float)mn[r];
  }
}

// The streamed unit of one row group for one lane: NB blocks (b0, b0 + 64,
// ...) of the group's 4 rows, their half scales and zero points; or, for
// WG_ZERO_Q4K, the 4 rows' (d, dmin) of the block's super-block and the
// block's 48 bits of 6-bit scales and mins.
template <int ZK, int NB>
struct Unit {
  uint4 q[NB][4];
  uint2 sc[NB];
  uint2 zr[NB];  // u8: .x holds 4 zero points; f16: 4 halves; Q4K: the 48 bits
  uint4 dd[ZK == WG_ZERO_Q4K ? NB : 1];
};

template <int ZK, int NB>
__device__ inline void load_unit(Unit<ZK, NB> &u, const uint4 *__restrict__ quants,
                                 const uint16_t *__restrict__ scales,
                                 const void *__restrict__ zeros, int g, int B, int b0, int b_end,
                                 bool live) {
#pragma unroll
  for (int j = 0; j < NB; j++) {
    int b = b0 + 64 * j;
    if (live && b < b_end) {
      int64_t si = ((int64_t)g * B + b) * 4;
      const uint4 *qp = quants + si;
      u.q[j][0] = qp[0];
      u.q[j][1] = qp[1];
      u.q[j][2] = qp[2];
      u.q[j][3] = qp[3];
      u.sc[j] = *reinterpret_cast<const uint2 *>(scales + si);
      if constexpr (ZK == WG_ZERO_U8)
        u.zr[j].x = *reinterpret_cast<const uint32_t *>((const uint8_t *)zeros + si);
      if constexpr (ZK == WG_ZERO_F16)
        u.zr[j] = *reinterpret_cast<const uint2 *>((const uint16_t *)zeros + si);
    } else {
      u.sc[j] = make_uint2(0u, 0u);  // scale 0: contributes nothing
      u.q[j][0] = u.q[j][1] = u.q[j][2] = u.q[j][3] = make_uint4(0u, 0u, 0u, 0u);
      u.zr[j] = make_uint2(0u, 0u);
    }
  }
}


// acc[r][m] += the unit's 4 rows times token m's activations (units of
// 2^-24): per block, d * (sum q a - z * sum a).
template <int M, int ZK, int NB>
__device__ inline void accumulate_unit(const Unit<ZK, NB> &u, const uint4 (&a)[M][NB][4],
                                       const float (&sa)[M][NB], float (&acc)[4][M]) {
#pragma unroll
  for (int j = 0; j < NB; j++) {
    float d[4] = {(float)as_h2(u.sc[j].x).x, (float)as_h2(u.sc[j].x).y,
                  (float)as_h2(u.sc[j].y).x, (float)as_h2(u.sc[j].y).y};
    float z[4];
    if constexpr (ZK == WG_ZERO_8) {
      z[0] = z[1] = z[2] = z[3] = 8.0f;
    } else if constexpr (ZK == WG_ZERO_U8) {
      uint32_t v = u.zr[j].x;
      z[0] = (float)(v & 0xffu);
      z[1] = (float)((v >> 8) & 0xffu);
      z[2] = (float)((v >> 16) & 0xffu);
      z[3] = (float)(v >> 24);
    } else {
      z[0] = (float)as_h2(u.zr[j].x).x;
      z[1] = (float)as_h2(u.zr[j].x).y;
      z[2] = (float)as_h2(u.zr[j].y).x;
      z[3] = (float)as_h2(u.zr[j].y).y;
    }
#pragma unroll
    for (int r = 0; r < 4; r++) {
      Nibbles n;
      unpack(u.q[j][r], n);
#pragma unroll
      for (int m = 0; m < M; m++) {
        float v = block_dot(n, a[m][j]);
        v = __builtin_fmaf(-z[r], sa[m][j], v);
        acc[r][m] = __builtin_fmaf(d[r], v, acc[r][m]);
      }
    }
  }
}

// The unit of row group g at blocks bj[j] (every index in range: the caller
// clamps), loaded with no branches.
template <int ZK, int NB>
__device__ inline void load_unit_at(Unit<ZK, NB> &u, const uint4 *__restrict__ quants,
                                    const uint16_t *__restrict__ scales,
                                    const void *__restrict__ zeros, int g, int B,
                                    const int (&bj)[NB]) {
#pragma unroll
  for (int j = 0; j < NB; j++) {
    const int64_t si = ((int64_t)g * B + bj[j]) * 4;
    const uint4 *qp = quants + si;
    u.q[j][0] = qp[0];
    u.q[j][1] = qp[1];
    u.q[j][2] = qp[2];
    u.q[j][3] = qp[3];
    if constexpr (ZK == WG_ZERO_Q4K) {
      q4k_load(scales, g, B, bj[j], u.dd[j], u.zr[j]);
    } else {
      u.sc[j] = *reinterpret_cast<const uint2 *>(scales + si);
    }
    if constexpr (ZK == WG_ZERO_U8)
      u.zr[j].x = *reinterpret_cast<const uint32_t *>((const uint8_t *)zeros + si);
    if constexpr (ZK == WG_ZERO_F16)
      u.zr[j] = *reinterpret_cast<const uint2 *>((const uint16_t *)zeros + si);
  }
}

// A block's 32 activations paired as the nibbles are unpacked below: for
// each of its halves (elements 0..15, then 16..31) and dword i < 4, even
// (a_4i, a_4i+2) and odd (a_4i+1, a_4i+3).
struct PairedActs {
  uint32_t e[2][4], o[2][4];
};

__device__ inline void pair_acts(const uint4 (&a)[4], PairedActs &p) {
  const uint32_t d[16] = {a[0].x, a[0].y, a[0].z, a[0].w, a[1].x, a[1].y, a[1].z, a[1].w,
                          a[2].x, a[2].y, a[2].z, a[2].w, a[3].x, a[3].y, a[3].z, a[3].w};
#pragma unroll
  for (int h = 0; h < 2; h++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      p.e[h][i] = __builtin_amdgcn_perm(d[8 * h + 2 * i + 1], d[8 * h + 2 * i], 0x05040100u);
      p.o[h][i] = __builtin_amdgcn_perm(d[8 * h + 2 * i + 1], d[8 * h + 2 * i], 0x07060302u);
    }
}

// v_perm_b32 selector: bytes 1 and 3 into the low byte of each half.
constexpr uint32_t SEL13 = 0x0c030c01u;

// sum q a over a block (times 2^-24) from one 16-byte block row: nibble
// dword i holds weights 4i..4i+3 low and 16+4i.. high; the pairs (q_4i,
// q_4i+2) take one mask, (q_4i+1, q_4i+3) a permute and a mask, and meet
// the activations paired by pair_acts.
__device__ inline float block_dot_paired(const uint4 &q, const PairedActs &p) {
  const uint32_t w[4] = {q.x, q.y, q.z, q.w};
  float lo = 0.0f, hi = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const uint32_t t = __builtin_amdgcn_perm(0u, w[i], SEL13);
    lo = dot2(w[i] & LO4, p.e[0][i], lo);
    hi = dot2(w[i] & HI4, p.e[1][i], hi);
    lo = dot2(t & LO4, p.o[0][i], lo);
    hi = dot2(t & HI4, p.o[1][i], hi);
  }
  return __builtin_fmaf(hi, 0.0625f, lo);
}

// acc[r][m] += the unit's 4 rows times token m's paired activations (units
// of 2^-24), blocks whose lane has no block (live[j] false) adding zero.
template <int M, int ZK, int NB>
__device__ inline void accumulate_unit_paired(const Unit<ZK, NB> &u,
                                              const PairedActs (&a)[M][NB],
                                              const float (&sa)[M][NB], const bool (&live)[NB],
                                              float (&acc)[4][M]) {
#pragma unroll
  for (int j = 0; j < NB; j++) {
    if constexpr (ZK == WG_ZERO_Q4K) {
      float d[4], c[4];
      q4k_dc(u.dd[j], u.zr[j], d, c);
#pragma unroll
      for (int r = 0; r < 4; r++) {
        d[r] = live[j] ? d[r] : 0.0f;
        c[r] = live[j] ? c[r] : 0.0f;
      }
#pragma unroll
      for (int r = 0; r < 4; r++)
#pragma unroll
        for (int m = 0; m < M; m++) {
          const float v = block_dot_paired(u.q[j][r], a[m][j]);
          acc[r][m] = __builtin_fmaf(d[r], v, acc[r][m]);
          acc[r][m] = __builtin_fmaf(-c[r], sa[m][j], acc[r][m]);
        }
      continue;
    }
    float d[4] = {(float)as_h2(u.sc[j].x).x, (float)as_h2(u.sc[j].x).y,
                  (float)as_h2(u.sc[j].y).x, (float)as_h2(u.sc[j].y).y};
#pragma unroll
    for (int r = 0; r < 4; r++) d[r] = live[j] ? d[r] : 0.0f;
    float z[4];
    if constexpr (ZK == WG_ZERO_8) {
      z[0] = z[1] = z[2] = z[3] = 8.0f;
    } else if constexpr (ZK == WG_ZERO_U8) {
      uint32_t v = u.zr[j].x;
      z[0] = (float)(v & 0xffu);
      z[1] = (float)((v >> 8) & 0xffu);
      z[2] = (float)((v >> 16) & 0xffu);
      z[3] = (float)(v >> 24);
    } else {
      z[0] = (float)as_h2(u.zr[j].x).x;
      z[1] = (float)as_h2(u.zr[j].x).y;
      z[2] = (float)as_h2(u.zr[j].y).x;
      z[3] = (float)as_h2(u.zr[j].y).y;
    }
#pragma unroll
    for (int r = 0; r < 4; r++)
#pragma unroll
      for (int m = 0; m < M; m++) {
        float v = block_dot_paired(u.q[j][r], a[m][j]);
        v = __builtin_fmaf(-z[r], sa[m][j], v);
        acc[r][m] = __builtin_fmaf(d[r], v, acc[r][m]);
      }
  }
}

}  // namespace wg
