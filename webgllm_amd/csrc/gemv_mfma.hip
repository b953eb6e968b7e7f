// The few-token GEMV on MFMA: 1 to 8 tokens (a speculative verify batch,
// the reference's split matmul at M <= 8, src/engine.ts:5316-5327) against
// a 4-bit row-group matrix, y = x W^T, with the same epilogues as the
// streaming GEMV.
//
// gfx950 mapping (v_mfma_f32_16x16x32_f16: D[16][16] += A[16][32] B[32][16];
// lane l holds A row l % 16 and B column l % 16 at k = 8 (l / 16) .. + 7, and
// D column l % 16 at rows 4 (l / 16) .. + 3):
//  - a tile is 16 weight rows (4 row groups), the B columns; an MFMA pair
//    covers two 32-weight blocks 2p, 2p + 1 of them. B's k = 0..15 are
//    block 2p (lane chunk c = 0, 1 takes bytes 8c..8c+7 of the row's
//    16-byte block row) and k = 16..31 block 2p + 1 (c = 2, 3). The first
//    MFMA takes those bytes' low nibbles (weights 8c' ..), the second their
//    high nibbles (weights 16 + 8c' ..);
//  - a nibble becomes an exact half with no conversion: for integer zero
//    points (Q4_0's 8, MatMulNBits' bytes) q - z itself, as the nibble under
//    a 1024 exponent (one and-or a pair) minus 1024 + z (one packed add; a
//    high nibble, 16 q under the exponent, takes one packed fma by 1/16);
//    for half zero points (the Q4_K repack) the subnormal q 2^-24 (a mask),
//    with -z sum(a) 2^-24 as the MFMA's float32 C operand. Every product is
//    exact in the f32 sums;
//  - A row t < 8 is token t over block 2p (k < 16, zero at k >= 16), row
//    t >= 8 token t - 8 over block 2p + 1 (k >= 16): D rows 0..7 are the
//    tokens' sums over block 2p, rows 8..15 over block 2p + 1, so each
//    lane's 4 sums are one block's and take that block's scale once;
//  - every wave holds its K slice's A operands (NP pairs, 8 registers
//    each) for the whole kernel; KS waves split K, and their sums meet in
//    LDS once a tile; persistent workgroups stream tiles through DEPTH
//    register sets, the next DEPTH - 1 tiles' weights in flight while one
//    is computed, each loaded from one address a tile (immediate offsets).
#include "common.h"
#include "dot.h"
#include "epilogue.h"
#include "kernels.h"
#include "lds_load.h"

namespace wg {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f4v __attribute__((ext_vector_type(4)));
typedef uint32_t u4v __attribute__((ext_vector_type(4)));

__device__ inline half8 h8(u4v v) { return __builtin_bit_cast(half8, v); }


// A lane's 8 activations (half pairs (a0 a1) (a2 a3) (a4 a5) (a6 a7)) as the
// nibbles unpack: (a0 a2) (a1 a3) (a4 a6) (a5 a7).
__device__ inline u4v pair_order(const uint4 &v) {
  u4v o;
  o[0] = __builtin_amdgcn_perm(v.y, v.x, 0x05040100u);
  o[1] = __builtin_amdgcn_perm(v.y, v.x, 0x07060302u);
  o[2] = __builtin_amdgcn_perm(v.w, v.z, 0x05040100u);
  o[3] = __builtin_amdgcn_perm(v.w, v.z, 0x07060302u);
  return o;
}

__device__ inline half2v as_hv(uint32_t u) { return __builtin_bit_cast(half2v, u); }
__device__ inline uint32_t bits(half2v v) { return __builtin_bit_cast(uint32_t, v); }

constexpr uint32_t BIAS = 0x64006400u;  // (1024, 1024) as halves

// (x & m) | c in one instruction (the compiler splits it in two: the
// three-operand encoding takes no literal, so m and c go in registers).
__device__ inline uint32_t and_or(uint32_t x, uint32_t m, uint32_t c) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "s"(m), "v"(c));
  return r;
}

// 8 nibble bytes (weights 8h'..8h'+7 low, 16+8h'.. high) as the two B
// operands, q - z exactly: lo = (w0 w2) (w1 w3) (w4 w6) (w5 w7), hi the
// same 16 higher. neg = -(1024 + z), neg16 = -(64 + z), both pairs.
__device__ inline void unpack_qz(uint2 q, uint32_t neg, uint32_t neg16, u4v &lo, u4v &hi) {
  const half2v n1 = as_hv(neg), n16 = as_hv(neg16);
  const half2v sixteenth = {(_Float16)0.0625f, (_Float16)0.0625f};
  const uint32_t w[2] = {q.x, q.y};
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const uint32_t t = w[i] >> 8;
    lo[2 * i] = bits(as_hv(and_or(w[i], LO4, BIAS)) + n1);
    lo[2 * i + 1] = bits(as_hv(and_or(t, LO4, BIAS)) + n1);
    hi[2 * i] = bits(__builtin_elementwise_fma(as_hv(and_or(w[i], HI4, BIAS)), sixteenth, n16));
    hi[2 * i + 1] = bits(__builtin_elementwise_fma(as_hv(and_or(t, HI4, BIAS)), sixteenth, n16));
  }
}

// The same bytes as subnormals q 2^-24 (no zero point).
__device__ inline void unpack_sub(uint2 q, u4v &lo, u4v &hi) {
  const uint32_t x0 = q.x, x1 = q.y;
  const uint32_t t0 = x0 >> 8, t1 = x1 >> 8;
  lo[0] = x0 & LO4;
  lo[1] = t0 & LO4;
  lo[2] = x1 & LO4;
  lo[3] = t1 & LO4;
  hi[0] = (x0 >> 4) & LO4;
  hi[1] = t0 >> 4 & LO4;
  hi[2] = (x1 >> 4) & LO4;
  hi[3] = t1 >> 4 & LO4;
}

// One wave's share of a tile in LDS: the nibble, scale and zero bytes of
// its NP block pairs over the tile's 4 row groups, each row group's run
// contiguous in memory and copied in the same order by direct-to-LDS loads
// (16 bytes a lane for nibbles, 4 for scales and zero points).
template <int ZK, int NP>
struct Slot {
  static constexpr int QB = NP * 512;  // 4 row groups x 2 NP blocks x 64 bytes
  static constexpr int SB = NP * 64;   // 4 x 2 NP blocks x 4 rows x 2 bytes
  static constexpr int ZB = ZK == WG_ZERO_U8 ? NP * 32 : ZK == WG_ZERO_F16 ? NP * 64 : 0;
  static constexpr int BYTES = QB + SB + ZB;
  static constexpr int NQ = QB / 1024;           // 16-byte loads of 64 lanes
  static constexpr int NS = (SB + 255) / 256;    // 4-byte loads
  static constexpr int NZ = (ZB + 255) / 256;
  static constexpr int LOADS = NQ + NS + NZ;     // load instructions a wave-tile
};

// Tiles whose K-slice sums wait in LDS before a round of epilogues: up to
// 8, as many as the LDS left by the ring holds (512 bytes a wave a tile).
template <int ZK, int NP, int KS, int S>
constexpr int mfma_round() {
  // (KS * 32: the norm's sums; KS * 128: the pick's parts)
  constexpr int ring = S * KS * Slot<ZK, NP>::BYTES, spare = 160 * 1024 - ring - KS * 160;
  constexpr int r = spare / (KS * 512);
  static_assert(r >= 1, "LDS");
  return r < 8 ? r : 8;
}

// The matrix, its shape and the activations lead the arguments, within the
// 14 dwords that arrive preloaded in scalar registers, so the first ring
// loads wait for no argument fetch.
template <int ZK, int NP, int KS, int S, int MODE>
__global__ __launch_bounds__(KS * 64) void gemv_mfma_kernel(
    const uint8_t *__restrict__ quants, const uint16_t *__restrict__ scales,
    const void *__restrict__ zeros, const uint16_t *__restrict__ x, int G, int B, int ldx, int M,
    float *__restrict__ y, int ldy, const wg_epilogue e) {
  using SL = Slot<ZK, NP>;
  constexpr bool SUB = ZK == WG_ZERO_F16;  // subnormal nibbles, zero point in C
  constexpr int R = mfma_round<ZK, NP, KS, S>();  // tiles a round (their sums wait in LDS)
  constexpr int RGF = (4 * R + KS - 1) / KS;  // row groups a wave finishes a round
  static_assert(NP % 2 == 0 && S >= 1 && (S - 1) * SL::LOADS < 64, "ring shape");
  extern __shared__ __align__(16) unsigned char smem[];
  float *red = reinterpret_cast<float *>(smem + S * KS * SL::BYTES);  // [R][KS][128]
  __shared__ float nred[KS * 8];
  __shared__ PickBest pick_lds[MODE == WG_EPI_STORE ? KS : 1][16];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 15, c = lane >> 4;
  const int bsel = c >> 1, h = c & 1;
  const int b0w = 2 * wave * NP;  // this wave's first block
  // SHORT_CONV: tile t holds the B, C and x row groups of channels 4 t ..
  // 4 t + 3 (row groups t, t + G / 3, t + 2 G / 3) in its first 3 row
  // groups; its 4th repeats the x row group's bytes (L2 hits, its sums
  // unread). G / 3 tiles, each finished on its own: 4 times as many work
  // units as tiles of whole row groups of one part would give.
  constexpr bool CONV = MODE == WG_EPI_SHORT_CONV;
  const int NT = CONV ? G / 3 : (G + 3) >> 2;
  const int ntiles = (NT - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x;
  auto tile_of = [&](int i) { return (int)blockIdx.x + i * (int)gridDim.x; };
  // row group q (0..3) of tile T
  auto rg_of = [&](int T, int q) {
    return CONV ? (uint32_t)(min(q, 2) * NT + T) : (uint32_t)min(4 * T + q, G - 1);
  };
  const uint32_t sbase = (uint32_t)(uintptr_t)smem;

  // This lane's piece of each load: row group and byte offset within the
  // row group's run (blocks past the row read the row's last one).
  int qrg[SL::NQ], srg[SL::NS], zrg[SL::NZ > 0 ? SL::NZ : 1];
  uint32_t qoff[SL::NQ], soff[SL::NS], zoff[SL::NZ > 0 ? SL::NZ : 1];
  bool slive[SL::NS], zlive[SL::NZ > 0 ? SL::NZ : 1];
#pragma unroll
  for (int i = 0; i < SL::NQ; i++) {
    const int o = (i * 64 + lane) * 16, w = o % (NP * 128);
    qrg[i] = o / (NP * 128);
    qoff[i] = (uint32_t)min(b0w + (w >> 6), B - 1) * 64 + (w & 63);
  }
#pragma unroll
  for (int i = 0; i < SL::NS; i++) {
    const int o = (i * 64 + lane) * 4, w = o % (NP * 16);
    slive[i] = o < SL::SB;
    srg[i] = min(o / (NP * 16), 3);
    soff[i] = (uint32_t)min(b0w + (w >> 3), B - 1) * 8 + (w & 7);
  }
  if constexpr (SL::NZ > 0) {
    constexpr int ZPB = ZK == WG_ZERO_U8 ? 4 : 8;  // zero-point bytes a block
#pragma unroll
    for (int i = 0; i < SL::NZ; i++) {
      const int o = (i * 64 + lane) * 4, w = o % (NP * 2 * ZPB);
      zlive[i] = o < SL::ZB;
      zrg[i] = min(o / (NP * 2 * ZPB), 3);
      zoff[i] = (uint32_t)min(b0w + w / ZPB, B - 1) * ZPB + (w % ZPB);
    }
  }
  // The loads of the WG's tile i (< ntiles) into ring stage i % S: exactly
  // SL::LOADS instructions, which the waits below count. Nothing is loaded
  // past the last tile: a wait for an epilogue operand (the compiler's,
  // which does not see these loads and waits for all) would wait for it.
  auto issue = [&](int i) {
    const int T = tile_of(i);
    const uint32_t live = ~0u;
    const uint32_t slot = sbase + (uint32_t)(((i % S) * KS + wave) * SL::BYTES);
#pragma unroll
    for (int k = 0; k < SL::NQ; k++) {
      const uint32_t g = rg_of(T, qrg[k]);
      dma16(quants, (g * (uint32_t)B * 64u + qoff[k]) & live, slot + k * 1024);
    }
#pragma unroll
    for (int k = 0; k < SL::NS; k++) {
      const uint32_t g = rg_of(T, srg[k]);
      if (slive[k]) dma4(scales, (g * (uint32_t)B * 8u + soff[k]) & live, slot + SL::QB + k * 256);
    }
    if constexpr (SL::NZ > 0) {
      constexpr uint32_t ZPB = ZK == WG_ZERO_U8 ? 4 : 8;
#pragma unroll
      for (int k = 0; k < SL::NZ; k++) {
        const uint32_t g = rg_of(T, zrg[k]);
        if (zlive[k])
          dma4(zeros, (g * (uint32_t)B * ZPB + zoff[k]) & live, slot + SL::QB + SL::SB + k * 256);
      }
    }
  };
#pragma unroll
  for (int i = 0; i < S - 1; i++)
    if (i < ntiles) issue(i);

  // A, once: row t = n is token t % 8 over block 2 p + t / 8, on the
  // diagonal chunks only (c / 2 == t / 8). Its loads go out with the norm's
  // parts before either is waited for.
  const int tok = n & 7;
  const bool arow = (n >> 3) == bsel && tok < M;
  uint4 ra[NP], rb[NP];
#pragma unroll
  for (int j = 0; j < NP; j++) {
    const int b = b0w + 2 * j + bsel;
    ra[j] = rb[j] = make_uint4(0u, 0u, 0u, 0u);
    if (arow && b < B) {
      const uint4 *xp = reinterpret_cast<const uint4 *>(x + (int64_t)tok * ldx + 32 * b + 8 * h);
      ra[j] = xp[0];
      rb[j] = xp[2];
    }
  }
  // The norm's parts: this lane's piece of each token's, loaded with A and
  // summed with it (waiting for A waits for every load so far), the waves'
  // sums left in LDS for the first round's barrier; no wave waits for
  // another before the first tile. Parts that a workgroup cannot take in
  // one piece a lane are summed here, behind a barrier.
  float scale[8];
  float4 pt[8];
  const int ip = wave * 64 + lane;
  const bool deferred = e.norm_parts && (((uintptr_t)e.norm_parts) & 15) == 0 &&
                        (e.n_parts & 3) == 0 && (e.ld_parts_in & 3) == 0 &&
                        (e.n_parts >> 2) <= 64 * KS;
  if (deferred) {
#pragma unroll
    for (int t = 0; t < 8; t++) {
      pt[t] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if (t < M && ip < (e.n_parts >> 2))
        pt[t] = reinterpret_cast<const float4 *>(e.norm_parts + (int64_t)t * e.ld_parts_in)[ip];
    }
  } else {
    input_scales_wg<8, KS>(e, scale, nred, M);
  }
  const int pos0 = epi_pos0<MODE>(e);

  if (deferred) {  // token t's sum on lanes 8 t .. 8 t + 7
    float v[8];
#pragma unroll
    for (int t = 0; t < 8; t++) v[t] = (pt[t].x + pt[t].y) + (pt[t].z + pt[t].w);
    const float sum = wave_sum8(v);
    if ((lane & 7) == 0) nred[wave * 8 + (lane >> 3)] = sum;
  }
  u4v alo[NP], ahi[NP];
  float sa[NP];
#pragma unroll
  for (int j = 0; j < NP; j++) {
    const uint4 r0 = ra[j], r1 = rb[j];
    alo[j] = pair_order(r0);
    ahi[j] = pair_order(r1);
    if constexpr (SUB) {  // the block's activation sum (this lane's 16 and the partner chunk's)
      float s = dot2(r0.x, ONES, 0.0f);
      s = dot2(r0.y, ONES, s);
      s = dot2(r0.z, ONES, s);
      s = dot2(r0.w, ONES, s);
      float t = dot2(r1.x, ONES, 0.0f);
      t = dot2(r1.y, ONES, t);
      t = dot2(r1.z, ONES, t);
      t = dot2(r1.w, ONES, t);
      s += t;
      sa[j] = s + xor16(s);
    }
  }
  // SUB: -sum(a) 2^-24 in the D layout (times z a pair): lane (n, c) sums
  // tokens 4 h + i of block 2 p + bsel, whose sum the A lane
  // (8 bsel + 4 h + i) + 32 bsel holds.
  f4v cz[SUB ? NP : 1];
  if constexpr (SUB) {
#pragma unroll
    for (int j = 0; j < NP; j++)
#pragma unroll
      for (int i = 0; i < 4; i++)
        cz[j][i] = -0x1p-24f * __shfl(sa[j], 8 * bsel + 4 * h + i + 32 * bsel, 64);
  }

  // This lane's bytes in a slot: nibbles of (row group n / 4, row n % 4,
  // block 2 j + bsel, half h), then its scale and zero point.
  const uint32_t q_lane = (uint32_t)((n >> 2) * (NP * 128) + bsel * 64 + (n & 3) * 16 + 8 * h);
  const uint32_t s_lane = (uint32_t)(SL::QB + (n >> 2) * (NP * 16) + bsel * 8 + (n & 3) * 2);
  constexpr int ZPB = ZK == WG_ZERO_U8 ? 4 : 8;
  const uint32_t z_lane =
      (uint32_t)(SL::QB + SL::SB + (n >> 2) * (NP * 2 * ZPB) + bsel * ZPB + (n & 3) * (ZPB / 4));

  const int m = lane & 15;
  float my_scale = 0.0f;
  if (!deferred) my_scale = pick<8>(scale, m < 8 ? m : 0) * (SUB ? 0x1p24f : 1.0f);
  const int D = 4 * NT;  // (SHORT_CONV) channels: 4 a tile
  PickBest pbest{PICK_FLOOR, PICK_NONE};  // (pick_parts) this lane's token's best row
  for (int r0 = 0; r0 < ntiles; r0 += R) {
    const int rn = min(R, ntiles - r0);
    // row groups to finish: every one, or a tile's channels (SHORT_CONV)
    const int nfin = CONV ? rn : 4 * rn;
    // the round's epilogue operands, in flight under its tiles (waves w,
    // w + KS, ... of its row groups to finish)
    EpiPre pe[RGF];
#pragma unroll
    for (int f = 0; f < RGF; f++) {
      const int qg = wave + f * KS;
      if constexpr (CONV) {
        if (qg < nfin)
          conv_prefetch(e, 4 * tile_of(r0 + qg) + ((lane >> 4) & 3), D, m < M, pe[f]);
      } else if (qg < nfin) {
        epi_prefetch<8, MODE>(e, 4 * tile_of(r0 + qg / 4) + (qg & 3), G, pos0, pe[f], M);
      }
    }
    for (int i = r0; i < r0 + rn; i++) {
      // tile i's loads are done once at most the later tiles' are in flight
      const int later = min(S - 1, ntiles - 1 - i);
      if (later == S - 1) {
        issue(i + S - 1);
        wait_vm<(S - 1) * SL::LOADS>();
      } else if (S > 2 && later == 1) {
        wait_vm<SL::LOADS>();
      } else if (later == 0) {
        wait_vm<0>();
      } else {
        wait_vm<(S > 3 ? 2 : 1) * SL::LOADS>();  // S = 4, later = 2
      }
      asm volatile("" ::: "memory");
      const unsigned char *slot = smem + ((i % S) * KS + wave) * SL::BYTES;
      f4v acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int j = 0; j < NP; j++) {
        const uint2 q = *reinterpret_cast<const uint2 *>(slot + q_lane + 128 * j);
        const uint16_t sc = *reinterpret_cast<const uint16_t *>(slot + s_lane + 16 * j);
        u4v lo, hi;
        f4v cin = {0.0f, 0.0f, 0.0f, 0.0f};
        if constexpr (SUB) {
          unpack_sub(q, lo, hi);
          const uint16_t zh = *reinterpret_cast<const uint16_t *>(slot + z_lane + 16 * j);
          cin = cz[j] * (float)__builtin_bit_cast(_Float16, zh);
        } else if constexpr (ZK == WG_ZERO_8) {
          unpack_qz(q, 0xE408E408u, 0xD480D480u, lo, hi);  // -1032, -72
        } else {
          const uint32_t zb = slot[z_lane + 8 * j];
          const uint32_t n1 = (0xE400u | zb) * 0x10001u;  // -(1024 + z): ulp 1 there
          const uint32_t n16 =
              (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(-64.0f - (float)zb)) * 0x10001u;
          unpack_qz(q, n1, n16, lo, hi);
        }
        f4v d = __builtin_amdgcn_mfma_f32_16x16x32_f16(h8(alo[j]), h8(lo), cin, 0, 0, 0);
        d = __builtin_amdgcn_mfma_f32_16x16x32_f16(h8(ahi[j]), h8(hi), d, 0, 0, 0);
        acc += (float)__builtin_bit_cast(_Float16, sc) * d;
      }
      // lanes l and l ^ 32: the same row and tokens, blocks 2p and 2p + 1
#pragma unroll
      for (int k = 0; k < 4; k++) acc[k] += xor32(acc[k]);
      if (lane < 32) *reinterpret_cast<f4v *>(red + ((i - r0) * KS + wave) * 128 + lane * 4) = acc;
    }
    // The round's sums are in LDS: finish its 4 rn row groups.
    __builtin_amdgcn_s_waitcnt(0xc07f);  // this wave's LDS writes done
    barrier();
    if (deferred && r0 == 0) {  // this lane's token only
      const int t = m < M ? m : 0;
      float a = 0.0f;
#pragma unroll
      for (int w = 0; w < KS; w++) a += nred[w * 8 + t];
      float v = e.norm_mult / sqrtf(a / (float)e.norm_count + e.eps);
      if (e.row_scale) v *= e.row_scale[t];
      my_scale = v * (SUB ? 0x1p24f : 1.0f);
    }
#pragma unroll
    for (int f = 0; f < RGF; f++) {
      const int qg = wave + f * KS;
      if (qg < nfin) {
        const int r = (lane >> 4) & 3;
        // row 4 jr + r of the round's tile t for token m: at lane (4 jr + r)
        // + 16 (m / 4), slot m % 4
        auto sum_of = [&](int t, int jr) {
          const int src = ((4 * jr + r) + 16 * ((m >> 2) & 1)) * 4 + (m & 3);
          float v = 0.0f;
#pragma unroll
          for (int w = 0; w < KS; w++) v += red[(t * KS + w) * 128 + src];
          return v * my_scale;
        };
        if constexpr (CONV) {
          conv_finish(e, 4 * tile_of(r0 + qg) + r, D, M, sum_of(qg, 0), sum_of(qg, 1),
                      sum_of(qg, 2), m < M, pe[f]);
        } else {
          const int t = qg / 4, jr = qg & 3;
          const int g = 4 * tile_of(r0 + t) + jr;
          const float val = sum_of(t, jr);
          finish_value<MODE>(e, g, val, g < G && m < M, y, ldy, pe[f], pos0);
          if constexpr (MODE == WG_EPI_STORE)
            if (e.pick_parts) pick_take(pbest, val, 4 * g + r, g < G && m < M);
        }
      }
    }
    barrier();  // the sums are read before the next round writes them
  }
  if constexpr (MODE == WG_EPI_STORE)
    if (e.pick_parts) pick_flush<KS>(e, pbest, M, pick_lds);
}

template <int ZK, int NP, int KS, int S>
int launch_mfma(const wg_q4_matrix *w, const uint16_t *x, int M, int ldx, float *y, int ldy,
                const wg_epilogue &e, hipStream_t s) {
  const int G = w->N / 4, B = w->K / 32, NT = (G + 3) / 4;
  constexpr size_t LDS =
      (size_t)S * KS * Slot<ZK, NP>::BYTES + mfma_round<ZK, NP, KS, S>() * KS * 128 * 4;
  static_assert(LDS + KS * 160 <= 160 * 1024, "LDS");
  // (SHORT_CONV: a tile a channel quad.) Workgroups a CU: the knob, or by
  // default 1, and 2 where each still takes 8 tiles or more and two fit the
  // LDS (a 65536-row head at 5 tokens: the verify step 1897 -> 1902 steps/s;
  // with 4 tiles a workgroup, 16384 x 2048, the step was slower)
  const int units = e.mode == WG_EPI_SHORT_CONV ? G / 3 : NT;
  int per_cu = tuning("gemv_mfma_wg_per_cu");
  if (!per_cu)
    per_cu = 2 * (LDS + KS * 160) <= 160 * 1024 && units >= 16 * persistent_grid(1 << 30, 1) ? 2 : 1;
  const int grid = persistent_grid(units, per_cu);
  if (e.pick_parts && grid > WG_PICK_SLOTS)
    return fail(WG_ERR_UNSUPPORTED, "wg_q4_gemv: %d workgroups for the pick's parts", grid);
  auto q = (const uint8_t *)w->quants;
  auto sc = (const uint16_t *)w->scales;
#define WG_MFMA_LAUNCH(MODE)                                                                    \
  do {                                                                                         \
    if (LDS > 64 * 1024) {                                                                     \
      const int rc = raise_lds((const void *)gemv_mfma_kernel<ZK, NP, KS, S, MODE>, (int)LDS); \
      if (rc) return rc;                                                                       \
    }                                                                                          \
    gemv_mfma_kernel<ZK, NP, KS, S, MODE>                                                      \
        <<<grid, KS * 64, LDS, s>>>(q, sc, w->zeros, x, G, B, ldx, M, y, ldy, e);              \
  } while (0)
  if (e.mode == WG_EPI_SHORT_CONV) WG_MFMA_LAUNCH(WG_EPI_SHORT_CONV);
  else if (e.mode == WG_EPI_SWIGLU) WG_MFMA_LAUNCH(WG_EPI_SWIGLU);
  else if (e.mode == WG_EPI_ROPE_KV) WG_MFMA_LAUNCH(WG_EPI_ROPE_KV);
  else WG_MFMA_LAUNCH(WG_EPI_STORE);
#undef WG_MFMA_LAUNCH
  return launched("wg_q4_gemv");
}

template <int ZK>
int launch_mfma_k(const wg_q4_matrix *w, const uint16_t *x, int M, int ldx, float *y, int ldy,
                  const wg_epilogue &e, hipStream_t s) {
  const int P = (w->K / 32 + 1) / 2;  // block pairs a row
  if (P < 2 || (int64_t)w->N * (w->K / 32) >= (1 << 26)) return -1;  // 32-bit byte offsets
  // pairs a wave (8 registers of A each): fewer give more waves a workgroup
  const int np = tuning("gemv_mfma_pairs");
  if (P <= 8) return launch_mfma<ZK, 2, 4, 4>(w, x, M, ldx, y, ldy, e, s);
  if (P <= 16) return np <= 2 ? launch_mfma<ZK, 2, 8, 4>(w, x, M, ldx, y, ldy, e, s)
                              : launch_mfma<ZK, 4, 4, 4>(w, x, M, ldx, y, ldy, e, s);
  // (8 waves of 4 pairs: a 2-stage ring, measured faster than 3 to 6 stages
  // on every 2048-deep matrix from 2048 to 65536 rows at 3, 5 and 8 tokens)
  if (P <= 32) return np <= 4 ? launch_mfma<ZK, 4, 8, 2>(w, x, M, ldx, y, ldy, e, s)
                              : launch_mfma<ZK, 8, 4, 3>(w, x, M, ldx, y, ldy, e, s);
  if (P <= 64) return np <= 4 ? launch_mfma<ZK, 4, 16, 3>(w, x, M, ldx, y, ldy, e, s)
                              : launch_mfma<ZK, 8, 8, 3>(w, x, M, ldx, y, ldy, e, s);
  // 16 waves of 8 pairs: a tile's 16 rows fill most of the LDS, so the ring
  // holds two (one with zero-point bytes); half zero points' C terms do not
  // fit the registers a wave of 16 has
  if constexpr (ZK != WG_ZERO_F16)
    if (P <= 128) return launch_mfma<ZK, 8, 16, ZK == WG_ZERO_8 ? 2 : 1>(w, x, M, ldx, y, ldy, e, s);
  return -1;
}

}  // namespace

int launch_gemv_mfma(const wg_q4_matrix *w, const uint16_t *x, int M, int ldx, float *y,
                     int ldy, const wg_epilogue &e, hipStream_t s) {
  const int mode = tuning("gemv_mfma");
  if (!mode || M < 1 || M > 8 || (M <= 2 && mode < 2)) return -1;
  if (w->zero == WG_ZERO_Q4K) return -1;  // (Q4_K records: the streaming kernels)
  switch (w->zero) {
    case WG_ZERO_8: return launch_mfma_k<WG_ZERO_8>(w, x, M, ldx, y, ldy, e, s);
    case WG_ZERO_U8: return launch_mfma_k<WG_ZERO_U8>(w, x, M, ldx, y, ldy, e, s);
    default: return launch_mfma_k<WG_ZERO_F16>(w, x, M, ldx, y, ldy, e, s);
  }
}

}  // namespace wg
