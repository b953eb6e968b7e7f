// Prefill GEMM for 4-bit weights on MFMA (the reference's Engine.matmul ->
// matmulQuad, or dequant + matmulF16, src/gpu/kernels.ts:370-429,
// :436-735, planned by Engine.f16Plan, src/engine.ts:980-995):
// C[m][n] = sum_k A[m][k] W[n][k], A half activations [M][K], W a row-group
// 4-bit matrix, C float32.
//
// gfx950 mapping:
//  - a workgroup owns a BM x BN tile of C (128 x 256, 128 x 128 or 64 x 128
//    by shape); its waves split the tile's columns, 32 each, so a wave owns
//    BM x 32 as BM / 32 MFMA tiles of 32 x 32 (v_mfma_f32_32x32x16_f16,
//    float32 accumulation) and every weight is dequantized once per
//    workgroup, feeding BM / 32 MFMAs (the vector work per MFMA, not HBM or
//    LDS, is what bounds this kernel at M = 512);
//  - K goes in steps of 64 (two 32-weight blocks) through an S-stage ring
//    in LDS: each stage holds the A tile (16-byte chunk c of row r at
//    position c ^ (r / 2 % 8), so the 16 rows an operand read takes at once
//    fill all 64 banks), the
//    weight tile's raw nibbles (a row group's two blocks are 128 contiguous
//    bytes), its half scales and its zero points;
//  - stages are filled by direct global-to-LDS loads
//    (global_load_lds_dwordx4, per-lane offsets fixed for the whole K loop
//    from scalar bases that step by a constant), issued S - 1 steps ahead
//    of their use, so
//    every step computes while the next ones stream in. Every wave issues
//    the same number of loads a stage, so "this wave's loads of stage kt
//    have landed" is one vmcnt wait; a workgroup barrier then covers the
//    other waves'. The loads are issued from inline assembly: the compiler
//    cannot tell which in-flight stage a later LDS read depends on and would
//    otherwise wait for all of them;
//  - the K loop is unrolled by S, so every LDS address is an immediate
//    offset;
//  - weights are dequantized from LDS to halves in registers, d (q - z)
//    rounded once as the reference's dequantOut does: 1024 + q as a half
//    (a nibble byte under a 0x64 exponent byte, one byte permute a pair)
//    minus 1024 + z is exact in packed f16, then one multiply by d. A
//    32-weight block is two K = 16 MFMA steps: lane half h takes bytes
//    8h..8h+7 of the block's row, whose low nibbles are weights 8h.. (the
//    first step) and high nibbles 16 + 8h.. (the second) - natural K order
//    on both operands;
//  - workgroups on one XCD (ids equal mod 8, as the dispatcher deals them
//    round-robin) take the M tiles of one weight tile one after another, so
//    it is read from HBM once into that XCD's L2;
//  - when the tiles are fewer than the compute units (M = 512 at N = 4096
//    gives 128 tiles of 128 x 128), K is split KS ways (2 or 4): each
//    workgroup runs one K range of one tile; the splits' float32 sums meet
//    in a fixed pairwise tree (coherent stores and loads, counters put back
//    to zero by their last arriver), and the tile's last workgroup runs the
//    epilogue. The result does not depend on which split ends last.
#include <algorithm>
#include <mutex>
#include <vector>

#include "common.h"
#include "dot.h"
#include "kernels.h"
#include "lds_load.h"

namespace wg {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float16v __attribute__((ext_vector_type(16)));

// 8 nibble bytes of one weight row and block -> the two K = 16 operands
// (low nibbles, high nibbles) as d (q - z), one rounding to half.
template <int ZK>
__device__ inline void dequant8(uint2 bytes, uint16_t scale_bits, float zero, half8 &lo,
                                half8 &hi) {
  const _Float16 d = __builtin_bit_cast(_Float16, scale_bits);
  uint32_t w[2] = {bytes.x, bytes.y};
  if constexpr (ZK != WG_ZERO_F16) {
    // 1024 + q as a half (q in the low mantissa bits), minus 1024 + z: exact.
    const _Float16 off = (_Float16)(1024.0f + zero);
    half2v off2 = {off, off}, d2 = {d, d};
    // The nibbles of a word masked once, low and high; then each half pair
    // is one byte permute that takes two nibble bytes and puts the 0x64
    // exponent byte (from k64) above each.
    const uint32_t k64 = 0x64646464u;
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const uint32_t lo4 = w[i] & 0x0f0f0f0fu, hi4 = (w[i] >> 4) & 0x0f0f0f0fu;
      half2v l0 = as_h2(__builtin_amdgcn_perm(k64, lo4, 0x04010400u)) - off2;
      half2v l1 = as_h2(__builtin_amdgcn_perm(k64, lo4, 0x04030402u)) - off2;
      half2v h0 = as_h2(__builtin_amdgcn_perm(k64, hi4, 0x04010400u)) - off2;
      half2v h1 = as_h2(__builtin_amdgcn_perm(k64, hi4, 0x04030402u)) - off2;
      l0 = l0 * d2;
      l1 = l1 * d2;
      h0 = h0 * d2;
      h1 = h1 * d2;
      lo[4 * i + 0] = l0.x;
      lo[4 * i + 1] = l0.y;
      lo[4 * i + 2] = l1.x;
      lo[4 * i + 3] = l1.y;
      hi[4 * i + 0] = h0.x;
      hi[4 * i + 1] = h0.y;
      hi[4 * i + 2] = h1.x;
      hi[4 * i + 3] = h1.y;
    }
  } else {
    // A fractional zero point: (q - z) in float32 (exact), times d, to half.
    const float df = (float)d;
#pragma unroll
    for (int t = 0; t < 8; t++) {
      uint32_t byte = (w[t >> 2] >> (8 * (t & 3))) & 0xffu;
      lo[t] = (_Float16)(((float)(byte & 15u) - zero) * df);
      hi[t] = (_Float16)(((float)(byte >> 4) - zero) * df);
    }
  }
}

// The weight form of a launch: the three zero-point kinds of 4-bit row
// groups, or Q8 for WG_LAYOUT_Q8 (signed bytes, no zero point).
constexpr int Q8 = 3;

// 8 code bytes of one weight row for each K = 16 step of a block (weights
// 8h.. and 16 + 8h..) -> the two operands as half(d q), rounded once:
// q + 128 (one xor a dword) under a 0x64 exponent byte is the half 1024 +
// q + 128, minus 1152 exact, then one multiply by d.
__device__ inline void dequant8_q8(uint2 b0, uint2 b1, uint16_t scale_bits, half8 &lo,
                                   half8 &hi) {
  const _Float16 d = __builtin_bit_cast(_Float16, scale_bits);
  const half2v off2 = {(_Float16)1152.0f, (_Float16)1152.0f}, d2 = {d, d};
  const uint32_t k64 = 0x64646464u;
  const uint32_t w[4] = {b0.x ^ 0x80808080u, b0.y ^ 0x80808080u, b1.x ^ 0x80808080u,
                         b1.y ^ 0x80808080u};
#pragma unroll
  for (int i = 0; i < 4; i++) {
    half2v p0 = (as_h2(__builtin_amdgcn_perm(k64, w[i], 0x04010400u)) - off2) * d2;
    half2v p1 = (as_h2(__builtin_amdgcn_perm(k64, w[i], 0x04030402u)) - off2) * d2;
    half8 &o = i < 2 ? lo : hi;
    const int t = (i & 1) * 4;
    o[t + 0] = p0.x;
    o[t + 1] = p0.y;
    o[t + 2] = p1.x;
    o[t + 3] = p1.y;
  }
}

template <int ZK, int BN>
struct Stage {
  // weights: BN / 4 row groups x 128 nibble bytes, or x 256 code bytes
  static constexpr int WQ = ZK == Q8 ? BN * 64 : BN * 32;
  static constexpr int WS = BN * 4;   // scales: BN / 4 row groups x 8 halves
  static constexpr int WZ = ZK == WG_ZERO_F16 ? BN * 4 : ZK == WG_ZERO_U8 ? BN * 2 : 0;
};

// Waves a SIMD holds at once, as the LDS ring allows (160 KB a compute
// unit, 4 SIMDs): the register budget the compiler may spend.
template <int ZK, int BM, int BN, int S, int NWV>
constexpr int gemm_waves_per_simd() {
  constexpr int stage = BM * 128 + Stage<ZK, BN>::WQ + Stage<ZK, BN>::WS + Stage<ZK, BN>::WZ;
  constexpr int wgs = (160 * 1024) / (S * stage);
  constexpr int w = (wgs * NWV + 3) / 4;
  return w < 1 ? 1 : w > 8 ? 8 : w;
}

__device__ inline uint16_t half_clamped(float v) {
  v = fminf(fmaxf(v, -65504.0f), 65504.0f);
  return __builtin_bit_cast(uint16_t, (_Float16)v);
}

// How split-K partials pass between the workgroups of one tile, which may
// run on different XCDs (whose L2s are not coherent with each other):
// 16-byte stores with sc1, which reach the point every compute unit sees,
// loads with sc1, which read past the L2, and the count at agent scope.
typedef float f4v __attribute__((ext_vector_type(4)));
__device__ inline void store_part(float *p, f4v v) {
  asm volatile("global_store_dwordx4 %0, %1, off sc1" ::"v"(p), "v"(v) : "memory");
}
// a buffer resource over [base, base + 2^31) (raw 32-bit loads)
__device__ inline __amdgpu_buffer_rsrc_t rsrc_over(const float *base) {
  return __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, 0x7fffffff, 0x00020000);
}
__device__ inline f4v load_part(__amdgpu_buffer_rsrc_t r, size_t floats) {
  return __builtin_bit_cast(
      f4v, __builtin_amdgcn_raw_buffer_load_b128(r, (int)(floats * 4), 0, 16 /* sc1 */));
}
// Counts a group in; true for the one that completes the count, which puts
// the counter back to zero for the next launch.
__device__ inline bool count_in(int *count, int expect) {
  if (__hip_atomic_fetch_add(count, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != expect - 1)
    return false;
  __hip_atomic_store(count, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return true;
}

// BM x BN tiles, S stages of BK = 64, a WGM x WGN grid of waves. With SW the
// matrix's rows come in groups of 4 as (gate 2i, gate 2i + 1, up 2i, up 2i
// + 1) and C is a half output [M][ldc] of N / 2 columns: half(silu(gate) *
// up), as REDUCE_SWIGLU (src/gpu/kernels.ts:1066-1077) computes it from
// the float32 sums.
template <int ZK, int BM, int BN, int S, int WGM, int WGN, bool SW = false, bool PP = false>
__global__ __launch_bounds__(WGM * WGN * 64) __attribute__((amdgpu_waves_per_eu(
    1, gemm_waves_per_simd<ZK, BM, BN, S, WGM * WGN>()))) void gemm_q4_kernel(const uint8_t *__restrict__ quants,
                                                      const uint16_t *__restrict__ scales,
                                                      const void *__restrict__ zeros,
                                                      const uint16_t *__restrict__ A, int lda,
                                                      float *__restrict__ C, int ldc,
                                                      const float *residual, int ldr,
                                                      const float *row_scale,
                                                      const int32_t *col_of, int M, int N,
                                                      int K, int ks, float *part, int *count) {
  constexpr int NWV = WGM * WGN;  // waves
  constexpr int WM = BM / WGM, WN = BN / WGN, MT = WM / 32, NT = WN / 32;
  static_assert(MT >= 1 && NT >= 1 && WM % 32 == 0 && WN % 32 == 0, "32 x 32 MFMA tiles");
  constexpr int A_BYTES = BM * 128;
  constexpr int WQ = Stage<ZK, BN>::WQ, WS = Stage<ZK, BN>::WS, WZ = Stage<ZK, BN>::WZ;
  constexpr int STAGE = A_BYTES + WQ + WS + WZ;
  constexpr int IA = BM * 128 / 1024 / NWV;  // A loads (1 KB each) a wave issues a stage
  static_assert(IA >= 1 && IA * NWV * 1024 == A_BYTES, "A tile splits evenly over the waves");
  // weight pieces (16 bytes) a stage; RGP of them a row group
  constexpr int RGP = ZK == Q8 ? 16 : 8, QP = BN / 4 * RGP;
  constexpr int QSTEP = RGP * 16;  // weight bytes a row group moves a step
  constexpr int IQ = QP > 64 * NWV ? QP / (64 * NWV) : 1;  // nibble loads a wave issues
  constexpr int NW = IA + IQ + 1 + (ZK == WG_ZERO_U8 ? 1 : 0);  // loads a wave issues a stage
  extern __shared__ __align__(16) unsigned char smem[];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WGN, wn = wave % WGN, h = lane >> 5;
  // the ping-pong group: waves 0-3 and 4-7 (wave w runs on SIMD w % 4)
  static_assert(!PP || NWV == 8, "the ping-pong schedule pairs 8 waves");
  [[maybe_unused]] const int group = wave >> 2;
  // Tile order: ids equal mod 8 (one XCD) run the M tiles of one weight
  // tile in turn, so it is read from HBM once into that XCD's L2.
  const int tiles_m = (M + BM - 1) / BM, tiles_n = N / BN, tiles = tiles_m * tiles_n;
  int id = blockIdx.x, tm, tn, split = 0;
  if (ks > 1) {  // workgroup id = split * tiles + tile
    split = id / tiles;
    id -= split * tiles;
  }
  const int tile = id;
  if (tiles_n % 8 == 0) {
    const int x = id % 8, j = id / 8;
    tm = j % tiles_m;
    tn = (j / tiles_m) * 8 + x;
  } else {
    tm = id % tiles_m;
    tn = id / tiles_m;
  }
  const int m0 = tm * BM, n0 = tn * BN, g0 = n0 / 4;
  // this workgroup's K steps of 64: KT of them from step kb
  const int B = K / 32, KT = K / 64 / ks, kb = split * KT;
  const uint32_t sbase = (uint32_t)(uintptr_t)smem;

  // This wave's loads of a step: per-lane byte offsets fixed for the whole
  // K loop, from wave-uniform bases that step kt moves by a fixed stride
  // (A: 64 halves; nibbles: two blocks of 64 bytes a row group; scales and
  // half zero points: 8 halves; u8 zero points: 8 bytes).
  constexpr int PWQ = QP > 64 * NWV ? 64 : QP / NWV;  // lanes a nibble load
  static_assert(PWQ >= 1 && IQ * NWV * PWQ == QP, "nibble pieces");
  constexpr int NSC = BN / 4, PIECES = ZK == WG_ZERO_F16 ? 2 * NSC : NSC, PWS = PIECES / NWV;
  static_assert(PWS >= 1 && PWS * NWV == PIECES && NSC % PWS == 0, "scale pieces");
  constexpr int PWZ = ZK == WG_ZERO_U8 ? 2 * BN / 4 / NWV : 1;
  static_assert(ZK != WG_ZERO_U8 || (PWZ >= 1 && PWZ * NWV * 4 == 2 * BN), "zero-point pieces");
  uint32_t off_a[IA];
#pragma unroll
  for (int i = 0; i < IA; i++) {
    const int p = (i * NWV + wave) * 64 + lane;  // 16-byte piece of the A tile
    const int row = p >> 3, c = (p & 7) ^ ((row >> 1) & 7);
    const int m = min(m0 + row, M - 1);
    off_a[i] = (uint32_t)(((int64_t)m * lda + c * 8) * 2);
  }
  uint32_t off_q[IQ];
#pragma unroll
  for (int i = 0; i < IQ; i++) {
    const int qq = (i * NWV + wave) * PWQ + lane;
    off_q[i] = (uint32_t)(((int64_t)(g0 + qq / RGP) * B) * (QSTEP / 2) + (qq % RGP) * 16);
  }
  const int qs = wave * PWS + lane;
  const bool s_is_zero = wave * PWS >= NSC;  // wave-uniform
  const uint32_t off_s = (uint32_t)((int64_t)(g0 + (s_is_zero ? qs - NSC : qs)) * B * 8);
  const int qz = wave * PWZ + lane;
  const uint32_t off_z = (uint32_t)(((int64_t)(g0 + (qz >> 1)) * B) * 4 + (qz & 1) * 4);
  const unsigned char *s_base =
      s_is_zero ? (const unsigned char *)zeros : (const unsigned char *)scales;
  auto issue = [&](int kt, int st) {
    kt += kb;
    const uint32_t base = sbase + st * STAGE;
#pragma unroll
    for (int i = 0; i < IA; i++)
      dma16((const unsigned char *)A + kt * 128, off_a[i],
            __builtin_amdgcn_readfirstlane(base + (i * NWV + wave) * 1024));
#pragma unroll
    for (int i = 0; i < IQ; i++)
      if (lane < PWQ)
        dma16(quants + kt * QSTEP, off_q[i],
              __builtin_amdgcn_readfirstlane(base + A_BYTES + (i * NWV + wave) * PWQ * 16));
    if (lane < PWS)
      dma16(s_base + kt * 16, off_s,
            __builtin_amdgcn_readfirstlane(base + A_BYTES + WQ + wave * PWS * 16));
    if constexpr (ZK == WG_ZERO_U8) {  // 8 zero-point bytes a row group, 4 at a time
      if (lane < PWZ)
        dma4((const uint8_t *)zeros + kt * 8, off_z,
             __builtin_amdgcn_readfirstlane(base + A_BYTES + WQ + WS + wave * PWZ * 4));
    }
  };

  float16v acc[MT][NT];
#pragma unroll
  for (int t = 0; t < MT; t++)
#pragma unroll
    for (int u = 0; u < NT; u++)
#pragma unroll
      for (int j = 0; j < 16; j++) acc[t][u][j] = 0.0f;

  // A step's dequantized weights (its two blocks), kept in registers from
  // their LDS reads to the step's MFMAs.
  half8 blo[2][NT], bhi[2][NT];
  // The step's weight, scale and zero-point reads from LDS and the dequant.
  auto wreads = [&](const unsigned char *st) {
    const unsigned char *Wq = st + A_BYTES;
    const uint16_t *Ws = reinterpret_cast<const uint16_t *>(st + A_BYTES + WQ);
    uint2 wbytes[2][NT], wbytes2[2][NT];
    uint16_t wsc[2][NT];
    float wz[2][NT];
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int u = 0; u < NT; u++) {
        const int nl = wn * WN + u * 32 + (lane & 31);  // tile-local weight row
        const int rg = nl >> 2, r = nl & 3;
        if constexpr (ZK == Q8) {  // a block row is 32 code bytes, weight j in byte j
          const unsigned char *row = Wq + rg * 256 + j * 128 + r * 32 + 8 * h;
          wbytes[j][u] = *reinterpret_cast<const uint2 *>(row);
          wbytes2[j][u] = *reinterpret_cast<const uint2 *>(row + 16);
        } else {
          wbytes[j][u] =
              *reinterpret_cast<const uint2 *>(Wq + rg * 128 + j * 64 + r * 16 + 8 * h);
        }
        wsc[j][u] = Ws[rg * 8 + j * 4 + r];
        if constexpr (ZK == WG_ZERO_8 || ZK == Q8) wz[j][u] = 8.0f;
        else if constexpr (ZK == WG_ZERO_U8)
          wz[j][u] = (float)(st + A_BYTES + WQ + WS)[rg * 8 + j * 4 + r];
        else
          wz[j][u] = (float)__builtin_bit_cast(
              _Float16, reinterpret_cast<const uint16_t *>(st + A_BYTES + WQ + WS)[rg * 8 + j * 4 + r]);
      }
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int u = 0; u < NT; u++) {
        if constexpr (ZK == Q8) dequant8_q8(wbytes[j][u], wbytes2[j][u], wsc[j][u], blo[j][u], bhi[j][u]);
        else dequant8<ZK>(wbytes[j][u], wsc[j][u], wz[j][u], blo[j][u], bhi[j][u]);
      }
  };
  // The step's A chunks from LDS and its MFMAs.
  auto amfmas = [&](const unsigned char *st) {
    const uint16_t *As = reinterpret_cast<const uint16_t *>(st);
#pragma unroll
    for (int j = 0; j < 2; j++)  // the two blocks of the step
#pragma unroll
      for (int step = 0; step < 2; step++) {  // low nibbles: K 0..15, high: 16..31
        const int c = 4 * j + 2 * step + h;   // 16-byte chunk of the A rows
        half8 av[MT];
#pragma unroll
        for (int t = 0; t < MT; t++) {
          const int row = wm * WM + t * 32 + (lane & 31);
          av[t] = *reinterpret_cast<const half8 *>(As + row * 64 + (c ^ ((row >> 1) & 7)) * 8);
        }
#pragma unroll
        for (int t = 0; t < MT; t++)
#pragma unroll
          for (int u = 0; u < NT; u++)
            acc[t][u] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[t], step ? bhi[j][u] : blo[j][u],
                                                              acc[t][u], 0, 0, 0);
      }
  };
  // (every LDS read of the wave has returned: a stage another wave fills
  // next may follow the next barrier)
  auto reads_done = []() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); };

  for (int s = 0; s < S - 1; s++)
    if (s < KT) issue(s, s);
  // Unrolled by S: a step's stage is a constant, so its LDS addresses are
  // immediate offsets.
  for (int k0 = 0; k0 < KT; k0 += S) {
#pragma unroll
  for (int ss = 0; ss < S; ss++) {
    const int kt = k0 + ss;
    if (kt >= KT) break;
    // this wave's loads of step kt have landed (younger stages may fly on)
    if (kt + S - 2 < KT) wait_vm<NW * (S - 2)>();
    else wait_vm<0>();
    barrier();  // every wave's have, and every wave is done with step kt - 1
    const unsigned char *st = smem + ss * STAGE;
    if constexpr (PP) {
      // Two wave groups half a step apart, one wave of each on every SIMD:
      // between two barriers one group dequantizes while the other runs
      // MFMAs. Group 1 runs step kt - 1's MFMAs, then step kt's dequant;
      // every wave passes two barriers a step. Step kt + S - 1's loads go
      // into step kt - 1's stage after the second, once group 1's MFMAs
      // have read its A chunks. (Holding a step's weights across the
      // barrier takes ~200 registers, one workgroup a compute unit: 13-30%
      // slower than two lock-step workgroups at 512-2048 rows, K 4096.)
      __builtin_amdgcn_sched_barrier(0);
      if (group) {
        if (kt > 0) amfmas(smem + ((ss + S - 1) % S) * STAGE);
      } else {
        wreads(st);
      }
      reads_done();
      __builtin_amdgcn_sched_barrier(0);
      barrier();
      __builtin_amdgcn_sched_barrier(0);
      if (kt + S - 1 < KT) issue(kt + S - 1, (ss + S - 1) % S);
      if (group) wreads(st);
      else amfmas(st);
      reads_done();
      __builtin_amdgcn_sched_barrier(0);
    } else {
      if (kt + S - 1 < KT) issue(kt + S - 1, (ss + S - 1) % S);
      wreads(st);
      amfmas(st);
    }
  }
  }
  if constexpr (PP) {
    if (group && KT > 0) amfmas(smem + ((KT - 1) % S) * STAGE);  // group 1's last step
  }

  if (ks > 1) {
    // The splits' sums meet in a fixed pairwise tree: at level l, group g
    // (the 2^l splits from g 2^l) publishes its sum in slot 2 ks - 2 ks /
    // 2^l + g, and the last of each pair of groups adds its partner's. An
    // addition of two values does not depend on their order, so neither
    // does the result on which workgroup arrives last. Every slot is
    // written once a launch, before anything reads it.
    // A slot holds a tile's sums as fragments: fragment (wave, t, u) is 16
    // floats a lane, stored as four 16-byte pieces a lane (1 KB a store).
    constexpr int FRAG = 16 * 64;  // floats a fragment
    const size_t tile_floats = (size_t)BM * BN;
    auto at = [&](int slot, int t, int u, int j4) {
      return (size_t)(slot * tiles + tile) * tile_floats +
             (size_t)((wave * MT + t) * NT + u) * FRAG + (j4 * 64 + lane) * 4;
    };
    const __amdgpu_buffer_rsrc_t rs = rsrc_over(part);
    __shared__ int last;
    for (int l = 0; (1 << l) < ks; l++) {
      const int g = split >> l;                    // this workgroup's group at level l
      const int level = 2 * ks - ((2 * ks) >> l);  // the level's first slot
#pragma unroll
      for (int t = 0; t < MT; t++)
#pragma unroll
        for (int u = 0; u < NT; u++)
#pragma unroll
          for (int j4 = 0; j4 < 4; j4++) {
            const f4v v = {acc[t][u][4 * j4], acc[t][u][4 * j4 + 1], acc[t][u][4 * j4 + 2],
                           acc[t][u][4 * j4 + 3]};
            store_part(part + at(level + g, t, u, j4), v);
          }
      wait_vm<0>();     // this wave's stores are done
      __syncthreads();  // every wave's are
      if (tid == 0) last = count_in(count + tile * 8 + (ks - (ks >> l)) + (g >> 1), 2);
      // (a full __syncthreads: it waits for the LDS write of `last` before
      // the barrier, which a bare s_barrier does not, and the other waves
      // would read the flag stale)
      __syncthreads();
      if (!last) return;
      const int partner = level + (g ^ 1);
#pragma unroll
      for (int t = 0; t < MT; t++)
#pragma unroll
        for (int u = 0; u < NT; u++) {
          f4v got[4];
#pragma unroll
          for (int j4 = 0; j4 < 4; j4++) got[j4] = load_part(rs, at(partner, t, u, j4));
#pragma unroll
          for (int j4 = 0; j4 < 4; j4++)
#pragma unroll
            for (int e = 0; e < 4; e++) acc[t][u][4 * j4 + e] += got[j4][e];
        }
    }
  }

  // D[j] of lane i: row 8 (j / 4) + 4 (i / 32) + j % 4, column i % 32.
  if constexpr (SW) {
    // Column i % 32's row in its group is i % 4: the gate rows' lanes (0, 1)
    // meet their up rows (2, 3) by a swap within each quad (DPP [2,3,0,1]),
    // which every lane takes part in.
    uint16_t *out16 = reinterpret_cast<uint16_t *>(C);
    const int r = lane & 3;
#pragma unroll
    for (int u = 0; u < NT; u++) {
      const int n = n0 + wn * WN + u * 32 + (lane & 31);
#pragma unroll
      for (int t = 0; t < MT; t++)
#pragma unroll
        for (int j = 0; j < 16; j++) {
          const int m = m0 + wm * WM + t * 32 + 8 * (j >> 2) + 4 * h + (j & 3);
          float v = acc[t][u][j];
          if (row_scale) v *= row_scale[m < M ? m : M - 1];
          const float up = dpp_f<0x4e, 0xf>(v, 0.0f);
          if (m < M && r < 2)
            out16[(int64_t)m * ldc + 2 * (n >> 2) + r] =
                half_clamped(v / (1.0f + __expf(-v)) * up);
        }
    }
    return;
  }
#pragma unroll
  for (int u = 0; u < NT; u++) {
    const int n = n0 + wn * WN + u * 32 + (lane & 31);
    const int col = col_of ? col_of[n] : n;
    if ((unsigned)col >= (unsigned)N) continue;
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
      for (int j = 0; j < 16; j++) {
        const int m = m0 + wm * WM + t * 32 + 8 * (j >> 2) + 4 * h + (j & 3);
        if (m < M) {
          float v = acc[t][u][j];
          if (row_scale) v *= row_scale[m];
          if (residual) v += residual[(int64_t)m * ldr + col];
          C[(int64_t)m * ldc + col] = v;
        }
      }
  }
}

// Puts the split-K counters to zero by the atomic stores the counting uses.
__global__ void split_zero_kernel(int *count, int n) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
    __hip_atomic_store(count + i, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// A split-K workspace per device and stream (launches on one stream run in
// turn; other streams get their own): the partial slots and the tree's
// counters, grown on demand. The counters start at zero and every launch
// leaves them so. A launch recorded into a graph never takes it: a graph
// may replay on another stream, beside eager launches on this one, and
// must not outlive a workspace that grows (is freed and allocated again)
// after the capture; captured GEMMs run unsplit.
struct SplitSpace {
  int dev;
  hipStream_t stream;
  float *part;
  size_t floats;
  int *count;
  int counters;
};

// The workspace for `floats` partial floats and `counters` counters on
// stream s; part stays null while s is being captured into a graph (the
// launch runs unsplit).
int split_space(hipStream_t s, size_t floats, int counters, float **part, int **count) {
  static std::mutex mu;
  static std::vector<SplitSpace *> spaces;
  *part = nullptr;
  *count = nullptr;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &cs) != hipSuccess) {
    (void)hipGetLastError();
    return WG_OK;
  }
  if (cs != hipStreamCaptureStatusNone) return WG_OK;
  int dev = 0;
  WG_HIP(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lock(mu);
  SplitSpace *sp = nullptr;
  for (SplitSpace *x : spaces)
    if (x->dev == dev && x->stream == s) sp = x;
  if (!sp || sp->floats < floats || sp->counters < counters) {
    if (!sp) {
      sp = new SplitSpace{dev, s, nullptr, 0, nullptr, 0};
      spaces.push_back(sp);
    }
    const size_t want = std::max(floats, sp->floats);
    const int want_counters = std::max(counters, sp->counters);
    if (sp->part) {  // launches queued on s may still use the old buffers
      WG_HIP(hipStreamSynchronize(s));
      WG_HIP(hipFree(sp->part));
      WG_HIP(hipFree(sp->count));
      sp->part = nullptr;
      sp->count = nullptr;
      sp->floats = 0;
      sp->counters = 0;
    }
    const size_t round = (want + (1 << 20) - 1) & ~(size_t)((1 << 20) - 1);
    float *p = nullptr;
    int *c = nullptr;
    if (hipMalloc(&p, round * sizeof(float)) != hipSuccess ||
        hipMalloc(&c, (size_t)want_counters * sizeof(int)) != hipSuccess) {
      (void)hipGetLastError();
      if (p) (void)hipFree(p);
      return fail(WG_ERR_OOM, "prefill GEMM: split-K workspace of %zu floats not allocated", round);
    }
    split_zero_kernel<<<(want_counters + 255) / 256, 256, 0, s>>>(c, want_counters);
    WG_HIP(hipGetLastError());
    sp->part = p;
    sp->floats = round;
    sp->count = c;
    sp->counters = want_counters;
  }
  *part = sp->part;
  *count = sp->count;
  return WG_OK;
}

// The halves a WG_ZERO_Q4K matrix's (d', z') are rebuilt into before its
// GEMM, per device and stream as the split-K workspace, grown on demand,
// and never taken by a launch being captured (a graph would keep pointing
// at it after it grows, and may replay beside eager launches).
struct ExpandSpace {
  int dev;
  hipStream_t stream;
  uint16_t *halves;
  size_t count;
};

// `count` halves on stream s, or null while s is being captured.
int expand_space(hipStream_t s, size_t count, uint16_t **out) {
  static std::mutex mu;
  static std::vector<ExpandSpace *> spaces;
  *out = nullptr;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &cs) != hipSuccess) {
    (void)hipGetLastError();
    return WG_OK;
  }
  if (cs != hipStreamCaptureStatusNone) return WG_OK;
  int dev = 0;
  WG_HIP(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lock(mu);
  ExpandSpace *sp = nullptr;
  for (ExpandSpace *x : spaces)
    if (x->dev == dev && x->stream == s) sp = x;
  if (!sp) {
    sp = new ExpandSpace{dev, s, nullptr, 0};
    spaces.push_back(sp);
  }
  if (sp->count < count) {
    if (sp->halves) {  // launches queued on s may still read the old halves
      WG_HIP(hipStreamSynchronize(s));
      WG_HIP(hipFree(sp->halves));
      sp->halves = nullptr;
      sp->count = 0;
    }
    uint16_t *p = nullptr;
    if (hipMalloc(&p, count * sizeof(uint16_t)) != hipSuccess) {
      (void)hipGetLastError();
      return fail(WG_ERR_OOM, "prefill GEMM: %zu halves for Q4_K scales not allocated", count);
    }
    sp->halves = p;
    sp->count = count;
  }
  *out = sp->halves;
  return WG_OK;
}

template <int ZK, int BM, int BN, int S, int WGM = 2, int WGN = 2, bool SW = false,
          bool PP = false>
int launch_tiles(const wg_q4_matrix *w, const uint16_t *A, int M, int lda, float *C, int ldc,
                 const float *residual, int ldr, const float *row_scale, const int32_t *col_of,
                 hipStream_t s) {
  constexpr int STAGE = BM * 128 + Stage<ZK, BN>::WQ + Stage<ZK, BN>::WS + Stage<ZK, BN>::WZ;
  constexpr size_t LDS = (size_t)S * STAGE;
  if (LDS > 64 * 1024) {  // more than 64 KiB of dynamic LDS
    const int rc =
        raise_lds((const void *)gemm_q4_kernel<ZK, BM, BN, S, WGM, WGN, SW, PP>, (int)LDS);
    if (rc) return rc;
  }
  const int tiles = ((M + BM - 1) / BM) * (w->N / BN), steps = w->K / 64;
  // K splits: the knob gemm_splits forces 1, 2, 4 or 8; 0 doubles them (up
  // to 4) while the workgroups stay within two a compute unit (one for the
  // 8-wave tile) and every split keeps at least S steps.
  int ks = tuning("gemm_splits");
  if (ks == 0) {
    const int64_t room = (int64_t)persistent_grid(1 << 30, 1) * (WGM * WGN > 4 ? 1 : 2);
    ks = 1;
    while (ks < 4 && (int64_t)tiles * ks * 2 <= room && steps % (2 * ks) == 0 &&
           steps / (2 * ks) >= S)
      ks *= 2;
  }
  // (the slots are read by 32-bit buffer offsets: under 2 GiB of them)
  if ((ks & (ks - 1)) || ks > 8 || steps % ks ||
      (int64_t)(2 * ks - 2) * tiles * BM * BN * 4 >= ((int64_t)1 << 31))
    ks = 1;
  float *part = nullptr;
  int *count = nullptr;
  if (ks > 1) {
    const int rc =
        split_space(s, (size_t)(2 * ks - 2) * tiles * BM * BN, tiles * 8, &part, &count);
    if (rc) return rc;
    if (!part) ks = 1;
  }
  gemm_q4_kernel<ZK, BM, BN, S, WGM, WGN, SW, PP><<<tiles * ks, WGM * WGN * 64, LDS, s>>>(
      (const uint8_t *)w->quants, (const uint16_t *)w->scales, w->zeros, A, lda, C, ldc,
      residual, ldr, row_scale, col_of, M, w->N, w->K, ks, part, count);
  return launched(SW ? "wg_q4_gemm_swiglu" : "wg_q4_gemm");
}

template <int ZK, bool SW = false>
int launch(const wg_q4_matrix *w, const uint16_t *A, int M, int lda, float *C, int ldc,
           const float *residual, int ldr, const float *row_scale, const int32_t *col_of,
           hipStream_t s) {
  // Each weight is dequantized once per tile, so taller tiles (more rows a
  // wave) spend fewer vector instructions per MFMA: 128 x 256 where its
  // tiles cover most compute units, else 128 x 128 from 512 rows, else 64 x
  // 128; splitting K makes up the workgroups that few tiles leave short.
  // The knob gemm_tile forces one (1: 64 x 128, 2: 128 x 128, 3: 128 x 256).
  const int cus = persistent_grid(1 << 30, 1);
  int t = tuning("gemm_tile");
  if (t == 0) {
    if (w->N % 256 == 0 && (int64_t)((M + 127) / 128) * (w->N / 256) * 4 >= (int64_t)cus * 3) t = 3;
    else if (M >= 512 && w->N % 128 == 0) t = 2;
    else if (w->N % 128 == 0) t = 1;
  }
  if (t == 3 && w->N % 256 == 0) {
    if (tuning("gemm_pingpong"))
      return launch_tiles<ZK, 128, 256, 3, 1, 8, SW, true>(w, A, M, lda, C, ldc, residual, ldr,
                                                           row_scale, col_of, s);
    return launch_tiles<ZK, 128, 256, 3, 1, 8, SW>(w, A, M, lda, C, ldc, residual, ldr, row_scale, col_of, s);
  }
  if (t == 2 && w->N % 128 == 0)
    return launch_tiles<ZK, 128, 128, 3, 1, 4, SW>(w, A, M, lda, C, ldc, residual, ldr, row_scale, col_of, s);
  if (w->N % 128 == 0)
    return launch_tiles<ZK, 64, 128, 4, 1, 4, SW>(w, A, M, lda, C, ldc, residual, ldr, row_scale, col_of, s);
  return launch_tiles<ZK, 64, 64, 5, 1, 2, SW>(w, A, M, lda, C, ldc, residual, ldr, row_scale, col_of, s);
}

}  // namespace
}  // namespace wg

using namespace wg;

static int check_gemm(const wg_q4_matrix *w, const uint16_t *A, int32_t M, int32_t lda,
                      const void *C, const char *who) {
  int rc = check_matrix(w, who);
  if (rc) return rc;
  WG_REQUIRE(w->layout == WG_LAYOUT_ROWGROUP || w->layout == WG_LAYOUT_Q8,
             "%s: the prefill GEMM reads 4-bit and 8-bit row-group matrices", who);
  WG_REQUIRE(w->K % 64 == 0, "%s: columns (%d) must be a multiple of 64", who, w->K);
  WG_REQUIRE(w->N % 64 == 0, "%s: rows (%d) must be a multiple of 64", who, w->N);
  WG_REQUIRE(A && C && M >= 1, "%s: bad arguments", who);
  WG_REQUIRE(lda >= w->K && lda % 8 == 0 && ((uintptr_t)A & 15) == 0,
             "%s: activations need a 16-byte aligned stride >= K", who);
  WG_REQUIRE((int64_t)M * lda * 2 < ((int64_t)1 << 31) && (int64_t)w->N * w->K < ((int64_t)1 << 32),
             "%s: %d x %d activations or a %d x %d matrix past 2 GiB", who, M, lda, w->N, w->K);
  return WG_OK;
}

template <bool SW>
static int dispatch(const wg_q4_matrix *w, const uint16_t *A, int M, int lda, float *C, int ldc,
                    const float *residual, int ldr, const float *row_scale,
                    const int32_t *col_of, hipStream_t s) {
  if (w->layout == WG_LAYOUT_Q8)
    return launch<Q8, SW>(w, A, M, lda, C, ldc, residual, ldr, row_scale, col_of, s);
  if (w->zero == WG_ZERO_Q4K) {
    // packQ4_K's halves rebuilt from the records, then the half-zero-point
    // GEMM over the same quants: the bits of a WG_ZERO_F16 matrix's GEMM
    const size_t blocks = (size_t)w->N * (w->K / 32);
    uint16_t *halves = nullptr;
    int rc = expand_space(s, 2 * blocks, &halves);
    if (rc) return rc;
    if (!halves)
      return fail(WG_ERR_UNSUPPORTED, "%s: a Q4_K-record matrix is not taken under capture",
                  SW ? "wg_q4_gemm_swiglu" : "wg_q4_gemm");
    wg_q4_matrix f = *w;
    f.zero = WG_ZERO_F16;
    f.scales = halves;
    f.zeros = halves + blocks;
    if ((rc = launch_q4k_expand(w, halves, halves + blocks, s))) return rc;
    return launch<WG_ZERO_F16, SW>(&f, A, M, lda, C, ldc, residual, ldr, row_scale, col_of, s);
  }
  switch (w->zero) {
    case WG_ZERO_8: return launch<WG_ZERO_8, SW>(w, A, M, lda, C, ldc, residual, ldr, row_scale, col_of, s);
    case WG_ZERO_U8: return launch<WG_ZERO_U8, SW>(w, A, M, lda, C, ldc, residual, ldr, row_scale, col_of, s);
    default: return launch<WG_ZERO_F16, SW>(w, A, M, lda, C, ldc, residual, ldr, row_scale, col_of, s);
  }
}

extern "C" {

int wg_q4_gemm_swiglu(const wg_q4_matrix *w, const uint16_t *A, int32_t M, int32_t lda,
                      uint16_t *out16, int32_t ldo, const float *row_scale, void *stream) {
  int rc = check_gemm(w, A, M, lda, out16, "wg_q4_gemm_swiglu");
  if (rc) return rc;
  WG_REQUIRE(ldo >= w->N / 2, "wg_q4_gemm_swiglu: ldo %d < N / 2 = %d", ldo, w->N / 2);
  WG_REQUIRE(!overlaps(A, (size_t)M * lda * 2, out16, (size_t)M * ldo * 2),
             "wg_q4_gemm_swiglu: activations and output overlap");
  return dispatch<true>(w, A, M, lda, reinterpret_cast<float *>(out16), ldo, nullptr, 0,
                        row_scale, nullptr, as_stream(stream));
}

int wg_q4_gemm(const wg_q4_matrix *w, const uint16_t *A, int32_t M, int32_t lda, float *C,
               int32_t ldc, const float *residual, int32_t ldr, const float *row_scale,
               const int32_t *col_of, void *stream) {
  int rc = check_matrix(w, "wg_q4_gemm");
  if (rc) return rc;
  WG_REQUIRE(w->layout == WG_LAYOUT_ROWGROUP || w->layout == WG_LAYOUT_Q8,
             "wg_q4_gemm: the prefill GEMM reads 4-bit and 8-bit row-group matrices");
  WG_REQUIRE(w->K % 64 == 0, "wg_q4_gemm: columns (%d) must be a multiple of 64", w->K);
  WG_REQUIRE(w->N % 64 == 0, "wg_q4_gemm: rows (%d) must be a multiple of 64", w->N);
  WG_REQUIRE(A && C && M >= 1, "wg_q4_gemm: bad arguments");
  WG_REQUIRE(lda >= w->K && lda % 8 == 0 && ((uintptr_t)A & 15) == 0,
             "wg_q4_gemm: activations need a 16-byte aligned stride >= K");
  WG_REQUIRE(ldc >= w->N, "wg_q4_gemm: ldc %d < N %d", ldc, w->N);
  WG_REQUIRE((int64_t)M * lda * 2 < ((int64_t)1 << 31) && (int64_t)w->N * w->K < ((int64_t)1 << 32),
             "wg_q4_gemm: %d x %d activations or a %d x %d matrix past 2 GiB", M, lda, w->N,
             w->K);
  WG_REQUIRE(!overlaps(A, (size_t)M * lda * 2, C, (size_t)M * ldc * 4),
             "wg_q4_gemm: activations and output overlap");
  if (residual) {
    WG_REQUIRE(ldr >= w->N, "wg_q4_gemm: residual stride %d < N %d", ldr, w->N);
    WG_REQUIRE(residual == C || !overlaps(residual, (size_t)M * ldr * 4, C, (size_t)M * ldc * 4),
               "wg_q4_gemm: residual overlaps the output");
  }
  return dispatch<false>(w, A, M, lda, C, ldc, residual, ldr, row_scale, col_of,
                         as_stream(stream));
}

}  // extern "C"
