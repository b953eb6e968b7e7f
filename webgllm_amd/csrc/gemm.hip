// Prefill GEMM for 4-bit weights on MFMA (the reference's Engine.matmul ->
// matmulQuad, or dequant + matmulF16, src/gpu/kernels.ts:370-429,
// :436-735, planned by Engine.f16Plan, src/engine.ts:980-995):
// C[m][n] = sum_k A[m][k] W[n][k], A half activations [M][K], W a row-group
// 4-bit matrix, C float32.
//
// gfx950 mapping:
//  - a workgroup (4 waves) owns a BM x BN tile of C (BM = 128 tokens; BN =
//    128 features, or 64 for narrow matrices so the grid still covers the
//    256 compute units); each wave owns WM x 32 of it (WM = 128 or 64);
//  - A goes through LDS, BK = 64 at a time, double-buffered; each wave
//    loads its 32 weight rows straight into registers (8 nibble bytes a
//    lane a block) and dequantizes there to halves, d (q - z) rounded once
//    to half as the reference's dequantOut does (packed f16 math: q - z is
//    exact, the product is rounded once);
//  - v_mfma_f32_32x32x16_f16 with float32 accumulation. A 32-weight block
//    is two K = 16 steps: lane half h holds bytes 8h..8h+7, whose low
//    nibbles are weights 8h..8h+7 (the first step) and high nibbles
//    weights 16+8h.. (the second) - natural K order on both operands;
//  - workgroups on one XCD (dispatch order mod 8) take the M tiles of one
//    weight tile one after another, so it is read from HBM once into that
//    XCD's L2.
#include "common.h"
#include "dot.h"

namespace wg {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float16v __attribute__((ext_vector_type(16)));

constexpr int BM = 128, BK = 64;
constexpr int ASTR = BK + 8;  // LDS row stride of the A tile, in halves

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
#pragma unroll
    for (int i = 0; i < 2; i++) {
      uint32_t p0 = __builtin_amdgcn_perm(0u, w[i], SEL01);
      uint32_t p1 = __builtin_amdgcn_perm(0u, w[i], SEL23);
      half2v l0 = as_h2((p0 & LO4) | 0x64006400u) - off2;
      half2v l1 = as_h2((p1 & LO4) | 0x64006400u) - off2;
      half2v h0 = as_h2(((p0 >> 4) & LO4) | 0x64006400u) - off2;
      half2v h1 = as_h2(((p1 >> 4) & LO4) | 0x64006400u) - off2;
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

template <int ZK>
__device__ inline float zero_of(const void *zeros, int64_t si) {
  if constexpr (ZK == WG_ZERO_8) return 8.0f;
  else if constexpr (ZK == WG_ZERO_U8) return (float)((const uint8_t *)zeros)[si];
  else return (float)__builtin_bit_cast(_Float16, ((const uint16_t *)zeros)[si]);
}

// WAVES_N waves across N (32 columns each), 4 / WAVES_N across M (WM rows).
template <int ZK, int WAVES_N>
__global__ __launch_bounds__(256) void gemm_q4_kernel(const uint8_t *__restrict__ quants,
                                                      const uint16_t *__restrict__ scales,
                                                      const void *__restrict__ zeros,
                                                      const uint16_t *__restrict__ A, int lda,
                                                      float *__restrict__ C, int ldc,
                                                      const float *residual, int ldr, int M,
                                                      int N, int K) {
  constexpr int BN = 32 * WAVES_N;
  constexpr int WAVES_M = 4 / WAVES_N;
  constexpr int WM = BM / WAVES_M;
  constexpr int MT = WM / 32;  // 32-row MFMA tiles a wave owns
  __shared__ __align__(16) uint16_t As[2][BM * ASTR];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wn = wave % WAVES_N, wm = wave / WAVES_N;
  // Tile order: XCD x = id % 8 runs the M tiles of weight tile 8 q + x in turn.
  const int tiles_m = (M + BM - 1) / BM, tiles_n = N / BN;
  int id = blockIdx.x, tm, tn;
  if (tiles_n % 8 == 0) {
    const int x = id % 8, j = id / 8;
    tm = j % tiles_m;
    tn = (j / tiles_m) * 8 + x;
  } else {
    tm = id % tiles_m;
    tn = id / tiles_m;
  }
  const int m0 = tm * BM, n0 = tn * BN;
  const int B = K / 32;

  // This lane's weight row and 8-byte half of each block.
  const int n = n0 + wn * 32 + (lane & 31), h = lane >> 5;
  const int64_t row_base = (int64_t)(n >> 2) * B * 4 + (n & 3);  // scale index at block 0
  auto wq = [&](int b) -> uint2 {
    return *reinterpret_cast<const uint2 *>(quants + (row_base + 4 * (int64_t)b) * 16 + 8 * h);
  };

  // A tile loader: 128 rows x 64 halves = 1024 pieces of 16 bytes, 4 a thread.
  uint4 stage[4];
  auto load_a = [&](int kt) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      int piece = tid + 256 * i;
      int r = piece >> 3, c = piece & 7;
      int m = m0 + r;
      stage[i] = m < M ? *reinterpret_cast<const uint4 *>(A + (int64_t)m * lda + kt * BK + 8 * c)
                       : make_uint4(0u, 0u, 0u, 0u);
    }
  };
  auto store_a = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      int piece = tid + 256 * i;
      int r = piece >> 3, c = piece & 7;
      *reinterpret_cast<uint4 *>(&As[buf][r * ASTR + 8 * c]) = stage[i];
    }
  };

  float16v acc[MT];
#pragma unroll
  for (int t = 0; t < MT; t++)
#pragma unroll
    for (int j = 0; j < 16; j++) acc[t][j] = 0.0f;

  const int KT = K / BK;
  uint2 wcur[2], wnext[2];
  uint16_t scur[2], snext[2];
  float zcur[2], znext[2];
  auto load_w = [&](int kt, uint2 *wv, uint16_t *sv, float *zv) {
#pragma unroll
    for (int j = 0; j < 2; j++) {
      int b = kt * 2 + j;
      wv[j] = wq(b);
      int64_t si = row_base + 4 * (int64_t)b;
      sv[j] = scales[si];
      zv[j] = zero_of<ZK>(zeros, si);
    }
  };

  load_a(0);
  load_w(0, wcur, scur, zcur);
  store_a(0);
  for (int kt = 0; kt < KT; kt++) {
    __syncthreads();  // tile kt is in LDS; tile kt - 1's buffer is free
    const bool more = kt + 1 < KT;
    if (more) {
      load_a(kt + 1);
      load_w(kt + 1, wnext, snext, znext);
    }
    const uint16_t *Ab = As[kt & 1];
#pragma unroll
    for (int j = 0; j < 2; j++) {  // the two blocks of this BK
      half8 blo, bhi;
      dequant8<ZK>(wcur[j], scur[j], zcur[j], blo, bhi);
#pragma unroll
      for (int step = 0; step < 2; step++) {  // low nibbles: K 0..15, high: 16..31
        const int k = j * 32 + step * 16 + 8 * h;
#pragma unroll
        for (int t = 0; t < MT; t++) {
          const int r = wm * WM + t * 32 + (lane & 31);
          half8 a = *reinterpret_cast<const half8 *>(&Ab[r * ASTR + k]);
          acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, step ? bhi : blo, acc[t], 0, 0, 0);
        }
      }
    }
    if (more) {
      store_a((kt + 1) & 1);
      wcur[0] = wnext[0];
      wcur[1] = wnext[1];
      scur[0] = snext[0];
      scur[1] = snext[1];
      zcur[0] = znext[0];
      zcur[1] = znext[1];
    }
  }

  // D[j] of lane i: row 8 (j / 4) + 4 (i / 32) + j % 4, column i % 32.
  const int col = n0 + wn * 32 + (lane & 31);
#pragma unroll
  for (int t = 0; t < MT; t++)
#pragma unroll
    for (int j = 0; j < 16; j++) {
      int m = m0 + wm * WM + t * 32 + 8 * (j >> 2) + 4 * h + (j & 3);
      if (m < M) {
        float v = acc[t][j];
        if (residual) v += residual[(int64_t)m * ldr + col];
        C[(int64_t)m * ldc + col] = v;
      }
    }
}

template <int ZK>
int launch(const wg_q4_matrix *w, const uint16_t *A, int M, int lda, float *C, int ldc,
           const float *residual, int ldr, hipStream_t s) {
  const int tiles_m = (M + BM - 1) / BM;
  // 128-wide tiles when they alone cover the compute units, else 64.
  if ((int64_t)tiles_m * (w->N / 128) >= 256 && w->N % 128 == 0) {
    int grid = tiles_m * (w->N / 128);
    gemm_q4_kernel<ZK, 4><<<grid, 256, 0, s>>>((const uint8_t *)w->quants,
                                                (const uint16_t *)w->scales, w->zeros, A, lda,
                                                C, ldc, residual, ldr, M, w->N, w->K);
  } else {
    int grid = tiles_m * (w->N / 64);
    gemm_q4_kernel<ZK, 2><<<grid, 256, 0, s>>>((const uint8_t *)w->quants,
                                                (const uint16_t *)w->scales, w->zeros, A, lda,
                                                C, ldc, residual, ldr, M, w->N, w->K);
  }
  return launched("wg_q4_gemm");
}

}  // namespace
}  // namespace wg

using namespace wg;

extern "C" {

int wg_q4_gemm(const wg_q4_matrix *w, const uint16_t *A, int32_t M, int32_t lda, float *C,
               int32_t ldc, const float *residual, int32_t ldr, void *stream) {
  int rc = check_matrix(w, "wg_q4_gemm");
  if (rc) return rc;
  WG_REQUIRE(w->layout == WG_LAYOUT_ROWGROUP,
             "wg_q4_gemm: the prefill GEMM reads row-group matrices");
  WG_REQUIRE(w->K % 64 == 0, "wg_q4_gemm: columns (%d) must be a multiple of 64", w->K);
  WG_REQUIRE(w->N % 64 == 0, "wg_q4_gemm: rows (%d) must be a multiple of 64", w->N);
  WG_REQUIRE(A && C && M >= 1, "wg_q4_gemm: bad arguments");
  WG_REQUIRE(lda >= w->K && lda % 8 == 0 && ((uintptr_t)A & 15) == 0,
             "wg_q4_gemm: activations need a 16-byte aligned stride >= K");
  WG_REQUIRE(ldc >= w->N, "wg_q4_gemm: ldc %d < N %d", ldc, w->N);
  WG_REQUIRE(!overlaps(A, (size_t)M * lda * 2, C, (size_t)M * ldc * 4),
             "wg_q4_gemm: activations and output overlap");
  if (residual) {
    WG_REQUIRE(ldr >= w->N, "wg_q4_gemm: residual stride %d < N %d", ldr, w->N);
    WG_REQUIRE(residual == C || !overlaps(residual, (size_t)M * ldr * 4, C, (size_t)M * ldc * 4),
               "wg_q4_gemm: residual overlaps the output");
  }
  hipStream_t s = as_stream(stream);
  switch (w->zero) {
    case WG_ZERO_8: return launch<WG_ZERO_8>(w, A, M, lda, C, ldc, residual, ldr, s);
    case WG_ZERO_U8: return launch<WG_ZERO_U8>(w, A, M, lda, C, ldc, residual, ldr, s);
    default: return launch<WG_ZERO_F16>(w, A, M, lda, C, ldc, residual, ldr, s);
  }
}

}  // extern "C"
