// LFM2's gated short convolution for a batch of tokens, with the state after
// every prefix kept for speculative rollback (the reference's convFused and
// convPrefixes, src/gpu/kernels.ts:1447-1523; Engine.convolve and accept,
// src/engine.ts:5806-5899, :8063-8086, with COPY_ROWS, kernels.ts:2177-2183).
// In_proj rows come as B | C | x (src/weights.ts:180-190); y_t = B_t x_t; the
// output z_t = C_t * sum_k taps[c][k] y[t - (W-1) + k], earlier tokens' y
// from the state (W - 1 rows, oldest first). The state stays float32, as
// the reference's state textures are.
#include "common.h"

namespace wg {
namespace {

constexpr int MAX_W = 8;

__device__ inline uint16_t to_h(float v) {
  v = fminf(fmaxf(v, -65504.0f), 65504.0f);
  return __builtin_bit_cast(uint16_t, (_Float16)v);
}

// Thread = channel c: it reads its channel's old state before writing, so
// state_out may be the state itself.
// A workgroup takes CONV_CH channels and all the batch's tokens, CONV_TOK
// at a time: each thread computes one token's output from the W values of
// y = B x it needs (from the batch, or the state for the first W - 1), so
// the tokens of a channel do not wait on each other. The new state is
// written after a barrier, when every read of the old one (which it may
// replace in place) is done.
constexpr int CONV_CH = 32, CONV_TOK = 8;

template <int W>
__global__ __launch_bounds__(CONV_CH * CONV_TOK) void short_conv_kernel(
    const float *bcx, int M, int D, int ldb, const float *taps, const float *state,
    float *state_out, float *prefixes, uint16_t *out, int ldo) {
  const int tl = threadIdx.x / CONV_CH, c = blockIdx.x * CONV_CH + threadIdx.x % CONV_CH;
  const bool live = c < D;
  // y of token s (s < 0: row W - 1 + s of the state, oldest first)
  auto yval = [&](int s) -> float {
    if (s >= 0) {
      const float *row = bcx + (int64_t)s * ldb;
      return row[c] * row[2 * D + c];
    }
    return state[(int64_t)(W - 1 + s) * D + c];
  };
  if (live) {
    float tp[W];
#pragma unroll
    for (int k = 0; k < W; k++) tp[k] = taps[(int64_t)c * W + k];
    for (int t = tl; t < M; t += CONV_TOK) {
      float y[W];
#pragma unroll
      for (int k = 0; k < W; k++) y[k] = yval(t - (W - 1) + k);
      const float gate = bcx[(int64_t)t * ldb + D + c];
      float a = 0.0f;
#pragma unroll
      for (int k = 0; k < W; k++) a += tp[k] * y[k];
      out[(int64_t)t * ldo + c] = to_h(gate * a);
      if (prefixes)  // the state after the first t + 1 tokens
#pragma unroll
        for (int i = 0; i < W - 1; i++) prefixes[((int64_t)t * (W - 1) + i) * D + c] = y[i + 1];
    }
  }
  float ns[W - 1];
  if (tl == 0 && live)
#pragma unroll
    for (int i = 0; i < W - 1; i++) ns[i] = yval(M - (W - 1) + i);
  __syncthreads();
  if (tl == 0 && live)
#pragma unroll
    for (int i = 0; i < W - 1; i++) state_out[(int64_t)i * D + c] = ns[i];
}

template <int W>
void launch_short_conv(const float *bcx, int M, int D, int ldb, const float *taps,
                       const float *state, float *state_out, float *prefixes, uint16_t *out,
                       int ldo, hipStream_t s) {
  short_conv_kernel<W><<<(D + CONV_CH - 1) / CONV_CH, CONV_CH * CONV_TOK, 0, s>>>(
      bcx, M, D, ldb, taps, state, state_out, prefixes, out, ldo);
}

__global__ void copy_rows_kernel(const float *src, float *dst, int64_t n) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) dst[i] = src[i];
}

}  // namespace
}  // namespace wg

using namespace wg;

extern "C" {

int wg_short_conv(const float *bcx, int32_t M, int32_t D, int32_t ldb, int32_t W,
                  const float *taps, const float *state, float *state_out, float *prefixes,
                  uint16_t *out, int32_t ldo, void *stream) {
  WG_REQUIRE(bcx && taps && state && state_out && out, "wg_short_conv: null argument");
  WG_REQUIRE(M >= 1, "wg_short_conv: %d tokens", M);
  WG_REQUIRE(W >= 2 && W <= MAX_W, "wg_short_conv: width %d (2 to %d)", W, MAX_W);
  WG_REQUIRE(D >= 1 && ldb >= 3 * D && ldo >= D, "wg_short_conv: bad shape");
  WG_REQUIRE(state == state_out || !overlaps(state, (size_t)(W - 1) * D * 4, state_out,
                                             (size_t)(W - 1) * D * 4),
             "wg_short_conv: state and new state partly overlap");
  hipStream_t s = as_stream(stream);
  switch (W) {
#define WG_CONV_W(n) \
  case n: launch_short_conv<n>(bcx, M, D, ldb, taps, state, state_out, prefixes, out, ldo, s); break;
    WG_CONV_W(2) WG_CONV_W(3) WG_CONV_W(4) WG_CONV_W(5) WG_CONV_W(6) WG_CONV_W(7) WG_CONV_W(8)
#undef WG_CONV_W
    default: return wg::fail(WG_ERR_INVALID, "wg_short_conv: width %d", W);
  }
  return launched("wg_short_conv");
}

int wg_conv_accept(const float *prefixes, int32_t kept, int32_t rows, int32_t D, int32_t W,
                   float *state, void *stream) {
  WG_REQUIRE(prefixes && state, "wg_conv_accept: null argument");
  WG_REQUIRE(kept >= 1 && kept <= rows, "wg_conv_accept: can't keep %d of a %d-token batch",
             kept, rows);
  int64_t n = (int64_t)(W - 1) * D;
  copy_rows_kernel<<<(unsigned)((n + 255) / 256), 256, 0, as_stream(stream)>>>(
      prefixes + (int64_t)(kept - 1) * n, state, n);
  return launched("wg_conv_accept");
}

}  // extern "C"
