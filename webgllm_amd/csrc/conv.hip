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
__global__ void short_conv_kernel(const float *bcx, int M, int D, int ldb, int W,
                                  const float *taps, const float *state, float *state_out,
                                  float *prefixes, uint16_t *out, int ldo) {
  int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= D) return;
  const int w1 = W - 1;
  // win: the last W - 1 values of y (oldest first), slid along the tokens
  float win[MAX_W - 1];
  for (int i = 0; i < w1; i++) win[i] = state[(int64_t)i * D + c];
  float tp[MAX_W];
  for (int k = 0; k < W; k++) tp[k] = taps[(int64_t)c * W + k];
  for (int t = 0; t < M; t++) {
    const float *row = bcx + (int64_t)t * ldb;
    const float y = row[c] * row[2 * D + c];
    float a = 0.0f;
    for (int k = 0; k < w1; k++) a += tp[k] * win[k];
    a += tp[w1] * y;
    out[(int64_t)t * ldo + c] = to_h(row[D + c] * a);
    for (int k = 0; k + 1 < w1; k++) win[k] = win[k + 1];
    win[w1 - 1] = y;
    if (prefixes)  // the state after the first t + 1 tokens
      for (int i = 0; i < w1; i++) prefixes[((int64_t)t * w1 + i) * D + c] = win[i];
  }
  for (int i = 0; i < w1; i++) state_out[(int64_t)i * D + c] = win[i];
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
  short_conv_kernel<<<(D + 255) / 256, 256, 0, as_stream(stream)>>>(
      bcx, M, D, ldb, W, taps, state, state_out, prefixes, out, ldo);
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
