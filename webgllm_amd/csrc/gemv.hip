// Decode / few-token GEMV for 4-bit weights (the reference's
// matmulSplitRgba4 and split matmul, src/gpu/kernels.ts:744-895, :163-296,
// dispatched by Engine.splitPartials, src/engine.ts:5241-5377).
//
// Bandwidth-bound, no MFMA. Mapping on gfx950 (wave64):
//  - one wave per row group of 4 rows (the layout keeps a row group's block
//    rows together: 64 contiguous bytes per block);
//  - lane l takes blocks l, l + 64, ...: per block it loads the 4 rows'
//    16-byte nibble rows (4 x 128-bit loads, 64 B contiguous), their 4 half
//    scales (one 64-bit load) and zero points, and the block's 32 half
//    activations per token (4 x 128-bit loads, L1/L2 hits: every wave reads
//    the same x);
//  - nibbles are unpacked as fp16 subnormals: a byte permute puts two
//    bytes' nibbles in the two halves of a dword, and masking 0x000f000f
//    (0x00f000f0) leaves q * 2^-24 (16 q * 2^-24) in each half, exactly. One
//    v_dot2_f32_f16 then multiplies two weights by two activations with
//    float32 accumulation, so the block sum b = sum q a costs ~1.25 VALU
//    ops a weight;
//  - per block and row, acc += d * (b - z * sa) with sa = sum a (the same
//    identity the reference's shaders use), kept in units of 2^-24 until the
//    epilogue;
//  - a butterfly over the 64 lanes reduces the 4 rows x M tokens.
#include "common.h"
#include "dot.h"
#include "kernels.h"
#include "epilogue.h"
#include "gemv_core.h"
#include "gemv_stream.h"

namespace wg {
namespace {

template <int M, int ZK, int MODE>
__global__ __launch_bounds__(256) void gemv_rowgroup_kernel(
    const uint4 *__restrict__ quants, const uint16_t *__restrict__ scales,
    const void *__restrict__ zeros, const uint16_t *__restrict__ x, int ldx,
    float *__restrict__ y, int ldy, const wg_epilogue e, int G, int B) {
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

  const uint4 *qg = quants + (int64_t)g * B * 4;
  const uint16_t *sg = scales + (int64_t)g * B * 4;
  for (int b = lane; b < B; b += 64) {
    const uint4 *qp = qg + (int64_t)b * 4;
    uint4 q[4] = {qp[0], qp[1], qp[2], qp[3]};
    // per row, d (b - z sa), or for Q4_K records d' b - c sa (z := c / d')
    float z[4], d[4], c[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (ZK == WG_ZERO_Q4K) {
      uint4 dd;
      uint2 bits;
      q4k_load(scales, g, B, b, dd, bits);
      q4k_dc(dd, bits, d, c);
      z[0] = z[1] = z[2] = z[3] = 0.0f;
    } else {
      uint2 sc = *reinterpret_cast<const uint2 *>(sg + (int64_t)b * 4);
      load_zeros<ZK>(zeros, ((int64_t)g * B + b) * 4, z);
      d[0] = (float)as_h2(sc.x).x;
      d[1] = (float)as_h2(sc.x).y;
      d[2] = (float)as_h2(sc.y).x;
      d[3] = (float)as_h2(sc.y).y;
    }
    uint4 a[M][4];
#pragma unroll
    for (int m = 0; m < M; m++) {
      const uint4 *xp = reinterpret_cast<const uint4 *>(x + (int64_t)m * ldx + b * 32);
      a[m][0] = xp[0];
      a[m][1] = xp[1];
      a[m][2] = xp[2];
      a[m][3] = xp[3];
    }
    float sa[M];
#pragma unroll
    for (int m = 0; m < M; m++) sa[m] = block_sum(a[m]) * 0x1p-24f;
#pragma unroll
    for (int r = 0; r < 4; r++) {
      Nibbles n;
      unpack(q[r], n);
#pragma unroll
      for (int m = 0; m < M; m++) {
        float v = block_dot(n, a[m]);
        if constexpr (ZK == WG_ZERO_Q4K) {
          acc[r][m] = __builtin_fmaf(d[r], v, acc[r][m]);
          acc[r][m] = __builtin_fmaf(-c[r], sa[m], acc[r][m]);
        } else {
          v = __builtin_fmaf(-z[r], sa[m], v);
          acc[r][m] = __builtin_fmaf(d[r], v, acc[r][m]);
        }
      }
    }
  }
  float scale[M], tot[M];
  input_scales<M>(e, scale);
#pragma unroll
  for (int m = 0; m < M; m++) tot[m] = wave_sum4(acc[0][m], acc[1][m], acc[2][m], acc[3][m]);
  finish<M, MODE>(e, g, G, tot, scale, y, ldy, pre, pos0);
}

// K split so a lane holds at most 2 blocks' activations, and further (while
// every part keeps 64 blocks) when the row groups alone would give fewer
// than gemv_min_waves waves.
template <int M, int ZK>
int launch_stream_k(const wg_q4_matrix *w, const uint16_t *x, int ldx, float *y, int ldy,
                    const wg_epilogue &ep, hipStream_t s) {
  int B = w->K / 32, G = w->N / 4;
  int ks = B <= 128 ? 1 : B <= 256 ? 2 : B <= 512 ? 4 : 0;
  if (!ks) return -1;
  while (ks < 4 && G * ks < tuning("gemv_min_waves") && B / (2 * ks) >= 64) ks *= 2;
  int nb = (B + ks - 1) / ks > 64 ? 2 : 1;
  if (ks == 1) return nb == 1 ? launch_stream<M, ZK, 1, 1>(w, x, ldx, y, ldy, ep, s)
                              : launch_stream<M, ZK, 2, 1>(w, x, ldx, y, ldy, ep, s);
  if (ks == 2) return nb == 1 ? launch_stream<M, ZK, 1, 2>(w, x, ldx, y, ldy, ep, s)
                              : launch_stream<M, ZK, 2, 2>(w, x, ldx, y, ldy, ep, s);
  return nb == 1 ? launch_stream<M, ZK, 1, 4>(w, x, ldx, y, ldy, ep, s)
                 : launch_stream<M, ZK, 2, 4>(w, x, ldx, y, ldy, ep, s);
}

template <int M>
int launch_stream_m(const wg_q4_matrix *w, const uint16_t *x, int ldx, float *y, int ldy,
                    const wg_epilogue &ep, hipStream_t s) {
  switch (w->zero) {
    case WG_ZERO_8: return launch_stream_k<M, WG_ZERO_8>(w, x, ldx, y, ldy, ep, s);
    case WG_ZERO_U8: return launch_stream_k<M, WG_ZERO_U8>(w, x, ldx, y, ldy, ep, s);
    case WG_ZERO_Q4K: return launch_stream_k<M, WG_ZERO_Q4K>(w, x, ldx, y, ldy, ep, s);
    default: return launch_stream_k<M, WG_ZERO_F16>(w, x, ldx, y, ldy, ep, s);
  }
}

template <int M, int ZK, int MODE>
void launch_rowgroup(const wg_q4_matrix *w, const uint16_t *x, int ldx, float *y, int ldy,
                     const wg_epilogue &e, hipStream_t s) {
  int G = w->N / 4, B = w->K / 32;
  gemv_rowgroup_kernel<M, ZK, MODE><<<(G + 3) / 4, 256, 0, s>>>(
      (const uint4 *)w->quants, (const uint16_t *)w->scales, w->zeros, x, ldx, y, ldy, e, G, B);
}

template <int M, int ZK>
void launch_rowgroup_mode(const wg_q4_matrix *w, const uint16_t *x, int ldx, float *y, int ldy,
                          const wg_epilogue &e, hipStream_t s) {
  if (e.mode == WG_EPI_SWIGLU) launch_rowgroup<M, ZK, WG_EPI_SWIGLU>(w, x, ldx, y, ldy, e, s);
  else if (e.mode == WG_EPI_ROPE_KV) launch_rowgroup<M, ZK, WG_EPI_ROPE_KV>(w, x, ldx, y, ldy, e, s);
  else launch_rowgroup<M, ZK, WG_EPI_STORE>(w, x, ldx, y, ldy, e, s);
}

template <int M>
int launch_gemv_m(const wg_q4_matrix *w, const uint16_t *x, int ldx, float *y, int ldy,
                  const wg_epilogue &e, hipStream_t s) {
  switch (w->zero) {
    case WG_ZERO_8: launch_rowgroup_mode<M, WG_ZERO_8>(w, x, ldx, y, ldy, e, s); break;
    case WG_ZERO_U8: launch_rowgroup_mode<M, WG_ZERO_U8>(w, x, ldx, y, ldy, e, s); break;
    case WG_ZERO_Q4K: launch_rowgroup_mode<M, WG_ZERO_Q4K>(w, x, ldx, y, ldy, e, s); break;
    default: launch_rowgroup_mode<M, WG_ZERO_F16>(w, x, ldx, y, ldy, e, s); break;
  }
  return launched("wg_q4_gemv");
}

__global__ void f32_to_f16_kernel(const float *x, uint16_t *out, int64_t n) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float v = fminf(fmaxf(x[i], -65504.0f), 65504.0f);
  out[i] = __builtin_bit_cast(uint16_t, (_Float16)v);
}

}  // namespace

// Checks an epilogue against the matrix and the row count.
int check_epilogue(const wg_q4_matrix *w, int M, const float *y, int ldy,
                          const wg_epilogue &e) {
  const int N = w->N, G = N / 4;
  WG_REQUIRE(e.mode == WG_EPI_STORE || e.mode == WG_EPI_SWIGLU || e.mode == WG_EPI_ROPE_KV ||
                 e.mode == WG_EPI_SHORT_CONV,
             "wg_q4_gemv: unknown epilogue mode %d", e.mode);
  if (e.norm_parts) {
    WG_REQUIRE(e.n_parts >= 1 && e.norm_count >= 1 && e.ld_parts_in >= e.n_parts &&
                   e.norm_mult != 0.0f,
               "wg_q4_gemv: input norm needs parts, their count and a prescale");
  }
  if (e.pick_parts) {
    WG_REQUIRE(e.mode == WG_EPI_STORE && !e.residual,
               "wg_q4_gemv: the pick's parts come from a plain store (no residual)");
    WG_REQUIRE(((uintptr_t)e.pick_parts & 15) == 0,
               "wg_q4_gemv: the pick's parts must be 16-byte aligned");
  }
  if (e.mode == WG_EPI_STORE) {
    WG_REQUIRE(y, "wg_q4_gemv: no output");
    WG_REQUIRE(ldy >= N, "wg_q4_gemv: ldy %d < N %d", ldy, N);
    if (e.residual) {
      WG_REQUIRE(e.ld_residual >= N, "wg_q4_gemv: residual stride %d < N %d", e.ld_residual, N);
      // An in-place add reads and writes the same element in one thread:
      // allowed. Any other overlap would race.
      WG_REQUIRE(e.residual == y || !overlaps(e.residual, (size_t)M * e.ld_residual * 4, y,
                                              (size_t)M * ldy * 4),
                 "wg_q4_gemv: residual overlaps the output");
    }
    if (e.out16)
      WG_REQUIRE(e.out16_w && e.ld_out16 >= N && e.norm_mult_out != 0.0f,
                 "wg_q4_gemv: the prescaled half output needs weights, a stride and a prescale");
    if (e.parts_out) WG_REQUIRE(e.ld_parts_out >= G, "wg_q4_gemv: parts stride too small");
  } else if (e.mode == WG_EPI_SWIGLU) {
    WG_REQUIRE(e.out16 && e.ld_out16 >= N / 2, "wg_q4_gemv: SwiGLU needs a half output of N/2");
  } else if (e.mode == WG_EPI_SHORT_CONV) {
    const int D = N / 3, W = e.conv_width;
    WG_REQUIRE(N % 48 == 0, "wg_q4_gemv: short-conv epilogue: %d rows are not B | C | x of a "
               "multiple of 16 channels", N);
    WG_REQUIRE(W >= 2 && W <= 4, "wg_q4_gemv: short-conv epilogue: width %d (2 to 4)", W);
    WG_REQUIRE(e.conv_taps && e.conv_state && e.conv_state_out && e.out16,
               "wg_q4_gemv: short-conv epilogue: null pointer");
    WG_REQUIRE(e.ld_out16 >= D, "wg_q4_gemv: short-conv epilogue: ld_out16 %d < %d channels",
               e.ld_out16, D);
    WG_REQUIRE(e.conv_state == e.conv_state_out ||
                   !overlaps(e.conv_state, (size_t)(W - 1) * D * 4, e.conv_state_out,
                             (size_t)(W - 1) * D * 4),
               "wg_q4_gemv: short-conv epilogue: state and new state partly overlap");
  } else {
    const int hd = e.head_dim;
    WG_REQUIRE(e.kv_heads > 0 && e.heads % e.kv_heads == 0 && hd >= 4 && hd % 4 == 0,
               "wg_q4_gemv: RoPE epilogue: %d heads over %d KV heads of %d", e.heads,
               e.kv_heads, hd);
    WG_REQUIRE(N == (e.heads + 2 * e.kv_heads) * hd,
               "wg_q4_gemv: RoPE epilogue: %d rows for %d q + 2 x %d kv heads of %d", N,
               e.heads, e.kv_heads, hd);
    WG_REQUIRE(e.rope && e.pos0 && e.q_out && e.k_cache && e.v_cache,
               "wg_q4_gemv: RoPE epilogue: null pointer");
    WG_REQUIRE(e.ld_q_out >= e.heads * hd, "wg_q4_gemv: q stride too small");
    WG_REQUIRE(e.ctx >= 1 && e.rope_rows >= 1024 + (e.ctx + 1023) / 1024,
               "wg_q4_gemv: a rope table of %d rows for a %d-position cache", e.rope_rows, e.ctx);
  }
  return WG_OK;
}
}  // namespace wg

using namespace wg;

extern "C" {

int wg_q4_gemv(const wg_q4_matrix *w, const uint16_t *x, int32_t M, int32_t ldx, float *y,
               int32_t ldy, const wg_epilogue *ep, void *stream) {
  int rc = check_matrix(w, "wg_q4_gemv");
  if (rc) return rc;
  WG_REQUIRE(M >= 1 && M <= 8, "wg_q4_gemv: %d rows; a few-token matmul takes 1 to 8", M);
  WG_REQUIRE(x, "wg_q4_gemv: null activations");
  WG_REQUIRE(ldx >= w->K && ldx % 8 == 0, "wg_q4_gemv: ldx %d (K %d) must be >= K and a multiple of 8",
             ldx, w->K);
  WG_REQUIRE(((uintptr_t)x & 15) == 0, "wg_q4_gemv: activations must be 16-byte aligned");
  wg_epilogue e = {};
  e.mode = WG_EPI_STORE;
  if (ep) e = *ep;
  if ((rc = check_epilogue(w, M, y, ldy, e))) return rc;
  if (y) WG_REQUIRE(!overlaps(x, (size_t)M * ldx * 2, y, (size_t)M * ldy * 4),
                    "wg_q4_gemv: activations and output overlap");
  if (e.out16)
    WG_REQUIRE(!overlaps(x, (size_t)M * ldx * 2, e.out16, (size_t)M * e.ld_out16 * 2),
               "wg_q4_gemv: activations and half output overlap");
  hipStream_t s = as_stream(stream);
  if (e.mode == WG_EPI_SHORT_CONV) {
    // the kernels that take it: the MFMA and the streaming GEMVs
    if (w->layout != WG_LAYOUT_ROWGROUP)
      return fail(WG_ERR_UNSUPPORTED, "wg_q4_gemv: short-conv epilogue: 4-bit row groups only");
    if ((rc = launch_gemv_mfma(w, x, M, ldx, y, ldy, e, s)) != -1) return rc;
    if (M <= 2 && w->K <= 512 * 32) {
      rc = M == 1 ? launch_stream_m<1>(w, x, ldx, y, ldy, e, s)
                  : launch_stream_m<2>(w, x, ldx, y, ldy, e, s);
      if (rc != -1) return rc;
    }
    if (M >= 3 && (rc = launch_gemv_few(w, x, M, ldx, y, ldy, e, s)) != -1) return rc;
    return fail(WG_ERR_UNSUPPORTED, "wg_q4_gemv: short-conv epilogue: not for this shape");
  }
  // (the pick's first stage: the MFMA and the streaming GEMVs)
  if (e.pick_parts && w->layout != WG_LAYOUT_ROWGROUP)
    return fail(WG_ERR_UNSUPPORTED, "wg_q4_gemv: the pick's parts: 4-bit row groups only");
  if (w->layout == WG_LAYOUT_Q4K) return launch_gemv_q4k(w, x, M, ldx, y, ldy, e, s);
  if (w->layout == WG_LAYOUT_Q8 || w->layout == WG_LAYOUT_Q6K)
    return launch_gemv_wide(w, x, M, ldx, y, ldy, e, s);
  if ((rc = launch_gemv_mfma(w, x, M, ldx, y, ldy, e, s)) != -1) return rc;
  if (M <= 2 && w->K <= 512 * 32) {
    rc = M == 1 ? launch_stream_m<1>(w, x, ldx, y, ldy, e, s)
                : launch_stream_m<2>(w, x, ldx, y, ldy, e, s);
    if (rc != -1) return rc;
  }
  if (M >= 3 && M <= 8) {
    rc = launch_gemv_few(w, x, M, ldx, y, ldy, e, s);
    if (rc != -1) return rc;
  }
  if (e.pick_parts)
    return fail(WG_ERR_UNSUPPORTED, "wg_q4_gemv: the pick's parts: not for this shape");
  switch (M) {
    case 1: return launch_gemv_m<1>(w, x, ldx, y, ldy, e, s);
    case 2: return launch_gemv_m<2>(w, x, ldx, y, ldy, e, s);
    case 3: return launch_gemv_m<3>(w, x, ldx, y, ldy, e, s);
    case 4: return launch_gemv_m<4>(w, x, ldx, y, ldy, e, s);
    case 5: return launch_gemv_m<5>(w, x, ldx, y, ldy, e, s);
    case 6: return launch_gemv_m<6>(w, x, ldx, y, ldy, e, s);
    case 7: return launch_gemv_m<7>(w, x, ldx, y, ldy, e, s);
    default: return launch_gemv_m<8>(w, x, ldx, y, ldy, e, s);
  }
}

int wg_f32_to_f16(const float *x, uint16_t *out, int64_t n, void *stream) {
  WG_REQUIRE(x && out && n >= 0, "wg_f32_to_f16: bad arguments");
  if (!n) return WG_OK;
  f32_to_f16_kernel<<<(unsigned)((n + 255) / 256), 256, 0, as_stream(stream)>>>(x, out, n);
  return launched("wg_f32_to_f16");
}

}  // extern "C"
