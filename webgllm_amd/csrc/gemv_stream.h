// The streaming GEMV kernel for 4-bit row-group matrices, shared by the
// decode launcher (1 or 2 tokens, gemv.hip) and the few-token one (3 to 8
// tokens, gemv_few.hip), each translation unit instantiating its own forms.
#pragma once

#include "common.h"
#include "dot.h"
#include "epilogue.h"
#include "gemv_core.h"

namespace wg {
namespace {

// ---------------------------------------------------------------------------
// Streaming variant (decode, and verify batches of up to 8 tokens): persistent
// workgroups of 4 waves. The K range is split into KS parts (a wave per
// part, KS waves per row group, reduced through LDS); lane l of a part
// takes its blocks l and l + 64 (NB of them), whose activations (paired as
// the nibbles unpack, see pair_acts) and block sums it loads once into
// registers: they are the same for every row group. Row groups are
// streamed through two register sets, the loop unrolled by 2, so the next
// row group's nibbles, scales and zero points are in flight while the
// current one is computed and are never copied. Loads past the matrix
// read an in-range row group or block (a clamped index): a row group past
// the end is not stored, a block past the part adds zero.
// The arguments the first loads need (the matrix, its shape, the
// activations) lead the list: the first 14 dwords of the arguments arrive
// in scalar registers with the wave, so the first loads wait for no
// argument fetch.
template <int M, int ZK, int NB, int KS, int MODE, bool LATE = false>
__global__ __launch_bounds__(256) void gemv_stream_kernel(
    const uint4 *__restrict__ quants, const uint16_t *__restrict__ scales,
    const void *__restrict__ zeros, const uint16_t *__restrict__ x, int G, int B, int ldx,
    float *__restrict__ y, int ldy, const wg_epilogue e) {
  constexpr int RGW = 4 / KS;  // row groups a workgroup takes at a time
  __shared__ float red[2][4][4 * M];
  __shared__ float nred[4 * M];
  __shared__ PickBest pick_lds[MODE == WG_EPI_STORE ? 4 : 1][16];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int part = wave % KS, slot = wave / KS;
  const int BP = (B + KS - 1) / KS;
  const int b0 = part * BP + lane;
  const int b_end = min(B, (part + 1) * BP);
  int bj[NB];
  bool live[NB];
#pragma unroll
  for (int j = 0; j < NB; j++) {
    live[j] = b0 + 64 * j < b_end;
    bj[j] = live[j] ? b0 + 64 * j : 0;
  }

  // The first row group's weights go out first: they need no input, and
  // everything after them (activations, sums, the norm's parts) overlaps
  // their flight.
  const int stride = gridDim.x * RGW;
  const int g_first = blockIdx.x * RGW + slot;
  Unit<ZK, NB> U0, U1;
  load_unit_at<ZK, NB>(U0, quants, scales, zeros, min(g_first, G - 1), B, bj);
  // and the first row group's epilogue operands (the waves that finish).
  // LATE (the rotation, where waves have later row groups to hide them
  // behind): the table rows hang on the position, a pointer chase, so they
  // go out after the activations and the norm's parts, whose waits would
  // otherwise take in that chase too. Where every wave has one row group,
  // nothing is left to hide them behind, and they go out first.
  const int pos0 = epi_pos0<MODE>(e);
  EpiPre pnext = {};
  if (!LATE && part == 0) epi_prefetch<M, MODE>(e, g_first, G, pos0, pnext);

  // This lane's activations, paired, and their block sums (times 2^-24), once.
  PairedActs a[M][NB];
  float sa[M][NB];
#pragma unroll
  for (int m = 0; m < M; m++)
#pragma unroll
    for (int j = 0; j < NB; j++) {
      uint4 raw[4];
      if (live[j]) {
        const uint4 *xp = reinterpret_cast<const uint4 *>(x + (int64_t)m * ldx + bj[j] * 32);
        raw[0] = xp[0];
        raw[1] = xp[1];
        raw[2] = xp[2];
        raw[3] = xp[3];
      } else {
        raw[0] = raw[1] = raw[2] = raw[3] = make_uint4(0u, 0u, 0u, 0u);
      }
      sa[m][j] = block_sum(raw) * 0x1p-24f;
      pair_acts(raw, a[m][j]);
    }
  float scale[M];
  input_scales_wg<M, 4>(e, scale, nred);
  if (LATE && part == 0) epi_prefetch<M, MODE>(e, g_first, G, pos0, pnext);

  // one row group: the 4 rows' sums for each token, reduced (into part 0's
  // lanes' tot)
  auto sums = [&](const Unit<ZK, NB> &u, int it, float (&tot)[M]) {
    float acc[4][M];
#pragma unroll
    for (int r = 0; r < 4; r++)
#pragma unroll
      for (int m = 0; m < M; m++) acc[r][m] = 0.0f;
    accumulate_unit_paired<M, ZK, NB>(u, a, sa, live, acc);
    const int row = wave_sum4_row();
#pragma unroll
    for (int m = 0; m < M; m++) tot[m] = wave_sum4(acc[0][m], acc[1][m], acc[2][m], acc[3][m]);
    if constexpr (KS > 1) {
      // Parts 1.. hand their sums to part 0 through LDS (double-buffered by
      // iteration parity, so one barrier a row group suffices).
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
  };

  if constexpr (MODE == WG_EPI_SHORT_CONV) {
    // The slot's steps walk triples of row groups, the B, C and x rows of
    // the same 4 channels (part k % 3 of triple t = blockIdx RGW + slot +
    // (k / 3) stride, a row group of each part holding 4 channels): the B
    // and C sums wait in registers for the x step, which convolves.
    const int T = G / 3, D = 4 * T;
    auto rg = [&](int k) {
      const int t = (int)blockIdx.x * RGW + slot + (k / 3) * stride;
      return t < T ? (k % 3) * T + t : G;
    };
    auto base = [&](int k) { return (int)blockIdx.x * RGW + (k / 3) * stride; };  // uniform
    const int r = (lane >> 4) & 3, m = lane & 15, mm = m < M ? m : 0;
    float bv = 0.0f, cv = 0.0f;
    EpiPre cp = {};
    auto conv_step = [&](const Unit<ZK, NB> &u, int k, int it) {
      float tot[M];
      sums(u, it, tot);
      if (part == 0) {
        const float v = pick<M>(tot, mm) * 0x1p24f * pick<M>(scale, mm);
        const int g = rg(k);
        const int c = 4 * (g - (k % 3) * T) + r;  // the lane's channel (g < G)
        const bool live = g < G && m < M;
        if (k % 3 == 0) {
          bv = v;
          conv_prefetch(e, c, D, live, cp);
        } else if (k % 3 == 1) {
          cv = v;
        } else {
          conv_finish(e, c, D, M, bv, cv, v, live, cp);
        }
      }
    };
    // U0 holds step 0's row group (g_first)
    for (int k = 0; base(k) < T; k += 2) {
      load_unit_at<ZK, NB>(U1, quants, scales, zeros, min(rg(k + 1), G - 1), B, bj);
      conv_step(U0, k, 0);
      if (base(k + 1) >= T) break;
      load_unit_at<ZK, NB>(U0, quants, scales, zeros, min(rg(k + 2), G - 1), B, bj);
      conv_step(U1, k + 1, 1);
    }
    return;
  }

  PickBest pbest{PICK_FLOOR, PICK_NONE};  // (pick_parts) this lane's token's best row
  auto step = [&](const Unit<ZK, NB> &u, int g, int it, const EpiPre &pe) {
    float tot[M];
    sums(u, it, tot);
    if (part == 0) {
      finish<M, MODE>(e, g, G, tot, scale, y, ldy, pe, pos0);
      if constexpr (MODE == WG_EPI_STORE)
        if (e.pick_parts) {  // the value finish stored (no residual)
          const int m = lane & 15, mm = m < M ? m : 0;
          const float v = pick<M>(tot, mm) * 0x1p24f * pick<M>(scale, mm);
          pick_take(pbest, v, 4 * g + ((lane >> 4) & 3), g < G && m < M);
        }
    }
  };

  // g0 is the same for every wave of the workgroup, so all of them run the
  // same iterations (the reductions' barriers); g >= G is an idle slot
  for (int g0 = blockIdx.x * RGW, g = g_first; g0 < G; g0 += 2 * stride, g += 2 * stride) {
    load_unit_at<ZK, NB>(U1, quants, scales, zeros, min(g + stride, G - 1), B, bj);
    EpiPre pe = pnext;
    if (part == 0) epi_prefetch<M, MODE>(e, g + stride, G, pos0, pnext);
    step(U0, g, 0, pe);
    if (g0 + stride >= G) break;
    load_unit_at<ZK, NB>(U0, quants, scales, zeros, min(g + 2 * stride, G - 1), B, bj);
    pe = pnext;
    if (part == 0) epi_prefetch<M, MODE>(e, g + 2 * stride, G, pos0, pnext);
    step(U1, g + stride, 1, pe);
  }
  if constexpr (MODE == WG_EPI_STORE)
    if (e.pick_parts) pick_flush<4>(e, pbest, M, pick_lds);
}

template <int M, int ZK, int NB, int KS>
int launch_stream(const wg_q4_matrix *w, const uint16_t *x, int ldx, float *y, int ldy,
                  const wg_epilogue &e, hipStream_t s) {
  int G = w->N / 4, B = w->K / 32;
  constexpr int RGW = 4 / KS;
  // 3 tokens and more: one workgroup a CU (each wave then takes more row
  // groups for the activations it holds). One or two tokens, by the row
  // groups (8B-shape matrices, µs a launch over 12 distinct ones at 1 / 2 /
  // 3 / 4 a CU): 1024 or fewer, one a CU (4096 x 4096: 4.56 / 4.86 / 4.80 /
  // 4.77; 4096 x 14336 10.66 / 10.62 / 11.27 / 11.56); from 4096, three
  // (28672 x 4096: 21.4 / 14.58 / 13.88 / 14.72); from 16384 (the head),
  // eight; two between (6144 x 4096: 5.95 / 5.40 / 5.68 / 5.65)
  const char *knob = M >= 3        ? "gemv_few_wg_per_cu"
                     : G >= 16384  ? "gemv_wg_per_cu_wide"
                     : G >= 4096   ? "gemv_wg_per_cu_deep"
                     : G <= 1024   ? "gemv_wg_per_cu_small"
                                   : "gemv_wg_per_cu";
  int grid = persistent_grid((G + RGW - 1) / RGW, tuning(knob));
  auto q = (const uint4 *)w->quants;
  auto sc = (const uint16_t *)w->scales;
  if (e.pick_parts && grid > WG_PICK_SLOTS)
    return fail(WG_ERR_UNSUPPORTED, "wg_q4_gemv: %d workgroups for the pick's parts", grid);
  if (e.mode == WG_EPI_SHORT_CONV) {
    // a slot takes triples of row groups: G / 3 of them
    grid = persistent_grid((G / 3 + RGW - 1) / RGW, tuning(knob));
    gemv_stream_kernel<M, ZK, NB, KS, WG_EPI_SHORT_CONV><<<grid, 256, 0, s>>>(
        q, sc, w->zeros, x, G, B, ldx, y, ldy, e);
  } else if (e.mode == WG_EPI_SWIGLU)
    gemv_stream_kernel<M, ZK, NB, KS, WG_EPI_SWIGLU><<<grid, 256, 0, s>>>(q, sc, w->zeros, x, G, B, ldx,
                                                                         y, ldy, e);
  else if (e.mode == WG_EPI_ROPE_KV && G > grid * RGW)
    gemv_stream_kernel<M, ZK, NB, KS, WG_EPI_ROPE_KV, true><<<grid, 256, 0, s>>>(
        q, sc, w->zeros, x, G, B, ldx, y, ldy, e);
  else if (e.mode == WG_EPI_ROPE_KV)
    gemv_stream_kernel<M, ZK, NB, KS, WG_EPI_ROPE_KV><<<grid, 256, 0, s>>>(q, sc, w->zeros, x, G, B,
                                                                          ldx, y, ldy, e);
  else
    gemv_stream_kernel<M, ZK, NB, KS, WG_EPI_STORE><<<grid, 256, 0, s>>>(q, sc, w->zeros, x, G, B, ldx,
                                                                        y, ldy, e);
  return launched("wg_q4_gemv");
}

}  // namespace
}  // namespace wg
