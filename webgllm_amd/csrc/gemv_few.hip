// The few-token GEMV (3 to 8 tokens: a speculative verify batch, the
// reference's split matmul at M <= 8, src/engine.ts:5316-5327) on the
// streaming kernel: persistent workgroups, each lane's activations of all
// M tokens held in registers for every row group, the next row group's
// weights loaded before the current one is computed. The K split keeps
// one block a lane (64 or fewer blocks a part), so the activations take
// 16 M registers; matrices of more than 256 blocks a row take the
// row-group kernel instead.
#include "gemv_stream.h"
#include "kernels.h"

namespace wg {
namespace {

template <int M, int ZK>
int launch_few_k(const wg_q4_matrix *w, const uint16_t *x, int ldx, float *y, int ldy,
                 const wg_epilogue &e, hipStream_t s) {
  const int B = w->K / 32, G = w->N / 4;
  int ks = B <= 64 ? 1 : B <= 128 ? 2 : B <= 256 ? 4 : 0;
  if (!ks) return -1;
  while (ks < 4 && G * ks < tuning("gemv_min_waves") && B / (2 * ks) >= 64) ks *= 2;
  if (ks == 1) return launch_stream<M, ZK, 1, 1>(w, x, ldx, y, ldy, e, s);
  if (ks == 2) return launch_stream<M, ZK, 1, 2>(w, x, ldx, y, ldy, e, s);
  return launch_stream<M, ZK, 1, 4>(w, x, ldx, y, ldy, e, s);
}

template <int M>
int launch_few_m(const wg_q4_matrix *w, const uint16_t *x, int ldx, float *y, int ldy,
                 const wg_epilogue &e, hipStream_t s) {
  switch (w->zero) {
    case WG_ZERO_8: return launch_few_k<M, WG_ZERO_8>(w, x, ldx, y, ldy, e, s);
    case WG_ZERO_U8: return launch_few_k<M, WG_ZERO_U8>(w, x, ldx, y, ldy, e, s);
    case WG_ZERO_Q4K: return launch_few_k<M, WG_ZERO_Q4K>(w, x, ldx, y, ldy, e, s);
    default: return launch_few_k<M, WG_ZERO_F16>(w, x, ldx, y, ldy, e, s);
  }
}

}  // namespace

int launch_gemv_few(const wg_q4_matrix *w, const uint16_t *x, int M, int ldx, float *y,
                    int ldy, const wg_epilogue &e, hipStream_t s) {
  if (!tuning("gemv_few_stream")) return -1;
  switch (M) {
    case 3: return launch_few_m<3>(w, x, ldx, y, ldy, e, s);
    case 4: return launch_few_m<4>(w, x, ldx, y, ldy, e, s);
    case 5: return launch_few_m<5>(w, x, ldx, y, ldy, e, s);
    case 6: return launch_few_m<6>(w, x, ldx, y, ldy, e, s);
    case 7: return launch_few_m<7>(w, x, ldx, y, ldy, e, s);
    case 8: return launch_few_m<8>(w, x, ldx, y, ldy, e, s);
    default: return -1;
  }
}

}  // namespace wg
