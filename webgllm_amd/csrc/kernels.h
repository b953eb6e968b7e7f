// Launchers shared between the library's source files (not part of the C ABI).
#pragma once

#include "common.h"

namespace wg {

// The epilogue checks of wg_q4_gemv for M rows (0, or a status with the
// error message set).
int check_epilogue(const wg_q4_matrix *w, int M, const float *y, int ldy, const wg_epilogue &e);

int launch_gemv_q4k(const wg_q4_matrix *w, const uint16_t *x, int M, int ldx, float *y, int ldy,
                    const wg_epilogue &e, hipStream_t s);
// WG_LAYOUT_Q8 and WG_LAYOUT_Q6K matrices.
// 4-bit row-group GEMV of 3 to 8 tokens on the streaming kernel, or -1
// when the shape (more than 256 blocks a row) or the knob leaves it to the
// row-group kernel.
int launch_gemv_few(const wg_q4_matrix *w, const uint16_t *x, int M, int ldx, float *y,
                    int ldy, const wg_epilogue &e, hipStream_t s);
// 4-bit row-group GEMV of 1 to 8 tokens on MFMA, or -1 when the knob or
// the shape (more than 128 blocks a row) leaves it to the other kernels.
int launch_gemv_mfma(const wg_q4_matrix *w, const uint16_t *x, int M, int ldx, float *y,
                     int ldy, const wg_epilogue &e, hipStream_t s);
int launch_gemv_wide(const wg_q4_matrix *w, const uint16_t *x, int M, int ldx, float *y, int ldy,
                     const wg_epilogue &e, hipStream_t s);
// A WG_ZERO_Q4K matrix's packQ4_K (d', z') halves into scales and zeros
// (N * K / 32 halves each, the WG_ZERO_F16 arrays of the same quants).
int launch_q4k_expand(const wg_q4_matrix *w, uint16_t *scales, uint16_t *zeros, hipStream_t s);

}  // namespace wg
