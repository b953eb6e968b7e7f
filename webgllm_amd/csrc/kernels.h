// Launchers shared between the library's source files (not part of the C ABI).
#pragma once

#include "common.h"

namespace wg {

int launch_gemv_q4k(const wg_q4_matrix *w, const uint16_t *x, int M, int ldx, float *y, int ldy,
                    const wg_epilogue &e, hipStream_t s);

}  // namespace wg
