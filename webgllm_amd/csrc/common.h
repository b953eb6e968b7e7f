// Shared helpers of the HIP backend: status handling, half bits, and the
// argument checks every entry point runs before it launches anything.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "status.h"

namespace wg {

// After a launch: WG_OK, or WG_ERR_DEVICE with HIP's message.
int launched(const char *what);

#define WG_HIP(expr)                                                                   \
  do {                                                                                 \
    hipError_t e_ = (expr);                                                            \
    if (e_ != hipSuccess)                                                              \
      return ::wg::fail(WG_ERR_DEVICE, "%s: %s", #expr, hipGetErrorString(e_));        \
  } while (0)


inline hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

// Checks a matrix descriptor's shape and arrays (shared by every op).
int check_matrix(const wg_q4_matrix *m, const char *who);

// Two byte ranges [a, a + na) and [b, b + nb) overlap.
inline bool overlaps(const void *a, size_t na, const void *b, size_t nb) {
  auto pa = reinterpret_cast<uintptr_t>(a), pb = reinterpret_cast<uintptr_t>(b);
  return pa < pb + nb && pb < pa + na;
}

// ----------------------------------------------------------- half bits

// IEEE half bits -> float, exactly (subnormals included), in integer math so
// the result never depends on the device's denormal mode.
__host__ __device__ inline float half_to_float(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu, mant = h & 0x3ffu;
  uint32_t bits;
  if (exp == 0) {
    if (mant == 0) {
      bits = sign;
    } else {  // subnormal: normalise
      int e = -1;
      do {
        e++;
        mant <<= 1;
      } while (!(mant & 0x400u));
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((mant & 0x3ffu) << 13);
    }
  } else if (exp == 31) {
    bits = sign | 0x7f800000u | (mant << 13);
  } else {
    bits = sign | ((exp + 112u) << 23) | (mant << 13);
  }
  return __builtin_bit_cast(float, bits);
}

// A double as half bits the way the reference's toHalf does it
// (src/half.ts:7-32): stored as a float32 first (round to nearest), then
// rounded to nearest even, with subnormals, overflow to infinity and NaN
// to a quiet NaN. Integer math, so it does not depend on device modes.
__host__ __device__ inline uint16_t double_to_half_ref(double value) {
  float f = (float)value;
  uint32_t x = __builtin_bit_cast(uint32_t, f);
  uint32_t sign = (x >> 16) & 0x8000u;
  int exp = (int)((x >> 23) & 0xffu);
  uint32_t mant = x & 0x7fffffu;
  if (exp == 0xff) return (uint16_t)(sign | 0x7c00u | (mant ? 0x200u : 0u));
  int e = exp - 127 + 15;
  if (e >= 31) return (uint16_t)(sign | 0x7c00u);
  if (e <= 0) {
    if (e < -10) return (uint16_t)sign;
    mant |= 0x800000u;
    int shift = 14 - e;
    uint32_t half = 1u << (shift - 1);
    uint32_t rest = mant & ((1u << shift) - 1u);
    uint32_t h = mant >> shift;
    if (rest > half || (rest == half && (h & 1u))) h++;
    return (uint16_t)(sign | h);
  }
  uint32_t h = ((uint32_t)e << 10) | (mant >> 13);
  uint32_t rest = mant & 0x1fffu;
  if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h++;
  return (uint16_t)(sign | h);
}

// get_scale_min_k4 for sub-block j (0..7) of a Q4_K super-block's 12 scale
// bytes (as src/repack.ts:127-140 decodes pairs of them).
__host__ __device__ inline void q4k_scale_min(const uint8_t *sc, int j, int *s, int *m) {
  if (j < 4) {
    *s = sc[j] & 63;
    *m = sc[j + 4] & 63;
  } else {
    *s = (sc[j + 4] & 15) | ((sc[j - 4] >> 6) << 4);
    *m = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4);
  }
}

}  // namespace wg
