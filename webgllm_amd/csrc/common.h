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

// packQ4_K's per-block halves from a Q4_K scale and min (src/repack.ts:100-168):
// d' = toHalf(d sc); z' = toHalf(dmin m / d') with the quotient in doubles;
// where d' is 0 the block is constant: d' = toHalf(-dmin m / 15), z' = 0,
// and its quants are 15. Returns whether the block is constant.
__host__ __device__ inline bool q4k_block_dz(double d, double dmin, int sc, int mn, uint16_t *dq,
                                             uint16_t *zq) {
  const double mins = dmin * mn;
  const uint16_t h = double_to_half_ref(d * sc);
  const float hv = half_to_float(h);
  if (hv != 0.0f) {
    *dq = h;
    *zq = double_to_half_ref(mins / (double)hv);
    return false;
  }
  *dq = double_to_half_ref(-mins / 15.0);
  *zq = 0;
  return true;
}

// A WG_ZERO_Q4K record (64 bytes a row group and super-block): the rows'
// (half d, half dmin) in bytes 0-15, then block pair i's 96 bits at byte 16
// + 12 i (block 2i in bits 0-47, 2i + 1 in 48-95), a block's row r at bits
// 12 r (scale) and 12 r + 6 (min), 6 bits each.
constexpr int Q4K_REC = 64;
__host__ __device__ inline int q4k_rec_field(const uint8_t *rec, int j, int r, int which) {
  const int bit = 48 * (j & 1) + 12 * r + 6 * which;
  const uint8_t *p = rec + 16 + 12 * (j >> 1) + (bit >> 3);
  // (the second byte only where the field crosses into it: never past the record)
  const uint32_t v = (uint32_t)p[0] | ((bit & 7) > 2 ? (uint32_t)p[1] << 8 : 0u);
  return (int)((v >> (bit & 7)) & 63u);
}
__host__ __device__ inline void q4k_rec_put(uint8_t *rec, int j, int r, int sc, int mn) {
  for (int which = 0; which < 2; which++) {
    const int bit = 48 * (j & 1) + 12 * r + 6 * which;
    const uint32_t v = (uint32_t)(which ? mn : sc) & 63u;
    uint8_t *p = rec + 16 + 12 * (j >> 1) + (bit >> 3);
    const bool two = (bit & 7) > 2;
    const uint32_t word =
        ((uint32_t)p[0] | (two ? (uint32_t)p[1] << 8 : 0u)) & ~(63u << (bit & 7));
    const uint32_t out = word | (v << (bit & 7));
    p[0] = (uint8_t)out;
    if (two) p[1] = (uint8_t)(out >> 8);
  }
}
// packQ4_K's (d', z') of row r, block j (0..7) of a record.
__host__ __device__ inline bool q4k_rec_dz(const uint8_t *rec, int j, int r, uint16_t *dq,
                                           uint16_t *zq) {
  const uint16_t db = (uint16_t)(rec[4 * r] | (rec[4 * r + 1] << 8));
  const uint16_t mb = (uint16_t)(rec[4 * r + 2] | (rec[4 * r + 3] << 8));
  return q4k_block_dz(half_to_float(db), half_to_float(mb), q4k_rec_field(rec, j, r, 0),
                      q4k_rec_field(rec, j, r, 1), dq, zq);
}

}  // namespace wg
