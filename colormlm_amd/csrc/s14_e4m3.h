// f32 -> OCP e4m3fn (bias 7, no infinities, NaN 0x7f, largest finite 448),
// round to nearest even, magnitudes past 448 saturating to 448 — the prefill's
// activation requant (l42_reference.py:390-403 with group 32).
//
// Straight-line: both the normal and the subnormal encodings are formed and
// the result selected, so a wavefront never splits on the value's range (the
// branchy form cost the prefill's SwiGLU epilogue several microseconds per
// wavefront in divergent control flow).  Usable from host and device code;
// the CPU tests compare the host build with the oracle's encoder.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define S14_E4M3_HD __host__ __device__ inline
#else
#define S14_E4M3_HD static inline
#include <math.h>
#include <string.h>
#endif

namespace s14x {

S14_E4M3_HD uint32_t e4m3_rne_sat(float v) {
  uint32_t u;
#if defined(__HIP_DEVICE_COMPILE__)
  u = __float_as_uint(v);
#else
  memcpy(&u, &v, 4);
#endif
  const uint32_t sign = (u >> 24) & 0x80u;
  const uint32_t au = u & 0x7fffffffu;
  const bool nan = au > 0x7f800000u;
  const bool sat = au >= 0x43e00000u;  // |v| >= 448 (inf included)
  const bool sub = au < 0x3c800000u;   // |v| < 2^-6: the 2^-9 grid
  // normal: round the f32 mantissa to 3 bits, ties to even; a carry out of
  // the mantissa bumps the exponent
  const uint32_t e = au >> 23;
  uint32_t mant = (au >> 20) & 7u;
  const uint32_t rem = au & 0xfffffu;
  mant += (rem > 0x80000u || (rem == 0x80000u && (mant & 1u))) ? 1u : 0u;
  const uint32_t be = e - 120u + (mant >> 3);  // e4m3 biased exponent (valid when !sub)
  mant &= 7u;
  const bool over = !sub && (be > 15u || (be == 15u && mant == 7u));
  const uint32_t normal = (be << 3) | mant;
  // subnormal: |v| * 512 rounded to an integer 0..8 (8 is the smallest
  // normal, code 0x08); the scaling by 2^9 is exact
  float a;
#if defined(__HIP_DEVICE_COMPILE__)
  a = __uint_as_float(au);
  const uint32_t subc = uint32_t(__builtin_rintf(a * 512.0f));
#else
  memcpy(&a, &au, 4);
  const uint32_t subc = (uint32_t)rintf(a * 512.0f);
#endif
  uint32_t code = sub ? subc : normal;
  code = (sat || over) ? 0x7eu : code;
  return nan ? 0x7fu : (sign | code);
}

}  // namespace s14x
