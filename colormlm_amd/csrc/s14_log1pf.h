// log1pf that returns, bit for bit, what glibc 2.35's log1pf returns.
//
// The reference's score router (executor.py:642) is sqrt(softplus(z)) with
// torch's threshold 20: softplus(z) = log1p(exp(z)) below it.  The oracle
// evaluates it with the C library (expf, log1pf), so the device needs the
// same log1pf, not merely an accurate one: glibc 2.35's log1pf is not
// correctly rounded.
//
// Method: the published fdlibm/Sun log1p reduction (as in FreeBSD msun's
// s_log1pf.c, which glibc's flt-32 s_log1pf.c follows), restated here in
// single precision with every step explicit:
//   1 + x = 2^k (1 + f),  f in [sqrt(2)/2 - 1, sqrt(2) - 1),
//   with a correction c = (1 + x) - u for the rounding of u = 1 + x,
//   log1p(x) = k ln2_hi + (f - (hfsq - s (hfsq + R)) + (k ln2_lo + c)),
//   s = f / (2 + f),  hfsq = f^2 / 2,  R = z (Lp1 + z (Lp2 + ... + z Lp7)),
//   z = s^2 (the Remez polynomial of the fdlibm routine, its coefficients
//   the float roundings of that routine's published double coefficients).
// Every operation is a separately rounded f32 operation (no FMA; build with
// -ffp-contract=off), as the C code compiles on x86-64.  The host build of
// this header is compared with the C library in the CPU tests.
#pragma once

#include <stdint.h>

#include "s14_expf.h"  // f32_bits, S14_HD

namespace s14x {

S14_HD float f32_from_bits(uint32_t u) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __uint_as_float(u);
#else
  float f;
  memcpy(&f, &u, 4);
  return f;
#endif
}

// Correctly rounded f32 division on both sides (the device's `/` is too by
// default; this keeps it so whatever the build's division flags).
S14_HD float fdiv_rn(float a, float b) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __fdiv_rn(a, b);
#else
  return a / b;
#endif
}

S14_HD float log1pf_glibc(float x) {
  const float ln2_hi = f32_from_bits(0x3f317180u);  // 6.9313812256e-01
  const float ln2_lo = f32_from_bits(0x3717f7d1u);  // 9.0580006145e-06
  const float two25 = f32_from_bits(0x4c000000u);   // 2^25
  const float Lp1 = f32_from_bits(0x3f2aaaabu), Lp2 = f32_from_bits(0x3ecccccdu), Lp3 = f32_from_bits(0x3e924925u),
              Lp4 = f32_from_bits(0x3e638e29u), Lp5 = f32_from_bits(0x3e3a3325u), Lp6 = f32_from_bits(0x3e1cd04fu),
              Lp7 = f32_from_bits(0x3e178897u);
  const int32_t hx = (int32_t)f32_bits(x);
  const int32_t ax = hx & 0x7fffffff;
  float f = 0.0f, c = 0.0f;
  int32_t k = 1, hu = 0;
  if (hx < 0x3ed413d7) {        // x < 0.41422 (or negative)
    if (ax >= 0x3f800000) {     // x <= -1
      if (x == -1.0f) return fdiv_rn(-two25, 0.0f);  // -inf
      return fdiv_rn(x - x, x - x);                  // NaN
    }
    if (ax < 0x31000000) {  // |x| < 2^-29
      if (ax < 0x24800000) return x;  // |x| < 2^-54
      return x - x * x * 0.5f;
    }
    if (hx > 0 || hx <= (int32_t)0xbe95f61f) {  // -0.2929 < x < 0.41422
      k = 0;
      f = x;
      hu = 1;
    }
  }
  if (hx >= 0x7f800000) return x + x;  // +inf, NaN
  if (k != 0) {
    float u;
    if (hx < 0x5a000000) {
      u = 1.0f + x;
      hu = (int32_t)f32_bits(u);
      k = (hu >> 23) - 127;
      c = (k > 0) ? 1.0f - (u - x) : x - (u - 1.0f);  // correction term
      c = fdiv_rn(c, u);
    } else {
      u = x;
      hu = (int32_t)f32_bits(u);
      k = (hu >> 23) - 127;
      c = 0.0f;
    }
    hu &= 0x007fffff;
    if (hu < 0x3504f7) {
      u = f32_from_bits((uint32_t)hu | 0x3f800000u);  // normalise u
    } else {
      k += 1;
      u = f32_from_bits((uint32_t)hu | 0x3f000000u);  // normalise u / 2
      hu = (0x00800000 - hu) >> 2;
    }
    f = u - 1.0f;
  }
  const float hfsq = 0.5f * f * f;
  if (hu == 0) {  // |f| < 2^-20
    if (f == 0.0f) {
      if (k == 0) return 0.0f;
      c += (float)k * ln2_lo;
      return (float)k * ln2_hi + c;
    }
    const float R = hfsq * (1.0f - f32_from_bits(0x3f2aaaabu) * f);
    if (k == 0) return f - R;
    return (float)k * ln2_hi - ((R - ((float)k * ln2_lo + c)) - f);
  }
  const float s = fdiv_rn(f, 2.0f + f);
  const float z = s * s;
  const float R = z * (Lp1 + z * (Lp2 + z * (Lp3 + z * (Lp4 + z * (Lp5 + z * (Lp6 + z * Lp7))))));
  if (k == 0) return f - (hfsq - s * (hfsq + R));
  return (float)k * ln2_hi - ((hfsq - (s * (hfsq + R) + ((float)k * ln2_lo + c))) - f);
}

}  // namespace s14x
