// expf that returns, bit for bit, what glibc 2.35's expf returns.
//
// The reference oracle's SwiGLU (s14_vulkan_numeric.rs:1543-1556) calls Rust's
// f32::exp, which on Linux is the C library's expf.  glibc's expf is not
// correctly rounded (it differs from round-to-f32 of the exact value on about
// 1 in 25,000 inputs), so a device exp that is merely accurate would make the
// SwiGLU output, and everything downstream of it, drift from the oracle.
//
// Method (the published one used by glibc and ARM optimized-routines,
// "expf: table of 2^(i/32) plus a cubic in double precision"):
//   x*32/ln2 = k + r,  k integer (round-to-nearest via the 1.5*2^52 shift),
//   exp(x) = 2^(k/32) * p(r),  p(r) ~ 1 + C2 r + C1 r^2 + C0 r^3,
//   2^(k/32) assembled from the table entry for k mod 32 and the exponent k/32.
// The 32 table entries below were computed here from the mathematics
// (2^(i/32) rounded to the nearest double, by 60-digit decimal arithmetic);
// entry i is stored minus i<<47 so adding k<<47 yields 2^(k/32) directly.
// Which products are fused was settled by comparing against the system expf
// on every non-NaN f32 input: with r formed by one fused multiply-add and all
// other steps unfused, the two agree on all 4,278,190,080 of them.  The host
// build of this header is checked against the C library in the CPU tests.
//
// Usable from host and device code; every f64 step is written out so that
// neither compiler may contract or reassociate it (build with
// -ffp-contract=off).
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define S14_HD __host__ __device__ inline
#else
#define S14_HD static inline
#include <math.h>
#include <string.h>
#endif

namespace s14x {

struct ExpTable {
  uint64_t t[32];
};

S14_HD double exp_table_entry(uint32_t i) {
  // 2^(i/32) as a double, minus (i << 47), for i = 0..31.
  const uint64_t tab[32] = {
      0x3ff0000000000000ULL, 0x3fefd9b0d3158574ULL, 0x3fefb5586cf9890fULL,
      0x3fef9301d0125b51ULL, 0x3fef72b83c7d517bULL, 0x3fef54873168b9aaULL,
      0x3fef387a6e756238ULL, 0x3fef1e9df51fdee1ULL, 0x3fef06fe0a31b715ULL,
      0x3feef1a7373aa9cbULL, 0x3feedea64c123422ULL, 0x3feece086061892dULL,
      0x3feebfdad5362a27ULL, 0x3feeb42b569d4f82ULL, 0x3feeab07dd485429ULL,
      0x3feea47eb03a5585ULL, 0x3feea09e667f3bcdULL, 0x3fee9f75e8ec5f74ULL,
      0x3feea11473eb0187ULL, 0x3feea589994cce13ULL, 0x3feeace5422aa0dbULL,
      0x3feeb737b0cdc5e5ULL, 0x3feec49182a3f090ULL, 0x3feed503b23e255dULL,
      0x3feee89f995ad3adULL, 0x3feeff76f2fb5e47ULL, 0x3fef199bdd85529cULL,
      0x3fef3720dcef9069ULL, 0x3fef5818dcfba487ULL, 0x3fef7c97337b9b5fULL,
      0x3fefa4afa2a490daULL, 0x3fefd0765b6e4540ULL};
  uint64_t u = tab[i & 31];
  double d;
#if defined(__HIP_DEVICE_COMPILE__)
  d = __longlong_as_double((long long)u);
#else
  memcpy(&d, &u, 8);
#endif
  return d;
}

S14_HD uint32_t f32_bits(float f) {
#if defined(__HIP_DEVICE_COMPILE__)
  return (uint32_t)__float_as_uint(f);
#else
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
#endif
}

S14_HD uint64_t f64_bits(double d) {
#if defined(__HIP_DEVICE_COMPILE__)
  return (uint64_t)__double_as_longlong(d);
#else
  uint64_t u;
  memcpy(&u, &d, 8);
  return u;
#endif
}

S14_HD double f64_from_bits(uint64_t u) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __longlong_as_double((long long)u);
#else
  double d;
  memcpy(&d, &u, 8);
  return d;
#endif
}

// The method with the table lookup supplied by the caller: tab(i) must return
// exp_table_entry(i).  Device kernels that call it many times keep the 32
// entries in LDS; read from the constant table each call is a dependent
// global load.
template <class Tab>
S14_HD float expf_glibc_with(float x, const Tab &tab) {
  const double kInvLn2N = 0x1.71547652b82fep+0 * 32.0;  // 32/ln(2)
  const double kShift = 0x1.8p+52;
  // cubic coefficients of 2^(r/32), pre-divided by 32^3, 32^2, 32
  const double kC0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
  const double kC1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
  const double kC2 = 0x1.62e42ff0c52d6p-1 / 32.0;

  const uint32_t abstop = (f32_bits(x) >> 20) & 0x7ff;
  if (abstop >= (0x42b00000u >> 20)) {  // |x| >= 88 or x is NaN/inf
    if (f32_bits(x) == 0xff800000u) return 0.0f;  // -inf
    if (abstop >= (0x7f800000u >> 20)) return x + x;  // +inf, NaN
    if (x > 0x1.62e42ep6f) return __builtin_inff();   // overflow
    if (x < -0x1.9fe368p6f) return 0.0f;              // underflow
  }
  const double xd = (double)x;
  double z = kInvLn2N * xd;
  double kd = z + kShift;
  const uint64_t ki = f64_bits(kd);
  kd = kd - kShift;
  const double r = fma(kInvLn2N, xd, -kd);
  uint64_t t = f64_bits(tab((uint32_t)(ki % 32)));
  t += ki << 47;
  const double s = f64_from_bits(t);
  z = kC0 * r + kC1;
  const double r2 = r * r;
  double y = kC2 * r + 1.0;
  y = z * r2 + y;
  y = y * s;
  return (float)y;
}

struct ConstExpTable {
#if defined(__HIPCC__)
  __host__ __device__
#endif
  double operator()(uint32_t i) const { return exp_table_entry(i); }
};

S14_HD float expf_glibc(float x) { return expf_glibc_with(x, ConstExpTable{}); }

}  // namespace s14x
