// Host build of the device expf (colormlm_amd/csrc/s14_expf.h) for the CPU
// test: counts inputs where it differs from the C library's expf.
#include <math.h>
#include <stdint.h>
#include <string.h>

#include "s14_expf.h"

extern "C" uint64_t expf_mismatches(uint64_t start, uint64_t stop, uint64_t step, uint32_t *first_bad) {
  uint64_t bad = 0;
  for (uint64_t u = start; u < stop; u += step) {
    uint32_t b = (uint32_t)u;
    float x;
    memcpy(&x, &b, 4);
    if (isnan(x)) continue;
    volatile float xv = x;
    float a = expf(xv), m = s14x::expf_glibc(xv);
    if (memcmp(&a, &m, 4) != 0) {
      if (bad == 0 && first_bad) *first_bad = b;
      ++bad;
    }
  }
  return bad;
}

extern "C" float expf_device_restated(float x) { return s14x::expf_glibc(x); }
