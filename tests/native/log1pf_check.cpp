// Host build of the device log1pf (colormlm_amd/csrc/s14_log1pf.h) for the
// CPU test: counts inputs where it differs from the C library's log1pf.
#include <math.h>
#include <stdint.h>
#include <string.h>

#include "s14_log1pf.h"

extern "C" uint64_t log1pf_mismatches(uint64_t start, uint64_t stop, uint64_t step, uint32_t *first_bad) {
  uint64_t bad = 0;
  for (uint64_t u = start; u < stop; u += step) {
    uint32_t b = (uint32_t)u;
    float x;
    memcpy(&x, &b, 4);
    if (isnan(x)) continue;
    volatile float xv = x;
    float a = log1pf(xv), m = s14x::log1pf_glibc(xv);
    if (memcmp(&a, &m, 4) != 0) {
      if (bad == 0 && first_bad) *first_bad = b;
      ++bad;
    }
  }
  return bad;
}
