// Host build of the device e4m3 encoder (colormlm_amd/csrc/s14_e4m3.h) for
// the CPU test: counts inputs where it differs from the oracle's encoder
// (passed in as a function pointer).
#include <stdint.h>
#include <string.h>

#include "s14_e4m3.h"

typedef uint8_t (*enc_fn)(float);

extern "C" uint64_t e4m3_mismatches(uint64_t start, uint64_t stop, uint64_t step, void *oracle, uint32_t *first_bad) {
  const enc_fn ref = (enc_fn)oracle;
  uint64_t bad = 0;
  for (uint64_t u = start; u < stop; u += step) {
    uint32_t b = (uint32_t)u;
    float x;
    memcpy(&x, &b, 4);
    if (uint32_t(ref(x)) != s14x::e4m3_rne_sat(x)) {
      if (bad == 0 && first_bad) *first_bad = b;
      ++bad;
    }
  }
  return bad;
}
