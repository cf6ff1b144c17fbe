// Host build of the FAST fp8_linear launch plan (colormlm_amd/csrc/
// s14_linear_plan.h) for the CPU test of its sizing.
#include <stdint.h>

#include "s14_linear_plan.h"

extern "C" void lin_plan(uint32_t m, uint32_t n, uint32_t groups, uint32_t *cw, uint32_t *blocks) {
  const s14::LinFastPlan p = s14::lin_fast_plan(m, n, groups);
  *cw = p.cw;
  *blocks = p.blocks;
}

extern "C" uint32_t lin_chunks(uint32_t groups, uint32_t tiles, uint32_t blocks, uint32_t ntok) {
  return s14::lin_fast_chunks(groups, tiles, blocks, ntok);
}

extern "C" void lin_limits(uint64_t *part_bytes, uint32_t *counters, uint32_t *stage_bytes, uint32_t *tile) {
  *part_bytes = s14::kLinPartBytes;
  *counters = s14::kLinMaxCounters;
  *stage_bytes = s14::kLinStageBytes;
  *tile = s14::kLinTile;
}
