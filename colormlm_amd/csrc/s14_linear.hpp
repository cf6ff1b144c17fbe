// Activation-quantised FP8 linear (the adjacent FP8 projections wq_b, wkv,
// wo_a, wo_b) and the group-wise activation requant that feeds it: shared
// between s14_linear.hip and the host translation units.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "s14_linear_plan.h"

namespace s14 {

constexpr uint32_t kLinMaxK = 128u * 1024u;  // EXACT keeps a row's group partials in LDS

struct LinearArgs {
  uint32_t m, n, k, groups;  // tokens, output rows, input features, ceil(k / 128)
  const uint8_t *x;          // e4m3 codes [m][k]
  const void *x_scale;       // [m][groups]: UE8M0 codes or f32
  int x_scale_f32;
  const uint8_t *w;          // e4m3 codes [n][k]
  const void *w_scale;       // [ceil(n / 128)][groups]: UE8M0 codes or f32
  int w_scale_f32;
  const float *bias;         // [n] or NULL
  float *y;                  // [m][n]
  int round_bf16;            // y rounded to bf16 (the official linear's output)
};

// FAST's split-K state: partial tiles and arrival counters (zero between
// launches: the last wavefront of each tile resets its counter).
struct LinearWorkspace {
  float *part;
  uint32_t *count;
};

// EXACT: fp8.py:173-191's order with the group's products summed k
// ascending; FAST: bf16 MFMA on exactly decoded operands, not order-exact.
hipError_t launch_fp8_linear(hipStream_t s, const LinearArgs &a, int mode, const LinearWorkspace &ws);
// x f32 [rows][k] -> q e4m3 [rows][k] + E8M0 scales [rows][k / group]
// (l42_reference.py:390-403 for any group dividing k).
hipError_t launch_act_quant(hipStream_t s, uint32_t rows, uint32_t k, uint32_t group, const float *x, uint8_t *q,
                            uint8_t *scales);

}  // namespace s14
