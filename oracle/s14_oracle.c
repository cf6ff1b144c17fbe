/*
 * CPU F32 oracle for the S14 quantized expert path — TEST INFRASTRUCTURE ONLY.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * this; the product never does.  Build with -O2 -ffp-contract=off and no
 * fast-math so every f32 operation rounds exactly as written (the Rust
 * reference never contracts to FMA).  File-level provenance is in
 * s14_oracle.h; each function cites the reference line it restates.
 */
#include "s14_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

int s14o_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

void s14o_set_num_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}

/* ------------------------------------------------------------------ */
/* decoders                                                            */
/* ------------------------------------------------------------------ */

/* s14_vulkan_numeric.rs:1716-1724: magnitude table, sign from bit 3. */
float s14o_e2m1(uint8_t code) {
  static const float mag[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
  float v = mag[code & 7];
  return (code & 8) == 0 ? v : -v;
}

/* s14_vulkan_numeric.rs:1726-1728: 2^(code-127); code 0 gives the f32
 * subnormal 2^-127 exactly, code 255 gives +inf (rejected upstream). */
float s14o_ue8m0(uint8_t code) { return ldexpf(1.0f, (int)code - 127); }

/* s14_vulkan_numeric.rs:1730-1743. */
float s14o_e4m3fn(uint8_t code) {
  int exponent = (code >> 3) & 0x0f;
  int mantissa = code & 7;
  float magnitude;
  if (exponent == 0) {
    magnitude = (float)mantissa * ldexpf(1.0f, -9);
  } else {
    magnitude = (1.0f + (float)mantissa / 8.0f) * ldexpf(1.0f, exponent - 7);
  }
  return (code & 0x80) == 0 ? magnitude : -magnitude;
}

float s14o_bf16_to_f32(uint16_t bits) {
  uint32_t u = (uint32_t)bits << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

uint16_t s14o_f32_to_bf16_rne(float v) {
  uint32_t u;
  memcpy(&u, &v, 4);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

/* OCP e4m3fn (bias 7, no infinities, NaN = 0x7f/0xff, max 448), RNE,
 * magnitudes above 448 saturate to 448. */
uint8_t s14o_f32_to_e4m3fn_rne_sat(float v) {
  if (isnan(v)) return 0x7f;
  uint8_t sign = signbit(v) ? 0x80 : 0x00;
  float a = fabsf(v);
  if (a >= 448.0f) return sign | 0x7e;
  if (a < 0x1p-6f) {
    /* subnormal grid m * 2^-9; m == 8 is the min normal, code 0x08 */
    float q = rintf(a * 512.0f);
    return sign | (uint8_t)q;
  }
  int e;
  float m = frexpf(a, &e); /* a = m * 2^e, m in [0.5, 1) */
  m *= 2.0f;
  e -= 1; /* a = m * 2^e, m in [1, 2) */
  float mant = rintf((m - 1.0f) * 8.0f);
  if (mant >= 8.0f) {
    mant = 0.0f;
    e += 1;
  }
  int biased = e + 7;
  if (biased > 15 || (biased == 15 && mant >= 7.0f)) return sign | 0x7e;
  return sign | (uint8_t)((biased << 3) | (int)mant);
}

void s14o_dequant_mxfp4(uint32_t n, uint32_t k, const uint8_t *packed,
                        const uint8_t *scale, float *out) {
  size_t pk = k / 2, groups = k / 32;
  for (size_t r = 0; r < n; ++r) {
    for (size_t kk = 0; kk < k; ++kk) {
      uint8_t byte = packed[r * pk + kk / 2];
      uint8_t code = (kk & 1) ? (byte >> 4) : (byte & 0x0f);
      out[r * k + kk] = s14o_e2m1(code) * s14o_ue8m0(scale[r * groups + kk / 32]);
    }
  }
}

void s14o_dequant_fp8_ue8m0(uint32_t n, uint32_t k, const uint8_t *w,
                            const uint8_t *scale, float *out) {
  size_t kg = (k + 127) / 128;
  for (size_t r = 0; r < n; ++r)
    for (size_t kk = 0; kk < k; ++kk)
      out[r * k + kk] = s14o_e4m3fn(w[r * k + kk]) * s14o_ue8m0(scale[(r / 128) * kg + kk / 128]);
}

/* ------------------------------------------------------------------ */
/* matvecs                                                             */
/* ------------------------------------------------------------------ */

/* cpu_mxfp4_matvec, s14_vulkan_numeric.rs:1669-1696: per row, groups outer,
 * 16 packed pairs inner; low nibble (even k) then high nibble (odd k);
 * sum += (x * e2m1) * scale, f32, no FMA. */
void s14o_mxfp4_matvec(uint32_t n, uint32_t k, const float *x,
                       const uint8_t *packed, const uint8_t *scale, float *y) {
  const size_t packed_k = k / 2;
  const size_t groups = k / 32;
  long long rows = (long long)n;
#pragma omp parallel for schedule(static)
  for (long long r = 0; r < rows; ++r) {
    float sum = 0.0f;
    for (size_t group = 0; group < groups; ++group) {
      float s = s14o_ue8m0(scale[(size_t)r * groups + group]);
      size_t pair_base = group * 16;
      for (size_t pig = 0; pig < 16; ++pig) {
        size_t pair = pair_base + pig;
        uint8_t codes = packed[(size_t)r * packed_k + pair];
        size_t k0 = pair * 2;
        sum += x[k0] * s14o_e2m1(codes & 0x0f) * s;
        sum += x[k0 + 1] * s14o_e2m1(codes >> 4) * s;
      }
    }
    y[r] = sum;
  }
}

/* cpu_fp8_matvec, s14_vulkan_numeric.rs:1698-1714: scale row n/128,
 * sum += (x * e4m3fn) * scale, k ascending. */
void s14o_fp8_matvec_ue8m0(uint32_t n, uint32_t k, const float *x,
                           const uint8_t *w, const uint8_t *scale, float *y) {
  const size_t k_groups = (k + 127) / 128;
  long long rows = (long long)n;
#pragma omp parallel for schedule(static)
  for (long long r = 0; r < rows; ++r) {
    size_t scale_row = ((size_t)r / 128) * k_groups;
    size_t weight_row = (size_t)r * k;
    float sum = 0.0f;
    for (size_t kk = 0; kk < k; ++kk) {
      float s = s14o_ue8m0(scale[scale_row + kk / 128]);
      sum += x[kk] * s14o_e4m3fn(w[weight_row + kk]) * s;
    }
    y[r] = sum;
  }
}

/* The same loop for the wq_a config: bf16 activations widened exactly to
 * f32 and one f32 scale per 128x128 tile. */
void s14o_fp8_matvec_f32scale_bf16x(uint32_t n, uint32_t k, const uint16_t *x_bf16,
                                    const uint8_t *w, const float *scale, float *y) {
  const size_t k_groups = (k + 127) / 128;
  long long rows = (long long)n;
#pragma omp parallel for schedule(static)
  for (long long r = 0; r < rows; ++r) {
    size_t scale_row = ((size_t)r / 128) * k_groups;
    size_t weight_row = (size_t)r * k;
    float sum = 0.0f;
    for (size_t kk = 0; kk < k; ++kk) {
      float s = scale[scale_row + kk / 128];
      float xv = s14o_bf16_to_f32(x_bf16[kk]);
      sum += xv * s14o_e4m3fn(w[weight_row + kk]) * s;
    }
    y[r] = sum;
  }
}

/* swiglu_limit, s14_vulkan_numeric.rs:1543-1556.  Rust f32::min returns the
 * non-NaN operand (fminf does too); clamp passes NaN through. */
void s14o_swiglu_limit(uint32_t n, const float *gate, const float *up, float *h) {
  for (size_t i = 0; i < n; ++i) {
    float g = fminf(gate[i], 10.0f);
    float u = up[i];
    if (u < -10.0f) u = -10.0f;
    if (u > 10.0f) u = 10.0f;
    h[i] = (g / (1.0f + expf(-g))) * u;
  }
}

/* ------------------------------------------------------------------ */
/* expert chain, layer                                                 */
/* ------------------------------------------------------------------ */

void s14o_mxfp4_expert_down(uint32_t hidden, uint32_t inter, const float *x,
                            const s14o_mxfp4_expert *e, float *down) {
  float *gate = (float *)malloc(sizeof(float) * inter * 3);
  float *up = gate + inter, *h = up + inter;
  s14o_mxfp4_matvec(inter, hidden, x, e->w1, e->s1, gate);
  s14o_mxfp4_matvec(inter, hidden, x, e->w3, e->s3, up);
  s14o_swiglu_limit(inter, gate, up, h);
  s14o_mxfp4_matvec(hidden, inter, h, e->w2, e->s2, down);
  free(gate);
}

void s14o_fp8_expert_down(uint32_t hidden, uint32_t inter, const float *x,
                          const s14o_fp8_expert *e, float *down) {
  float *gate = (float *)malloc(sizeof(float) * inter * 3);
  float *up = gate + inter, *h = up + inter;
  s14o_fp8_matvec_ue8m0(inter, hidden, x, e->w1, e->s1, gate);
  s14o_fp8_matvec_ue8m0(inter, hidden, x, e->w3, e->s3, up);
  s14o_swiglu_limit(inter, gate, up, h);
  s14o_fp8_matvec_ue8m0(hidden, inter, h, e->w2, e->s2, down);
  free(gate);
}

/* run_mxfp4_expert_chain's CPU half, s14_vulkan_numeric.rs:1294-1300. */
void s14o_expert_chain(uint32_t hidden, uint32_t inter, const float *x,
                       const s14o_mxfp4_expert *e, float route_w, float *y) {
  float *down = (float *)malloc(sizeof(float) * hidden);
  s14o_mxfp4_expert_down(hidden, inter, x, e, down);
  for (size_t i = 0; i < hidden; ++i) y[i] = route_w * down[i];
  free(down);
}

/* run_top6_shared_moe_batch's CPU half, s14_vulkan_numeric.rs:929-946. */
void s14o_moe_layer(uint32_t hidden, uint32_t inter, const float *x, uint32_t topk,
                    const s14o_mxfp4_expert *routed, const float *weights,
                    const s14o_mxfp4_expert *shared_mx, const s14o_fp8_expert *shared_fp8,
                    float *y) {
  float *down = (float *)malloc(sizeof(float) * hidden);
  for (size_t i = 0; i < hidden; ++i) y[i] = 0.0f;
  for (uint32_t e = 0; e < topk; ++e) {
    s14o_mxfp4_expert_down(hidden, inter, x, &routed[e], down);
    for (size_t i = 0; i < hidden; ++i) y[i] += weights[e] * down[i];
  }
  if (shared_fp8) {
    s14o_fp8_expert_down(hidden, inter, x, shared_fp8, down);
  } else {
    s14o_mxfp4_expert_down(hidden, inter, x, shared_mx, down);
  }
  for (size_t i = 0; i < hidden; ++i) y[i] += down[i];
  free(down);
}

/* ------------------------------------------------------------------ */
/* router                                                              */
/* ------------------------------------------------------------------ */

void s14o_router_logits(uint32_t n_experts, uint32_t k, const float *wr,
                        const float *x, float *z) {
  long long rows = (long long)n_experts;
#pragma omp parallel for schedule(static)
  for (long long e = 0; e < rows; ++e) {
    float p[64];
    const float *row = wr + (size_t)e * k;
    for (int l = 0; l < 64; ++l) {
      float acc = 0.0f;
      for (size_t c = 0; c < k / 256; ++c) {
        for (int j = 0; j < 4; ++j) {
          size_t kk = c * 256 + (size_t)l * 4 + (size_t)j;
          acc = fmaf(row[kk], x[kk], acc);
        }
      }
      p[l] = acc;
    }
    for (int m = 32; m >= 1; m >>= 1) {
      float q[64];
      for (int l = 0; l < 64; ++l) q[l] = p[l] + p[l ^ m];
      memcpy(p, q, sizeof(q));
    }
    z[e] = p[0];
  }
}

/* Score, biased top-k and weights.  BASELINE: sigmoid, weights renormalised
 * to 1.  Reference (executor.py:641-667): sqrt(softplus) with torch's
 * threshold-20 softplus, weights renormalised then scaled by 1.5. */
/* Scores of every expert and, in b, the biased scores (executor.py:641-645). */
static void router_scores(uint32_t n_experts, uint32_t k, const float *wr, const float *bias,
                          const float *x, int score_fn, float *scores_out, float *b) {
  float *z = (float *)malloc(sizeof(float) * n_experts);
  s14o_router_logits(n_experts, k, wr, x, z);
  for (uint32_t e = 0; e < n_experts; ++e) {
    float s;
    if (score_fn == S14O_SCORE_SIGMOID) {
      s = 1.0f / (1.0f + expf(-z[e]));
    } else {
      float sp = z[e] > 20.0f ? z[e] : log1pf(expf(z[e]));
      s = sqrtf(sp);
    }
    scores_out[e] = s;
    b[e] = s + bias[e];
  }
  free(z);
}

/* Weights of a chosen route: s[id] / sum with the sum sequential in route
 * order from 0, times route_scale if != 1 (executor.py:664-667). */
static void route_weights(const float *scores, const uint16_t *ids, uint32_t topk, float route_scale,
                          float *weights_out) {
  float sum = 0.0f;
  for (uint32_t i = 0; i < topk; ++i) sum += scores[ids[i]];
  for (uint32_t i = 0; i < topk; ++i) {
    float w = scores[ids[i]] / sum;
    if (route_scale != 1.0f) w = w * route_scale;
    weights_out[i] = w;
  }
}

int s14o_route_hash(uint32_t n_experts, uint32_t k, const float *wr, const float *bias, const float *x,
                    const int64_t *row, int score_fn, uint32_t topk, float route_scale, float *scores_out,
                    uint16_t *ids_out, float *weights_out) {
  float *b = (float *)malloc(sizeof(float) * n_experts);
  router_scores(n_experts, k, wr, bias, x, score_fn, scores_out, b);
  free(b);
  int bad = 0;
  for (uint32_t i = 0; i < topk; ++i) {
    if (row[i] < 0 || row[i] >= (int64_t)n_experts) bad = 1;
    for (uint32_t j = 0; j < i; ++j)
      if (row[j] == row[i]) bad = 1;
  }
  if (bad) return 1;
  for (uint32_t i = 0; i < topk; ++i) ids_out[i] = (uint16_t)row[i];
  route_weights(scores_out, ids_out, topk, route_scale, weights_out);
  return 0;
}

int s14o_route_valid(const uint16_t *ids, const float *w, uint32_t topk, uint32_t n_experts, float route_scale) {
  float sum = 0.0f;
  for (uint32_t i = 0; i < topk; ++i) {
    if (ids[i] >= n_experts) return 0;
    if (!isfinite(w[i]) || w[i] < 0.0f) return 0;
    for (uint32_t j = 0; j < i; ++j)
      if (ids[j] == ids[i]) return 0;
    sum += w[i];
  }
  return fabsf(sum - route_scale) <= 1e-4f;
}

void s14o_route(uint32_t n_experts, uint32_t k, const float *wr, const float *bias,
                const float *x, int score_fn, uint32_t topk, float route_scale,
                float *scores_out, uint16_t *ids_out, float *weights_out) {
  float *b = (float *)malloc(sizeof(float) * n_experts);
  router_scores(n_experts, k, wr, bias, x, score_fn, scores_out, b);
  unsigned char taken[1024];
  memset(taken, 0, sizeof(taken));
  for (uint32_t i = 0; i < topk; ++i) {
    int best = -1;
    for (uint32_t e = 0; e < n_experts; ++e) {
      if (taken[e]) continue;
      if (best < 0 || b[e] > b[best]) best = (int)e;
    }
    taken[best] = 1;
    ids_out[i] = (uint16_t)best;
  }
  route_weights(scores_out, ids_out, topk, route_scale, weights_out);
  free(b);
}

/* ------------------------------------------------------------------ */
/* error statistics                                                    */
/* ------------------------------------------------------------------ */

/* error_stats, s14_vulkan_numeric.rs:1745-1771. */
void s14o_error_stats_compute(size_t n, const float *actual, const float *expected,
                              s14o_error_stats *out) {
  float max_abs = 0.0f, max_rel = 0.0f;
  double sum_abs = 0.0, sum_sq = 0.0;
  out->finite = 1;
  for (size_t i = 0; i < n; ++i) {
    float a = actual[i], e = expected[i];
    if (!isfinite(a) || !isfinite(e)) {
      out->finite = 0;
      break;
    }
    float delta = fabsf(a - e);
    if (delta > max_abs) max_abs = delta;
    sum_abs += (double)delta;
    sum_sq += (double)delta * (double)delta;
    if (fabsf(e) > 1.0e-5f) {
      float rel = delta / fabsf(e);
      if (rel > max_rel) max_rel = rel;
    }
  }
  out->max_abs = max_abs;
  out->mean_abs = n ? sum_abs / (double)n : 0.0;
  out->rmse = n ? sqrt(sum_sq / (double)n) : 0.0;
  out->max_rel_abs_ref_gt_1e_5 = max_rel;
}

/* ------------------------------------------------------------------ */
/* activation requant                                                  */
/* ------------------------------------------------------------------ */

/* ceil(log2(r)) for finite r > 0, exactly: r = m * 2^e with m in [0.5,1). */
static int ceil_log2_exact(float r) {
  int e;
  float m = frexpf(r, &e);
  return m == 0.5f ? e - 1 : e;
}

void s14o_requant_e4m3(uint32_t rows, uint32_t k, uint32_t group, const float *x,
                       uint8_t *q, uint8_t *scale_codes) {
  size_t groups = k / group;
  for (size_t r = 0; r < rows; ++r) {
    for (size_t g = 0; g < groups; ++g) {
      const float *blk = x + r * k + g * group;
      float amax = 0.0f;
      for (size_t i = 0; i < group; ++i) {
        float a = fabsf(blk[i]);
        if (a > amax) amax = a;
      }
      if (amax < 1.0e-4f) amax = 1.0e-4f;
      int e = ceil_log2_exact(amax / 448.0f);
      scale_codes[r * groups + g] = (uint8_t)(e + 127);
      float inv = ldexpf(1.0f, -e);
      for (size_t i = 0; i < group; ++i) {
        float v = blk[i] * inv;
        if (v > 448.0f) v = 448.0f;
        if (v < -448.0f) v = -448.0f;
        q[r * k + g * group + i] = s14o_f32_to_e4m3fn_rne_sat(v);
      }
    }
  }
}

void s14o_dequant_requant(uint32_t rows, uint32_t k, uint32_t group, const uint8_t *q,
                          const uint8_t *scale_codes, float *out) {
  size_t groups = k / group;
  for (size_t r = 0; r < rows; ++r)
    for (size_t i = 0; i < k; ++i)
      out[r * k + i] = ldexpf(s14o_e4m3fn(q[r * k + i]), (int)scale_codes[r * groups + i / group] - 127);
}

void s14o_mxfp4_expert_down_requant(uint32_t hidden, uint32_t inter, uint32_t group,
                                    const float *x, const s14o_mxfp4_expert *e, float *down) {
  size_t big = hidden > inter ? hidden : inter;
  float *xd = (float *)malloc(sizeof(float) * (big + 3 * inter));
  float *gate = xd + big, *up = gate + inter, *h = up + inter;
  uint8_t *q = (uint8_t *)malloc(big + big / group);
  uint8_t *sc = q + big;
  s14o_requant_e4m3(1, hidden, group, x, q, sc);
  s14o_dequant_requant(1, hidden, group, q, sc, xd);
  s14o_mxfp4_matvec(inter, hidden, xd, e->w1, e->s1, gate);
  s14o_mxfp4_matvec(inter, hidden, xd, e->w3, e->s3, up);
  s14o_swiglu_limit(inter, gate, up, h);
  s14o_requant_e4m3(1, inter, group, h, q, sc);
  s14o_dequant_requant(1, inter, group, q, sc, xd);
  s14o_mxfp4_matvec(hidden, inter, xd, e->w2, e->s2, down);
  free(q);
  free(xd);
}

/* ------------------------------------------------------------------ */
/* official expert semantics                                           */
/* ------------------------------------------------------------------ */

/* act_quant of l42_reference.py:390-403 with group 128, dequantised: the
 * activation every official linear multiplies (exact f32 values). */
static void act_quant_128(uint32_t n, const float *x, float *xd) {
  uint8_t *q = (uint8_t *)malloc(n + n / 128);
  uint8_t *sc = q + n;
  s14o_requant_e4m3(1, n, 128, x, q, sc);
  s14o_dequant_requant(1, n, 128, q, sc, xd);
  free(q);
}

static float bf16_round(float v) { return s14o_bf16_to_f32(s14o_f32_to_bf16_rne(v)); }

void s14o_expert_official(uint32_t hidden, uint32_t inter, const float *x, const s14o_mxfp4_expert *mx,
                          const s14o_fp8_expert *f8, float weight, int apply_weight, float *out) {
  size_t big = hidden > inter ? hidden : inter;
  float *xd = (float *)malloc(sizeof(float) * (big + 3 * inter));
  float *g = xd + big, *u = g + inter, *h = u + inter;
  act_quant_128(hidden, x, xd);
  if (mx) {
    s14o_mxfp4_matvec(inter, hidden, xd, mx->w1, mx->s1, g);
    s14o_mxfp4_matvec(inter, hidden, xd, mx->w3, mx->s3, u);
  } else {
    s14o_fp8_matvec_ue8m0(inter, hidden, xd, f8->w1, f8->s1, g);
    s14o_fp8_matvec_ue8m0(inter, hidden, xd, f8->w3, f8->s3, u);
  }
  for (uint32_t i = 0; i < inter; ++i) {
    g[i] = bf16_round(g[i]);
    u[i] = bf16_round(u[i]);
  }
  s14o_swiglu_limit(inter, g, u, h);
  for (uint32_t i = 0; i < inter; ++i) h[i] = bf16_round(apply_weight ? h[i] * weight : h[i]);
  act_quant_128(inter, h, xd);
  if (mx)
    s14o_mxfp4_matvec(hidden, inter, xd, mx->w2, mx->s2, out);
  else
    s14o_fp8_matvec_ue8m0(hidden, inter, xd, f8->w2, f8->s2, out);
  for (uint32_t i = 0; i < hidden; ++i) out[i] = bf16_round(out[i]);
  free(xd);
}

void s14o_moe_layer_official(uint32_t hidden, uint32_t inter, const float *x, uint32_t topk,
                             const s14o_mxfp4_expert *routed, const float *weights,
                             const s14o_mxfp4_expert *shared_mx, const s14o_fp8_expert *shared_fp8, float *y,
                             float *y_f32) {
  float *acc = (float *)calloc(hidden, sizeof(float));
  float *out = (float *)malloc(sizeof(float) * hidden);
  for (uint32_t e = 0; e < topk; ++e) {
    s14o_expert_official(hidden, inter, x, &routed[e], NULL, weights[e], 1, out);
    for (uint32_t i = 0; i < hidden; ++i) acc[i] += out[i];
  }
  if (shared_mx || shared_fp8) {
    s14o_expert_official(hidden, inter, x, shared_mx, shared_fp8, 1.0f, 0, out);
    for (uint32_t i = 0; i < hidden; ++i) acc[i] += out[i];
  }
  for (uint32_t i = 0; i < hidden; ++i) {
    if (y_f32) y_f32[i] = acc[i];
    y[i] = bf16_round(acc[i]);
  }
  free(out);
  free(acc);
}

static float linear_scale(const void *s, size_t i, int is_f32) {
  return is_f32 ? ((const float *)s)[i] : s14o_ue8m0(((const uint8_t *)s)[i]);
}

void s14o_fp8_linear(uint32_t m, uint32_t n, uint32_t k, const uint8_t *x, const void *x_scale, int x_scale_f32,
                     const uint8_t *w, const void *w_scale, int w_scale_f32, const float *bias, int round_bf16,
                     float *y) {
  const uint32_t groups = (k + 127) / 128;
#pragma omp parallel for schedule(static)
  for (int64_t rr = 0; rr < (int64_t)n; ++rr) {
    const uint32_t r = (uint32_t)rr;
    for (uint32_t t = 0; t < m; ++t) {
      float acc = 0.0f;
      for (uint32_t g = 0; g < groups; ++g) {
        const float sa = linear_scale(x_scale, (size_t)t * groups + g, x_scale_f32);
        const float sb = linear_scale(w_scale, (size_t)(r / 128) * groups + g, w_scale_f32);
        const uint32_t k0 = 128 * g, k1 = k0 + 128 < k ? k0 + 128 : k;
        float partial = 0.0f;
        for (uint32_t kk = k0; kk < k1; ++kk) {
          const float a = s14o_e4m3fn(x[(size_t)t * k + kk]) * sa;
          const float b = s14o_e4m3fn(w[(size_t)r * k + kk]) * sb;
          partial += a * b;
        }
        acc += partial;
      }
      if (bias) acc += bias[r];
      y[(size_t)t * n + r] = round_bf16 ? bf16_round(acc) : acc;
    }
  }
}
