/*
 * CPU F32 oracle for the S14 quantized expert path — TEST INFRASTRUCTURE ONLY.
 *
 * This library is the checker the parity tests, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg compare the HIP path against.  Nothing in the
 * product (colormlm_amd/) links, loads or calls it.
 *
 * It restates the reference's CPU F32 oracle from
 *   scheduler/ssd_inference/examples/s14_vulkan_numeric.rs
 * with the identical operation order (strictly sequential k, mul-then-add,
 * no FMA contraction: build with -ffp-contract=off, never -ffast-math):
 *   e2m1            :1716-1724     ue8m0      :1726-1728     e4m3fn :1730-1743
 *   cpu_mxfp4_matvec:1669-1696     cpu_fp8_matvec :1698-1714
 *   swiglu_limit    :1543-1556     chain route mix :1300
 *   layer accumulate:929-946       error_stats    :1745-1771
 * Rows are independent (rayon into_par_iter in the reference, OpenMP here),
 * so results do not depend on the thread count.
 *
 * Functions the reference has no f32 loop for (router, token block, requant)
 * follow the semantics the north-star configs and executor.py:638-668 give;
 * where the reference leaves an order open (torch's BLAS order for the router
 * dot product) this file fixes one and says so at the function.
 *
 * Pinning (what checks each function; see tests/test_oracle_*.py):
 *   decoders      known-answer vectors of local_s14_primitives/tests/
 *                 test_primitives.py:37-94 and selftest.py:28-38; torch's
 *                 float8_e4m3fn decode for all 254 finite codes.
 *   matvecs       f64 brute force on small shapes; single-code closed forms;
 *                 an order-sensitive construction whose sequential-f32 value
 *                 is known in closed form; sign symmetry.
 *   swiglu/router libm identities; top-k against numpy argsort; tie rule.
 *   layer/block   composition identities against the pinned parts and f64.
 *   requant       RNE e4m3 encoder against torch's float8_e4m3fn cast.
 *   fp8_linear    the reference's own known-answer case (torch-seeded codes,
 *                 tolerance 2e-5 against decoded x @ decoded w.T); f64 brute
 *                 force; a group-order construction (per-group partials
 *                 differ from one flat sum) in closed form; power-of-two
 *                 scale identities.
 */
#ifndef S14_ORACLE_H
#define S14_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- decoders (s14_vulkan_numeric.rs:1716-1743) ---- */
float s14o_e2m1(uint8_t code);
float s14o_ue8m0(uint8_t code);
float s14o_e4m3fn(uint8_t code);
float s14o_bf16_to_f32(uint16_t bits);
/* OCP e4m3fn encoder, round-to-nearest-even, saturating to +-448. */
uint8_t s14o_f32_to_e4m3fn_rne_sat(float v);
uint16_t s14o_f32_to_bf16_rne(float v);

/* Dequantise one MXFP4 matrix [n, k] to f32 (w = e2m1 * ue8m0, exact). */
void s14o_dequant_mxfp4(uint32_t n, uint32_t k, const uint8_t *packed,
                        const uint8_t *scale, float *out);
/* Dequantise one FP8 matrix [n, k] with UE8M0 128x128 tile scales. */
void s14o_dequant_fp8_ue8m0(uint32_t n, uint32_t k, const uint8_t *w,
                            const uint8_t *scale, float *out);

/* ---- matvecs ---- */
/* cpu_mxfp4_matvec, s14_vulkan_numeric.rs:1669-1696. */
void s14o_mxfp4_matvec(uint32_t n, uint32_t k, const float *x,
                       const uint8_t *packed, const uint8_t *scale, float *y);
/* cpu_fp8_matvec, s14_vulkan_numeric.rs:1698-1714 (UE8M0 tile scales). */
void s14o_fp8_matvec_ue8m0(uint32_t n, uint32_t k, const float *x,
                           const uint8_t *w, const uint8_t *scale, float *y);
/* Same loop with f32 128x128 tile scales and bf16 activations (the wq_a
 * config): sum += (bf16(x[k]) * e4m3(w)) * scale_f32, k ascending. */
void s14o_fp8_matvec_f32scale_bf16x(uint32_t n, uint32_t k, const uint16_t *x_bf16,
                                    const uint8_t *w, const float *scale, float *y);

/* swiglu_limit, s14_vulkan_numeric.rs:1543-1556 (libm expf, as Rust's
 * f32::exp resolves to on Linux). */
void s14o_swiglu_limit(uint32_t n, const float *gate, const float *up, float *h);

/* ---- expert pages ---- */
/* MXFP4 page: [w1 | s1 | w3 | s3 | w2 | s2] for hidden=k_in, inter=n_mid. */
typedef struct {
  const uint8_t *w1, *s1, *w3, *s3, *w2, *s2;
} s14o_mxfp4_expert;
/* FP8 page (UE8M0 tile scales): the reference's shared expert. */
typedef struct {
  const uint8_t *w1, *s1, *w3, *s3, *w2, *s2;
} s14o_fp8_expert;

/* Expert without route weight: down = w2 . swiglu(w1.x, w3.x). */
void s14o_mxfp4_expert_down(uint32_t hidden, uint32_t inter, const float *x,
                            const s14o_mxfp4_expert *e, float *down);
void s14o_fp8_expert_down(uint32_t hidden, uint32_t inter, const float *x,
                          const s14o_fp8_expert *e, float *down);
/* Config-0 chain: y = route_w * down (s14_vulkan_numeric.rs:1294-1300). */
void s14o_expert_chain(uint32_t hidden, uint32_t inter, const float *x,
                       const s14o_mxfp4_expert *e, float route_w, float *y);

/* Top-k routed + shared layer with routing given
 * (s14_vulkan_numeric.rs:929-946): acc = 0; acc += w_i*down_i in route
 * order; acc += shared_down.  shared_fp8 selects the reference's FP8 shared
 * expert (shared_fp8 != NULL) instead of an MXFP4 one (shared_mx). */
void s14o_moe_layer(uint32_t hidden, uint32_t inter, const float *x, uint32_t topk,
                    const s14o_mxfp4_expert *routed, const float *weights,
                    const s14o_mxfp4_expert *shared_mx, const s14o_fp8_expert *shared_fp8,
                    float *y);

/* Official expert semantics (executor.py:712-744, l42_reference.py:390-419):
 * every linear multiplies the activation requantised by act_quant (e4m3, one
 * E8M0 scale 2^ceil(log2(max(amax,1e-4)/448)) per 128 values, dequantised:
 * exact f32) in the oracle's row order and rounds its output to bf16 (RNE).
 * Expert: g = bf16(W1 xq), u = bf16(W3 xq); h = bf16(swiglu(g, u) * weight)
 * for a routed expert (the route weight before w2, executor.py:720-722),
 * h = bf16(swiglu(g, u)) for the shared one (apply_weight = 0); out =
 * bf16(W2 hq).  mx or f8 selects the page format. */
void s14o_expert_official(uint32_t hidden, uint32_t inter, const float *x, const s14o_mxfp4_expert *mx,
                          const s14o_fp8_expert *f8, float weight, int apply_weight, float *out);
/* Official layer: acc = 0; acc += out_e (f32) for the routed experts in route
 * order, then the shared one; y = bf16(acc) (and y_f32 = acc if not NULL). */
void s14o_moe_layer_official(uint32_t hidden, uint32_t inter, const float *x, uint32_t topk,
                             const s14o_mxfp4_expert *routed, const float *weights,
                             const s14o_mxfp4_expert *shared_mx, const s14o_fp8_expert *shared_fp8, float *y,
                             float *y_f32);

/* ---- router ---- */
enum { S14O_SCORE_SIGMOID = 0, S14O_SCORE_SQRT_SOFTPLUS = 1 };
/* Router logits z[e] = W_r[e,:] . x.  The reference computes this with
 * torch F.linear (executor.py:641), whose summation order is the BLAS's and
 * unspecified; this oracle fixes it: 64 lane partials, lane l summing
 * k = 256c + 4l + j (c ascending, j = 0..3) sequentially, each term one
 * fused multiply-add acc = fmaf(w_k, x_k, acc) (one rounding per term, as a
 * BLAS dot kernel's FMA), then a xor butterfly of plain adds
 * p[l] = p[l] + p[l ^ m] for m = 32,16,8,4,2,1.  Requires k%256==0. */
void s14o_router_logits(uint32_t n_experts, uint32_t k, const float *wr,
                        const float *x, float *z);
/* scores, top-k of (score + bias) with ties to the lower index, weights =
 * s[id]/sum (sum sequential in selection order) times route_scale if != 1. */
/* Hash route (executor.py:643-667, the reference's layers 0-2): ids = the
 * token's tid2eid row, in row order; weights as for s14o_route.  Returns 0,
 * or 1 (outputs other than the scores untouched) when an entry is outside
 * [0, n_experts) or repeats an earlier one (the executor's ContractError). */
int s14o_route_hash(uint32_t n_experts, uint32_t k, const float *wr, const float *bias, const float *x,
                    const int64_t *row, int score_fn, uint32_t topk, float route_scale, float *scores_out,
                    uint16_t *ids_out, float *weights_out);
/* RouteDecision::validate_for's route checks (runner.rs:128-180): ids in
 * range and distinct, weights finite and >= 0, f32 sum (sequential) within
 * 1e-4 of route_scale (the reference's 1.5).  1 = valid. */
int s14o_route_valid(const uint16_t *ids, const float *w, uint32_t topk, uint32_t n_experts, float route_scale);
void s14o_route(uint32_t n_experts, uint32_t k, const float *wr, const float *bias,
                const float *x, int score_fn, uint32_t topk, float route_scale,
                float *scores_out, uint16_t *ids_out, float *weights_out);

/* ---- error statistics (s14_vulkan_numeric.rs:1745-1771) ---- */
typedef struct {
  float max_abs;
  double mean_abs;
  double rmse;
  float max_rel_abs_ref_gt_1e_5;
  int finite;
} s14o_error_stats;
void s14o_error_stats_compute(size_t n, const float *actual, const float *expected,
                              s14o_error_stats *out);

/* ---- activation requant (prefill): e4m3 with per-group E8M0 scales ----
 * scale = 2^ceil(log2(max(amax, 1e-4) / 448)) per group
 * (l42_reference.py:390-403), q = e4m3_rne_sat(x / scale). */
void s14o_requant_e4m3(uint32_t rows, uint32_t k, uint32_t group, const float *x,
                       uint8_t *q, uint8_t *scale_codes);

/* Dequantise requantised activations: x = e4m3(q) * 2^(code-127), exact. */
void s14o_dequant_requant(uint32_t rows, uint32_t k, uint32_t group, const uint8_t *q,
                          const uint8_t *scale_codes, float *out);

/* Prefill expert (config 4, BASELINE: FP8-requantised activations, per-32
 * E8M0 scales): xd = dequant(requant(x)); g = w1.xd, u = w3.xd in the oracle
 * order; h = swiglu(g, u); hd = dequant(requant(h)); down = w2.hd.  The
 * route weight and the accumulation are applied by the caller in the layer
 * order (s14_vulkan_numeric.rs:929-946).  This is the reference CPU order
 * applied to the quantised operands; the GPU's MFMA sums them in another
 * order, so parity for this config is a measured tolerance. */
void s14o_mxfp4_expert_down_requant(uint32_t hidden, uint32_t inter, uint32_t group,
                                    const float *x, const s14o_mxfp4_expert *e, float *down);

/* ---- activation-quantised FP8 linear (local_s14_primitives/fp8.py:111-193) ----
 * x e4m3 [m, k] with scales [m, G], weight e4m3 [n, k] with scales
 * [ceil(n/128), G], G = ceil(k/128); a scale is a UE8M0 code (f32 flag 0)
 * or an f32 (flag 1).  For each output: acc = 0; for each 128-k group g
 * ascending: partial = sum over the group's k of (e4m3(x) * sa) * (e4m3(w) *
 * sb), each product and sum rounded to f32; acc += partial (fp8.py:173-191,
 * one addmm per group); then acc += bias (if not NULL); y = acc, rounded to
 * bf16 if round_bf16.  The reference's addmm sums a group's products in its
 * BLAS's order; this oracle fixes k ascending. */
void s14o_fp8_linear(uint32_t m, uint32_t n, uint32_t k, const uint8_t *x, const void *x_scale, int x_scale_f32,
                     const uint8_t *w, const void *w_scale, int w_scale_f32, const float *bias, int round_bf16,
                     float *y);

int s14o_num_threads(void);
void s14o_set_num_threads(int n);

#ifdef __cplusplus
}
#endif
#endif
