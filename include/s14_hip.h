/*
 * s14_hip.h — C ABI of the MI355X (gfx950) S14 quantized expert path.
 *
 * Drop-in replacement for the Rust/Vulkan hot path of
 * scheduler/ssd_inference (reference files cited per entry point):
 *   src/s14_vulkan.rs   shape/byte contract, code validation, the
 *                       S14NumericPipelines bind_* / cmd_* dispatch API and the
 *                       S14VulkanMoePages route page batches
 *   src/vram_pool.rs    the fenced VRAM page pool (VramPool)
 *   shaders/s14_*.comp  the five kernels (re-designed, not translated)
 *   s14_runner/src/runner.rs RouteDecision::validate_for
 *
 * Conventions (mirroring the reference and its moe_scheduler.h precedent):
 *   - every function returns S14_OK (0) or a negative S14_ERR_* code; the
 *     calling thread's last message is available from s14_last_error();
 *   - device pointers are caller-owned; the library never frees them;
 *   - s14_bind_* validate shapes and capacities exactly like the reference's
 *     bind_* (s14_vulkan.rs:206-334) and fill a plain dispatch record;
 *     s14_cmd_* only enqueue the kernel on the given stream (the reference's
 *     cmd_* "record only the dispatch", s14_vulkan.rs:336-416);
 *   - stream arguments are hipStream_t values passed as void*; NULL is the
 *     device's null (default) stream, as everywhere in HIP; the context's own
 *     streams come from s14_ctx_compute_stream / s14_ctx_copy_stream;
 *   - no internal locking: a pool or page set is used by one thread at a time
 *     (the reference's &mut discipline); contexts may be used from several
 *     threads only with distinct streams and workspaces.
 */
#ifndef S14_HIP_H
#define S14_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define S14_ABI_VERSION 2

/* ---- status codes: one per anyhow::bail! category of the reference ---- */
enum {
  S14_OK = 0,
  S14_ERR_SHAPE = -1,      /* N/K zero, alignment, overflow (s14_vulkan.rs:44-114) */
  S14_ERR_CAPACITY = -2,   /* buffer smaller than required (s14_vulkan.rs:128-140) */
  S14_ERR_NAN_CODE = -3,   /* UE8M0 0xff / E4M3FN 0x7f,0xff (s14_vulkan.rs:143-156) */
  S14_ERR_STALE = -4,      /* stale generation / binding (vram_pool.rs:263-360) */
  S14_ERR_POOL_FULL = -5,  /* all slots Loading or pinned (vram_pool.rs:193-201) */
  S14_ERR_INVALID = -6,    /* invalid argument: weight, NULL, state, duplicate */
  S14_ERR_ROUTE = -7,      /* RouteDecision contract (runner.rs:128-180) */
  S14_ERR_HIP = -8,        /* HIP runtime failure */
  S14_ERR_NOT_READY = -9   /* transfer / compute fence not yet complete */
};

/* Thread-local message of the last failing call on this thread. */
const char *s14_last_error(void);
int s14_abi_version(void);

/* ======================================================================
 * Shape / byte contract — S14MatvecShape, s14_vulkan.rs:39-114
 * ====================================================================== */
typedef struct {
  uint32_t n;
  uint32_t k;
} s14_shape;

typedef struct {
  uint64_t input_bytes;   /* fp32 x: 4*K */
  uint64_t output_bytes;  /* fp32 y: 4*N */
  uint64_t weight_bytes;  /* MXFP4: N*K/2; FP8: N*K */
  uint64_t scale_bytes;   /* MXFP4: N*K/32; FP8: ceil(N/128)*ceil(K/128) */
} s14_shape_bytes;

/* S14MatvecShape::validate_mxfp4 (s14_vulkan.rs:52-66): N,K > 0, K % 128 == 0. */
int s14_shape_validate_mxfp4(s14_shape shape, s14_shape_bytes *out);
/* S14MatvecShape::validate_fp8 (s14_vulkan.rs:68-78). */
int s14_shape_validate_fp8(s14_shape shape, s14_shape_bytes *out);
/* validate_ue8m0_codes (s14_vulkan.rs:143-148): first 0xff → S14_ERR_NAN_CODE,
 * *bad_index set.  Host memory. */
int s14_validate_ue8m0_codes(const uint8_t *codes, size_t n, size_t *bad_index);
/* validate_e4m3fn_codes (s14_vulkan.rs:151-156): 0x7f/0xff rejected. */
int s14_validate_e4m3fn_codes(const uint8_t *codes, size_t n, size_t *bad_index);

/* ======================================================================
 * Context — replaces VulkanContext + S14NumericPipelines::new/destroy
 * (device.rs:26-76, s14_vulkan.rs:196-204, :418-424)
 * ====================================================================== */
typedef struct s14_ctx s14_ctx;

/* Creates a context on `device`: a compute stream, a copy stream and a
 * device workspace sized for the largest layer/block launch.  The fused
 * launches of one context share that workspace (pair table, h, route
 * counters that each launch leaves at zero): launches of one context must
 * not overlap on the device, so issue them on one stream (or order the
 * streams with events), and use one context per concurrent stream. */
int s14_ctx_create(int device, s14_ctx **out);
void s14_ctx_destroy(s14_ctx *ctx);
/* hipStream_t of the context's compute / copy stream, as void*. */
void *s14_ctx_compute_stream(s14_ctx *ctx);
void *s14_ctx_copy_stream(s14_ctx *ctx);
int s14_ctx_synchronize(s14_ctx *ctx);
/* Stage timing (the role of the reference's Vulkan timestamp queries,
 * s14_vulkan_numeric.rs:1088-1101): when enabled, each fused entry point
 * (chain, layer, block) attaches start/stop hipEvents to each of its kernel
 * launches, timing the kernels' own execution.  s14_ctx_stage_times waits
 * for the last such launch and returns up to 3 stage durations in ms:
 * {route (router scores and top-k plan, one launch), phase 1 (w1, w3,
 * SwiGLU), phase 2 (w2, mix)}; a stage the last launch did not run (chain
 * and given-route layers have no route) reads 0.  An EXACT block's phase 1
 * and phase 2 are those of the half of its pairs run on the caller's stream
 * (the other half runs beside it); its phase 2 includes the combine. */
int s14_ctx_enable_stage_timing(s14_ctx *ctx, int enable);
int s14_ctx_stage_times(s14_ctx *ctx, float *ms, uint32_t cap, uint32_t *n_stages);

/* A device buffer view: the GpuBuffer of the reference (buffer.rs:21-70)
 * reduced to what the kernels need.  `bytes` is the capacity checked by the
 * bind calls, like GpuBuffer::size(). */
typedef struct {
  void *ptr;
  uint64_t bytes;
} s14_buffer;

/* Reduction order.  S14_MODE_EXACT reproduces the reference CPU oracle's
 * order (one output row per lane, k ascending, multiply then add, no FMA),
 * so results are bit-identical to it.  S14_MODE_FAST splits K across a
 * wavefront and reduces with cross-lane adds: HBM-bound, not bit-identical.
 * S14_MODE_OFFICIAL (fused expert entry points only: expert chain, MoE
 * layer, routed layer/block, no-alloc block, and the prefill, whose dot
 * products are the MFMA's) computes the model's official
 * expert (executor.py:712-744, l42_reference.py:390-419): each linear's
 * activation requantised to e4m3 with one power-of-two scale per 128
 * values, each linear's output rounded to bf16, the route weight applied to
 * h before w2 (shared expert: none), expert outputs summed in f32 in route
 * order with the shared expert last, the layer output rounded to bf16; dot
 * products in the EXACT order, so results are bit-identical to the oracle's
 * official restatement.  The expert chain in this mode applies its weight
 * the same way, to h before w2. */
enum { S14_MODE_EXACT = 0, S14_MODE_FAST = 1, S14_MODE_OFFICIAL = 2 };

/* ---- dispatch records (bind → cmd) ---- */
typedef struct {
  s14_shape shape;
  const float *x;
  const uint8_t *weight;
  const uint8_t *scale;
  float *y;
  int mode;
} s14_mxfp4_dispatch;

enum { S14_X_F32 = 0, S14_X_BF16 = 1 };
enum { S14_SCALE_UE8M0 = 0, S14_SCALE_F32 = 1 };
typedef struct {
  s14_shape shape;
  const void *x;          /* f32[K] or bf16[K] per x_dtype */
  const uint8_t *weight;  /* e4m3fn [N,K] */
  const void *scale;      /* ue8m0 or f32, [ceil(N/128), ceil(K/128)] */
  float *y;
  int x_dtype;
  int scale_dtype;
  int mode;
} s14_fp8_dispatch;

typedef struct {
  uint32_t n;
  const float *gate;
  const float *up;
  float *y;
} s14_swiglu_dispatch;

typedef struct {
  uint32_t n;
  float weight;
  const float *expert;
  float *out; /* route_mix: routed (written); moe_accumulate: acc (+=) */
} s14_scale_dispatch;

/* bind_mxfp4, s14_vulkan.rs:206-235 (capacities rounded to 4-byte words as
 * storage_bytes, :124-126). */
int s14_bind_mxfp4(s14_shape shape, s14_buffer x, s14_buffer packed_weight,
                   s14_buffer weight_scale, s14_buffer y, int mode, s14_mxfp4_dispatch *out);
/* bind_fp8, s14_vulkan.rs:237-266; extended with bf16 x / f32 tile scales. */
int s14_bind_fp8(s14_shape shape, s14_buffer x, int x_dtype, s14_buffer weight,
                 s14_buffer weight_scale, int scale_dtype, s14_buffer y, int mode,
                 s14_fp8_dispatch *out);
/* bind_swiglu_limit, s14_vulkan.rs:268-289. */
int s14_bind_swiglu_limit(uint32_t n, s14_buffer gate, s14_buffer up, s14_buffer y,
                          s14_swiglu_dispatch *out);
/* bind_route_mix, s14_vulkan.rs:291-312 (weight finite and >= 0). */
int s14_bind_route_mix(uint32_t n, float route_weight, s14_buffer expert, s14_buffer routed,
                       s14_scale_dispatch *out);
/* bind_moe_accumulate, s14_vulkan.rs:314-334. */
int s14_bind_moe_accumulate(uint32_t n, float weight, s14_buffer expert,
                            s14_buffer accumulator, s14_scale_dispatch *out);

/* cmd_*, s14_vulkan.rs:338-416: enqueue one kernel on `stream`. */
int s14_cmd_mxfp4_matvec(s14_ctx *ctx, void *stream, const s14_mxfp4_dispatch *d);
int s14_cmd_fp8_matvec(s14_ctx *ctx, void *stream, const s14_fp8_dispatch *d);
int s14_cmd_swiglu_limit(s14_ctx *ctx, void *stream, const s14_swiglu_dispatch *d);
int s14_cmd_route_mix(s14_ctx *ctx, void *stream, const s14_scale_dispatch *d);
int s14_cmd_moe_accumulate(s14_ctx *ctx, void *stream, const s14_scale_dispatch *d);

/* Debug dequantisers (bit-exact decode check): out f32 [N,K]. */
int s14_dequant_mxfp4(s14_ctx *ctx, void *stream, s14_shape shape, const uint8_t *packed,
                      const uint8_t *scale, float *out);
int s14_dequant_fp8(s14_ctx *ctx, void *stream, s14_shape shape, const uint8_t *weight,
                    const void *scale, int scale_dtype, float *out);

/* ======================================================================
 * Expert pages and fused expert entry points
 * ====================================================================== */
/* In-page layout (the reference treats pages as opaque EXPERT_PAGE_BYTES,
 * s14_runner memory.rs:3; this fixes it):
 *   MXFP4 page: [w1 N*K/2 | s1 N*K/32 | w3 | s3 | w2 K*N/2 | s2 K*N/32]
 *               = 13,369,344 B at hidden 4096, inter 2048 (EXPERT_PAGE_BYTES)
 *   FP8 page:   [w1 N*K | s1 tiles | w3 | s3 | w2 | s2]
 *               = 25,167,360 B (S14_SHARED_EXPERT_PAGE_BYTES, s14_vulkan.rs:18)
 * Each matrix starts at the byte offset given by s14_page_layout. */
enum { S14_PAGE_MXFP4 = 0, S14_PAGE_FP8 = 1 };
typedef struct {
  uint64_t w1, s1, w3, s3, w2, s2; /* byte offsets */
  uint64_t total_bytes;
} s14_page_layout;
int s14_page_layout_get(int page_format, uint32_t hidden, uint32_t inter, s14_page_layout *out);

#define S14_EXPERT_PAGE_BYTES 13369344ULL
#define S14_SHARED_EXPERT_PAGE_BYTES 25167360ULL
#define S14_HIDDEN 4096u
#define S14_INTER 2048u
#define S14_N_ROUTED_EXPERTS 256u
#define S14_TOP_K 6u
#define S14_MAX_BLOCK_TOKENS 8u

/* Single routed expert chain (the 5-dispatch sequence of
 * s14_vulkan_numeric.rs:1404-1447): y = route_w * (w2 . swiglu(w1.x, w3.x)). */
int s14_expert_chain(s14_ctx *ctx, void *stream, const uint8_t *page, const float *x,
                     float route_w, float *y, int mode);

/* Top-k routed + shared layer with the route given (the 35-dispatch batch of
 * s14_vulkan_numeric.rs:895-1269): y = sum_i w_i*down_i (route order), then
 * + shared_down.  routed_pages: `topk` device page pointers (host array). */
int s14_moe_layer(s14_ctx *ctx, void *stream, uint32_t topk, const uint8_t *const *routed_pages,
                  const float *route_weights, const uint8_t *shared_page, int shared_format,
                  const float *x, float *y, int mode);

/* Router parameters for the routed entry points. */
enum { S14_SCORE_SIGMOID = 0, S14_SCORE_SQRT_SOFTPLUS = 1 };
typedef struct {
  const float *weight;   /* device f32 [n_experts, hidden] */
  const float *bias;     /* device f32 [n_experts] */
  uint32_t n_experts;    /* 256 */
  uint32_t topk;         /* 6 */
  int score_fn;          /* S14_SCORE_* */
  float route_scale;     /* 1.0 (BASELINE) or 1.5 (reference route_scale) */
  /* Hash routing, the reference's layers 0-2 (executor.py:643-656,
   * contract.rs:81-90): when tid2eid is not NULL, token t's experts are the
   * row tid2eid[token_ids[t]] (device int64 [vocab][topk]) in row order
   * instead of the biased top-k; the weights are still the chosen experts'
   * scores renormalised (times route_scale).  A token id outside [0, vocab),
   * an entry outside [0, n_experts) or a repeated entry fails that token's
   * route (see s14_launch_status).  NULL tid2eid: score routing. */
  const int64_t *tid2eid;
  uint32_t vocab;
  const int32_t *token_ids; /* device int32 [tokens] of the launch */
} s14_router;

/* Router + routed + shared for one token.  expert_pages: device array of
 * n_experts page pointers (uint64).  ids_out/weights_out: device outputs
 * (topk each), may be NULL. */
int s14_moe_layer_route(s14_ctx *ctx, void *stream, const s14_router *router,
                        const uint64_t *expert_pages_dev, const uint8_t *shared_page,
                        int shared_format, const float *x, float *y, uint16_t *ids_out,
                        float *weights_out, int mode);

/* Speculative-verify block: T <= 8 tokens X[T, hidden] through the routed
 * layer, grouped expert-major so each distinct expert page is read once per
 * block.  ids_out [T, topk] u16 and weights_out [T, topk] f32 (device, may be
 * NULL); s14_last_block_distinct reports the distinct routed page count.
 * An EXACT block of T >= 2 runs half of its pairs on the context's own side
 * stream, joined back into `stream` (event wait) before the output is
 * written: work queued on `stream` afterwards sees y complete, and a graph
 * capture of `stream` takes the side branch in. */
int s14_moe_block_route(s14_ctx *ctx, void *stream, uint32_t tokens, const s14_router *router,
                        const uint64_t *expert_pages_dev, const uint8_t *shared_page,
                        int shared_format, const float *x, float *y, uint16_t *ids_out,
                        float *weights_out, int mode);
/* Distinct routed pages read by the last routed launch on this context
 * (synchronises the device). */
int s14_last_block_distinct(s14_ctx *ctx, uint32_t *n_distinct);

/* No counterpart in the reference: the routed layer/block of
 * s14_moe_block_route (same arguments without a context, same kernels,
 * bit-identical results) for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  It calls no hipMalloc/hipFree: its workspace is a static
 * device array of s14_noalloc_scratch_bytes() bytes (about 1.6 MB) per GPU,
 * held until the process ends, whose device address the first call on each
 * GPU looks up (hipGetSymbolAddress) with that GPU current.  The limit is
 * the block size: tokens > S14_MAX_BLOCK_TOKENS is S14_ERR_SHAPE.  Launches
 * go to `stream` on the current device.  Every call on a GPU shares that
 * GPU's array, so calls that overlap on one GPU (other streams or threads)
 * race on it. */
int s14_moe_block_route_noalloc(void *stream, uint32_t tokens, const s14_router *router,
                                const uint64_t *expert_pages_dev, const uint8_t *shared_page,
                                int shared_format, const float *x, float *y, uint16_t *ids_out,
                                float *weights_out, int mode);
uint64_t s14_noalloc_scratch_bytes(void);

/* Device-side status of the routed launches on this context since the last
 * call (synchronises the device, then clears it).  The routed entry points
 * read each chosen expert's page address from expert_pages_dev on the
 * device; every entry of that table must be the address of a resident,
 * pinned page of the layer (lease it through s14_moe_pages_* and release it
 * only after the launch's compute fence).  A launch that finds a 0 entry
 * reads no memory through it, writes NaN for the affected outputs and leaves
 * a status that this call reports as S14_ERR_INVALID.  Every routed
 * launch also runs RouteDecision::validate_for's checks (runner.rs:128-180)
 * on each token's device-chosen route: expert ids inside [0, n_experts) and
 * distinct, weights finite and >= 0, their f32 sum within 1e-4 of
 * route_scale.  A token whose route fails them gets NaN outputs and this
 * call reports S14_ERR_ROUTE. */
int s14_launch_status(s14_ctx *ctx);

/* Router only (scores f32 [n_experts], ids u16 [topk], weights f32 [topk]). */
int s14_route(s14_ctx *ctx, void *stream, const s14_router *router, uint32_t tokens,
              const float *x, float *scores_out, uint16_t *ids_out, float *weights_out);

/* Prefill (config 4; the reference has no GPU code for it, its layer
 * semantics are s14_vulkan_numeric.rs:929-946): tokens <= 1024 through the
 * router and the top-6 routed + shared MXFP4 experts as grouped GEMMs on
 * the bf16 MFMA, both operands decoded exactly to bf16 by the gfx950 scaled
 * converters (products exact, f32 sums), activations requantised to e4m3 with per-32 E8M0
 * scales 2^ceil(log2(max(amax,1e-4)/448)) (l42_reference.py:390-403 with
 * group 32) before w1/w3 and again (h) before w2.  Not order-exact: results
 * agree with the CPU oracle to a measured tolerance.  The shared page must
 * be MXFP4.  ids_out [T, 6] u16 and weights_out [T, 6] f32 may be NULL.
 * mode: S14_MODE_EXACT or S14_MODE_FAST run the semantics above (one
 * numeric path, the MFMA's); S14_MODE_OFFICIAL the model's official expert
 * (executor.py:712-744): act_quant group 128 before every linear, g, u and
 * each expert output rounded to bf16, the route weight applied to h before
 * w2, y = bf16(f32 sum of the outputs in route order, shared last).
 * The first call on a context allocates its prefill workspace. */
int s14_moe_prefill(s14_ctx *ctx, void *stream, uint32_t tokens, const s14_router *router,
                    const uint64_t *expert_pages_dev, const uint8_t *shared_page, const float *x,
                    float *y, uint16_t *ids_out, float *weights_out, int mode);
/* Distinct routed experts, the largest tokens-per-expert and the number of
 * GEMM work items of the last prefill (synchronises the device). */
int s14_last_prefill_stats(s14_ctx *ctx, uint32_t *distinct, uint32_t *max_tokens,
                           uint32_t *n_items);
#define S14_MAX_PREFILL_TOKENS 1024u
/* Read-only device view of the last prefill's intermediates on this context
 * (valid until the next prefill on it), for stage-by-stage verification.
 * No counterpart in the reference, whose GPU code has no prefill.
 *   xq [tokens][4096] e4m3 and xs [tokens][128] E8M0: the requantised
 *     activations;
 *   ht, hts: the SwiGLU output of each (token, expert) pair, requantised
 *     the same way, in work-item tiles: item i's tile is 65536 bytes at
 *     ht + 65536 i, byte (s, part, lane, b) at 2048 s + 1024 part +
 *     16 lane + b holding the code of h value 64 s + 32 (lane / 32) +
 *     16 part + b of the pair first_i + (lane % 32); its scales are 2048
 *     bytes at hts + 2048 i, u32 [s / 4][lane] with byte s % 4 = the E8M0
 *     of h values 64 s + 32 (lane / 32) .. +31;
 *   down [n_pairs][4096] f32: each pair's w2 output, route weight not applied;
 *   pair_token [n_pairs]: the token of each pair; token_pair [tokens][7]:
 *     each token's pairs in route order, the shared expert's last;
 *   items [n_items][3]: {expert, first pair, pairs} of each GEMM work item.
 * Pairs are grouped by routed expert ascending, the shared expert's last. */
typedef struct s14_prefill_view {
  const uint8_t *xq, *xs, *ht, *hts;
  const float *down;
  const uint32_t *pair_token, *token_pair, *items;
  uint32_t tokens, n_pairs, n_items;
} s14_prefill_view;
int s14_last_prefill_view(s14_ctx *ctx, s14_prefill_view *out);
/* The prefill's activation requant as a standalone dispatch (natural
 * layout): x f32 [rows, k] -> q e4m3 [rows, k] and scales E8M0
 * [rows, k/32], bit-identical to the CPU oracle's requant. */
int s14_requant_e4m3(s14_ctx *ctx, void *stream, uint32_t rows, uint32_t k, const float *x,
                     uint8_t *q, uint8_t *scales);

/* ======================================================================
 * Adjacent FP8 projections: activation-quantised FP8 linear
 * ====================================================================== */

/* The official activation quant (l42_reference.py:390-403,
 * _activation_quant): x f32 [rows, k] -> q e4m3 [rows, k] (RNE,
 * saturating at 448) and E8M0 scale codes [rows, k / group], one scale
 * 2^ceil(log2(max(amax, 1e-4) / 448)) per group of `group` consecutive
 * values; group is 32, 64 or 128 and divides k (the reference raises
 * otherwise).  Group 128 feeds s14_fp8_linear; s14_requant_e4m3 is group
 * 32.  Bit-identical to the CPU oracle's requant. */
int s14_act_quant_e4m3(s14_ctx *ctx, void *stream, uint32_t rows, uint32_t k, uint32_t group,
                       const float *x, uint8_t *q, uint8_t *scales);

/* Round each output to bf16 (as an f32 value): the official linear's
 * output rounding (l42_reference.py:405-411, _linear_fp8). */
enum { S14_LINEAR_ROUND_BF16 = 1 };

/* fp8_linear (local_s14_primitives/fp8.py:111-193): y [m, n] f32 from
 *   x            e4m3 codes [m, k]
 *   x_scale      [m, ceil(k/128)]  UE8M0 codes or f32 (x_scale_dtype)
 *   weight       e4m3 codes [n, k]
 *   weight_scale [ceil(n/128), ceil(k/128)]  UE8M0 codes or f32, one per
 *                128 x 128 weight tile
 *   bias         f32 [n], or ptr NULL for none
 * y[t][r] = sum over 128-k groups g, ascending, of
 *   partial_g = sum_k (dec(x) * x_scale[t][g]) * (dec(w) * w_scale[r/128][g])
 * (acc = 0; acc += partial_g; then acc += bias[r]), f32 throughout.  A
 * ragged last group (k % 128 != 0) holds the remaining k.
 *
 * S14_MODE_EXACT sums each group's products k ascending (multiply, then
 * add; the reference's addmm leaves that order to the BLAS): bit-identical
 * to the CPU oracle's s14o_fp8_linear.  S14_MODE_FAST computes the group
 * dot products in another order (within the reference's own 2e-5 relative
 * tolerance of it): for one or two tokens (up to four where n <= 1024) and
 * k % 1024 == 0 as a VALU GEMV, otherwise on the MFMA; it needs k % 512 == 0
 * and otherwise runs the EXACT kernel.  Both modes keep partial sums in a
 * 32 MiB context workspace
 * (FAST: split-K partials and arrival counters; EXACT: per-group partials)
 * allocated on the first call: fp8_linear calls on one context must not
 * overlap (serialise them on one stream).
 *
 * Errors (fp8.py:141-171): S14_ERR_SHAPE for m, n or k zero, k > 131072,
 * or sizes past 32-bit addressing; S14_ERR_CAPACITY for a buffer smaller
 * than its shape; S14_ERR_INVALID for NULL buffers, an unknown scale dtype,
 * flag or mode.  E4M3FN NaN codes (0x7f, 0xff) are the caller's to reject
 * first (s14_validate_e4m3fn_codes; fp8.py:73-75 raises on them), as are
 * non-finite f32 scales (fp8.py:43-44). */
int s14_fp8_linear(s14_ctx *ctx, void *stream, uint32_t m, uint32_t n, uint32_t k, s14_buffer x,
                   s14_buffer x_scale, int x_scale_dtype, s14_buffer weight, s14_buffer weight_scale,
                   int weight_scale_dtype, s14_buffer bias, s14_buffer y, int flags, int mode);

/* ======================================================================
 * Synthetic page fill (bench / tests): integer hash, same spec as the
 * oracle's generator, computed on the device.
 * ====================================================================== */
int s14_fill_mxfp4_page(s14_ctx *ctx, void *stream, uint8_t *page, uint64_t seed,
                        uint32_t layer, uint32_t expert, uint32_t hidden, uint32_t inter,
                        int lo_exp, int hi_exp);

/* ======================================================================
 * VRAM page pool — VramPool, vram_pool.rs:62-405
 * ====================================================================== */
typedef struct {
  uint32_t layer;
  uint8_t kind; /* 0x53 routed, 0x54 shared (s14_vulkan.rs:14-15) */
  uint32_t slot;
} s14_expert_key;

#define S14_ROUTED_EXPERT_KIND 0x53
#define S14_SHARED_EXPERT_KIND 0x54

/* SlotBinding (vram_pool.rs:30-37); a lease is the binding of a pinned page. */
typedef struct {
  s14_expert_key key;
  uint32_t slot;
  uint64_t generation;
} s14_slot_binding;

/* LoadingReservation (vram_pool.rs:53-60). */
typedef struct {
  s14_expert_key key;
  uint32_t slot;
  uint64_t generation;
  int has_evicted;
  s14_expert_key evicted;
} s14_loading_reservation;

typedef struct s14_pool s14_pool;

/* VramPool::new (vram_pool.rs:78-111): one hipMalloc of n_slots*slot_bytes on
 * ctx's device.  ctx == NULL creates a host-only bookkeeping pool with no
 * device arena (the reference's new_for_tests, vram_pool.rs:407-421). */
int s14_pool_create(s14_ctx *ctx, uint32_t n_slots, uint64_t slot_bytes, s14_pool **out);
void s14_pool_destroy(s14_pool *pool);
uint32_t s14_pool_capacity(const s14_pool *pool);
uint64_t s14_pool_slot_bytes(const s14_pool *pool);
uint32_t s14_pool_n_loaded(const s14_pool *pool);
uint64_t s14_pool_total_bytes(const s14_pool *pool);
/* slot_offset (vram_pool.rs:399-401). */
uint64_t s14_pool_slot_offset(const s14_pool *pool, uint32_t slot);
/* Device address of a slot (NULL for a host-only pool). */
void *s14_pool_slot_ptr(const s14_pool *pool, uint32_t slot);
/* lookup (vram_pool.rs:127-135): 1 and *slot if Ready, 0 if absent. */
int s14_pool_lookup(s14_pool *pool, s14_expert_key key, uint32_t *slot);
/* lookup_and_pin (vram_pool.rs:138-161): *found = 0 if absent. */
int s14_pool_lookup_and_pin(s14_pool *pool, s14_expert_key key, int *found,
                            s14_slot_binding *lease);
/* reserve_loading (vram_pool.rs:166-169). */
int s14_pool_reserve_loading(s14_pool *pool, s14_expert_key key, uint32_t *slot,
                             int *has_evicted, s14_expert_key *evicted);
/* reserve_loading_generation (vram_pool.rs:172-235). */
int s14_pool_reserve_loading_generation(s14_pool *pool, s14_expert_key key,
                                        s14_loading_reservation *out);
/* mark_ready (vram_pool.rs:238-260). */
int s14_pool_mark_ready(s14_pool *pool, uint32_t slot, s14_expert_key key);
/* validate_publish_batch (vram_pool.rs:263-306). */
int s14_pool_validate_publish_batch(const s14_pool *pool, const s14_loading_reservation *r,
                                    size_t n);
/* publish_batch_and_pin (vram_pool.rs:310-339): leases_out[n]. */
int s14_pool_publish_batch_and_pin(s14_pool *pool, const s14_loading_reservation *r, size_t n,
                                   s14_slot_binding *leases_out);
/* validate_binding (vram_pool.rs:343-360). */
int s14_pool_validate_binding(const s14_pool *pool, s14_slot_binding binding);
/* release_after_compute_fence (vram_pool.rs:362-366). */
int s14_pool_release_after_compute_fence(s14_pool *pool, s14_slot_binding lease);
/* cancel_loading (vram_pool.rs:369-375): no-op unless Loading(key). */
void s14_pool_cancel_loading(s14_pool *pool, uint32_t slot, s14_expert_key key);
/* cancel_reservation (vram_pool.rs:377-396). */
int s14_pool_cancel_reservation(s14_pool *pool, s14_loading_reservation r);
/* Copy host bytes into a Loading slot on ctx's copy stream and record the
 * transfer fence (a hipEvent).  The fence replaces the Vulkan transfer
 * fence of expert_loader.rs:198-263; the page may be published only after
 * s14_fence_query reports it complete. */
typedef struct s14_fence s14_fence;
int s14_pool_upload(s14_ctx *ctx, s14_pool *pool, const s14_loading_reservation *r,
                    const void *host, uint64_t bytes, s14_fence **fence_out);
/* Record a fence on `stream` (e.g. after the compute that consumes a lease). */
int s14_fence_record(s14_ctx *ctx, void *stream, s14_fence **fence_out);
/* S14_OK if complete, S14_ERR_NOT_READY if pending. */
int s14_fence_query(s14_fence *fence);
int s14_fence_wait(s14_fence *fence);
void s14_fence_destroy(s14_fence *fence);

/* ======================================================================
 * Expert page uploader — ExpertLoader, expert_loader.rs:1-474
 * ====================================================================== */

/* A ring of pipeline_depth pinned host staging slots (hipHostMalloc) of
 * staging_bytes each, one hipEvent transfer fence per slot, copies on ctx's
 * copy stream (ExpertLoader::new_with_staging_bytes, expert_loader.rs:51-104).
 * A loader is used by one thread at a time, like the reference's &mut self. */
typedef struct s14_loader s14_loader;
/* Fills dst with the page of `key` (bytes long); returns 0 on success.  The
 * role of ExpertReader::read_into (expert_loader.rs:209-218). */
typedef int (*s14_read_fn)(void *user, s14_expert_key key, void *dst, uint64_t bytes);
int s14_loader_create(s14_ctx *ctx, uint32_t pipeline_depth, uint64_t staging_bytes, s14_loader **out);
/* Waits only for submitted transfers, then frees the ring (expert_loader.rs:444-458). */
void s14_loader_destroy(s14_loader *loader);
/* enqueue (expert_loader.rs:163-284): a Ready key returns its slot; a key
 * still in the ring has its transfer completed and returns its slot;
 * otherwise the next ring slot's previous transfer is completed (fence wait,
 * then mark_ready), a Loading slot is reserved (may evict), the page is read
 * into the staging slot and its hipMemcpyAsync and fence are submitted.  The
 * page is visible through s14_pool_lookup only after its fence completes
 * (a later enqueue reusing the ring slot, s14_loader_wait_all, or a repeat
 * enqueue of the key).  A failed read cancels the reservation.
 * S14_ERR_CAPACITY if bytes exceed the staging slot or the pool slot. */
int s14_loader_enqueue(s14_loader *loader, s14_pool *pool, s14_expert_key key, uint64_t bytes,
                       s14_read_fn read, void *user, uint32_t *slot_out);
/* enqueue_from_buf (expert_loader.rs:362-442): the same from bytes already in host memory. */
int s14_loader_enqueue_from_buf(s14_loader *loader, s14_pool *pool, s14_expert_key key, const void *data,
                                uint64_t bytes, uint32_t *slot_out);
/* wait_all (expert_loader.rs:286-291): complete and publish every transfer in the ring. */
int s14_loader_wait_all(s14_loader *loader, s14_pool *pool);
/* batch_enqueue (expert_loader.rs:299-360): settle the ring, deduplicate the
 * keys, reject more distinct keys than the pool has slots (S14_ERR_CAPACITY),
 * then enqueue in waves no deeper than the ring, draining between waves; the
 * last wave stays in flight.  slots_out[i] is the VRAM slot of keys[i]. */
int s14_loader_batch_enqueue(s14_loader *loader, s14_pool *pool, const s14_expert_key *keys,
                             const uint64_t *bytes, size_t n, s14_read_fn read, void *user, uint32_t *slots_out);
/* The same with every page's bytes already in host memory (data[i], bytes[i]). */
int s14_loader_batch_enqueue_from_bufs(s14_loader *loader, s14_pool *pool, const s14_expert_key *keys,
                                       const void *const *data, const uint64_t *bytes, size_t n,
                                       uint32_t *slots_out);
/* stat_loads / stat_bytes (expert_loader.rs:38-40) and transfers in flight. */
int s14_loader_stats(const s14_loader *loader, uint64_t *loads, uint64_t *bytes, uint32_t *in_flight);

/* ======================================================================
 * Route decisions and two-pool page batches — s14_vulkan.rs:500-819
 * ====================================================================== */
enum { S14_PROFILE_S14_TOP6 = 0, S14_PROFILE_FULL_DEPTH43_TOP6 = 1 };
enum { S14_ROUTER_HASH = 0, S14_ROUTER_SCORE = 1 };
typedef struct {
  uint8_t layer;
  int kind;               /* S14_ROUTER_* */
  uint32_t n;             /* number of ids/weights (must equal 6) */
  uint16_t expert_ids[16];
  float weights[16];
} s14_route_decision;

/* RouteDecision::validate_for (runner.rs:128-180); the weight-sum target is
 * a parameter: 1.5 for the reference's route_scale, 1.0 for renormalised
 * weights.  Tolerance 1e-4 as in the reference. */
int s14_route_validate_for(const s14_route_decision *route, int profile, float weight_sum);

typedef struct s14_moe_pages s14_moe_pages;
typedef struct s14_route_load_batch s14_route_load_batch;
typedef struct s14_moe_lease_batch s14_moe_lease_batch;

/* S14VulkanMoePages::new (s14_vulkan.rs:710-734): routed slots must hold
 * EXPERT_PAGE_BYTES; shared slots S14_SHARED_EXPERT_PAGE_BYTES for the
 * reference's FP8 shared page (S14_PAGE_FP8) or EXPERT_PAGE_BYTES for an
 * MXFP4 shared page (S14_PAGE_MXFP4).  weight_sum: see s14_route_validate_for. */
int s14_moe_pages_create(s14_pool *routed, s14_pool *shared, int profile, int shared_format,
                         float weight_sum, s14_moe_pages **out);
void s14_moe_pages_destroy(s14_moe_pages *pages);
/* begin_after_official_route (s14_vulkan.rs:736-774): validate, then pin
 * cached pages or reserve Loading slots for the 6 routed pages and the
 * layer's shared page; on any failure roll everything back. */
int s14_moe_pages_begin_after_official_route(s14_moe_pages *pages,
                                             const s14_route_decision *route,
                                             s14_route_load_batch **out);
/* Pages of a batch: index 0..n-2 routed in route order, n-1 shared.
 * *loading = 1 if the page still needs an upload into its reservation. */
uint32_t s14_route_load_batch_size(const s14_route_load_batch *b);
int s14_route_load_batch_page(const s14_route_load_batch *b, uint32_t i, int *loading,
                              s14_loading_reservation *reservation, s14_slot_binding *cached);
/* publish_after_transfer_fence (s14_vulkan.rs:777-800): preflight both pools,
 * then publish+pin all; otherwise roll back everything.  Consumes the batch
 * (freed whether or not it succeeds). */
int s14_moe_pages_publish_after_transfer_fence(s14_moe_pages *pages, s14_route_load_batch *batch,
                                               s14_moe_lease_batch **out);
/* Bindings of a lease batch: routed[6] then shared. */
int s14_moe_lease_batch_bindings(const s14_moe_lease_batch *lease, s14_slot_binding *routed,
                                 uint32_t n_routed, s14_slot_binding *shared);
/* release_after_compute_fence (s14_vulkan.rs:802-812).  Consumes the lease
 * batch on success; on failure the batch stays valid. */
int s14_moe_pages_release_after_compute_fence(s14_moe_pages *pages, s14_moe_lease_batch *lease);
/* cancel (s14_vulkan.rs:814-818).  Consumes the batch. */
int s14_moe_pages_cancel(s14_moe_pages *pages, s14_route_load_batch *batch);
/* Test hook mirroring the reference test that reaches into the pool
 * (s14_vulkan.rs:962-996): the shared page's reservation, if Loading. */
int s14_route_load_batch_shared_reservation(const s14_route_load_batch *b,
                                            s14_loading_reservation *out);

#ifdef __cplusplus
}
#endif
#endif /* S14_HIP_H */
