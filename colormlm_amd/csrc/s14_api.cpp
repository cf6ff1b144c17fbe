// C ABI of the S14 path: contexts, bind/cmd dispatch, fused expert entry
// points, the pool's device arena and the hipEvent fences.
//
// Replaces scheduler/ssd_inference/src/s14_vulkan.rs:187-498 (pipelines,
// bind_*, cmd_*) and the Vulkan substrate it sits on (device.rs, buffer.rs,
// compute.rs): a context owns a compute stream, a copy stream and one device
// workspace; "binding" is validation into a plain record; "recording" is a
// kernel launch on a stream; fences are hipEvents.
#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstring>
#include <new>

#include "s14_device.hpp"
#include "s14_internal.hpp"
#include "s14_linear.hpp"
#include "s14_prefill.hpp"

using s14::fail;

namespace {
// stages of a fused launch timed by per-kernel start/stop events
enum { kStageRoute = 0, kStagePhase1 = 1, kStagePhase2 = 2, kStages = 3 };
}  // namespace

struct s14_ctx {
  int device = 0;
  hipStream_t compute = nullptr;
  hipStream_t copy = nullptr;
  s14::BlockFork fork{};  // side stream and events of EXACT blocks
  void *ws_base = nullptr;
  void *prefill_base = nullptr;  // prefill workspace, made on the first prefill call
  void *lin_base = nullptr;      // fp8_linear FAST split-K workspace, made on the first FAST call
  s14::LinearWorkspace lws{};
  uint32_t prefill_tokens = 0;   // token count of the last prefill
  s14::PrefillWorkspace pws{};
  s14::Workspace ws{};
  s14::PageOffsets mx{}, fp8{};
  // optional per-kernel timing of the fused entry points (the role of the
  // reference's Vulkan timestamp queries): router scores, plan, phase 1,
  // phase 2
  bool stage_timing = false;
  hipEvent_t stage_ev[2 * kStages] = {};  // start/stop per stage kernel
  uint32_t stage_mask = 0;                 // stages the last fused launch ran
  bool stage_valid = false;
};

struct s14_fence {
  hipEvent_t ev = nullptr;
};

namespace {

int hip_fail(hipError_t e, const char *what) {
  return fail(S14_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

#define S14_HIP(call, what)                       \
  do {                                            \
    hipError_t _e = (call);                       \
    if (_e != hipSuccess) return hip_fail(_e, what); \
  } while (0)

// Streams follow HIP's convention: NULL is the device's null (default)
// stream; the context's own streams are passed explicitly.
hipStream_t pick(s14_ctx *ctx, void *stream) {
  (void)ctx;
  return reinterpret_cast<hipStream_t>(stream);
}

uint64_t storage_bytes(uint64_t logical) { return (logical + 3) / 4 * 4; }

int require_capacity(const s14_buffer &b, uint64_t required, const char *label) {
  if (!b.ptr) return fail(S14_ERR_INVALID, "%s buffer is NULL", label);
  if (b.bytes < required)
    return fail(S14_ERR_CAPACITY, "%s buffer is %llu B, requires at least %llu B", label,
                (unsigned long long)b.bytes, (unsigned long long)required);
  return S14_OK;
}

s14::PageOffsets offsets_of(const s14_page_layout &l) { return {l.w1, l.s1, l.w3, l.s3, l.w2, l.s2}; }

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

int check_ctx(s14_ctx *ctx) {
  if (!ctx) return fail(S14_ERR_INVALID, "NULL context");
  return S14_OK;
}

// The standalone matvec kernels address weights and scales through 32-bit
// buffer descriptors and 32-bit row offsets (row * row_bytes < weight
// bytes): shapes whose weight or scale bytes reach 2^32 are rejected here
// rather than wrapping on the device.
int check_u32_extent(uint64_t weight_bytes, uint64_t scale_bytes, const char *label) {
  if (weight_bytes > UINT32_MAX || scale_bytes > UINT32_MAX)
    return fail(S14_ERR_SHAPE, "%s needs %llu weight / %llu scale bytes; at most %u each are addressable", label,
                (unsigned long long)weight_bytes, (unsigned long long)scale_bytes, UINT32_MAX);
  return S14_OK;
}

}  // namespace

// ---------------------------------------------------------------------------
// context
// ---------------------------------------------------------------------------

extern "C" int s14_ctx_create(int device, s14_ctx **out) {
  if (!out) return fail(S14_ERR_INVALID, "NULL context output");
  *out = nullptr;
  int count = 0;
  S14_HIP(hipGetDeviceCount(&count), "hipGetDeviceCount");
  if (device < 0 || device >= count) return fail(S14_ERR_INVALID, "device %d not present (%d visible)", device, count);
  S14_HIP(hipSetDevice(device), "hipSetDevice");
  s14_ctx *ctx = new (std::nothrow) s14_ctx();
  if (!ctx) return fail(S14_ERR_INVALID, "out of host memory");
  ctx->device = device;
  hipError_t e = hipStreamCreateWithFlags(&ctx->compute, hipStreamNonBlocking);
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&ctx->copy, hipStreamNonBlocking);
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&ctx->fork.side, hipStreamNonBlocking);
  if (e == hipSuccess) e = hipEventCreateWithFlags(&ctx->fork.fork, hipEventDisableTiming);
  if (e == hipSuccess) e = hipEventCreateWithFlags(&ctx->fork.join, hipEventDisableTiming);
  if (e != hipSuccess) {
    s14_ctx_destroy(ctx);
    return hip_fail(e, "hipStreamCreate");
  }
  // workspace: table | h | scores | biased | route counters | h windows
  const size_t off = s14::kWorkspaceBytes;
  e = hipMalloc(&ctx->ws_base, off);
  if (e != hipSuccess) {
    s14_ctx_destroy(ctx);
    return hip_fail(e, "hipMalloc(workspace)");
  }
  ctx->ws = s14::workspace_carve(ctx->ws_base);  // route counters zeroed below; each route launch leaves them 0
  // one clear at creation, outside any launch sequence
  e = hipMemset(ctx->ws_base, 0, off);
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e != hipSuccess) {
    s14_ctx_destroy(ctx);
    return hip_fail(e, "hipMemset(workspace)");
  }
  s14_page_layout l;
  s14_page_layout_get(S14_PAGE_MXFP4, S14_HIDDEN, S14_INTER, &l);
  ctx->mx = offsets_of(l);
  s14_page_layout_get(S14_PAGE_FP8, S14_HIDDEN, S14_INTER, &l);
  ctx->fp8 = offsets_of(l);
  *out = ctx;
  s14::clear_error();
  return S14_OK;
}

extern "C" void s14_ctx_destroy(s14_ctx *ctx) {
  if (!ctx) return;
  (void)hipSetDevice(ctx->device);
  if (ctx->compute) (void)hipStreamSynchronize(ctx->compute);
  if (ctx->copy) (void)hipStreamSynchronize(ctx->copy);
  if (ctx->fork.side) (void)hipStreamSynchronize(ctx->fork.side);
  if (ctx->ws_base) (void)hipFree(ctx->ws_base);
  if (ctx->prefill_base) (void)hipFree(ctx->prefill_base);
  if (ctx->lin_base) (void)hipFree(ctx->lin_base);
  if (ctx->compute) (void)hipStreamDestroy(ctx->compute);
  if (ctx->copy) (void)hipStreamDestroy(ctx->copy);
  if (ctx->fork.side) (void)hipStreamDestroy(ctx->fork.side);
  if (ctx->fork.fork) (void)hipEventDestroy(ctx->fork.fork);
  if (ctx->fork.join) (void)hipEventDestroy(ctx->fork.join);
  for (auto ev : ctx->stage_ev)
    if (ev) (void)hipEventDestroy(ev);
  delete ctx;
}

extern "C" void *s14_ctx_compute_stream(s14_ctx *ctx) { return ctx ? ctx->compute : nullptr; }
int s14::ctx_device(const s14_ctx *ctx) { return ctx->device; }
extern "C" void *s14_ctx_copy_stream(s14_ctx *ctx) { return ctx ? ctx->copy : nullptr; }

extern "C" int s14_ctx_synchronize(s14_ctx *ctx) {
  if (int rc = check_ctx(ctx)) return rc;
  S14_HIP(hipStreamSynchronize(ctx->compute), "hipStreamSynchronize(compute)");
  S14_HIP(hipStreamSynchronize(ctx->copy), "hipStreamSynchronize(copy)");
  S14_HIP(hipStreamSynchronize(ctx->fork.side), "hipStreamSynchronize(side)");
  return S14_OK;
}

namespace s14 {
int pool_alloc_arena(s14_ctx *ctx, uint64_t bytes, uint8_t **out, int *device) {
  S14_HIP(hipSetDevice(ctx->device), "hipSetDevice");
  void *p = nullptr;
  S14_HIP(hipMalloc(&p, bytes), "hipMalloc(pool arena)");
  *out = static_cast<uint8_t *>(p);
  *device = ctx->device;
  return S14_OK;
}
void pool_free_arena(int device, uint8_t *base) {
  if (device >= 0) (void)hipSetDevice(device);
  (void)hipFree(base);
}
}  // namespace s14

// ---------------------------------------------------------------------------
// bind (s14_vulkan.rs:206-334)
// ---------------------------------------------------------------------------

extern "C" int s14_bind_mxfp4(s14_shape shape, s14_buffer x, s14_buffer w, s14_buffer sc, s14_buffer y,
                              int mode, s14_mxfp4_dispatch *out) {
  if (!out) return fail(S14_ERR_INVALID, "NULL dispatch output");
  s14_shape_bytes b;
  if (int rc = s14_shape_validate_mxfp4(shape, &b)) return rc;
  if (mode != S14_MODE_EXACT && mode != S14_MODE_FAST) return fail(S14_ERR_INVALID, "unknown mode %d", mode);
  if (int rc = check_u32_extent(b.weight_bytes, b.scale_bytes, "S14 MXFP4 matvec")) return rc;
  if (int rc = require_capacity(x, b.input_bytes, "S14 MXFP4 input")) return rc;
  if (int rc = require_capacity(w, storage_bytes(b.weight_bytes), "S14 MXFP4 weight")) return rc;
  if (int rc = require_capacity(sc, storage_bytes(b.scale_bytes), "S14 MXFP4 scale")) return rc;
  if (int rc = require_capacity(y, b.output_bytes, "S14 MXFP4 output")) return rc;
  if (reinterpret_cast<uintptr_t>(x.ptr) % 16 || reinterpret_cast<uintptr_t>(w.ptr) % 16 ||
      reinterpret_cast<uintptr_t>(sc.ptr) % 4)
    return fail(S14_ERR_INVALID, "S14 MXFP4 buffers need 16-byte x/weight and 4-byte scale alignment");
  *out = s14_mxfp4_dispatch{shape, static_cast<const float *>(x.ptr), static_cast<const uint8_t *>(w.ptr),
                            static_cast<const uint8_t *>(sc.ptr), static_cast<float *>(y.ptr), mode};
  return S14_OK;
}

extern "C" int s14_bind_fp8(s14_shape shape, s14_buffer x, int x_dtype, s14_buffer w, s14_buffer sc,
                            int scale_dtype, s14_buffer y, int mode, s14_fp8_dispatch *out) {
  if (!out) return fail(S14_ERR_INVALID, "NULL dispatch output");
  s14_shape_bytes b;
  if (int rc = s14_shape_validate_fp8(shape, &b)) return rc;
  if (mode != S14_MODE_EXACT && mode != S14_MODE_FAST) return fail(S14_ERR_INVALID, "unknown mode %d", mode);
  if (x_dtype != S14_X_F32 && x_dtype != S14_X_BF16) return fail(S14_ERR_INVALID, "unknown x dtype %d", x_dtype);
  if (scale_dtype != S14_SCALE_UE8M0 && scale_dtype != S14_SCALE_F32)
    return fail(S14_ERR_INVALID, "unknown scale dtype %d", scale_dtype);
  const uint64_t x_bytes = x_dtype == S14_X_BF16 ? uint64_t(shape.k) * 2 : b.input_bytes;
  const uint64_t s_bytes = scale_dtype == S14_SCALE_F32 ? b.scale_bytes * 4 : storage_bytes(b.scale_bytes);
  if (int rc = check_u32_extent(b.weight_bytes, s_bytes, "S14 FP8 matvec")) return rc;
  if (int rc = require_capacity(x, x_bytes, "S14 FP8 input")) return rc;
  if (int rc = require_capacity(w, storage_bytes(b.weight_bytes), "S14 FP8 weight")) return rc;
  if (int rc = require_capacity(sc, s_bytes, "S14 FP8 scale")) return rc;
  if (int rc = require_capacity(y, b.output_bytes, "S14 FP8 output")) return rc;
  *out = s14_fp8_dispatch{shape, x.ptr, static_cast<const uint8_t *>(w.ptr), sc.ptr,
                          static_cast<float *>(y.ptr), x_dtype, scale_dtype, mode};
  return S14_OK;
}

extern "C" int s14_bind_swiglu_limit(uint32_t n, s14_buffer gate, s14_buffer up, s14_buffer y,
                                     s14_swiglu_dispatch *out) {
  if (!out) return fail(S14_ERR_INVALID, "NULL dispatch output");
  if (n == 0) return fail(S14_ERR_SHAPE, "S14 SwiGLU requires non-zero length");
  const uint64_t bytes = uint64_t(n) * 4;
  if (int rc = require_capacity(gate, bytes, "S14 SwiGLU gate")) return rc;
  if (int rc = require_capacity(up, bytes, "S14 SwiGLU up")) return rc;
  if (int rc = require_capacity(y, bytes, "S14 SwiGLU output")) return rc;
  *out = s14_swiglu_dispatch{n, static_cast<const float *>(gate.ptr), static_cast<const float *>(up.ptr),
                             static_cast<float *>(y.ptr)};
  return S14_OK;
}

extern "C" int s14_bind_route_mix(uint32_t n, float w, s14_buffer expert, s14_buffer routed,
                                  s14_scale_dispatch *out) {
  if (!out) return fail(S14_ERR_INVALID, "NULL dispatch output");
  if (n == 0 || !std::isfinite(w) || w < 0.0f)
    return fail(S14_ERR_INVALID, "S14 route mix requires non-zero length and finite non-negative weight");
  const uint64_t bytes = uint64_t(n) * 4;
  if (int rc = require_capacity(expert, bytes, "S14 route mix expert")) return rc;
  if (int rc = require_capacity(routed, bytes, "S14 route mix output")) return rc;
  *out = s14_scale_dispatch{n, w, static_cast<const float *>(expert.ptr), static_cast<float *>(routed.ptr)};
  return S14_OK;
}

extern "C" int s14_bind_moe_accumulate(uint32_t n, float w, s14_buffer expert, s14_buffer acc,
                                       s14_scale_dispatch *out) {
  if (!out) return fail(S14_ERR_INVALID, "NULL dispatch output");
  if (n == 0 || !std::isfinite(w) || w < 0.0f)
    return fail(S14_ERR_INVALID, "S14 MoE accumulate requires non-zero length and finite non-negative weight");
  const uint64_t bytes = uint64_t(n) * 4;
  if (int rc = require_capacity(expert, bytes, "S14 MoE accumulate expert")) return rc;
  if (int rc = require_capacity(acc, bytes, "S14 MoE accumulator")) return rc;
  *out = s14_scale_dispatch{n, w, static_cast<const float *>(expert.ptr), static_cast<float *>(acc.ptr)};
  return S14_OK;
}

// ---------------------------------------------------------------------------
// cmd (s14_vulkan.rs:338-416)
// ---------------------------------------------------------------------------

#define S14_LAUNCH(call, what)                      \
  do {                                              \
    hipError_t _e = (call);                         \
    if (_e != hipSuccess) return hip_fail(_e, what); \
    return S14_OK;                                  \
  } while (0)

extern "C" int s14_cmd_mxfp4_matvec(s14_ctx *ctx, void *stream, const s14_mxfp4_dispatch *d) {
  if (int rc = check_ctx(ctx)) return rc;
  if (!d) return fail(S14_ERR_INVALID, "NULL dispatch");
  S14_LAUNCH(s14::launch_mxfp4_matvec(pick(ctx, stream), *d), "mxfp4_matvec launch");
}
extern "C" int s14_cmd_fp8_matvec(s14_ctx *ctx, void *stream, const s14_fp8_dispatch *d) {
  if (int rc = check_ctx(ctx)) return rc;
  if (!d) return fail(S14_ERR_INVALID, "NULL dispatch");
  S14_LAUNCH(s14::launch_fp8_matvec(pick(ctx, stream), *d), "fp8_matvec launch");
}
extern "C" int s14_cmd_swiglu_limit(s14_ctx *ctx, void *stream, const s14_swiglu_dispatch *d) {
  if (int rc = check_ctx(ctx)) return rc;
  if (!d) return fail(S14_ERR_INVALID, "NULL dispatch");
  S14_LAUNCH(s14::launch_swiglu(pick(ctx, stream), *d), "swiglu launch");
}
extern "C" int s14_cmd_route_mix(s14_ctx *ctx, void *stream, const s14_scale_dispatch *d) {
  if (int rc = check_ctx(ctx)) return rc;
  if (!d) return fail(S14_ERR_INVALID, "NULL dispatch");
  S14_LAUNCH(s14::launch_route_mix(pick(ctx, stream), *d), "route_mix launch");
}
extern "C" int s14_cmd_moe_accumulate(s14_ctx *ctx, void *stream, const s14_scale_dispatch *d) {
  if (int rc = check_ctx(ctx)) return rc;
  if (!d) return fail(S14_ERR_INVALID, "NULL dispatch");
  S14_LAUNCH(s14::launch_moe_accumulate(pick(ctx, stream), *d), "moe_accumulate launch");
}

extern "C" int s14_dequant_mxfp4(s14_ctx *ctx, void *stream, s14_shape shape, const uint8_t *packed,
                                 const uint8_t *scale, float *out) {
  if (int rc = check_ctx(ctx)) return rc;
  if (int rc = s14_shape_validate_mxfp4(shape, nullptr)) return rc;
  if (!packed || !scale || !out) return fail(S14_ERR_INVALID, "NULL dequant buffer");
  S14_LAUNCH(s14::launch_dequant_mxfp4(pick(ctx, stream), shape, packed, scale, out), "dequant launch");
}

extern "C" int s14_dequant_fp8(s14_ctx *ctx, void *stream, s14_shape shape, const uint8_t *weight,
                               const void *scale, int scale_dtype, float *out) {
  if (int rc = check_ctx(ctx)) return rc;
  if (int rc = s14_shape_validate_fp8(shape, nullptr)) return rc;
  if (!weight || !scale || !out) return fail(S14_ERR_INVALID, "NULL dequant buffer");
  S14_LAUNCH(s14::launch_dequant_fp8(pick(ctx, stream), shape, weight, scale, scale_dtype, out),
             "dequant launch");
}

extern "C" int s14_fill_mxfp4_page(s14_ctx *ctx, void *stream, uint8_t *page, uint64_t seed, uint32_t layer,
                                   uint32_t expert, uint32_t hidden, uint32_t inter, int lo_exp, int hi_exp) {
  if (int rc = check_ctx(ctx)) return rc;
  if (!page) return fail(S14_ERR_INVALID, "NULL page");
  if (hi_exp < lo_exp || 127 + lo_exp < 0 || 127 + hi_exp > 254)
    return fail(S14_ERR_INVALID, "scale exponent range [%d, %d] invalid", lo_exp, hi_exp);
  s14_page_layout l;
  if (int rc = s14_page_layout_get(S14_PAGE_MXFP4, hidden, inter, &l)) return rc;
  if (reinterpret_cast<uintptr_t>(page) % 8) return fail(S14_ERR_INVALID, "page must be 8-byte aligned");
  S14_LAUNCH(s14::launch_fill_mxfp4_page(pick(ctx, stream), page, seed, layer, expert, hidden, inter, lo_exp,
                                         hi_exp, offsets_of(l)),
             "fill launch");
}

// ---------------------------------------------------------------------------
// fused expert entry points
// ---------------------------------------------------------------------------

namespace {

// Fused expert entry points also take the official expert semantics.
int check_mode(int mode) {
  if (mode != S14_MODE_EXACT && mode != S14_MODE_FAST && mode != S14_MODE_OFFICIAL)
    return fail(S14_ERR_INVALID, "unknown mode %d", mode);
  return S14_OK;
}

int check_router(const s14_router *r) {
  if (!r || !r->weight || !r->bias) return fail(S14_ERR_INVALID, "router weight/bias missing");
  if (r->n_experts == 0 || r->n_experts > uint32_t(s14::kMaxExperts))
    return fail(S14_ERR_SHAPE, "router n_experts=%u outside 1..%d", r->n_experts, s14::kMaxExperts);
  if (r->topk == 0 || r->topk > uint32_t(s14::kTopK) || r->topk > r->n_experts)
    return fail(S14_ERR_SHAPE, "router topk=%u outside 1..%d", r->topk, s14::kTopK);
  if (r->score_fn != S14_SCORE_SIGMOID && r->score_fn != S14_SCORE_SQRT_SOFTPLUS)
    return fail(S14_ERR_INVALID, "unknown score function %d", r->score_fn);
  if (!std::isfinite(r->route_scale) || r->route_scale <= 0.0f)
    return fail(S14_ERR_INVALID, "route_scale must be finite and positive");
  if (r->tid2eid && (!r->token_ids || r->vocab == 0))
    return fail(S14_ERR_INVALID, "hash routing needs token ids and a non-empty tid2eid table");
  return S14_OK;
}

s14::RouterArgs router_args(const s14_router *r) {
  return s14::RouterArgs{r->weight, r->bias,    r->n_experts, r->topk,     r->score_fn,
                         r->route_scale, r->tid2eid, r->vocab, r->token_ids};
}

// Stage-timing events for stage i of a fused launch (none when off).
s14::KernelEvents stage_events(s14_ctx *ctx, int i) {
  if (!ctx->stage_timing) return {};
  ctx->stage_mask |= 1u << i;
  return {ctx->stage_ev[2 * i], ctx->stage_ev[2 * i + 1]};
}
void stage_begin(s14_ctx *ctx) {
  ctx->stage_mask = 0;
  ctx->stage_valid = false;
}

// phase 1 -> phase 2 (the router and plan stages, when any, precede).
int run_layer(s14_ctx *ctx, hipStream_t st, const s14::PairTable *host_plan, uint32_t n_pairs, uint32_t tokens,
              const float *x, float *y, int mode) {
  hipError_t e = s14::launch_phase1(st, ctx->ws, host_plan, n_pairs, tokens, ctx->mx, ctx->fp8, x, mode,
                                    stage_events(ctx, kStagePhase1));
  if (e != hipSuccess) return hip_fail(e, "phase 1 launch");
  e = s14::launch_phase2(st, ctx->ws, tokens, ctx->mx, ctx->fp8, y, mode, stage_events(ctx, kStagePhase2));
  if (e != hipSuccess) return hip_fail(e, "phase 2 launch");
  ctx->stage_valid = ctx->stage_timing;
  return S14_OK;
}

}  // namespace

extern "C" int s14_expert_chain(s14_ctx *ctx, void *stream, const uint8_t *page, const float *x, float route_w,
                                float *y, int mode) {
  if (int rc = check_ctx(ctx)) return rc;
  if (int rc = check_mode(mode)) return rc;
  if (!page || !x || !y) return fail(S14_ERR_INVALID, "NULL chain buffer");
  if (!std::isfinite(route_w) || route_w < 0.0f)
    return fail(S14_ERR_INVALID, "S14 route mix requires a finite non-negative weight");
  s14::PairTable t{};
  t.n_pairs = 1;
  t.n_tokens = 1;
  t.n_distinct = 1;
  t.chain = 1;
  s14::plan_pair(t, 0, page, S14_PAGE_MXFP4, 0, 0, route_w, false);
  t.npairs[0] = 1;
  hipStream_t st = pick(ctx, stream);
  stage_begin(ctx);
  if (mode == S14_MODE_EXACT) {
    // one pair: lane quads, so that the rows spread over the SIMDs
    const hipError_t e = s14::launch_chain_quad(st, ctx->ws, page, ctx->mx, x, route_w, y,
                                                stage_events(ctx, kStagePhase1), stage_events(ctx, kStagePhase2));
    if (e != hipSuccess) return hip_fail(e, "chain launch");
    ctx->stage_valid = ctx->stage_timing;
    return S14_OK;
  }
  return run_layer(ctx, st, &t, 1, 1, x, y, mode);
}

extern "C" int s14_moe_layer(s14_ctx *ctx, void *stream, uint32_t topk, const uint8_t *const *routed_pages,
                             const float *route_weights, const uint8_t *shared_page, int shared_format,
                             const float *x, float *y, int mode) {
  if (int rc = check_ctx(ctx)) return rc;
  if (int rc = check_mode(mode)) return rc;
  if (topk > uint32_t(s14::kTopK)) return fail(S14_ERR_SHAPE, "topk=%u exceeds %d", topk, s14::kTopK);
  if (topk == 0 && !shared_page) return fail(S14_ERR_SHAPE, "layer needs at least one expert");
  if (!x || !y || (topk && (!routed_pages || !route_weights))) return fail(S14_ERR_INVALID, "NULL layer buffer");
  if (shared_page && shared_format != S14_PAGE_MXFP4 && shared_format != S14_PAGE_FP8)
    return fail(S14_ERR_INVALID, "unknown shared page format %d", shared_format);
  s14::PairTable t{};
  for (uint32_t i = 0; i < topk; ++i) {
    if (!routed_pages[i]) return fail(S14_ERR_INVALID, "routed page %u is NULL", i);
    const float w = route_weights[i];
    if (!std::isfinite(w) || w < 0.0f)
      return fail(S14_ERR_INVALID, "S14 MoE accumulate requires finite non-negative weight (route %u)", i);
    s14::plan_pair(t, i, routed_pages[i], S14_PAGE_MXFP4, 0, i, w, false);
  }
  uint32_t n = topk;
  if (shared_page) {
    s14::plan_pair(t, n, shared_page, uint32_t(shared_format), 0, n, 1.0f, true);
    ++n;
  }
  t.n_pairs = n;
  t.n_tokens = 1;
  t.n_distinct = topk;
  t.npairs[0] = n;
  hipStream_t st = pick(ctx, stream);
  stage_begin(ctx);
  return run_layer(ctx, st, &t, n, 1, x, y, mode);
}

namespace s14 {

int block_route_validate(uint32_t tokens, const s14_router *router, const uint64_t *expert_pages_dev,
                         const uint8_t *shared_page, int shared_format, const float *x, float *y, int mode) {
  if (int rc = check_mode(mode)) return rc;
  if (int rc = check_router(router)) return rc;
  if (router->topk != uint32_t(kTopK)) return fail(S14_ERR_SHAPE, "routed layer requires topk=%d", kTopK);
  if (tokens == 0 || tokens > uint32_t(kMaxTokens))
    return fail(S14_ERR_SHAPE, "block size %u outside 1..%d", tokens, kMaxTokens);
  if (!expert_pages_dev || !shared_page || !x || !y) return fail(S14_ERR_INVALID, "NULL layer buffer");
  if (shared_format != S14_PAGE_MXFP4 && shared_format != S14_PAGE_FP8)
    return fail(S14_ERR_INVALID, "unknown shared page format %d", shared_format);
  return S14_OK;
}

int block_route_launch(hipStream_t st, const Workspace &ws, uint32_t tokens, const s14_router *router,
                       const uint64_t *expert_pages_dev, const uint8_t *shared_page, int shared_format,
                       const float *x, float *y, uint16_t *ids_out, float *weights_out, int mode,
                       const KernelEvents *ev, const BlockFork *fork) {
  s14_page_layout l;
  s14_page_layout_get(S14_PAGE_MXFP4, S14_HIDDEN, S14_INTER, &l);
  const PageOffsets mx = offsets_of(l);
  s14_page_layout_get(S14_PAGE_FP8, S14_HIDDEN, S14_INTER, &l);
  const PageOffsets f8 = offsets_of(l);
  const RouteSpec rs{router_args(router), tokens,      shared_format,  expert_pages_dev, shared_page,
                     ids_out,              weights_out, status_word(ws)};
  const uint32_t n_pairs = tokens * (kTopK + 1);
  if (tokens == 1) {
    // one token: the route launch only scores, and every phase-1 workgroup
    // of a routed pair selects the top-k itself (no last-arrival hand-off)
    hipError_t e = launch_route_scores(st, ws, rs, x, ev ? ev[kStageRoute] : KernelEvents{}, mode == S14_MODE_OFFICIAL);
    if (e != hipSuccess) return hip_fail(e, "router launch");
    e = launch_phase1(st, ws, nullptr, n_pairs, tokens, mx, f8, x, mode, ev ? ev[kStagePhase1] : KernelEvents{}, &rs);
    if (e != hipSuccess) return hip_fail(e, "phase 1 launch");
    e = launch_phase2(st, ws, tokens, mx, f8, y, mode, ev ? ev[kStagePhase2] : KernelEvents{});
    if (e != hipSuccess) return hip_fail(e, "phase 2 launch");
    return S14_OK;
  }
  const bool official = mode == S14_MODE_OFFICIAL;
  // official: the route launch also writes x's act_quant for phase 1
  hipError_t e = launch_route(st, ws, rs, x, ev ? ev[kStageRoute] : KernelEvents{}, official);
  if (e != hipSuccess) return hip_fail(e, "router launch");
  if (tokens > 1 && (mode == S14_MODE_EXACT || official)) {
    // blocks: one row per lane (enough (token, expert) chains to fill the
    // GPU).  With a side stream the pairs run as two halves, one per stream,
    // so that the SIMDs one half's phase-1 tail leaves idle (3.5 equal
    // wavefronts per SIMD, two resident at a time) take the other half's
    // work: K=8 182.9 -> 170.7 us per block (an even split measured best; three
    // or four streams were slower).  Stage events time the first half.
    const uint32_t na = fork ? n_pairs / 2 : n_pairs, nb = n_pairs - na;
    if (fork) {
      if ((e = hipEventRecord(fork->fork, st)) != hipSuccess) return hip_fail(e, "hipEventRecord(fork)");
      if ((e = hipStreamWaitEvent(fork->side, fork->fork, 0)) != hipSuccess) return hip_fail(e, "hipStreamWaitEvent");
    }
    const char *failed = nullptr;
    e = launch_block_phase1(st, ws, 0, na, mx, f8, x, official, ev ? ev[kStagePhase1] : KernelEvents{});
    if (e == hipSuccess && nb) e = launch_block_phase1(fork->side, ws, na, nb, mx, f8, x, official);
    if (e != hipSuccess) {
      failed = "phase 1 launch";
    } else {
      e = launch_block_phase2(st, ws, 0, na, mx, f8, official, ev ? ev[kStagePhase2].start : nullptr);
      if (e == hipSuccess && nb) e = launch_block_phase2(fork->side, ws, na, nb, mx, f8, official);
      if (e != hipSuccess) failed = "phase 2 launch";
    }
    if (fork) {
      // the side stream joins the caller's also after a failed launch, so a
      // capture never ends with an unjoined branch (the launch error is the
      // one reported)
      hipError_t j = hipEventRecord(fork->join, fork->side);
      if (j == hipSuccess) j = hipStreamWaitEvent(st, fork->join, 0);
      if (!failed && j != hipSuccess) {
        e = j;
        failed = "side stream join";
      }
    }
    if (failed) return hip_fail(e, failed);
    e = launch_block_combine(st, ws, tokens, y, official, ev ? ev[kStagePhase2].stop : nullptr);
    if (e != hipSuccess) return hip_fail(e, "combine launch");
    return S14_OK;
  }
  e = launch_phase1(st, ws, nullptr, n_pairs, tokens, mx, f8, x, mode, ev ? ev[kStagePhase1] : KernelEvents{});
  if (e != hipSuccess) return hip_fail(e, "phase 1 launch");
  e = launch_phase2(st, ws, tokens, mx, f8, y, mode, ev ? ev[kStagePhase2] : KernelEvents{});
  if (e != hipSuccess) return hip_fail(e, "phase 2 launch");
  return S14_OK;
}

}  // namespace s14

extern "C" int s14_moe_block_route(s14_ctx *ctx, void *stream, uint32_t tokens, const s14_router *router,
                                   const uint64_t *expert_pages_dev, const uint8_t *shared_page,
                                   int shared_format, const float *x, float *y, uint16_t *ids_out,
                                   float *weights_out, int mode) {
  if (int rc = check_ctx(ctx)) return rc;
  if (int rc = s14::block_route_validate(tokens, router, expert_pages_dev, shared_page, shared_format, x, y, mode))
    return rc;
  stage_begin(ctx);
  s14::KernelEvents ev[kStages];
  if (ctx->stage_timing)
    for (int i = 0; i < kStages; ++i) ev[i] = {ctx->stage_ev[2 * i], ctx->stage_ev[2 * i + 1]};
  const int rc = s14::block_route_launch(pick(ctx, stream), ctx->ws, tokens, router, expert_pages_dev, shared_page,
                                         shared_format, x, y, ids_out, weights_out, mode,
                                         ctx->stage_timing ? ev : nullptr, &ctx->fork);
  if (rc == S14_OK && ctx->stage_timing) {
    ctx->stage_mask = (1u << kStageRoute) | (1u << kStagePhase1) | (1u << kStagePhase2);
    ctx->stage_valid = true;
  }
  return rc;
}

extern "C" int s14_moe_layer_route(s14_ctx *ctx, void *stream, const s14_router *router,
                                   const uint64_t *expert_pages_dev, const uint8_t *shared_page,
                                   int shared_format, const float *x, float *y, uint16_t *ids_out,
                                   float *weights_out, int mode) {
  return s14_moe_block_route(ctx, stream, 1, router, expert_pages_dev, shared_page, shared_format, x, y,
                             ids_out, weights_out, mode);
}

extern "C" int s14_last_block_distinct(s14_ctx *ctx, uint32_t *n_distinct) {
  if (int rc = check_ctx(ctx)) return rc;
  if (!n_distinct) return fail(S14_ERR_INVALID, "NULL output");
  // the launch may have gone to any stream of the device
  S14_HIP(hipSetDevice(ctx->device), "hipSetDevice");
  S14_HIP(hipDeviceSynchronize(), "hipDeviceSynchronize");
  S14_HIP(hipMemcpy(n_distinct, &ctx->ws.table->n_distinct, sizeof(uint32_t), hipMemcpyDeviceToHost),
          "hipMemcpy(n_distinct)");
  return S14_OK;
}

namespace s14 {
int read_launch_status(const Workspace &ws, int device) {
  S14_HIP(hipSetDevice(device), "hipSetDevice");
  S14_HIP(hipDeviceSynchronize(), "hipDeviceSynchronize");
  uint32_t *word = ws.sync + kSyncStatusLine * kRouteCounterStride;
  uint32_t bits = 0;
  S14_HIP(hipMemcpy(&bits, word, sizeof(bits), hipMemcpyDeviceToHost), "hipMemcpy(status)");
  if (!bits) return S14_OK;
  const uint32_t zero = 0;
  S14_HIP(hipMemcpy(word, &zero, sizeof(zero), hipMemcpyHostToDevice), "hipMemcpy(status clear)");
  if (bits & kStatusNullPage)
    return fail(S14_ERR_INVALID, "a routed expert's page address was 0 (page not resident); outputs are NaN");
  return fail(S14_ERR_ROUTE,
              "a token's route failed RouteDecision::validate_for (expert id out of range or repeated, weight "
              "not finite or negative, or weight sum off route_scale by more than 1e-4); its outputs are NaN");
}
}  // namespace s14

extern "C" int s14_launch_status(s14_ctx *ctx) {
  if (int rc = check_ctx(ctx)) return rc;
  return s14::read_launch_status(ctx->ws, ctx->device);
}

extern "C" int s14_route(s14_ctx *ctx, void *stream, const s14_router *router, uint32_t tokens,
                         const float *x, float *scores_out, uint16_t *ids_out, float *weights_out) {
  if (int rc = check_ctx(ctx)) return rc;
  if (int rc = check_router(router)) return rc;
  if (tokens == 0 || tokens > uint32_t(s14::kMaxTokens))
    return fail(S14_ERR_SHAPE, "token count %u outside 1..%d", tokens, s14::kMaxTokens);
  if (!x) return fail(S14_ERR_INVALID, "NULL router input");
  hipStream_t st = pick(ctx, stream);
  const s14::RouteSpec rs{router_args(router), tokens,      S14_PAGE_MXFP4,              nullptr, nullptr,
                          ids_out,              weights_out, s14::status_word(ctx->ws)};
  hipError_t e = s14::launch_route(st, ctx->ws, rs, x);
  if (e != hipSuccess) return hip_fail(e, "router launch");
  if (scores_out) {
    for (uint32_t t = 0; t < tokens; ++t) {
      e = hipMemcpyAsync(scores_out + size_t(t) * router->n_experts, ctx->ws.scores + size_t(t) * s14::kMaxExperts,
                         sizeof(float) * router->n_experts, hipMemcpyDeviceToDevice, st);
      if (e != hipSuccess) return hip_fail(e, "hipMemcpyAsync(scores)");
    }
  }
  return S14_OK;
}

// ---------------------------------------------------------------------------
// prefill (config 4)
// ---------------------------------------------------------------------------

namespace {

// The prefill workspace for kMaxPrefillTokens tokens, allocated once per
// context on first use (no allocation on later calls).
int prefill_workspace(s14_ctx *ctx) {
  if (ctx->prefill_base) return S14_OK;
  using namespace s14;
  const uint32_t T = kMaxPrefillTokens, P = kSlots * kMaxPrefillTokens;
  size_t off = 0;
  auto take = [&off](size_t bytes) {
    const size_t o = off;
    off = align_up(off + bytes, 256);
    return o;
  };
  const size_t o_scores = take(sizeof(float) * T * kMaxExperts);
  const size_t o_biased = take(sizeof(float) * T * kMaxExperts);
  const size_t o_ids = take(sizeof(uint32_t) * T * kTopK);
  const size_t o_w = take(sizeof(float) * T * kTopK);
  const size_t o_bits = take(sizeof(uint32_t) * kMaxExperts * kPrefillBitWords);
  const size_t o_items = take(sizeof(PrefillItem) * prefill_max_items(T));
  const size_t o_stats = take(sizeof(uint32_t) * 4);
  const size_t o_pt = take(sizeof(uint32_t) * P);
  const size_t o_tp = take(sizeof(uint32_t) * T * kSlots);
  const size_t o_xq = take(size_t(T) * kHidden);
  const size_t o_xs = take(size_t(T) * (kHidden / 32));
  const size_t n_items = prefill_max_items(T);
  const size_t o_xt = take(n_items * kXTileBytes);
  const size_t o_xts = take(n_items * kXScaleBytes);
  const size_t o_ht = take(n_items * kHTileBytes);
  const size_t o_hts = take(n_items * kHScaleBytes);
  const size_t o_down = take(sizeof(float) * size_t(P) * kHidden);
  const size_t o_pw = take(sizeof(float) * size_t(P));
  const size_t o_hf = take(sizeof(float) * size_t(P) * kInter);
  S14_HIP(hipSetDevice(ctx->device), "hipSetDevice");
  S14_HIP(hipMalloc(&ctx->prefill_base, off), "hipMalloc(prefill workspace)");
  // the token bitmaps start clear; every prefill's grouping step clears them again
  S14_HIP(hipMemset(static_cast<uint8_t *>(ctx->prefill_base) + o_bits, 0,
                    sizeof(uint32_t) * kMaxExperts * kPrefillBitWords),
          "hipMemset(prefill bitmaps)");
  S14_HIP(hipDeviceSynchronize(), "hipDeviceSynchronize");
  uint8_t *b = static_cast<uint8_t *>(ctx->prefill_base);
  PrefillWorkspace &w = ctx->pws;
  w.scores = reinterpret_cast<float *>(b + o_scores);
  w.biased = reinterpret_cast<float *>(b + o_biased);
  w.ids = reinterpret_cast<uint32_t *>(b + o_ids);
  w.weights = reinterpret_cast<float *>(b + o_w);
  w.token_bits = reinterpret_cast<uint32_t *>(b + o_bits);
  w.items = reinterpret_cast<PrefillItem *>(b + o_items);
  w.stats = reinterpret_cast<uint32_t *>(b + o_stats);
  w.pair_token = reinterpret_cast<uint32_t *>(b + o_pt);
  w.token_pair = reinterpret_cast<uint32_t *>(b + o_tp);
  w.xq = b + o_xq;
  w.xs = b + o_xs;
  w.xt = b + o_xt;
  w.xts = b + o_xts;
  w.ht = b + o_ht;
  w.hts = b + o_hts;
  w.down = reinterpret_cast<float *>(b + o_down);
  w.pair_weight = reinterpret_cast<float *>(b + o_pw);
  w.hf = reinterpret_cast<float *>(b + o_hf);
  w.bytes = off;
  return S14_OK;
}

}  // namespace

extern "C" int s14_moe_prefill(s14_ctx *ctx, void *stream, uint32_t tokens, const s14_router *router,
                               const uint64_t *expert_pages_dev, const uint8_t *shared_page, const float *x,
                               float *y, uint16_t *ids_out, float *weights_out, int mode) {
  if (int rc = check_ctx(ctx)) return rc;
  if (mode != S14_MODE_EXACT && mode != S14_MODE_FAST && mode != S14_MODE_OFFICIAL)
    return fail(S14_ERR_INVALID, "unknown mode %d", mode);
  if (int rc = check_router(router)) return rc;
  if (router->topk != uint32_t(s14::kTopK))
    return fail(S14_ERR_SHAPE, "prefill requires topk=%d", s14::kTopK);
  if (tokens == 0 || tokens > s14::kMaxPrefillTokens)
    return fail(S14_ERR_SHAPE, "prefill token count %u outside 1..%u", tokens, s14::kMaxPrefillTokens);
  if (!expert_pages_dev || !shared_page || !x || !y) return fail(S14_ERR_INVALID, "NULL prefill buffer");
  if (int rc = prefill_workspace(ctx)) return rc;
  hipStream_t st = pick(ctx, stream);
  const s14::PrefillArgs a{router_args(router), tokens,      expert_pages_dev,          shared_page,
                           ctx->mx,              x,           y,                         ids_out,
                           weights_out,          s14::status_word(ctx->ws), mode == S14_MODE_OFFICIAL ? 1 : 0};
  const hipError_t e = s14::launch_prefill(st, a, ctx->pws);
  if (e != hipSuccess) return hip_fail(e, "prefill launch");
  ctx->prefill_tokens = tokens;
  return S14_OK;
}

extern "C" int s14_act_quant_e4m3(s14_ctx *ctx, void *stream, uint32_t rows, uint32_t k, uint32_t group,
                                  const float *x, uint8_t *q, uint8_t *scales) {
  if (int rc = check_ctx(ctx)) return rc;
  if (group != 32 && group != 64 && group != 128) return fail(S14_ERR_SHAPE, "requant group %u is not 32, 64 or 128", group);
  if (rows == 0 || k == 0 || k % group != 0)
    return fail(S14_ERR_SHAPE, "requant needs rows > 0 and k a multiple of the group (%u)", group);
  if (uint64_t(rows) * k >= (uint64_t(1) << 32))
    return fail(S14_ERR_SHAPE, "requant of %u x %u values exceeds 2^32 values", rows, k);
  if (!x || !q || !scales) return fail(S14_ERR_INVALID, "NULL requant buffer");
  const hipError_t e = s14::launch_act_quant(pick(ctx, stream), rows, k, group, x, q, scales);
  if (e != hipSuccess) return hip_fail(e, "requant launch");
  return S14_OK;
}

extern "C" int s14_requant_e4m3(s14_ctx *ctx, void *stream, uint32_t rows, uint32_t k, const float *x,
                                uint8_t *q, uint8_t *scales) {
  return s14_act_quant_e4m3(ctx, stream, rows, k, 32, x, q, scales);
}

// ---------------------------------------------------------------------------
// activation-quantised FP8 linear (fp8.py:111-193)
// ---------------------------------------------------------------------------

namespace {

// FAST's split-K partials and arrival counters, and EXACT's group partials,
// allocated on the first fp8_linear call (counters zeroed once; every launch
// leaves them zero).
int linear_workspace(s14_ctx *ctx) {
  if (ctx->lin_base) return S14_OK;
  const size_t cnt_bytes = sizeof(uint32_t) * s14::kLinMaxCounters;
  S14_HIP(hipSetDevice(ctx->device), "hipSetDevice");
  S14_HIP(hipMalloc(&ctx->lin_base, s14::kLinPartBytes + cnt_bytes), "hipMalloc(linear workspace)");
  uint8_t *b = static_cast<uint8_t *>(ctx->lin_base);
  S14_HIP(hipMemset(b + s14::kLinPartBytes, 0, cnt_bytes), "hipMemset(linear counters)");
  S14_HIP(hipDeviceSynchronize(), "hipDeviceSynchronize");
  ctx->lws.part = reinterpret_cast<float *>(b);
  ctx->lws.count = reinterpret_cast<uint32_t *>(b + s14::kLinPartBytes);
  return S14_OK;
}

}  // namespace

extern "C" int s14_fp8_linear(s14_ctx *ctx, void *stream, uint32_t m, uint32_t n, uint32_t k, s14_buffer x,
                              s14_buffer x_scale, int x_scale_dtype, s14_buffer weight, s14_buffer weight_scale,
                              int weight_scale_dtype, s14_buffer bias, s14_buffer y, int flags, int mode) {
  if (int rc = check_ctx(ctx)) return rc;
  if (mode != S14_MODE_EXACT && mode != S14_MODE_FAST) return fail(S14_ERR_INVALID, "unknown mode %d", mode);
  if (flags & ~S14_LINEAR_ROUND_BF16) return fail(S14_ERR_INVALID, "unknown linear flags 0x%x", flags);
  if (m == 0 || n == 0 || k == 0) return fail(S14_ERR_SHAPE, "fp8_linear needs m, n and k > 0 (m=%u n=%u k=%u)", m, n, k);
  if (k > s14::kLinMaxK) return fail(S14_ERR_SHAPE, "fp8_linear k=%u exceeds %u", k, s14::kLinMaxK);
  const bool xs_f32 = x_scale_dtype == S14_SCALE_F32, ws_f32 = weight_scale_dtype == S14_SCALE_F32;
  if ((!xs_f32 && x_scale_dtype != S14_SCALE_UE8M0) || (!ws_f32 && weight_scale_dtype != S14_SCALE_UE8M0))
    return fail(S14_ERR_INVALID, "unknown scale dtype");
  const uint64_t G = (k + 127) / 128;
  // 32-bit buffer offsets: weight rows of the last 32-row tile, and every
  // activation offset below the out-of-range marker the FAST kernel uses
  if (uint64_t(n + 31) * k > UINT32_MAX || uint64_t(m) * k >= 0xFFFFFF00ull || uint64_t(m) * n > UINT32_MAX)
    return fail(S14_ERR_SHAPE, "fp8_linear m=%u n=%u k=%u exceeds 32-bit addressing", m, n, k);
  if (int rc = require_capacity(x, uint64_t(m) * k, "x")) return rc;
  if (int rc = require_capacity(x_scale, uint64_t(m) * G * (xs_f32 ? 4 : 1), "activation_scale")) return rc;
  if (int rc = require_capacity(weight, uint64_t(n) * k, "weight")) return rc;
  if (int rc = require_capacity(weight_scale, (uint64_t(n) + 127) / 128 * G * (ws_f32 ? 4 : 1), "weight_scale"))
    return rc;
  if (bias.ptr)
    if (int rc = require_capacity(bias, uint64_t(n) * 4, "bias")) return rc;
  if (int rc = require_capacity(y, uint64_t(m) * n * 4, "y")) return rc;
  if (int rc = linear_workspace(ctx)) return rc;
  const s14::LinearArgs a{m,
                          n,
                          k,
                          uint32_t(G),
                          static_cast<const uint8_t *>(x.ptr),
                          x_scale.ptr,
                          xs_f32,
                          static_cast<const uint8_t *>(weight.ptr),
                          weight_scale.ptr,
                          ws_f32,
                          static_cast<const float *>(bias.ptr),
                          static_cast<float *>(y.ptr),
                          (flags & S14_LINEAR_ROUND_BF16) ? 1 : 0};
  const hipError_t e = s14::launch_fp8_linear(pick(ctx, stream), a, mode, ctx->lws);
  if (e != hipSuccess) return hip_fail(e, "fp8_linear launch");
  return S14_OK;
}

extern "C" int s14_last_prefill_stats(s14_ctx *ctx, uint32_t *distinct, uint32_t *max_tokens, uint32_t *n_items) {
  if (int rc = check_ctx(ctx)) return rc;
  if (!ctx->prefill_base) return fail(S14_ERR_NOT_READY, "no prefill launched on this context");
  S14_HIP(hipSetDevice(ctx->device), "hipSetDevice");
  S14_HIP(hipDeviceSynchronize(), "hipDeviceSynchronize");
  uint32_t st[4];
  S14_HIP(hipMemcpy(st, ctx->pws.stats, sizeof(st), hipMemcpyDeviceToHost), "hipMemcpy(prefill stats)");
  if (distinct) *distinct = st[1];
  if (max_tokens) *max_tokens = st[2];
  if (n_items) *n_items = st[0];
  return S14_OK;
}

extern "C" int s14_last_prefill_view(s14_ctx *ctx, s14_prefill_view *out) {
  if (int rc = check_ctx(ctx)) return rc;
  if (!out) return fail(S14_ERR_INVALID, "NULL prefill view");
  if (!ctx->prefill_base || !ctx->prefill_tokens) return fail(S14_ERR_NOT_READY, "no prefill launched on this context");
  S14_HIP(hipSetDevice(ctx->device), "hipSetDevice");
  S14_HIP(hipDeviceSynchronize(), "hipDeviceSynchronize");
  uint32_t st[4];
  S14_HIP(hipMemcpy(st, ctx->pws.stats, sizeof(st), hipMemcpyDeviceToHost), "hipMemcpy(prefill stats)");
  const s14::PrefillWorkspace &w = ctx->pws;
  *out = s14_prefill_view{w.xq,
                          w.xs,
                          w.ht,
                          w.hts,
                          w.down,
                          w.pair_token,
                          w.token_pair,
                          reinterpret_cast<const uint32_t *>(w.items),
                          ctx->prefill_tokens,
                          st[3],
                          st[0]};
  return S14_OK;
}

// ---------------------------------------------------------------------------
// uploads and fences (replacing the Vulkan transfer/compute fences)
// ---------------------------------------------------------------------------

extern "C" int s14_pool_upload(s14_ctx *ctx, s14_pool *pool, const s14_loading_reservation *r,
                               const void *host, uint64_t bytes, s14_fence **fence_out) {
  if (int rc = check_ctx(ctx)) return rc;
  if (!pool || !r || !host || !fence_out) return fail(S14_ERR_INVALID, "NULL upload argument");
  *fence_out = nullptr;
  if (!pool->base) return fail(S14_ERR_INVALID, "pool has no device arena");
  if (r->slot >= pool->n_slots) return fail(S14_ERR_INVALID, "invalid VRAM slot %u", r->slot);
  if (pool->states[r->slot] != SlotState::Loading || !s14::key_eq(pool->state_keys[r->slot], r->key) ||
      pool->generations[r->slot] != r->generation)
    return fail(S14_ERR_STALE, "upload target slot %u is not the reservation's Loading generation", r->slot);
  if (bytes > pool->slot_bytes)
    return fail(S14_ERR_CAPACITY, "upload of %llu B exceeds slot of %llu B", (unsigned long long)bytes,
                (unsigned long long)pool->slot_bytes);
  S14_HIP(hipSetDevice(ctx->device), "hipSetDevice");
  S14_HIP(hipMemcpyAsync(pool->base + uint64_t(r->slot) * pool->slot_bytes, host, bytes, hipMemcpyHostToDevice,
                         ctx->copy),
          "hipMemcpyAsync(upload)");
  return s14_fence_record(ctx, ctx->copy, fence_out);
}

extern "C" int s14_fence_record(s14_ctx *ctx, void *stream, s14_fence **fence_out) {
  if (int rc = check_ctx(ctx)) return rc;
  if (!fence_out) return fail(S14_ERR_INVALID, "NULL fence output");
  *fence_out = nullptr;
  s14_fence *f = new (std::nothrow) s14_fence();
  if (!f) return fail(S14_ERR_INVALID, "out of host memory");
  hipError_t e = hipEventCreateWithFlags(&f->ev, hipEventDisableTiming);
  if (e == hipSuccess) e = hipEventRecord(f->ev, pick(ctx, stream));
  if (e != hipSuccess) {
    if (f->ev) (void)hipEventDestroy(f->ev);
    delete f;
    return hip_fail(e, "hipEventRecord");
  }
  *fence_out = f;
  return S14_OK;
}

extern "C" int s14_fence_query(s14_fence *fence) {
  if (!fence) return fail(S14_ERR_INVALID, "NULL fence");
  hipError_t e = hipEventQuery(fence->ev);
  if (e == hipSuccess) return S14_OK;
  if (e == hipErrorNotReady) return fail(S14_ERR_NOT_READY, "fence not yet signalled");
  return hip_fail(e, "hipEventQuery");
}

extern "C" int s14_fence_wait(s14_fence *fence) {
  if (!fence) return fail(S14_ERR_INVALID, "NULL fence");
  S14_HIP(hipEventSynchronize(fence->ev), "hipEventSynchronize");
  return S14_OK;
}

extern "C" void s14_fence_destroy(s14_fence *fence) {
  if (!fence) return;
  if (fence->ev) (void)hipEventDestroy(fence->ev);
  delete fence;
}

// ---------------------------------------------------------------------------
// stage timestamps
// ---------------------------------------------------------------------------

extern "C" int s14_ctx_enable_stage_timing(s14_ctx *ctx, int enable) {
  if (int rc = check_ctx(ctx)) return rc;
  if (enable && !ctx->stage_ev[0]) {
    for (auto &ev : ctx->stage_ev) S14_HIP(hipEventCreate(&ev), "hipEventCreate(stage)");
  }
  ctx->stage_timing = enable != 0;
  ctx->stage_valid = false;
  return S14_OK;
}

extern "C" int s14_ctx_stage_times(s14_ctx *ctx, float *ms, uint32_t cap, uint32_t *n_stages) {
  if (int rc = check_ctx(ctx)) return rc;
  if (!ms || !n_stages) return fail(S14_ERR_INVALID, "NULL stage-time output");
  if (!ctx->stage_valid) return fail(S14_ERR_NOT_READY, "no timed launch recorded");
  const uint32_t n = cap < uint32_t(kStages) ? cap : uint32_t(kStages);
  for (uint32_t i = 0; i < n; ++i) {
    ms[i] = 0.0f;
    if (!(ctx->stage_mask & (1u << i))) continue;
    S14_HIP(hipEventSynchronize(ctx->stage_ev[2 * i + 1]), "hipEventSynchronize(stage)");
    S14_HIP(hipEventElapsedTime(&ms[i], ctx->stage_ev[2 * i], ctx->stage_ev[2 * i + 1]), "hipEventElapsedTime");
  }
  *n_stages = uint32_t(kStages);
  return S14_OK;
}
