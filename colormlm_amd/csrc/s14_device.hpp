// Launchers of the gfx950 kernels in s14_device.hip, called by the C ABI in
// s14_api.cpp.  All pointers are device pointers; every launcher enqueues on
// `stream` and returns the hipError_t of the launch.
#pragma once

#include <hip/hip_runtime_api.h>
#include <stdint.h>

#include "s14_hip.h"

namespace s14 {

constexpr int kMaxTokens = 8;
constexpr int kTopK = 6;
constexpr int kMaxPairs = kMaxTokens * (kTopK + 1);  // (token, expert) pairs incl. shared
constexpr int kHidden = 4096;
constexpr int kInter = 2048;
constexpr int kMaxExperts = 256;

// Exact-mode tiles (one row per lane pair): phase 1 = 16 rows of w1 + the
// same 16 rows of w3 per wavefront; phase 2 = 16 rows of w2 for each of the
// token's pairs, two pairs per wavefront.
constexpr int kP1ExactRows = 16;
constexpr int kP1ExactWaves = 4;  // phase-1 row tiles per workgroup, sharing one staged x
constexpr int kP2ExactRows = 16;
constexpr int kP2ExactWaves = 4;
// Fast-mode tiles: phase 1 = 4 wavefronts x R rows of w1 and w3 (streamed, two row
// pairs of codes in flight per wavefront; R = 8 for single-token launches, 16 for blocks,
// the measured best of 4 / 8 / 16 rows at depths 1-6); phase 2 = 16 rows of w2 per
// wavefront (one wavefront per pair of the token).
constexpr int p1_fast_rows_per_wave(int tier) { return tier == 1 ? 8 : 16; }
constexpr int kP1FastDepth = 2;  // row pairs of codes in flight per wavefront
constexpr int kFastWaves = 4;
constexpr int p1_fast_rows(int tier) { return p1_fast_rows_per_wave(tier) * kFastWaves; }
constexpr int kP2FastRows = 16;

constexpr int kSlots = kTopK + 1;  // pairs of one token: routed + shared
// Route completion counters: groups, then <= 16 groups of 16 workgroups,
// each on its own 128-byte line (atomics to one line serialize).
constexpr uint32_t kRouteCounterStride = 32;
constexpr uint32_t kRouteCounters = (1 + 16) * kRouteCounterStride;

// Work of a layer or block launch.  Phase 1 runs one grid row per
// (token, expert) pair: routed pairs first, sorted by expert id so that all
// tokens of one expert page are consecutive in the grid, the shared
// expert's pairs last.  Phase 2 walks each token's pairs in accumulation
// order (routed in route order, shared last) through per-token slot records,
// so that a workgroup finds everything about its token with one round trip.
struct PairTable {
  uint32_t n_pairs;
  uint32_t n_tokens;
  uint32_t n_distinct;  // distinct routed pages
  uint32_t chain;       // 1: output = weight * down (the single-expert chain)
  // per pair (phase 1)
  uint64_t page[kMaxPairs];
  uint32_t fmt[kMaxPairs];
  uint32_t token[kMaxPairs];
  float weight[kMaxPairs];  // route weight (1 for the shared expert): official mode applies it in phase 1
  // per token and slot (phase 2)
  uint32_t npairs[kMaxTokens];
  uint32_t slot_pair[kMaxTokens][kSlots];  // pair index: row of the h buffer
  uint32_t slot_fmt[kMaxTokens][kSlots];
  uint32_t slot_shared[kMaxTokens][kSlots];
  float slot_weight[kMaxTokens][kSlots];  // route weight; 1 for the shared expert
  uint64_t slot_page[kMaxTokens][kSlots];
};

// Host-built plans (fixed routes): pair p runs `page` for `token`, and is
// slot j of that token's accumulation.
inline void plan_pair(PairTable &t, uint32_t p, const void *page, uint32_t fmt, uint32_t token, uint32_t j,
                      float weight, bool shared) {
  t.page[p] = reinterpret_cast<uint64_t>(page);
  t.fmt[p] = fmt;
  t.token[p] = token;
  t.weight[p] = shared ? 1.0f : weight;
  t.slot_pair[token][j] = p;
  t.slot_page[token][j] = reinterpret_cast<uint64_t>(page);
  t.slot_fmt[token][j] = fmt;
  t.slot_weight[token][j] = weight;
  t.slot_shared[token][j] = shared ? 1u : 0u;
}

// Device workspace of a context (one allocation, carved by s14_api.cpp).
struct Workspace {
  PairTable *table;
  float *h;       // [kMaxPairs][kInter]
  float *scores;  // [kMaxTokens][kMaxExperts]
  float *biased;  // [kMaxTokens][kMaxExperts]
  uint32_t *route_count;  // [kRouteCounters]: groups, then per-group workgroups, of the running route launch that are done (one per 128-byte line)
  uint32_t *hwin;         // [kMaxPairs][kInter / kP1ExactRows]: exponent range (lo | hi << 16) of each exact phase-1 tile's h
  uint32_t *xwin;         // [kMaxTokens]: exponent range (lo | hi << 16) of each token's x (official: of its act_quant), written by the block route
  // kSyncLines lines of kRouteCounterStride words: the status word (kStatus*
  // bits) that launches leave for s14_launch_status.
  uint32_t *sync;
  float *down;  // [kMaxPairs][kHidden]: each pair's w2 output of a block launch (before its route weight)
  float *xq;    // [kMaxTokens][kHidden]: official mode's act_quant of x (dequantised), written by the route launch
  size_t bytes;
};
constexpr uint32_t kSyncLines = 1;
constexpr uint32_t kSyncStatusLine = kSyncLines - 1;  // the status word's line
inline uint32_t *status_word(const Workspace &ws) { return ws.sync + kSyncStatusLine * kRouteCounterStride; }
// Status bits a launch leaves in the status line of ws.sync (sticky until
// read by s14_launch_status).
enum : uint32_t { kStatusNullPage = 1u, kStatusBadRoute = 2u };

// Layout of the workspace in one device allocation (each region 256-byte
// aligned): table | h | scores | biased | route counters | h windows | x
// windows | status line | w2 rows | requantised x.
struct WorkspaceLayout {
  size_t table, h, scores, biased, count, hwin, xwin, sync, down, xq, bytes;
};
constexpr size_t ws_align(size_t v) { return (v + 255) / 256 * 256; }
constexpr WorkspaceLayout workspace_layout() {
  WorkspaceLayout l{};
  size_t off = 0;
  l.table = off;
  off = ws_align(off + sizeof(PairTable));
  l.h = off;
  off = ws_align(off + sizeof(float) * kMaxPairs * kInter);
  l.scores = off;
  off = ws_align(off + sizeof(float) * kMaxTokens * kMaxExperts);
  l.biased = off;
  off = ws_align(off + sizeof(float) * kMaxTokens * kMaxExperts);
  l.count = off;
  off = ws_align(off + sizeof(uint32_t) * kRouteCounters);
  l.hwin = off;
  off = ws_align(off + sizeof(uint32_t) * kMaxPairs * (kInter / kP1ExactRows));
  l.xwin = off;
  off = ws_align(off + sizeof(uint32_t) * kMaxTokens);
  l.sync = off;
  off = ws_align(off + sizeof(uint32_t) * kSyncLines * kRouteCounterStride);
  l.down = off;
  off = ws_align(off + sizeof(float) * kMaxPairs * kHidden);
  l.xq = off;
  off = ws_align(off + sizeof(float) * kMaxTokens * kHidden);
  l.bytes = off;
  return l;
}
constexpr size_t kWorkspaceBytes = workspace_layout().bytes;

// The workspace views of the allocation at `base` (kWorkspaceBytes bytes,
// 256-byte aligned).
inline Workspace workspace_carve(void *base) {
  constexpr WorkspaceLayout l = workspace_layout();
  uint8_t *b = static_cast<uint8_t *>(base);
  Workspace ws{};
  ws.table = reinterpret_cast<PairTable *>(b + l.table);
  ws.h = reinterpret_cast<float *>(b + l.h);
  ws.scores = reinterpret_cast<float *>(b + l.scores);
  ws.biased = reinterpret_cast<float *>(b + l.biased);
  ws.route_count = reinterpret_cast<uint32_t *>(b + l.count);
  ws.hwin = reinterpret_cast<uint32_t *>(b + l.hwin);
  ws.xwin = reinterpret_cast<uint32_t *>(b + l.xwin);
  ws.sync = reinterpret_cast<uint32_t *>(b + l.sync);
  ws.down = reinterpret_cast<float *>(b + l.down);
  ws.xq = reinterpret_cast<float *>(b + l.xq);
  ws.bytes = l.bytes;
  return ws;
}

struct PageOffsets {
  uint64_t w1, s1, w3, s3, w2, s2;
};

struct RouterArgs {
  const float *weight;
  const float *bias;
  uint32_t n_experts;
  uint32_t topk;
  int score_fn;
  float route_scale;
  const int64_t *tid2eid;  // hash routing: [vocab][topk] expert rows; NULL: biased top-k
  uint32_t vocab;
  const int32_t *token_ids;  // [tokens] (hash routing)
};

// Where a device-routed launch finds its pages and reports its routes.
struct RouteSpec {
  RouterArgs r;
  uint32_t tokens;
  int shared_fmt;
  const uint64_t *expert_pages;
  const uint8_t *shared_page;
  uint16_t *ids_out;
  float *weights_out;
  uint32_t *status;  // the workspace's status word (kStatus* bits)
};

// Optional start/stop events a fused launcher attaches to its kernel launch
// (hipExtLaunchKernelGGL): they time the kernel's own execution.
struct KernelEvents {
  hipEvent_t start = nullptr;
  hipEvent_t stop = nullptr;
};

// --- standalone dispatches (bind/cmd API) ---
hipError_t launch_mxfp4_matvec(hipStream_t s, const s14_mxfp4_dispatch &d);
hipError_t launch_fp8_matvec(hipStream_t s, const s14_fp8_dispatch &d);
hipError_t launch_swiglu(hipStream_t s, const s14_swiglu_dispatch &d);
hipError_t launch_route_mix(hipStream_t s, const s14_scale_dispatch &d);
hipError_t launch_moe_accumulate(hipStream_t s, const s14_scale_dispatch &d);
hipError_t launch_dequant_mxfp4(hipStream_t s, s14_shape shape, const uint8_t *w,
                                const uint8_t *sc, float *out);
hipError_t launch_dequant_fp8(hipStream_t s, s14_shape shape, const uint8_t *w, const void *sc,
                              int scale_dtype, float *out);
hipError_t launch_fill_mxfp4_page(hipStream_t s, uint8_t *page, uint64_t seed, uint32_t layer,
                                  uint32_t expert, uint32_t hidden, uint32_t inter, int lo, int hi,
                                  const PageOffsets &off);

// Zeroes the route kernel's completion counters and the status word of a
// workspace (the counters start at 0 and every route launch leaves them at
// 0).
hipError_t launch_clear_route_counters(hipStream_t s, const Workspace &ws);

// --- fused layer / block path: route (router + plan) -> phase 1 -> phase 2 ---
// Scores and biased scores of every (token, expert) into ws.scores/biased
// (the prefill's router; the layer path uses launch_route).  requant 1 / 2:
// the same launch also requantises x into q [tokens][4096] e4m3 and qs
// [tokens][128] E8M0 (groups of 32 / the official groups of 128).
hipError_t launch_router_scores(hipStream_t s, const Workspace &ws, const RouterArgs &r,
                                uint32_t tokens, const float *x, KernelEvents ev = {}, int requant = 0,
                                uint8_t *q = nullptr, uint8_t *qs = nullptr);
// Scores, then the top-k and weights of every token to rs.ids_out /
// weights_out when given; with rs.expert_pages also the pair table in
// ws.table.  One launch (the last workgroup plans).  requant_x: one more
// workgroup per token writes the official act_quant of x (group 128,
// dequantised) to ws.xq and its exponent range to ws.xwin, for the official
// block engine.
hipError_t launch_route(hipStream_t s, const Workspace &ws, const RouteSpec &rs, const float *x,
                        KernelEvents ev = {}, bool requant_x = false);
// The same launch's scoring alone (no plan, no table): for one routed
// token, whose phase 1 plans from the scores itself (launch_phase1 with
// `route`).  official: one more workgroup writes the official act_quant of
// x (group 128, dequantised) to ws.xq, which the official phase 1 stages
// instead of requantising x in every workgroup.
hipError_t launch_route_scores(hipStream_t s, const Workspace &ws, const RouteSpec &rs, const float *x,
                               KernelEvents ev = {}, bool official = false);
// w1/w3 + SwiGLU of every pair.  host_plan != NULL: the pairs are given and
// workgroup (0,0) publishes them for phase 2; route != NULL (one token):
// every workgroup of a routed pair selects the top-k from the scores of
// launch_route_scores, and workgroup (0,0) reports the route and publishes
// the table; otherwise the pairs are read from the table launch_route wrote.
// More than one token: FAST only (EXACT and official blocks run the block
// engine below); other modes return hipErrorInvalidValue.
hipError_t launch_phase1(hipStream_t s, const Workspace &ws, const PairTable *host_plan,
                         uint32_t n_pairs, uint32_t tokens, const PageOffsets &mx,
                         const PageOffsets &fp8, const float *x, int mode, KernelEvents ev = {},
                         const RouteSpec *route = nullptr);
// Blocks of 2..8 tokens in EXACT order, one row per lane (s14_block.hip):
// phase 1 and phase 2 of the pairs [p0, p0 + n_pairs) of the table the route
// kernel wrote, then each token's route-order accumulation of its pairs'
// outputs into y [tokens][hidden].  official: the official expert semantics
// (x from ws.xq, which launch_route with requant_x wrote; bf16 g, u, h and
// w2 outputs, the route weight before w2, h's act_quant inside phase 1).
hipError_t launch_block_phase1(hipStream_t s, const Workspace &ws, uint32_t p0, uint32_t n_pairs,
                               const PageOffsets &mx, const PageOffsets &fp8, const float *x, bool official,
                               KernelEvents ev = {});
hipError_t launch_block_phase2(hipStream_t s, const Workspace &ws, uint32_t p0, uint32_t n_pairs,
                               const PageOffsets &mx, const PageOffsets &fp8, bool official,
                               hipEvent_t ev_start = nullptr);
hipError_t launch_block_combine(hipStream_t s, const Workspace &ws, uint32_t tokens, float *y, bool official,
                                hipEvent_t ev_stop = nullptr);
// The single-expert chain (one MXFP4 page, y = weight * down) in EXACT
// order with lane quads: its phase 1 and phase 2.
hipError_t launch_chain_quad(hipStream_t s, const Workspace &ws, const uint8_t *page, const PageOffsets &mx,
                             const float *x, float weight, float *y, KernelEvents ev1 = {}, KernelEvents ev2 = {});
// w2 of every pair and the per-token accumulation into y [tokens][hidden]
// (more than one token: FAST only, as launch_phase1).
hipError_t launch_phase2(hipStream_t s, const Workspace &ws, uint32_t tokens,
                         const PageOffsets &mx, const PageOffsets &fp8, float *y, int mode,
                         KernelEvents ev = {});

}  // namespace s14
