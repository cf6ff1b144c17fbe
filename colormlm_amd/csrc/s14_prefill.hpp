// Prefill (config 4) launcher and its device workspace, used by the C ABI in
// s14_api.cpp; kernels in s14_prefill.hip.
#pragma once

#include <hip/hip_runtime_api.h>
#include <stdint.h>

#include "s14_device.hpp"

namespace s14 {

constexpr uint32_t kMaxPrefillTokens = 1024;
constexpr uint32_t kPrefillBitWords = kMaxPrefillTokens / 32;  // token bitmap words per expert
constexpr uint32_t kItemTokens = 32;  // tokens of one expert per GEMM work item: one MFMA column tile
constexpr uint32_t kNarrowTokens = 16;  // items of at most this many tokens run one 16-column half

// One GEMM work item: `count` consecutive pairs of one expert, starting at
// pair `first` (expert kMaxExperts is the shared expert).
struct PrefillItem {
  uint32_t expert;
  uint32_t first;
  uint32_t count;
};

// Item tiles: the activation operand (B) of one work item laid out so each
// 128-k super-step is two coalesced 1 KiB loads per 16-column half:
// tile[super-step][half][plane p][lane][16 bytes], lane = c + 16 q holding
// the e4m3 codes of k 32 q + 16 p .. +15 of the super-step for column 16 half
// + c, one E8M0 block (q) per lane (columns past the item's count are
// neither written nor read; an item of at most kNarrowTokens pairs has only
// half 0).  Scales: [chunk of kChunkSteps 64-k steps][half][lane] u32, byte u
// (0, 1) = the E8M0 of the chunk's super-step u for the lane's block.
constexpr uint32_t kChunkSteps = 4;
constexpr uint32_t kXTileBytes = (kHidden / 64) * 2048;                      // phase 1: 128 KiB
constexpr uint32_t kXScaleBytes = (kHidden / 64 / kChunkSteps) * 2 * 64 * 4; // 8 KiB
constexpr uint32_t kHTileBytes = (kInter / 64) * 2048;                       // phase 2: 64 KiB
constexpr uint32_t kHScaleBytes = (kInter / 64 / kChunkSteps) * 2 * 64 * 4;  // 4 KiB

// Upper bound of the work items of T tokens: every expert contributes at
// most one partial item beyond its full ones.
constexpr uint32_t prefill_max_items(uint32_t tokens) {
  return (kTopK * tokens + kItemTokens - 1) / kItemTokens + kMaxExperts + (tokens + kItemTokens - 1) / kItemTokens;
}

struct PrefillArgs {
  RouterArgs r;
  uint32_t tokens;
  const uint64_t *expert_pages;  // device [256] page addresses
  const uint8_t *shared_page;
  PageOffsets mx;
  const float *x;  // [tokens][4096]
  float *y;        // [tokens][4096]
  uint16_t *ids_out;
  float *weights_out;
  uint32_t *status;  // the context workspace's status word (kStatus* bits)
  int official;      // 1: the official expert semantics (S14_MODE_OFFICIAL)
};

// Device workspace for up to kMaxPrefillTokens tokens (one allocation per
// context, made on the first prefill call).
struct PrefillWorkspace {
  float *scores;          // [T][256]
  float *biased;          // [T][256]
  uint32_t *ids;          // [T][kTopK]
  float *weights;         // [T][kTopK]
  uint32_t *token_bits;   // [256][kPrefillBitWords]
  PrefillItem *items;     // [prefill_max_items]
  uint32_t *stats;        // {items, distinct routed experts, max tokens per expert, pairs}
  uint32_t *pair_token;   // [7T]
  uint32_t *token_pair;   // [T][kSlots]
  uint8_t *xq;            // [T][4096] e4m3
  uint8_t *xs;            // [T][128] E8M0
  uint8_t *xt;            // [items][kXTileBytes] x of each item's pairs, item tile
  uint8_t *xts;           // [items][kXScaleBytes]
  uint8_t *ht;            // [items][kHTileBytes] e4m3 SwiGLU output, item tile
  uint8_t *hts;           // [items][kHScaleBytes]
  float *down;            // [7T][4096]
  float *pair_weight;     // [7T]: each pair's route weight (1 for the shared expert)
  float *hf;              // [7T][2048]: official mode's h (bf16 values) before its group-128 requant
  size_t bytes;
};

hipError_t launch_prefill(hipStream_t s, const PrefillArgs &a, const PrefillWorkspace &ws);

}  // namespace s14
