// Internal declarations shared by the host-side translation units of
// libs14hip.so.  Not part of the public ABI (include/s14_hip.h is).
#pragma once

#include <cstdarg>
#include <cstdint>
#include <string>
#include <unordered_map>
#include <vector>

#include "s14_device.hpp"
#include "s14_hip.h"

namespace s14 {

// Argument checks of the routed layer/block entry points (s14_api.cpp).
int block_route_validate(uint32_t tokens, const s14_router *router, const uint64_t *expert_pages_dev,
                         const uint8_t *shared_page, int shared_format, const float *x, float *y, int mode);
// A second stream and two events (all on the context's device) over which
// an EXACT block runs half of its pairs beside the caller's stream.
struct BlockFork {
  hipStream_t side;
  hipEvent_t fork, join;
};
// Route -> phase 1 -> phase 2 of a routed layer/block on `st` with workspace
// `ws` (arguments already validated); ev: per-stage timing events or NULL;
// fork: the side stream for EXACT blocks, or NULL to run everything on `st`.
int block_route_launch(hipStream_t st, const Workspace &ws, uint32_t tokens, const s14_router *router,
                       const uint64_t *expert_pages_dev, const uint8_t *shared_page, int shared_format,
                       const float *x, float *y, uint16_t *ids_out, float *weights_out, int mode,
                       const KernelEvents *ev, const BlockFork *fork);
// Status bits the last launches left in ws (synchronises the device and
// clears them): S14_OK, or the error they stand for.
int read_launch_status(const Workspace &ws, int device);

// The device a context was created on.
int ctx_device(const s14_ctx *ctx);

// Records `msg` as this thread's last error and returns `code`.
int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

struct KeyHash {
  size_t operator()(const s14_expert_key &k) const noexcept {
    uint64_t v = (uint64_t(k.layer) << 40) ^ (uint64_t(k.kind) << 32) ^ uint64_t(k.slot);
    v ^= v >> 33;
    v *= 0xff51afd7ed558ccdULL;
    v ^= v >> 33;
    return size_t(v);
  }
};
struct KeyEq {
  bool operator()(const s14_expert_key &a, const s14_expert_key &b) const noexcept {
    return a.layer == b.layer && a.kind == b.kind && a.slot == b.slot;
  }
};
inline bool key_eq(const s14_expert_key &a, const s14_expert_key &b) { return KeyEq()(a, b); }

}  // namespace s14

// Slot lifecycle of vram_pool.rs:23-28: Empty, Loading(key), Ready(key).
enum class SlotState : uint8_t { Empty, Loading, Ready };

struct s14_pool {
  int device = -1;          // device of the arena; -1 for a host-only bookkeeping pool
  uint8_t *base = nullptr;  // device arena (one allocation), NULL if host-only
  uint64_t slot_bytes = 0;
  uint32_t n_slots = 0;
  std::vector<SlotState> states;
  std::vector<s14_expert_key> state_keys;  // key of Loading/Ready slots
  std::vector<uint64_t> last_access;
  std::vector<uint32_t> pin_count;
  std::vector<uint64_t> generations;
  std::unordered_map<s14_expert_key, uint32_t, s14::KeyHash, s14::KeyEq> index;
  uint64_t clock = 0;
  uint32_t n_loaded = 0;
};

namespace s14 {
// The pool's device arena, allocated on ctx's device (implemented in
// s14_api.cpp).  The pool keeps the device id, not the context: it may
// outlive the context that created it.
int pool_alloc_arena(s14_ctx *ctx, uint64_t bytes, uint8_t **out, int *device);
void pool_free_arena(int device, uint8_t *base);
}  // namespace s14
