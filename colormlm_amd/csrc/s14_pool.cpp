// Host-side contracts of the S14 path: shape/byte validation, quantised-code
// validation, the fenced VRAM page pool and the two-pool route page batches.
//
// Restates, with the same state machine and error cases:
//   scheduler/ssd_inference/src/s14_vulkan.rs:39-156   S14MatvecShape, validate_*
//   scheduler/ssd_inference/src/vram_pool.rs:62-405    VramPool
//   scheduler/ssd_inference/src/s14_vulkan.rs:500-819  PageState, rollback,
//                                                      S14VulkanMoePages
//   scheduler/s14_runner/src/runner.rs:128-180         RouteDecision::validate_for
// The device arena is one hipMalloc (s14_api.cpp); everything here is plain
// bookkeeping, so a pool created without a context runs on any host.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <limits>
#include <memory>
#include <unordered_set>

#include "s14_internal.hpp"

namespace s14 {

static thread_local std::string g_last_error;

int fail(int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

void clear_error() { g_last_error.clear(); }

}  // namespace s14

using s14::fail;

extern "C" const char *s14_last_error(void) { return s14::g_last_error.c_str(); }
extern "C" int s14_abi_version(void) { return S14_ABI_VERSION; }

// ---------------------------------------------------------------------------
// Shape / byte contract (s14_vulkan.rs:39-140)
// ---------------------------------------------------------------------------

static constexpr uint32_t kFp4Group = 32;
static constexpr uint32_t kFp8Tile = 128;

static uint64_t div_ceil(uint64_t a, uint64_t b) { return (a + b - 1) / b; }

extern "C" int s14_shape_validate_mxfp4(s14_shape shape, s14_shape_bytes *out) {
  if (shape.n == 0 || shape.k == 0) return fail(S14_ERR_SHAPE, "S14 matvec requires non-zero N and K");
  if (shape.k % kFp8Tile != 0)
    return fail(S14_ERR_SHAPE, "S14 MXFP4 K=%u must be a multiple of 128", shape.k);
  // k % 128 == 0 implies the even-K (:86-88) and group-of-32 (:94-99) checks.
  if (out) {
    out->input_bytes = uint64_t(shape.k) * 4;
    out->output_bytes = uint64_t(shape.n) * 4;
    out->weight_bytes = uint64_t(shape.n) * shape.k / 2;
    out->scale_bytes = uint64_t(shape.n) * (shape.k / kFp4Group);
  }
  return S14_OK;
}

extern "C" int s14_shape_validate_fp8(s14_shape shape, s14_shape_bytes *out) {
  if (shape.n == 0 || shape.k == 0) return fail(S14_ERR_SHAPE, "S14 matvec requires non-zero N and K");
  if (out) {
    out->input_bytes = uint64_t(shape.k) * 4;
    out->output_bytes = uint64_t(shape.n) * 4;
    out->weight_bytes = uint64_t(shape.n) * shape.k;
    out->scale_bytes = div_ceil(shape.n, kFp8Tile) * div_ceil(shape.k, kFp8Tile);
  }
  return S14_OK;
}

extern "C" int s14_validate_ue8m0_codes(const uint8_t *codes, size_t n, size_t *bad_index) {
  if (!codes && n) return fail(S14_ERR_INVALID, "NULL UE8M0 code buffer");
  for (size_t i = 0; i < n; ++i) {
    if (codes[i] == 0xff) {
      if (bad_index) *bad_index = i;
      return fail(S14_ERR_NAN_CODE, "UE8M0 scale contains 0xff NaN at byte %zu", i);
    }
  }
  return S14_OK;
}

extern "C" int s14_validate_e4m3fn_codes(const uint8_t *codes, size_t n, size_t *bad_index) {
  if (!codes && n) return fail(S14_ERR_INVALID, "NULL E4M3FN code buffer");
  for (size_t i = 0; i < n; ++i) {
    if (codes[i] == 0x7f || codes[i] == 0xff) {
      if (bad_index) *bad_index = i;
      return fail(S14_ERR_NAN_CODE, "E4M3FN weight contains NaN code at byte %zu", i);
    }
  }
  return S14_OK;
}

extern "C" int s14_page_layout_get(int page_format, uint32_t hidden, uint32_t inter,
                                   s14_page_layout *out) {
  if (!out) return fail(S14_ERR_INVALID, "NULL layout output");
  if (hidden == 0 || inter == 0) return fail(S14_ERR_SHAPE, "page shape must be non-zero");
  uint64_t up_w, up_s, dn_w, dn_s;
  if (page_format == S14_PAGE_MXFP4) {
    if (hidden % kFp8Tile || inter % kFp8Tile)
      return fail(S14_ERR_SHAPE, "MXFP4 page needs hidden and inter multiples of 128");
    up_w = uint64_t(inter) * hidden / 2;
    up_s = uint64_t(inter) * hidden / kFp4Group;
    dn_w = uint64_t(hidden) * inter / 2;
    dn_s = uint64_t(hidden) * inter / kFp4Group;
  } else if (page_format == S14_PAGE_FP8) {
    up_w = uint64_t(inter) * hidden;
    up_s = div_ceil(inter, kFp8Tile) * div_ceil(hidden, kFp8Tile);
    dn_w = uint64_t(hidden) * inter;
    dn_s = div_ceil(hidden, kFp8Tile) * div_ceil(inter, kFp8Tile);
  } else {
    return fail(S14_ERR_INVALID, "unknown page format %d", page_format);
  }
  out->w1 = 0;
  out->s1 = up_w;
  out->w3 = out->s1 + up_s;
  out->s3 = out->w3 + up_w;
  out->w2 = out->s3 + up_s;
  out->s2 = out->w2 + dn_w;
  out->total_bytes = out->s2 + dn_s;
  return S14_OK;
}

// ---------------------------------------------------------------------------
// VramPool (vram_pool.rs:62-405)
// ---------------------------------------------------------------------------

static inline uint64_t sat_add1(uint64_t v) {
  return v == std::numeric_limits<uint64_t>::max() ? v : v + 1;
}

static const char *state_name(SlotState s) {
  switch (s) {
    case SlotState::Empty: return "Empty";
    case SlotState::Loading: return "Loading";
    default: return "Ready";
  }
}

static bool state_is(const s14_pool *p, uint32_t slot, SlotState st, const s14_expert_key &key) {
  return p->states[slot] == st && s14::key_eq(p->state_keys[slot], key);
}

extern "C" int s14_pool_create(s14_ctx *ctx, uint32_t n_slots, uint64_t slot_bytes, s14_pool **out) {
  if (!out) return fail(S14_ERR_INVALID, "NULL pool output");
  *out = nullptr;
  if (n_slots == 0) return fail(S14_ERR_INVALID, "VRAM pool must contain at least one slot");
  if (slot_bytes == 0) return fail(S14_ERR_INVALID, "VRAM slot size must be greater than zero");
  if (slot_bytes > std::numeric_limits<uint64_t>::max() / n_slots)
    return fail(S14_ERR_INVALID, "VRAM pool size overflow");
  std::unique_ptr<s14_pool> p(new s14_pool());
  p->device = -1;
  p->slot_bytes = slot_bytes;
  p->n_slots = n_slots;
  p->states.assign(n_slots, SlotState::Empty);
  p->state_keys.assign(n_slots, s14_expert_key{0, 0, 0});
  p->last_access.assign(n_slots, 0);
  p->pin_count.assign(n_slots, 0);
  p->generations.assign(n_slots, 0);
  p->index.reserve(n_slots);
  if (ctx) {
    int rc = s14::pool_alloc_arena(ctx, uint64_t(n_slots) * slot_bytes, &p->base, &p->device);
    if (rc != S14_OK) return rc;
  }
  *out = p.release();
  return S14_OK;
}

extern "C" void s14_pool_destroy(s14_pool *pool) {
  if (!pool) return;
  if (pool->base) s14::pool_free_arena(pool->device, pool->base);
  delete pool;
}

extern "C" uint32_t s14_pool_capacity(const s14_pool *p) { return p ? p->n_slots : 0; }
extern "C" uint64_t s14_pool_slot_bytes(const s14_pool *p) { return p ? p->slot_bytes : 0; }
extern "C" uint32_t s14_pool_n_loaded(const s14_pool *p) { return p ? p->n_loaded : 0; }
extern "C" uint64_t s14_pool_total_bytes(const s14_pool *p) {
  return p ? uint64_t(p->n_slots) * p->slot_bytes : 0;
}
extern "C" uint64_t s14_pool_slot_offset(const s14_pool *p, uint32_t slot) {
  return p ? uint64_t(slot) * p->slot_bytes : 0;
}
extern "C" void *s14_pool_slot_ptr(const s14_pool *p, uint32_t slot) {
  if (!p || !p->base || slot >= p->n_slots) return nullptr;
  return p->base + uint64_t(slot) * p->slot_bytes;
}

extern "C" int s14_pool_lookup(s14_pool *p, s14_expert_key key, uint32_t *slot) {
  if (!p) return 0;
  auto it = p->index.find(key);
  if (it == p->index.end()) return 0;
  p->clock = sat_add1(p->clock);
  p->last_access[it->second] = p->clock;
  if (slot) *slot = it->second;
  return 1;
}

extern "C" int s14_pool_lookup_and_pin(s14_pool *p, s14_expert_key key, int *found,
                                       s14_slot_binding *lease) {
  if (!p || !found) return fail(S14_ERR_INVALID, "NULL pool argument");
  *found = 0;
  auto it = p->index.find(key);
  if (it == p->index.end()) return S14_OK;
  uint32_t slot = it->second;
  if (!state_is(p, slot, SlotState::Ready, key))
    return fail(S14_ERR_STALE, "VRAM index for (%u,%u,%u) points at non-ready slot %u", key.layer,
                key.kind, key.slot, slot);
  if (p->pin_count[slot] == std::numeric_limits<uint32_t>::max())
    return fail(S14_ERR_INVALID, "VRAM slot %u pin count overflow", slot);
  p->pin_count[slot] += 1;
  p->clock = sat_add1(p->clock);
  p->last_access[slot] = p->clock;
  *found = 1;
  if (lease) *lease = s14_slot_binding{key, slot, p->generations[slot]};
  return S14_OK;
}

extern "C" int s14_pool_reserve_loading_generation(s14_pool *p, s14_expert_key key,
                                                   s14_loading_reservation *out) {
  if (!p || !out) return fail(S14_ERR_INVALID, "NULL pool argument");
  if (p->index.count(key))
    return fail(S14_ERR_INVALID, "expert (%u,%u,%u) is already ready", key.layer, key.kind, key.slot);
  for (uint32_t i = 0; i < p->n_slots; ++i)
    if (state_is(p, i, SlotState::Loading, key))
      return fail(S14_ERR_INVALID, "expert (%u,%u,%u) is already loading", key.layer, key.kind,
                  key.slot);
  // First Empty slot; otherwise the least recently used unpinned Ready slot
  // (the first one on ties, as Iterator::min_by_key).
  int64_t chosen = -1;
  for (uint32_t i = 0; i < p->n_slots; ++i)
    if (p->states[i] == SlotState::Empty) {
      chosen = i;
      break;
    }
  if (chosen < 0) {
    uint64_t best = 0;
    for (uint32_t i = 0; i < p->n_slots; ++i) {
      if (p->states[i] == SlotState::Ready && p->pin_count[i] == 0) {
        if (chosen < 0 || p->last_access[i] < best) {
          chosen = i;
          best = p->last_access[i];
        }
      }
    }
    if (chosen < 0)
      return fail(S14_ERR_POOL_FULL, "all %u VRAM slots are Loading or pinned Ready", p->n_slots);
  }
  const uint32_t slot = uint32_t(chosen);
  if (p->generations[slot] == std::numeric_limits<uint64_t>::max())
    return fail(S14_ERR_INVALID, "VRAM slot %u generation overflow", slot);
  out->has_evicted = 0;
  out->evicted = s14_expert_key{0, 0, 0};
  if (p->states[slot] == SlotState::Ready) {
    out->has_evicted = 1;
    out->evicted = p->state_keys[slot];
    p->index.erase(p->state_keys[slot]);
  } else {
    p->n_loaded += 1;
  }
  const uint64_t generation = p->generations[slot] + 1;
  p->generations[slot] = generation;
  p->pin_count[slot] = 0;
  p->states[slot] = SlotState::Loading;
  p->state_keys[slot] = key;
  out->key = key;
  out->slot = slot;
  out->generation = generation;
  return S14_OK;
}

extern "C" int s14_pool_reserve_loading(s14_pool *p, s14_expert_key key, uint32_t *slot,
                                        int *has_evicted, s14_expert_key *evicted) {
  s14_loading_reservation r;
  int rc = s14_pool_reserve_loading_generation(p, key, &r);
  if (rc != S14_OK) return rc;
  if (slot) *slot = r.slot;
  if (has_evicted) *has_evicted = r.has_evicted;
  if (evicted) *evicted = r.evicted;
  return S14_OK;
}

extern "C" int s14_pool_validate_publish_batch(const s14_pool *p, const s14_loading_reservation *rs,
                                               size_t n) {
  if (!p) return fail(S14_ERR_INVALID, "NULL pool");
  if (n == 0 || !rs) return fail(S14_ERR_INVALID, "cannot publish an empty VRAM batch");
  std::unordered_set<uint32_t> slots;
  std::unordered_set<s14_expert_key, s14::KeyHash, s14::KeyEq> keys;
  for (size_t i = 0; i < n; ++i) {
    const s14_loading_reservation &r = rs[i];
    if (!slots.insert(r.slot).second || !keys.insert(r.key).second)
      return fail(S14_ERR_INVALID, "VRAM publish batch contains a duplicate slot or key");
    if (r.slot >= p->n_slots) return fail(S14_ERR_INVALID, "invalid VRAM slot %u", r.slot);
    const uint64_t cur = p->generations[r.slot];
    if (!state_is(p, r.slot, SlotState::Loading, r.key) || cur != r.generation)
      return fail(S14_ERR_STALE,
                  "stale VRAM generation for (%u,%u,%u): slot=%u generation=%llu "
                  "current_state=%s current_generation=%llu",
                  r.key.layer, r.key.kind, r.key.slot, r.slot, (unsigned long long)r.generation,
                  state_name(p->states[r.slot]), (unsigned long long)cur);
    if (p->pin_count[r.slot] != 0)
      return fail(S14_ERR_INVALID, "Loading slot %u unexpectedly has compute pins", r.slot);
    if (p->index.count(r.key))
      return fail(S14_ERR_INVALID, "cannot publish (%u,%u,%u): key is already visible",
                  r.key.layer, r.key.kind, r.key.slot);
  }
  return S14_OK;
}

// publish_prevalidated_batch_and_pin (vram_pool.rs:318-339).
static void publish_prevalidated(s14_pool *p, const s14_loading_reservation *rs, size_t n,
                                 s14_slot_binding *leases_out) {
  for (size_t i = 0; i < n; ++i) {
    const s14_loading_reservation &r = rs[i];
    p->states[r.slot] = SlotState::Ready;
    p->state_keys[r.slot] = r.key;
    p->index[r.key] = r.slot;
    p->pin_count[r.slot] = 1;
    p->clock = sat_add1(p->clock);
    p->last_access[r.slot] = p->clock;
    if (leases_out) leases_out[i] = s14_slot_binding{r.key, r.slot, r.generation};
  }
}

extern "C" int s14_pool_publish_batch_and_pin(s14_pool *p, const s14_loading_reservation *rs,
                                              size_t n, s14_slot_binding *leases_out) {
  int rc = s14_pool_validate_publish_batch(p, rs, n);
  if (rc != S14_OK) return rc;
  publish_prevalidated(p, rs, n, leases_out);
  return S14_OK;
}

extern "C" int s14_pool_validate_binding(const s14_pool *p, s14_slot_binding b) {
  if (!p) return fail(S14_ERR_INVALID, "NULL pool");
  if (b.slot >= p->n_slots) return fail(S14_ERR_INVALID, "invalid VRAM slot %u", b.slot);
  if (!state_is(p, b.slot, SlotState::Ready, b.key) || p->generations[b.slot] != b.generation ||
      p->pin_count[b.slot] == 0)
    return fail(S14_ERR_STALE, "stale or unpinned VRAM binding for (%u,%u,%u): slot=%u generation=%llu",
                b.key.layer, b.key.kind, b.key.slot, b.slot, (unsigned long long)b.generation);
  return S14_OK;
}

extern "C" int s14_pool_release_after_compute_fence(s14_pool *p, s14_slot_binding lease) {
  int rc = s14_pool_validate_binding(p, lease);
  if (rc != S14_OK) return rc;
  p->pin_count[lease.slot] -= 1;
  return S14_OK;
}

extern "C" int s14_pool_mark_ready(s14_pool *p, uint32_t slot, s14_expert_key key) {
  if (!p) return fail(S14_ERR_INVALID, "NULL pool");
  if (slot >= p->n_slots) return fail(S14_ERR_INVALID, "invalid VRAM slot %u", slot);
  if (!state_is(p, slot, SlotState::Loading, key))
    return fail(S14_ERR_STALE, "slot %u cannot publish (%u,%u,%u): current state is %s", slot,
                key.layer, key.kind, key.slot, state_name(p->states[slot]));
  s14_loading_reservation r{key, slot, p->generations[slot], 0, {0, 0, 0}};
  s14_slot_binding lease;
  int rc = s14_pool_publish_batch_and_pin(p, &r, 1, &lease);
  if (rc != S14_OK) return rc;
  return s14_pool_release_after_compute_fence(p, lease);
}

extern "C" void s14_pool_cancel_loading(s14_pool *p, uint32_t slot, s14_expert_key key) {
  if (!p || slot >= p->n_slots) return;
  if (state_is(p, slot, SlotState::Loading, key)) {
    p->states[slot] = SlotState::Empty;
    p->pin_count[slot] = 0;
    if (p->n_loaded) p->n_loaded -= 1;
  }
}

extern "C" int s14_pool_cancel_reservation(s14_pool *p, s14_loading_reservation r) {
  if (!p) return fail(S14_ERR_INVALID, "NULL pool");
  if (r.slot >= p->n_slots) return fail(S14_ERR_INVALID, "invalid VRAM slot %u", r.slot);
  if (!state_is(p, r.slot, SlotState::Loading, r.key) || p->generations[r.slot] != r.generation)
    return fail(S14_ERR_STALE, "stale VRAM cancellation for (%u,%u,%u): slot=%u generation=%llu",
                r.key.layer, r.key.kind, r.key.slot, r.slot, (unsigned long long)r.generation);
  p->states[r.slot] = SlotState::Empty;
  p->pin_count[r.slot] = 0;
  if (p->n_loaded) p->n_loaded -= 1;
  return S14_OK;
}

// ---------------------------------------------------------------------------
// RouteDecision::validate_for (runner.rs:128-180; contract.rs:4-12, 77-90)
// ---------------------------------------------------------------------------

static const uint8_t kSelectedLayers[14] = {0, 1, 2, 6, 7, 14, 15, 22, 23, 30, 31, 40, 41, 42};
static constexpr uint8_t kNLayers = 43;
static constexpr uint32_t kExpertsPerToken = 6;
static constexpr uint32_t kNRoutedExperts = 256;

extern "C" int s14_route_validate_for(const s14_route_decision *route, int profile,
                                      float weight_sum) {
  if (!route) return fail(S14_ERR_INVALID, "NULL route");
  bool in_profile = false;
  if (profile == S14_PROFILE_S14_TOP6) {
    for (uint8_t l : kSelectedLayers) in_profile |= (l == route->layer);
  } else if (profile == S14_PROFILE_FULL_DEPTH43_TOP6) {
    in_profile = route->layer < kNLayers;
  } else {
    return fail(S14_ERR_INVALID, "unknown graph profile %d", profile);
  }
  if (!in_profile)
    return fail(S14_ERR_ROUTE, "route layer %u is not in the registered profile %d", route->layer,
                profile);
  if (route->n != kExpertsPerToken)
    return fail(S14_ERR_ROUTE, "profile %d requires top-%u, got ids=%u weights=%u", profile,
                kExpertsPerToken, route->n, route->n);
  if (route->layer >= kNLayers)
    return fail(S14_ERR_ROUTE, "layer %u outside the official 0..42", route->layer);
  const int expected_kind = route->layer < 3 ? S14_ROUTER_HASH : S14_ROUTER_SCORE;
  if (route->kind != expected_kind)
    return fail(S14_ERR_ROUTE, "L%u router kind must be %s", route->layer,
                expected_kind == S14_ROUTER_HASH ? "Hash" : "Score");
  for (uint32_t i = 0; i < route->n; ++i) {
    const uint16_t e = route->expert_ids[i];
    const float w = route->weights[i];
    if (e >= kNRoutedExperts) return fail(S14_ERR_ROUTE, "route[%u] expert %u out of range", i, e);
    if (!std::isfinite(w) || w < 0.0f)
      return fail(S14_ERR_ROUTE, "route[%u] weight is not finite and non-negative", i);
    for (uint32_t j = 0; j < i; ++j)
      if (route->expert_ids[j] == e) return fail(S14_ERR_ROUTE, "route expert %u repeated", e);
  }
  float sum = -0.0f;
  for (uint32_t i = 0; i < route->n; ++i) sum += route->weights[i];
  if (std::fabs(sum - weight_sum) > 1e-4f)
    return fail(S14_ERR_ROUTE, "normalized weights*route_scale must sum to %g, got %g",
                (double)weight_sum, (double)sum);
  return S14_OK;
}

// ---------------------------------------------------------------------------
// Route page batches (s14_vulkan.rs:500-819)
// ---------------------------------------------------------------------------

namespace {
// PageState (s14_vulkan.rs:500-504).
struct PageState {
  bool loading = false;
  s14_loading_reservation reservation{};
  s14_slot_binding lease{};
};

int acquire_page(s14_pool *pool, s14_expert_key key, PageState *out) {
  int found = 0;
  int rc = s14_pool_lookup_and_pin(pool, key, &found, &out->lease);
  if (rc != S14_OK) return rc;
  if (found) {
    out->loading = false;
    return S14_OK;
  }
  out->loading = true;
  return s14_pool_reserve_loading_generation(pool, key, &out->reservation);
}

std::vector<s14_loading_reservation> loading_reservations(const std::vector<PageState> &pages) {
  std::vector<s14_loading_reservation> out;
  for (const auto &p : pages)
    if (p.loading) out.push_back(p.reservation);
  return out;
}

int validate_page_publish(const s14_pool *pool, const std::vector<PageState> &pages) {
  auto rs = loading_reservations(pages);
  if (rs.empty()) return S14_OK;
  return s14_pool_validate_publish_batch(pool, rs.data(), rs.size());
}

std::vector<s14_slot_binding> publish_prevalidated_pages(s14_pool *pool,
                                                         const std::vector<PageState> &pages) {
  auto rs = loading_reservations(pages);
  std::vector<s14_slot_binding> published(rs.size());
  if (!rs.empty()) publish_prevalidated(pool, rs.data(), rs.size(), published.data());
  std::vector<s14_slot_binding> out;
  size_t next = 0;
  for (const auto &p : pages) out.push_back(p.loading ? published[next++] : p.lease);
  return out;
}

// rollback_pages (s14_vulkan.rs:552-567): release cached pins, cancel
// reservations, report the first error but keep going.
int rollback_pages(s14_pool *pool, const std::vector<PageState> &pages) {
  int first = S14_OK;
  std::string first_msg;
  for (const auto &p : pages) {
    int rc = p.loading ? s14_pool_cancel_reservation(pool, p.reservation)
                       : s14_pool_release_after_compute_fence(pool, p.lease);
    if (rc != S14_OK && first == S14_OK) {
      first = rc;
      first_msg = s14_last_error();
    }
  }
  if (first != S14_OK) fail(first, "%s", first_msg.c_str());
  return first;
}
}  // namespace

struct s14_moe_pages {
  s14_pool *routed = nullptr;
  s14_pool *shared = nullptr;
  int profile = 0;
  float weight_sum = 1.5f;
};

struct s14_route_load_batch {
  uint8_t layer = 0;
  std::vector<uint16_t> expert_ids;
  std::vector<float> route_weights;
  std::vector<PageState> routed_pages;
  PageState shared_page;
};

struct s14_moe_lease_batch {
  uint8_t layer = 0;
  std::vector<uint16_t> expert_ids;
  std::vector<float> route_weights;
  std::vector<s14_slot_binding> routed;
  s14_slot_binding shared{};
};

extern "C" int s14_moe_pages_create(s14_pool *routed, s14_pool *shared, int profile,
                                    int shared_format, float weight_sum, s14_moe_pages **out) {
  if (!routed || !shared || !out) return fail(S14_ERR_INVALID, "NULL page-set argument");
  *out = nullptr;
  if (routed->slot_bytes < S14_EXPERT_PAGE_BYTES)
    return fail(S14_ERR_CAPACITY, "S14 routed slot is %llu B, requires at least %llu B",
                (unsigned long long)routed->slot_bytes, (unsigned long long)S14_EXPERT_PAGE_BYTES);
  const uint64_t need_shared =
      shared_format == S14_PAGE_FP8 ? S14_SHARED_EXPERT_PAGE_BYTES : S14_EXPERT_PAGE_BYTES;
  if (shared_format != S14_PAGE_FP8 && shared_format != S14_PAGE_MXFP4)
    return fail(S14_ERR_INVALID, "unknown shared page format %d", shared_format);
  if (shared->slot_bytes < need_shared)
    return fail(S14_ERR_CAPACITY, "S14 shared slot is %llu B, requires at least %llu B",
                (unsigned long long)shared->slot_bytes, (unsigned long long)need_shared);
  auto *p = new s14_moe_pages();
  p->routed = routed;
  p->shared = shared;
  p->profile = profile;
  p->weight_sum = weight_sum;
  *out = p;
  return S14_OK;
}

extern "C" void s14_moe_pages_destroy(s14_moe_pages *pages) { delete pages; }

extern "C" int s14_moe_pages_begin_after_official_route(s14_moe_pages *pages,
                                                        const s14_route_decision *route,
                                                        s14_route_load_batch **out) {
  if (!pages || !route || !out) return fail(S14_ERR_INVALID, "NULL argument");
  *out = nullptr;
  int rc = s14_route_validate_for(route, pages->profile, pages->weight_sum);
  if (rc != S14_OK) return rc;
  std::unique_ptr<s14_route_load_batch> b(new s14_route_load_batch());
  for (uint32_t i = 0; i < route->n; ++i) {
    s14_expert_key key{route->layer, S14_ROUTED_EXPERT_KIND, route->expert_ids[i]};
    PageState page;
    rc = acquire_page(pages->routed, key, &page);
    if (rc != S14_OK) {
      std::string msg = s14_last_error();
      rollback_pages(pages->routed, b->routed_pages);
      return fail(rc, "%s", msg.c_str());
    }
    b->routed_pages.push_back(page);
  }
  s14_expert_key shared_key{route->layer, S14_SHARED_EXPERT_KIND, 0};
  rc = acquire_page(pages->shared, shared_key, &b->shared_page);
  if (rc != S14_OK) {
    std::string msg = s14_last_error();
    rollback_pages(pages->routed, b->routed_pages);
    return fail(rc, "%s", msg.c_str());
  }
  b->layer = route->layer;
  b->expert_ids.assign(route->expert_ids, route->expert_ids + route->n);
  b->route_weights.assign(route->weights, route->weights + route->n);
  *out = b.release();
  return S14_OK;
}

extern "C" uint32_t s14_route_load_batch_size(const s14_route_load_batch *b) {
  return b ? uint32_t(b->routed_pages.size() + 1) : 0;
}

extern "C" int s14_route_load_batch_page(const s14_route_load_batch *b, uint32_t i, int *loading,
                                         s14_loading_reservation *reservation,
                                         s14_slot_binding *cached) {
  if (!b || !loading) return fail(S14_ERR_INVALID, "NULL argument");
  if (i > b->routed_pages.size()) return fail(S14_ERR_INVALID, "batch page %u out of range", i);
  const PageState &p = i < b->routed_pages.size() ? b->routed_pages[i] : b->shared_page;
  *loading = p.loading ? 1 : 0;
  if (p.loading && reservation) *reservation = p.reservation;
  if (!p.loading && cached) *cached = p.lease;
  return S14_OK;
}

extern "C" int s14_route_load_batch_shared_reservation(const s14_route_load_batch *b,
                                                       s14_loading_reservation *out) {
  if (!b || !out) return fail(S14_ERR_INVALID, "NULL argument");
  if (!b->shared_page.loading) return fail(S14_ERR_INVALID, "shared page is not Loading");
  *out = b->shared_page.reservation;
  return S14_OK;
}

extern "C" int s14_moe_pages_publish_after_transfer_fence(s14_moe_pages *pages,
                                                          s14_route_load_batch *batch,
                                                          s14_moe_lease_batch **out) {
  if (!pages || !batch || !out) return fail(S14_ERR_INVALID, "NULL argument");
  std::unique_ptr<s14_route_load_batch> b(batch);
  *out = nullptr;
  std::vector<PageState> shared_pages{b->shared_page};
  int rc = validate_page_publish(pages->routed, b->routed_pages);
  if (rc == S14_OK) rc = validate_page_publish(pages->shared, shared_pages);
  if (rc != S14_OK) {
    std::string msg = s14_last_error();
    rollback_pages(pages->routed, b->routed_pages);
    rollback_pages(pages->shared, shared_pages);
    return fail(rc, "%s", msg.c_str());
  }
  std::unique_ptr<s14_moe_lease_batch> l(new s14_moe_lease_batch());
  l->routed = publish_prevalidated_pages(pages->routed, b->routed_pages);
  l->shared = publish_prevalidated_pages(pages->shared, shared_pages)[0];
  l->layer = b->layer;
  l->expert_ids = b->expert_ids;
  l->route_weights = b->route_weights;
  *out = l.release();
  return S14_OK;
}

extern "C" int s14_moe_lease_batch_bindings(const s14_moe_lease_batch *lease,
                                            s14_slot_binding *routed, uint32_t n_routed,
                                            s14_slot_binding *shared) {
  if (!lease) return fail(S14_ERR_INVALID, "NULL lease batch");
  if (routed) {
    if (n_routed < lease->routed.size())
      return fail(S14_ERR_CAPACITY, "binding output holds %u, batch has %zu", n_routed,
                  lease->routed.size());
    for (size_t i = 0; i < lease->routed.size(); ++i) routed[i] = lease->routed[i];
  }
  if (shared) *shared = lease->shared;
  return S14_OK;
}

extern "C" int s14_moe_pages_release_after_compute_fence(s14_moe_pages *pages,
                                                         s14_moe_lease_batch *lease) {
  if (!pages || !lease) return fail(S14_ERR_INVALID, "NULL argument");
  for (const auto &b : lease->routed) {
    int rc = s14_pool_validate_binding(pages->routed, b);
    if (rc != S14_OK) return rc;
  }
  int rc = s14_pool_validate_binding(pages->shared, lease->shared);
  if (rc != S14_OK) return rc;
  for (const auto &b : lease->routed) {
    rc = s14_pool_release_after_compute_fence(pages->routed, b);
    if (rc != S14_OK) return rc;
  }
  rc = s14_pool_release_after_compute_fence(pages->shared, lease->shared);
  if (rc != S14_OK) return rc;
  delete lease;
  return S14_OK;
}

extern "C" int s14_moe_pages_cancel(s14_moe_pages *pages, s14_route_load_batch *batch) {
  if (!pages || !batch) return fail(S14_ERR_INVALID, "NULL argument");
  std::unique_ptr<s14_route_load_batch> b(batch);
  int routed_rc = rollback_pages(pages->routed, b->routed_pages);
  std::string routed_msg = routed_rc != S14_OK ? s14_last_error() : "";
  int shared_rc = rollback_pages(pages->shared, std::vector<PageState>{b->shared_page});
  if (routed_rc != S14_OK) return fail(routed_rc, "%s", routed_msg.c_str());
  return shared_rc;
}
