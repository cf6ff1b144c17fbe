// Expert page uploader: the transfer side of ExpertLoader
// (scheduler/ssd_inference/src/expert_loader.rs:1-474) on HIP.
//
// A ring of `pipeline_depth` pinned host staging slots (hipHostMalloc, so the
// copy engine reads them without a driver bounce) feeds hipMemcpyAsync
// transfers into the VRAM pool's arena on the context's copy stream, which
// runs beside the compute stream.  Each ring slot has one hipEvent as its
// transfer fence.  A page becomes visible through the pool (mark_ready) only
// once its fence has completed; until then the pool holds its slot as
// Loading, so lookups miss and eviction skips it.  Reusing a ring slot first
// completes its previous transfer, so a staging slot is never rewritten while
// the copy engine may still read it.  batch_enqueue deduplicates keys and
// issues them in waves no deeper than the ring (expert_loader.rs:293-298:
// the reference's fix for staging aliasing); the last wave stays in flight
// for the caller's wait_all.
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cstring>
#include <new>
#include <thread>
#include <unordered_map>
#include <vector>

#include "s14_internal.hpp"

using s14::fail;

namespace {

int hip_fail(hipError_t e, const char *what) { return fail(S14_ERR_HIP, "%s: %s", what, hipGetErrorString(e)); }

// Source of one page's bytes: pre-read host memory (enqueue_from_buf) or the
// caller's reader (enqueue with ExpertReader::read_into).
struct PageSource {
  const void *data;
  s14_read_fn read;
  void *user;
};

// Host copy into pinned staging.  One thread moves ~10 GB/s here, a fifth of
// a PCIe Gen5 x16 link, so large pages are split over a few threads.
void staging_copy(uint8_t *dst, const uint8_t *src, uint64_t bytes) {
  constexpr uint64_t kSplit = 4ull << 20;  // below this one thread is cheaper than spawning
  const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
  const unsigned n = unsigned(std::min<uint64_t>(std::min(8u, hw), bytes / kSplit));
  if (n <= 1) {
    std::memcpy(dst, src, bytes);
    return;
  }
  const uint64_t part = (bytes / n + 63) & ~uint64_t(63);
  std::vector<std::thread> threads;
  threads.reserve(n - 1);
  for (unsigned i = 1; i < n; ++i) {
    const uint64_t off = std::min<uint64_t>(bytes, uint64_t(i) * part);
    const uint64_t len = std::min<uint64_t>(bytes - off, part);
    threads.emplace_back([=] { std::memcpy(dst + off, src + off, len); });
  }
  std::memcpy(dst, src, std::min(bytes, part));
  for (auto &t : threads) t.join();
}

}  // namespace

struct s14_loader {
  int device = 0;
  hipStream_t stream = nullptr;  // the context's copy stream
  uint32_t depth = 0;
  uint64_t staging_bytes = 0;
  std::vector<uint8_t *> staging;  // pinned host slots
  std::vector<hipEvent_t> fences;  // transfer fence of each slot
  struct Pending {
    bool live = false;
    s14_expert_key key{};
    uint32_t vram_slot = 0;
  };
  std::vector<Pending> pending;
  uint32_t next = 0;
  uint64_t stat_loads = 0, stat_bytes = 0;
};

namespace {

// complete_pipeline_slot (expert_loader.rs:124-140): wait the slot's fence,
// then publish its page.
int complete_slot(s14_loader *l, s14_pool *pool, uint32_t pip) {
  s14_loader::Pending &p = l->pending[pip];
  if (!p.live) return S14_OK;
  const hipError_t e = hipEventSynchronize(l->fences[pip]);
  if (e != hipSuccess) return hip_fail(e, "hipEventSynchronize(transfer fence)");
  p.live = false;
  return s14_pool_mark_ready(pool, p.vram_slot, p.key);
}

// complete_pending_key (expert_loader.rs:142-157).
int complete_pending_key(s14_loader *l, s14_pool *pool, s14_expert_key key, bool *found, uint32_t *slot) {
  *found = false;
  for (uint32_t pip = 0; pip < l->depth; ++pip) {
    if (!l->pending[pip].live || !s14::key_eq(l->pending[pip].key, key)) continue;
    if (int rc = complete_slot(l, pool, pip)) return rc;
    *found = s14_pool_lookup(pool, key, slot) == 1;
    return S14_OK;
  }
  return S14_OK;
}

int check_pool(const s14_loader *l, const s14_pool *pool) {
  if (!l || !pool) return fail(S14_ERR_INVALID, "NULL loader or pool");
  if (!pool->base) return fail(S14_ERR_INVALID, "pool has no device arena");
  if (pool->device != l->device)
    return fail(S14_ERR_INVALID, "pool is on device %d, loader on device %d", pool->device, l->device);
  return S14_OK;
}

// enqueue / enqueue_from_buf (expert_loader.rs:163-284, 362-442).
int enqueue(s14_loader *l, s14_pool *pool, s14_expert_key key, uint64_t bytes, const PageSource &src,
            uint32_t *slot_out) {
  uint32_t slot = 0;
  if (s14_pool_lookup(pool, key, &slot) == 1) {  // already loaded
    *slot_out = slot;
    return S14_OK;
  }
  bool found = false;
  if (int rc = complete_pending_key(l, pool, key, &found, &slot)) return rc;
  if (found) {
    *slot_out = slot;
    return S14_OK;
  }
  // validate_transfer_size (expert_loader.rs:106-122)
  if (bytes > l->staging_bytes)
    return fail(S14_ERR_CAPACITY, "expert page is too large for staging slot: %llu > %llu bytes",
                (unsigned long long)bytes, (unsigned long long)l->staging_bytes);
  if (bytes > pool->slot_bytes)
    return fail(S14_ERR_CAPACITY, "expert page is too large for VRAM slot: %llu > %llu bytes",
                (unsigned long long)bytes, (unsigned long long)pool->slot_bytes);
  const uint32_t pip = l->next;
  l->next = (l->next + 1) % l->depth;
  if (int rc = complete_slot(l, pool, pip)) return rc;
  // a hidden Loading slot (may evict); lookups miss it until the fence completes
  int evicted = 0;
  s14_expert_key evicted_key{};
  if (int rc = s14_pool_reserve_loading(pool, key, &slot, &evicted, &evicted_key)) return rc;
  uint8_t *stage = l->staging[pip];
  if (src.read) {
    if (src.read(src.user, key, stage, bytes) != 0) {
      s14_pool_cancel_loading(pool, slot, key);
      return fail(S14_ERR_INVALID, "reading expert (%u,%u,%u) failed", key.layer, key.kind, key.slot);
    }
  } else {
    staging_copy(stage, static_cast<const uint8_t *>(src.data), bytes);
  }
  hipError_t e = hipMemcpyAsync(pool->base + uint64_t(slot) * pool->slot_bytes, stage, bytes, hipMemcpyHostToDevice,
                                l->stream);
  if (e == hipSuccess) e = hipEventRecord(l->fences[pip], l->stream);
  if (e != hipSuccess) {
    // the copy may be queued: settle the stream before the slot can be reused
    (void)hipStreamSynchronize(l->stream);
    s14_pool_cancel_loading(pool, slot, key);
    return hip_fail(e, "transfer submit");
  }
  l->pending[pip] = {true, key, slot};
  l->stat_loads += 1;
  l->stat_bytes += bytes;
  *slot_out = slot;
  return S14_OK;
}

int wait_all(s14_loader *l, s14_pool *pool) {
  for (uint32_t pip = 0; pip < l->depth; ++pip)
    if (int rc = complete_slot(l, pool, pip)) return rc;
  return S14_OK;
}

// batch_enqueue (expert_loader.rs:299-360).
int batch_enqueue(s14_loader *l, s14_pool *pool, const s14_expert_key *keys, const uint64_t *bytes, size_t n,
                  const PageSource *sources, uint32_t *slots_out) {
  if (n == 0) return S14_OK;
  if (!keys || !bytes || !slots_out) return fail(S14_ERR_INVALID, "NULL batch argument");
  // settle earlier work so duplicate detection sees the pool's Ready index
  if (int rc = wait_all(l, pool)) return rc;
  std::unordered_map<s14_expert_key, size_t, s14::KeyHash, s14::KeyEq> distinct;
  std::vector<size_t> unique, input_to_unique(n);
  for (size_t i = 0; i < n; ++i) {
    auto it = distinct.emplace(keys[i], unique.size());
    if (it.second) unique.push_back(i);
    input_to_unique[i] = it.first->second;
  }
  if (unique.size() > pool->n_slots)
    return fail(S14_ERR_CAPACITY, "batch requests %zu distinct experts but VRAM pool has only %u slots",
                unique.size(), pool->n_slots);
  std::vector<uint32_t> unique_slots(unique.size());
  const size_t waves = (unique.size() + l->depth - 1) / l->depth;
  for (size_t w = 0; w < waves; ++w) {
    const size_t lo = w * l->depth, hi = std::min(unique.size(), lo + l->depth);
    for (size_t u = lo; u < hi; ++u) {
      const size_t i = unique[u];
      if (int rc = enqueue(l, pool, keys[i], bytes[i], sources[i], &unique_slots[u])) return rc;
    }
    // a later wave reuses the staging slots: publish and drain this one first
    if (w + 1 < waves)
      if (int rc = wait_all(l, pool)) return rc;
  }
  for (size_t i = 0; i < n; ++i) slots_out[i] = unique_slots[input_to_unique[i]];
  return S14_OK;
}

}  // namespace

extern "C" int s14_loader_create(s14_ctx *ctx, uint32_t pipeline_depth, uint64_t staging_bytes, s14_loader **out) {
  if (!out) return fail(S14_ERR_INVALID, "NULL loader output");
  *out = nullptr;
  if (!ctx) return fail(S14_ERR_INVALID, "NULL context");
  if (pipeline_depth == 0) return fail(S14_ERR_INVALID, "pipeline depth must be greater than zero");
  if (staging_bytes == 0) return fail(S14_ERR_INVALID, "staging slot size must be greater than zero");
  s14_loader *l = new (std::nothrow) s14_loader();
  if (!l) return fail(S14_ERR_INVALID, "out of host memory");
  l->device = s14::ctx_device(ctx);
  l->stream = static_cast<hipStream_t>(s14_ctx_copy_stream(ctx));
  l->depth = pipeline_depth;
  l->staging_bytes = staging_bytes;
  l->pending.resize(pipeline_depth);
  hipError_t e = hipSetDevice(l->device);
  for (uint32_t i = 0; e == hipSuccess && i < pipeline_depth; ++i) {
    void *p = nullptr;
    e = hipHostMalloc(&p, staging_bytes, hipHostMallocDefault);
    if (e == hipSuccess) l->staging.push_back(static_cast<uint8_t *>(p));
    hipEvent_t ev = nullptr;
    if (e == hipSuccess) e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    if (e == hipSuccess) l->fences.push_back(ev);
  }
  if (e != hipSuccess) {
    s14_loader_destroy(l);
    return hip_fail(e, "loader staging ring");
  }
  *out = l;
  return S14_OK;
}

extern "C" void s14_loader_destroy(s14_loader *l) {
  if (!l) return;
  (void)hipSetDevice(l->device);
  // only submitted transfers have a fence to wait for (expert_loader.rs:444-458)
  for (uint32_t pip = 0; pip < l->fences.size() && pip < l->pending.size(); ++pip)
    if (l->pending[pip].live) (void)hipEventSynchronize(l->fences[pip]);
  for (hipEvent_t ev : l->fences) (void)hipEventDestroy(ev);
  for (uint8_t *p : l->staging) (void)hipHostFree(p);
  delete l;
}

extern "C" int s14_loader_enqueue(s14_loader *l, s14_pool *pool, s14_expert_key key, uint64_t bytes,
                                  s14_read_fn read, void *user, uint32_t *slot_out) {
  if (int rc = check_pool(l, pool)) return rc;
  if (!read || !slot_out) return fail(S14_ERR_INVALID, "NULL reader or slot output");
  return enqueue(l, pool, key, bytes, PageSource{nullptr, read, user}, slot_out);
}

extern "C" int s14_loader_enqueue_from_buf(s14_loader *l, s14_pool *pool, s14_expert_key key, const void *data,
                                           uint64_t bytes, uint32_t *slot_out) {
  if (int rc = check_pool(l, pool)) return rc;
  if (!data || !slot_out) return fail(S14_ERR_INVALID, "NULL page bytes or slot output");
  return enqueue(l, pool, key, bytes, PageSource{data, nullptr, nullptr}, slot_out);
}

extern "C" int s14_loader_wait_all(s14_loader *l, s14_pool *pool) {
  if (!l || !pool) return fail(S14_ERR_INVALID, "NULL loader or pool");
  return wait_all(l, pool);
}

extern "C" int s14_loader_batch_enqueue(s14_loader *l, s14_pool *pool, const s14_expert_key *keys,
                                        const uint64_t *bytes, size_t n, s14_read_fn read, void *user,
                                        uint32_t *slots_out) {
  if (int rc = check_pool(l, pool)) return rc;
  if (n && !read) return fail(S14_ERR_INVALID, "NULL reader");
  std::vector<PageSource> src(n, PageSource{nullptr, read, user});
  return batch_enqueue(l, pool, keys, bytes, n, src.data(), slots_out);
}

extern "C" int s14_loader_batch_enqueue_from_bufs(s14_loader *l, s14_pool *pool, const s14_expert_key *keys,
                                                  const void *const *data, const uint64_t *bytes, size_t n,
                                                  uint32_t *slots_out) {
  if (int rc = check_pool(l, pool)) return rc;
  if (n && !data) return fail(S14_ERR_INVALID, "NULL page bytes");
  std::vector<PageSource> src(n);
  for (size_t i = 0; i < n; ++i) {
    if (!data[i]) return fail(S14_ERR_INVALID, "page %zu has NULL bytes", i);
    src[i] = PageSource{data[i], nullptr, nullptr};
  }
  return batch_enqueue(l, pool, keys, bytes, n, src.data(), slots_out);
}

extern "C" int s14_loader_stats(const s14_loader *l, uint64_t *loads, uint64_t *bytes, uint32_t *in_flight) {
  if (!l) return fail(S14_ERR_INVALID, "NULL loader");
  if (loads) *loads = l->stat_loads;
  if (bytes) *bytes = l->stat_bytes;
  if (in_flight) {
    uint32_t n = 0;
    for (const auto &p : l->pending) n += p.live ? 1u : 0u;
    *in_flight = n;
  }
  return S14_OK;
}
