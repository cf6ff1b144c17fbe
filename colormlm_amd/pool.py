"""Page pool and route page batches — Python face of the C ABI.

Mirrors, name for name, the reference's Rust interface so callers and tests
read the same:
  VramPool                 scheduler/ssd_inference/src/vram_pool.rs:62-405
  ExpertLoader             scheduler/ssd_inference/src/expert_loader.rs:26-474
  S14MoePages              scheduler/ssd_inference/src/s14_vulkan.rs:703-819
  RouteDecision.validate_for  scheduler/s14_runner/src/runner.rs:128-180
All state lives in the C++ library; this module only marshals arguments and
raises S14Error where the Rust code would `bail!`.
"""

from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field
from enum import Enum
from typing import List, Optional, Sequence

from . import _native as N
from ._native import S14Error, check, lib


@dataclass(frozen=True)
class ExpertKey:
    layer: int
    kind: int
    slot: int

    def c(self) -> N.ExpertKeyC:
        return N.ExpertKeyC(self.layer, self.kind, self.slot)

    @staticmethod
    def from_c(k: N.ExpertKeyC) -> "ExpertKey":
        return ExpertKey(int(k.layer), int(k.kind), int(k.slot))


@dataclass(frozen=True)
class SlotBinding:
    key: ExpertKey
    slot: int
    generation: int

    def c(self) -> N.SlotBindingC:
        return N.SlotBindingC(self.key.c(), self.slot, self.generation)

    @staticmethod
    def from_c(b: N.SlotBindingC) -> "SlotBinding":
        return SlotBinding(ExpertKey.from_c(b.key), int(b.slot), int(b.generation))


@dataclass(frozen=True)
class SlotLease:
    """A compute-side pin (vram_pool.rs:39-50)."""

    binding: SlotBinding


@dataclass(frozen=True)
class LoadingReservation:
    key: ExpertKey
    slot: int
    generation: int
    evicted: Optional[ExpertKey] = None

    def c(self) -> N.LoadingReservationC:
        ev = self.evicted.c() if self.evicted else N.ExpertKeyC(0, 0, 0)
        return N.LoadingReservationC(self.key.c(), self.slot, self.generation, 1 if self.evicted else 0, ev)

    @staticmethod
    def from_c(r: N.LoadingReservationC) -> "LoadingReservation":
        ev = ExpertKey.from_c(r.evicted) if r.has_evicted else None
        return LoadingReservation(ExpertKey.from_c(r.key), int(r.slot), int(r.generation), ev)


class VramPool:
    """VramPool (vram_pool.rs:62-405).  ``ctx=None`` gives the bookkeeping-only
    pool of the reference's ``new_for_tests`` (no device arena)."""

    def __init__(self, n_slots: int, slot_bytes: int, ctx=None):
        self._h = C.c_void_p()
        # the pool's fences and uploads go through ctx: keep it alive as long as the pool
        self._ctx = ctx
        check(lib().s14_pool_create(ctx.handle if ctx is not None else None, n_slots, slot_bytes, C.byref(self._h)))

    @classmethod
    def new_for_tests(cls, n_slots: int, slot_bytes: int) -> "VramPool":
        return cls(n_slots, slot_bytes, None)

    @property
    def handle(self):
        return self._h

    def destroy(self) -> None:
        if self._h:
            lib().s14_pool_destroy(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass

    def capacity(self) -> int:
        return int(lib().s14_pool_capacity(self._h))

    def slot_bytes(self) -> int:
        return int(lib().s14_pool_slot_bytes(self._h))

    def n_loaded(self) -> int:
        return int(lib().s14_pool_n_loaded(self._h))

    def total_bytes(self) -> int:
        return int(lib().s14_pool_total_bytes(self._h))

    def slot_offset(self, slot: int) -> int:
        return int(lib().s14_pool_slot_offset(self._h, slot))

    def slot_ptr(self, slot: int) -> Optional[int]:
        p = lib().s14_pool_slot_ptr(self._h, slot)
        return int(p) if p else None

    def slot_tensor(self, slot: int):
        """A torch uint8 view of one slot of the device arena (no copy)."""
        import torch

        ptr = self.slot_ptr(slot)
        if ptr is None:
            raise S14Error(N.S14_ERR_INVALID, "pool has no device arena")
        return torch.as_tensor(_DeviceBytes(ptr, self.slot_bytes(), self), device="cuda")

    def lookup(self, key: ExpertKey) -> Optional[int]:
        slot = C.c_uint32()
        return int(slot.value) if lib().s14_pool_lookup(self._h, key.c(), C.byref(slot)) else None

    def lookup_and_pin(self, key: ExpertKey) -> Optional[SlotLease]:
        found = C.c_int()
        b = N.SlotBindingC()
        check(lib().s14_pool_lookup_and_pin(self._h, key.c(), C.byref(found), C.byref(b)))
        return SlotLease(SlotBinding.from_c(b)) if found.value else None

    def reserve_loading(self, key: ExpertKey):
        slot, has_ev, ev = C.c_uint32(), C.c_int(), N.ExpertKeyC()
        check(lib().s14_pool_reserve_loading(self._h, key.c(), C.byref(slot), C.byref(has_ev), C.byref(ev)))
        return int(slot.value), (ExpertKey.from_c(ev) if has_ev.value else None)

    def reserve_loading_generation(self, key: ExpertKey) -> LoadingReservation:
        r = N.LoadingReservationC()
        check(lib().s14_pool_reserve_loading_generation(self._h, key.c(), C.byref(r)))
        return LoadingReservation.from_c(r)

    def mark_ready(self, slot: int, key: ExpertKey) -> None:
        check(lib().s14_pool_mark_ready(self._h, slot, key.c()))

    def validate_publish_batch(self, reservations: Sequence[LoadingReservation]) -> None:
        arr = (N.LoadingReservationC * max(1, len(reservations)))(*[r.c() for r in reservations])
        check(lib().s14_pool_validate_publish_batch(self._h, arr, len(reservations)))

    def publish_batch_and_pin(self, reservations: Sequence[LoadingReservation]) -> List[SlotLease]:
        n = len(reservations)
        arr = (N.LoadingReservationC * max(1, n))(*[r.c() for r in reservations])
        out = (N.SlotBindingC * max(1, n))()
        check(lib().s14_pool_publish_batch_and_pin(self._h, arr, n, out))
        return [SlotLease(SlotBinding.from_c(out[i])) for i in range(n)]

    def validate_binding(self, binding: SlotBinding) -> None:
        check(lib().s14_pool_validate_binding(self._h, binding.c()))

    def release_after_compute_fence(self, lease: SlotLease) -> None:
        check(lib().s14_pool_release_after_compute_fence(self._h, lease.binding.c()))

    def cancel_loading(self, slot: int, key: ExpertKey) -> None:
        lib().s14_pool_cancel_loading(self._h, slot, key.c())

    def cancel_reservation(self, reservation: LoadingReservation) -> None:
        check(lib().s14_pool_cancel_reservation(self._h, reservation.c()))

    def upload(self, ctx, reservation: LoadingReservation, host_bytes) -> "Fence":
        """hipMemcpyAsync into the reserved slot on ctx's copy stream; the
        returned transfer fence must complete before publication."""
        import numpy as np

        buf = np.ascontiguousarray(np.frombuffer(host_bytes, dtype=np.uint8))
        fence = C.c_void_p()
        r = reservation.c()
        check(lib().s14_pool_upload(ctx.handle, self._h, C.byref(r), buf.ctypes.data, buf.nbytes, C.byref(fence)))
        return Fence(fence, keepalive=buf)


class ExpertLoader:
    """ExpertLoader (expert_loader.rs:26-474): a pinned staging ring of
    ``pipeline_depth`` slots feeding the VRAM pool over the context's copy
    stream, one transfer fence per slot.

    ``reader(key, dst_view)`` fills a writable memoryview of the page's size
    (the role of ExpertReader::read_into) and returns nothing; an exception
    cancels the reservation and surfaces as S14Error."""

    def __init__(self, ctx, pipeline_depth: int, staging_bytes: int):
        self._h = C.c_void_p()
        check(lib().s14_loader_create(ctx.handle, pipeline_depth, staging_bytes, C.byref(self._h)))
        self.pipeline_depth = pipeline_depth
        self.staging_bytes = staging_bytes

    def destroy(self) -> None:
        if self._h:
            lib().s14_loader_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass

    @staticmethod
    def _reader(reader):
        def cb(user, key, dst, nbytes):
            try:
                reader(ExpertKey.from_c(key), (C.c_ubyte * nbytes).from_address(dst))
                return 0
            except Exception:
                return 1

        return N.READ_FN(cb)

    def enqueue(self, pool: VramPool, key: ExpertKey, nbytes: int, reader) -> int:
        """enqueue (expert_loader.rs:163-284): the page's VRAM slot."""
        slot = C.c_uint32()
        fn = self._reader(reader)
        check(lib().s14_loader_enqueue(self._h, pool.handle, key.c(), nbytes, fn, None, C.byref(slot)))
        return int(slot.value)

    def enqueue_from_buf(self, pool: VramPool, key: ExpertKey, data) -> int:
        """enqueue_from_buf (expert_loader.rs:362-442): bytes already in host memory."""
        import numpy as np

        buf = np.ascontiguousarray(np.frombuffer(data, dtype=np.uint8))
        slot = C.c_uint32()
        check(lib().s14_loader_enqueue_from_buf(self._h, pool.handle, key.c(), buf.ctypes.data, buf.nbytes,
                                                C.byref(slot)))
        return int(slot.value)

    def wait_all(self, pool: VramPool) -> None:
        check(lib().s14_loader_wait_all(self._h, pool.handle))

    def batch_enqueue(self, pool: VramPool, keys: Sequence[ExpertKey], sizes: Sequence[int], reader) -> List[int]:
        """batch_enqueue (expert_loader.rs:299-360): VRAM slots in input order."""
        n = len(keys)
        kc = (N.ExpertKeyC * max(1, n))(*[k.c() for k in keys])
        sz = (C.c_uint64 * max(1, n))(*sizes)
        out = (C.c_uint32 * max(1, n))()
        fn = self._reader(reader)
        check(lib().s14_loader_batch_enqueue(self._h, pool.handle, kc, sz, n, fn, None, out))
        return [int(out[i]) for i in range(n)]

    def batch_enqueue_from_bufs(self, pool: VramPool, keys: Sequence[ExpertKey], datas) -> List[int]:
        """batch_enqueue with every page's bytes in host memory."""
        import numpy as np

        bufs = [np.ascontiguousarray(np.frombuffer(d, dtype=np.uint8)) for d in datas]
        n = len(keys)
        kc = (N.ExpertKeyC * max(1, n))(*[k.c() for k in keys])
        ptrs = (C.c_void_p * max(1, n))(*[b.ctypes.data for b in bufs])
        sz = (C.c_uint64 * max(1, n))(*[b.nbytes for b in bufs])
        out = (C.c_uint32 * max(1, n))()
        check(lib().s14_loader_batch_enqueue_from_bufs(self._h, pool.handle, kc, ptrs, sz, n, out))
        return [int(out[i]) for i in range(n)]

    def stats(self) -> dict:
        loads, nbytes, inflight = C.c_uint64(), C.c_uint64(), C.c_uint32()
        check(lib().s14_loader_stats(self._h, C.byref(loads), C.byref(nbytes), C.byref(inflight)))
        return {"stat_loads": int(loads.value), "stat_bytes": int(nbytes.value), "in_flight": int(inflight.value)}


class _DeviceBytes:
    """__cuda_array_interface__ of a byte range of device memory."""

    def __init__(self, ptr: int, nbytes: int, owner):
        self._owner = owner
        self.__cuda_array_interface__ = {"shape": (nbytes,), "typestr": "|u1", "data": (ptr, False), "version": 3}


class Fence:
    """A hipEvent standing in for the reference's Vulkan fences."""

    def __init__(self, handle, keepalive=None):
        self._h = handle
        self._keep = keepalive

    @classmethod
    def record(cls, ctx, stream=None) -> "Fence":
        h = C.c_void_p()
        check(lib().s14_fence_record(ctx.handle, stream, C.byref(h)))
        return cls(h)

    def is_complete(self) -> bool:
        rc = lib().s14_fence_query(self._h)
        if rc == N.S14_ERR_NOT_READY:
            return False
        check(rc)
        return True

    def wait(self) -> None:
        check(lib().s14_fence_wait(self._h))
        self._keep = None

    def destroy(self) -> None:
        if self._h:
            lib().s14_fence_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


class RouterKind(Enum):
    HASH = N.S14_ROUTER_HASH
    SCORE = N.S14_ROUTER_SCORE


class GraphProfile(Enum):
    S14_TOP6 = N.S14_PROFILE_S14_TOP6
    FULL_DEPTH43_NATIVE_TOP6 = N.S14_PROFILE_FULL_DEPTH43_TOP6


REFERENCE_ROUTE_SCALE = 1.5  # route_scale "1.5_exact" (s14_contract.json:12)


@dataclass
class RouteDecision:
    layer: int
    kind: RouterKind
    expert_ids: List[int]
    weights: List[float]

    def c(self) -> N.RouteDecisionC:
        r = N.RouteDecisionC()
        r.layer = self.layer
        r.kind = self.kind.value
        same = len(self.expert_ids) == len(self.weights) and len(self.expert_ids) <= 16
        # a length mismatch fails validate_for's top-k check, as in runner.rs:137-147
        r.n = len(self.expert_ids) if same else 0xFFFFFFFF
        for i, e in enumerate(self.expert_ids[:16]):
            r.expert_ids[i] = e
        for i, w in enumerate(self.weights[:16]):
            r.weights[i] = w
        return r

    def validate_for(self, profile: GraphProfile, weight_sum: float = REFERENCE_ROUTE_SCALE) -> None:
        r = self.c()
        check(lib().s14_route_validate_for(C.byref(r), profile.value, weight_sum))


class RouteLoadBatch:
    """Pages of one route: routed (route order) then shared; each either a
    cached pinned page or a Loading reservation awaiting its upload."""

    def __init__(self, handle):
        self._h = handle

    def pages(self):
        out = []
        n = lib().s14_route_load_batch_size(self._h)
        for i in range(n):
            loading = C.c_int()
            r = N.LoadingReservationC()
            b = N.SlotBindingC()
            check(lib().s14_route_load_batch_page(self._h, i, C.byref(loading), C.byref(r), C.byref(b)))
            out.append(LoadingReservation.from_c(r) if loading.value else SlotLease(SlotBinding.from_c(b)))
        return out

    def shared_reservation(self) -> LoadingReservation:
        r = N.LoadingReservationC()
        check(lib().s14_route_load_batch_shared_reservation(self._h, C.byref(r)))
        return LoadingReservation.from_c(r)


class S14MoeComputeLeaseBatch:
    def __init__(self, handle, n_routed: int):
        self._h = handle
        self._n = n_routed

    def routed_bindings(self) -> List[SlotBinding]:
        arr = (N.SlotBindingC * self._n)()
        check(lib().s14_moe_lease_batch_bindings(self._h, arr, self._n, None))
        return [SlotBinding.from_c(arr[i]) for i in range(self._n)]

    def shared_binding(self) -> SlotBinding:
        b = N.SlotBindingC()
        check(lib().s14_moe_lease_batch_bindings(self._h, None, 0, C.byref(b)))
        return SlotBinding.from_c(b)


class S14MoePages:
    """S14VulkanMoePages (s14_vulkan.rs:703-819) over two pools."""

    def __init__(
        self,
        routed_pool: VramPool,
        shared_pool: VramPool,
        profile: GraphProfile,
        shared_format: int = N.S14_PAGE_FP8,
        weight_sum: float = REFERENCE_ROUTE_SCALE,
    ):
        self._h = C.c_void_p()
        self.routed_pool = routed_pool
        self.shared_pool = shared_pool
        check(
            lib().s14_moe_pages_create(
                routed_pool.handle, shared_pool.handle, profile.value, shared_format, weight_sum, C.byref(self._h)
            )
        )

    def __del__(self):
        try:
            if self._h:
                lib().s14_moe_pages_destroy(self._h)
                self._h = C.c_void_p()
        except Exception:
            pass

    def begin_after_official_route(self, route: RouteDecision) -> RouteLoadBatch:
        r = route.c()
        h = C.c_void_p()
        check(lib().s14_moe_pages_begin_after_official_route(self._h, C.byref(r), C.byref(h)))
        return RouteLoadBatch(h)

    def publish_after_transfer_fence(self, batch: RouteLoadBatch) -> S14MoeComputeLeaseBatch:
        n_routed = lib().s14_route_load_batch_size(batch._h) - 1
        h = C.c_void_p()
        try:
            check(lib().s14_moe_pages_publish_after_transfer_fence(self._h, batch._h, C.byref(h)))
        finally:
            batch._h = None  # consumed either way
        return S14MoeComputeLeaseBatch(h, n_routed)

    def release_after_compute_fence(self, lease: S14MoeComputeLeaseBatch) -> None:
        check(lib().s14_moe_pages_release_after_compute_fence(self._h, lease._h))
        lease._h = None

    def cancel(self, batch: RouteLoadBatch) -> None:
        try:
            check(lib().s14_moe_pages_cancel(self._h, batch._h))
        finally:
            batch._h = None


__all__ = [
    "ExpertKey",
    "SlotBinding",
    "SlotLease",
    "LoadingReservation",
    "VramPool",
    "ExpertLoader",
    "Fence",
    "RouterKind",
    "GraphProfile",
    "RouteDecision",
    "RouteLoadBatch",
    "S14MoeComputeLeaseBatch",
    "S14MoePages",
    "S14Error",
    "REFERENCE_ROUTE_SCALE",
]
