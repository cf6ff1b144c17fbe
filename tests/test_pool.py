"""Host contracts through the C ABI, on the CPU: every test of
scheduler/ssd_inference/src/vram_pool.rs:437-616 and
scheduler/ssd_inference/src/s14_vulkan.rs:834-996, plus the route contract
of scheduler/s14_runner/src/runner.rs:128-180.  Pools are created without a
device arena (the reference's new_for_tests)."""

from __future__ import annotations

import pytest

from colormlm_amd import _native as N
from colormlm_amd.pool import (
    ExpertKey,
    GraphProfile,
    LoadingReservation,
    RouteDecision,
    RouterKind,
    S14MoePages,
    SlotLease,
    VramPool,
)
from colormlm_amd.s14 import S14Error, S14MatvecShape, validate_e4m3fn_codes, validate_ue8m0_codes

ROUTED = N.S14_ROUTED_EXPERT_KIND
SHARED = N.S14_SHARED_EXPERT_KIND


def key(l, k, s):
    return ExpertKey(l, k, s)


# ---------------------------------------------------------------- vram_pool.rs


def test_reserve_eviction_logic(native):
    p = VramPool.new_for_tests(3, 1024)
    k1, k2, k3, k4 = (key(0, 0, i) for i in (1, 2, 3, 4))
    s1, e1 = p.reserve_loading(k1)
    assert s1 == 0 and e1 is None
    assert p.lookup(k1) is None
    p.mark_ready(s1, k1)
    s2, e2 = p.reserve_loading(k2)
    assert s2 == 1 and e2 is None
    p.mark_ready(s2, k2)
    s3, e3 = p.reserve_loading(k3)
    assert s3 == 2 and e3 is None
    p.mark_ready(s3, k3)
    assert p.n_loaded() == 3
    p.lookup(k2)  # touch k2 so k1 is the oldest
    s4, e4 = p.reserve_loading(k4)
    assert s4 == 0 and e4 == k1
    assert p.lookup(k4) is None
    p.mark_ready(s4, k4)
    assert p.n_loaded() == 3
    assert p.lookup(k1) is None
    assert p.lookup(k2) is not None and p.lookup(k3) is not None and p.lookup(k4) is not None


def test_loading_slots_are_hidden_and_never_evicted(native):
    p = VramPool.new_for_tests(1, 1024)
    loading, other = key(1, 0, 7), key(1, 0, 8)
    slot, _ = p.reserve_loading(loading)
    assert p.lookup(loading) is None
    with pytest.raises(S14Error):
        p.reserve_loading(other)
    p.cancel_loading(slot, loading)
    replacement, _ = p.reserve_loading(other)
    assert replacement == slot
    p.mark_ready(replacement, other)
    assert p.lookup(other) == slot


def test_pinned_ready_slot_cannot_be_evicted_until_compute_fence_release(native):
    p = VramPool.new_for_tests(1, 1024)
    resident, replacement = key(42, 0x53, 126), key(42, 0x53, 12)
    r = p.reserve_loading_generation(resident)
    lease = p.publish_batch_and_pin([r])[0]
    with pytest.raises(S14Error) as err:
        p.reserve_loading_generation(replacement)
    assert err.value.code == N.S14_ERR_POOL_FULL
    p.release_after_compute_fence(lease)
    p.reserve_loading_generation(replacement)


def test_stale_generation_is_rejected_after_slot_reuse(native):
    p = VramPool.new_for_tests(1, 1024)
    first, second = key(42, 0x53, 126), key(42, 0x53, 12)
    lease = p.publish_batch_and_pin([p.reserve_loading_generation(first)])[0]
    stale = lease.binding
    p.release_after_compute_fence(lease)
    p.publish_batch_and_pin([p.reserve_loading_generation(second)])
    with pytest.raises(S14Error) as err:
        p.validate_binding(stale)
    assert err.value.code == N.S14_ERR_STALE
    with pytest.raises(S14Error):
        p.release_after_compute_fence(SlotLease(stale))


def test_batch_publish_preflight_prevents_partial_visibility(native):
    p = VramPool.new_for_tests(2, 1024)
    first, second = key(42, 0x53, 126), key(42, 0x53, 12)
    r1 = p.reserve_loading_generation(first)
    r2 = p.reserve_loading_generation(second)
    stale2 = LoadingReservation(r2.key, r2.slot, r2.generation + 1, r2.evicted)
    with pytest.raises(S14Error):
        p.publish_batch_and_pin([r1, stale2])
    assert p.lookup(first) is None and p.lookup(second) is None
    p.cancel_reservation(r1)
    p.cancel_reservation(r2)


def test_pool_constructor_and_accounting(native):
    with pytest.raises(S14Error):
        VramPool.new_for_tests(0, 1024)
    with pytest.raises(S14Error):
        VramPool.new_for_tests(4, 0)
    p = VramPool.new_for_tests(4, N.EXPERT_PAGE_BYTES)
    assert p.capacity() == 4 and p.slot_bytes() == N.EXPERT_PAGE_BYTES
    assert p.total_bytes() == 4 * N.EXPERT_PAGE_BYTES
    assert p.slot_offset(3) == 3 * N.EXPERT_PAGE_BYTES
    assert p.slot_ptr(0) is None  # bookkeeping-only pool has no arena
    with pytest.raises(S14Error):
        p.validate_publish_batch([])
    r = p.reserve_loading_generation(key(1, 1, 1))
    with pytest.raises(S14Error):
        p.publish_batch_and_pin([r, r])  # duplicate slot/key
    with pytest.raises(S14Error):
        p.reserve_loading_generation(key(1, 1, 1))  # already loading
    p.mark_ready(r.slot, r.key)
    with pytest.raises(S14Error):
        p.reserve_loading_generation(key(1, 1, 1))  # already ready
    lease = p.lookup_and_pin(key(1, 1, 1))
    assert lease is not None and lease.binding.generation == r.generation
    p.validate_binding(lease.binding)
    p.release_after_compute_fence(lease)
    with pytest.raises(S14Error):
        p.release_after_compute_fence(lease)  # pin already released
    assert p.lookup_and_pin(key(9, 9, 9)) is None
    with pytest.raises(S14Error):
        p.cancel_reservation(r)  # slot is Ready now


# ---------------------------------------------------------------- s14_vulkan.rs


def test_real_sample_shapes_have_exact_byte_contracts(native, known_answers):
    bc = known_answers["byte_contracts"]
    w1 = S14MatvecShape.new(2048, 4096).validate_mxfp4()
    assert w1.mxfp4_weight_bytes() == bc["w1"]["weight_bytes"]
    assert w1.mxfp4_scale_bytes() == bc["w1"]["scale_bytes"]
    w2 = S14MatvecShape.new(4096, 2048).validate_mxfp4()
    assert w2.mxfp4_weight_bytes() == bc["w2"]["weight_bytes"]
    assert w2.mxfp4_scale_bytes() == bc["w2"]["scale_bytes"]
    wq = S14MatvecShape.new(1024, 4096).validate_fp8()
    assert wq.fp8_weight_bytes() == bc["wq_a"]["fp8_weight_bytes"]
    assert wq.fp8_scale_bytes() == bc["wq_a"]["fp8_scale_bytes"]
    from colormlm_amd.s14 import page_layout

    assert page_layout(N.S14_PAGE_MXFP4).total_bytes == bc["expert_page_bytes"]
    assert page_layout(N.S14_PAGE_FP8).total_bytes == bc["shared_expert_page_bytes"]


def test_rejects_invalid_quantized_codes(native):
    validate_ue8m0_codes([0, 127, 254])
    with pytest.raises(S14Error) as err:
        validate_ue8m0_codes([127, 255])
    assert err.value.code == N.S14_ERR_NAN_CODE
    validate_e4m3fn_codes([0x00, 0x01, 0x7E, 0xFE])
    for bad in ([0x7F], [0xFF]):
        with pytest.raises(S14Error):
            validate_e4m3fn_codes(bad)
    validate_ue8m0_codes([])  # empty is valid


def test_mxfp4_rejects_non_native_k_alignment(native):
    with pytest.raises(S14Error) as err:
        S14MatvecShape.new(1, 32).validate_mxfp4()
    assert err.value.code == N.S14_ERR_SHAPE
    with pytest.raises(S14Error):
        S14MatvecShape.new(0, 128)
    S14MatvecShape.new(1, 130).validate_fp8()  # FP8 accepts any K


def _route(ids, w=0.25, layer=42):
    return RouteDecision(layer, RouterKind.SCORE, list(ids), [w] * len(ids))


REF_IDS = [126, 12, 205, 149, 227, 174]


def test_route_load_batch_rolls_back_every_reservation_on_capacity_failure(native):
    routed = VramPool.new_for_tests(5, N.EXPERT_PAGE_BYTES)
    shared = VramPool.new_for_tests(1, N.SHARED_EXPERT_PAGE_BYTES)
    pages = S14MoePages(routed, shared, GraphProfile.S14_TOP6)
    with pytest.raises(S14Error):
        pages.begin_after_official_route(_route(REF_IDS))
    assert routed.n_loaded() == 0 and shared.n_loaded() == 0


def test_route_load_batch_rejects_duplicate_or_weight_drift_before_reservation(native):
    routed = VramPool.new_for_tests(6, N.EXPERT_PAGE_BYTES)
    shared = VramPool.new_for_tests(1, N.SHARED_EXPERT_PAGE_BYTES)
    pages = S14MoePages(routed, shared, GraphProfile.S14_TOP6)
    with pytest.raises(S14Error) as err:
        pages.begin_after_official_route(_route([126, 126, 205, 149, 227, 174]))
    assert err.value.code == N.S14_ERR_ROUTE
    drift = _route(REF_IDS)
    drift.weights[0] = 0.0
    with pytest.raises(S14Error):
        pages.begin_after_official_route(drift)
    assert routed.n_loaded() == 0 and shared.n_loaded() == 0


def test_route_load_batch_capacity_failure_releases_cached_pin(native):
    resident = key(42, ROUTED, 126)
    routed = VramPool.new_for_tests(1, N.EXPERT_PAGE_BYTES)
    lease = routed.publish_batch_and_pin([routed.reserve_loading_generation(resident)])[0]
    routed.release_after_compute_fence(lease)
    shared = VramPool.new_for_tests(1, N.SHARED_EXPERT_PAGE_BYTES)
    pages = S14MoePages(routed, shared, GraphProfile.S14_TOP6)
    with pytest.raises(S14Error):
        pages.begin_after_official_route(_route(REF_IDS))
    routed.reserve_loading_generation(key(42, ROUTED, 7))  # the cached pin was released


def test_route_load_batch_publishes_all_then_holds_compute_fence_pins(native):
    routed = VramPool.new_for_tests(6, N.EXPERT_PAGE_BYTES)
    shared = VramPool.new_for_tests(1, N.SHARED_EXPERT_PAGE_BYTES)
    pages = S14MoePages(routed, shared, GraphProfile.S14_TOP6)
    batch = pages.begin_after_official_route(_route(REF_IDS))
    compute = pages.publish_after_transfer_fence(batch)
    assert len(compute.routed_bindings()) == 6
    assert [b.key.slot for b in compute.routed_bindings()] == REF_IDS
    assert compute.shared_binding().key == key(42, SHARED, 0)
    with pytest.raises(S14Error):
        pages.begin_after_official_route(_route([1, 2, 3, 4, 5, 6]))
    pages.release_after_compute_fence(compute)
    replacement = pages.begin_after_official_route(_route([1, 2, 3, 4, 5, 6]))
    pages.cancel(replacement)


def test_stale_shared_generation_prevents_partial_routed_publication(native):
    routed = VramPool.new_for_tests(6, N.EXPERT_PAGE_BYTES)
    shared = VramPool.new_for_tests(1, N.SHARED_EXPERT_PAGE_BYTES)
    pages = S14MoePages(routed, shared, GraphProfile.S14_TOP6)
    batch = pages.begin_after_official_route(_route(REF_IDS))
    stale_shared = batch.shared_reservation()
    shared.cancel_reservation(stale_shared)
    unrelated = shared.reserve_loading_generation(key(42, SHARED, 1))
    with pytest.raises(S14Error):
        pages.publish_after_transfer_fence(batch)
    for e in REF_IDS:
        assert routed.lookup(key(42, ROUTED, e)) is None
    shared.cancel_reservation(unrelated)


def test_cached_pages_are_pinned_not_reloaded(native):
    routed = VramPool.new_for_tests(7, N.EXPERT_PAGE_BYTES)
    shared = VramPool.new_for_tests(1, N.SHARED_EXPERT_PAGE_BYTES)
    pages = S14MoePages(routed, shared, GraphProfile.S14_TOP6)
    lease = pages.publish_after_transfer_fence(pages.begin_after_official_route(_route(REF_IDS)))
    pages.release_after_compute_fence(lease)
    batch = pages.begin_after_official_route(_route([126, 12, 205, 149, 227, 5]))
    kinds = [isinstance(p, SlotLease) for p in batch.pages()]
    assert kinds == [True] * 5 + [False, True]  # expert 5 loads, shared page is cached
    lease = pages.publish_after_transfer_fence(batch)
    pages.release_after_compute_fence(lease)


def test_moe_pages_slot_size_checks(native):
    small = VramPool.new_for_tests(6, N.EXPERT_PAGE_BYTES - 1)
    shared = VramPool.new_for_tests(1, N.SHARED_EXPERT_PAGE_BYTES)
    with pytest.raises(S14Error) as err:
        S14MoePages(small, shared, GraphProfile.S14_TOP6)
    assert err.value.code == N.S14_ERR_CAPACITY
    routed = VramPool.new_for_tests(6, N.EXPERT_PAGE_BYTES)
    mx_shared = VramPool.new_for_tests(1, N.EXPERT_PAGE_BYTES)
    with pytest.raises(S14Error):
        S14MoePages(routed, mx_shared, GraphProfile.S14_TOP6)  # FP8 shared page needs 25,167,360 B
    S14MoePages(routed, mx_shared, GraphProfile.S14_TOP6, shared_format=N.S14_PAGE_MXFP4, weight_sum=1.0)


# ---------------------------------------------------------------- runner.rs


def test_route_decision_validate_for(native):
    ok = _route(REF_IDS)
    ok.validate_for(GraphProfile.S14_TOP6)
    ok.validate_for(GraphProfile.FULL_DEPTH43_NATIVE_TOP6)
    with pytest.raises(S14Error):
        _route(REF_IDS, layer=5).validate_for(GraphProfile.S14_TOP6)  # layer not selected
    _route(REF_IDS, layer=5).validate_for(GraphProfile.FULL_DEPTH43_NATIVE_TOP6)
    with pytest.raises(S14Error):
        _route(REF_IDS, layer=43).validate_for(GraphProfile.FULL_DEPTH43_NATIVE_TOP6)
    with pytest.raises(S14Error):
        RouteDecision(42, RouterKind.HASH, REF_IDS, [0.25] * 6).validate_for(GraphProfile.S14_TOP6)
    RouteDecision(1, RouterKind.HASH, REF_IDS, [0.25] * 6).validate_for(GraphProfile.S14_TOP6)
    with pytest.raises(S14Error):
        RouteDecision(1, RouterKind.SCORE, REF_IDS, [0.25] * 6).validate_for(GraphProfile.S14_TOP6)
    with pytest.raises(S14Error):
        _route(REF_IDS[:5], w=0.3).validate_for(GraphProfile.S14_TOP6)  # top-5
    with pytest.raises(S14Error):
        RouteDecision(42, RouterKind.SCORE, REF_IDS, [0.25] * 5).validate_for(GraphProfile.S14_TOP6)
    with pytest.raises(S14Error):
        _route([256, 12, 205, 149, 227, 174]).validate_for(GraphProfile.S14_TOP6)
    bad = _route(REF_IDS)
    bad.weights[2] = float("nan")
    with pytest.raises(S14Error):
        bad.validate_for(GraphProfile.S14_TOP6)
    neg = _route(REF_IDS)
    neg.weights = [0.3, 0.3, 0.3, 0.3, 0.35, -0.05]
    with pytest.raises(S14Error):
        neg.validate_for(GraphProfile.S14_TOP6)
    # renormalised (BASELINE) weights sum to 1
    _route(REF_IDS, w=1 / 6).validate_for(GraphProfile.S14_TOP6, weight_sum=1.0)
    with pytest.raises(S14Error):
        _route(REF_IDS, w=1 / 6).validate_for(GraphProfile.S14_TOP6)
