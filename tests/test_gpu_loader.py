"""GPU tests of the expert page uploader (ExpertLoader, expert_loader.rs:
26-474): pinned staging ring, transfers and fences on the context's copy
stream, publication into the VRAM pool only after each fence, waves no deeper
than the ring, and a MoE layer computed from uploaded pages against the CPU
oracle bit for bit."""

from __future__ import annotations

import sys

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from colormlm_amd import _native as N  # noqa: E402
from colormlm_amd import s14, synth  # noqa: E402
from colormlm_amd.pool import ExpertKey, ExpertLoader, S14Error, VramPool  # noqa: E402

pytestmark = pytest.mark.gpu

SLOT = 1 << 20  # small slots keep the ring tests fast; the layer test uses full pages


def say(msg: str) -> None:
    print(f"[gpu-test] {msg}", file=sys.stderr, flush=True)


@pytest.fixture(scope="module")
def ctx():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    c = s14.Context(0)
    yield c
    torch.cuda.synchronize()
    c.destroy()


def page(i: int, nbytes: int = SLOT) -> np.ndarray:
    return np.random.default_rng(1000 + i).integers(0, 256, nbytes, dtype=np.uint8)


def on_device(pool: VramPool, slot: int, nbytes: int) -> np.ndarray:
    torch.cuda.synchronize()
    return pool.slot_tensor(slot)[:nbytes].cpu().numpy()


def test_ring_publishes_after_fences_and_bytes_arrive(ctx):
    say("loader ring: 10 pages through 3 staging slots")
    pool = VramPool(12, SLOT, ctx)
    loader = ExpertLoader(ctx, pipeline_depth=3, staging_bytes=SLOT)
    keys = [ExpertKey(1, 0, i) for i in range(10)]
    slots = [loader.enqueue_from_buf(pool, k, page(i)) for i, k in enumerate(keys)]
    # the last ring slot's page is still Loading: invisible until its fence completes
    assert pool.lookup(keys[-1]) is None
    assert loader.stats()["in_flight"] >= 1
    loader.wait_all(pool)
    assert loader.stats() == {"stat_loads": 10, "stat_bytes": 10 * SLOT, "in_flight": 0}
    for i, (k, s) in enumerate(zip(keys, slots)):
        assert pool.lookup(k) == s
        assert np.array_equal(on_device(pool, s, SLOT), page(i)), i
    # Ready keys come back without a transfer
    assert loader.enqueue_from_buf(pool, keys[3], page(99)) == slots[3]
    assert loader.stats()["stat_loads"] == 10
    loader.destroy()
    pool.destroy()


def test_pending_key_completes_instead_of_reloading(ctx):
    pool = VramPool(4, SLOT, ctx)
    loader = ExpertLoader(ctx, pipeline_depth=2, staging_bytes=SLOT)
    k = ExpertKey(0, 0, 7)
    s = loader.enqueue_from_buf(pool, k, page(7))
    assert loader.enqueue_from_buf(pool, k, page(8)) == s  # completes the pending transfer
    assert pool.lookup(k) == s and loader.stats()["stat_loads"] == 1
    assert np.array_equal(on_device(pool, s, SLOT), page(7))
    loader.destroy()
    pool.destroy()


def test_batch_dedupes_waves_and_capacity(ctx):
    say("loader batch: duplicates, waves, capacity")
    pool = VramPool(8, SLOT, ctx)
    loader = ExpertLoader(ctx, pipeline_depth=3, staging_bytes=SLOT)
    ids = [5, 1, 5, 2, 3, 1, 4, 6, 7]  # 7 distinct keys: waves of 3, 3, 1
    keys = [ExpertKey(2, 0, i) for i in ids]
    slots = loader.batch_enqueue_from_bufs(pool, keys, [page(i) for i in ids])
    assert slots[0] == slots[2] and slots[1] == slots[5] and len(set(slots)) == 7
    assert loader.stats()["stat_loads"] == 7
    loader.wait_all(pool)
    for i, s in zip(ids, slots):
        assert np.array_equal(on_device(pool, s, SLOT), page(i))
    # more distinct keys than slots: rejected before anything is reserved
    before = pool.n_loaded()
    with pytest.raises(S14Error) as err:
        loader.batch_enqueue_from_bufs(pool, [ExpertKey(3, 0, i) for i in range(9)], [page(i) for i in range(9)])
    assert err.value.code == N.S14_ERR_CAPACITY and pool.n_loaded() == before
    loader.destroy()
    pool.destroy()


def test_reader_path_failure_cancels_and_oversize_rejected(ctx):
    pool = VramPool(4, SLOT, ctx)
    loader = ExpertLoader(ctx, pipeline_depth=2, staging_bytes=SLOT)
    seen = []

    def reader(key, dst):
        seen.append(key)
        dst[:] = page(key.slot).tobytes()

    keys = [ExpertKey(4, 0, i) for i in (11, 12, 13)]
    slots = loader.batch_enqueue(pool, keys, [SLOT] * 3, reader)
    loader.wait_all(pool)
    assert seen == keys
    for k, s in zip(keys, slots):
        assert np.array_equal(on_device(pool, s, SLOT), page(k.slot))

    def broken(key, dst):
        raise IOError("disk")

    bad = ExpertKey(4, 0, 20)
    n = pool.n_loaded()
    with pytest.raises(S14Error):
        loader.enqueue(pool, bad, SLOT, broken)
    assert pool.lookup(bad) is None and pool.n_loaded() == n  # reservation cancelled
    with pytest.raises(S14Error) as err:
        loader.enqueue_from_buf(pool, ExpertKey(4, 0, 21), np.zeros(SLOT + 1, np.uint8))
    assert err.value.code == N.S14_ERR_CAPACITY
    loader.destroy()
    pool.destroy()


def test_eviction_skips_pinned_pages(ctx):
    """Four slots, six pages: the loader's reservations evict the least
    recently used Ready pages, never a pinned one."""
    pool = VramPool(4, SLOT, ctx)
    loader = ExpertLoader(ctx, pipeline_depth=2, staging_bytes=SLOT)
    first = [ExpertKey(5, 0, i) for i in range(4)]
    for i, k in enumerate(first):
        loader.enqueue_from_buf(pool, k, page(i))
    loader.wait_all(pool)
    lease = pool.lookup_and_pin(first[0])
    assert lease is not None
    for i in (4, 5):
        loader.enqueue_from_buf(pool, ExpertKey(5, 0, i), page(i))
    loader.wait_all(pool)
    assert pool.lookup(first[0]) == lease.binding.slot  # pinned: kept
    assert pool.lookup(first[1]) is None and pool.lookup(first[2]) is None  # least recently used: evicted
    pool.release_after_compute_fence(lease)
    loader.destroy()
    pool.destroy()


def test_layer_from_loader_uploaded_pages(ctx, oracle):
    """Six routed pages and the shared page uploaded through the loader
    (13.4 MB each, ring of 2), then the MoE layer from their slot addresses,
    bit for bit against the oracle on the same pages."""
    say("loader: 7 full pages -> layer")
    ids = [126, 12, 205, 149, 227, 174]
    hosts = {e: synth.gen_mxfp4_page(0, 0, e) for e in ids}
    hosts[256] = synth.gen_mxfp4_page(0, 0, synth.SHARED_EXPERT)
    pool = VramPool(8, N.EXPERT_PAGE_BYTES, ctx)
    loader = ExpertLoader(ctx, pipeline_depth=2, staging_bytes=N.EXPERT_PAGE_BYTES)
    keys = [ExpertKey(0, 0, e) for e in ids] + [ExpertKey(0, 0x54, 0)]
    slots = loader.batch_enqueue_from_bufs(pool, keys, [hosts[e] for e in ids + [256]])
    loader.wait_all(pool)
    x = synth.token(seed=6)
    w = np.array([0.3, 0.2, 0.15, 0.15, 0.1, 0.1], np.float32)
    y = torch.empty(N.HIDDEN, dtype=torch.float32, device="cuda")
    s14.moe_layer(ctx, [pool.slot_ptr(s) for s in slots[:6]], w.tolist(), pool.slot_ptr(slots[6]),
                  torch.from_numpy(x).cuda(), y, mode=s14.EXACT)
    torch.cuda.synchronize()
    want = oracle.moe_layer(x, [hosts[e] for e in ids], w, hosts[256])
    assert np.array_equal(y.cpu().numpy().view(np.uint32), want.view(np.uint32))
    loader.destroy()
    pool.destroy()
