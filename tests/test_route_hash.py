"""The oracle's hash router (the reference's layers 0-2: experts from the
tid2eid row of the token, executor.py:643-667) and RouteDecision's
validate_for checks (runner.rs:128-180), on the CPU.

Pinned by: the reference's own test routes (runner.rs:709-714,
tests/range_bridge.rs:33-38: six ids with weights 0.25 each, which
validate_for accepts at route scale 1.5); a closed form (zero router weights
give logit 0, sigmoid score exactly 0.5, weight exactly f32(0.5 / 3.0)); the
score router's own top-6 row, for which the hash route must reproduce the
score route's ids and weights bit for bit; f64 renormalisation; and every
rejection case of validate_for and of the executor's row checks."""

from __future__ import annotations

import numpy as np
import pytest

from colormlm_amd import synth


def test_validate_for_reference_routes(oracle):
    w = np.full(6, 0.25, np.float32)
    for ids in ([0, 1, 2, 3, 4, 5], [126, 12, 205, 149, 227, 174]):
        assert oracle.route_valid(ids, w, route_scale=1.5)
        assert not oracle.route_valid(ids, w, route_scale=1.0)  # sums to 1.5, not 1
    ids = [126, 12, 205, 149, 227, 174]
    assert not oracle.route_valid([126, 12, 205, 149, 227, 126], w, route_scale=1.5)  # repeated expert
    assert not oracle.route_valid([126, 12, 205, 149, 227, 256], w, route_scale=1.5)  # out of range
    for bad in (np.nan, np.inf, -0.25):
        wb = w.copy()
        wb[3] = bad
        assert not oracle.route_valid(ids, wb, route_scale=1.5)
    wb = w.copy()
    wb[0] += np.float32(2e-4)  # sum off by more than 1e-4
    assert not oracle.route_valid(ids, wb, route_scale=1.5)
    wb = w.copy()
    wb[0] += np.float32(5e-5)
    assert oracle.route_valid(ids, wb, route_scale=1.5)


def test_hash_route_closed_form(oracle):
    wr = np.zeros((256, 4096), np.float32)
    bias = synth.gen_normal(3, 9, 256, 0.0, 0.01)
    x = synth.token(seed=3)
    row = np.array([17, 3, 250, 99, 0, 128], np.int64)
    scores, ids, w = oracle.route_hash(wr, bias, x, row)
    assert np.all(scores == np.float32(0.5))
    assert ids.tolist() == row.tolist()
    assert np.all(w == np.float32(0.5) / np.float32(3.0))
    _, _, w15 = oracle.route_hash(wr, bias, x, row, route_scale=1.5)
    assert np.all(w15 == (np.float32(0.5) / np.float32(3.0)) * np.float32(1.5))


@pytest.mark.parametrize("score_fn,scale", [(0, 1.0), (1, 1.5)])
def test_hash_route_reproduces_score_route(oracle, score_fn, scale):
    wr, bias = synth.router(seed=0, layer=2)
    for i in range(4):
        x = synth.token(seed=0, index=i)
        s_sc, ids, w = oracle.route(wr, bias, x, score_fn=score_fn, route_scale=scale)
        s_h, ids_h, w_h = oracle.route_hash(wr, bias, x, ids.astype(np.int64), score_fn=score_fn, route_scale=scale)
        assert np.array_equal(s_sc.view(np.uint32), s_h.view(np.uint32))
        assert ids_h.tolist() == ids.tolist()
        assert np.array_equal(w_h.view(np.uint32), w.view(np.uint32))


def test_hash_route_weights_f64_and_valid(oracle):
    wr, bias = synth.router(seed=0, layer=1)
    rng = np.random.default_rng(11)
    for i in range(8):
        x = synth.token(seed=1, index=i)
        row = rng.choice(256, size=6, replace=False).astype(np.int64)
        scores, ids, w = oracle.route_hash(wr, bias, x, row, score_fn=1, route_scale=1.5)
        s = scores[row].astype(np.float64)
        np.testing.assert_allclose(w.astype(np.float64), s / s.sum() * 1.5, rtol=1e-6)
        assert oracle.route_valid(ids, w, route_scale=1.5)


def test_hash_route_rejects_bad_rows(oracle):
    wr, bias = synth.router(seed=0, layer=0)
    x = synth.token(seed=2)
    for row in ([1, 2, 3, 4, 5, 1], [1, 2, 3, 4, 5, 256], [-1, 2, 3, 4, 5, 6]):
        scores, ids, w = oracle.route_hash(wr, bias, x, np.array(row, np.int64))
        assert ids is None and w is None and scores.shape == (256,)
