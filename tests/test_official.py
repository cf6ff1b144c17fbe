"""The oracle's official expert semantics (executor.py:712-744,
l42_reference.py:390-419) against an independent evaluation, on the CPU.

The independent side takes its roundings from torch (the bfloat16 cast and
the float8_e4m3fn cast, both round-to-nearest-even, which the reference
itself calls) and its dot products from float64 over the dequantised weights
(oracle.dequant_*, pinned bit for bit elsewhere).  The oracle sums each
product in the reference CPU oracle's f32 order, so the two differ only by
that order's rounding before each bf16 rounding: outputs must agree within
one bf16 step everywhere and exactly almost everywhere.  What this pins: the
group-128 requant of every linear's activation, bf16 rounding of every
linear's output, the route weight applied to h before w2 and only for routed
experts, the sum of expert outputs in f32, and the layer's final bf16."""

from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from colormlm_amd import synth  # noqa: E402

H, I = 512, 256  # small hidden / inter: the page layout scales with them


def bf16(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16).float().numpy()


def act_quant(a, group=128):
    """e4m3 with one power-of-two scale per group (torch's float8 cast)."""
    a = np.asarray(a, np.float32).reshape(-1, group)
    amax = np.maximum(np.abs(a).max(1, keepdims=True), np.float32(1e-4)).astype(np.float64)
    e = np.ceil(np.log2(amax / 448.0))
    e = np.where(np.exp2(e - 1) >= amax / 448.0, e - 1, e)  # exact ceil(log2) of the f32 quotient's value
    scale = np.exp2(e).astype(np.float32)
    q = torch.from_numpy(np.clip(a / scale, -448, 448).astype(np.float32)).to(torch.float8_e4m3fn).float().numpy()
    return (q * scale).reshape(-1)


def swiglu(g, u):
    g = np.minimum(g, np.float32(10)).astype(np.float64)
    u = np.clip(u, -10, 10).astype(np.float64)
    return (g / (1 + np.exp(-g)) * u).astype(np.float32)


def weights_of(oracle, page, fmt):
    o = synth.page_offsets(fmt, H, I)
    if fmt == "mxfp4":
        def m(w, s, n, k):
            return oracle.dequant_mxfp4(page[o[w]:o[w] + n * k // 2].reshape(n, k // 2),
                                        page[o[s]:o[s] + n * k // 32].reshape(n, k // 32))
    else:
        def m(w, s, n, k):
            return oracle.dequant_fp8_ue8m0(page[o[w]:o[w] + n * k].reshape(n, k),
                                            page[o[s]:o[s] + (n // 128) * (k // 128)].reshape(n // 128, k // 128))
    return m("w1", "s1", I, H), m("w3", "s3", I, H), m("w2", "s2", H, I)


def expert_independent(oracle, x, page, fmt, weight, routed):
    w1, w3, w2 = weights_of(oracle, page, fmt)
    xq = act_quant(x).astype(np.float64)
    g = bf16(w1.astype(np.float64) @ xq)
    u = bf16(w3.astype(np.float64) @ xq)
    h = swiglu(g, u)
    h = bf16(h * np.float32(weight)) if routed else bf16(h)
    return bf16(w2.astype(np.float64) @ act_quant(h).astype(np.float64))


def close_in_bf16(a, b, frac=0.02):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    step = np.maximum(np.abs(b), 1e-30) * 2.0 ** -7  # one bf16 step (8 significant bits)
    assert np.all(np.abs(a - b) <= step * 1.0001), np.max(np.abs(a - b) / step)
    assert np.mean(a != b) <= frac, np.mean(a != b)


@pytest.mark.parametrize("fmt,routed", [("mxfp4", True), ("mxfp4", False), ("fp8", False)])
def test_expert_official_matches_independent(oracle, fmt, routed):
    page = (synth.gen_mxfp4_page(3, 0, 7, hidden=H, inter=I) if fmt == "mxfp4"
            else synth.gen_fp8_page(3, 0, hidden=H, inter=I, w_std=0.05))
    x = synth.gen_normal(3, 77, H, 0.0, 1.0)
    w = 0.23
    got = oracle.expert_official(x, page, w, routed, fmt, H, I)
    close_in_bf16(got, expert_independent(oracle, x, page, fmt, w, routed))
    assert np.array_equal(got, bf16(got))  # outputs are bf16 values


def test_route_weight_applies_before_w2(oracle):
    """The weight scales h before its bf16 rounding and requant, so the output
    is not the weight times the unweighted output (the chain's order), and a
    routed expert with weight 1 equals the shared form."""
    page = synth.gen_mxfp4_page(4, 0, 9, hidden=H, inter=I)
    x = synth.gen_normal(4, 5, H, 0.0, 1.0)
    one = oracle.expert_official(x, page, 1.0, True, "mxfp4", H, I)
    assert np.array_equal(one, oracle.expert_official(x, page, 1.0, False, "mxfp4", H, I))
    w = np.float32(0.3)
    weighted = oracle.expert_official(x, page, w, True, "mxfp4", H, I)
    assert not np.array_equal(weighted, bf16(w * one))
    close_in_bf16(weighted, expert_independent(oracle, x, page, "mxfp4", w, True))


def test_moe_layer_official_composition(oracle):
    pages = [synth.gen_mxfp4_page(5, 0, e, hidden=H, inter=I) for e in range(6)]
    shared = synth.gen_fp8_page(5, 0, hidden=H, inter=I, w_std=0.05)
    x = synth.gen_normal(5, 1, H, 0.0, 1.0)
    w = np.array([0.4, 0.3, 0.25, 0.2, 0.2, 0.15], np.float32)  # sums to 1.5, the reference's route scale
    y, y32 = oracle.moe_layer_official(x, pages, w, shared, "fp8", H, I, with_f32=True)
    outs = [oracle.expert_official(x, p, wi, True, "mxfp4", H, I) for p, wi in zip(pages, w)]
    outs.append(oracle.expert_official(x, shared, 1.0, False, "fp8", H, I))
    acc = np.zeros(H, np.float32)
    for o in outs:  # f32, route order, shared last
        acc = (acc + o).astype(np.float32)
    assert np.array_equal(y32, acc) and np.array_equal(y, bf16(acc))
    indep = sum(expert_independent(oracle, x, p, "mxfp4", wi, True).astype(np.float64) for p, wi in zip(pages, w))
    indep = bf16(indep + expert_independent(oracle, x, shared, "fp8", 1.0, False))
    close_in_bf16(y, indep, frac=0.05)


def test_act_quant_group_128_bit_exact(oracle):
    """The requant every official linear applies, on its own: group 128
    (l42_reference.py:390-403's default) against torch's float8_e4m3fn cast,
    bit for bit on the dequantised values; group 32 (the prefill's) differs."""
    rng = np.random.default_rng(8)
    x = (rng.standard_normal(4096) * np.exp(rng.uniform(-6, 6, 4096))).astype(np.float32)
    x[:128] *= 1e-7  # a group below the 1e-4 amax floor
    q, sc = oracle.requant_e4m3(x, group=128)
    got = oracle.dequant_requant(q, sc, group=128).reshape(-1)
    want = act_quant(x, 128)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    q32, sc32 = oracle.requant_e4m3(x, group=32)
    assert not np.array_equal(oracle.dequant_requant(q32, sc32, group=32).reshape(-1), want)
