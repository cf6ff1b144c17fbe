"""Pin the oracle's decoders and encoders against the reference's own
known-answer vectors (tests/golden/known_answers.json) and against library
routines that implement the same formats (torch's float8_e4m3fn/bfloat16)."""

from __future__ import annotations

import numpy as np
import pytest
import torch


def _bits(v) -> np.ndarray:
    return np.asarray(v, dtype=np.float32).view(np.uint32)


def _unpack(oracle, packed):
    out = []
    for b in packed:
        out += [oracle.e2m1(b & 0x0F), oracle.e2m1(b >> 4)]
    return np.array(out, dtype=np.float32)


def test_e2m1_all_codes_and_container_order(oracle, known_answers):
    case = known_answers["e2m1_all_codes"]
    got = _unpack(oracle, case["packed"])
    assert np.array_equal(_bits(got), _bits(case["values"]))
    assert np.signbit(got[case["negative_zero_index"]])
    case = known_answers["e2m1_container_order"]
    assert np.array_equal(_bits(_unpack(oracle, case["packed"])), _bits(case["values"]))


def test_ue8m0_edges(oracle, known_answers):
    case = known_answers["ue8m0_edges"]
    for code, l2 in zip(case["codes"], case["log2_values"]):
        got = oracle.ue8m0(code)
        assert got == np.float32(np.ldexp(np.float64(1.0), l2)), code
    # code 0 is the f32 subnormal 2^-127, exactly
    assert oracle.ue8m0(0).view(np.uint32) == 0x00400000
    assert np.isinf(oracle.ue8m0(case["nan_code"]))  # rejected upstream; decodes as 2^128
    case = known_answers["ue8m0_known_bits"]
    assert [oracle.ue8m0(c) for c in case["codes"]] == [np.float32(v) for v in case["values"]]


def test_e4m3_known_values_and_torch(oracle, known_answers):
    for key in ("e4m3_known_values", "e4m3_selftest"):
        case = known_answers[key]
        got = np.array([oracle.e4m3fn(c) for c in case["codes"]], dtype=np.float32)
        assert np.array_equal(_bits(got), _bits(case["values"])), key
    # every finite code against torch's OCP float8_e4m3fn decode
    codes = np.array([c for c in range(256) if c not in (0x7F, 0xFF)], dtype=np.uint8)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    got = np.array([oracle.e4m3fn(int(c)) for c in codes], dtype=np.float32)
    assert np.array_equal(_bits(got), _bits(ref))


def test_e4m3_encoder_matches_torch_cast(oracle):
    rng = np.random.default_rng(3)
    vals = np.concatenate(
        [
            rng.normal(0, 0.02, 4000),
            rng.normal(0, 50, 2000),
            rng.uniform(-2**-6, 2**-6, 2000),
            # exact midpoints between adjacent e4m3 values: RNE ties
            [0.5 * (a + b) for a, b in zip(range(1, 8), range(2, 9))],
            [2**-10, 3 * 2**-10, 1.0625, 1.1875, 448.0, -448.0, 0.0, -0.0],
        ]
    ).astype(np.float32)
    vals = vals[np.abs(vals) <= 448]
    ref = torch.from_numpy(vals).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    got = np.array([oracle.e4m3fn_encode(v) for v in vals], dtype=np.uint8)
    assert np.array_equal(got, ref)
    # saturation above the format's maximum
    assert oracle.e4m3fn_encode(1000.0) == 0x7E and oracle.e4m3fn_encode(-1e6) == 0xFE


def test_bf16_encoder_matches_torch(oracle):
    rng = np.random.default_rng(5)
    vals = rng.normal(0, 1, 5000).astype(np.float32)
    ref = torch.from_numpy(vals).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = np.array([oracle.bf16_encode(v) for v in vals], dtype=np.uint16)
    assert np.array_equal(got, ref)


def test_mxfp4_decode_case_from_reference(oracle, known_answers):
    """test_primitives.py:58-72: arange(192) packed codes, the given scale
    table, x = sin(arange(256) * 0.013); the dequantised matrix against the
    closed-form e2m1 * 2^(code-127) and the matvec against float64."""
    case = known_answers["mxfp4_decode_case"]
    packed = np.arange(192, dtype=np.uint8).reshape(3, 64)
    scales = np.array(case["scales"], dtype=np.uint8)
    w = oracle.dequant_mxfp4(packed, scales)
    table = np.array([0, .5, 1, 1.5, 2, 3, 4, 6, -0.0, -.5, -1, -1.5, -2, -3, -4, -6], dtype=np.float64)
    codes = np.empty((3, 128), dtype=np.int64)
    codes[:, 0::2] = packed & 0x0F
    codes[:, 1::2] = packed >> 4
    expect = table[codes] * np.exp2(np.repeat(scales.astype(np.float64) - 127, 32, axis=1))
    assert np.array_equal(w.astype(np.float64), expect)
    x = np.sin(np.arange(256, dtype=np.float32) * np.float32(0.013)).reshape(2, 128)
    for row in x:
        y = oracle.mxfp4_matvec(row, packed, scales)
        ref = expect @ row.astype(np.float64)
        np.testing.assert_allclose(y, ref, rtol=case["rtol"], atol=case["atol"])


def test_dequant_fp8_tiles(oracle):
    rng = np.random.default_rng(9)
    w = rng.integers(0, 255, (200, 130), dtype=np.uint8)
    w[w == 0x7F] = 0x7E
    s = rng.integers(120, 130, (2, 2), dtype=np.uint8)
    got = oracle.dequant_fp8_ue8m0(w, s)
    dec = torch.from_numpy(w).view(torch.float8_e4m3fn).double().numpy()
    sc = np.exp2(s.astype(np.float64) - 127).repeat(128, 0).repeat(128, 1)[:200, :130]
    assert np.array_equal(got.astype(np.float64), dec * sc)
