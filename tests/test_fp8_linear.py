"""The oracle's activation-quantised FP8 linear (local_s14_primitives/fp8.py:
111-193) and the C-ABI's argument checks for it, on the CPU.

Pinned by: the reference's own known-answer case (test_primitives.py:97-109:
torch.manual_seed(7) codes, UE8M0 scales [[127, 128], [126, 127]], within
rtol = atol = 2e-5 of decoded x @ decoded w.T), reproduced here with the same
torch generator; f64 brute force over ragged shapes and f32 scales; a
construction whose value is fixed in closed form by the group structure
(per-group partials, then acc += partial) and the in-group order (k
ascending); and exact identities (power-of-two scales, sign, bias last,
bf16 output rounding)."""

from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from colormlm_amd import _native as N  # noqa: E402

ONE = 0x38  # e4m3 code of 1.0


def decode_e4m3(codes) -> np.ndarray:
    """Independent decode: torch's float8_e4m3fn view."""
    t = torch.from_numpy(np.ascontiguousarray(codes, np.uint8)).view(torch.float8_e4m3fn)
    return t.float().numpy()


def decode_ue8m0(codes) -> np.ndarray:
    return np.exp2(np.asarray(codes, np.float64) - 127)


def expand(scales, rows, k, row_group):
    s = np.repeat(np.repeat(scales, row_group, 0), 128, 1)
    return s[:rows, :k]


def test_reference_known_answer(oracle):
    torch.manual_seed(7)
    raw_x = torch.randint(0, 255, (2, 130), dtype=torch.uint8)
    raw_w = torch.randint(0, 255, (129, 130), dtype=torch.uint8)
    raw_x[raw_x == 0x7F] = 0x7E
    raw_w[raw_w == 0x7F] = 0x7E
    scale_a = np.array([[127, 128], [126, 127]], np.uint8)
    scale_w = np.array([[127, 128], [126, 127]], np.uint8)
    xd = decode_e4m3(raw_x.numpy()) * expand(decode_ue8m0(scale_a), 2, 130, 1)
    wd = decode_e4m3(raw_w.numpy()) * expand(decode_ue8m0(scale_w), 129, 130, 128)
    expected = (torch.from_numpy(xd.astype(np.float32)) @ torch.from_numpy(wd.astype(np.float32)).T).numpy()
    got = oracle.fp8_linear(raw_x.numpy(), scale_a, raw_w.numpy(), scale_w)
    np.testing.assert_allclose(got, expected, rtol=2e-5, atol=2e-5)


@pytest.mark.parametrize("m,n,k,f32", [(1, 7, 130, False), (3, 200, 384, True), (2, 129, 1000, False)])
def test_f64_brute_force(oracle, m, n, k, f32):
    rng = np.random.default_rng(m * 1000 + k)
    x = rng.integers(0, 256, (m, k), dtype=np.uint8)
    w = rng.integers(0, 256, (n, k), dtype=np.uint8)
    x[(x & 0x7F) == 0x7F] = 0x7E
    w[(w & 0x7F) == 0x7F] = 0x7E
    g = -(-k // 128)
    if f32:
        xs = rng.uniform(0.01, 0.1, (m, g)).astype(np.float32)
        ws = rng.uniform(0.001, 0.01, (-(-n // 128), g)).astype(np.float32)
        xsv, wsv = xs.astype(np.float64), ws.astype(np.float64)
    else:
        xs = rng.integers(118, 130, (m, g), dtype=np.uint8)
        ws = rng.integers(115, 125, (-(-n // 128), g), dtype=np.uint8)
        xsv, wsv = decode_ue8m0(xs), decode_ue8m0(ws)
    bias = rng.standard_normal(n).astype(np.float32)
    xd = decode_e4m3(x).astype(np.float64) * expand(xsv, m, k, 1)
    wd = decode_e4m3(w).astype(np.float64) * expand(wsv, n, k, 128)
    want = xd @ wd.T + bias
    got = oracle.fp8_linear(x, xs, w, ws, bias=bias)
    bound = (np.abs(xd) @ np.abs(wd).T + np.abs(bias)) * (k + 2) * 2.0 ** -23
    assert np.all(np.abs(got - want) <= bound)


def one_row(oracle, x_codes, x_scales, w_codes, w_scales):
    return oracle.fp8_linear(np.array([x_codes], np.uint8), np.array([x_scales], np.uint8),
                             np.array([w_codes], np.uint8), np.array([w_scales], np.uint8))[0, 0]


def test_group_partials_then_add(oracle):
    """Group 0 holds one product 2^24, group 1 two products of 1.  Per-group
    partials give 2^24 + 2 (representable); one flat f32 sum would round
    2^24 + 1 back to 2^24 twice."""
    x = np.zeros(256, np.uint8)
    w = np.zeros(256, np.uint8)
    x[0] = x[128] = x[129] = ONE
    w[0] = w[128] = w[129] = ONE
    assert one_row(oracle, x, [127 + 24, 127], w, [127, 127]) == np.float32(2.0 ** 24 + 2)


def test_in_group_order_k_ascending(oracle):
    """Inside one group: products 2^24, 1, 1 (codes 256 * 256 and 2^-4 * 2^-4
    under scales 2^8 and 1).  k ascending rounds each 1 away (2^24); the same
    products in the other order sum to 2^24 + 2."""
    x = np.zeros(128, np.uint8)
    w = np.zeros(128, np.uint8)
    x[0] = w[0] = 0x78  # 256
    x[1] = x[2] = w[1] = w[2] = 0x18  # 2^-4
    assert one_row(oracle, x, [127 + 8], w, [127]) == np.float32(2.0 ** 24)
    x[[0, 2]] = x[[2, 0]]
    w[[0, 2]] = w[[2, 0]]
    assert one_row(oracle, x, [127 + 8], w, [127]) == np.float32(2.0 ** 24 + 2)


def test_exact_identities(oracle):
    rng = np.random.default_rng(3)
    m, n, k = 3, 70, 512
    x = rng.integers(0, 256, (m, k), dtype=np.uint8)
    w = rng.integers(0, 256, (n, k), dtype=np.uint8)
    x[(x & 0x7F) == 0x7F] = 0x7E
    w[(w & 0x7F) == 0x7F] = 0x7E
    xs = rng.integers(120, 130, (m, 4), dtype=np.uint8)
    ws = rng.integers(118, 126, (1, 4), dtype=np.uint8)
    y = oracle.fp8_linear(x, xs, w, ws)
    # power-of-two scales: every product doubles exactly
    assert np.array_equal(oracle.fp8_linear(x, xs + 1, w, ws), 2 * y)
    # sign: flipping every activation sign negates every product and sum
    assert np.array_equal(oracle.fp8_linear(x ^ 0x80, xs, w, ws), -y)
    # bias added after the groups (f32), bf16 rounding last
    b = rng.standard_normal(n).astype(np.float32)
    yb = oracle.fp8_linear(x, xs, w, ws, bias=b)
    assert np.array_equal(yb, (y + b).astype(np.float32))
    yr = oracle.fp8_linear(x, xs, w, ws, bias=b, round_bf16=True)
    assert np.array_equal(yr, torch.from_numpy(yb).to(torch.bfloat16).float().numpy())
    # zero codes: zero output
    assert not np.any(oracle.fp8_linear(np.zeros_like(x), xs, w, ws))


# -- C-ABI argument checks (no launch happens: every case fails validation) --


def buf(ptr, nbytes):
    return N.Buffer(ptr, nbytes)


def linear(m, n, k, xb, xsb, wb, wsb, yb, bias=None, xsd=N.S14_SCALE_UE8M0, wsd=N.S14_SCALE_UE8M0, flags=0,
           mode=N.S14_MODE_EXACT):
    return N.lib().s14_fp8_linear(C.c_void_p(1), None, m, n, k, xb, xsb, xsd, wb, wsb, wsd,
                                  bias if bias is not None else buf(None, 0), yb, flags, mode)


def test_fp8_linear_argument_checks(native):
    A = 0x10000
    m, n, k = 2, 129, 130
    ok = dict(xb=buf(A, m * k), xsb=buf(A, m * 2), wb=buf(A, n * k), wsb=buf(A, 2 * 2), yb=buf(A, 4 * m * n))
    # each capacity one byte short of its shape (fp8.py:141-171's shape errors)
    for key, short in (("xb", m * k - 1), ("xsb", m * 2 - 1), ("wb", n * k - 1), ("wsb", 3), ("yb", 4 * m * n - 1)):
        args = dict(ok)
        args[key] = buf(A, short)
        assert linear(m, n, k, **args) == N.S14_ERR_CAPACITY, (key, N.last_error())
    args = dict(ok)
    args["xsb"] = buf(A, m * 2 * 4 - 1)
    assert linear(m, n, k, xsd=N.S14_SCALE_F32, **args) == N.S14_ERR_CAPACITY
    assert linear(m, n, k, bias=buf(A, 4 * n - 1), **ok) == N.S14_ERR_CAPACITY
    assert linear(0, n, k, **ok) == N.S14_ERR_SHAPE
    assert linear(m, n, 0, **ok) == N.S14_ERR_SHAPE
    assert linear(m, n, 128 * 1024 + 1, **ok) == N.S14_ERR_SHAPE
    assert linear(m, 1 << 20, 8192, **ok) == N.S14_ERR_SHAPE  # weight bytes past 32-bit offsets
    assert linear(m, n, k, xsd=7, **ok) == N.S14_ERR_INVALID
    assert linear(m, n, k, flags=2, **ok) == N.S14_ERR_INVALID
    assert linear(m, n, k, mode=N.S14_MODE_OFFICIAL, **ok) == N.S14_ERR_INVALID
    args = dict(ok)
    args["xb"] = buf(None, m * k)
    assert linear(m, n, k, **args) == N.S14_ERR_INVALID


def test_act_quant_argument_checks(native):
    L = N.lib()
    ctx = C.c_void_p(1)
    assert L.s14_act_quant_e4m3(ctx, None, 1, 256, 48, 1, 1, 1) == N.S14_ERR_SHAPE  # group not 32/64/128
    assert L.s14_act_quant_e4m3(ctx, None, 1, 192, 128, 1, 1, 1) == N.S14_ERR_SHAPE  # k % group
    assert L.s14_act_quant_e4m3(ctx, None, 0, 256, 128, 1, 1, 1) == N.S14_ERR_SHAPE
    assert L.s14_act_quant_e4m3(ctx, None, 1, 256, 128, None, 1, 1) == N.S14_ERR_INVALID
