"""GPU parity of the activation-quantised FP8 linear (fp8.py:111-193) at the
adjacent projections' shapes (l42_reference.py:89-102) and of the group-128
activation quant that feeds it (l42_reference.py:390-403).

EXACT is compared bit for bit with the oracle's s14o_fp8_linear (k
ascending inside each 128-k group, then acc += partial).  FAST (MFMA) is
compared with the same oracle within the reference's own tolerance for this
function (test_primitives.py:109: rtol 2e-5), taken relative to the row's
sum of |products| so that cancellation in a row cannot hide or fake an
error."""

from __future__ import annotations

import sys

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from colormlm_amd import s14  # noqa: E402

pytestmark = pytest.mark.gpu

SHAPES = {"wq_b": (32768, 1024), "wkv": (512, 4096), "wo_a": (8192, 4096), "wo_b": (4096, 8192)}


def say(msg: str) -> None:
    print(f"[gpu-test] {msg}", file=sys.stderr, flush=True)


def dev(a: np.ndarray) -> "torch.Tensor":
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t) -> np.ndarray:
    torch.cuda.synchronize()
    return t.cpu().numpy()


@pytest.fixture(scope="module")
def ctx():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    c = s14.Context(0)
    yield c
    torch.cuda.synchronize()
    c.destroy()


def codes(rng, shape) -> np.ndarray:
    c = rng.integers(0, 256, shape, dtype=np.uint8)
    c[(c & 0x7F) == 0x7F] = 0x7E  # no NaN codes (the caller's to reject)
    return c


def weight(n, k, seed):
    rng = np.random.default_rng(seed)
    return codes(rng, (n, k)), rng.integers(114, 122, (-(-n // 128), -(-k // 128)), dtype=np.uint8)


def decoded(oracle, c, scales, row_group):
    n, k = c.shape
    lut = np.array([oracle.e4m3fn(i) for i in range(256)], np.float64)
    s = scales.astype(np.float64) if scales.dtype == np.float32 else np.exp2(scales.astype(np.float64) - 127)
    s = np.repeat(np.repeat(s, row_group, 0), 128, 1)[:n, :k]
    return lut[c] * s


def check_fast(oracle, got, want, x, xs, w, ws, what):
    """|fast - oracle| <= 2e-6 * sum_k |x_k w_k| of the row (f32 summation
    error; measured <= 3.2e-7)."""
    l1 = np.abs(decoded(oracle, x, xs, 1)) @ np.abs(decoded(oracle, w, ws, 128)).T
    err = np.abs(got.astype(np.float64) - want)
    ratio = float(np.max(err / np.maximum(l1, 1e-30)))
    say(f"  {what}: fast max |err| / row L1 = {ratio:.3g}")
    assert np.all(np.isfinite(got)) and ratio <= 2e-6


def test_act_quant_group128_bit_exact(ctx, oracle):
    say("act quant, groups of 128 (and 64, 32)")
    rng = np.random.default_rng(2)
    x = (rng.standard_normal((5, 8192)) * np.exp(rng.uniform(-8, 8, (5, 8192)))).astype(np.float32)
    x[0, :128] *= 1e-9  # below the 1e-4 amax floor
    x[1, 5] = 1e30  # saturating group
    x[2, 7] = np.nan  # ignored by the amax scan
    for group in (128, 64, 32):
        q, s = torch.empty((5, 8192), dtype=torch.uint8, device="cuda"), torch.empty(
            (5, 8192 // group), dtype=torch.uint8, device="cuda")
        s14.act_quant_e4m3(ctx, dev(x), q, s, group=group)
        qo, so = oracle.requant_e4m3(x, group=group)
        assert np.array_equal(host(q), qo) and np.array_equal(host(s), so), group


@pytest.mark.parametrize("m", [1, 4])
@pytest.mark.parametrize("name", list(SHAPES))
def test_fp8_linear_projection_shapes(ctx, oracle, name, m):
    n, k = SHAPES[name]
    say(f"fp8_linear {name} [{n}, {k}] m={m}")
    w, ws = weight(n, k, seed=list(SHAPES).index(name))
    rng = np.random.default_rng(m)
    xf = rng.standard_normal((m, k)).astype(np.float32)
    q = torch.empty((m, k), dtype=torch.uint8, device="cuda")
    qs = torch.empty((m, k // 128), dtype=torch.uint8, device="cuda")
    s14.act_quant_e4m3(ctx, dev(xf), q, qs, group=128)
    xq, xs = host(q), host(qs)
    want = oracle.fp8_linear(xq, xs, w, ws)
    wd, wsd = dev(w), dev(ws)
    y = torch.empty((m, n), dtype=torch.float32, device="cuda")
    s14.fp8_linear(ctx, q, qs, wd, wsd, y, mode=s14.EXACT)
    assert np.array_equal(host(y).view(np.uint32), want.view(np.uint32)), "exact"
    y.fill_(np.nan)
    s14.fp8_linear(ctx, q, qs, wd, wsd, y, mode=s14.FAST)
    fast = host(y)
    check_fast(oracle, fast, want, xq, xs, w, ws, name)
    # a second FAST launch (split-K counters reset by the first) gives the same bits
    s14.fp8_linear(ctx, q, qs, wd, wsd, y, mode=s14.FAST)
    assert np.array_equal(host(y).view(np.uint32), fast.view(np.uint32))


def test_fp8_linear_reference_known_answer_shape(ctx, oracle):
    """test_primitives.py:97-109's shapes and scales (x [2, 130], w [129, 130],
    ragged last group and row tile): both modes run the EXACT kernel here."""
    say("fp8_linear reference KAT shape")
    torch.manual_seed(7)
    raw_x = torch.randint(0, 255, (2, 130), dtype=torch.uint8)
    raw_w = torch.randint(0, 255, (129, 130), dtype=torch.uint8)
    raw_x[raw_x == 0x7F] = 0x7E
    raw_w[raw_w == 0x7F] = 0x7E
    sa = np.array([[127, 128], [126, 127]], np.uint8)
    sw = np.array([[127, 128], [126, 127]], np.uint8)
    want = oracle.fp8_linear(raw_x.numpy(), sa, raw_w.numpy(), sw)
    y = torch.empty((2, 129), dtype=torch.float32, device="cuda")
    for mode in (s14.EXACT, s14.FAST):
        s14.fp8_linear(ctx, raw_x.cuda(), dev(sa), raw_w.cuda(), dev(sw), y, mode=mode)
        assert np.array_equal(host(y).view(np.uint32), want.view(np.uint32)), mode


@pytest.mark.parametrize("m", [1, 3])
def test_fp8_linear_f32_scales_bias_bf16(ctx, oracle, m):
    """f32 scales (fp8.py:37-46's float form), a bias and the official bf16
    output rounding, at wkv's shape (one token: the single-token kernels)."""
    say(f"fp8_linear f32 scales + bias + bf16 output, m={m}")
    n, k = 512, 4096
    rng = np.random.default_rng(9)
    w = codes(rng, (n, k))
    ws = rng.uniform(1e-3, 4e-3, (n // 128, k // 128)).astype(np.float32)
    x = codes(rng, (m, k))
    xs = rng.uniform(1e-2, 3e-2, (m, k // 128)).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    y = torch.empty((m, n), dtype=torch.float32, device="cuda")
    for rb in (False, True):
        want = oracle.fp8_linear(x, xs, w, ws, bias=b, round_bf16=rb)
        s14.fp8_linear(ctx, dev(x), dev(xs), dev(w), dev(ws), y, bias=dev(b), round_bf16=rb, mode=s14.EXACT)
        assert np.array_equal(host(y).view(np.uint32), want.view(np.uint32)), rb
    want = oracle.fp8_linear(x, xs, w, ws, bias=b)
    s14.fp8_linear(ctx, dev(x), dev(xs), dev(w), dev(ws), y, bias=dev(b), mode=s14.FAST)
    got = host(y) - b
    check_fast(oracle, got, (want - b).astype(np.float64), x, xs, w, ws, "f32 scales")


@pytest.mark.parametrize("m,n,k", [(33, 100, 1536), (1, 4000, 512), (8, 96, 16384), (2, 300, 1024), (8, 4096, 8192),
                                   (3, 130, 16384), (1, 4099, 2048), (4, 1000, 4096)])
def test_fp8_linear_fast_edges(ctx, oracle, m, n, k):
    """Row tiles cut by n, two token blocks (m = 33), 12 groups (chunks per
    wavefront 4 or 12), one group-chunk round (k = 512), k = 16384, two
    tokens, and eight tokens at wo_b's shape; for the few-token GEMV, three
    tokens over k = 16384 (two batches of eight chunks) with rows cut by n,
    a last four-row group cut by n, and four tokens at a short n."""
    say(f"fp8_linear fast edges m={m} n={n} k={k}")
    rng = np.random.default_rng(n)
    w, ws = codes(rng, (n, k)), rng.integers(114, 122, (-(-n // 128), k // 128), dtype=np.uint8)
    x, xs = codes(rng, (m, k)), rng.integers(120, 128, (m, k // 128), dtype=np.uint8)
    want = oracle.fp8_linear(x, xs, w, ws)
    y = torch.empty((m, n), dtype=torch.float32, device="cuda")
    s14.fp8_linear(ctx, dev(x), dev(xs), dev(w), dev(ws), y, mode=s14.EXACT)
    assert np.array_equal(host(y).view(np.uint32), want.view(np.uint32))
    s14.fp8_linear(ctx, dev(x), dev(xs), dev(w), dev(ws), y, mode=s14.FAST)
    check_fast(oracle, host(y), want, x, xs, w, ws, f"m={m} n={n} k={k}")


@pytest.mark.parametrize("k", [1024, 2048, 8192])
def test_fp8_linear_exact_one_token_extreme_scales(ctx, oracle, k):
    """The single-token EXACT kernel at each of its four k (4,096 in the
    shape tests) with UE8M0 codes 0..12 mixed with ordinary ones, so that
    products fall to subnormals or zero (the kernel's separate-multiply
    branch; the top of the code range would overflow to inf and NaN, whose
    payloads the CPU and the GPU form differently), rows cut by n; bit for
    bit."""
    say(f"fp8_linear exact m=1 extreme scales k={k}")
    n = 777
    rng = np.random.default_rng(k)
    w, x = codes(rng, (n, k)), codes(rng, (1, k))
    ends = np.arange(0, 13).astype(np.uint8)
    ws = rng.integers(118, 124, (-(-n // 128), k // 128), dtype=np.uint8)
    xs = rng.integers(118, 124, (1, k // 128), dtype=np.uint8)
    sel = rng.random(ws.shape) < 0.4
    ws[sel] = rng.choice(ends, size=int(sel.sum()))
    sel = rng.random(xs.shape) < 0.4
    xs[sel] = rng.choice(ends, size=int(sel.sum()))
    want = oracle.fp8_linear(x, xs, w, ws)
    y = torch.empty((1, n), dtype=torch.float32, device="cuda")
    s14.fp8_linear(ctx, dev(x), dev(xs), dev(w), dev(ws), y, mode=s14.EXACT)
    got = host(y)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), np.count_nonzero(got != want)


def test_fp8_linear_exact_token_chunks(ctx, oracle):
    """EXACT keeps every group partial of a launch in the context's 32 MiB
    workspace: at wq_b's shape (8 groups x 32768 rows x 4 bytes per token)
    40 tokens take two launches of the tiled kernel, 32 tokens then 8."""
    say("fp8_linear exact token chunks: wq_b m=40")
    n, k, m = 32768, 1024, 40
    w, ws = weight(n, k, seed=11)
    rng = np.random.default_rng(12)
    x, xs = codes(rng, (m, k)), rng.integers(120, 128, (m, k // 128), dtype=np.uint8)
    want = oracle.fp8_linear(x, xs, w, ws)
    y = torch.empty((m, n), dtype=torch.float32, device="cuda")
    s14.fp8_linear(ctx, dev(x), dev(xs), dev(w), dev(ws), y, mode=s14.EXACT)
    assert np.array_equal(host(y).view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("m", [129, 512])
def test_fp8_linear_fast_token_blocks_in_several_launches(ctx, oracle, m):
    """wq_b's FAST split-K partials take 8 MiB per 32-token block, so the
    32 MiB workspace holds 4 blocks: 129 tokens run as launches of 96 and 33
    tokens, 512 as four of 128.  Every token's row matches the oracle."""
    n, k = SHAPES["wq_b"]
    say(f"fp8_linear fast wq_b m={m} (several launches)")
    w, ws = weight(n, k, seed=21)
    rng = np.random.default_rng(m)
    x, xs = codes(rng, (m, k)), rng.integers(120, 128, (m, k // 128), dtype=np.uint8)
    want = oracle.fp8_linear(x, xs, w, ws)
    y = torch.full((m, n), np.nan, dtype=torch.float32, device="cuda")
    s14.fp8_linear(ctx, dev(x), dev(xs), dev(w), dev(ws), y, mode=s14.FAST)
    check_fast(oracle, host(y), want, x, xs, w, ws, f"wq_b m={m}")
