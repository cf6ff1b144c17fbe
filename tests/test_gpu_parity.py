"""GPU parity: the HIP path through its C ABI against the CPU oracle on the
same seeded inputs.  EXACT mode must be bit-identical (integer/decode work
and the oracle-order f32 reductions); FAST mode is checked against the
north-star tolerance where it applies (FP8: max-abs 2e-5, RMSE 2e-6) and
otherwise against the reference's own Vulkan gates
(s14_vulkan_numeric.rs:1039 layer 1e-3/1.5e-4, :1347 chain 2e-4/2.5e-5)."""

from __future__ import annotations

import sys

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

from colormlm_amd import _native as N  # noqa: E402
from colormlm_amd import s14, synth  # noqa: E402

HIDDEN, INTER = N.HIDDEN, N.INTER


def say(msg: str) -> None:
    print(f"[gpu-test] {msg}", file=sys.stderr, flush=True)


def dev(a: np.ndarray) -> "torch.Tensor":
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).cuda()
    return torch.from_numpy(a).cuda()


def host(t) -> np.ndarray:
    torch.cuda.synchronize()
    return t.cpu().numpy()


def bits(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def assert_bit_exact(got, want, what):
    g, w = bits(got), bits(want)
    bad = np.flatnonzero(g != w)
    assert bad.size == 0, f"{what}: {bad.size} of {g.size} differ; first {bad[:5]} got {np.asarray(got).reshape(-1)[bad[:3]]} want {np.asarray(want).reshape(-1)[bad[:3]]}"


@pytest.fixture(scope="module")
def ctx():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    say("context on cuda:0")
    c = s14.Context(0)
    yield c
    torch.cuda.synchronize()
    c.destroy()


@pytest.fixture(scope="module")
def pipes(ctx):
    return s14.S14NumericPipelines(ctx)


def mx_parts(page: np.ndarray):
    o = synth.page_offsets("mxfp4")
    return {
        "w1": page[o["w1"]:o["s1"]].reshape(INTER, HIDDEN // 2),
        "s1": page[o["s1"]:o["w3"]].reshape(INTER, HIDDEN // 32),
        "w3": page[o["w3"]:o["s3"]].reshape(INTER, HIDDEN // 2),
        "s3": page[o["s3"]:o["w2"]].reshape(INTER, HIDDEN // 32),
        "w2": page[o["w2"]:o["s2"]].reshape(HIDDEN, INTER // 2),
        "s2": page[o["s2"]:o["total"]].reshape(HIDDEN, INTER // 32),
    }


# --------------------------------------------------------------------------
# synthetic page fill and decoders
# --------------------------------------------------------------------------


def test_device_fill_matches_host_generator(ctx):
    say("fill page seed=3 layer=1 expert=5")
    page = torch.empty(N.EXPERT_PAGE_BYTES, dtype=torch.uint8, device="cuda")
    s14.fill_mxfp4_page(ctx, page, 3, 1, 5)
    assert np.array_equal(host(page), synth.gen_mxfp4_page(3, 1, 5))


def test_dequant_mxfp4_bit_exact_every_byte_and_scale(pipes, oracle):
    say("dequant mxfp4 all codes x all scales")
    n, k = 256, 128
    packed = ((np.arange(n)[:, None] * 7 + np.arange(k // 2)[None, :]) % 256).astype(np.uint8)
    scale = (np.arange(n * 4).reshape(n, 4) % 255).astype(np.uint8)  # every code 0..254
    out = torch.empty((n, k), dtype=torch.float32, device="cuda")
    pipes.dequant_mxfp4(s14.S14MatvecShape(n, k), dev(packed), dev(scale), out)
    assert_bit_exact(host(out), oracle.dequant_mxfp4(packed, scale), "dequant mxfp4")


def test_dequant_fp8_bit_exact_every_code(pipes, oracle):
    say("dequant fp8 all codes")
    n, k = 256, 256
    w = ((np.arange(n)[:, None] + np.arange(k)[None, :]) % 256).astype(np.uint8)
    w[(w & 0x7F) == 0x7F] = 0x7E
    s = np.array([[0, 127], [130, 254]], dtype=np.uint8)
    out = torch.empty((n, k), dtype=torch.float32, device="cuda")
    pipes.dequant_fp8(s14.S14MatvecShape(n, k), dev(w), dev(s), out)
    assert_bit_exact(host(out), oracle.dequant_fp8_ue8m0(w, s), "dequant fp8")


# --------------------------------------------------------------------------
# standalone dispatches (bind / cmd)
# --------------------------------------------------------------------------


@pytest.mark.parametrize("n,k", [(2048, 4096), (4096, 2048), (64, 128), (100, 384), (7, 8192)])
def test_mxfp4_matvec_exact_bit_exact(pipes, oracle, n, k):
    say(f"mxfp4 exact n={n} k={k}")
    packed = synth.gen_bytes(11, 1 + n, n * k // 2).reshape(n, k // 2)
    scale = synth.gen_ue8m0(11, 2 + n, n * k // 32).reshape(n, k // 32)
    x = synth.gen_normal(11, 3 + n, k)
    y = torch.empty(n, dtype=torch.float32, device="cuda")
    shape = s14.S14MatvecShape.new(n, k)
    d = pipes.bind_mxfp4(shape, dev(x), dev(packed), dev(scale), y, mode=s14.EXACT)
    pipes.cmd_mxfp4_matvec(d)
    assert_bit_exact(host(y), oracle.mxfp4_matvec(x, packed, scale), f"mxfp4 exact {n}x{k}")


def test_mxfp4_matvec_exact_slow_decode_paths(pipes, oracle):
    """Scale codes outside the scaled-decode window (tiny and huge), tiny and
    subnormal activations, zeros and infinities in x."""
    say("mxfp4 exact edge codes")
    n, k = 64, 256
    packed = synth.gen_bytes(12, 1, n * k // 2).reshape(n, k // 2)
    scale = synth.gen_ue8m0(12, 2, n * k // 32, -127, 127).reshape(n, k // 32)
    scale[0, :] = 0
    scale[1, :] = 254
    x = synth.gen_normal(12, 3, k)
    x[5] = 0.0
    x[6] = -0.0
    x[7] = np.float32(1e-40)  # subnormal
    x[8] = np.float32(3e-38)
    y = torch.empty(n, dtype=torch.float32, device="cuda")
    d = pipes.bind_mxfp4(s14.S14MatvecShape(n, k), dev(x), dev(packed), dev(scale), y, mode=s14.EXACT)
    pipes.cmd_mxfp4_matvec(d)
    assert_bit_exact(host(y), oracle.mxfp4_matvec(x, packed, scale), "mxfp4 exact edge")


@pytest.mark.parametrize("n,k", [(2048, 4096), (4096, 2048), (100, 384)])
def test_mxfp4_matvec_fast_close(pipes, oracle, n, k):
    say(f"mxfp4 fast n={n} k={k}")
    packed = synth.gen_bytes(13, 1, n * k // 2).reshape(n, k // 2)
    scale = synth.gen_ue8m0(13, 2, n * k // 32).reshape(n, k // 32)
    x = synth.gen_normal(13, 3, k)
    y = torch.empty(n, dtype=torch.float32, device="cuda")
    d = pipes.bind_mxfp4(s14.S14MatvecShape(n, k), dev(x), dev(packed), dev(scale), y, mode=s14.FAST)
    pipes.cmd_mxfp4_matvec(d)
    got, want = host(y), oracle.mxfp4_matvec(x, packed, scale)
    st = oracle.error_stats(got, want)
    say(f"  fast vs oracle {st}")
    # order-changed f32 sums over k terms: bounded by k * eps * sum|terms|
    assert st["max_abs"] < 2e-4 and st["rmse"] < 5e-5


def test_fp8_wq_a_config(pipes, oracle):
    """Config 1: W e4m3 [1024, 4096], f32 128x128 tile scales, bf16 x."""
    say("fp8 wq_a config: exact and fast")
    cfg = synth.config1(seed=0)
    want = oracle.fp8_matvec_f32scale_bf16x(cfg["x_bf16"], cfg["w"], cfg["scale"])
    x = dev(cfg["x_bf16"]).view(torch.bfloat16)
    shape = s14.S14MatvecShape.new(1024, 4096).validate_fp8()
    for mode in (s14.EXACT, s14.FAST):
        y = torch.empty(1024, dtype=torch.float32, device="cuda")
        d = pipes.bind_fp8(shape, x, dev(cfg["w"]), dev(cfg["scale"]), y, mode=mode)
        pipes.cmd_fp8_matvec(d)
        got = host(y)
        if mode == s14.EXACT:
            assert_bit_exact(got, want, "fp8 exact")
        else:
            st = oracle.error_stats(got, want)
            say(f"  fp8 fast vs oracle {st}")
            assert st["max_abs"] <= 2e-5 and st["rmse"] <= 2e-6


# lane quads take k % 1024 == 0 up to 8192 (ragged n included); lane pairs the
# other k % 32 == 0; whole-row lanes the rest
@pytest.mark.parametrize("n,k", [(2048, 4096), (4096, 2048), (200, 1024), (96, 8192), (130, 1056), (129, 130)])
def test_fp8_ue8m0_reference_variant_exact(pipes, oracle, n, k):
    say(f"fp8 ue8m0 f32-x exact n={n} k={k}")
    w = synth.e4m3fn_encode(synth.gen_normal(14, 1, n * k)).reshape(n, k)
    s = synth.gen_ue8m0(14, 2, (-(-n // 128)) * (-(-k // 128)), -7, -5).reshape(-(-n // 128), -(-k // 128))
    x = synth.gen_normal(14, 3, k)
    y = torch.empty(n, dtype=torch.float32, device="cuda")
    # buffers hold whole 4-byte words, as storage_bytes requires (s14_vulkan.rs:124-126)
    w_words = np.zeros(-(-w.size // 4) * 4, dtype=np.uint8)
    w_words[: w.size] = w.reshape(-1)
    s_words = np.zeros(-(-s.size // 4) * 4, dtype=np.uint8)
    s_words[: s.size] = s.reshape(-1)
    d = pipes.bind_fp8(s14.S14MatvecShape(n, k), dev(x), dev(w_words), dev(s_words), y, mode=s14.EXACT)
    pipes.cmd_fp8_matvec(d)
    assert_bit_exact(host(y), oracle.fp8_matvec_ue8m0(x, w, s), "fp8 ue8m0 exact")


def test_fp8_quad_exact_every_code(pipes, oracle):
    """The lane-quad EXACT FP8 matvec (k % 1024 == 0) over every finite e4m3
    code in every byte position of a lane's words, with zeros, -0 and
    subnormal x, and scales small enough that products fall into the f32
    subnormal range: both scale kinds and both x kinds."""
    say("fp8 quad exact: every code, subnormal products")
    n, k = 256, 2048
    w = ((np.arange(n)[:, None] * 5 + np.arange(k)[None, :]) % 256).astype(np.uint8)
    w[(w & 0x7F) == 0x7F] = 0x7E  # the NaN codes
    tiles = (n // 128, k // 128)
    # f32 x with zeros, -0 and subnormals; UE8M0 codes down to 2^-126
    x = synth.gen_normal(16, 1, k)
    x[::97] = 0.0
    x[5::97] = -0.0
    x[11::53] = np.float32(1e-40)
    x[13::61] = np.float32(-3e-39)
    s = (np.arange(tiles[0] * tiles[1]).reshape(tiles) * 17 % 140 + 1).astype(np.uint8)
    s_words = np.zeros(-(-s.size // 4) * 4, dtype=np.uint8)
    s_words[: s.size] = s.reshape(-1)
    y = torch.empty(n, dtype=torch.float32, device="cuda")
    d = pipes.bind_fp8(s14.S14MatvecShape.new(n, k).validate_fp8(), dev(x), dev(w), dev(s_words), y, mode=s14.EXACT)
    pipes.cmd_fp8_matvec(d)
    assert_bit_exact(host(y), oracle.fp8_matvec_ue8m0(x, w, s), "fp8 quad ue8m0 every code")
    # bf16 x with zeros, -0 and subnormals; f32 scales from 2^-120 to 1
    xb = (synth.gen_bytes(16, 2, 2 * k).view(np.uint16) & 0x3FFF) | ((np.arange(k) % 2) << 15).astype(np.uint16)
    xb[::89] = 0x0000
    xb[7::89] = 0x8000
    xb[3::41] = 0x0001 | ((np.arange(k)[3::41] % 2) << 15).astype(np.uint16)
    sf = np.exp2(-(np.arange(tiles[0] * tiles[1]) * 29 % 121)).astype(np.float32).reshape(tiles)
    y2 = torch.empty(n, dtype=torch.float32, device="cuda")
    d2 = pipes.bind_fp8(
        s14.S14MatvecShape.new(n, k).validate_fp8(), dev(xb).view(torch.bfloat16), dev(w), dev(sf), y2, mode=s14.EXACT
    )
    pipes.cmd_fp8_matvec(d2)
    assert_bit_exact(host(y2), oracle.fp8_matvec_f32scale_bf16x(xb, w, sf), "fp8 quad f32-scale bf16-x every code")


def test_swiglu_route_mix_accumulate_bit_exact(pipes, oracle):
    say("swiglu / route_mix / moe_accumulate")
    n = 1 << 20
    g = synth.gen_normal(15, 1, n, 0.0, 8.0)
    u = synth.gen_normal(15, 2, n, 0.0, 8.0)
    g[:6] = [0.0, -0.0, 10.0, 1e30, -200.0, np.nan]
    u[6:8] = [np.nan, 1e20]
    gt, ut, yt = dev(g), dev(u), torch.empty(n, dtype=torch.float32, device="cuda")
    pipes.cmd_swiglu_limit(pipes.bind_swiglu_limit(n, gt, ut, yt))
    assert_bit_exact(host(yt), oracle.swiglu_limit(g, u), "swiglu")
    e = synth.gen_normal(15, 3, 4096)
    acc0 = synth.gen_normal(15, 4, 4096)
    et, rt = dev(e), torch.empty(4096, dtype=torch.float32, device="cuda")
    pipes.cmd_route_mix(pipes.bind_route_mix(4096, 0.17, et, rt))
    assert_bit_exact(host(rt), (np.float32(0.17) * e).astype(np.float32), "route_mix")
    at = dev(acc0)
    pipes.cmd_moe_accumulate(pipes.bind_moe_accumulate(4096, 0.3, et, at))
    assert_bit_exact(host(at), (acc0 + (np.float32(0.3) * e).astype(np.float32)).astype(np.float32), "accumulate")


# --------------------------------------------------------------------------
# fused expert paths
# --------------------------------------------------------------------------


def test_expert_chain_config0(ctx, oracle):
    say("config 0 expert chain exact + fast")
    cfg = synth.config0(seed=0)
    want = oracle.expert_chain(cfg["x"], cfg["page"], float(cfg["route_w"]))
    page, x = dev(cfg["page"]), dev(cfg["x"])
    y = torch.empty(HIDDEN, dtype=torch.float32, device="cuda")
    s14.expert_chain(ctx, page, x, float(cfg["route_w"]), y, mode=s14.EXACT)
    assert_bit_exact(host(y), want, "chain exact")
    s14.expert_chain(ctx, page, x, float(cfg["route_w"]), y, mode=s14.FAST)
    st = oracle.error_stats(host(y), want)
    say(f"  chain fast vs oracle {st}")
    assert st["max_abs"] <= 2e-4 and st["rmse"] <= 2.5e-5


@pytest.mark.parametrize("tiny_x", [False, True])
def test_expert_chain_edge_scale_codes(ctx, oracle, tiny_x):
    """Rows whose scale codes leave the scaled-decode window (tiny scales:
    subnormal products) in w1, w3 and w2, among rows that stay inside, so
    that some wavefronts take the literal decode for all their rows; with
    tiny_x a subnormal activation narrows the window for every row."""
    say(f"expert chain edge codes tiny_x={tiny_x}")
    cfg = synth.config0(seed=3)
    page = cfg["page"].copy()
    o = synth.page_offsets("mxfp4")
    g_up, g_dn = HIDDEN // 32, INTER // 32
    page[o["s1"] + 5 * g_up: o["s1"] + 5 * g_up + 7] = [0, 1, 2, 3, 4, 5, 6]
    page[o["s3"] + 40 * g_up + 100] = 9
    page[o["s1"] + 2047 * g_up + 127] = 1
    page[o["s2"] + 77 * g_dn: o["s2"] + 77 * g_dn + 3] = [3, 0, 8]
    page[o["s2"] + 4095 * g_dn + 63] = 2
    x = cfg["x"].copy()
    if tiny_x:
        x[11] = np.float32(1e-39)
    want = oracle.expert_chain(x, page, float(cfg["route_w"]))
    y = torch.empty(HIDDEN, dtype=torch.float32, device="cuda")
    s14.expert_chain(ctx, dev(page), dev(x), float(cfg["route_w"]), y, mode=s14.EXACT)
    assert_bit_exact(host(y), want, "chain exact edge codes")


@pytest.fixture(scope="module")
def bank(ctx):
    """256 routed MXFP4 pages + 1 MXFP4 shared page of layer 0, on device."""
    say("filling 257-page bank (3.4 GB)")
    pages = torch.empty((257, N.EXPERT_PAGE_BYTES), dtype=torch.uint8, device="cuda")
    for e in range(256):
        s14.fill_mxfp4_page(ctx, pages[e], 0, 0, e)
    s14.fill_mxfp4_page(ctx, pages[256], 0, 0, synth.SHARED_EXPERT)
    table = torch.tensor([pages[e].data_ptr() for e in range(256)], dtype=torch.int64, device="cuda")
    wr, bias = synth.router(seed=0, layer=0)
    torch.cuda.synchronize()
    return {"pages": pages, "table": table, "wr": wr, "bias": bias, "wr_d": dev(wr), "bias_d": dev(bias)}


def page_host(bank, e) -> np.ndarray:
    return host(bank["pages"][e])


def test_moe_layer_route_given(ctx, oracle, bank):
    say("moe layer, route given, mxfp4 shared, exact + fast")
    ids = [126, 12, 205, 149, 227, 174]
    w = np.array([0.3, 0.2, 0.15, 0.15, 0.1, 0.1], dtype=np.float32)
    x = synth.token(seed=1)
    want = oracle.moe_layer(x, [page_host(bank, e) for e in ids], w, page_host(bank, 256))
    y = torch.empty(HIDDEN, dtype=torch.float32, device="cuda")
    routed = [bank["pages"][e] for e in ids]
    s14.moe_layer(ctx, routed, w.tolist(), bank["pages"][256], dev(x), y, mode=s14.EXACT)
    assert_bit_exact(host(y), want, "layer exact")
    s14.moe_layer(ctx, routed, w.tolist(), bank["pages"][256], dev(x), y, mode=s14.FAST)
    st = oracle.error_stats(host(y), want)
    say(f"  layer fast vs oracle {st}")
    assert st["max_abs"] <= 1e-3 and st["rmse"] <= 1.5e-4


def test_moe_layer_fp8_shared_reference_variant(ctx, oracle, bank):
    say("moe layer with the reference's FP8 shared page, exact")
    sh = synth.gen_fp8_page(0, 0)
    ids = [1, 2, 3, 4, 5, 6]
    w = np.full(6, 0.25, dtype=np.float32)  # reference route_scale 1.5
    x = synth.token(seed=2)
    want = oracle.moe_layer(x, [page_host(bank, e) for e in ids], w, sh, shared_fmt="fp8")
    y = torch.empty(HIDDEN, dtype=torch.float32, device="cuda")
    s14.moe_layer(ctx, [bank["pages"][e] for e in ids], w.tolist(), dev(sh), dev(x), y,
                  shared_format=N.S14_PAGE_FP8, mode=s14.EXACT)
    assert_bit_exact(host(y), want, "layer fp8-shared exact")
    s14.moe_layer(ctx, [bank["pages"][e] for e in ids], w.tolist(), dev(sh), dev(x), y,
                  shared_format=N.S14_PAGE_FP8, mode=s14.FAST)
    st = oracle.error_stats(host(y), want)
    say(f"  layer fp8-shared fast vs oracle {st}")
    assert st["max_abs"] <= 1e-3 and st["rmse"] <= 1.5e-4


def test_router_matches_oracle(ctx, oracle, bank):
    say("router sigmoid + sqrt-softplus")
    xs = synth.block_tokens(seed=3, tokens=8)
    router = s14.Router(bank["wr_d"], bank["bias_d"])
    scores = torch.empty((8, 256), dtype=torch.float32, device="cuda")
    ids = torch.empty((8, 6), dtype=torch.int16, device="cuda")
    wts = torch.empty((8, 6), dtype=torch.float32, device="cuda")
    s14.route(ctx, router, 8, dev(xs), scores, ids, wts)
    sc_h, ids_h, w_h = host(scores), host(ids).astype(np.uint16), host(wts)
    for t in range(8):
        s_o, i_o, w_o = oracle.route(bank["wr"], bank["bias"], xs[t])
        assert_bit_exact(sc_h[t], s_o, f"scores t={t}")
        assert ids_h[t].tolist() == i_o.tolist()
        assert_bit_exact(w_h[t], w_o, f"weights t={t}")
    ref = s14.Router(bank["wr_d"], bank["bias_d"], score_fn=N.S14_SCORE_SQRT_SOFTPLUS, route_scale=1.5)
    s14.route(ctx, ref, 1, dev(xs[0]), scores, ids, wts)
    s_o, i_o, w_o = oracle.route(bank["wr"], bank["bias"], xs[0], score_fn=oracle.SCORE_SQRT_SOFTPLUS, route_scale=1.5)
    # exp and log1p are the C library's bit for bit (s14_expf.h, s14_log1pf.h)
    assert_bit_exact(host(scores)[0], s_o, "sqrt-softplus scores")
    assert host(ids).astype(np.uint16)[0].tolist() == i_o.tolist()
    assert_bit_exact(host(wts)[0], w_o, "sqrt-softplus weights")


def test_router_ties_and_expert_counts(ctx, oracle, bank):
    say("router exact ties (lowest index wins) and n_experts < 256")
    x = synth.token(seed=5)
    wr = bank["wr"].copy()
    bias = bank["bias"].copy()
    # four identical rows with identical (large) bias tie for the top places;
    # a fifth pair ties further down the list
    for e in (200, 5, 77, 130):
        wr[e] = wr[42]
        bias[e] = 3.0
    wr[9], bias[9] = wr[250], 2.0
    wr[250], bias[250] = wr[9], 2.0
    scores = torch.empty((1, 256), dtype=torch.float32, device="cuda")
    ids = torch.empty((1, 6), dtype=torch.int16, device="cuda")
    wts = torch.empty((1, 6), dtype=torch.float32, device="cuda")
    for n in (256, 100, 6):
        wr_n, b_n = np.ascontiguousarray(wr[:n]), np.ascontiguousarray(bias[:n])
        router = s14.Router(dev(wr_n), dev(b_n), n_experts=n)
        s14.route(ctx, router, 1, dev(x), scores, ids, wts)
        s_o, i_o, w_o = oracle.route(wr_n, b_n, x)
        assert host(ids).astype(np.uint16)[0].tolist() == i_o.tolist(), f"n={n}"
        assert_bit_exact(host(wts)[0], w_o, f"weights n={n}")
        assert_bit_exact(host(scores)[0][:n], s_o, f"scores n={n}")
    # the tie group occupies the first four places in index order
    _, i_o, _ = oracle.route(wr, bias, x)
    assert i_o.tolist() == [5, 77, 130, 200, 9, 250]


def test_moe_layer_route_config2(ctx, oracle, bank):
    say("config 2 layer with device router, exact + fast")
    x = synth.token(seed=0)
    _, i_o, w_o = oracle.route(bank["wr"], bank["bias"], x)
    want = oracle.moe_layer(x, [page_host(bank, int(e)) for e in i_o], w_o, page_host(bank, 256))
    router = s14.Router(bank["wr_d"], bank["bias_d"])
    y = torch.empty(HIDDEN, dtype=torch.float32, device="cuda")
    ids = torch.empty(6, dtype=torch.int16, device="cuda")
    wts = torch.empty(6, dtype=torch.float32, device="cuda")
    s14.moe_layer_route(ctx, router, bank["table"], bank["pages"][256], dev(x), y, ids, wts, mode=s14.EXACT)
    assert host(ids).astype(np.uint16).tolist() == i_o.tolist()
    assert_bit_exact(host(wts), w_o, "route weights")
    assert_bit_exact(host(y), want, "config2 exact")
    s14.moe_layer_route(ctx, router, bank["table"], bank["pages"][256], dev(x), y, ids, wts, mode=s14.FAST)
    st = oracle.error_stats(host(y), want)
    say(f"  config2 fast vs oracle {st}")
    assert st["max_abs"] <= 1e-3 and st["rmse"] <= 1.5e-4


@pytest.mark.parametrize("tokens", [8, 7, 3, 2])
def test_moe_block_route_config3(ctx, oracle, bank, tokens):
    say(f"config 3 verify block T={tokens}, exact + fast")
    xs = synth.block_tokens(seed=4, tokens=tokens)
    router = s14.Router(bank["wr_d"], bank["bias_d"])
    y = torch.empty((tokens, HIDDEN), dtype=torch.float32, device="cuda")
    ids = torch.empty((tokens, 6), dtype=torch.int16, device="cuda")
    s14.moe_block_route(ctx, tokens, router, bank["table"], bank["pages"][256], dev(xs), y, ids, mode=s14.EXACT)
    got = host(y)
    distinct = s14.last_block_distinct(ctx)
    ids_h = host(ids).astype(np.uint16)
    cache = {}
    shared = page_host(bank, 256)
    for t in range(tokens):
        _, i_o, w_o = oracle.route(bank["wr"], bank["bias"], xs[t])
        assert ids_h[t].tolist() == i_o.tolist()
        for e in i_o:
            if int(e) not in cache:
                cache[int(e)] = page_host(bank, int(e))
        want = oracle.moe_layer(xs[t], [cache[int(e)] for e in i_o], w_o, shared)
        assert_bit_exact(got[t], want, f"block token {t}")
    assert distinct == len(cache)
    say(f"  distinct routed pages D={distinct}")
    s14.moe_block_route(ctx, tokens, router, bank["table"], bank["pages"][256], dev(xs), y, mode=s14.FAST)
    fast = host(y)
    for t in range(tokens):
        assert np.max(np.abs(fast[t] - got[t])) <= 1e-3


def test_moe_block_graph_replays(ctx, bank):
    """An EXACT block captured in a HIP graph (its side-stream half joins the
    capture through the fork/join events), replayed three times with other
    eager block launches and new inputs in between: every replay equals the
    eager launch on the same inputs bit for bit."""
    say("config 3 block T=8 captured in a HIP graph, three replays against eager launches")
    router = s14.Router(bank["wr_d"], bank["bias_d"])
    blocks = [synth.block_tokens(seed=40 + i, tokens=8) for i in range(3)]
    x_static = dev(blocks[0])
    y_graph = torch.empty((8, HIDDEN), dtype=torch.float32, device="cuda")
    y_eager = torch.empty_like(y_graph)

    def launch(x, y):
        s14.moe_block_route(ctx, 8, router, bank["table"], bank["pages"][256], x, y, mode=s14.EXACT)

    launch(x_static, y_graph)  # warm-up outside the capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        launch(x_static, y_graph)
    for i, xs in enumerate(blocks):
        x_static.copy_(dev(xs))
        g.replay()
        torch.cuda.synchronize()
        got = host(y_graph)
        launch(dev(xs), y_eager)  # eager work between the replays, on the same context
        torch.cuda.synchronize()
        assert_bit_exact(got, host(y_eager), f"graph replay {i}")
    del g


def test_moe_block_on_caller_stream(ctx, bank):
    """An EXACT block launched on a caller's own stream (not torch's current
    one), with that stream's earlier work writing the block's input: the side
    stream forks after that work and joins before the output, so the result
    equals the launch on the current stream bit for bit."""
    say("config 3 block T=8 on a caller stream, input written on that stream just before")
    router = s14.Router(bank["wr_d"], bank["bias_d"])
    xs = synth.block_tokens(seed=50, tokens=8)
    y_ref = torch.empty((8, HIDDEN), dtype=torch.float32, device="cuda")
    s14.moe_block_route(ctx, 8, router, bank["table"], bank["pages"][256], dev(xs), y_ref, mode=s14.EXACT)
    torch.cuda.synchronize()
    src = dev(xs)
    x = torch.zeros_like(src)
    y = torch.empty_like(y_ref)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        x.copy_(src)  # the block's input, written on the caller's stream
        s14.moe_block_route(ctx, 8, router, bank["table"], bank["pages"][256], x, y, mode=s14.EXACT,
                            stream=stream.cuda_stream)
    stream.synchronize()
    assert_bit_exact(host(y), host(y_ref), "block on a caller stream")


def test_moe_block_fp8_shared_and_edge_codes(ctx, oracle, bank):
    """Block launches (T=4) with the reference's FP8 shared page, so every
    phase-2 wavefront that serves a routed slot beside the shared one mixes
    MXFP4 and FP8 halves; exact mode against the oracle token by token."""
    tokens = 4
    say(f"config 3 block T={tokens} with FP8 shared page, exact")
    sh = synth.gen_fp8_page(0, 0)
    xs = synth.block_tokens(seed=7, tokens=tokens)
    router = s14.Router(bank["wr_d"], bank["bias_d"])
    y = torch.empty((tokens, HIDDEN), dtype=torch.float32, device="cuda")
    ids = torch.empty((tokens, 6), dtype=torch.int16, device="cuda")
    s14.moe_block_route(ctx, tokens, router, bank["table"], dev(sh), dev(xs), y, ids,
                        shared_format=N.S14_PAGE_FP8, mode=s14.EXACT)
    got, ids_h = host(y), host(ids).astype(np.uint16)
    for t in range(tokens):
        _, i_o, w_o = oracle.route(bank["wr"], bank["bias"], xs[t])
        assert ids_h[t].tolist() == i_o.tolist()
        want = oracle.moe_layer(xs[t], [page_host(bank, int(e)) for e in i_o], w_o, sh, shared_fmt="fp8")
        assert_bit_exact(got[t], want, f"block fp8-shared token {t}")
    # FAST mode's block kernels on the same inputs (FP8 rows in both phases), against the exact result
    s14.moe_block_route(ctx, tokens, router, bank["table"], dev(sh), dev(xs), y, shared_format=N.S14_PAGE_FP8,
                        mode=s14.FAST)
    fast = host(y)
    for t in range(tokens):
        assert np.max(np.abs(fast[t] - got[t])) <= 1e-3


@pytest.mark.parametrize("mode", [s14.EXACT, s14.OFFICIAL])
def test_moe_block_edge_scale_codes(ctx, oracle, bank, mode):
    """Block launches (T=3) whose routed pages carry scale codes outside the
    scaled-decode window in w1, w3 and w2 rows (copies of the chosen pages,
    substituted in the page table), against the oracle on the same pages, in
    EXACT and official mode (whose windows come from the requantised x and h)."""
    tokens = 3
    say(f"config 3 block T={tokens} with out-of-window scale codes, mode={mode}")
    xs = synth.block_tokens(seed=9, tokens=tokens)
    routes = [oracle.route(bank["wr"], bank["bias"], xs[t]) for t in range(tokens)]
    chosen = sorted({int(e) for _, i_o, _ in routes for e in i_o})
    o = synth.page_offsets("mxfp4")
    g_up, g_dn = HIDDEN // 32, INTER // 32
    edited, keep = {}, []
    table = bank["table"].clone()
    for n, e in enumerate(chosen[:4]):
        pg = page_host(bank, e).copy()
        pg[o["s1"] + (3 + 40 * n) * g_up + 5] = 1
        pg[o["s3"] + (700 + n) * g_up: o["s3"] + (700 + n) * g_up + 3] = [0, 2, 4]
        pg[o["s2"] + (33 * n + 1) * g_dn + 60] = 3
        d = dev(pg)
        keep.append(d)
        table[e] = d.data_ptr()
        edited[e] = pg
    router = s14.Router(bank["wr_d"], bank["bias_d"])
    y = torch.empty((tokens, HIDDEN), dtype=torch.float32, device="cuda")
    s14.moe_block_route(ctx, tokens, router, table, bank["pages"][256], dev(xs), y, mode=mode)
    got = host(y)
    shared = page_host(bank, 256)
    layer = oracle.moe_layer_official if mode == s14.OFFICIAL else oracle.moe_layer
    for t, (_, i_o, w_o) in enumerate(routes):
        pages = [edited[int(e)] if int(e) in edited else page_host(bank, int(e)) for e in i_o]
        assert_bit_exact(got[t], layer(xs[t], pages, w_o, shared), f"block edge codes token {t}")


def test_pool_upload_publish_compute_release(ctx, oracle, bank):
    """The page contract end to end on the device: reserve, upload on the copy
    stream, wait the transfer fence, publish, compute from slot addresses,
    release after the compute fence."""
    say("pool upload -> fence -> publish -> layer -> release")
    from colormlm_amd.pool import Fence, GraphProfile, RouteDecision, RouterKind, S14MoePages, VramPool

    routed = VramPool(7, N.EXPERT_PAGE_BYTES, ctx)
    shared = VramPool(1, N.EXPERT_PAGE_BYTES, ctx)
    pages = S14MoePages(routed, shared, GraphProfile.S14_TOP6, shared_format=N.S14_PAGE_MXFP4, weight_sum=1.0)
    ids = [126, 12, 205, 149, 227, 174]
    w = [1 / 6] * 6
    batch = pages.begin_after_official_route(RouteDecision(42, RouterKind.SCORE, ids, w))
    fences = []
    hosts = {}
    for i, p in enumerate(batch.pages()):
        e = ids[i] if i < 6 else 256
        hosts[e] = page_host(bank, e)
        fences.append((routed if i < 6 else shared).upload(ctx, p, hosts[e].tobytes()))
    for f in fences:
        f.wait()
        assert f.is_complete()
    lease = pages.publish_after_transfer_fence(batch)
    slots = [b.slot for b in lease.routed_bindings()]
    ptrs = [routed.slot_ptr(s) for s in slots]
    x = synth.token(seed=5)
    y = torch.empty(HIDDEN, dtype=torch.float32, device="cuda")
    xd = dev(x)
    torch.cuda.synchronize()  # torch's copies are on its stream; the layer runs on the context's
    s14.moe_layer(ctx, ptrs, np.array(w, np.float32).tolist(), shared.slot_ptr(lease.shared_binding().slot), xd, y,
                  mode=s14.EXACT, stream=ctx.compute_stream)
    done = Fence.record(ctx, ctx.compute_stream)
    done.wait()
    pages.release_after_compute_fence(lease)
    want = oracle.moe_layer(x, [hosts[e] for e in ids], np.array(w, np.float32), hosts[256])
    assert_bit_exact(host(y), want, "layer from pool slots")


# ---------------------------------------------------------------------------
# prefill (config 4): e4m3 requant + grouped scaled-MFMA GEMM
# ---------------------------------------------------------------------------


def _requant_edge_rows(k: int) -> np.ndarray:
    """Rows exercising the requant's special cases: zeros and -0 (amax clamp
    to 1e-4), a tiny row, amax/448 an exact power of two (ceil(log2) must not
    round up), values on e4m3 round-half-even midpoints, the subnormal grid,
    NaN (ignored by amax, coded 0x7f) and +-inf-free huge values."""
    rows = [np.zeros(k, np.float32), np.full(k, -0.0, np.float32), np.full(k, 3e-5, np.float32)]
    r = np.linspace(-1.0, 1.0, k, dtype=np.float32)
    r[::32] = 448.0 * 2.0 ** -3  # amax = 56 -> amax / 448 = 2^-3 exactly
    rows.append(r)
    # midpoints between adjacent e4m3 values at scale 1 (amax 448 in each group)
    mids = np.array([1.0625, 1.1875, 3.25 + 0.125, 0.001953125 * 1.5, 0.009765625 * 0.5 + 0.0078125 * 0.5, 240.0 + 8.0],
                    np.float32)
    m = np.resize(mids, k).astype(np.float32)
    m[::32] = 448.0
    m[1::64] *= -1
    rows.append(m)
    sub = (np.arange(k, dtype=np.float32) % 17) * np.float32(2.0 ** -10)  # subnormal e4m3 at scale 1
    sub[::32] = 448.0
    rows.append(sub)
    nan = np.linspace(-3.0, 3.0, k, dtype=np.float32)
    nan[5::97] = np.nan
    rows.append(nan)
    rows.append(np.linspace(-3e30, 3e30, k, dtype=np.float32))
    return np.stack(rows)


def test_requant_e4m3_bit_exact(ctx, oracle):
    say("e4m3 requant (per-32 E8M0) vs oracle, random + edge rows")
    k = 4096
    rng = np.random.default_rng(7)
    rand = rng.standard_normal((56, k)).astype(np.float32)
    rand *= np.float32(2.0) ** rng.integers(-30, 20, size=(56, 1)).astype(np.float32)
    x = np.concatenate([rand, _requant_edge_rows(k)]).astype(np.float32)
    for rows, kk in ((x.shape[0], k), (3, 96), (1, 32)):
        xs = np.ascontiguousarray(x[:rows, :kk])
        q = torch.empty((rows, kk), dtype=torch.uint8, device="cuda")
        sc = torch.empty((rows, kk // 32), dtype=torch.uint8, device="cuda")
        s14.requant_e4m3(ctx, rows, kk, dev(xs), q, sc)
        q_o, s_o = oracle.requant_e4m3(xs)
        assert np.array_equal(host(sc), s_o), f"scales {rows}x{kk}"
        qh = host(q)
        bad = np.argwhere(qh != q_o)
        assert bad.size == 0, f"codes {rows}x{kk}: {len(bad)} differ, first {bad[:3].tolist()}"
    with pytest.raises(N.S14Error):
        s14.requant_e4m3(ctx, 1, 48, dev(x[0, :48]), q, sc)


@pytest.fixture(scope="module")
def prefill_router(bank):
    wr, bias = synth.prefill_router(seed=0, layer=0)
    assert np.array_equal(wr, bank["wr"])
    return {"wr": wr, "bias": bias, "router": s14.Router(bank["wr_d"], dev(bias))}


def _run_prefill(ctx, bank, pr, xs):
    T = xs.shape[0]
    y = torch.empty((T, HIDDEN), dtype=torch.float32, device="cuda")
    ids = torch.empty((T, 6), dtype=torch.int16, device="cuda")
    wts = torch.empty((T, 6), dtype=torch.float32, device="cuda")
    s14.moe_prefill(ctx, T, pr["router"], bank["table"], bank["pages"][256], dev(xs), y, ids, wts)
    return host(y), host(ids).astype(np.uint16), host(wts)


# End-to-end tolerance of the MFMA path against the CPU oracle, relative to
# the output's scale (|y| reaches ~290 here, where one f32 ulp is 3e-5, so an
# absolute 2e-5 gate cannot hold even between two CPU summation orders).
# The GEMMs decode both operands exactly to bf16 and multiply them on the
# bf16 MFMA: every product is exact and only the f32 summation order differs
# from the oracle's (measured: 8.4e-7 of the pair's largest output at worst).
# An h value can still land on the other side of an e4m3 rounding boundary
# from the oracle's when its f32 g/u differ in the last bits (none seen in
# the sampled pairs); one such flip is one e4m3 step of h and would move the
# layer output by that step times a w2 column (~0.5 % of max|y| for a large
# element), which the flip count and the one-step check below bound.
# Gates about 2x the measured worst cases (deterministic runs): end to end
# max_rel 6.4e-7 / rmse_rel 2.5e-7 (tokens 0, 21, 63, 509, 511); GEMM 8.4e-7;
# h flips 0 of 151,552 checked codes.
PREFILL_MAX_REL = 1.5e-6   # max |y - y_ref| / max |y_ref|
PREFILL_RMSE_REL = 5e-7    # rmse(y - y_ref) / rms(y_ref)
GEMM_REL = 2e-6            # a grouped GEMM given the GPU's own operands, vs the oracle's f32 matvec
FLIP_FRACTION = 2e-5       # h codes allowed to differ from the oracle's requant (each by one e4m3 step)


def _prefill_close(oracle, got, want, what):
    st = oracle.error_stats(got, want)
    scale = float(np.max(np.abs(want)))
    rms = float(np.sqrt(np.mean(want.astype(np.float64) ** 2)))
    rel = {"max_rel": st["max_abs"] / scale, "rmse_rel": st["rmse"] / rms}
    say(f"  {what}: max_abs {st['max_abs']:.3g} rmse {st['rmse']:.3g} max|y| {scale:.1f} -> {rel}")
    assert st["finite"]
    assert rel["max_rel"] <= PREFILL_MAX_REL and rel["rmse_rel"] <= PREFILL_RMSE_REL, f"{what}: {rel}"
    return rel


def _e4m3_values(oracle):
    vals = np.array([oracle.e4m3fn(c) for c in range(256)], np.float64)
    finite = np.unique(vals[np.isfinite(vals)])
    return vals, finite


def _check_prefill_stages(oracle, bank, view, xs, ids, wts, y, pairs_to_check):
    """x requant bit-exact; pair bookkeeping; each checked pair's w1/w3 GEMM +
    SwiGLU + h requant (codes equal to the oracle's or one e4m3 step away, at
    most FLIP_FRACTION of them) and w2 GEMM (given the GPU's own h, within
    GEMM_REL); the combine bit-exact for every token."""
    T = xs.shape[0]
    q_o, s_o = oracle.requant_e4m3(xs)
    assert np.array_equal(view["xq"], q_o), "x requant codes"
    assert np.array_equal(view["xs"], s_o), "x requant scales"
    tp, pt = view["token_pair"], view["pair_token"]
    assert view["n_pairs"] == 7 * T
    # pairs grouped by expert ascending, the shared expert's last; token order within an expert
    expert_of = np.empty(7 * T, np.int64)
    for t in range(T):
        for s_ in range(7):
            p = tp[t, s_]
            assert pt[p] == t
            expert_of[p] = ids[t, s_] if s_ < 6 else 256
    assert np.all(np.diff(expert_of) >= 0)
    same = np.diff(expert_of) == 0
    assert np.all(np.diff(pt)[same] > 0)
    # combine: acc = 0; acc += w * down in route order; acc += shared down
    down = view["down"]
    for t in range(T):
        acc = np.zeros(HIDDEN, np.float32)
        for s_ in range(6):
            acc = (acc + np.float32(wts[t, s_]) * down[tp[t, s_]]).astype(np.float32)
        acc = (acc + down[tp[t, 6]]).astype(np.float32)
        assert_bit_exact(y[t], acc, f"combine token {t}")
    vals, grid = _e4m3_values(oracle)
    flips = codes = scale_miss = 0
    worst_gemm = 0.0
    pages = {}
    for p in pairs_to_check:
        e = int(expert_of[p])
        if e not in pages:
            pages[e] = mx_parts(page_host(bank, e))
        m = pages[e]
        t = int(pt[p])
        xd = oracle.dequant_requant(q_o[t], s_o[t])[0]
        h_ref = oracle.swiglu_limit(oracle.mxfp4_matvec(xd, m["w1"], m["s1"]), oracle.mxfp4_matvec(xd, m["w3"], m["s3"]))
        hq_ref, hs_ref = oracle.requant_e4m3(h_ref)
        hq = view["hq"][p]
        ok_scale = view["hs"][p] == hs_ref[0]
        scale_miss += int(np.count_nonzero(~ok_scale))
        in_ok = np.repeat(ok_scale, 32)
        diff = np.flatnonzero((hq != hq_ref[0]) & in_ok)
        steps = np.abs(np.searchsorted(grid, vals[hq[diff]]) - np.searchsorted(grid, vals[hq_ref[0][diff]]))
        assert np.all(steps <= 1), f"pair {p}: h codes more than one e4m3 step off at {diff[steps > 1][:5]}"
        flips += diff.size
        codes += int(np.count_nonzero(in_ok))
        hd = oracle.dequant_requant(hq[None], view["hs"][p][None])[0]
        d_ref = oracle.mxfp4_matvec(hd, m["w2"], m["s2"])
        rel = float(np.max(np.abs(down[p] - d_ref)) / np.max(np.abs(d_ref)))
        worst_gemm = max(worst_gemm, rel)
        assert rel <= GEMM_REL, f"pair {p} (expert {e}, token {t}): w2 GEMM rel {rel:.3g}"
    say(f"  stages: {len(pairs_to_check)} pairs, w2 GEMM worst rel {worst_gemm:.3g}, h flips {flips}/{codes}, "
        f"h scale groups off {scale_miss}")
    assert flips <= FLIP_FRACTION * codes
    assert scale_miss <= 2e-3 * len(pairs_to_check) * 64


def test_prefill_config4_against_oracle(ctx, oracle, bank, prefill_router):
    T = 64
    say(f"config 4 prefill T={T}: routes exact, stages, outputs vs oracle")
    xs = synth.prefill_tokens(seed=0, tokens=T)
    y, ids, wts = _run_prefill(ctx, bank, prefill_router, xs)
    counts = np.zeros(256, np.int64)
    for t in range(T):
        _, i_o, w_o = oracle.route(prefill_router["wr"], prefill_router["bias"], xs[t])
        assert ids[t].tolist() == i_o.tolist(), f"route t={t}"
        assert_bit_exact(wts[t], w_o, f"route weights t={t}")
        counts[i_o] += 1
    st = s14.last_prefill_stats(ctx)
    assert st["distinct"] == int(np.count_nonzero(counts))
    assert st["max_tokens_per_expert"] == int(counts.max())
    assert st["items"] == int(np.sum((counts + 31) // 32)) + (T + 31) // 32
    say(f"  stats {st}")
    view = s14.last_prefill_view(ctx)
    check = sorted({int(p) for t in range(0, T, 8) for p in view["token_pair"][t]})
    _check_prefill_stages(oracle, bank, view, xs, ids, wts, y, check)
    shared = page_host(bank, 256)
    for t in (0, 21, 63):
        want = oracle.moe_prefill_token(xs[t], [page_host(bank, int(e)) for e in ids[t]], wts[t], shared)
        _prefill_close(oracle, y[t], want, f"token {t}")


def test_prefill_config4_512_properties(ctx, oracle, bank, prefill_router):
    """Full config-4 size.  Each token's output depends only on its own row
    (an MFMA column does not see its neighbours), so the first 64 tokens
    must equal a 64-token run bit for bit, whatever tiles and work items the
    grouping gave them; repeat runs are identical; all 512 routes match the
    oracle; and the stages check out for one pair of every 32-token work
    item of the busiest expert (the routes follow Zipf(1.1) popularity, so
    that expert takes about 380 of the 512 tokens: 12 work items streaming
    its page) and for pairs of the shared expert."""
    T = 512
    say(f"config 4 prefill T={T}: properties, stages of the busiest experts")
    xs = synth.prefill_tokens(seed=0, tokens=T)
    y, ids, wts = _run_prefill(ctx, bank, prefill_router, xs)
    st = s14.last_prefill_stats(ctx)
    view = s14.last_prefill_view(ctx)
    counts = np.zeros(256, np.int64)
    for t in range(T):
        _, i_o, w_o = oracle.route(prefill_router["wr"], prefill_router["bias"], xs[t])
        assert ids[t].tolist() == i_o.tolist(), f"route t={t}"
        counts[i_o] += 1
    assert st["distinct"] == int(np.count_nonzero(counts))
    assert st["max_tokens_per_expert"] == int(counts.max())
    assert st["items"] == int(np.sum((counts + 31) // 32)) + (T + 31) // 32
    say(f"  stats {st}; tokens/expert mean {counts[counts > 0].mean():.2f}")
    busiest = int(np.argmax(counts))
    on_busiest = np.flatnonzero((ids == busiest).any(axis=1))
    assert len(on_busiest) >= 300, f"busiest expert has {len(on_busiest)} tokens (Zipf(1.1) head: ~380)"
    firsts = list(on_busiest[::32]) + [on_busiest[-1]]
    check = [int(view["token_pair"][t][list(ids[t]).index(busiest)]) for t in firsts]
    check += [int(view["token_pair"][t][6]) for t in (0, 127, 128, 300, 511)]
    _check_prefill_stages(oracle, bank, view, xs, ids, wts, y, sorted(check))
    y2, ids2, _ = _run_prefill(ctx, bank, prefill_router, xs)
    assert_bit_exact(y2, y, "repeat run")
    assert np.array_equal(ids2, ids)
    y64, ids64, _ = _run_prefill(ctx, bank, prefill_router, np.ascontiguousarray(xs[:64]))
    assert np.array_equal(ids64, ids[:64])
    assert_bit_exact(y64, y[:64], "first 64 tokens of T=512 vs T=64")
    shared = page_host(bank, 256)
    for t in (int(on_busiest[-1]), 511):
        want = oracle.moe_prefill_token(xs[t], [page_host(bank, int(e)) for e in ids[t]], wts[t], shared)
        _prefill_close(oracle, y[t], want, f"token {t}")


def _bf16(a) -> np.ndarray:
    """Round f32 values to bf16 (RNE, torch's cast; the oracle's own bf16
    rounding is pinned to it in tests/test_official.py)."""
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16).to(torch.float32).numpy()


def _bf16_ulp(v) -> np.ndarray:
    """Spacing of bf16 values at |v| (8 significand bits)."""
    _, e = np.frexp(np.abs(np.asarray(v, np.float64)))
    return np.ldexp(1.0, e - 8)


# Official end to end: each expert output and y are rounded to bf16, so an
# f32 difference in the last bits can round one of them to the neighbouring
# bf16 value: a token may differ by up to one bf16 step of its largest
# output (2 at |y| >= 256).  Measured (tokens 0, 2, 4, 32, 63 of seeds 2):
# max-abs <= 0.0625, rmse_rel <= 1.4e-5, most tokens bit-identical.
OFFICIAL_RMSE_REL = 5e-5


def _prefill_close_official(oracle, got, want, what):
    st = oracle.error_stats(got, want)
    scale = float(np.max(np.abs(want)))
    rms = float(np.sqrt(np.mean(want.astype(np.float64) ** 2)))
    bound = PREFILL_MAX_REL * scale + float(_bf16_ulp(scale))
    rel = {"max_rel": st["max_abs"] / scale, "rmse_rel": st["rmse"] / rms}
    say(f"  {what}: max_abs {st['max_abs']:.3g} (bound {bound:.3g}) rmse {st['rmse']:.3g} max|y| {scale:.1f} -> {rel}")
    assert st["finite"]
    assert st["max_abs"] <= bound and rel["rmse_rel"] <= OFFICIAL_RMSE_REL, f"{what}: {rel}"
    return rel


def _run_prefill_official(ctx, bank, pr, xs):
    T = xs.shape[0]
    y = torch.empty((T, HIDDEN), dtype=torch.float32, device="cuda")
    ids = torch.empty((T, 6), dtype=torch.int16, device="cuda")
    wts = torch.empty((T, 6), dtype=torch.float32, device="cuda")
    s14.moe_prefill(ctx, T, pr["router"], bank["table"], bank["pages"][256], dev(xs), y, ids, wts,
                    mode=s14.OFFICIAL)
    return host(y), host(ids).astype(np.uint16), host(wts)


def _check_prefill_official_stages(oracle, bank, view, xs, ids, wts, y, pairs_to_check):
    """Official prefill (executor.py:712-744 on the MFMA path): x act_quant
    (group 128) bit-exact; every token's combine (f32 sum of the bf16 expert
    outputs in route order, shared last, then bf16) bit-exact; each checked
    pair's h (bf16 g and u, SwiGLU times the route weight, bf16, act_quant
    group 128) equal to the oracle's from the same x codes or one e4m3 step
    away, at most FLIP_FRACTION of them; its bf16 w2 output, given the GPU's
    own h, within two bf16 steps plus GEMM_REL of the oracle's."""
    T = xs.shape[0]
    q_o, s_o = oracle.requant_e4m3(xs, 128)
    assert np.array_equal(view["xq"], q_o), "x act_quant codes"
    assert np.array_equal(view["xs"], np.repeat(s_o, 4, axis=1)), "x act_quant scales"
    tp, pt = view["token_pair"], view["pair_token"]
    down = view["down"]
    for t in range(T):
        acc = np.zeros(HIDDEN, np.float32)
        for s_ in range(7):
            acc = (acc + down[tp[t, s_]]).astype(np.float32)
        assert_bit_exact(y[t], _bf16(acc), f"official combine token {t}")
    vals, grid = _e4m3_values(oracle)
    flips = codes = scale_miss = 0
    worst_gemm = 0.0
    pages = {}
    for p in pairs_to_check:
        t = int(pt[p])
        slot = list(tp[t]).index(p)
        e = int(ids[t, slot]) if slot < 6 else 256
        if e not in pages:
            pages[e] = mx_parts(page_host(bank, e))
        m = pages[e]
        w = np.float32(wts[t, slot]) if slot < 6 else np.float32(1.0)
        xd = oracle.dequant_requant(q_o[t], s_o[t], 128)[0]
        g = _bf16(oracle.mxfp4_matvec(xd, m["w1"], m["s1"]))
        u = _bf16(oracle.mxfp4_matvec(xd, m["w3"], m["s3"]))
        h_ref = _bf16((oracle.swiglu_limit(g, u) * w).astype(np.float32))
        hq_ref, hs_ref = oracle.requant_e4m3(h_ref, 128)
        hq, hs = view["hq"][p], view["hs"][p]
        assert np.all(hs.reshape(16, 4) == hs.reshape(16, 4)[:, :1]), f"pair {p}: scales differ within a group of 128"
        ok_scale = hs.reshape(16, 4)[:, 0] == hs_ref[0]
        scale_miss += int(np.count_nonzero(~ok_scale))
        in_ok = np.repeat(ok_scale, 128)
        diff = np.flatnonzero((hq != hq_ref[0]) & in_ok)
        steps = np.abs(np.searchsorted(grid, vals[hq[diff]]) - np.searchsorted(grid, vals[hq_ref[0][diff]]))
        assert np.all(steps <= 1), f"pair {p}: h codes more than one e4m3 step off at {diff[steps > 1][:5]}"
        flips += diff.size
        codes += int(np.count_nonzero(in_ok))
        hd = oracle.dequant_requant(hq[None], hs[None])[0]
        d_ref = oracle.mxfp4_matvec(hd, m["w2"], m["s2"])
        scale = float(np.max(np.abs(d_ref)))
        err = np.abs(down[p].astype(np.float64) - _bf16(d_ref))
        worst_gemm = max(worst_gemm, float(np.max(err / (2.0 * _bf16_ulp(d_ref) + GEMM_REL * scale))))
        assert np.all(err <= 2.0 * _bf16_ulp(d_ref) + GEMM_REL * scale), f"pair {p} (expert {e}, token {t}): w2"
    say(f"  official stages: {len(pairs_to_check)} pairs, w2 worst {worst_gemm:.3g} of its bound, "
        f"h flips {flips}/{codes}, h scale groups off {scale_miss}")
    assert flips <= FLIP_FRACTION * codes
    assert scale_miss <= 2e-3 * len(pairs_to_check) * 16


@pytest.mark.parametrize("tokens", [64, 5])
def test_prefill_official(ctx, oracle, bank, prefill_router, tokens):
    """The official expert semantics on the prefill's MFMA path: routes as the
    default prefill's, the stage checks above, and each checked token's output
    against the oracle's official layer (s14o_moe_layer_official)."""
    say(f"config 4 prefill T={tokens}, official semantics")
    xs = synth.prefill_tokens(seed=2, tokens=tokens)
    y, ids, wts = _run_prefill_official(ctx, bank, prefill_router, xs)
    for t in range(tokens):
        _, i_o, w_o = oracle.route(prefill_router["wr"], prefill_router["bias"], xs[t])
        assert ids[t].tolist() == i_o.tolist(), f"route t={t}"
        assert_bit_exact(wts[t], w_o, f"route weights t={t}")
    view = s14.last_prefill_view(ctx)
    check = sorted({int(p) for t in range(0, tokens, 8) for p in view["token_pair"][t]})
    _check_prefill_official_stages(oracle, bank, view, xs, ids, wts, y, check)
    shared = page_host(bank, 256)
    worst = {"max_rel": 0.0, "rmse_rel": 0.0}
    for t in sorted({0, tokens // 2, tokens - 1}):
        want = oracle.moe_layer_official(xs[t], [page_host(bank, int(e)) for e in ids[t]], wts[t], shared)
        rel = _prefill_close_official(oracle, y[t], want, f"official token {t}")
        worst = {k: max(worst[k], rel[k]) for k in worst}
    say(f"  official end to end worst {worst}")
    y2, _, _ = _run_prefill_official(ctx, bank, prefill_router, xs)
    assert_bit_exact(y2, y, "official repeat run")
    # tokens are independent: a subset's rows equal their rows in the full run
    pick = sorted({0, tokens // 2, tokens - 1})
    y3, ids3, _ = _run_prefill_official(ctx, bank, prefill_router, np.ascontiguousarray(xs[pick]))
    assert np.array_equal(ids3, ids[pick])
    assert_bit_exact(y3, y[pick], f"official rows {pick} vs a {len(pick)}-token run")


@pytest.mark.parametrize("tokens", [1, 5, 1024])
def test_prefill_ragged_and_max_tokens(ctx, oracle, bank, prefill_router, tokens):
    """1 and 5 tokens (partial MFMA column tiles) and the 1024-token maximum:
    each token's row equals its row in a separate run of a different size."""
    say(f"prefill T={tokens} vs per-token consistency")
    xs = synth.prefill_tokens(seed=1, tokens=tokens)
    y, ids, wts = _run_prefill(ctx, bank, prefill_router, xs)
    if tokens <= 5:
        view = s14.last_prefill_view(ctx)
        _check_prefill_stages(oracle, bank, view, xs, ids, wts, y, list(view["token_pair"][tokens - 1]))
    pick = sorted({0, tokens // 2, tokens - 1})
    y1, ids1, _ = _run_prefill(ctx, bank, prefill_router, np.ascontiguousarray(xs[pick]))
    assert np.array_equal(ids1, ids[pick])
    assert_bit_exact(y1, y[pick], f"T={tokens} rows {pick} vs a {len(pick)}-token run")
    with pytest.raises(N.S14Error):
        s14.moe_prefill(ctx, 1025, prefill_router["router"], bank["table"], bank["pages"][256], dev(xs[:1]),
                        torch.empty(1, device="cuda"))


def _boundary_routes(T: int, targets) -> np.ndarray:
    """T rows of six distinct experts in which expert e appears exactly
    targets[e] times (the rest of the 6T slots spread over the other
    experts): each token takes the six experts with the most slots left."""
    left = np.zeros(256, np.int64)
    for e, c in targets.items():
        left[e] = c
    others = [e for e in range(256) if e not in targets]
    rest, k = 6 * T - int(left.sum()), 0
    while rest > 0:
        left[others[k % len(others)]] += 1
        rest -= 1
        k += 1
    rows = np.zeros((T, 6), np.int64)
    for t in range(T):
        order = np.lexsort((np.arange(256), -left))[:6]  # most slots left, lowest id first
        rows[t] = np.sort(order)
        left[order] -= 1
    assert (left == 0).all()
    return rows


def test_prefill_item_width_boundaries(ctx, oracle, bank):
    """The prefill GEMMs run a work item of at most 16 pairs as one 16-column
    half and a wider one as two halves; an expert's tokens split into items
    of 32.  Hash-routed tokens (tid2eid rows built here) give experts exactly
    1, 15, 16, 17, 31, 32, 33, 47, 48 and 49 tokens, so items of 1, 15, 16,
    17, 31 and 32 pairs and every split across the 32 and 16 boundaries
    occur: routes as built, stage checks (h codes, w2 GEMM, combine) on every
    pair of those experts, outputs within the prefill's gates, and the first
    40 tokens of the run equal a 40-token run bit for bit although their
    experts' items (and widths) differ between the two runs."""
    T = 64
    targets = {3: 1, 11: 15, 29: 16, 47: 17, 60: 31, 77: 32, 95: 33, 120: 47, 150: 48, 201: 49}
    say(f"prefill item widths T={T}: expert token counts {sorted(targets.values())}")
    rows = _boundary_routes(T, targets)
    counts = np.bincount(rows.ravel(), minlength=256)
    assert all(counts[e] == c for e, c in targets.items())
    xs = synth.prefill_tokens(seed=3, tokens=T)
    tok = np.arange(T, dtype=np.int32)
    router = s14.Router(bank["wr_d"], bank["bias_d"], tid2eid=torch.from_numpy(rows).cuda(), token_ids=dev(tok))
    y = torch.empty((T, HIDDEN), dtype=torch.float32, device="cuda")
    ids = torch.empty((T, 6), dtype=torch.int16, device="cuda")
    wts = torch.empty((T, 6), dtype=torch.float32, device="cuda")
    s14.moe_prefill(ctx, T, router, bank["table"], bank["pages"][256], dev(xs), y, ids, wts)
    got, ids_h, wts_h = host(y), host(ids).astype(np.int64), host(wts)
    assert (ids_h == rows).all(), "hash routes"
    st = s14.last_prefill_stats(ctx)
    assert st["items"] == int(np.sum((counts + 31) // 32)) + (T + 31) // 32
    view = s14.last_prefill_view(ctx)
    widths = sorted({int(c) for c in view["items"][:, 2]})
    for w in (1, 15, 16, 17, 31, 32):
        assert w in widths, f"no item of {w} pairs: {widths}"
    check = sorted(int(view["token_pair"][t][s_]) for t in range(T) for s_ in range(6) if int(rows[t, s_]) in targets)
    _check_prefill_stages(oracle, bank, view, xs, ids_h, wts_h, got, check)
    shared = page_host(bank, 256)
    for t in (0, 37, 63):
        want = oracle.moe_prefill_token(xs[t], [page_host(bank, int(e)) for e in rows[t]], wts_h[t], shared)
        _prefill_close(oracle, got[t], want, f"token {t}")
    # batch invariance across item widths
    T2 = 40
    y2 = torch.empty((T2, HIDDEN), dtype=torch.float32, device="cuda")
    s14.moe_prefill(ctx, T2, router, bank["table"], bank["pages"][256], dev(np.ascontiguousarray(xs[:T2])), y2)
    assert_bit_exact(host(y2), got[:T2], f"first {T2} tokens of T={T} vs T={T2}")
    ctx.launch_status()


def test_nonresident_page_is_reported_not_read(ctx, oracle, bank, prefill_router):
    """A routed expert whose page-table entry is 0 (not resident): the one-token
    single-launch kernel, a block launch and a prefill each read the shared
    page in its place (mapped memory), write NaN for the tokens that chose it,
    and leave a status that s14_launch_status reports as S14_ERR_INVALID; a
    clean launch afterwards reports S14_OK.  The entry zeroed is one the
    oracle's router picks for token 0."""
    ctx.launch_status()  # clear anything earlier tests left
    router = s14.Router(bank["wr_d"], bank["bias_d"])
    shared = bank["pages"][256]
    xs = synth.block_tokens(seed=21, tokens=4)
    _, i0, _ = oracle.route(bank["wr"], bank["bias"], xs[0])
    gone = int(i0[2])
    table = bank["table"].clone()
    table[gone] = 0
    chose = [gone in oracle.route(bank["wr"], bank["bias"], xs[t])[1].tolist() for t in range(4)]
    say(f"non-resident expert {gone}: K=1 exact, K=1 fast, block T=4, prefill T=4")
    for mode in (s14.EXACT, s14.FAST):
        y = torch.zeros(HIDDEN, dtype=torch.float32, device="cuda")
        s14.moe_layer_route(ctx, router, table, shared, dev(xs[0]), y, mode=mode)
        assert np.isnan(host(y)).all()
        with pytest.raises(s14.S14Error) as err:
            ctx.launch_status()
        assert err.value.code == N.S14_ERR_INVALID
    yb = torch.zeros((4, HIDDEN), dtype=torch.float32, device="cuda")
    s14.moe_block_route(ctx, 4, router, table, shared, dev(xs), yb, mode=s14.EXACT)
    got = host(yb)
    for t in range(4):
        assert np.isnan(got[t]).all() == chose[t] and (chose[t] or not np.isnan(got[t]).any())
    with pytest.raises(s14.S14Error):
        ctx.launch_status()
    yp = torch.zeros((4, HIDDEN), dtype=torch.float32, device="cuda")
    s14.moe_prefill(ctx, 4, prefill_router["router"], table, shared, dev(xs), yp)
    got = host(yp)
    p_chose = [gone in oracle.route(prefill_router["wr"], prefill_router["bias"], xs[t])[1].tolist() for t in range(4)]
    for t in range(4):
        assert np.isnan(got[t]).all() == p_chose[t]
    if any(p_chose):
        with pytest.raises(s14.S14Error):
            ctx.launch_status()
    # a clean launch leaves no status
    y = torch.zeros(HIDDEN, dtype=torch.float32, device="cuda")
    s14.moe_layer_route(ctx, router, bank["table"], shared, dev(xs[0]), y, mode=s14.EXACT)
    ctx.launch_status()
    assert not np.isnan(host(y)).any()


def _tid2eid(vocab: int = 1000, seed: int = 5) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return np.stack([rng.choice(256, 6, replace=False) for _ in range(vocab)]).astype(np.int64)


@pytest.mark.parametrize("score_fn,scale", [(N.S14_SCORE_SIGMOID, 1.0), (N.S14_SCORE_SQRT_SOFTPLUS, 1.5)])
def test_hash_router_layer_block_prefill(ctx, oracle, bank, score_fn, scale):
    """Hash routing (the reference's layers 0-2: experts from tid2eid[token],
    weights from the chosen scores, executor.py:643-667) through the one-token
    layer (exact and fast), a block of 4, the route-only entry point and a
    prefill of 4, against the oracle's hash route and layer, bit for bit
    for both score functions."""
    say(f"hash router score_fn={score_fn} scale={scale}")
    tab_h = _tid2eid()
    tab_d = torch.from_numpy(tab_h).cuda()
    tok = np.array([17, 999, 0, 523], np.int32)
    xs = synth.block_tokens(seed=31, tokens=4)
    router = s14.Router(bank["wr_d"], bank["bias_d"], score_fn=score_fn, route_scale=scale, tid2eid=tab_d,
                        token_ids=dev(tok))
    shared = page_host(bank, 256)
    want, routes = [], []
    for t in range(4):
        sc, i_o, w_o = oracle.route_hash(bank["wr"], bank["bias"], xs[t], tab_h[tok[t]], score_fn=score_fn,
                                         route_scale=scale)
        assert i_o.tolist() == tab_h[tok[t]].tolist()
        routes.append((i_o, w_o))
        want.append(oracle.moe_layer(xs[t], [page_host(bank, int(e)) for e in i_o], w_o, shared))
    # route only
    ids = torch.empty((4, 6), dtype=torch.int16, device="cuda")
    wts = torch.empty((4, 6), dtype=torch.float32, device="cuda")
    s14.route(ctx, router, 4, dev(xs), ids_out=ids, weights_out=wts)
    ids_h, wts_h = host(ids).astype(np.uint16), host(wts)
    for t in range(4):
        assert ids_h[t].tolist() == routes[t][0].tolist()
        assert_bit_exact(wts_h[t], routes[t][1], f"hash weights t={t}")
    # one token (exact, then fast) and a block of 4 (exact)
    y = torch.empty(HIDDEN, dtype=torch.float32, device="cuda")
    s14.moe_layer_route(ctx, router, bank["table"], bank["pages"][256], dev(xs[0]), y, mode=s14.EXACT)
    assert_bit_exact(host(y), want[0], "hash layer exact")
    s14.moe_layer_route(ctx, router, bank["table"], bank["pages"][256], dev(xs[0]), y, mode=s14.FAST)
    st = oracle.error_stats(host(y), want[0])
    assert st["max_abs"] <= 1e-3 and st["rmse"] <= 1.5e-4, st
    yb = torch.empty((4, HIDDEN), dtype=torch.float32, device="cuda")
    s14.moe_block_route(ctx, 4, router, bank["table"], bank["pages"][256], dev(xs), yb, mode=s14.EXACT)
    got = host(yb)
    for t in range(4):
        assert_bit_exact(got[t], want[t], f"hash block t={t}")
    # prefill of the same 4 tokens: routes bit for bit, outputs within the prefill's gates
    yp = torch.empty((4, HIDDEN), dtype=torch.float32, device="cuda")
    pids = torch.empty((4, 6), dtype=torch.int16, device="cuda")
    s14.moe_prefill(ctx, 4, router, bank["table"], bank["pages"][256], dev(xs), yp, ids_out=pids)
    assert (host(pids).astype(np.uint16) == np.stack([r[0] for r in routes])).all()
    gp = host(yp)
    for t in range(4):
        wp = oracle.moe_prefill_token(xs[t], [page_host(bank, int(e)) for e in routes[t][0]], routes[t][1], shared)
        _prefill_close(oracle, gp[t], wp, f"hash prefill token {t}")
    ctx.launch_status()  # every route passed validate_for


def test_hash_router_bad_row_poisons_only_its_token(ctx, oracle, bank):
    """A tid2eid row with a repeated expert, and a token id past the table:
    those tokens' outputs are NaN and s14_launch_status reports
    S14_ERR_ROUTE; the other tokens of the block are exact."""
    tab_h = _tid2eid()
    tab_h[999] = [5, 9, 5, 200, 31, 77]  # repeated expert
    tok = np.array([17, 999, 0, 5000], np.int32)  # 5000 is past the 1000-row table
    xs = synth.block_tokens(seed=33, tokens=4)
    router = s14.Router(bank["wr_d"], bank["bias_d"], tid2eid=torch.from_numpy(tab_h).cuda(), token_ids=dev(tok))
    ctx.launch_status()
    yb = torch.empty((4, HIDDEN), dtype=torch.float32, device="cuda")
    s14.moe_block_route(ctx, 4, router, bank["table"], bank["pages"][256], dev(xs), yb, mode=s14.EXACT)
    got = host(yb)
    shared = page_host(bank, 256)
    for t in (0, 2):
        _, i_o, w_o = oracle.route_hash(bank["wr"], bank["bias"], xs[t], tab_h[tok[t]])
        assert_bit_exact(got[t], oracle.moe_layer(xs[t], [page_host(bank, int(e)) for e in i_o], w_o, shared), f"t={t}")
    assert np.isnan(got[1]).all() and np.isnan(got[3]).all()
    with pytest.raises(s14.S14Error) as err:
        ctx.launch_status()
    assert err.value.code == N.S14_ERR_ROUTE


# --------------------------------------------------------------------------
# official expert semantics (executor.py:712-744, l42_reference.py:390-419)


def _is_bf16(a) -> bool:
    b = bits(a)
    return bool(np.all((b & 0xFFFF) == 0))


def test_official_config2_device_router(ctx, oracle, bank):
    """Config 2 in S14_MODE_OFFICIAL: the device router's route, then each
    linear's activation requantised in groups of 128, bf16 outputs, the route
    weight on h before w2, f32 sum in route order with the shared expert
    last, bf16 layer output; bit for bit against the oracle's official
    layer."""
    say("config 2 official, device router, MXFP4 shared")
    x = synth.token(seed=0)
    _, i_o, w_o = oracle.route(bank["wr"], bank["bias"], x)
    want = oracle.moe_layer_official(x, [page_host(bank, int(e)) for e in i_o], w_o, page_host(bank, 256))
    router = s14.Router(bank["wr_d"], bank["bias_d"])
    y = torch.empty(HIDDEN, dtype=torch.float32, device="cuda")
    ids = torch.empty(6, dtype=torch.int16, device="cuda")
    wts = torch.empty(6, dtype=torch.float32, device="cuda")
    s14.moe_layer_route(ctx, router, bank["table"], bank["pages"][256], dev(x), y, ids, wts, mode=s14.OFFICIAL)
    assert host(ids).astype(np.uint16).tolist() == i_o.tolist()
    assert_bit_exact(host(wts), w_o, "route weights")
    got = host(y)
    assert_bit_exact(got, want, "config2 official")
    assert _is_bf16(got)
    # not the exact mode's layer (the modes must differ)
    exact = oracle.moe_layer(x, [page_host(bank, int(e)) for e in i_o], w_o, page_host(bank, 256))
    assert not np.array_equal(got, exact)


def test_official_route_given_fp8_shared(ctx, oracle, bank):
    """Official layer with a given route and the reference's FP8 shared page
    (e4m3 weights, 128x128 block scales): the FP8 rows see the requantised
    activation too."""
    say("official layer, route given, FP8 shared")
    ids = [126, 12, 205, 149, 227, 174]
    w = np.array([0.3, 0.2, 0.15, 0.15, 0.1, 0.1], dtype=np.float32)
    sh = synth.gen_fp8_page(0, 0)
    x = synth.token(seed=2)
    want = oracle.moe_layer_official(x, [page_host(bank, e) for e in ids], w, sh, shared_fmt="fp8")
    y = torch.empty(HIDDEN, dtype=torch.float32, device="cuda")
    s14.moe_layer(ctx, [bank["pages"][e] for e in ids], w.tolist(), dev(sh), dev(x), y,
                  shared_format=N.S14_PAGE_FP8, mode=s14.OFFICIAL)
    assert_bit_exact(host(y), want, "official fp8 shared")


def test_official_chain_weight_before_w2(ctx, oracle, bank):
    """The expert chain in official mode: one routed expert, its weight on h
    before w2, no shared expert."""
    say("official expert chain")
    cfg = synth.config0(seed=5)
    w = float(cfg["route_w"])
    want = oracle.moe_layer_official(cfg["x"], [cfg["page"]], np.array([w], np.float32), None)
    y = torch.empty(HIDDEN, dtype=torch.float32, device="cuda")
    s14.expert_chain(ctx, dev(cfg["page"]), dev(cfg["x"]), w, y, mode=s14.OFFICIAL)
    assert_bit_exact(host(y), want, "official chain")


@pytest.mark.parametrize("score_fn,scale,tokens", [(N.S14_SCORE_SIGMOID, 1.0, 8),
                                                   (N.S14_SCORE_SQRT_SOFTPLUS, 1.5, 3),
                                                   (N.S14_SCORE_SIGMOID, 1.0, 2)])
def test_official_block(ctx, oracle, bank, score_fn, scale, tokens):
    """Official blocks through the device router, token by token against the
    oracle: ids and weights bit for bit with the oracle's own route (both
    score functions), and the output bit for bit with the oracle's official
    layer evaluated on that route."""
    say(f"official block T={tokens} score_fn={score_fn}")
    xs = synth.block_tokens(seed=9, tokens=tokens)
    router = s14.Router(bank["wr_d"], bank["bias_d"], score_fn=score_fn, route_scale=scale)
    y = torch.empty((tokens, HIDDEN), dtype=torch.float32, device="cuda")
    ids = torch.empty((tokens, 6), dtype=torch.int16, device="cuda")
    wts = torch.empty((tokens, 6), dtype=torch.float32, device="cuda")
    s14.moe_block_route(ctx, tokens, router, bank["table"], bank["pages"][256], dev(xs), y, ids, wts,
                        mode=s14.OFFICIAL)
    got, ids_h, wts_h = host(y), host(ids).astype(np.uint16), host(wts)
    shared = page_host(bank, 256)
    for t in range(tokens):
        _, i_o, w_o = oracle.route(bank["wr"], bank["bias"], xs[t], score_fn=score_fn, route_scale=scale)
        assert ids_h[t].tolist() == i_o.tolist()
        assert_bit_exact(wts_h[t], w_o, f"weights t={t}")
        want = oracle.moe_layer_official(xs[t], [page_host(bank, int(e)) for e in i_o], w_o, shared)
        assert_bit_exact(got[t], want, f"official block t={t}")


def test_official_block_fp8_shared(ctx, oracle, bank):
    """Official block (T=5) with the reference's FP8 shared page: the FP8
    rows of both phases read the requantised x and h, and phase-2 wavefronts
    whose halves mix MXFP4 and FP8 rows round each to bf16; token by token
    against the oracle's official layer on the device's route."""
    tokens = 5
    say(f"official block T={tokens} with FP8 shared page")
    sh = synth.gen_fp8_page(0, 0)
    xs = synth.block_tokens(seed=12, tokens=tokens)
    router = s14.Router(bank["wr_d"], bank["bias_d"])
    y = torch.empty((tokens, HIDDEN), dtype=torch.float32, device="cuda")
    ids = torch.empty((tokens, 6), dtype=torch.int16, device="cuda")
    wts = torch.empty((tokens, 6), dtype=torch.float32, device="cuda")
    s14.moe_block_route(ctx, tokens, router, bank["table"], dev(sh), dev(xs), y, ids, wts,
                        shared_format=N.S14_PAGE_FP8, mode=s14.OFFICIAL)
    got, ids_h, wts_h = host(y), host(ids).astype(np.uint16), host(wts)
    for t in range(tokens):
        _, i_o, w_o = oracle.route(bank["wr"], bank["bias"], xs[t])
        assert ids_h[t].tolist() == i_o.tolist()
        assert_bit_exact(wts_h[t], w_o, f"weights t={t}")
        want = oracle.moe_layer_official(xs[t], [page_host(bank, int(e)) for e in i_o], w_o, sh, shared_fmt="fp8")
        assert_bit_exact(got[t], want, f"official block fp8-shared t={t}")

