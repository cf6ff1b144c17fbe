"""Seeded synthetic inputs for the benchmark configurations.

One counter-based generator (SplitMix64 finaliser over (seed, stream,
index)) feeds every config, so the host (numpy, here) and the device fill
kernel (k_fill_page in csrc/s14_device.hip) produce identical integer data.
Normal variates use Box-Muller in float64 and are only drawn on the host;
both the GPU run and the CPU oracle consume the same host arrays.

Configs (the north-star list):
  0  one MXFP4 expert chain, x ~ N(0,1), e2m1 codes uniform, UE8M0 scale
     exponents uniform in [-10, -4], route_w = 0.17
  1  FP8 wq_a [1024 x 4096]: W = e4m3(N(0, 0.02)) RNE-saturated, f32 tile
     scales 2^U(-6, 0), x = bf16(N(0, 1))
  2  top-6 + shared layer: 256 routed MXFP4 pages + 1 shared (MXFP4), router
     W_r ~ N(0, 0.02), bias ~ N(0, 0.01), sigmoid scores
  3  K = 8 verify block through the config-2 layer, adjacent tokens
     correlated (x_t = a x_{t-1} + sqrt(1 - a^2) z_t)
"""

from __future__ import annotations

import functools

import numpy as np

MASK = (1 << 64) - 1
GOLDEN = np.uint64(0x9E3779B97F4A7C15)
C1 = np.uint64(0xBF58476D1CE4E5B9)
C2 = np.uint64(0x94D049BB133111EB)
STEP = np.uint64(0xD1B54A32D192ED03)

HIDDEN = 4096
INTER = 2048
N_EXPERTS = 256
SHARED_EXPERT = 256  # expert index used for the shared page's streams

# stream ids of the non-page inputs
STREAM_X = 1 << 48
STREAM_ROUTER_W = (1 << 48) + 1
STREAM_ROUTER_B = (1 << 48) + 2
STREAM_FP8_W = (1 << 48) + 3
STREAM_FP8_S = (1 << 48) + 4
STREAM_FP8_X = (1 << 48) + 5
STREAM_BLOCK = (1 << 48) + 16  # + token


def _mix64(z: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        z = z + GOLDEN
        z = (z ^ (z >> np.uint64(30))) * C1
        z = (z ^ (z >> np.uint64(27))) * C2
        return z ^ (z >> np.uint64(31))


def stream_key(seed: int, stream: int) -> np.uint64:
    s = _mix64(np.array([stream & MASK], dtype=np.uint64))
    return _mix64(np.array([seed & MASK], dtype=np.uint64) ^ s)[0]


def rand_u64(seed: int, stream: int, index) -> np.ndarray:
    """mix64(mix64(seed ^ mix64(stream)) + index * STEP), vectorised."""
    key = stream_key(seed, stream)
    idx = np.asarray(index, dtype=np.uint64)
    with np.errstate(over="ignore"):
        return _mix64(key + idx * STEP)


def gen_bytes(seed: int, stream: int, n: int) -> np.ndarray:
    words = rand_u64(seed, stream, np.arange((n + 7) // 8, dtype=np.uint64))
    return words.astype("<u8").view(np.uint8)[:n].copy()


def gen_ue8m0(seed: int, stream: int, n: int, lo_exp: int = -10, hi_exp: int = -4) -> np.ndarray:
    span = np.uint64(hi_exp - lo_exp + 1)
    r = rand_u64(seed, stream, np.arange(n, dtype=np.uint64))
    return (127 + lo_exp + (r % span).astype(np.int64)).astype(np.uint8)


def _unit(r: np.ndarray, open_low: bool) -> np.ndarray:
    top = (r >> np.uint64(11)).astype(np.float64)
    return (top + 1.0) * 2.0**-53 if open_low else top * 2.0**-53


def gen_normal(seed: int, stream: int, n: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    i = np.arange(n, dtype=np.uint64)
    u1 = _unit(rand_u64(seed, stream, 2 * i), True)
    u2 = _unit(rand_u64(seed, stream, 2 * i + np.uint64(1)), False)
    z = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
    return (mean + std * z).astype(np.float32)


def gen_log2_uniform(seed: int, stream: int, n: int, lo_exp: float = -6.0, hi_exp: float = 0.0) -> np.ndarray:
    u = _unit(rand_u64(seed, stream, np.arange(n, dtype=np.uint64)), False)
    return np.exp2(lo_exp + (hi_exp - lo_exp) * u).astype(np.float32)


def e4m3fn_encode(v) -> np.ndarray:
    """OCP e4m3fn, round-to-nearest-even, |v| > 448 saturates to 448."""
    v = np.asarray(v, dtype=np.float32)
    sign = np.signbit(v).astype(np.uint8) << 7
    a = np.abs(v).astype(np.float64)
    out = np.zeros(v.shape, dtype=np.uint8)
    sub = a < 2.0**-6
    out[sub] = np.rint(a[sub] * 512.0).astype(np.uint8)  # m * 2^-9, m = 8 is min normal
    nrm = ~sub
    m, e = np.frexp(a[nrm])  # a = m * 2^e, m in [0.5, 1)
    mant = np.rint((m * 2.0 - 1.0) * 8.0)
    e = e - 1 + (mant >= 8)
    mant = np.where(mant >= 8, 0, mant)
    biased = e + 7
    sat = (biased > 15) | ((biased == 15) & (mant >= 7))
    code = np.where(sat, 0x7E, (np.clip(biased, 0, 15) << 3) | mant.astype(np.int64))
    out[nrm] = code.astype(np.uint8)
    nan = np.isnan(v)
    out = out | sign
    out[nan] = 0x7F
    return out


def bf16_encode(v) -> np.ndarray:
    u = np.asarray(v, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = (u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16)
    return r.astype(np.uint16)


def bf16_decode(b) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint32) << 16).view(np.float32)


def page_stream(layer: int, expert: int, part: int) -> int:
    return (layer << 32) | (expert << 8) | part


def page_offsets(fmt: str = "mxfp4", hidden: int = HIDDEN, inter: int = INTER) -> dict:
    if fmt == "mxfp4":
        up_w, up_s = inter * hidden // 2, inter * hidden // 32
        dn_w, dn_s = hidden * inter // 2, hidden * inter // 32
    else:
        up_w, up_s = inter * hidden, -(-inter // 128) * -(-hidden // 128)
        dn_w, dn_s = hidden * inter, -(-hidden // 128) * -(-inter // 128)
    o = {"w1": 0, "s1": up_w}
    o["w3"] = o["s1"] + up_s
    o["s3"] = o["w3"] + up_w
    o["w2"] = o["s3"] + up_s
    o["s2"] = o["w2"] + dn_w
    o["total"] = o["s2"] + dn_s
    return o


def gen_mxfp4_page(seed: int, layer: int, expert: int, lo_exp: int = -10, hi_exp: int = -4,
                   hidden: int = HIDDEN, inter: int = INTER) -> np.ndarray:
    """[w1|s1|w3|s3|w2|s2] with codes uniform and scale exponents uniform in
    [lo_exp, hi_exp]; the same bytes the device fill kernel writes."""
    o = page_offsets("mxfp4", hidden, inter)
    page = np.empty(o["total"], dtype=np.uint8)
    parts = [("w1", "s1", 0), ("w3", "s3", 2), ("w2", "s2", 4)]
    ends = {"w1": o["s1"], "s1": o["w3"], "w3": o["s3"], "s3": o["w2"], "w2": o["s2"], "s2": o["total"]}
    for w, s, part in parts:
        page[o[w]:ends[w]] = gen_bytes(seed, page_stream(layer, expert, part), ends[w] - o[w])
        page[o[s]:ends[s]] = gen_ue8m0(seed, page_stream(layer, expert, part + 1), ends[s] - o[s], lo_exp, hi_exp)
    return page


def gen_fp8_page(seed: int, layer: int, expert: int = SHARED_EXPERT, hidden: int = HIDDEN, inter: int = INTER,
                 w_std: float = 1.0, lo_exp: int = -7, hi_exp: int = -5) -> np.ndarray:
    """Reference-faithful FP8 shared page: e4m3(N(0, w_std)) weights with
    UE8M0 128x128 tile scales, exponents uniform in [lo_exp, hi_exp]."""
    o = page_offsets("fp8", hidden, inter)
    page = np.empty(o["total"], dtype=np.uint8)
    ends = {"w1": o["s1"], "s1": o["w3"], "w3": o["s3"], "s3": o["w2"], "w2": o["s2"], "s2": o["total"]}
    for w, s, part in [("w1", "s1", 0), ("w3", "s3", 2), ("w2", "s2", 4)]:
        n = ends[w] - o[w]
        page[o[w]:ends[w]] = e4m3fn_encode(gen_normal(seed, page_stream(layer, expert, part), n, 0.0, w_std))
        page[o[s]:ends[s]] = gen_ue8m0(seed, page_stream(layer, expert, part + 1), ends[s] - o[s], lo_exp, hi_exp)
    return page


# ---------------------------------------------------------------------------
# configs
# ---------------------------------------------------------------------------


def config0(seed: int = 0):
    return {
        "x": gen_normal(seed, STREAM_X, HIDDEN),
        "page": gen_mxfp4_page(seed, 0, 0),
        "route_w": np.float32(0.17),
    }


def config1(seed: int = 0, n: int = 1024, k: int = HIDDEN):
    w = e4m3fn_encode(gen_normal(seed, STREAM_FP8_W, n * k, 0.0, 0.02)).reshape(n, k)
    tiles = (-(-n // 128), -(-k // 128))
    s = gen_log2_uniform(seed, STREAM_FP8_S, tiles[0] * tiles[1], -6.0, 0.0).reshape(tiles)
    x = bf16_encode(gen_normal(seed, STREAM_FP8_X, k))
    return {"w": w, "scale": s, "x_bf16": x}


def router(seed: int = 0, layer: int = 0):
    wr = gen_normal(seed, STREAM_ROUTER_W + (layer << 8), N_EXPERTS * HIDDEN, 0.0, 0.02).reshape(N_EXPERTS, HIDDEN)
    bias = gen_normal(seed, STREAM_ROUTER_B + (layer << 8), N_EXPERTS, 0.0, 0.01)
    return wr, bias


def token(seed: int = 0, index: int = 0) -> np.ndarray:
    return gen_normal(seed, STREAM_X + index, HIDDEN)


# Correlation of adjacent block tokens: a = 0.315 gives a mean adjacent-token
# top-6 overlap of 9.5 % through the config-2 routers (measured over the
# bench's 64 seeded blocks and 12 layer routers: 0.30 -> 9.3 %, 0.32 -> 9.7 %),
# the 8 / 84 = 9.52 % the reference observed (README.md:92).  Tokens two or
# more apart also share experts by chance (two independent top-6 sets of 256
# share 6 * 6 / 256 = 0.14 experts on average), so a block of 8 reads about
# 41 distinct routed pages, not the 48 - 7 * 6 * 0.095 = 44 that adjacent
# repeats alone would leave.
BLOCK_CORRELATION = 0.315


def block_tokens(seed: int = 0, tokens: int = 8, a: float = BLOCK_CORRELATION) -> np.ndarray:
    """x_t = a x_{t-1} + sqrt(1 - a^2) z_t: marginally N(0,1), adjacent
    tokens correlated so that some routed experts repeat."""
    xs = np.empty((tokens, HIDDEN), dtype=np.float32)
    xs[0] = gen_normal(seed, STREAM_BLOCK, HIDDEN)
    b = np.float32(np.sqrt(1.0 - a * a))
    for t in range(1, tokens):
        z = gen_normal(seed, STREAM_BLOCK + t, HIDDEN)
        xs[t] = np.float32(a) * xs[t - 1] + b * z
    return xs


STREAM_PREFILL = (1 << 48) + (1 << 40)  # + token
STREAM_ZIPF_PERM = (1 << 48) + 32


def prefill_tokens(seed: int = 0, tokens: int = 512) -> np.ndarray:
    """Config 4 activations X[tokens, 4096] ~ N(0, 1), one stream per token."""
    return np.stack([gen_normal(seed, STREAM_PREFILL + t, HIDDEN) for t in range(tokens)])


@functools.lru_cache(maxsize=4)
def zipf_top6_inclusion(s: float = 1.1, n_experts: int = N_EXPERTS, topk: int = 6, samples: int = 40000) -> np.ndarray:
    """P(rank r is among a token's topk experts) when each token draws its
    topk distinct experts with probability proportional to Zipf(s) over
    ranks (sampling without replacement, drawn as the top-k of log p + Gumbel
    noise; seeded Monte Carlo)."""
    rng = np.random.default_rng(0x5A1F)
    logp = -s * np.log(np.arange(1, n_experts + 1, dtype=np.float64))
    hits = np.zeros(n_experts)
    for lo in range(0, samples, 10000):
        g = rng.gumbel(size=(min(10000, samples - lo), n_experts)) + logp
        hits += np.bincount(np.argpartition(-g, topk, axis=1)[:, :topk].ravel(), minlength=n_experts)
    return hits / samples


def prefill_router(seed: int = 0, layer: int = 0, s: float = 1.1, iters: int = 300):
    """Config 4 router: W_r as config 2 and a bias per expert calibrated so
    that top6(sigmoid(W_r x) + bias) over x ~ N(0, 1) picks each expert as
    often as top-6 sampling under Zipf(s) popularity would (experts ranked by
    a seeded permutation).  The calibration nudges each expert's bias by the
    log ratio of its target and observed inclusion rates over 4,096 seeded
    calibration tokens.  Measured on the bench's 512 prefill tokens (seed 0):
    busiest expert 376-389 tokens and 235-243 distinct experts over layers
    0-3, per-expert tokens p50 4 and p90 21-25; pure Zipf(1.1) top-6
    sampling gives 394, 242, 4 and 22 on average."""
    wr, _ = router(seed, layer)
    keys = rand_u64(seed, STREAM_ZIPF_PERM + (layer << 8), np.arange(N_EXPERTS, dtype=np.uint64))
    rank = np.empty(N_EXPERTS, dtype=np.int64)
    rank[np.argsort(keys, kind="stable")] = np.arange(N_EXPERTS)
    target = zipf_top6_inclusion(s)[rank]
    rng = np.random.default_rng([seed & 0xFFFFFFFF, layer, 0x2F])
    xc = rng.standard_normal((4096, HIDDEN), dtype=np.float32)
    scores = 1.0 / (1.0 + np.exp(-(xc @ wr.T).astype(np.float64)))
    bias = 0.05 * np.log(target)
    lt = np.log(target + 1e-4)
    for _ in range(iters):
        top = np.argpartition(-(scores + bias), 6, axis=1)[:, :6]
        seen = np.bincount(top.ravel(), minlength=N_EXPERTS) / scores.shape[0]
        bias += 0.025 * (lt - np.log(seen + 1e-4))
    return wr, bias.astype(np.float32)
