#!/usr/bin/env python3
"""Benchmark of the S14 quantized MoE layer on one MI355X.

Metric: MoE layer us/token and achieved HBM GB/s (% of the
8 TB/s peak) at K=1 and K=8.  A step is one pass of the hot path over one
batch: K=1 is one token through router + top-6 routed + shared MXFP4 experts
(config 2, the headline); K=8 is one speculative-verify block of 8 tokens
(config 3).  Beside them: config 0 (one expert chain), config 1 (the FP8
wq_a matvec) and config 4 (the 512-token prefill).

Every leg times the EXACT (oracle-order, bit-identical) kernels and the FAST
(order-changed) ones.  Each leg's figure is the median of --trials trials;
a trial times exactly --steps steps (after --warmup untimed ones) between
two events on the launch stream, queued behind an untimed pre-roll of the
same steps so that the events bracket the device's work and not the host's
submission.  The
steps of a trial are recorded once into a HIP graph and each trial replays
it (the K=1 and K=8 legs also report eager launches, one host launch
sequence per step).  Inputs are resident in HBM before timing: `--layers`
layer banks of 257 expert pages live in one device arena (a VramPool), and
consecutive steps rotate banks, pages and tokens so that the working set
between reuses (> 1 GB) exceeds the 256 MB MALL; config 1 rotates 96 copies
of its 4 MiB weight.  The `variants` legs time the reference's published
layer configuration (route given, FP8 shared page), official expert
semantics at K=1 and K=8, a hash-routed layer and a MALL-resident layer.

Prints one JSON line.
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "MoE layer µs/token + achieved HBM GB/s (% peak) at K=1 and K=8, 1 MI355X"
HBM_PEAK_GBPS = 8000.0

PAGE = 13_369_344
UP = 2 * (4_194_304 + 262_144)  # w1 + s1 + w3 + s3
DOWN = 4_194_304 + 262_144  # w2 + s2
ROUTER = 256 * 4096 * 4 + 256 * 4
X_BYTES = 4096 * 4
H_BYTES = 2048 * 4
CHAIN_BYTES = PAGE + 2 * X_BYTES  # config 0: page, x in, y out
WQA_N, WQA_K = 1024, 4096
WQA_BYTES = WQA_N * WQA_K + 8 * 32 * 4 + WQA_K * 2 + WQA_N * 4  # config 1: W, f32 tile scales, bf16 x, f32 y
WQA_COPIES = 96


def layer_bytes_k1() -> int:
    # 6 routed + 1 shared page, router weights + bias, x in, y out
    return 7 * PAGE + ROUTER + X_BYTES + X_BYTES


def block_bytes(distinct: float, tokens: int, shared_page: int = PAGE) -> float:
    # each distinct routed page (D, the measured mean) and the shared page once; router once; x, y per token
    return distinct * PAGE + shared_page + ROUTER + tokens * 2 * X_BYTES


PREFILL_TOKENS = 512
BF16_MFMA_PEAK_TFLOPS = 2500.0  # dense bf16: the prefill GEMMs run v_mfma_f32_32x32x16_bf16 on exactly decoded operands


def prefill_bytes(distinct: float, tokens: int) -> float:
    # each distinct routed page and the shared page once; router once; x in, y out
    return (distinct + 1) * PAGE + ROUTER + tokens * 2 * X_BYTES


def prefill_flops(tokens: int) -> int:
    # 7 experts per token, w1 + w3 + w2 (3 x 2048 x 4096 MACs each), plus the router
    return tokens * (7 * 3 * 2 * 2048 * 4096 + 2 * 256 * 4096)


def phase1_bytes(pairs: int, tokens: int) -> int:
    # w1/s1/w3/s3 of every (token, expert) pair as launched, x read, h written
    return pairs * UP + tokens * X_BYTES + pairs * H_BYTES


LEGS = ("k1", "k8", "config0", "config1", "variants", "prefill", "linear", "upload")


def parse():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200, help="timed steps per trial")
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--trials", type=int, default=5, help="trials per leg; each leg reports the median")
    ap.add_argument("--mode", choices=["exact", "fast"], default="exact")
    ap.add_argument("--layers", type=int, default=12, help="layer banks of 257 pages rotated across steps")
    ap.add_argument("--tokens", type=int, default=64, help="distinct tokens rotated across steps")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--profile-steps", type=int, default=64)
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="bound on the CPU baseline's work per config")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain 256 MiB device copy 10 times (the known-size kernel that "
                         "scales the FETCH_SIZE / WRITE_SIZE counters) and exit")
    ap.add_argument("--prefill-steps", type=int, default=20)
    ap.add_argument("--only", default="all",
                    help="restrict the timed work (for profiler runs): a comma-separated subset of " + ",".join(LEGS))
    return ap.parse_args()


def progress(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


class Timer:
    """Median-of-trials timing of a step function on torch's current stream
    (the stream the library launches on).

    Each trial first queues a pre-roll, the same steps once more, untimed,
    then the start event, the trial's steps and the end event.  The device
    is still running the pre-roll while the host submits the timed steps, so
    the two events bracket the device's work alone, as the reference's
    timestamps do (s14_vulkan_numeric.rs:1088-1101), and a trial's figure
    depends little on how many steps it holds (what is left is one kernel
    boundary per event, ~9 us per trial).  A trial whose start event had
    already completed when the host finished submitting (the device idled
    waiting for work) is discarded and rerun with a longer pre-roll, up to
    three times; after that it is kept and the figure is flagged
    (submission_covered false: the host's launch rate paced the device)."""

    def __init__(self, torch, trials: int, warm_ms: float = 100.0):
        self.torch = torch
        self.trials = max(1, trials)
        self.warm_ms = warm_ms

    def _trials(self, preroll, submit) -> tuple:
        """Per-trial (device ms between the events, host submission ms), the
        pre-roll repeats used and whether every trial's submission was
        covered.  Before the first trial the pre-roll runs back to back for
        warm_ms of wall time: after an idle spell the device's first
        milliseconds of work run slower (a 20-step K=1 trial measured 43.1
        us/step right after one second idle and 42.2 after 100 ms busy)."""
        torch = self.torch
        t0 = time.perf_counter()
        while True:
            preroll()
            torch.cuda.synchronize()
            if (time.perf_counter() - t0) * 1e3 >= self.warm_ms:
                break
        per, host = [], []
        n, attempts, covered_all = 1, 0, True
        while len(per) < self.trials:
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            for _ in range(n):
                preroll()
            start.record()
            t0 = time.perf_counter()
            submit()
            end.record()
            host_ms = (time.perf_counter() - t0) * 1e3
            covered = not start.query()
            torch.cuda.synchronize()
            if not covered and attempts < 3:
                # the device idled waiting for the host: a longer pre-roll,
                # unless the host's launch rate is what paces the device
                attempts += 1
                n *= 2
                continue
            covered_all &= covered
            per.append(start.elapsed_time(end))
            host.append(host_ms)
        return per, host, n, covered_all

    @staticmethod
    def _summary(per: list, host: list, n: int, covered: bool, units: int, **extra) -> dict:
        per = [p / units for p in per]
        out = {"ms": statistics.median(per), "ms_min": min(per), "ms_max": max(per), "trials": len(per),
               "host_submit_ms_max": max(host), "preroll_repeats": n, "submission_covered": covered}
        out.update(extra)
        return out

    def run(self, fn, steps: int, warmup: int) -> dict:
        """Eager: the host launches every step inside the trial."""
        torch = self.torch
        steps = max(1, steps)
        for i in range(warmup):
            fn(i)
        torch.cuda.synchronize()
        k = [warmup]

        def submit():
            for i in range(steps):
                fn(k[0] + i)
            k[0] += steps

        per, host, n, cov = self._trials(submit, submit)
        return self._summary(per, host, n, cov, steps, steps_per_trial=steps, timing="eager launches")

    def run_graph(self, fn, launches: int, warmup: int) -> dict:
        """Median per-launch time of `launches` calls captured in one HIP
        graph and replayed once per trial.  The pre-roll is a second graph
        of the next `launches` steps (other layer banks, pages and tokens),
        so that a trial does not find the previous trial's inputs in the
        MALL however few steps it holds."""
        torch = self.torch
        for i in range(max(1, warmup)):
            fn(i)
        torch.cuda.synchronize()
        graphs = []
        for base in (0, launches):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for i in range(launches):
                    fn(base + i)
            g.replay()  # the first replay uploads the graph
            graphs.append(g)
        torch.cuda.synchronize()
        per, host, n, cov = self._trials(graphs[1].replay, graphs[0].replay)
        del graphs
        return self._summary(per, host, n, cov, launches, launches_per_trial=launches, timing="hip graph replay")


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one MI355X only; --gpus {args.gpus} is not supported "
              "(the S14 path is single-GPU; multi-GPU sharding is design-only)", file=sys.stderr)
        return 2
    only = set(args.only.split(","))
    bad = only - set(LEGS) - {"all"}
    if bad:
        print(f"unknown --only legs {sorted(bad)}; choose from {', '.join(LEGS)} or all", file=sys.stderr)
        return 2
    if "all" in only:
        only = set(LEGS)

    import numpy as np
    import torch

    from colormlm_amd import _native as N
    from colormlm_amd import s14, synth
    from colormlm_amd.pool import VramPool

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    torch.cuda.init()
    if args.copy_calibration:
        return copy_calibration(torch)
    ctx = s14.Context(0)
    NL, P = args.layers, args.tokens
    timer = Timer(torch, args.trials)

    # ---- resident inputs ----
    progress(f"filling {NL} x 257 expert pages")
    bank = VramPool(NL * 257, N.EXPERT_PAGE_BYTES, ctx)
    for L in range(NL):
        for e in range(257):
            s14.fill_mxfp4_page(ctx, bank.slot_ptr(L * 257 + e), args.seed, L, e if e < 256 else synth.SHARED_EXPERT)
    tables = torch.tensor([[bank.slot_ptr(L * 257 + e) for e in range(256)] for L in range(NL)],
                          dtype=torch.int64, device="cuda")
    shared = [bank.slot_ptr(L * 257 + 256) for L in range(NL)]
    pages_flat = [bank.slot_ptr(i) for i in range(NL * 257)]
    routers_h = [synth.router(args.seed, L) for L in range(NL)]
    wr = torch.stack([torch.from_numpy(w) for w, _ in routers_h]).cuda()
    bias = torch.stack([torch.from_numpy(b) for _, b in routers_h]).cuda()
    routers = [s14.Router(wr[L], bias[L]) for L in range(NL)]
    X = torch.from_numpy(np.stack([synth.token(args.seed, i) for i in range(P)])).cuda()
    XB = torch.from_numpy(np.stack([synth.block_tokens(args.seed + 1000 + i, 8) for i in range(P)])).cuda()
    Y = torch.empty(4096, dtype=torch.float32, device="cuda")
    YB = torch.empty((8, 4096), dtype=torch.float32, device="cuda")
    IDS = torch.empty((8, 6), dtype=torch.int16, device="cuda")
    torch.cuda.synchronize()

    def step_k1(m):
        def f(i):
            L = i % NL
            s14.moe_layer_route(ctx, routers[L], tables[L], shared[L], X[i % P], Y, mode=m)
        return f

    def step_k8(m):
        def f(i):
            L = i % NL
            s14.moe_block_route(ctx, 8, routers[L], tables[L], shared[L], XB[i % P], YB, mode=m)
        return f

    def step_chain(m):
        def f(i):
            # a different page (and layer bank) every step: > 1 GB between reuses
            page = pages_flat[(i * 37) % len(pages_flat)]
            s14.expert_chain(ctx, page, X[i % P], 0.17, Y, mode=m)
        return f

    def stages(fn, steps):
        ctx.enable_stage_timing(True)
        acc = np.zeros(3)
        for i in range(steps):
            fn(i)
            acc += np.array(ctx.stage_times())
        ctx.enable_stage_timing(False)
        return (acc / steps).tolist()

    def block_routes(m):
        """Distinct routed pages and the adjacent-token top-6 overlap of the
        bench's blocks, from the routes the device itself chose."""
        ds, ov = [], []
        for i in range(min(P, 32)):
            L = i % NL
            s14.moe_block_route(ctx, 8, routers[L], tables[L], shared[L], XB[i % P], YB, ids_out=IDS, mode=m)
            ds.append(s14.last_block_distinct(ctx))
            ids = [set(int(v) for v in row) for row in IDS.cpu().numpy().astype(np.int64) & 0xffff]
            ov += [len(ids[t] & ids[t - 1]) / 6.0 for t in range(1, 8)]
        return float(np.mean(ds)), float(np.mean(ov))

    out = {}
    for name, m in (("exact", s14.EXACT), ("fast", s14.FAST)):
        r = {}
        if "k1" in only:
            progress(f"config 2 (K=1) {name}")
            t = timer.run_graph(step_k1(m), args.steps, args.warmup)
            t["eager"] = timer.run(step_k1(m), args.steps, args.warmup)
            st = stages(step_k1(m), args.profile_steps)
            us = t["ms"] * 1e3
            r["k1"] = {"us_per_token": us, "timing": t, "hbm_gbps": layer_bytes_k1() / (us * 1e-6) / 1e9,
                       "stage_ms": {"route": st[0], "phase1": st[1], "phase2": st[2]}}
            r["k1"]["hbm_frac"] = r["k1"]["hbm_gbps"] / HBM_PEAK_GBPS
        if "k8" in only:
            progress(f"config 3 (K=8) {name}")
            t = timer.run_graph(step_k8(m), max(args.steps // 4, 10), max(args.warmup // 4, 5))
            t["eager"] = timer.run(step_k8(m), max(args.steps // 4, 10), max(args.warmup // 4, 5))
            st = stages(step_k8(m), max(args.profile_steps // 4, 8))
            d, ov = block_routes(m)
            ms = t["ms"]
            r["k8"] = {"us_per_token": ms * 1e3 / 8, "ms_per_block": ms, "timing": t, "distinct_pages": d,
                       "adjacent_overlap": ov, "hbm_gbps": block_bytes(d, 8) / (ms * 1e-3) / 1e9,
                       "stage_ms": {"route": st[0], "phase1": st[1], "phase2": st[2]}}
            if name == "exact":
                r["k8"]["stage_note"] = ("phase1/phase2: the kernels of the half of the pairs on the caller's "
                                         "stream (phase2 up to the combine's end); the other half runs beside "
                                         "them on the context's side stream")
            r["k8"]["hbm_frac"] = r["k8"]["hbm_gbps"] / HBM_PEAK_GBPS
        if "config0" in only:
            progress(f"config 0 (chain) {name}")
            t = timer.run_graph(step_chain(m), args.steps, args.warmup)
            st = stages(step_chain(m), args.profile_steps)
            us = t["ms"] * 1e3
            r["config0"] = {"us_per_chain": us, "timing": t, "hbm_gbps": CHAIN_BYTES / (us * 1e-6) / 1e9,
                            "stage_ms": {"phase1": st[1], "phase2": st[2]}, "algorithmic_bytes": CHAIN_BYTES}
            r["config0"]["hbm_frac"] = r["config0"]["hbm_gbps"] / HBM_PEAK_GBPS
        out[name] = r

    if "config1" in only:
        progress("config 1 (wq_a fp8)")
        c1 = bench_config1(args, ctx, timer, torch, np, s14, synth)
        for name in ("exact", "fast"):
            out[name]["config1"] = c1[name]

    variants = None
    if "variants" in only:
        progress("layer variants: reference layer, official, hash-routed, MALL-resident")
        variants = bench_variants(args, ctx, timer, torch, np, s14, synth, N, bank, tables, shared, routers_h, wr,
                                  bias, X, XB, NL, P, stages)
    prefill = None
    if "prefill" in only:
        progress("config 4 (prefill)")
        prefill = bench_prefill(args, ctx, tables, shared, NL, torch, np, s14, synth)
    linear = None
    if "linear" in only:
        progress("adjacent FP8 projections (fp8_linear)")
        linear = bench_linear(args, ctx, timer, torch, s14)
    upload = None
    if "upload" in only:
        progress("page upload (ExpertLoader)")
        upload = bench_upload(args, ctx, torch, np, N, step_k1(s14.EXACT))
    if "k1" not in only:
        print(json.dumps({"only": sorted(only), "legs": out, "variants": variants, "prefill": prefill,
                          "fp8_linear": linear, "upload": upload}),
              flush=True)
        return 0

    main_r = out[args.mode]
    headline = main_r["k1"]
    # dominant kernel of the timed path: phase 1 (w1, w3 of all pairs)
    st = headline["stage_ms"]
    kernel, k_ms, k_bytes = f"k_phase1_{args.mode}", st["phase1"], phase1_bytes(7, 1)
    achieved = k_bytes / (k_ms * 1e-3) / 1e9
    roofline = {
        "bound": "hbm",
        "kernel": kernel,
        "achieved": achieved,
        "peak": HBM_PEAK_GBPS,
        "unit": "GB/s",
        "frac": achieved / HBM_PEAK_GBPS,
        "traffic": measured_traffic(kernel),
        "algorithmic_bytes": k_bytes,
        "avg_ms": k_ms,
    }

    cpu = None
    if not args.no_cpu_baseline:
        progress("CPU baseline")
        cpu = cpu_baseline(args, bank, routers_h, X, ctx, np, torch, synth)

    line = {
        "metric": METRIC,
        "value": headline["us_per_token"],
        "unit": "us/token",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": headline["us_per_token"] * 1e-3,
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded; MXFP4 codes uniform, UE8M0 exponents in [-10,-4], x ~ N(0,1))",
        "config": {
            "workload": "config2: router + top-6 routed + shared MXFP4 MoE layer, batch 1 (hidden 4096, "
                        "inter 2048, 256 experts); K=8 verify block, config 0 chain, config 1 wq_a and "
                        "config 4 prefill reported beside it",
            "mode": args.mode,
            "parity": "bit-identical to the CPU oracle" if args.mode == "exact" else "order-changed f32",
            "timing": f"median of {args.trials} trials, each one replay of a HIP graph of {args.steps} steps "
                      "between two events queued behind an untimed pre-roll of the same steps (the events "
                      "bracket the device's work; the eager figure, one host launch sequence per step, is in "
                      "k1.timing.eager)",
            "layer_banks": NL,
            "tokens_rotated": P,
            "layer_bytes_k1": layer_bytes_k1(),
        },
        "hbm_gbps": headline["hbm_gbps"],
        "hbm_frac": headline["hbm_frac"],
        "k1": main_r.get("k1"),
        "k8": main_r.get("k8"),
        "config0": main_r.get("config0"),
        "config1": main_r.get("config1"),
        "other_mode": {k: v for k, v in out.items() if k != args.mode},
        "variants": variants,
        "prefill": prefill,
        "fp8_linear": linear,
        "upload": upload,
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    ctx.synchronize()
    return 0


def bench_config1(args, ctx, timer, torch, np, s14, synth):
    """Config 1: the FP8 wq_a matvec (W e4m3 [1024, 4096], f32 128x128 tile
    scales, bf16 x), rotated over WQA_COPIES copies of W (403 MB, past the
    MALL)."""
    cfg = synth.config1(seed=args.seed)
    w1 = torch.from_numpy(cfg["w"].reshape(-1)).cuda()
    W = w1.unsqueeze(0).repeat(WQA_COPIES, 1)
    S = torch.from_numpy(cfg["scale"].reshape(-1)).cuda()
    xb = torch.from_numpy(cfg["x_bf16"]).cuda().view(torch.bfloat16)
    y = torch.empty(WQA_N, dtype=torch.float32, device="cuda")
    pipes = s14.S14NumericPipelines(ctx)
    shape = s14.S14MatvecShape.new(WQA_N, WQA_K).validate_fp8()
    res = {}
    for name, m in (("exact", s14.EXACT), ("fast", s14.FAST)):
        ds = [pipes.bind_fp8(shape, xb, W[c], S, y, mode=m) for c in range(WQA_COPIES)]

        def f(i, ds=ds):
            pipes.cmd_fp8_matvec(ds[(i * 7) % WQA_COPIES])

        t = timer.run_graph(f, WQA_COPIES, args.warmup)
        us = t["ms"] * 1e3
        res[name] = {"us_per_matvec": us, "timing": t, "algorithmic_bytes": WQA_BYTES,
                     "hbm_gbps": WQA_BYTES / (us * 1e-6) / 1e9, "hbm_frac": WQA_BYTES / (us * 1e-6) / 1e9 / HBM_PEAK_GBPS}
    return res


# The reference's one published layer figure: six routed MXFP4 experts with
# the FP8 shared page, route [126, 12, 205, 149, 227, 174] weighted by the
# sqrt-softplus scores x 1.5, 35 dispatches, 1.3696 ms on an RX 5700 XT
# (evidence/s14_vulkan_numeric_rx5700xt.json:49-53).
REF_ROUTE = [126, 12, 205, 149, 227, 174]
REF_LAYER_US = 1369.6
FP8_SHARED_PAGE = 25_167_360


def fp8_shared_pages(torch, n: int, seed: int):
    """n device copies of an FP8 shared page ([w1|s1|w3|s3|w2|s2], e4m3 of
    N(0,1) weights, UE8M0 128x128 tile scales 2^-7..2^-5), made with torch's
    casts on the host: timing inputs only (parity tests use the seeded
    generator and the oracle)."""
    g = torch.Generator().manual_seed(seed)
    parts = []
    for _ in range(3):
        w = torch.randn(2048 * 4096, generator=g).clamp_(-448.0, 448.0)
        parts.append(w.to(torch.float8_e4m3fn).view(torch.uint8))
        parts.append(torch.randint(120, 123, (512,), dtype=torch.uint8, generator=g))
    page = torch.cat(parts)
    assert page.numel() == FP8_SHARED_PAGE
    out = torch.empty((n, FP8_SHARED_PAGE), dtype=torch.uint8, device="cuda")
    for i in range(n):
        out[i].copy_(page)
    return out


def bench_variants(args, ctx, timer, torch, np, s14, synth, N, bank, tables, shared, routers_h, wr, bias, X, XB, NL,
                   P, stages):
    """Layer configurations beside the headline, each a HIP graph of --steps
    steps rotating layer banks and tokens as the headline does:
    - the reference's published layer (route given, FP8 shared page), EXACT
      and FAST, beside its 1.3696 ms;
    - the same with the route chosen on the device (sqrt-softplus x 1.5);
    - official expert semantics (executor.py:705-744) at K=1 and K=8, with
      the config-2 router and MXFP4 shared page, and with the reference's
      router and FP8 shared page;
    - a hash-routed K=1 layer (tid2eid rows, executor.py:643-667);
    - the headline layer with its 97.8 MB resident in the MALL (one layer
      bank, one token repeated), against the rotated figure."""
    res = {}
    steps, warm = args.steps, args.warmup
    f8 = fp8_shared_pages(torch, NL, args.seed)
    Y = torch.empty(4096, dtype=torch.float32, device="cuda")
    YB = torch.empty((8, 4096), dtype=torch.float32, device="cuda")
    x0 = X[0].cpu().numpy().astype(np.float64)

    def ref_weights(L):
        z = routers_h[L][0].astype(np.float64) @ x0
        sc = np.sqrt(np.where(z > 20, z, np.log1p(np.exp(np.minimum(z, 20)))))
        w = sc[REF_ROUTE]
        return (w / w.sum() * 1.5).astype(np.float32).tolist()

    k1_ref_bytes = 6 * PAGE + FP8_SHARED_PAGE + 2 * X_BYTES
    k1_ref_routed_bytes = 6 * PAGE + FP8_SHARED_PAGE + ROUTER + 2 * X_BYTES

    def record(name, t, nbytes, tokens=1, **extra):
        us = t["ms"] * 1e3 / tokens
        gbps = nbytes / (t["ms"] * 1e-3) / 1e9
        res[name] = {"us_per_token": us, "algorithmic_bytes": nbytes, "hbm_gbps": gbps,
                     "hbm_frac": gbps / HBM_PEAK_GBPS, "timing": t, **extra}
        progress(f"  {name}: {us:.2f} us/token, {gbps:.0f} GB/s")

    # reference layer, route given
    pages = [[bank.slot_ptr(L * 257 + e) for e in REF_ROUTE] for L in range(NL)]
    wts = [ref_weights(L) for L in range(NL)]
    for name, m in (("exact", s14.EXACT), ("fast", s14.FAST)):
        def f(i, m=m):
            L = i % NL
            s14.moe_layer(ctx, pages[L], wts[L], f8[L], X[i % P], Y, shared_format=N.S14_PAGE_FP8, mode=m)
        t = timer.run_graph(f, steps, warm)
        record(f"k1_reference_layer_{name}", t, k1_ref_bytes, route=REF_ROUTE,
               reference_rx5700xt_us=REF_LAYER_US, speedup_vs_reference=REF_LAYER_US / (t["ms"] * 1e3))

    ref_routers = [s14.Router(wr[L], bias[L], score_fn=N.S14_SCORE_SQRT_SOFTPLUS, route_scale=1.5)
                   for L in range(NL)]
    cfg_routers = [s14.Router(wr[L], bias[L]) for L in range(NL)]

    def k1(routers, sh, fmt, m):
        def f(i):
            L = i % NL
            s14.moe_layer_route(ctx, routers[L], tables[L], sh[L], X[i % P], Y, shared_format=fmt, mode=m)
        return f

    def k8(routers, sh, fmt, m):
        def f(i):
            L = i % NL
            s14.moe_block_route(ctx, 8, routers[L], tables[L], sh[L], XB[i % P], YB, shared_format=fmt, mode=m)
        return f

    def distinct(routers, sh, fmt, m):
        ds = []
        for i in range(min(P, 16)):
            k8(routers, sh, fmt, m)(i)
            ds.append(s14.last_block_distinct(ctx))
        return float(np.mean(ds))

    t = timer.run_graph(k1(ref_routers, f8, N.S14_PAGE_FP8, s14.EXACT), steps, warm)
    record("k1_reference_routed_exact", t, k1_ref_routed_bytes, router="sqrt-softplus x 1.5", shared="fp8")

    for label, routers, sh, fmt, nb, shared_bytes in (
            ("", cfg_routers, shared, N.S14_PAGE_MXFP4, layer_bytes_k1(), PAGE),
            ("_reference", ref_routers, f8, N.S14_PAGE_FP8, k1_ref_routed_bytes, FP8_SHARED_PAGE)):
        fn = k1(routers, sh, fmt, s14.OFFICIAL)
        t = timer.run_graph(fn, steps, warm)
        st = stages(fn, args.profile_steps)
        record(f"k1_official{label}", t, nb, stage_ms={"route": st[0], "phase1": st[1], "phase2": st[2]})
        fn = k8(routers, sh, fmt, s14.OFFICIAL)
        t = timer.run_graph(fn, max(steps // 4, 10), max(warm // 4, 5))
        d = distinct(routers, sh, fmt, s14.OFFICIAL)
        record(f"k8_official{label}", t, block_bytes(d, 8, shared_bytes), tokens=8, distinct_pages=d,
               ms_per_block=t["ms"])

    # hash routing: tid2eid rows of six distinct experts, token ids rotated
    rng = np.random.default_rng(args.seed + 7)
    vocab = 4096
    tab = torch.from_numpy(np.stack([rng.choice(256, 6, replace=False) for _ in range(vocab)]).astype(np.int64)).cuda()
    tok = torch.from_numpy(rng.integers(0, vocab, P).astype(np.int32)).cuda()
    hash_routers = [[s14.Router(wr[L], bias[L], score_fn=N.S14_SCORE_SQRT_SOFTPLUS, route_scale=1.5, tid2eid=tab,
                                token_ids=tok[p:p + 1]) for p in range(P)] for L in range(NL)]

    def f_hash(i):
        L = i % NL
        s14.moe_layer_route(ctx, hash_routers[L][i % P], tables[L], shared[L], X[i % P], Y, mode=s14.EXACT)

    t = timer.run_graph(f_hash, steps, warm)
    record("k1_hash_exact", t, layer_bytes_k1(), router="tid2eid hash rows, sqrt-softplus x 1.5 weights")

    def f_hot(i):
        s14.moe_layer_route(ctx, cfg_routers[0], tables[0], shared[0], X[0], Y, mode=s14.EXACT)

    t = timer.run_graph(f_hot, steps, warm)
    record("k1_exact_mall_resident", t, layer_bytes_k1(),
           note="one layer bank and one token repeated: the layer's 97.8 MB stay in the 256 MB MALL")
    del f8
    return res


LINEAR_SHAPES = {"wq_b": (32768, 1024), "wkv": (512, 4096), "wo_a": (8192, 4096), "wo_b": (4096, 8192)}


def linear_bytes(m: int, n: int, k: int) -> int:
    """Algorithmic bytes of one fp8_linear: e4m3 weight, UE8M0 tile scales,
    e4m3 activations and their scales, f32 output."""
    g = -(-k // 128)
    return n * k + -(-n // 128) * g + m * k + m * g + 4 * m * n


def bench_linear(args, ctx, timer, torch, s14):
    """The adjacent FP8 projections (fp8_linear, fp8.py:111-193) at wq_b,
    wkv, wo_a and wo_b (l42_reference.py:89-102) for 1 and 8 tokens, each
    mode timed as a HIP graph of launches over weight copies that total at
    least 512 MB (past the 256 MB MALL)."""
    res = {}
    gen = torch.Generator(device="cuda")
    gen.manual_seed(args.seed)
    for name, (n, k) in LINEAR_SHAPES.items():
        copies = max(2, -(-(512 << 20) // (n * k)))
        W = torch.randint(0, 256, (copies, n, k), dtype=torch.uint8, device="cuda", generator=gen)
        W[(W & 0x7F) == 0x7F] = 0x7E
        WS = torch.randint(114, 122, (copies, -(-n // 128), k // 128), dtype=torch.uint8, device="cuda", generator=gen)
        for m in (1, 8):
            X = torch.randint(0, 256, (m, k), dtype=torch.uint8, device="cuda", generator=gen)
            X[(X & 0x7F) == 0x7F] = 0x7E
            XS = torch.randint(120, 128, (m, k // 128), dtype=torch.uint8, device="cuda", generator=gen)
            y = torch.empty((m, n), dtype=torch.float32, device="cuda")
            nbytes = linear_bytes(m, n, k)
            for mode_name, mode in (("exact", s14.EXACT), ("fast", s14.FAST)):
                def f(i, mode=mode):
                    c = i % copies
                    s14.fp8_linear(ctx, X, XS, W[c], WS[c], y, mode=mode)

                t = timer.run_graph(f, copies, 3)
                us = t["ms"] * 1e3
                gbps = nbytes / (us * 1e-6) / 1e9
                res[f"{name}_m{m}_{mode_name}"] = {"n": n, "k": k, "m": m, "us": us, "algorithmic_bytes": nbytes,
                                                   "hbm_gbps": gbps, "hbm_frac": gbps / HBM_PEAK_GBPS, "timing": t}
                progress(f"  {name} m={m} {mode_name}: {us:.2f} us, {gbps:.0f} GB/s")
        del W, WS
        torch.cuda.synchronize()
    return res


UPLOAD_PAGES = 48  # 642 MB per batch


def bench_upload(args, ctx, torch, np, N, layer_step):
    """The page upload path (ExpertLoader, expert_loader.rs:299-360): a batch
    of UPLOAD_PAGES distinct pages from host memory (the enqueue_from_buf
    path: bytes already read) through a ring of pinned staging slots into a
    VramPool on the context's copy stream, until the last transfer fence.
    Alone, then while the K=1 exact layer replays from a HIP graph on the
    compute side; overlap = (t_layer + t_upload - t_both) / min(t_layer,
    t_upload), 1 when the two hide each other completely."""
    from colormlm_amd.pool import ExpertKey, ExpertLoader, VramPool

    rng = np.random.default_rng(args.seed)
    sources = [rng.integers(0, 256, PAGE, dtype=np.uint8) for _ in range(8)]  # cycled: 107 MB of distinct bytes
    pool = VramPool(UPLOAD_PAGES, PAGE, ctx)
    res = {"pages": UPLOAD_PAGES, "page_bytes": PAGE, "sources": "host memory (numpy), 8 distinct 13.4 MB buffers"}
    batch = [0]

    def upload(loader):
        b = batch[0]
        batch[0] += 1
        keys = [ExpertKey(b % 60, 0, i) for i in range(UPLOAD_PAGES)]
        t0 = time.perf_counter()
        loader.batch_enqueue_from_bufs(pool, keys, [sources[i % 8] for i in range(UPLOAD_PAGES)])
        loader.wait_all(pool)
        return time.perf_counter() - t0

    for depth in (2, 4, 8):
        loader = ExpertLoader(ctx, depth, PAGE)
        upload(loader)  # warm: pool slots and staging touched once
        ts = [upload(loader) for _ in range(max(3, args.trials))]
        t = statistics.median(ts)
        res[f"depth{depth}"] = {"s_per_batch": t, "h2d_gbps": UPLOAD_PAGES * PAGE / t / 1e9}
        loader.destroy()
        progress(f"  upload depth {depth}: {UPLOAD_PAGES * PAGE / t / 1e9:.1f} GB/s")
    # raw copy-engine rate from pinned memory, for comparison
    src = torch.empty(UPLOAD_PAGES * PAGE, dtype=torch.uint8, pin_memory=True)
    dst = torch.empty(UPLOAD_PAGES * PAGE, dtype=torch.uint8, device="cuda")
    dst.copy_(src, non_blocking=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    dst.copy_(src, non_blocking=True)
    torch.cuda.synchronize()
    res["pinned_memcpy_gbps"] = UPLOAD_PAGES * PAGE / (time.perf_counter() - t0) / 1e9
    del src, dst
    # overlap with the layer: 100 K=1 exact steps per graph replay
    loader = ExpertLoader(ctx, 4, PAGE)
    upload(loader)
    for i in range(3):
        layer_step(i)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(100):
            layer_step(i)
    g.replay()
    torch.cuda.synchronize()
    t_up = statistics.median([upload(loader) for _ in range(3)])
    t0 = time.perf_counter()
    for _ in range(8):
        g.replay()
    torch.cuda.synchronize()
    reps = max(1, round(8 * t_up / (time.perf_counter() - t0)))  # layer time ~ upload time
    t0 = time.perf_counter()
    for _ in range(reps):
        g.replay()
    torch.cuda.synchronize()
    t_layer = time.perf_counter() - t0
    t0 = time.perf_counter()
    for _ in range(reps):
        g.replay()
    t_up_both = upload(loader)
    torch.cuda.synchronize()
    t_both = time.perf_counter() - t0
    loader.destroy()
    del g
    res["overlap"] = {"layer_steps": 100 * reps, "t_layer_s": t_layer, "t_upload_s": t_up, "t_both_s": t_both,
                      "upload_during_layer_gbps": UPLOAD_PAGES * PAGE / t_up_both / 1e9,
                      "layer_us_per_token_during_upload": t_both / (100 * reps) * 1e6,
                      "overlap": (t_layer + t_up - t_both) / min(t_layer, t_up)}
    progress(f"  overlap {res['overlap']['overlap']:.2f} (layer {t_layer * 1e3:.1f} ms, upload {t_up * 1e3:.1f} ms, "
             f"both {t_both * 1e3:.1f} ms)")
    pool.destroy()
    return res


PREFILL_LAYERS = 4  # layer banks rotated by the prefill leg (each prefill reads ~240 pages, 3.2 GB)


def bench_prefill(args, ctx, tables, shared, NL, torch, np, s14, synth):
    """Config 4: 512 tokens through the layer as grouped scaled-MFMA GEMMs,
    routed under Zipf(1.1) expert popularity (synth.prefill_router: the
    busiest expert takes ~380 of the 512 tokens), layers rotated across
    steps.  Reports the per-expert token counts (M_e) the routes gave."""
    T = PREFILL_TOKENS
    NP = min(NL, PREFILL_LAYERS)
    routers = []
    keep = []
    for L in range(NP):
        w, b = synth.prefill_router(args.seed, L)
        wt, bias = torch.from_numpy(w).cuda(), torch.from_numpy(b).cuda()
        keep += [wt, bias]
        routers.append(s14.Router(wt, bias))
    xs = torch.from_numpy(synth.prefill_tokens(args.seed, T)).cuda()
    y = torch.empty((T, 4096), dtype=torch.float32, device="cuda")
    ids = torch.empty((T, 6), dtype=torch.int16, device="cuda")

    def step(i):
        L = i % NP
        s14.moe_prefill(ctx, T, routers[L], tables[L], shared[L], xs, y)

    def step_official(i):
        L = i % NP
        s14.moe_prefill(ctx, T, routers[L], tables[L], shared[L], xs, y, mode=s14.OFFICIAL)

    stats, me = [], []
    for L in range(NP):
        s14.moe_prefill(ctx, T, routers[L], tables[L], shared[L], xs, y, ids_out=ids)
        stats.append(s14.last_prefill_stats(ctx))
        c = np.bincount(ids.cpu().numpy().astype(np.int64).ravel() & 0xFFFF, minlength=256)
        me.append(c[c > 0])
    t = Timer(torch, args.trials).run(step, max(args.prefill_steps, 1), 2)
    t_off = Timer(torch, args.trials).run(step_official, max(args.prefill_steps, 1), 2)
    ms = t["ms"]
    d = float(np.mean([s["distinct"] for s in stats]))
    nbytes = prefill_bytes(d, T)
    flops = prefill_flops(T)
    allme = np.concatenate(me)
    return {
        "tokens": T,
        "ms_per_prefill": ms,
        "us_per_token": ms * 1e3 / T,
        "timing": t,
        "layers_rotated": NP,
        "routing": "sigmoid router with per-expert bias calibrated to Zipf(1.1) top-6 popularity",
        "distinct_experts": d,
        "max_tokens_per_expert": max(s["max_tokens_per_expert"] for s in stats),
        "tokens_per_expert": {"max_per_layer": [int(m.max()) for m in me],
                              "p50": float(np.percentile(allme, 50)), "p90": float(np.percentile(allme, 90)),
                              "mean": float(allme.mean())},
        "work_items": float(np.mean([s["items"] for s in stats])),
        "algorithmic_bytes": nbytes,
        "hbm_gbps": nbytes / (ms * 1e-3) / 1e9,
        "hbm_frac": nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS,
        "tflops": flops / (ms * 1e-3) / 1e12,
        "mfma_frac_bf16": flops / (ms * 1e-3) / 1e12 / BF16_MFMA_PEAK_TFLOPS,
        "official": {"ms_per_prefill": t_off["ms"], "us_per_token": t_off["ms"] * 1e3 / T, "timing": t_off,
                     "hbm_gbps": nbytes / (t_off["ms"] * 1e-3) / 1e9},
    }


COPY_BYTES = 256 << 20


def copy_calibration(torch) -> int:
    """A plain device copy of COPY_BYTES, 10 times: under rocprofv3 --pmc its
    FETCH_SIZE / WRITE_SIZE per dispatch should read COPY_BYTES / 1024 KiB;
    the ratio scales the counters of the S14 kernels."""
    src = torch.empty(COPY_BYTES, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": COPY_BYTES, "reps": 10}), flush=True)
    return 0


def measured_traffic(kernel: str):
    """HBM bytes per launch of `kernel` (read + written) from the committed
    counter summary: lines 'traffic <kernel> <fetch_bytes> <write_bytes>'
    in profiles/*.md, already scaled by the copy calibration.  None when no
    summary covers the kernel."""
    for f in sorted((ROOT / "profiles").glob("*.md")):
        for ln in f.read_text().splitlines():
            parts = ln.strip().strip("`").split()
            if len(parts) == 4 and parts[0] == "traffic" and parts[1] == kernel:
                return int(parts[2]) + int(parts[3])
    return None


def cpu_model() -> str:
    try:
        for ln in Path("/proc/cpuinfo").read_text().splitlines():
            if ln.startswith("model name"):
                return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def _median_runs(fn, seconds: float, min_runs: int = 5, max_runs: int = 15):
    """Wall times of fn() after one warm-up run: at least min_runs, more while
    under `seconds` of total work."""
    fn()
    times = []
    spent = 0.0
    while len(times) < max_runs and (len(times) < min_runs or spent < seconds):
        t0 = time.perf_counter()
        fn()
        dt = time.perf_counter() - t0
        times.append(dt)
        spent += dt
        if len(times) >= min_runs and spent >= seconds:
            break
    return statistics.median(times), len(times)


def cpu_baseline(args, bank, routers_h, X, ctx, np, torch, synth):
    """The CPU oracle (the C restatement of the reference's CPU F32 path) on
    the host cores: config 2 (route + layer), config 0 (chain) and config 1
    (wq_a), each on all host cores and on one core, median of >= 5 runs
    after a warm-up run, each config's work bounded by --cpu-seconds."""
    import oracle

    xs = X.cpu().numpy()
    wr, b = routers_h[0]
    _, ids, w = oracle.route(wr, b, xs[0])
    torch.cuda.synchronize()
    routed = [bank.slot_tensor(int(e))[:PAGE].cpu().numpy() for e in ids]
    sh = bank.slot_tensor(256)[:PAGE].cpu().numpy()
    c1 = synth.config1(seed=args.seed)

    def layer():
        oracle.route(wr, b, xs[0])
        oracle.moe_layer(xs[0], routed, w, sh)

    def chain():
        oracle.expert_chain(xs[0], routed[0], 0.17)

    def wqa():
        oracle.fp8_matvec_f32scale_bf16x(c1["x_bf16"], c1["w"], c1["scale"])

    all_cores = oracle.num_threads()
    res = {}
    for label, n in (("all_cores", all_cores), ("one_core", 1)):
        oracle.set_num_threads(n)
        share = args.cpu_seconds / 2
        t_layer, n_layer = _median_runs(layer, share * 0.7)
        t_chain, n_chain = _median_runs(chain, share * 0.2)
        t_wqa, n_wqa = _median_runs(wqa, share * 0.1)
        res[label] = {"cores": n, "config2_us_per_token": t_layer * 1e6, "config2_runs": n_layer,
                      "config0_us_per_chain": t_chain * 1e6, "config0_runs": n_chain,
                      "config1_us_per_matvec": t_wqa * 1e6, "config1_runs": n_wqa}
    oracle.set_num_threads(all_cores)
    return {
        "value": res["all_cores"]["config2_us_per_token"],
        "unit": "us/token",
        "cores": all_cores,
        "kind": "port",
        "cpu_model": cpu_model(),
        "host_cpus": os.cpu_count(),
        "sample": "config 2: one token (router + 6 routed + shared MXFP4 pages, f32 oracle order, OpenMP over "
                  "rows), median of >= 5 runs after a warm-up; configs 0 and 1 likewise",
        "all_cores": res["all_cores"],
        "one_core": res["one_core"],
    }


if __name__ == "__main__":
    sys.exit(main())
