"""The no-allocation entry point (s14_moe_block_route_noalloc) against the
context entry point it varies (s14_moe_block_route): same inputs, outputs,
routes and weights bit for bit, on two calls in a row, the second with a
smaller block, in each mode (EXACT, FAST, official)."""

from __future__ import annotations

import sys

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

from colormlm_amd import _native as N  # noqa: E402
from colormlm_amd import s14, synth  # noqa: E402

HIDDEN = N.HIDDEN


def say(msg: str) -> None:
    print(f"[gpu-test] {msg}", file=sys.stderr, flush=True)


def bits(t) -> np.ndarray:
    torch.cuda.synchronize()
    return np.ascontiguousarray(t.cpu().numpy()).view(np.uint8)


@pytest.fixture(scope="module")
def setup():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    say("no-alloc: context and 257-page bank")
    ctx = s14.Context(0)
    pages = torch.empty((257, N.EXPERT_PAGE_BYTES), dtype=torch.uint8, device="cuda")
    for e in range(256):
        s14.fill_mxfp4_page(ctx, pages[e], 5, 1, e)
    s14.fill_mxfp4_page(ctx, pages[256], 5, 1, synth.SHARED_EXPERT)
    table = torch.tensor([pages[e].data_ptr() for e in range(256)], dtype=torch.int64, device="cuda")
    wr, bias = synth.router(seed=5, layer=1)
    router = s14.Router(torch.from_numpy(wr).cuda(), torch.from_numpy(bias).cuda())
    torch.cuda.synchronize()
    yield ctx, pages, table, router
    torch.cuda.synchronize()
    ctx.destroy()


@pytest.mark.parametrize("mode", [s14.EXACT, s14.FAST, s14.OFFICIAL])
def test_noalloc_matches_context_entry(setup, mode):
    ctx, pages, table, router = setup
    assert N.lib().s14_noalloc_scratch_bytes() > 0
    # each call smaller than the one before; one token runs the single-launch layer kernel
    for call, tokens in enumerate((8, 3, 1)):
        say(f"no-alloc call {call}: T={tokens} mode={mode}")
        x = torch.from_numpy(synth.block_tokens(seed=40 + call, tokens=tokens)).cuda()
        y_ref = torch.full((tokens, HIDDEN), np.nan, dtype=torch.float32, device="cuda")
        y_new = torch.full((tokens, HIDDEN), np.nan, dtype=torch.float32, device="cuda")
        ids_ref = torch.zeros((tokens, 6), dtype=torch.int16, device="cuda")
        ids_new = torch.zeros((tokens, 6), dtype=torch.int16, device="cuda")
        w_ref = torch.zeros((tokens, 6), dtype=torch.float32, device="cuda")
        w_new = torch.zeros((tokens, 6), dtype=torch.float32, device="cuda")
        s14.moe_block_route(ctx, tokens, router, table, pages[256], x, y_ref, ids_ref, w_ref, mode=mode)
        s14.moe_block_route_noalloc(tokens, router, table, pages[256], x, y_new, ids_new, w_new, mode=mode)
        assert np.array_equal(bits(ids_new), bits(ids_ref))
        assert np.array_equal(bits(w_new), bits(w_ref))
        assert np.array_equal(bits(y_new), bits(y_ref)), f"call {call}: outputs differ"
        assert not np.isnan(y_new.cpu().numpy()).any()


def test_noalloc_rejects_oversized_block(setup):
    ctx, pages, table, router = setup
    x = torch.zeros((9, HIDDEN), dtype=torch.float32, device="cuda")
    y = torch.zeros((9, HIDDEN), dtype=torch.float32, device="cuda")
    with pytest.raises(s14.S14Error) as err:
        s14.moe_block_route_noalloc(9, router, table, pages[256], x, y)
    assert err.value.code == N.S14_ERR_SHAPE


CAPTURE_CHILD = r"""
import sys
import numpy as np
import torch
from colormlm_amd import _native as N
from colormlm_amd import s14, synth

def say(m):
    print(m, file=sys.stderr, flush=True)

ctx = s14.Context(0)
# eight distinct pages behind the 256-entry table (routes are compared
# between the two entry points, which share the table)
pages = torch.empty((9, N.EXPERT_PAGE_BYTES), dtype=torch.uint8, device="cuda")
for e in range(8):
    s14.fill_mxfp4_page(ctx, pages[e], 6, 1, e)
s14.fill_mxfp4_page(ctx, pages[8], 6, 1, synth.SHARED_EXPERT)
table = torch.tensor([pages[e % 8].data_ptr() for e in range(256)], dtype=torch.int64, device="cuda")
wr, bias = synth.router(seed=6, layer=1)
router = s14.Router(torch.from_numpy(wr).cuda(), torch.from_numpy(bias).cuda())
T = 8
x_static = torch.from_numpy(synth.block_tokens(seed=60, tokens=T)).cuda()
y_graph = torch.full((T, N.HIDDEN), np.nan, dtype=torch.float32, device="cuda")
torch.cuda.synchronize()
say("capture: the process's first no-alloc call")
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g):
    s14.moe_block_route_noalloc(T, router, table, pages[8], x_static, y_graph, mode=s14.EXACT)
for i in range(3):
    xs = torch.from_numpy(synth.block_tokens(seed=61 + i, tokens=T)).cuda()
    x_static.copy_(xs)
    y_graph.fill_(np.nan)
    g.replay()
    torch.cuda.synchronize()
    got = y_graph.cpu().numpy().copy()
    y_ctx = torch.full_like(y_graph, np.nan)
    s14.moe_block_route(ctx, T, router, table, pages[8], xs, y_ctx, mode=s14.EXACT)
    y_eager = torch.full_like(y_graph, np.nan)
    s14.moe_block_route_noalloc(T, router, table, pages[8], xs, y_eager, mode=s14.EXACT)
    torch.cuda.synchronize()
    want = y_ctx.cpu().numpy()
    assert not np.isnan(got).any(), f"replay {i}: NaN outputs"
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"replay {i} differs from the context entry"
    assert np.array_equal(y_eager.cpu().numpy().view(np.uint32), want.view(np.uint32)), f"eager {i}"
    say(f"replay {i}: bit-identical to the context entry and to an eager no-alloc call")
del g
torch.cuda.synchronize()
ctx.destroy()
print("CAPTURE-OK", flush=True)
"""


def test_noalloc_first_call_under_graph_capture():
    """A process whose first no-allocation call is made while its stream is
    being captured into a HIP graph (the per-device set-up then runs under
    capture): three replays with new inputs, each bit-identical to the
    context entry point and to an eager no-allocation call between the
    replays.  Runs in a child process so that the call is the process's
    first whatever ran before it here."""
    import subprocess
    from pathlib import Path

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    root = Path(__file__).resolve().parents[1]
    say("no-alloc: first call under graph capture (child process)")
    r = subprocess.run([sys.executable, "-c", CAPTURE_CHILD], cwd=root, capture_output=True, text=True, timeout=300)
    sys.stderr.write(r.stderr[-4000:])
    assert r.returncode == 0 and "CAPTURE-OK" in r.stdout, r.stdout[-2000:]
