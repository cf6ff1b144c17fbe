"""The FAST fp8_linear's launch plan (csrc/s14_linear_plan.h), compiled for
the host: every launch it makes keeps its split-K partials within the
context's 32 MiB workspace and its (row tile, token block) arrival counters
within the 65,536 the workspace holds, its staged activations within the
wavefront's LDS budget, and its K split whole (chunk widths are multiples
of 4 dividing the group count).  Checked for m = 1..1024 tokens at the
adjacent projections' shapes (l42_reference.py:89-102) and at shapes that
force the token blocks into several launches or FAST off altogether."""

from __future__ import annotations

import ctypes as C
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]

SHAPES = {"wq_b": (32768, 1024), "wkv": (512, 4096), "wo_a": (8192, 4096), "wo_b": (4096, 8192)}


@pytest.fixture(scope="module")
def plan_lib(tmp_path_factory):
    if not shutil.which("g++"):
        pytest.skip("g++ not available")
    out = tmp_path_factory.mktemp("linplan") / "liblinplan.so"
    subprocess.run(
        ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", f"-I{ROOT / 'colormlm_amd' / 'csrc'}",
         str(ROOT / "tests" / "native" / "linear_plan_check.cpp"), "-o", str(out)],
        check=True,
    )
    lib = C.CDLL(str(out))
    u32p = C.POINTER(C.c_uint32)
    lib.lin_plan.argtypes = [C.c_uint32, C.c_uint32, C.c_uint32, u32p, u32p]
    lib.lin_chunks.argtypes = [C.c_uint32] * 4
    lib.lin_chunks.restype = C.c_uint32
    lib.lin_limits.argtypes = [C.POINTER(C.c_uint64), u32p, u32p, u32p]
    return lib


def launches(lib, m, n, k):
    """The launches launch_fp8_linear makes: [(tokens, chunk width, splits)]
    or None when FAST hands the shape to EXACT."""
    groups = -(-k // 128)
    cw, blocks = C.c_uint32(), C.c_uint32()
    lib.lin_plan(m, n, groups, C.byref(cw), C.byref(blocks))
    if cw.value == 0:
        return None
    tiles, per = -(-n // 32), blocks.value * 32
    out = []
    for m0 in range(0, m, per):
        mc = min(per, m - m0)
        c = lib.lin_chunks(groups, tiles, -(-mc // 32), min(mc, 32))
        out.append((mc, c, groups // c if c else 0))
    return out


def check(lib, m, n, k):
    part, cnt, stage, tile = C.c_uint64(), C.c_uint32(), C.c_uint32(), C.c_uint32()
    lib.lin_limits(C.byref(part), C.byref(cnt), C.byref(stage), C.byref(tile))
    groups = -(-k // 128)
    tiles = -(-n // 32)
    plan = launches(lib, m, n, k)
    if plan is None:
        return None
    assert sum(mc for mc, _, _ in plan) == m
    for mc, cw, splits in plan:
        assert cw > 0 and cw % 4 == 0 and groups % cw == 0, (m, n, k, cw)
        ncb, ntok = -(-mc // 32), min(mc, 32)
        assert ntok * cw * (128 * 2 + 4) <= stage.value, (m, n, k, cw)
        if splits > 1:
            assert tiles * ncb <= cnt.value, (m, n, k)
            assert tiles * ncb * splits * 32 * 32 * 4 <= part.value, (m, n, k, mc, cw)
    return plan


@pytest.mark.parametrize("name", list(SHAPES))
def test_fast_plan_fits_the_workspace_for_every_token_count(plan_lib, name):
    n, k = SHAPES[name]
    for m in range(1, 1025):
        plan = check(plan_lib, m, n, k)
        # the projections always run FAST (a shape FAST cannot plan goes to EXACT)
        assert plan is not None, (name, m)


def test_fast_plan_splits_token_blocks_where_partials_would_overflow(plan_lib):
    # wq_b: 1,024 row tiles x 2 splits x 4 KiB = 8 MiB of partials per token
    # block, so at most 4 blocks (128 tokens) per launch
    assert launches(plan_lib, 128, 32768, 1024) == [(128, 4, 2)]
    assert launches(plan_lib, 129, 32768, 1024) == [(96, 4, 2), (33, 4, 2)]
    plan = launches(plan_lib, 1024, 32768, 1024)
    assert len(plan) == 8 and all(mc == 128 for mc, _, _ in plan)
    # wkv's partials are small: 1,024 tokens in one launch
    assert len(launches(plan_lib, 1024, 512, 4096)) == 1


def test_fast_plan_hands_unplannable_shapes_to_exact(plan_lib):
    # G = 6 is not a multiple of 4; 32 tokens at k = 131072 split K 256 ways
    # over 2,048 row tiles: 2 GiB of partials for a single block
    assert launches(plan_lib, 4, 1024, 768) is None
    assert launches(plan_lib, 32, 65536, 131072) is None
    for m in (1, 2, 31, 32, 33, 300, 1024):
        for n, k in ((65536, 16384), (100, 131072), (131072, 512), (4096, 65536)):
            check(plan_lib, m, n, k)
