"""The device log1pf used by the sqrt-softplus router (csrc/s14_log1pf.h)
must return exactly what the C library's log1pf returns, because the oracle
(executor.py:642's softplus, evaluated with the C library) calls it.  The
header is compiled for the host here and compared bit for bit; the same
comparison over every non-NaN f32 found no difference."""

from __future__ import annotations

import ctypes as C
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]


@pytest.fixture(scope="module")
def lib(tmp_path_factory):
    if not shutil.which("g++"):
        pytest.skip("g++ not available")
    out = tmp_path_factory.mktemp("log1pf") / "liblog1pf.so"
    subprocess.run(
        ["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-fPIC", "-shared",
         f"-I{ROOT / 'colormlm_amd' / 'csrc'}", str(ROOT / "tests" / "native" / "log1pf_check.cpp"),
         "-o", str(out)],
        check=True,
    )
    h = C.CDLL(str(out))
    h.log1pf_mismatches.restype = C.c_uint64
    h.log1pf_mismatches.argtypes = [C.c_uint64, C.c_uint64, C.c_uint64, C.POINTER(C.c_uint32)]
    return h


def bits(v: float) -> int:
    return int(np.array([v], np.float32).view(np.uint32)[0])


def test_log1pf_matches_libc_on_a_stride_of_all_floats(lib):
    first = C.c_uint32(0)
    assert lib.log1pf_mismatches(0, 1 << 32, 61, C.byref(first)) == 0, hex(first.value)


def test_log1pf_matches_libc_on_the_softplus_range(lib):
    # log1p(exp(z)) for z <= 20 (torch's threshold): arguments in (0, e^20];
    # every float of [0.25, 4) (the reduction's branch points and 1 + x
    # carries) and a stride elsewhere
    first = C.c_uint32(0)
    assert lib.log1pf_mismatches(bits(0.25), bits(4.0), 1, C.byref(first)) == 0, hex(first.value)
    assert lib.log1pf_mismatches(1, bits(float(np.exp(np.float32(20)))) + 1, 7, C.byref(first)) == 0, hex(first.value)


def test_log1pf_branch_edges_and_specials(lib):
    # the reduction's thresholds (0.41422, -0.2929, 2^-29, 2^-54, 2^53, the
    # sqrt(2) normalisation) and the specials
    edges = [0x3ed413d7, 0xbe95f61f, 0x31000000, 0x24800000, 0x5a000000, 0x3504f7 | 0x3f800000,
             bits(-1.0), bits(-0.5), bits(-0.0), 0, bits(np.inf), bits(-np.inf), bits(1e-45), bits(3.4e38)]
    for b in edges:
        first = C.c_uint32(0)
        assert lib.log1pf_mismatches(max(b - 64, 0), min(b + 64, 1 << 32), 1, C.byref(first)) == 0, hex(b)
