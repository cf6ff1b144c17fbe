"""The device exp used by SwiGLU and the sigmoid router (csrc/s14_expf.h)
must return exactly what the C library's expf returns, because the oracle
(like the reference's Rust f32::exp on Linux) calls the C library.  The
header is compiled for the host here and compared bit for bit."""

from __future__ import annotations

import ctypes as C
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]


@pytest.fixture(scope="module")
def expf_lib(tmp_path_factory):
    if not shutil.which("g++"):
        pytest.skip("g++ not available")
    out = tmp_path_factory.mktemp("expf") / "libexpf.so"
    subprocess.run(
        ["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-fPIC", "-shared",
         f"-I{ROOT / 'colormlm_amd' / 'csrc'}", str(ROOT / "tests" / "native" / "expf_check.cpp"),
         "-o", str(out)],
        check=True,
    )
    lib = C.CDLL(str(out))
    lib.expf_mismatches.restype = C.c_uint64
    lib.expf_mismatches.argtypes = [C.c_uint64, C.c_uint64, C.c_uint64, C.POINTER(C.c_uint32)]
    lib.expf_device_restated.restype = C.c_float
    lib.expf_device_restated.argtypes = [C.c_float]
    return lib


def test_expf_matches_libc_on_a_stride_of_all_floats(expf_lib):
    first = C.c_uint32(0)
    bad = expf_lib.expf_mismatches(0, 1 << 32, 61, C.byref(first))
    assert bad == 0, hex(first.value)


def test_expf_matches_libc_on_swiglu_range(expf_lib):
    # every f32 in [-10, 0] and [0, 16]: the arguments SwiGLU's exp(-g) sees most
    lo = np.array([-10.0], np.float32).view(np.uint32)[0]
    first = C.c_uint32(0)
    assert expf_lib.expf_mismatches(0x80000000, int(lo) + 1, 1, C.byref(first)) == 0, hex(first.value)
    hi = np.array([16.0], np.float32).view(np.uint32)[0]
    assert expf_lib.expf_mismatches(0, int(hi) + 1, 1, C.byref(first)) == 0, hex(first.value)


def test_expf_known_hard_cases(expf_lib):
    # inputs where glibc differs from round-to-nearest of the exact value, and
    # where an all-unfused evaluation order differs from glibc
    for bits in (0x37FF7F01, 0x38AD9E29, 0x4202422F, 0xC27C65D9, 0x42B17218, 0xC2CFF1B5):
        first = C.c_uint32(0)
        assert expf_lib.expf_mismatches(int(bits), int(bits) + 1, 1, C.byref(first)) == 0, hex(bits)
    # overflow / underflow / specials
    inf = np.float32(np.inf)
    assert expf_lib.expf_device_restated(89.0) == inf
    assert expf_lib.expf_device_restated(-105.0) == 0.0
    assert expf_lib.expf_device_restated(float(-inf)) == 0.0
    assert np.isnan(expf_lib.expf_device_restated(float("nan")))
