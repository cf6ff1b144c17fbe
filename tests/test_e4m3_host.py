"""The device e4m3 encoder of the prefill requant (csrc/s14_e4m3.h), a
straight-line restatement, must encode every f32 exactly as the oracle's
branchy encoder (s14o_f32_to_e4m3fn_rne_sat) does.  The header is compiled
for the host here and compared bit for bit: a stride over all floats, every
float in the ranges where the encoding changes form, and every rounding tie."""

from __future__ import annotations

import ctypes as C
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest

import oracle as O

ROOT = Path(__file__).resolve().parents[1]


@pytest.fixture(scope="module")
def check():
    if not shutil.which("g++"):
        pytest.skip("g++ not available")
    import tempfile
    out = Path(tempfile.mkdtemp()) / "libe4m3.so"
    subprocess.run(
        ["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-fPIC", "-shared",
         f"-I{ROOT / 'colormlm_amd' / 'csrc'}", str(ROOT / "tests" / "native" / "e4m3_check.cpp"),
         "-o", str(out)],
        check=True,
    )
    lib = C.CDLL(str(out))
    lib.e4m3_mismatches.restype = C.c_uint64
    lib.e4m3_mismatches.argtypes = [C.c_uint64, C.c_uint64, C.c_uint64, C.c_void_p, C.POINTER(C.c_uint32)]
    ref = C.cast(O.lib().s14o_f32_to_e4m3fn_rne_sat, C.c_void_p).value

    def mismatches(start, stop, step=1):
        first = C.c_uint32(0)
        n = lib.e4m3_mismatches(int(start), int(stop), int(step), ref, C.byref(first))
        return n, hex(first.value)

    return mismatches


def bits(v):
    return int(np.array([v], np.float32).view(np.uint32)[0])


def test_stride_over_all_floats(check):
    assert check(0, 1 << 32, 97) == (0, "0x0")


@pytest.mark.parametrize("sign", [0, 0x80000000])
def test_every_float_where_the_form_changes(check, sign):
    # zero and the f32 subnormals up to the e4m3 subnormal grid's top (2^-6),
    # then around the largest finite (448) and past it to the infinities
    assert check(sign, sign + bits(2.0 ** -5) + 1) == (0, "0x0")
    assert check(sign + bits(400.0), sign + bits(520.0) + 1) == (0, "0x0")
    assert check(sign + 0x7F000000, sign + 0x80000000) == (0, "0x0")


def test_every_rounding_tie(check):
    # every normal e4m3 exponent and mantissa: the tie point halfway to the
    # next code, and one f32 ulp either side; and the subnormal grid's ties
    for e in range(121, 136):
        for m in range(8):
            for sign in (0, 0x80000000):
                tie = sign | (e << 23) | (m << 20) | 0x80000
                assert check(tie - 1, tie + 2) == (0, "0x0"), (e, m, sign)
    for k in range(0, 9):
        for sign in (0, 0x80000000):
            t = sign | bits((k + 0.5) / 512.0)
            assert check(t - 1, t + 2) == (0, "0x0"), k
