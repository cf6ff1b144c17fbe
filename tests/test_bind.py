"""bind_* validation (s14_vulkan.rs:206-334) runs on the host before any
launch: shape, alignment and capacity errors surface with the reference's
categories.  Device addresses are never dereferenced here."""

from __future__ import annotations

import ctypes as C

import pytest

from colormlm_amd import _native as N
from colormlm_amd.s14 import S14Error


def buf(ptr, nbytes):
    return N.Buffer(ptr, nbytes)


def bind_mx(n, k, xb, wb, sb, yb, mode=N.S14_MODE_EXACT):
    rec = N.Mxfp4Dispatch()
    rc = N.lib().s14_bind_mxfp4(N.Shape(n, k), xb, wb, sb, yb, mode, C.byref(rec))
    return rc, rec


def test_bind_mxfp4_capacities(native):
    A = 0x10000
    ok = bind_mx(2048, 4096, buf(A, 16384), buf(A, 4194304), buf(A, 262144), buf(A, 8192))
    assert ok[0] == 0 and ok[1].shape.n == 2048 and ok[1].mode == 0
    cases = [
        (buf(A, 16380), buf(A, 4194304), buf(A, 262144), buf(A, 8192)),
        (buf(A, 16384), buf(A, 4194303), buf(A, 262144), buf(A, 8192)),
        (buf(A, 16384), buf(A, 4194304), buf(A, 262143), buf(A, 8192)),
        (buf(A, 16384), buf(A, 4194304), buf(A, 262144), buf(A, 8188)),
    ]
    for c in cases:
        rc, _ = bind_mx(2048, 4096, *c)
        assert rc == N.S14_ERR_CAPACITY, N.last_error()
    assert "requires at least" in N.last_error()
    assert bind_mx(2048, 4000, *cases[0])[0] == N.S14_ERR_SHAPE
    assert bind_mx(2048, 4096, buf(None, 16384), *cases[0][1:])[0] == N.S14_ERR_INVALID
    assert bind_mx(2048, 4096, buf(A + 4, 16384), buf(A, 4194304), buf(A, 262144), buf(A, 8192))[0] == N.S14_ERR_INVALID
    assert bind_mx(2048, 4096, buf(A, 16384), buf(A, 4194304), buf(A, 262144), buf(A, 8192), mode=7)[0] == N.S14_ERR_INVALID
    # official semantics belong to the fused expert entry points, not to a plain matvec
    ok_bufs = (buf(A, 16384), buf(A, 4194304), buf(A, 262144), buf(A, 8192))
    assert bind_mx(2048, 4096, *ok_bufs, mode=N.S14_MODE_OFFICIAL)[0] == N.S14_ERR_INVALID


def test_bind_fp8_dtypes_and_tiles(native):
    A = 0x20000
    rec = N.Fp8Dispatch()
    L = N.lib()
    # wq_a: bf16 x (8 KiB), f32 tile scales 8x32 (1 KiB)
    assert L.s14_bind_fp8(N.Shape(1024, 4096), buf(A, 8192), N.S14_X_BF16, buf(A, 4194304), buf(A, 1024),
                          N.S14_SCALE_F32, buf(A, 4096), N.S14_MODE_FAST, C.byref(rec)) == 0
    assert L.s14_bind_fp8(N.Shape(1024, 4096), buf(A, 8192), N.S14_X_F32, buf(A, 4194304), buf(A, 1024),
                          N.S14_SCALE_F32, buf(A, 4096), N.S14_MODE_FAST, C.byref(rec)) == N.S14_ERR_CAPACITY
    assert L.s14_bind_fp8(N.Shape(1024, 4096), buf(A, 16384), N.S14_X_F32, buf(A, 4194304), buf(A, 256),
                          N.S14_SCALE_UE8M0, buf(A, 4096), N.S14_MODE_EXACT, C.byref(rec)) == 0
    assert L.s14_bind_fp8(N.Shape(1024, 4096), buf(A, 16384), N.S14_X_F32, buf(A, 4194304), buf(A, 255),
                          N.S14_SCALE_UE8M0, buf(A, 4096), N.S14_MODE_EXACT, C.byref(rec)) == N.S14_ERR_CAPACITY
    assert L.s14_bind_fp8(N.Shape(0, 4096), buf(A, 16384), N.S14_X_F32, buf(A, 4194304), buf(A, 256),
                          N.S14_SCALE_UE8M0, buf(A, 4096), N.S14_MODE_EXACT, C.byref(rec)) == N.S14_ERR_SHAPE


def test_bind_elementwise(native):
    L = N.lib()
    A = 0x30000
    sw = N.SwigluDispatch()
    assert L.s14_bind_swiglu_limit(2048, buf(A, 8192), buf(A, 8192), buf(A, 8192), C.byref(sw)) == 0
    assert L.s14_bind_swiglu_limit(0, buf(A, 8192), buf(A, 8192), buf(A, 8192), C.byref(sw)) == N.S14_ERR_SHAPE
    assert L.s14_bind_swiglu_limit(2048, buf(A, 8192), buf(A, 8191), buf(A, 8192), C.byref(sw)) == N.S14_ERR_CAPACITY
    sc = N.ScaleDispatch()
    assert L.s14_bind_route_mix(4096, 0.17, buf(A, 16384), buf(A, 16384), C.byref(sc)) == 0
    for bad in (float("nan"), float("inf"), -0.5):
        assert L.s14_bind_route_mix(4096, bad, buf(A, 16384), buf(A, 16384), C.byref(sc)) == N.S14_ERR_INVALID
        assert L.s14_bind_moe_accumulate(4096, bad, buf(A, 16384), buf(A, 16384), C.byref(sc)) == N.S14_ERR_INVALID
    assert L.s14_bind_moe_accumulate(4096, 1.0, buf(A, 16384), buf(A, 16000), C.byref(sc)) == N.S14_ERR_CAPACITY


def test_cmd_requires_context(native):
    rec = N.Mxfp4Dispatch()
    assert N.lib().s14_cmd_mxfp4_matvec(None, None, C.byref(rec)) == N.S14_ERR_INVALID
    with pytest.raises(S14Error):
        N.check(N.lib().s14_expert_chain(None, None, None, None, 0.17, None, 0))


def test_bind_rejects_shapes_past_32bit_addressing(native):
    """The standalone matvecs address weights through 32-bit buffer
    descriptors: a shape whose weight (or scale) bytes reach 2^32 is a shape
    error at bind time, not a silent wrap on the device."""
    A = 0x40000
    big = 1 << 40
    # MXFP4: N * K / 2 = 2^32 bytes exactly -> rejected; one row fewer -> accepted
    n, k = 1 << 20, 1 << 13
    assert bind_mx(n, k, buf(A, 4 * k), buf(A, big), buf(A, big), buf(A, 4 * n))[0] == N.S14_ERR_SHAPE
    assert "addressable" in N.last_error()
    assert bind_mx(n - 1, k, buf(A, 4 * k), buf(A, big), buf(A, big), buf(A, 4 * n))[0] == 0
    # FP8: N * K = 2^32 bytes -> rejected; f32 tile scales count 4 bytes each
    rec = N.Fp8Dispatch()
    L = N.lib()
    assert L.s14_bind_fp8(N.Shape(1 << 16, 1 << 16), buf(A, 1 << 18), N.S14_X_F32, buf(A, big), buf(A, big),
                          N.S14_SCALE_UE8M0, buf(A, 1 << 18), N.S14_MODE_EXACT, C.byref(rec)) == N.S14_ERR_SHAPE
    assert L.s14_bind_fp8(N.Shape((1 << 16) - 128, 1 << 16), buf(A, 1 << 18), N.S14_X_F32, buf(A, big),
                          buf(A, big), N.S14_SCALE_F32, buf(A, 1 << 18), N.S14_MODE_EXACT, C.byref(rec)) == 0
