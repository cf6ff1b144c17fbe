"""The C ABI library loads on a CPU-only host and exports every function
include/s14_hip.h declares; the Python binding declares the same set."""

from __future__ import annotations

import re
import subprocess
from pathlib import Path

from colormlm_amd import _native as N

ROOT = Path(__file__).resolve().parents[1]


def declared_functions():
    text = (ROOT / "include" / "s14_hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(s14_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol(native):
    out = subprocess.run(["nm", "-D", "--defined-only", str(N.library_path())], capture_output=True, text=True, check=True)
    exported = {line.split()[-1] for line in out.stdout.splitlines() if line.strip()}
    missing = [f for f in declared_functions() if f not in exported]
    assert not missing, missing


def test_binding_covers_the_header():
    assert sorted(N.SIGNATURES) == declared_functions()


def test_abi_version_and_error_channel(native):
    assert native.s14_abi_version() == 2
    rc = native.s14_shape_validate_mxfp4(N.Shape(0, 128), None)
    assert rc == N.S14_ERR_SHAPE
    assert "non-zero" in N.last_error()


def test_context_creation_fails_cleanly_without_a_gpu(native):
    import ctypes as C

    import torch

    if torch.cuda.is_available():
        return
    h = C.c_void_p()
    rc = native.s14_ctx_create(0, C.byref(h))
    assert rc in (N.S14_ERR_HIP, N.S14_ERR_INVALID) and not h.value


def test_loader_argument_checks(native):
    """ExpertLoader::new_with_staging_bytes's checks (expert_loader.rs:57-66),
    before any device call."""
    import ctypes as C

    from colormlm_amd import _native as N

    out = C.c_void_p()
    assert N.lib().s14_loader_create(None, 2, 1 << 20, C.byref(out)) == N.S14_ERR_INVALID
    assert N.lib().s14_loader_create(C.c_void_p(1), 0, 1 << 20, C.byref(out)) == N.S14_ERR_INVALID
    assert "pipeline depth" in N.last_error()
    assert N.lib().s14_loader_create(C.c_void_p(1), 2, 0, C.byref(out)) == N.S14_ERR_INVALID
    assert "staging slot size" in N.last_error()
    assert out.value is None
