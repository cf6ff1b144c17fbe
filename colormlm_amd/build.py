"""Build libs14hip.so in-tree for gfx950.

    python -m colormlm_amd.build

One hipcc invocation compiles the kernels (s14_device.hip), the C ABI
(s14_api.cpp) and the host contracts (s14_pool.cpp) into
colormlm_amd/lib/libs14hip.so.  -ffp-contract=off keeps the exact kernels'
multiply-then-add unfused; packed FP32 instructions are disabled.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OUT = PKG / "lib" / "libs14hip.so"
SOURCES = ["s14_device.hip", "s14_prefill.hip", "s14_api.cpp", "s14_pool.cpp"]
ARCH = os.environ.get("S14_OFFLOAD_ARCH", "gfx950")


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required)")


def command(out: Path = OUT) -> list:
    return [
        hipcc(),
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-shared",
        "-ffp-contract=off",
        "-Xclang",
        "-target-feature",
        "-Xclang",
        "-packed-fp32-ops",
        "-Wall",
        f"-I{ROOT / 'include'}",
        f"-I{CSRC}",
        *[str(CSRC / s) for s in SOURCES],
        "-o",
        str(out),
    ]


def build(verbose: bool = False) -> Path:
    OUT.parent.mkdir(parents=True, exist_ok=True)
    tmp = OUT.with_suffix(".so.tmp")
    cmd = command(tmp)
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"hipcc failed with status {proc.returncode}")
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
