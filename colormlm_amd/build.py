"""Build libs14hip.so in-tree for gfx950.

    python -m colormlm_amd.build

Each source is compiled to an object of its own (in parallel), then linked
into colormlm_amd/lib/libs14hip.so:

- the gfx950 kernel files (*.hip) with -ffp-contract=off (the exact kernels'
  multiply-then-add must stay unfused) and with packed FP32 instructions
  disabled (-Xclang -target-feature -Xclang -packed-fp32-ops).  Clang has no
  driver spelling that forwards an -Xclang pair to the device pass alone, so
  the host pass of these files prints a one-line notice that it does not
  know the feature; the device code objects are what the flag is for;
- the host-only translation units (*.cpp: the C ABI, the pool and loader
  contracts) without that flag.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OUT = PKG / "lib" / "libs14hip.so"
OBJ = PKG / "lib" / "obj"
DEVICE_SOURCES = ["s14_device.hip", "s14_block.hip", "s14_prefill.hip", "s14_static.hip", "s14_linear.hip"]
HOST_SOURCES = ["s14_api.cpp", "s14_pool.cpp", "s14_loader.cpp"]
SOURCES = DEVICE_SOURCES + HOST_SOURCES
ARCH = os.environ.get("S14_OFFLOAD_ARCH", "gfx950")
NO_PACKED_FP32 = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required)")


def common_flags() -> list:
    return [f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off", "-Wall",
            f"-I{ROOT / 'include'}", f"-I{CSRC}"]


def compile_command(src: str) -> list:
    extra = NO_PACKED_FP32 if src.endswith(".hip") else []
    return [hipcc(), *common_flags(), *extra, "-c", str(CSRC / src), "-o", str(OBJ / (src + ".o"))]


def link_command(out: Path) -> list:
    return [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *[str(OBJ / (s + ".o")) for s in SOURCES],
            "-o", str(out)]


def command(out: Path = OUT) -> list:
    """The single-invocation form of the build (kept for reference): every
    source on one hipcc line."""
    return [hipcc(), *common_flags(), *NO_PACKED_FP32, "-shared",
            *[str(CSRC / s) for s in SOURCES], "-o", str(out)]


def _run(cmd: list, verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"hipcc failed with status {proc.returncode}: {' '.join(cmd[-3:])}")
    notes = [ln for ln in (proc.stdout + proc.stderr).splitlines()
             if ln.strip() and "packed-fp32-ops' is not a recognized feature" not in ln]
    if notes:
        sys.stderr.write("\n".join(notes) + "\n")


def build(verbose: bool = False) -> Path:
    OUT.parent.mkdir(parents=True, exist_ok=True)
    OBJ.mkdir(parents=True, exist_ok=True)
    jobs = min(len(SOURCES), int(os.environ.get("MAX_JOBS", "8")))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        for f in [ex.submit(_run, compile_command(s), verbose) for s in SOURCES]:
            f.result()
    tmp = OUT.with_suffix(".so.tmp")
    _run(link_command(tmp), verbose)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
