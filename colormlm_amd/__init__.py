"""MI355X-native (gfx950) S14 quantized expert path.

A from-scratch HIP implementation of the MXFP4 routed-expert chain, the
top-6 routed + shared MoE layer (batch 1 and the K<=8 verify block) and the
FP8 block-scaled projection matvec of colormlm's scheduler/ssd_inference,
behind a C ABI (include/s14_hip.h) that keeps the reference's dispatch API
and fenced page-pool contract.
"""

from . import _native  # noqa: F401
from ._native import S14Error  # noqa: F401

__all__ = ["S14Error", "s14", "pool", "build"]
