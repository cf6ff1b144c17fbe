"""ctypes binding of libs14hip.so (the C ABI declared in include/s14_hip.h).

The shared library is built in-tree (``colormlm_amd/lib/libs14hip.so``) by
``colormlm_amd.build``.  Loading fails loudly if it is missing: there is no
CPU or PyTorch fallback for any entry point.
"""

from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

LIB_DIR = Path(__file__).resolve().parent / "lib"
LIB_PATH = LIB_DIR / "libs14hip.so"

# ---- status codes (s14_hip.h) ----
S14_OK = 0
S14_ERR_SHAPE = -1
S14_ERR_CAPACITY = -2
S14_ERR_NAN_CODE = -3
S14_ERR_STALE = -4
S14_ERR_POOL_FULL = -5
S14_ERR_INVALID = -6
S14_ERR_ROUTE = -7
S14_ERR_HIP = -8
S14_ERR_NOT_READY = -9

ERROR_NAMES = {
    S14_ERR_SHAPE: "shape",
    S14_ERR_CAPACITY: "capacity",
    S14_ERR_NAN_CODE: "nan_code",
    S14_ERR_STALE: "stale",
    S14_ERR_POOL_FULL: "pool_full",
    S14_ERR_INVALID: "invalid",
    S14_ERR_ROUTE: "route",
    S14_ERR_HIP: "hip",
    S14_ERR_NOT_READY: "not_ready",
}

S14_MODE_EXACT = 0
S14_MODE_FAST = 1
S14_MODE_OFFICIAL = 2
S14_LINEAR_ROUND_BF16 = 1
S14_X_F32 = 0
S14_X_BF16 = 1
S14_SCALE_UE8M0 = 0
S14_SCALE_F32 = 1
S14_PAGE_MXFP4 = 0
S14_PAGE_FP8 = 1
S14_SCORE_SIGMOID = 0
S14_SCORE_SQRT_SOFTPLUS = 1
S14_PROFILE_S14_TOP6 = 0
S14_PROFILE_FULL_DEPTH43_TOP6 = 1
S14_ROUTER_HASH = 0
S14_ROUTER_SCORE = 1
S14_ROUTED_EXPERT_KIND = 0x53
S14_SHARED_EXPERT_KIND = 0x54
EXPERT_PAGE_BYTES = 13_369_344
SHARED_EXPERT_PAGE_BYTES = 25_167_360
HIDDEN = 4096
INTER = 2048
N_ROUTED_EXPERTS = 256
TOP_K = 6
MAX_BLOCK_TOKENS = 8


class S14Error(RuntimeError):
    """A negative status from the C ABI, with the library's message."""

    def __init__(self, code: int, message: str):
        self.code = code
        self.kind = ERROR_NAMES.get(code, str(code))
        super().__init__(f"[{self.kind}] {message}")


# ---- structs (field order and types as in s14_hip.h) ----
class Shape(C.Structure):
    _fields_ = [("n", C.c_uint32), ("k", C.c_uint32)]


class ShapeBytes(C.Structure):
    _fields_ = [
        ("input_bytes", C.c_uint64),
        ("output_bytes", C.c_uint64),
        ("weight_bytes", C.c_uint64),
        ("scale_bytes", C.c_uint64),
    ]


class Buffer(C.Structure):
    _fields_ = [("ptr", C.c_void_p), ("bytes", C.c_uint64)]


class Mxfp4Dispatch(C.Structure):
    _fields_ = [
        ("shape", Shape),
        ("x", C.c_void_p),
        ("weight", C.c_void_p),
        ("scale", C.c_void_p),
        ("y", C.c_void_p),
        ("mode", C.c_int),
    ]


class Fp8Dispatch(C.Structure):
    _fields_ = [
        ("shape", Shape),
        ("x", C.c_void_p),
        ("weight", C.c_void_p),
        ("scale", C.c_void_p),
        ("y", C.c_void_p),
        ("x_dtype", C.c_int),
        ("scale_dtype", C.c_int),
        ("mode", C.c_int),
    ]


class SwigluDispatch(C.Structure):
    _fields_ = [("n", C.c_uint32), ("gate", C.c_void_p), ("up", C.c_void_p), ("y", C.c_void_p)]


class ScaleDispatch(C.Structure):
    _fields_ = [("n", C.c_uint32), ("weight", C.c_float), ("expert", C.c_void_p), ("out", C.c_void_p)]


class PageLayout(C.Structure):
    _fields_ = [
        ("w1", C.c_uint64),
        ("s1", C.c_uint64),
        ("w3", C.c_uint64),
        ("s3", C.c_uint64),
        ("w2", C.c_uint64),
        ("s2", C.c_uint64),
        ("total_bytes", C.c_uint64),
    ]


class Router(C.Structure):
    _fields_ = [
        ("weight", C.c_void_p),
        ("bias", C.c_void_p),
        ("n_experts", C.c_uint32),
        ("topk", C.c_uint32),
        ("score_fn", C.c_int),
        ("route_scale", C.c_float),
        ("tid2eid", C.c_void_p),
        ("vocab", C.c_uint32),
        ("token_ids", C.c_void_p),
    ]


class PrefillView(C.Structure):
    _fields_ = [
        ("xq", C.c_void_p),
        ("xs", C.c_void_p),
        ("ht", C.c_void_p),
        ("hts", C.c_void_p),
        ("down", C.c_void_p),
        ("pair_token", C.c_void_p),
        ("token_pair", C.c_void_p),
        ("items", C.c_void_p),
        ("tokens", C.c_uint32),
        ("n_pairs", C.c_uint32),
        ("n_items", C.c_uint32),
    ]


class ExpertKeyC(C.Structure):
    _fields_ = [("layer", C.c_uint32), ("kind", C.c_uint8), ("slot", C.c_uint32)]


class SlotBindingC(C.Structure):
    _fields_ = [("key", ExpertKeyC), ("slot", C.c_uint32), ("generation", C.c_uint64)]


class LoadingReservationC(C.Structure):
    _fields_ = [
        ("key", ExpertKeyC),
        ("slot", C.c_uint32),
        ("generation", C.c_uint64),
        ("has_evicted", C.c_int),
        ("evicted", ExpertKeyC),
    ]


class RouteDecisionC(C.Structure):
    _fields_ = [
        ("layer", C.c_uint8),
        ("kind", C.c_int),
        ("n", C.c_uint32),
        ("expert_ids", C.c_uint16 * 16),
        ("weights", C.c_float * 16),
    ]


P = C.c_void_p
I = C.c_int
U32 = C.c_uint32
U64 = C.c_uint64
F = C.c_float

# name -> (restype, argtypes); the complete export list of s14_hip.h
SIGNATURES = {
    "s14_last_error": (C.c_char_p, []),
    "s14_abi_version": (I, []),
    "s14_shape_validate_mxfp4": (I, [Shape, C.POINTER(ShapeBytes)]),
    "s14_shape_validate_fp8": (I, [Shape, C.POINTER(ShapeBytes)]),
    "s14_validate_ue8m0_codes": (I, [P, C.c_size_t, C.POINTER(C.c_size_t)]),
    "s14_validate_e4m3fn_codes": (I, [P, C.c_size_t, C.POINTER(C.c_size_t)]),
    "s14_ctx_create": (I, [I, C.POINTER(P)]),
    "s14_ctx_destroy": (None, [P]),
    "s14_ctx_compute_stream": (P, [P]),
    "s14_ctx_copy_stream": (P, [P]),
    "s14_ctx_synchronize": (I, [P]),
    "s14_ctx_enable_stage_timing": (I, [P, I]),
    "s14_ctx_stage_times": (I, [P, C.POINTER(F), U32, C.POINTER(U32)]),
    "s14_bind_mxfp4": (I, [Shape, Buffer, Buffer, Buffer, Buffer, I, C.POINTER(Mxfp4Dispatch)]),
    "s14_bind_fp8": (I, [Shape, Buffer, I, Buffer, Buffer, I, Buffer, I, C.POINTER(Fp8Dispatch)]),
    "s14_bind_swiglu_limit": (I, [U32, Buffer, Buffer, Buffer, C.POINTER(SwigluDispatch)]),
    "s14_bind_route_mix": (I, [U32, F, Buffer, Buffer, C.POINTER(ScaleDispatch)]),
    "s14_bind_moe_accumulate": (I, [U32, F, Buffer, Buffer, C.POINTER(ScaleDispatch)]),
    "s14_cmd_mxfp4_matvec": (I, [P, P, C.POINTER(Mxfp4Dispatch)]),
    "s14_cmd_fp8_matvec": (I, [P, P, C.POINTER(Fp8Dispatch)]),
    "s14_cmd_swiglu_limit": (I, [P, P, C.POINTER(SwigluDispatch)]),
    "s14_cmd_route_mix": (I, [P, P, C.POINTER(ScaleDispatch)]),
    "s14_cmd_moe_accumulate": (I, [P, P, C.POINTER(ScaleDispatch)]),
    "s14_dequant_mxfp4": (I, [P, P, Shape, P, P, P]),
    "s14_dequant_fp8": (I, [P, P, Shape, P, P, I, P]),
    "s14_page_layout_get": (I, [I, U32, U32, C.POINTER(PageLayout)]),
    "s14_expert_chain": (I, [P, P, P, P, F, P, I]),
    "s14_moe_layer": (I, [P, P, U32, C.POINTER(P), C.POINTER(F), P, I, P, P, I]),
    "s14_moe_layer_route": (I, [P, P, C.POINTER(Router), P, P, I, P, P, P, P, I]),
    "s14_moe_block_route": (I, [P, P, U32, C.POINTER(Router), P, P, I, P, P, P, P, I]),
    "s14_last_block_distinct": (I, [P, C.POINTER(U32)]),
    "s14_launch_status": (I, [P]),
    "s14_moe_block_route_noalloc": (I, [P, U32, C.POINTER(Router), P, P, I, P, P, P, P, I]),
    "s14_noalloc_scratch_bytes": (C.c_uint64, []),
    "s14_route": (I, [P, P, C.POINTER(Router), U32, P, P, P, P]),
    "s14_moe_prefill": (I, [P, P, U32, C.POINTER(Router), P, P, P, P, P, P, I]),
    "s14_last_prefill_stats": (I, [P, C.POINTER(U32), C.POINTER(U32), C.POINTER(U32)]),
    "s14_requant_e4m3": (I, [P, P, U32, U32, P, P, P]),
    "s14_act_quant_e4m3": (I, [P, P, U32, U32, U32, P, P, P]),
    "s14_fp8_linear": (I, [P, P, U32, U32, U32, Buffer, Buffer, I, Buffer, Buffer, I, Buffer, Buffer, I, I]),
    "s14_last_prefill_view": (I, [P, C.POINTER(PrefillView)]),
    "s14_fill_mxfp4_page": (I, [P, P, P, U64, U32, U32, U32, U32, I, I]),
    "s14_pool_create": (I, [P, U32, U64, C.POINTER(P)]),
    "s14_pool_destroy": (None, [P]),
    "s14_pool_capacity": (U32, [P]),
    "s14_pool_slot_bytes": (U64, [P]),
    "s14_pool_n_loaded": (U32, [P]),
    "s14_pool_total_bytes": (U64, [P]),
    "s14_pool_slot_offset": (U64, [P, U32]),
    "s14_pool_slot_ptr": (P, [P, U32]),
    "s14_pool_lookup": (I, [P, ExpertKeyC, C.POINTER(U32)]),
    "s14_pool_lookup_and_pin": (I, [P, ExpertKeyC, C.POINTER(I), C.POINTER(SlotBindingC)]),
    "s14_pool_reserve_loading": (I, [P, ExpertKeyC, C.POINTER(U32), C.POINTER(I), C.POINTER(ExpertKeyC)]),
    "s14_pool_reserve_loading_generation": (I, [P, ExpertKeyC, C.POINTER(LoadingReservationC)]),
    "s14_pool_mark_ready": (I, [P, U32, ExpertKeyC]),
    "s14_pool_validate_publish_batch": (I, [P, C.POINTER(LoadingReservationC), C.c_size_t]),
    "s14_pool_publish_batch_and_pin": (
        I,
        [P, C.POINTER(LoadingReservationC), C.c_size_t, C.POINTER(SlotBindingC)],
    ),
    "s14_pool_validate_binding": (I, [P, SlotBindingC]),
    "s14_pool_release_after_compute_fence": (I, [P, SlotBindingC]),
    "s14_pool_cancel_loading": (None, [P, U32, ExpertKeyC]),
    "s14_pool_cancel_reservation": (I, [P, LoadingReservationC]),
    "s14_pool_upload": (I, [P, P, C.POINTER(LoadingReservationC), P, U64, C.POINTER(P)]),
    "s14_fence_record": (I, [P, P, C.POINTER(P)]),
    "s14_fence_query": (I, [P]),
    "s14_fence_wait": (I, [P]),
    "s14_fence_destroy": (None, [P]),
    "s14_route_validate_for": (I, [C.POINTER(RouteDecisionC), I, F]),
    "s14_moe_pages_create": (I, [P, P, I, I, F, C.POINTER(P)]),
    "s14_moe_pages_destroy": (None, [P]),
    "s14_moe_pages_begin_after_official_route": (I, [P, C.POINTER(RouteDecisionC), C.POINTER(P)]),
    "s14_route_load_batch_size": (U32, [P]),
    "s14_route_load_batch_page": (
        I,
        [P, U32, C.POINTER(I), C.POINTER(LoadingReservationC), C.POINTER(SlotBindingC)],
    ),
    "s14_moe_pages_publish_after_transfer_fence": (I, [P, P, C.POINTER(P)]),
    "s14_moe_lease_batch_bindings": (I, [P, C.POINTER(SlotBindingC), U32, C.POINTER(SlotBindingC)]),
    "s14_moe_pages_release_after_compute_fence": (I, [P, P]),
    "s14_moe_pages_cancel": (I, [P, P]),
    "s14_route_load_batch_shared_reservation": (I, [P, C.POINTER(LoadingReservationC)]),
    "s14_loader_create": (I, [P, U32, U64, C.POINTER(P)]),
    "s14_loader_destroy": (None, [P]),
    "s14_loader_enqueue": (I, [P, P, ExpertKeyC, U64, P, P, C.POINTER(U32)]),
    "s14_loader_enqueue_from_buf": (I, [P, P, ExpertKeyC, P, U64, C.POINTER(U32)]),
    "s14_loader_wait_all": (I, [P, P]),
    "s14_loader_batch_enqueue": (I, [P, P, C.POINTER(ExpertKeyC), C.POINTER(U64), C.c_size_t, P, P, C.POINTER(U32)]),
    "s14_loader_batch_enqueue_from_bufs": (
        I,
        [P, P, C.POINTER(ExpertKeyC), C.POINTER(P), C.POINTER(U64), C.c_size_t, C.POINTER(U32)],
    ),
    "s14_loader_stats": (I, [P, C.POINTER(U64), C.POINTER(U64), C.POINTER(U32)]),
}

# s14_read_fn: int (*)(void *user, s14_expert_key key, void *dst, uint64_t bytes)
READ_FN = C.CFUNCTYPE(C.c_int, C.c_void_p, ExpertKeyC, C.c_void_p, C.c_uint64)

_lib = None


def library_path() -> Path:
    return Path(os.environ.get("S14_HIP_LIB", LIB_PATH))


def lib() -> C.CDLL:
    """Load libs14hip.so once and attach the declared signatures."""
    global _lib
    if _lib is not None:
        return _lib
    path = library_path()
    if not path.exists():
        raise ImportError(
            f"{path} is not built; run `python -m colormlm_amd.build` (there is no fallback path)"
        )
    handle = C.CDLL(str(path))
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = restype
        fn.argtypes = argtypes
    _lib = handle
    return handle


def last_error() -> str:
    msg = lib().s14_last_error()
    return msg.decode("utf-8", "replace") if msg else ""


def check(rc: int) -> int:
    if rc < 0:
        raise S14Error(rc, last_error())
    return rc
