"""CPU oracle (test infrastructure only) — ctypes wrapper of libs14oracle.so.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this package, and only as the checker.  The C source (s14_oracle.c) restates
the reference CPU F32 oracle of scheduler/ssd_inference/examples/
s14_vulkan_numeric.rs:1543-1784 in its exact operation order; see the header
of s14_oracle.h for what pins each function.
"""

from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "libs14oracle.so"

HIDDEN = 4096
INTER = 2048
SCORE_SIGMOID = 0
SCORE_SQRT_SOFTPLUS = 1

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        _lib = C.CDLL(str(LIB))
        _declare(_lib)
    return _lib


P = C.c_void_p
U32, U64, I, F, D = C.c_uint32, C.c_uint64, C.c_int, C.c_float, C.c_double


class _Expert(C.Structure):
    _fields_ = [(n, P) for n in ("w1", "s1", "w3", "s3", "w2", "s2")]


class ErrorStats(C.Structure):
    _fields_ = [
        ("max_abs", C.c_float),
        ("mean_abs", C.c_double),
        ("rmse", C.c_double),
        ("max_rel_abs_ref_gt_1e_5", C.c_float),
        ("finite", C.c_int),
    ]

    def as_dict(self):
        return {
            "max_abs": float(self.max_abs),
            "mean_abs": float(self.mean_abs),
            "rmse": float(self.rmse),
            "max_rel_abs_ref_gt_1e_5": float(self.max_rel_abs_ref_gt_1e_5),
            "finite": bool(self.finite),
        }


def _declare(L):
    sig = {
        "s14o_e2m1": (F, [C.c_uint8]),
        "s14o_ue8m0": (F, [C.c_uint8]),
        "s14o_e4m3fn": (F, [C.c_uint8]),
        "s14o_bf16_to_f32": (F, [C.c_uint16]),
        "s14o_f32_to_e4m3fn_rne_sat": (C.c_uint8, [F]),
        "s14o_f32_to_bf16_rne": (C.c_uint16, [F]),
        "s14o_dequant_mxfp4": (None, [U32, U32, P, P, P]),
        "s14o_dequant_fp8_ue8m0": (None, [U32, U32, P, P, P]),
        "s14o_mxfp4_matvec": (None, [U32, U32, P, P, P, P]),
        "s14o_fp8_matvec_ue8m0": (None, [U32, U32, P, P, P, P]),
        "s14o_fp8_matvec_f32scale_bf16x": (None, [U32, U32, P, P, P, P]),
        "s14o_swiglu_limit": (None, [U32, P, P, P]),
        "s14o_mxfp4_expert_down": (None, [U32, U32, P, C.POINTER(_Expert), P]),
        "s14o_fp8_expert_down": (None, [U32, U32, P, C.POINTER(_Expert), P]),
        "s14o_expert_chain": (None, [U32, U32, P, C.POINTER(_Expert), F, P]),
        "s14o_moe_layer": (None, [U32, U32, P, U32, P, P, P, P, P]),
        "s14o_router_logits": (None, [U32, U32, P, P, P]),
        "s14o_route": (None, [U32, U32, P, P, P, I, U32, F, P, P, P]),
        "s14o_route_hash": (I, [U32, U32, P, P, P, P, I, U32, F, P, P, P]),
        "s14o_expert_official": (None, [U32, U32, P, P, P, F, I, P]),
        "s14o_moe_layer_official": (None, [U32, U32, P, U32, P, P, P, P, P, P]),
        "s14o_fp8_linear": (None, [U32, U32, U32, P, P, I, P, P, I, P, I, P]),
        "s14o_route_valid": (I, [P, P, U32, U32, F]),
        "s14o_error_stats_compute": (None, [C.c_size_t, P, P, C.POINTER(ErrorStats)]),
        "s14o_requant_e4m3": (None, [U32, U32, U32, P, P, P]),
        "s14o_dequant_requant": (None, [U32, U32, U32, P, P, P]),
        "s14o_mxfp4_expert_down_requant": (None, [U32, U32, U32, P, C.POINTER(_Expert), P]),
        "s14o_num_threads": (I, []),
        "s14o_set_num_threads": (None, [I]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be contiguous"
    return a.ctypes.data


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _u8(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.uint8)


# ---------------------------------------------------------------------------
# decoders / encoders
# ---------------------------------------------------------------------------


def e2m1(code: int) -> float:
    return float(np.float32(lib().s14o_e2m1(code)))


def ue8m0(code: int) -> np.float32:
    return np.float32(lib().s14o_ue8m0(code))


def e4m3fn(code: int) -> np.float32:
    return np.float32(lib().s14o_e4m3fn(code))


def e4m3fn_encode(v: float) -> int:
    return int(lib().s14o_f32_to_e4m3fn_rne_sat(float(np.float32(v))))


def bf16_encode(v: float) -> int:
    return int(lib().s14o_f32_to_bf16_rne(float(np.float32(v))))


def dequant_mxfp4(packed: np.ndarray, scale: np.ndarray) -> np.ndarray:
    packed, scale = _u8(packed), _u8(scale)
    n, pk = packed.shape
    out = np.empty((n, pk * 2), dtype=np.float32)
    lib().s14o_dequant_mxfp4(n, pk * 2, _p(packed), _p(scale), _p(out))
    return out


def dequant_fp8_ue8m0(w: np.ndarray, scale: np.ndarray) -> np.ndarray:
    w, scale = _u8(w), _u8(scale)
    n, k = w.shape
    out = np.empty((n, k), dtype=np.float32)
    lib().s14o_dequant_fp8_ue8m0(n, k, _p(w), _p(scale), _p(out))
    return out


# ---------------------------------------------------------------------------
# matvecs, swiglu, experts, layer
# ---------------------------------------------------------------------------


def mxfp4_matvec(x, packed, scale) -> np.ndarray:
    x, packed, scale = _f32(x), _u8(packed), _u8(scale)
    n = packed.shape[0]
    k = x.shape[0]
    y = np.empty(n, dtype=np.float32)
    lib().s14o_mxfp4_matvec(n, k, _p(x), _p(packed), _p(scale), _p(y))
    return y


def fp8_matvec_ue8m0(x, w, scale) -> np.ndarray:
    x, w, scale = _f32(x), _u8(w), _u8(scale)
    n, k = w.shape
    y = np.empty(n, dtype=np.float32)
    lib().s14o_fp8_matvec_ue8m0(n, k, _p(x), _p(w), _p(scale), _p(y))
    return y


def fp8_matvec_f32scale_bf16x(x_bf16, w, scale) -> np.ndarray:
    x = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    w, scale = _u8(w), _f32(scale)
    n, k = w.shape
    y = np.empty(n, dtype=np.float32)
    lib().s14o_fp8_matvec_f32scale_bf16x(n, k, _p(x), _p(w), _p(scale), _p(y))
    return y


def swiglu_limit(gate, up) -> np.ndarray:
    gate, up = _f32(gate), _f32(up)
    h = np.empty_like(gate)
    lib().s14o_swiglu_limit(gate.size, _p(gate), _p(up), _p(h))
    return h


def page_offsets(fmt: str = "mxfp4", hidden: int = HIDDEN, inter: int = INTER):
    """[w1|s1|w3|s3|w2|s2] byte offsets of an expert page."""
    if fmt == "mxfp4":
        up_w, up_s = inter * hidden // 2, inter * hidden // 32
        dn_w, dn_s = hidden * inter // 2, hidden * inter // 32
    else:
        up_w, up_s = inter * hidden, -(-inter // 128) * -(-hidden // 128)
        dn_w, dn_s = hidden * inter, -(-hidden // 128) * -(-inter // 128)
    o = {"w1": 0}
    o["s1"] = up_w
    o["w3"] = o["s1"] + up_s
    o["s3"] = o["w3"] + up_w
    o["w2"] = o["s3"] + up_s
    o["s2"] = o["w2"] + dn_w
    o["total"] = o["s2"] + dn_s
    return o


def _expert(page: np.ndarray, fmt: str, hidden: int, inter: int) -> _Expert:
    o = page_offsets(fmt, hidden, inter)
    assert page.dtype == np.uint8 and page.size >= o["total"] and page.flags["C_CONTIGUOUS"]
    base = page.ctypes.data
    return _Expert(*[base + o[k] for k in ("w1", "s1", "w3", "s3", "w2", "s2")])


def expert_down(x, page, fmt="mxfp4", hidden=HIDDEN, inter=INTER) -> np.ndarray:
    x = _f32(x)
    e = _expert(page, fmt, hidden, inter)
    out = np.empty(hidden, dtype=np.float32)
    fn = lib().s14o_mxfp4_expert_down if fmt == "mxfp4" else lib().s14o_fp8_expert_down
    fn(hidden, inter, _p(x), C.byref(e), _p(out))
    return out


def expert_chain(x, page, route_w: float, hidden=HIDDEN, inter=INTER) -> np.ndarray:
    x = _f32(x)
    e = _expert(page, "mxfp4", hidden, inter)
    y = np.empty(hidden, dtype=np.float32)
    lib().s14o_expert_chain(hidden, inter, _p(x), C.byref(e), float(route_w), _p(y))
    return y


def moe_layer(x, routed_pages, weights, shared_page, shared_fmt="mxfp4", hidden=HIDDEN, inter=INTER) -> np.ndarray:
    x = _f32(x)
    k = len(routed_pages)
    arr = (_Expert * max(1, k))(*[_expert(p, "mxfp4", hidden, inter) for p in routed_pages])
    w = _f32(weights)
    y = np.empty(hidden, dtype=np.float32)
    sh = _expert(shared_page, shared_fmt, hidden, inter)
    sh_mx = C.byref(sh) if shared_fmt == "mxfp4" else None
    sh_f8 = C.byref(sh) if shared_fmt != "mxfp4" else None
    lib().s14o_moe_layer(hidden, inter, _p(x), k, C.cast(arr, P), _p(w), sh_mx, sh_f8, _p(y))
    return y


def expert_official(x, page, weight=1.0, apply_weight=True, fmt="mxfp4", hidden=HIDDEN, inter=INTER) -> np.ndarray:
    """One expert under the official semantics (executor.py:712-744): bf16
    linear outputs, group-128 e4m3 activation requant before every linear,
    the route weight applied to h before w2 (routed experts only)."""
    x = _f32(x)
    e = _expert(page, fmt, hidden, inter)
    out = np.empty(hidden, dtype=np.float32)
    mx = C.byref(e) if fmt == "mxfp4" else None
    f8 = C.byref(e) if fmt != "mxfp4" else None
    lib().s14o_expert_official(hidden, inter, _p(x), mx, f8, float(weight), int(apply_weight), _p(out))
    return out


def moe_layer_official(x, routed_pages, weights, shared_page, shared_fmt="mxfp4", hidden=HIDDEN, inter=INTER,
                       with_f32=False):
    """Official layer: bf16(sum of the routed experts' outputs in route order,
    then the shared expert's, in f32); shared_page None: routed experts only."""
    x = _f32(x)
    k = len(routed_pages)
    arr = (_Expert * max(1, k))(*[_expert(p, "mxfp4", hidden, inter) for p in routed_pages])
    w = _f32(weights)
    y = np.empty(hidden, dtype=np.float32)
    y32 = np.empty(hidden, dtype=np.float32)
    sh = _expert(shared_page, shared_fmt, hidden, inter) if shared_page is not None else None
    sh_mx = C.byref(sh) if sh is not None and shared_fmt == "mxfp4" else None
    sh_f8 = C.byref(sh) if sh is not None and shared_fmt != "mxfp4" else None
    lib().s14o_moe_layer_official(hidden, inter, _p(x), k, C.cast(arr, P), _p(w), sh_mx, sh_f8, _p(y), _p(y32))
    return (y, y32) if with_f32 else y


def router_logits(wr, x) -> np.ndarray:
    wr, x = _f32(wr), _f32(x)
    z = np.empty(wr.shape[0], dtype=np.float32)
    lib().s14o_router_logits(wr.shape[0], wr.shape[1], _p(wr), _p(x), _p(z))
    return z


def route(wr, bias, x, score_fn=SCORE_SIGMOID, topk=6, route_scale=1.0):
    wr, bias, x = _f32(wr), _f32(bias), _f32(x)
    n = wr.shape[0]
    scores = np.empty(n, dtype=np.float32)
    ids = np.empty(topk, dtype=np.uint16)
    w = np.empty(topk, dtype=np.float32)
    lib().s14o_route(n, wr.shape[1], _p(wr), _p(bias), _p(x), score_fn, topk, float(route_scale), _p(scores), _p(ids), _p(w))
    return scores, ids, w


def route_hash(wr, bias, x, row, score_fn=SCORE_SIGMOID, topk=6, route_scale=1.0):
    """Hash route of one token from its tid2eid row (executor.py:643-667):
    (scores, ids, weights), or (scores, None, None) when the row has an entry
    outside [0, n_experts) or a repeated one."""
    wr, bias, x = _f32(wr), _f32(bias), _f32(x)
    row = np.ascontiguousarray(row, dtype=np.int64)
    n = wr.shape[0]
    scores = np.empty(n, dtype=np.float32)
    ids = np.empty(topk, dtype=np.uint16)
    w = np.empty(topk, dtype=np.float32)
    bad = lib().s14o_route_hash(n, wr.shape[1], _p(wr), _p(bias), _p(x), _p(row), score_fn, topk,
                                float(route_scale), _p(scores), _p(ids), _p(w))
    return (scores, None, None) if bad else (scores, ids, w)


def route_valid(ids, w, n_experts=256, route_scale=1.0) -> bool:
    """RouteDecision::validate_for's id and weight checks (runner.rs:128-180)."""
    ids = np.ascontiguousarray(ids, dtype=np.uint16)
    w = _f32(w)
    return bool(lib().s14o_route_valid(_p(ids), _p(w), ids.size, n_experts, float(route_scale)))


def fp8_linear(x, x_scale, w, w_scale, bias=None, round_bf16=False) -> np.ndarray:
    """fp8_linear (fp8.py:111-193) with each group's products summed k
    ascending: x, w e4m3 codes [m, k] / [n, k]; scales UE8M0 codes (uint8)
    or float32, [m, ceil(k/128)] and [ceil(n/128), ceil(k/128)]."""
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.uint8)
    w = np.ascontiguousarray(w, dtype=np.uint8)
    m, k = x.shape
    n = w.shape[0]
    assert w.shape[1] == k
    g = (k + 127) // 128
    xs = np.ascontiguousarray(np.atleast_2d(x_scale))
    ws = np.ascontiguousarray(np.atleast_2d(w_scale))
    assert xs.shape == (m, g) and ws.shape == ((n + 127) // 128, g)
    assert xs.dtype in (np.uint8, np.float32) and ws.dtype in (np.uint8, np.float32)
    b = None if bias is None else _f32(bias)
    y = np.empty((m, n), dtype=np.float32)
    lib().s14o_fp8_linear(m, n, k, _p(x), _p(xs), int(xs.dtype == np.float32), _p(w), _p(ws),
                          int(ws.dtype == np.float32), None if b is None else _p(b), int(bool(round_bf16)), _p(y))
    return y


def error_stats(actual, expected) -> dict:
    a, e = _f32(actual).reshape(-1), _f32(expected).reshape(-1)
    assert a.size == e.size and a.size > 0
    st = ErrorStats()
    lib().s14o_error_stats_compute(a.size, _p(a), _p(e), C.byref(st))
    return st.as_dict()


def requant_e4m3(x, group: int = 32):
    x = _f32(np.atleast_2d(x))
    rows, k = x.shape
    q = np.empty((rows, k), dtype=np.uint8)
    s = np.empty((rows, k // group), dtype=np.uint8)
    lib().s14o_requant_e4m3(rows, k, group, _p(x), _p(q), _p(s))
    return q, s


def dequant_requant(q, scale_codes, group: int = 32):
    q = np.ascontiguousarray(np.atleast_2d(q), dtype=np.uint8)
    sc = np.ascontiguousarray(np.atleast_2d(scale_codes), dtype=np.uint8)
    rows, k = q.shape
    out = np.empty((rows, k), dtype=np.float32)
    lib().s14o_dequant_requant(rows, k, group, _p(q), _p(sc), _p(out))
    return out


def expert_down_requant(x, page, group: int = 32, hidden=HIDDEN, inter=INTER) -> np.ndarray:
    """Prefill expert on requantised activations (config 4), route weight not applied."""
    x = _f32(x)
    e = _expert(page, "mxfp4", hidden, inter)
    out = np.empty(hidden, dtype=np.float32)
    lib().s14o_mxfp4_expert_down_requant(hidden, inter, group, _p(x), C.byref(e), _p(out))
    return out


def moe_prefill_token(x, routed_pages, weights, shared_page, group: int = 32, hidden=HIDDEN, inter=INTER) -> np.ndarray:
    """One token of the config-4 layer: acc = 0; acc += w_i * down_i in route
    order; acc += shared_down (s14_vulkan_numeric.rs:929-946 order), each
    down computed by expert_down_requant."""
    acc = np.zeros(hidden, dtype=np.float32)
    for p, w in zip(routed_pages, _f32(weights)):
        acc = (acc + np.float32(w) * expert_down_requant(x, p, group, hidden, inter)).astype(np.float32)
    return (acc + expert_down_requant(x, shared_page, group, hidden, inter)).astype(np.float32)


def set_num_threads(n: int) -> None:
    lib().s14o_set_num_threads(n)


def num_threads() -> int:
    return int(lib().s14o_num_threads())
