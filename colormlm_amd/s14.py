"""S14 dispatch API — Python face of the C ABI in include/s14_hip.h.

Mirrors the reference's Rust surface (scheduler/ssd_inference/src/
s14_vulkan.rs): ``S14MatvecShape`` (:39-114), ``validate_ue8m0_codes`` /
``validate_e4m3fn_codes`` (:143-156) and ``S14NumericPipelines`` with
``bind_*`` (:206-334) and ``cmd_*`` (:338-416).  Buffers are device tensors
(anything with ``data_ptr()``; torch tensors in practice); "recording" a
command enqueues the gfx950 kernel on a HIP stream (by default torch's
current stream, so ordering with torch work is implicit).

Beyond the reference's five kernels it exposes the fused entry points the
hot path uses: the single-expert chain, the top-6 + shared layer (route
given or computed on the device), the token-grouped verify block and the
router alone.
"""

from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from typing import Optional, Sequence

import numpy as np

from . import _native as N
from ._native import S14Error, check, lib

EXACT = N.S14_MODE_EXACT
FAST = N.S14_MODE_FAST
OFFICIAL = N.S14_MODE_OFFICIAL  # fused expert entry points and the prefill only


def _ptr(t) -> int:
    if t is None:
        return 0
    if isinstance(t, int):
        return t
    return int(t.data_ptr())


def _nbytes(t) -> int:
    if hasattr(t, "untyped_storage"):
        return int(t.numel() * t.element_size())
    return int(t.nbytes)


def buffer(t, nbytes: Optional[int] = None) -> N.Buffer:
    """GpuBuffer view (buffer.rs:21-70): device address + capacity."""
    if t is None:
        return N.Buffer(None, 0)
    return N.Buffer(_ptr(t), _nbytes(t) if nbytes is None else nbytes)


_TORCH_CUDA = []  # [torch] once torch with a visible GPU is found, [None] if not


def _stream(stream):
    """The stream to launch on: the caller's, else torch's current stream
    (so that torch events and work order against the library's), else the
    null stream."""
    if stream is not None:
        return stream
    if not _TORCH_CUDA:
        try:
            import torch

            _TORCH_CUDA.append(torch if torch.cuda.is_available() else None)
        except Exception:  # pragma: no cover - torch is optional for the ABI
            _TORCH_CUDA.append(None)
    torch = _TORCH_CUDA[0]
    return torch.cuda.current_stream().cuda_stream if torch is not None else None


class Context:
    """Device context: compute + copy streams and the kernel workspace
    (replaces VulkanContext + S14NumericPipelines::new)."""

    def __init__(self, device: int = 0):
        self._h = C.c_void_p()
        check(lib().s14_ctx_create(device, C.byref(self._h)))
        self.device = device

    @property
    def handle(self):
        return self._h

    @property
    def compute_stream(self) -> int:
        return int(lib().s14_ctx_compute_stream(self._h) or 0)

    @property
    def copy_stream(self) -> int:
        return int(lib().s14_ctx_copy_stream(self._h) or 0)

    def synchronize(self) -> None:
        check(lib().s14_ctx_synchronize(self._h))

    def enable_stage_timing(self, enable: bool = True) -> None:
        check(lib().s14_ctx_enable_stage_timing(self._h, 1 if enable else 0))

    def stage_times(self):
        """Kernel ms of {route (router + plan), phase 1, phase 2} of the last
        fused launch (0 for a stage it did not run)."""
        ms = (C.c_float * 4)()
        n = C.c_uint32()
        check(lib().s14_ctx_stage_times(self._h, ms, 4, C.byref(n)))
        return [float(ms[i]) for i in range(n.value)]

    def launch_status(self) -> None:
        """Raises S14Error if a routed launch since the last call found a
        page address of 0 (synchronises)."""
        check(lib().s14_launch_status(self._h))

    def destroy(self) -> None:
        if self._h:
            lib().s14_ctx_destroy(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


# ---------------------------------------------------------------------------
# shape / code contracts
# ---------------------------------------------------------------------------


@dataclass(frozen=True)
class S14MatvecShape:
    n: int
    k: int

    @classmethod
    def new(cls, n: int, k: int) -> "S14MatvecShape":
        if n == 0 or k == 0:
            raise S14Error(N.S14_ERR_SHAPE, "S14 matvec requires non-zero N and K")
        return cls(n, k)

    def _c(self) -> N.Shape:
        return N.Shape(self.n, self.k)

    def _bytes(self, fn) -> N.ShapeBytes:
        out = N.ShapeBytes()
        check(fn(self._c(), C.byref(out)))
        return out

    def validate_mxfp4(self) -> "S14MatvecShape":
        self._bytes(lib().s14_shape_validate_mxfp4)
        return self

    def validate_fp8(self) -> "S14MatvecShape":
        self._bytes(lib().s14_shape_validate_fp8)
        return self

    def fp32_input_bytes(self) -> int:
        return 4 * self.k

    def fp32_output_bytes(self) -> int:
        return 4 * self.n

    def mxfp4_weight_bytes(self) -> int:
        return int(self._bytes(lib().s14_shape_validate_mxfp4).weight_bytes)

    def mxfp4_scale_bytes(self) -> int:
        return int(self._bytes(lib().s14_shape_validate_mxfp4).scale_bytes)

    def fp8_weight_bytes(self) -> int:
        return int(self._bytes(lib().s14_shape_validate_fp8).weight_bytes)

    def fp8_scale_bytes(self) -> int:
        return int(self._bytes(lib().s14_shape_validate_fp8).scale_bytes)


def _host_u8(codes) -> np.ndarray:
    a = np.ascontiguousarray(np.asarray(codes, dtype=np.uint8).reshape(-1))
    return a


def validate_ue8m0_codes(codes) -> None:
    a = _host_u8(codes)
    bad = C.c_size_t()
    check(lib().s14_validate_ue8m0_codes(a.ctypes.data if a.size else None, a.size, C.byref(bad)))


def validate_e4m3fn_codes(codes) -> None:
    a = _host_u8(codes)
    bad = C.c_size_t()
    check(lib().s14_validate_e4m3fn_codes(a.ctypes.data if a.size else None, a.size, C.byref(bad)))


def page_layout(page_format: int = N.S14_PAGE_MXFP4, hidden: int = N.HIDDEN, inter: int = N.INTER) -> N.PageLayout:
    out = N.PageLayout()
    check(lib().s14_page_layout_get(page_format, hidden, inter, C.byref(out)))
    return out


# ---------------------------------------------------------------------------
# bind / cmd
# ---------------------------------------------------------------------------


class _Dispatch:
    def __init__(self, rec, keep):
        self.rec = rec
        self._keep = keep  # keep the bound tensors alive while the record exists

    @property
    def shape(self):
        return S14MatvecShape(self.rec.shape.n, self.rec.shape.k) if hasattr(self.rec, "shape") else None


class S14NumericPipelines:
    """S14NumericPipelines (s14_vulkan.rs:187-425) on a Context."""

    def __init__(self, ctx: Context):
        self.ctx = ctx

    # -- bind: validation only, like the reference's descriptor binding --
    def bind_mxfp4(self, shape: S14MatvecShape, x, packed_weight, weight_scale, y, mode: int = EXACT):
        rec = N.Mxfp4Dispatch()
        check(lib().s14_bind_mxfp4(shape._c(), buffer(x), buffer(packed_weight), buffer(weight_scale), buffer(y), mode, C.byref(rec)))
        return _Dispatch(rec, (x, packed_weight, weight_scale, y))

    def bind_fp8(self, shape: S14MatvecShape, x, weight, weight_scale, y, mode: int = EXACT):
        x_dtype = N.S14_X_BF16 if str(getattr(x, "dtype", "")).endswith("bfloat16") else N.S14_X_F32
        s_dtype = N.S14_SCALE_F32 if str(getattr(weight_scale, "dtype", "")).endswith("float32") else N.S14_SCALE_UE8M0
        rec = N.Fp8Dispatch()
        check(
            lib().s14_bind_fp8(
                shape._c(), buffer(x), x_dtype, buffer(weight), buffer(weight_scale), s_dtype, buffer(y), mode, C.byref(rec)
            )
        )
        return _Dispatch(rec, (x, weight, weight_scale, y))

    def bind_swiglu_limit(self, n: int, gate, up, y):
        rec = N.SwigluDispatch()
        check(lib().s14_bind_swiglu_limit(n, buffer(gate), buffer(up), buffer(y), C.byref(rec)))
        return _Dispatch(rec, (gate, up, y))

    def bind_route_mix(self, n: int, route_weight: float, expert, routed):
        rec = N.ScaleDispatch()
        check(lib().s14_bind_route_mix(n, route_weight, buffer(expert), buffer(routed), C.byref(rec)))
        return _Dispatch(rec, (expert, routed))

    def bind_moe_accumulate(self, n: int, weight: float, expert, accumulator):
        rec = N.ScaleDispatch()
        check(lib().s14_bind_moe_accumulate(n, weight, buffer(expert), buffer(accumulator), C.byref(rec)))
        return _Dispatch(rec, (expert, accumulator))

    # -- cmd: enqueue only --
    def cmd_mxfp4_matvec(self, dispatch, stream=None) -> None:
        check(lib().s14_cmd_mxfp4_matvec(self.ctx.handle, _stream(stream), C.byref(dispatch.rec)))

    def cmd_fp8_matvec(self, dispatch, stream=None) -> None:
        check(lib().s14_cmd_fp8_matvec(self.ctx.handle, _stream(stream), C.byref(dispatch.rec)))

    def cmd_swiglu_limit(self, dispatch, stream=None) -> None:
        check(lib().s14_cmd_swiglu_limit(self.ctx.handle, _stream(stream), C.byref(dispatch.rec)))

    def cmd_route_mix(self, dispatch, stream=None) -> None:
        check(lib().s14_cmd_route_mix(self.ctx.handle, _stream(stream), C.byref(dispatch.rec)))

    def cmd_moe_accumulate(self, dispatch, stream=None) -> None:
        check(lib().s14_cmd_moe_accumulate(self.ctx.handle, _stream(stream), C.byref(dispatch.rec)))

    def destroy(self) -> None:
        """Nothing to free: records hold no device objects."""

    # -- debug dequantisers (bit-exact decode checks) --
    def dequant_mxfp4(self, shape: S14MatvecShape, packed, scale, out, stream=None) -> None:
        check(lib().s14_dequant_mxfp4(self.ctx.handle, _stream(stream), shape._c(), _ptr(packed), _ptr(scale), _ptr(out)))

    def dequant_fp8(self, shape: S14MatvecShape, weight, scale, out, stream=None) -> None:
        s_dtype = N.S14_SCALE_F32 if str(getattr(scale, "dtype", "")).endswith("float32") else N.S14_SCALE_UE8M0
        check(
            lib().s14_dequant_fp8(self.ctx.handle, _stream(stream), shape._c(), _ptr(weight), _ptr(scale), s_dtype, _ptr(out))
        )


# ---------------------------------------------------------------------------
# fused entry points
# ---------------------------------------------------------------------------


@dataclass
class Router:
    """Router parameters: W_r f32 [n_experts, 4096], bias f32 [n_experts]."""

    weight: object
    bias: object
    n_experts: int = N.N_ROUTED_EXPERTS
    topk: int = N.TOP_K
    score_fn: int = N.S14_SCORE_SIGMOID
    route_scale: float = 1.0
    tid2eid: object = None  # hash routing: device int64 [vocab, topk]
    token_ids: object = None  # hash routing: device int32 [tokens]

    def c(self) -> N.Router:
        vocab = int(self.tid2eid.shape[0]) if self.tid2eid is not None else 0
        return N.Router(_ptr(self.weight), _ptr(self.bias), self.n_experts, self.topk, self.score_fn, self.route_scale,
                        _ptr(self.tid2eid), vocab, _ptr(self.token_ids))


def expert_chain(ctx: Context, page, x, route_w: float, y, mode: int = EXACT, stream=None) -> None:
    """w1/w3 matvec -> limit-10 SwiGLU -> w2 -> route-weight mix for one
    MXFP4 page (s14_vulkan_numeric.rs:1271-1498)."""
    check(lib().s14_expert_chain(ctx.handle, _stream(stream), _ptr(page), _ptr(x), route_w, _ptr(y), mode))


def moe_layer(
    ctx: Context,
    routed_pages: Sequence,
    route_weights: Sequence[float],
    shared_page,
    x,
    y,
    shared_format: int = N.S14_PAGE_MXFP4,
    mode: int = EXACT,
    stream=None,
) -> None:
    """Top-k routed + shared layer with the route given
    (s14_vulkan_numeric.rs:895-1269)."""
    k = len(routed_pages)
    pages = (C.c_void_p * max(1, k))(*[_ptr(p) for p in routed_pages])
    weights = (C.c_float * max(1, k))(*route_weights)
    check(
        lib().s14_moe_layer(
            ctx.handle, _stream(stream), k, pages, weights, _ptr(shared_page), shared_format, _ptr(x), _ptr(y), mode
        )
    )


def moe_layer_route(
    ctx: Context,
    router: Router,
    expert_pages,
    shared_page,
    x,
    y,
    ids_out=None,
    weights_out=None,
    shared_format: int = N.S14_PAGE_MXFP4,
    mode: int = EXACT,
    stream=None,
) -> None:
    """Router + top-6 routed + shared for one token.  expert_pages: device
    int64 tensor of n_experts page addresses."""
    r = router.c()
    check(
        lib().s14_moe_layer_route(
            ctx.handle,
            _stream(stream),
            C.byref(r),
            _ptr(expert_pages),
            _ptr(shared_page),
            shared_format,
            _ptr(x),
            _ptr(y),
            _ptr(ids_out),
            _ptr(weights_out),
            mode,
        )
    )


def moe_block_route(
    ctx: Context,
    tokens: int,
    router: Router,
    expert_pages,
    shared_page,
    x,
    y,
    ids_out=None,
    weights_out=None,
    shared_format: int = N.S14_PAGE_MXFP4,
    mode: int = EXACT,
    stream=None,
) -> None:
    """Speculative-verify block of `tokens` <= 8 through the routed layer,
    grouped expert-major."""
    r = router.c()
    check(
        lib().s14_moe_block_route(
            ctx.handle,
            _stream(stream),
            tokens,
            C.byref(r),
            _ptr(expert_pages),
            _ptr(shared_page),
            shared_format,
            _ptr(x),
            _ptr(y),
            _ptr(ids_out),
            _ptr(weights_out),
            mode,
        )
    )


def moe_block_route_noalloc(
    tokens: int,
    router: Router,
    expert_pages,
    shared_page,
    x,
    y,
    ids_out=None,
    weights_out=None,
    shared_format: int = N.S14_PAGE_MXFP4,
    mode: int = EXACT,
    stream=None,
) -> None:
    """moe_block_route without a context: the workspace is the library's
    static per-GPU scratch array (no device allocation in the call)."""
    r = router.c()
    check(
        lib().s14_moe_block_route_noalloc(
            _stream(stream),
            tokens,
            C.byref(r),
            _ptr(expert_pages),
            _ptr(shared_page),
            shared_format,
            _ptr(x),
            _ptr(y),
            _ptr(ids_out),
            _ptr(weights_out),
            mode,
        )
    )


def last_block_distinct(ctx: Context) -> int:
    n = C.c_uint32()
    check(lib().s14_last_block_distinct(ctx.handle, C.byref(n)))
    return int(n.value)


def route(ctx: Context, router: Router, tokens: int, x, scores_out=None, ids_out=None, weights_out=None, stream=None) -> None:
    r = router.c()
    check(
        lib().s14_route(
            ctx.handle, _stream(stream), C.byref(r), tokens, _ptr(x), _ptr(scores_out), _ptr(ids_out), _ptr(weights_out)
        )
    )


def moe_prefill(ctx: Context, tokens: int, router: Router, expert_pages, shared_page, x, y, ids_out=None,
                weights_out=None, stream=None, mode: int = EXACT) -> None:
    """Config 4: `tokens` rows of x [tokens, 4096] through the router and the
    top-6 routed + shared MXFP4 experts as grouped scaled-MFMA GEMMs on
    e4m3-requantised activations (per-32 E8M0); y [tokens, 4096].  Not
    order-exact (the MFMA's own summation), see the C header.  mode=OFFICIAL:
    the official expert semantics (group-128 act_quant, bf16 outputs, route
    weight before w2)."""
    r = router.c()
    check(
        lib().s14_moe_prefill(
            ctx.handle, _stream(stream), tokens, C.byref(r), _ptr(expert_pages), _ptr(shared_page), _ptr(x), _ptr(y),
            _ptr(ids_out), _ptr(weights_out), mode
        )
    )


def last_prefill_stats(ctx: Context) -> dict:
    """Distinct routed experts, largest tokens-per-expert and GEMM work items of
    the last prefill (synchronises)."""
    d, m, n = C.c_uint32(), C.c_uint32(), C.c_uint32()
    check(lib().s14_last_prefill_stats(ctx.handle, C.byref(d), C.byref(m), C.byref(n)))
    return {"distinct": int(d.value), "max_tokens_per_expert": int(m.value), "items": int(n.value)}


def last_prefill_view(ctx: Context) -> dict:
    """Host copies of the last prefill's intermediates (synchronises): xq/xs
    and, per pair, hq/hs (codes and E8M0 scales of the requantised SwiGLU
    output), down [pairs, 4096], pair_token and token_pair [tokens, 7]."""
    import torch

    v = N.PrefillView()
    check(lib().s14_last_prefill_view(ctx.handle, C.byref(v)))
    T, P = int(v.tokens), int(v.n_pairs)

    def grab(ptr, n, typestr):
        class _Dev:  # a device range exposed to torch without a copy
            __cuda_array_interface__ = {"shape": (n,), "typestr": typestr, "data": (int(ptr), False), "version": 2}

        return torch.as_tensor(_Dev(), device="cuda").cpu().numpy()

    n_items = int(v.n_items)
    items = grab(v.items, 3 * n_items, "<u4").reshape(n_items, 3)
    supers = N.INTER // 128
    # tile [u][half][plane][b][c][byte]: k 128 u + 32 b + 16 plane + byte of
    # column 16 half + c; scales [chunk][half][b][c][byte]: byte u' < 2 is
    # the E8M0 of super-step 2 chunk + u', block b
    tiles = grab(v.ht, n_items * supers * 4096, "|u1").reshape(n_items, supers, 2, 2, 4, 16, 16)
    tscales = grab(v.hts, n_items * (supers // 2) * 512, "|u1").reshape(n_items, supers // 2, 2, 4, 16, 4)
    hq = np.zeros((P, N.INTER), np.uint8)
    hs = np.zeros((P, N.INTER // 32), np.uint8)
    for i, (_, first, count) in enumerate(items.tolist()):
        blk = tiles[i].transpose(1, 4, 0, 3, 2, 5).reshape(32, N.INTER)  # [half][c][u][b][plane][byte]
        hq[first:first + count] = blk[:count]
        sc = tscales[i][..., :2].transpose(1, 3, 0, 4, 2).reshape(32, N.INTER // 32)  # [half][c][chunk][u'][b]
        hs[first:first + count] = sc[:count]
    return {
        "tokens": T,
        "n_pairs": P,
        "xq": grab(v.xq, T * N.HIDDEN, "|u1").reshape(T, N.HIDDEN),
        "xs": grab(v.xs, T * (N.HIDDEN // 32), "|u1").reshape(T, N.HIDDEN // 32),
        "hq": hq,
        "hs": hs,
        "items": items,
        "down": grab(v.down, P * N.HIDDEN, "<f4").reshape(P, N.HIDDEN),
        "pair_token": grab(v.pair_token, P, "<i4"),
        "token_pair": grab(v.token_pair, T * 7, "<i4").reshape(T, 7),
    }


def requant_e4m3(ctx: Context, rows: int, k: int, x, q, scales, stream=None) -> None:
    """e4m3 requant with per-32 E8M0 scales, natural layout (the prefill's
    activation quantiser as a standalone dispatch)."""
    check(lib().s14_requant_e4m3(ctx.handle, _stream(stream), rows, k, _ptr(x), _ptr(q), _ptr(scales)))


def act_quant_e4m3(ctx: Context, x, q, scales, group: int = 128, stream=None) -> None:
    """The official activation quant (l42_reference.py:390-403): x f32
    [rows, k] -> q e4m3 [rows, k] and E8M0 codes [rows, k / group]."""
    rows, k = (1, x.shape[0]) if x.dim() == 1 else (x.shape[0], x.shape[-1])
    check(lib().s14_act_quant_e4m3(ctx.handle, _stream(stream), rows, k, group, _ptr(x), _ptr(q), _ptr(scales)))


def fp8_linear(
    ctx: Context,
    x,
    x_scale,
    weight,
    weight_scale,
    y,
    bias=None,
    round_bf16: bool = False,
    mode: int = EXACT,
    stream=None,
) -> None:
    """fp8_linear (fp8.py:111-193): x e4m3 codes [m, k] (uint8), weight
    [n, k]; scales uint8 UE8M0 codes or float32, [m, ceil(k/128)] and
    [ceil(n/128), ceil(k/128)]; y float32 [m, n]."""
    m, k = (1, x.shape[0]) if x.dim() == 1 else (x.shape[0], x.shape[-1])
    n = weight.shape[0]

    def sdt(t):
        return N.S14_SCALE_F32 if str(t.dtype).endswith("float32") else N.S14_SCALE_UE8M0

    flags = N.S14_LINEAR_ROUND_BF16 if round_bf16 else 0
    check(
        lib().s14_fp8_linear(
            ctx.handle, _stream(stream), m, n, k, buffer(x), buffer(x_scale), sdt(x_scale), buffer(weight),
            buffer(weight_scale), sdt(weight_scale), buffer(bias), buffer(y), flags, mode
        )
    )


def fill_mxfp4_page(
    ctx: Context,
    page,
    seed: int,
    layer: int,
    expert: int,
    lo_exp: int = -10,
    hi_exp: int = -4,
    hidden: int = N.HIDDEN,
    inter: int = N.INTER,
    stream=None,
) -> None:
    """Device fill of one MXFP4 page with the seeded synthetic generator."""
    check(
        lib().s14_fill_mxfp4_page(
            ctx.handle, _stream(stream), _ptr(page), seed, layer, expert, hidden, inter, lo_exp, hi_exp
        )
    )


__all__ = [
    "EXACT",
    "OFFICIAL",
    "act_quant_e4m3",
    "fp8_linear",
    "FAST",
    "Context",
    "S14MatvecShape",
    "S14NumericPipelines",
    "S14Error",
    "Router",
    "buffer",
    "validate_ue8m0_codes",
    "validate_e4m3fn_codes",
    "page_layout",
    "expert_chain",
    "moe_layer",
    "moe_layer_route",
    "moe_block_route",
    "last_block_distinct",
    "route",
    "fill_mxfp4_page",
]
