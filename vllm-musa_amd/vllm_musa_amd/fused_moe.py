"""Fused-MoE host driver (reference: vllm_musa/model_executor/layers/fused_moe/fused_moe.py).

This module keeps the reference's Python entry points:
  moe_align_block_size(topk_ids, block_size, num_experts, expert_map=None, pad_sorted_ids=False)
      upstream wrapper of the _moe_C op (sizing as fused_moe.py:881-884)
  fused_experts_impl(...)   fused_moe.py:1935-1965 / the dispatcher 2214-2240
  fused_experts(..., quant_config)
The whole layer is one C-ABI call (vmamd_fused_moe_*) that enqueues all of its
kernels on the current stream; Python only validates and allocates.
"""
from __future__ import annotations

import math

import torch

from . import _custom_ops as ops
from . import _lib, dispatch_policy
from ._lib import call, ptr, stream_of


def _round_up(x: int, m: int) -> int:
    return (x + m - 1) // m * m


def moe_align_block_size(topk_ids: torch.Tensor, block_size: int, num_experts: int,
                         expert_map: torch.Tensor | None = None, pad_sorted_ids: bool = False,
                         return_offsets: bool = False):
    """Group the routes of ``topk_ids`` [T, K] by expert, padded per expert to
    ``block_size``.  Returns (sorted_token_ids, expert_ids, num_tokens_post_pad)
    (and the per-expert segment offsets when ``return_offsets``)."""
    ids = topk_ids if topk_ids.dtype == torch.int32 else topk_ids.to(torch.int32)
    ids = ids.contiguous()
    numel = ids.numel()
    cap = numel + num_experts * (block_size - 1)
    if pad_sorted_ids:
        cap = _round_up(cap, block_size)
    dev = ids.device
    sorted_ids = torch.empty(cap, dtype=torch.int32, device=dev)
    expert_ids = torch.empty((cap + block_size - 1) // block_size, dtype=torch.int32, device=dev)
    ntpp = torch.empty(1, dtype=torch.int32, device=dev)
    offsets = torch.empty(num_experts + 1, dtype=torch.int32, device=dev) if return_offsets else None
    ops.moe_align_block_size(ids, num_experts, block_size, sorted_ids, expert_ids, ntpp, expert_map,
                             None, offsets)
    if return_offsets:
        return sorted_ids, expert_ids, ntpp, offsets
    return sorted_ids, expert_ids, ntpp


# ---------------------------------------------------------------- experts --
# Kernel paths of the fused layer (VMAMD_MOE_PATH_*): "gemv" / "gemm" force
# the W8A8 decode kernels / grouped GEMMs, "auto" lets the library pick by
# routes per expert, "native_gemv" computes the reference's native GEMV-MoE
# numerics (bf16 activations, gate and up in fp32 through the SwiGLU).
PATHS = {"auto": 0, "gemv": 1, "gemm": 2, "native_gemv": 3}
# Tokens per launch sequence: longer batches run in chunks of this many
# tokens with one chunk's workspace (fused_moe.py:2126-2128).
CHUNK_SIZE = 16384


def _per_expert_scale(scale: torch.Tensor, e: int) -> torch.Tensor | None:
    """The [E] per-expert view of a per-tensor / per-expert scale layout (0-d,
    one element, [E] or [E, 1]), or None for any other layout."""
    if scale.dim() == 0 or (scale.dim() == 1 and scale.numel() == 1):
        return scale.reshape(1).expand(e)
    if scale.dim() == 1 and scale.numel() == e:
        return scale
    if scale.dim() == 2 and tuple(scale.shape) == (e, 1):
        return scale[:, 0]
    return None


def fp8_moe_scale_layout_is_supported(scale: torch.Tensor | None, weight: torch.Tensor) -> bool:
    """True when this path takes ``scale`` for the fp8 expert stack ``weight``
    [E, N, K]: f32 and contiguous, K a multiple of 128, and either one of the
    per-tensor layouts (0-d, [1], [E], [E, 1]) or the 128x128 block grid
    [E, ceil(N/128), K/128].  Mirrors the reference's guard
    _musa_fp8_moe_scale_layout_is_supported (fused_moe.py:1262-1302) for the
    128-wide grid; its 64-wide grid (a 128x128 block holding four different
    scales) has no 128x128 view and is declined."""
    if scale is None or scale.dtype != torch.float32 or not scale.is_contiguous():
        return False
    e, n, k = weight.shape
    if k % 128 != 0:
        return False
    if _per_expert_scale(scale, e) is not None:
        return True
    return tuple(scale.shape) == (e, (n + 127) // 128, k // 128)


def _expand_fp8_scale(scale: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """Per-tensor / per-expert fp8 scales -> the [E, ceil(N/128), K/128] block
    view; a scale already on that grid passes through (reference:
    _maybe_expand_fp8_moe_per_tensor_scale, fused_moe.py:1212-1259, applied by
    fused_experts_impl at 2006-2008 whatever block_shape says)."""
    e, n, k = w.shape
    if k % 128 != 0:
        raise ValueError(f"fp8 MoE weights need an input size divisible by 128, got {k}")
    want = (e, (n + 127) // 128, k // 128)
    s = scale.to(torch.float32)
    if tuple(s.shape) == want:
        return s.contiguous()
    per_expert = _per_expert_scale(s, e)
    if per_expert is not None:
        return per_expert.reshape(e, 1, 1).expand(want).contiguous()
    raise ValueError(f"fp8 MoE scale of shape {tuple(scale.shape)} is neither per-tensor, "
                     f"per-expert nor the 128x128 block grid {want} (64-wide block scales "
                     "are not on this path)")


def fused_experts_impl(hidden_states: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor,
                       topk_weights: torch.Tensor, topk_ids: torch.Tensor,
                       activation: str = "silu", apply_router_weight_on_input: bool = False,
                       use_fp8_w8a8: bool = False, use_int8_w8a8: bool = False,
                       use_int8_w8a16: bool = False, use_int4_w4a16: bool = False,
                       ocp_mx_scheme: str | None = None, per_channel_quant: bool = False,
                       global_num_experts: int = -1, expert_map: torch.Tensor | None = None,
                       w1_scale: torch.Tensor | None = None, w2_scale: torch.Tensor | None = None,
                       w1_zp: torch.Tensor | None = None, w2_zp: torch.Tensor | None = None,
                       a1_scale: torch.Tensor | None = None, a2_scale: torch.Tensor | None = None,
                       block_shape: list[int] | None = None, w1_bias: torch.Tensor | None = None,
                       w2_bias: torch.Tensor | None = None,
                       gemm1_clamp_limit: float | None = None, *, inplace: bool = False,
                       path: str = "auto", chunk_size: int = CHUNK_SIZE) -> torch.Tensor:
    """Drop-in for the reference's fused_experts_impl
    (vllm_musa/model_executor/layers/fused_moe/fused_moe.py:1935-1965, 2214-2240):
    out[t] = sum_k w[t,k] * W2[e] . act(W13[e] . x[t]) with the reference's
    rounding points.  Supported: bf16 weights, and fp8 weights (use_fp8_w8a8)
    with 128x128 block scales (block_shape=[128, 128]) or per-tensor /
    per-expert scales (any block_shape; expanded to the 128x128 grid as the
    reference's fused_experts_impl does, fused_moe.py:2006-2008), with dynamic
    1x128 activation quantisation.  apply_router_weight_on_input multiplies
    the W13 output by the routed weight before the activation and leaves the
    W2 output unweighted (the reference's mul_routed_weight on its first GEMV,
    fused_moe.py:2148-2177).  ``path`` forces the W8A8 decode ("gemv") or
    prefill ("gemm") kernels, or the reference's native GEMV-MoE numerics
    ("native_gemv": x not quantised, gate and up in fp32 through the SwiGLU,
    one rounding; gemv.mu:249-514); "auto" computes what the reference computes
    for this call -- its native GEMV where its dispatcher would run it (its
    calibrated shapes, the VLLM_MUSA_FUSED_MOE_DISPATCH=gemv override),
    W8A8 elsewhere -- on the kernels MI355X's dispatch table picks.  Batches
    longer than ``chunk_size`` tokens run in chunks of that many tokens with
    one chunk's workspace, as the reference's driver loop does
    (fused_moe.py:2126-2128)."""
    if activation != "silu":
        raise NotImplementedError(f"activation {activation!r}: only silu (SwiGLU) is on this path")
    if use_int8_w8a8 or use_int8_w8a16 or use_int4_w4a16 or ocp_mx_scheme or per_channel_quant:
        raise NotImplementedError("int8 / int4-w4a16 / MX / per-channel MoE are not on this path")
    if w1_bias is not None or w2_bias is not None or w1_zp is not None or w2_zp is not None:
        raise NotImplementedError("expert biases / zero points are not on this path")
    if a1_scale is not None or a2_scale is not None:
        raise NotImplementedError("static activation scales: only dynamic 1x128 quantisation")
    if hidden_states.dim() != 2 or hidden_states.dtype != torch.bfloat16:
        raise ValueError("hidden_states must be bf16 [T, H]")
    if hidden_states.shape[1] != w1.shape[2]:
        raise ValueError(f"Hidden size mismatch {hidden_states.shape[1]} != {w1.shape[2]}")
    if topk_weights.shape != topk_ids.shape:
        raise ValueError("topk shape mismatch")
    if not hidden_states.is_contiguous():
        raise ValueError("Hidden_states must be contiguous")
    t, h = hidden_states.shape
    e, n2, _ = w1.shape
    i = n2 // 2
    if w2.shape != (e, h, i):
        raise ValueError(f"w2 must be [E, H, I] = {(e, h, i)}, got {tuple(w2.shape)}")
    topk = topk_ids.shape[1]
    out = hidden_states if (inplace and t > 0) else torch.empty_like(hidden_states)
    if t == 0:
        return out
    ids = topk_ids.to(torch.int32).contiguous()
    wts = topk_weights.to(torch.float32).contiguous()
    emap = None if expert_map is None else expert_map.to(torch.int32).contiguous()
    limit = 0.0 if gemm1_clamp_limit is None else float(gemm1_clamp_limit)
    on_input = int(bool(apply_router_weight_on_input))
    if use_fp8_w8a8:
        if block_shape is not None and list(block_shape) != [128, 128]:
            raise NotImplementedError("fp8 MoE on this path takes block_shape [128, 128] "
                                      "or per-tensor / per-expert scales")
        if w1_scale is None or w2_scale is None:
            raise ValueError("fp8 MoE needs w1_scale and w2_scale")
        w1_scale = _expand_fp8_scale(w1_scale, w1)
        w2_scale = _expand_fp8_scale(w2_scale, w2)
        block_shape = [128, 128]
    if path == "auto":
        path = dispatch_policy.resolve_path(
            hidden_states, w1, w2, w1_scale if use_fp8_w8a8 else None,
            w2_scale if use_fp8_w8a8 else None, topk, block_shape, expert_map,
            topk_weights=topk_weights, topk_ids=topk_ids, use_fp8_w8a8=use_fp8_w8a8,
            apply_router_weight_on_input=apply_router_weight_on_input,
            global_num_experts=global_num_experts)
    code = PATHS[path]
    if chunk_size <= 0:
        raise ValueError("chunk_size must be positive")
    if use_fp8_w8a8:
        if w1.dtype != torch.float8_e4m3fn or w2.dtype != torch.float8_e4m3fn:
            raise ValueError("fp8 MoE weights must be float8_e4m3fn")
        s1, s2 = w1_scale, w2_scale
        w1c, w2c = w1.contiguous(), w2.contiguous()
        _lib.check_cuda(hidden_states, w1c, w2c, s1, s2, wts, ids, emap)
        size = _lib.load().vmamd_fused_moe_fp8_workspace_size

        def launch(x, ci, cw, o, ws, nbytes):
            call("vmamd_fused_moe_fp8", ptr(x), _lib.DTYPE_BF16, x.shape[0], h, ptr(w1c), ptr(s1),
                 ptr(w2c), ptr(s2), e, i, ptr(cw), ptr(ci), topk, ptr(emap),
                 0 if emap is None else emap.numel(), limit, on_input, code, ptr(o), ptr(ws),
                 nbytes, stream_of(x))
    elif w1.dtype == torch.bfloat16 and w2.dtype == torch.bfloat16:
        if w1_scale is not None or w2_scale is not None:
            raise ValueError("bf16 MoE weights take no scales")
        w1c, w2c = w1.contiguous(), w2.contiguous()
        _lib.check_cuda(hidden_states, w1c, w2c, wts, ids, emap)
        size = _lib.load().vmamd_fused_moe_bf16_workspace_size

        def launch(x, ci, cw, o, ws, nbytes):
            call("vmamd_fused_moe_bf16", ptr(x), x.shape[0], h, ptr(w1c), ptr(w2c), e, i, ptr(cw),
                 ptr(ci), topk, ptr(emap), 0 if emap is None else emap.numel(), limit, on_input,
                 code, ptr(o), ptr(ws), nbytes, stream_of(x))
    else:
        raise NotImplementedError(f"MoE weights of dtype {w1.dtype} are not on this path")
    _run_chunked(hidden_states, ids, wts, out, chunk_size,
                 lambda tc: size(tc, topk, e, h, i, code), launch)
    return out


def _run_chunked(x, ids, wts, out, chunk, size, launch):
    """The layer over token chunks of at most ``chunk`` rows, in order, with
    one workspace sized for the largest chunk (the full-size ones and the
    remainder may take different kernels, so both are sized)."""
    t = x.shape[0]
    first = min(t, chunk)
    nbytes = max(size(first), size(t % chunk) if t > chunk and t % chunk else 0)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=x.device)
    for c0 in range(0, t, chunk):
        c1 = min(t, c0 + chunk)
        launch(x[c0:c1], ids[c0:c1], wts[c0:c1], out[c0:c1], ws, nbytes)


def _bf16_big_block(routes: int, experts: int) -> int:
    """The large route block of the bf16 grouped GEMMs: 320 where it needs
    fewer blocks for the expected largest expert (mean + 3 sqrt(mean)
    routes) than 256, each 320-route block counted 1.25x, else 256 -- the
    rule of bf16_big_block (csrc/moe_gemm.hip)."""
    mean = routes / experts
    top = mean + 3.0 * math.sqrt(mean)
    return 320 if 1.25 * math.ceil(top / 320) < math.ceil(top / 256) else 256


class MoeStages:
    """One MoE layer as its separate launches, in the order the fused call
    enqueues them: ``quant`` (1x128 of x; fp8 only), ``align``
    (moe_align_block_size), ``w13_stage`` (grouped W13 GEMM + SiLU-and-mul,
    + a2 quantisation for fp8), ``w2_stage`` (grouped W2 GEMM with the routed
    weight) and ``combine`` (top-k sum).  This is the upstream
    fused_experts_impl decomposition (quantize input ->
    invoke_fused_moe_kernel(W13) -> activation + a2 quant ->
    invoke_fused_moe_kernel(W2) -> moe_sum; patches/series/0144-…:22-78).
    Each method launches exactly its kernels on the current stream, so one
    stage can be timed or profiled on its own.  Buffers are allocated here.

    fp8 weights (float8_e4m3fn) need w13_scale / w2_scale (128x128 blocks);
    bf16 weights take none."""

    def __init__(self, hidden_states, w13, w13_scale, w2, w2_scale, topk_weights, topk_ids,
                 path: str = "auto", expert_map=None, swiglu_limit: float | None = None,
                 block_m: int | None = None):
        self.fp8 = w13.dtype == torch.float8_e4m3fn
        self.x = hidden_states
        t, self.h = hidden_states.shape
        self.e, n2, _ = w13.shape
        self.i = n2 // 2
        self.topk = topk_ids.shape[1]
        self.t = t
        numel = t * self.topk
        # `auto`: the rule of moe_block_m (csrc/moe_gemm.hip) -- decode kernels up to
        # 2.5 routes per expert for fp8, 12 for bf16 (measured crossovers).
        limit = (5 * self.e) // 2 if self.fp8 else 12 * self.e
        gemv = path == "gemv" or (path == "auto" and numel <= limit)
        # grouped GEMMs: large route blocks from 128 routes per expert (256, or
        # 320 for bf16 where that needs fewer blocks: bf16_big_block in
        # csrc/moe_gemm.hip)
        big = 256 if self.fp8 else _bf16_big_block(numel, self.e)
        self.block_m = 16 if gemv else big if numel >= 128 * self.e else 128
        if block_m is not None:  # the grouped GEMMs' route tile
            allowed = (128, 256) if self.fp8 else (128, 256, 320)
            if gemv or block_m not in allowed:
                raise ValueError(f"block_m {block_m} needs the grouped GEMMs {allowed}")
            self.block_m = block_m
        self.w13, self.w2 = w13.contiguous(), w2.contiguous()
        if self.fp8:
            self.s13 = _expand_fp8_scale(w13_scale, w13)
            self.s2 = _expand_fp8_scale(w2_scale, w2)
        self.ids = topk_ids.to(torch.int32).contiguous()
        self.wts = topk_weights.to(torch.float32).contiguous()
        self.emap = None if expert_map is None else expert_map.to(torch.int32).contiguous()
        self.limit = 0.0 if swiglu_limit is None else float(swiglu_limit)
        dev = hidden_states.device
        self.cap = numel + self.e * (self.block_m - 1)
        i32 = dict(dtype=torch.int32, device=dev)
        if self.fp8:
            self.xq = torch.empty(t, self.h, dtype=torch.float8_e4m3fn, device=dev)
            self.xs = torch.empty(t, self.h // 128, dtype=torch.float32, device=dev)
        self.sorted = torch.empty(self.cap, **i32)
        self.eids = torch.empty(-(-self.cap // self.block_m), **i32)
        self.ntpp = torch.empty(1, **i32)
        self.offsets = torch.empty(self.e + 1, **i32)
        self.active = torch.empty(self.e, **i32)
        self.nact = torch.empty(1, **i32)
        rows = numel if gemv else self.cap
        adt = torch.float8_e4m3fn if self.fp8 else torch.bfloat16
        self.a2 = torch.empty(rows, self.i, dtype=adt, device=dev)
        if self.fp8:
            self.a2s = torch.empty(rows, self.i // 128, dtype=torch.float32, device=dev)
        self.y = torch.empty(t, self.topk, self.h, dtype=torch.bfloat16, device=dev)
        self.out = torch.empty(t, self.h, dtype=torch.bfloat16, device=dev)
        q = "vmamd_moe_fp8_stage_workspace_size" if self.fp8 else \
            "vmamd_moe_bf16_stage_workspace_size"
        nbytes = getattr(_lib.load(), q)(t, self.topk, self.e, self.h, self.i, self.block_m)
        self.ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=dev)
        self.ws_bytes = nbytes

    def quant(self):
        if self.fp8:
            ops.per_token_group_quant_8bit_vec(self.x, self.xq, self.xs, 128, 1e-10, ops.FP8_MIN,
                                               ops.FP8_MAX)

    def align(self):
        ops.moe_align_block_size(self.ids, self.e, self.block_m, self.sorted, self.eids,
                                 self.ntpp, self.emap, None, self.offsets, self.active, self.nact)

    def _route_args(self):
        return (ptr(self.sorted), self.cap, self.block_m, ptr(self.offsets), ptr(self.ntpp),
                ptr(self.active), ptr(self.nact))

    def w13_stage(self):
        if self.fp8:
            call("vmamd_moe_fp8_w13", ptr(self.xq), ptr(self.xs), self.t, self.h, self.topk,
                 *self._route_args(), ptr(self.w13), ptr(self.s13), self.e, self.i, self.limit,
                 ptr(self.a2), ptr(self.a2s), ptr(self.ws), self.ws_bytes, stream_of(self.x))
        else:
            call("vmamd_moe_bf16_w13", ptr(self.x), self.t, self.h, self.topk,
                 *self._route_args(), ptr(self.w13), self.e, self.i, self.limit, ptr(self.a2),
                 ptr(self.ws), self.ws_bytes, stream_of(self.x))

    def w2_stage(self):
        tail = (ptr(self.wts), ptr(self.ids), ptr(self.emap),
                0 if self.emap is None else self.emap.numel(), ptr(self.y), ptr(self.ws),
                self.ws_bytes, stream_of(self.x))
        if self.fp8:
            call("vmamd_moe_fp8_w2", ptr(self.a2), ptr(self.a2s), self.t, self.topk,
                 *self._route_args(), ptr(self.w2), ptr(self.s2), self.e, self.h, self.i, *tail)
        else:
            call("vmamd_moe_bf16_w2", ptr(self.a2), self.t, self.topk, *self._route_args(),
                 ptr(self.w2), self.e, self.h, self.i, *tail)

    def combine(self):
        ops.moe_sum(self.y, self.out, self.ids, self.emap)

    def run(self) -> torch.Tensor:
        self.quant()
        self.align()
        self.w13_stage()
        self.w2_stage()
        self.combine()
        return self.out


Fp8MoeStages = MoeStages


def fused_experts(hidden_states: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor,
                  topk_weights: torch.Tensor, topk_ids: torch.Tensor, inplace: bool = False,
                  activation: str = "silu", apply_router_weight_on_input: bool = False,
                  global_num_experts: int = -1, expert_map: torch.Tensor | None = None,
                  quant_config=None) -> torch.Tensor:
    """Upstream fused_experts(..., quant_config) entry (called from the quant
    methods, quantization/fp8.py:261-272 and unquantized_fused_moe_method.py:119-130)."""
    qc = quant_config
    return fused_experts_impl(
        hidden_states, w1, w2, topk_weights, topk_ids, activation=activation,
        apply_router_weight_on_input=apply_router_weight_on_input,
        use_fp8_w8a8=bool(getattr(qc, "use_fp8_w8a8", False)),
        global_num_experts=global_num_experts, expert_map=expert_map,
        w1_scale=getattr(qc, "w1_scale", None), w2_scale=getattr(qc, "w2_scale", None),
        block_shape=getattr(qc, "block_shape", None),
        gemm1_clamp_limit=getattr(qc, "gemm1_clamp_limit", None), inplace=inplace)
