"""Parallel fp32 router-gate GEMM behind the reference's guard contract.

Reference: vllm_musa/model_executor/layers/fused_moe/router/musa_router_gemm.py
(router_gate_enabled 112-114, activation_count 117-128, the custom op 229-247,
router_gate_fp32 250-266).  The gate of the model the reference tuned for
(Nemotron-H, hidden 2688, 128 routed experts, fp32 weight) is computed by
vmamd_router_gate_fp32; every other gate shape, dtype, layout or device is
declined with ``None`` so the caller keeps its own path, and
``VLLM_MUSA_ROUTER_GATE_FP32=0`` turns the tier off.

The logits are bitwise reproducible: each one is summed in a fixed fp32 order
(one fused-multiply-add chain per lane over a fixed slice of K, then a fixed
64-way butterfly) that does not depend on the batch size, so a token's top-k
cannot change with the batch it is served in.

The platform decision is taken once at import and the per-call checks read
only tensor metadata that FakeTensors carry too (dtype, shape, contiguity);
"meta" is an accepted device, served by the op's fake implementation, so a
traced graph keeps the kernel (musa_router_gemm.py:44-57, 99-107).
"""
from __future__ import annotations

import os

import torch

from . import _custom_ops as ops

__all__ = ["router_gate_enabled", "router_gate_fp32", "activation_count"]

_HIDDEN, _EXPERTS = 2688, 128
SUPPORTED_WEIGHT_SHAPE = (_EXPERTS, _HIDDEN)

_ON_ROCM = torch.version.hip is not None
_ACCEPTED_DEVICES = ("cuda", "meta")
_ACTIVATIONS = 0


def router_gate_enabled() -> bool:
    """Kill switch, read per call (VLLM_MUSA_ROUTER_GATE_FP32=0 disables)."""
    return os.environ.get("VLLM_MUSA_ROUTER_GATE_FP32", "1") != "0"


def activation_count() -> int:
    """Router gates this process has served with the kernel (a graph replayed
    from a cache compiled with the tier off leaves it at 0)."""
    return _ACTIVATIONS


@torch.library.custom_op("vllm_musa_amd::router_gate_fp32", mutates_args=())
def _router_gate_op(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    global _ACTIVATIONS
    _ACTIVATIONS += 1
    out = torch.empty((x.shape[0], weight.shape[0]), dtype=torch.float32, device=x.device)
    ops.router_gate_fp32(x, weight, out)
    return out


@_router_gate_op.register_fake
def _router_gate_fake(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    return torch.empty((x.shape[0], weight.shape[0]), dtype=torch.float32, device=x.device)


def router_gate_fp32(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor | None:
    """fp32 logits [M, 128] of the [M, 2688] activations (bf16 or f32) against
    the [128, 2688] fp32 gate weight, or None when this tier does not apply
    (never an error).  An empty batch returns an empty [0, 128] tensor."""
    if not _ON_ROCM or not router_gate_enabled():
        return None
    if weight.dtype != torch.float32 or tuple(weight.shape) != SUPPORTED_WEIGHT_SHAPE:
        return None
    if x.dim() != 2 or x.shape[-1] != _HIDDEN:
        return None
    if x.dtype not in (torch.float32, torch.bfloat16):
        return None
    if x.device.type not in _ACCEPTED_DEVICES or weight.device.type != x.device.type:
        return None
    if not x.is_contiguous() or not weight.is_contiguous():
        return None
    return torch.ops.vllm_musa_amd.router_gate_fp32(x, weight)
