"""The MoE quant-method ``apply`` hooks with the reference's signatures.

Each reads the expert weights from the layer object the way the reference
method does and runs this package's fused layer:

  Fp8MoEMethod.apply               vllm_musa/model_executor/layers/quantization/fp8.py:212-291
                                   (block fp8: w13_weight / w2_weight with
                                   w13_weight_scale_inv / w2_weight_scale_inv)
  UnquantizedFusedMoEMethod.forward_oot
                                   model_executor/layers/fused_moe/unquantized_fused_moe_method.py:81-130
  W4AFp8MoEMethod.apply            model_executor/layers/quantization/w4afp8.py:147-170

Shared experts that the caller delegates (shared_experts with an input) are
added to the routed output, as the reference does when the runner hands them
to the quant method.  Expert-parallel all-to-all managers are not part of this
single-GPU path; layer.expert_map selects the local experts.
"""
from __future__ import annotations

import torch

from .fused_moe import fused_experts_impl
from .w4afp8_moe import w4afp8_moe


def _add_shared(routed, shared_experts, shared_experts_input, x):
    if shared_experts is None:
        return routed
    inp = shared_experts_input if shared_experts_input is not None else x
    return routed + shared_experts(inp)


def _activation(layer) -> str:
    act = getattr(layer, "activation", "silu")
    return getattr(act, "value", act) if not isinstance(act, str) else act


class Fp8MoEMethod:
    """Block-fp8 (128x128 weight blocks, dynamic 1x128 activations) experts."""

    def __init__(self, block_shape=(128, 128), swiglu_limit: float | None = None):
        self.block_shape = list(block_shape)
        self.swiglu_limit = swiglu_limit

    def apply(self, layer, x: torch.Tensor, topk_weights: torch.Tensor, topk_ids: torch.Tensor,
              shared_experts=None, shared_experts_input: torch.Tensor | None = None):
        routed = fused_experts_impl(
            x, layer.w13_weight, layer.w2_weight, topk_weights, topk_ids,
            activation=_activation(layer),
            apply_router_weight_on_input=getattr(layer, "apply_router_weight_on_input", False),
            use_fp8_w8a8=True, expert_map=getattr(layer, "expert_map", None),
            w1_scale=layer.w13_weight_scale_inv, w2_scale=layer.w2_weight_scale_inv,
            block_shape=self.block_shape, gemm1_clamp_limit=self.swiglu_limit)
        return _add_shared(routed, shared_experts, shared_experts_input, x)


class UnquantizedFusedMoEMethod:
    """bf16 experts."""

    def __init__(self, swiglu_limit: float | None = None):
        self.swiglu_limit = swiglu_limit

    def forward_oot(self, layer, x: torch.Tensor, topk_weights: torch.Tensor,
                    topk_ids: torch.Tensor, shared_experts=None,
                    shared_experts_input: torch.Tensor | None = None):
        routed = fused_experts_impl(
            x, layer.w13_weight, layer.w2_weight, topk_weights, topk_ids,
            activation=_activation(layer),
            apply_router_weight_on_input=getattr(layer, "apply_router_weight_on_input", False),
            expert_map=getattr(layer, "expert_map", None), gemm1_clamp_limit=self.swiglu_limit)
        return _add_shared(routed, shared_experts, shared_experts_input, x)

    apply = forward_oot


class W4AFp8MoEMethod:
    """Packed int4 experts with bf16 group-128 scales and dynamic per-row fp8
    activations."""

    def __init__(self, swiglu_limit: float | None = None):
        self.swiglu_limit = swiglu_limit

    def apply(self, layer, x: torch.Tensor, topk_weights: torch.Tensor, topk_ids: torch.Tensor,
              shared_experts=None, shared_experts_input: torch.Tensor | None = None):
        if getattr(layer, "apply_router_weight_on_input", False):
            raise NotImplementedError("W4AFP8 router weights must apply to the output")
        routed = w4afp8_moe(x, layer.w13_weight, layer.w2_weight, layer.w13_weight_scale_inv,
                            layer.w2_weight_scale_inv, topk_weights, topk_ids,
                            getattr(layer, "expert_map", None), swiglu_limit=self.swiglu_limit)
        return _add_shared(routed, shared_experts, shared_experts_input, x)
