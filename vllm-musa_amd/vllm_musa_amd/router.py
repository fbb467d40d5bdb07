"""Router entry points with the reference's Python signatures.

  topk_softmax / topk_sigmoid   vllm_musa/jit_kernel/csrc/topk.py:211-275
  fused_topk                    upstream fused_topk as called from
                                model_executor/layers/fused_moe/router/grouped_topk_router.py:219-225
  grouped_topk                  grouped_topk_router.py:388-469 (and _grouped_topk_general 257-357)
  extend_topk_with_shared       vllm_musa/jit_kernel/extend_topk_shared.py:49-73
"""
from __future__ import annotations

import torch

from . import _custom_ops as ops

topk_softmax = ops.topk_softmax
topk_sigmoid = ops.topk_sigmoid


def extend_topk_with_shared(topk_weights: torch.Tensor, topk_ids: torch.Tensor,
                            shared_logits: torch.Tensor,
                            shared_expert_id: int) -> tuple[torch.Tensor, torch.Tensor]:
    """[T, K] routing -> new [T, K + 1] tensors with the folded shared expert's
    always-selected slot (weight sigmoid(shared logit), rounded to the logit
    dtype; routed weights unchanged)."""
    return ops.extend_topk_with_shared(topk_weights, topk_ids, shared_logits, shared_expert_id)


def fused_topk(hidden_states: torch.Tensor, gating_output: torch.Tensor, topk: int,
               renormalize: bool, indices_type: torch.dtype | None = None,
               correction_bias: torch.Tensor | None = None, scoring_func: str = "softmax"):
    """Returns (topk_weights f32, topk_ids, token_expert_indices) like upstream fused_topk."""
    if hidden_states.shape[0] != gating_output.shape[0]:
        raise ValueError("Number of tokens mismatch")
    t = gating_output.shape[0]
    dev = gating_output.device
    w = torch.empty(t, topk, dtype=torch.float32, device=dev)
    ids = torch.empty(t, topk, dtype=torch.int32, device=dev)
    token_expert_indices = torch.empty(t, topk, dtype=torch.int32, device=dev)
    g = gating_output.contiguous()
    if scoring_func == "softmax":
        ops.topk_softmax(w, ids, g, renormalize, correction_bias=correction_bias,
                         token_expert_indices=token_expert_indices)
    elif scoring_func == "sigmoid":
        ops.topk_sigmoid(w, ids, g, renormalize, correction_bias=correction_bias,
                         token_expert_indices=token_expert_indices)
    else:
        raise ValueError(f"Unsupported scoring function: {scoring_func}")
    if indices_type is not None and indices_type != torch.int32:
        ids = ids.to(indices_type)
    return w, ids, token_expert_indices


def grouped_topk(hidden_states: torch.Tensor, gating_output: torch.Tensor, topk: int,
                 renormalize: bool, num_expert_group: int = 0, topk_group: int = 0,
                 scoring_func: str = "softmax", routed_scaling_factor: float = 1.0,
                 e_score_correction_bias: torch.Tensor | None = None,
                 num_fused_shared_experts: int = 0) -> tuple[torch.Tensor, torch.Tensor]:
    """Grouped top-k on the GPU kernel; returns (weights f32 [T, topk], ids i32 [T, topk])."""
    if num_fused_shared_experts:
        raise NotImplementedError("fused shared experts are not part of this path")
    if hidden_states.shape[0] != gating_output.shape[0]:
        raise ValueError("Number of tokens mismatch")
    t = gating_output.shape[0]
    w = torch.empty(t, topk, dtype=torch.float32, device=gating_output.device)
    ids = torch.empty(t, topk, dtype=torch.int32, device=gating_output.device)
    ops.grouped_topk_into(w, ids, gating_output.contiguous(), num_expert_group, topk_group,
                          renormalize, scoring_func, routed_scaling_factor,
                          e_score_correction_bias)
    return w, ids
