"""Fused-MoE host driver (reference: vllm_musa/model_executor/layers/fused_moe/fused_moe.py).

This module keeps the reference's Python entry points:
  moe_align_block_size(topk_ids, block_size, num_experts, expert_map=None, pad_sorted_ids=False)
      upstream wrapper of the _moe_C op (sizing as fused_moe.py:881-884)
"""
from __future__ import annotations

import torch

from . import _custom_ops as ops


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
