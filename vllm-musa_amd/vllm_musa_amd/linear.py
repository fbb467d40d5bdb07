"""Row-parallel linear hooks with the reference's interface.

  forward_swiglu_clamp(layer, gate_up, swiglu_limit)
      MusaRowParallelLinear.forward_swiglu_clamp
      (vllm_musa/model_executor/layers/linear.py:33-96): the clamp-aware SwiGLU
      and the layer's block-fp8 projection as one path, or None when the layer
      is not in the configuration that path covers (the model then runs its
      ordinary activation and linear path).

The layer is duck-typed on the attributes the reference reads: quant_method
(block_quant, fp8_linear), input_is_parallel, bias, input_size_per_partition,
output_size_per_partition, weight, weight_scale_inv (or weight_scale),
weight_block_size, reduce_results and tp_size.  The reference's second branch,
the fine-block GEMV kernel of DeepSeek-V4 (its own block layout), has no
counterpart here and is never taken.
"""
from __future__ import annotations

import os

import torch

from .block_fp8 import Fp8BlockScaledMMKernel, silu_clamp_block_fp8_matmul


def _batch_invariant() -> bool:
    return os.environ.get("VLLM_BATCH_INVARIANT", "0") not in ("", "0", "false", "False")


def _block_fp8(quant_method) -> bool:
    """Block-quantised fp8 linear whose kernel is the block-scaled MM kernel
    (reference: _deepgemm_block_fp8, linear.py:9-18)."""
    return (quant_method is not None and bool(getattr(quant_method, "block_quant", False))
            and isinstance(getattr(quant_method, "fp8_linear", None), Fp8BlockScaledMMKernel))


def forward_swiglu_clamp(layer, gate_up: torch.Tensor, swiglu_limit: float) -> torch.Tensor | None:
    """Clamp-aware SwiGLU + block-fp8 down projection for a row-parallel layer,
    with the reference's gates (linear.py:58-74): not batch-invariant, parallel
    input, no bias, gate_up [..., 2 * input_size_per_partition] contiguous bf16,
    128x128 weight blocks, swiglu_limit == 10.  With tensor parallelism the
    partial outputs are summed over the default process group."""
    fast = (not _batch_invariant()
            and getattr(layer, "input_is_parallel", False)
            and _block_fp8(getattr(layer, "quant_method", None))
            and getattr(layer, "bias", None) is None
            and gate_up.dim() >= 2
            and gate_up.shape[-1] == 2 * layer.input_size_per_partition
            and gate_up.dtype == torch.bfloat16
            and gate_up.is_contiguous()
            and tuple(getattr(layer, "weight_block_size", None) or ()) == (128, 128)
            and swiglu_limit == 10.0)
    if not fast:
        return None
    weight_scale = getattr(layer, "weight_scale_inv", None)
    if weight_scale is None:
        weight_scale = getattr(layer, "weight_scale", None)
    if weight_scale is None:
        return None
    gate_up_2d = gate_up.view(-1, gate_up.shape[-1])
    out = silu_clamp_block_fp8_matmul(gate_up_2d, layer.weight, weight_scale, 128, False,
                                      swiglu_limit).view(*gate_up.shape[:-1],
                                                         layer.output_size_per_partition)
    if getattr(layer, "reduce_results", True) and getattr(layer, "tp_size", 1) > 1:
        torch.distributed.all_reduce(out)
    return out
