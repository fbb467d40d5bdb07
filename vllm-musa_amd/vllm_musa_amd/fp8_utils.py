"""Activation quantisation and checkpoint scale handling with the
reference's Python signatures.

References (vllm_musa/model_executor/layers/quantization/utils/fp8_utils.py):
  per_token_group_quant_fp8                33-152
  _upcast_e8m0_to_fp32                     13-15
  deepgemm_post_process_fp8_weight_block   18-30
"""
from __future__ import annotations

import torch

from . import _custom_ops as ops

FP8_DTYPE = ops.FP8_DTYPE
E8M0_DTYPE = ops.E8M0_DTYPE


def upcast_e8m0_to_fp32(scale: torch.Tensor) -> torch.Tensor:
    """e8m0 exponent bytes -> float32 with the byte as the exponent field and a
    zero mantissa (0 -> +0.0, 255 -> +inf), on the GPU.  Reference:
    _upcast_e8m0_to_fp32 (fp8_utils.py:13-15)."""
    out = torch.empty(scale.shape, dtype=torch.float32, device=scale.device)
    ops.convert_scales(scale.contiguous(), out)
    return out


_upcast_e8m0_to_fp32 = upcast_e8m0_to_fp32


def deepgemm_post_process_fp8_weight_block(wq: torch.Tensor, ws: torch.Tensor,
                                           quant_block_shape: tuple[int, ...], use_e8m0: bool,
                                           is_bmm: bool = False, bmm_batch_size: int = 0
                                           ) -> tuple[torch.Tensor, torch.Tensor]:
    """Weights are kept as they are; e8m0 block scales become float32 unless the
    GEMM consumes e8m0 itself (use_e8m0).  Reference: fp8_utils.py:18-30."""
    del quant_block_shape, is_bmm, bmm_batch_size
    if E8M0_DTYPE is not None and ws.dtype == E8M0_DTYPE and not use_e8m0:
        return wq, upcast_e8m0_to_fp32(ws)
    return wq, ws


def per_token_group_quant_fp8(x: torch.Tensor, group_size: int, eps: float = 1e-10,
                              dtype: torch.dtype | None = None, column_major_scales: bool = False,
                              tma_aligned_scales: bool = False, out_q: torch.Tensor | None = None,
                              use_ue8m0: bool | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Quantise x [..., K] per 1 x group_size group to e4m3fn; returns (x_q, x_s)."""
    if use_ue8m0:
        raise NotImplementedError("UE8M0 scales are not part of this path")
    if tma_aligned_scales:
        raise NotImplementedError("TMA-aligned scales are a DeepGEMM layout; use row or column major")
    dtype = FP8_DTYPE if dtype is None else dtype
    if dtype != FP8_DTYPE:
        raise ValueError("only torch.float8_e4m3fn output is supported")
    if x.shape[-1] % group_size != 0:
        raise ValueError(f"the last dimension of `x` {x.shape[-1]} must be divisible by "
                         f"`group_size` {group_size}")
    if x.stride(-1) != 1:
        raise ValueError("`x` groups must be contiguous")
    x2 = x.reshape(-1, x.shape[-1])
    if not x2.is_contiguous() and x2.stride(0) < x2.shape[1]:
        x2 = x2.contiguous()
    x_q = out_q if out_q is not None else torch.empty(x.shape, device=x.device, dtype=dtype)
    if x_q.shape != x.shape:
        raise ValueError("out_q must have x's shape")
    m, k = x2.shape
    if column_major_scales:
        x_s = torch.empty((k // group_size, m), device=x.device, dtype=torch.float32).t()
    else:
        x_s = torch.empty((m, k // group_size), device=x.device, dtype=torch.float32)
    fp8_max = float(torch.finfo(dtype).max)
    ops.per_token_group_quant_8bit_vec(x2, x_q.view(m, k), x_s, group_size, eps, -fp8_max, fp8_max)
    x_s = x_s.reshape(*x.shape[:-1], k // group_size) if not column_major_scales else x_s
    return x_q, x_s


def silu_mul_per_token_group_quant_fp8(x: torch.Tensor, group_size: int = 128,
                                       swiglu_limit: float | None = None, eps: float = 1e-10):
    """Fused SiLU-and-mul + 1x128 quantisation of x [M, 2d] -> (q [M, d], s [M, d/128])."""
    m, d2 = x.shape
    d = d2 // 2
    q = torch.empty((m, d), dtype=FP8_DTYPE, device=x.device)
    s = torch.empty((m, d // group_size), dtype=torch.float32, device=x.device)
    fp8_max = float(torch.finfo(FP8_DTYPE).max)
    if swiglu_limit is None:
        ops.silu_and_mul_per_token_group_fp8_quant(x.contiguous(), q, s, group_size, eps,
                                                   -fp8_max, fp8_max)
    else:
        ops.silu_and_mul_clamp_per_token_group_fp8_quant(x.contiguous(), q, s, group_size, eps,
                                                         -fp8_max, fp8_max, swiglu_limit)
    return q, s
