"""Dense w8a8 block-fp8 linear with the reference's interfaces.

  w8a8_block_fp8_matmul(A, B, As, Bs, block_size, output_dtype)
      upstream w8a8_triton_block_scaled_mm as called at
      vllm_musa/deepseek_v4_jit/fp8_einsum.py:399-406
  apply_w8a8_block_fp8_linear(input, weight, weight_scale, block_size)
      quantise bf16 activations per 1x128 group, then the block GEMM
      (_musa_deepgemm_fp8_op, model_executor/kernels/linear/scaled_mm/deep_gemm.py:233-262)
  Fp8BlockScaledMMKernel.apply_block_scaled_mm(A, B, As, Bs, **kwargs)
      MUSADeepGemmFp8BlockScaledMMKernel.apply_block_scaled_mm (deep_gemm.py:177-197)
  silu_clamp_block_fp8_matmul(input, weight, weight_scale, group_size, use_deep_gemm_e8m0,
                              swiglu_limit)
      clamp-aware SwiGLU + 1x128 fp8 quantisation + block-fp8 down projection
      (_musa_silu_clamp_deepgemm_fp8_op, deep_gemm.py:336-409)
"""
from __future__ import annotations

import torch

from . import _lib
from ._lib import call, check_cuda, ptr, stream_of
from .fp8_utils import (FP8_DTYPE, deepgemm_post_process_fp8_weight_block,
                        per_token_group_quant_fp8)


def w8a8_block_fp8_matmul(A: torch.Tensor, B: torch.Tensor, As: torch.Tensor, Bs: torch.Tensor,
                          block_size: list[int], output_dtype: torch.dtype = torch.bfloat16,
                          out: torch.Tensor | None = None) -> torch.Tensor:
    """C = (A * As) @ (B * Bs)^T with 1x128 activation and 128x128 weight scales."""
    check_cuda(A, B, As, Bs, out)
    if output_dtype != torch.bfloat16:
        raise ValueError("only bfloat16 output is supported")
    if A.dtype != FP8_DTYPE or B.dtype != FP8_DTYPE:
        raise ValueError("A and B must be float8_e4m3fn")
    if list(block_size) != [128, 128]:
        raise ValueError(f"block_size must be [128, 128], got {block_size}")
    if B.dim() != 2 or not B.is_contiguous():
        raise ValueError("B must be a contiguous [N, K] matrix")
    n, k = B.shape
    if A.shape[-1] != k:
        raise ValueError(f"K mismatch: A has {A.shape[-1]}, B has {k}")
    lead = A.shape[:-1]
    a2 = A.reshape(-1, k).contiguous()
    m = a2.shape[0]
    as2 = As.reshape(-1, As.shape[-1])
    if as2.shape != (m, k // 128) or As.dtype != torch.float32:
        raise ValueError(f"As must be float32 [M, K/128] = {(m, k // 128)}, got {tuple(As.shape)}")
    if Bs.shape != ((n + 127) // 128, k // 128) or Bs.dtype != torch.float32:
        raise ValueError("Bs must be float32 [ceil(N/128), K/128]")
    Bs = Bs.contiguous()
    if out is None:
        out = torch.empty((m, n), dtype=torch.bfloat16, device=A.device)
    elif (tuple(out.shape) != (m, n) or out.dtype != torch.bfloat16 or not out.is_contiguous()
          or out.device != A.device):
        raise ValueError(f"out must be a contiguous bfloat16 [M, N] = {(m, n)} tensor on "
                         f"{A.device}, got {tuple(out.shape)} {out.dtype} on {out.device}")
    ws_bytes = _lib.load().vmamd_w8a8_block_fp8_matmul_workspace_size(m, n, k)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=A.device) if ws_bytes else None
    call("vmamd_w8a8_block_fp8_matmul", ptr(a2), ptr(as2), as2.stride(0), as2.stride(1), ptr(B),
         ptr(Bs), ptr(out), m, n, k, 128, 128, ptr(ws), ws_bytes, stream_of(A))
    return out.view(*lead, n)


def apply_w8a8_block_fp8_linear(input: torch.Tensor, weight: torch.Tensor,
                                weight_scale: torch.Tensor, block_size: list[int] = (128, 128),
                                bias: torch.Tensor | None = None) -> torch.Tensor:
    """bf16 input -> 1x128 fp8 quantisation -> block-fp8 GEMM (+ bias)."""
    q, s = per_token_group_quant_fp8(input.reshape(-1, input.shape[-1]), block_size[1])
    out = w8a8_block_fp8_matmul(q, weight, s, weight_scale, list(block_size))
    if bias is not None:
        out = out + bias
    return out.view(*input.shape[:-1], weight.shape[0])


class Fp8BlockScaledMMKernel:
    """Drop-in for the reference's block-scaled MM kernel object: its
    apply_block_scaled_mm receives the bf16 activations A, the fp8 weight B,
    (unused) As and the weight scales Bs, quantises A itself and returns bf16."""

    def __init__(self, weight_group_shape=(128, 128)):
        self.weight_group_shape = tuple(weight_group_shape)
        self.use_deep_gemm_e8m0 = False

    def process_weights_after_loading(self, layer) -> None:
        """Once after loading: block scales stored as e8m0 (weight_scale_inv, else
        weight_scale) are replaced by their float32 values, which the GEMM reads.
        Reference: MUSADeepGemmFp8BlockScaledMMKernel.process_weights_after_loading
        (model_executor/kernels/linear/scaled_mm/deep_gemm.py:112-146)."""
        name = ("weight_scale_inv" if getattr(layer, "weight_scale_inv", None) is not None
                else "weight_scale")
        block = tuple(getattr(layer, "weight_block_size", None) or self.weight_group_shape)
        old = getattr(layer, name)
        weight, scale = deepgemm_post_process_fp8_weight_block(
            layer.weight, old, block, self.use_deep_gemm_e8m0,
            getattr(layer, "is_bmm", False), getattr(layer, "bmm_batch_size", 0))
        if scale is not old:
            if isinstance(old, torch.nn.Parameter):
                scale = torch.nn.Parameter(scale, requires_grad=False)
            setattr(layer, name, scale)

    def apply_block_scaled_mm(self, A: torch.Tensor, B: torch.Tensor, As: torch.Tensor | None,
                              Bs: torch.Tensor, **kwargs) -> torch.Tensor:
        out = apply_w8a8_block_fp8_linear(A, B, Bs, list(self.weight_group_shape))
        dst = kwargs.get("output")
        if dst is not None:
            dst.copy_(out)
            return dst
        return out


def silu_clamp_block_fp8_matmul(input: torch.Tensor, weight: torch.Tensor,
                                weight_scale: torch.Tensor, group_size: int = 128,
                                use_deep_gemm_e8m0: bool = False,
                                swiglu_limit: float = 10.0) -> torch.Tensor:
    """down = block_fp8( quant1x128( silu(min(gate, L)) * clamp(up, -L, L) ) ) for
    input = [gate | up] of shape [M, 2D] (bf16 / f16) and weight [N, D] e4m3fn with
    128x128 block scales; returns [M, N] bf16.

    The activation is rounded to the input dtype before its group absmax, as the
    materialised activation of the ordinary path is (the quantiser is bit-exact
    to torch's clamp / sigmoid / multiply in bf16 followed by the 1x128
    quantiser).  Shapes the fused quantiser does not take run the reference's
    fallback: the activation in torch, then the quantiser and the block GEMM.
    Reference: _musa_silu_clamp_deepgemm_fp8_op (scaled_mm/deep_gemm.py:336-409)."""
    if use_deep_gemm_e8m0:
        raise NotImplementedError("power-of-two (ue8m0) activation scales are not supported")
    hidden = input.shape[-1] // 2 if input.dim() == 2 else 0
    supported = (group_size == 128 and input.dim() == 2
                 and input.shape[-1] % (2 * group_size) == 0 and hidden == weight.shape[-1]
                 and input.dtype in (torch.bfloat16, torch.float16) and input.is_contiguous()
                 and swiglu_limit > 0.0)
    if not supported:
        d = input.shape[-1] // 2
        gate = torch.clamp(input[..., :d], max=swiglu_limit)
        up = torch.clamp(input[..., d:], min=-swiglu_limit, max=swiglu_limit)
        activated = gate * torch.sigmoid(gate) * up
        return apply_w8a8_block_fp8_linear(activated, weight, weight_scale, [group_size, group_size])
    from . import _custom_ops as ops
    check_cuda(input, weight, weight_scale)
    m = input.shape[0]
    q = torch.empty((m, hidden), dtype=FP8_DTYPE, device=input.device)
    s = torch.empty((m, hidden // group_size), dtype=torch.float32, device=input.device)
    ops.silu_and_mul_clamp_per_token_group_fp8_quant(input, q, s, group_size, 1e-10, -448.0, 448.0,
                                                     swiglu_limit)
    return w8a8_block_fp8_matmul(q, weight, s, weight_scale, [128, 128])
