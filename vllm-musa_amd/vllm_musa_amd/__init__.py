"""vllm_musa_amd: the quantized fused-MoE / block-fp8 matmul hot path of
vllm-musa, rebuilt for AMD Instinct MI355X (gfx950).

Python on PyTorch-ROCm hosts the reference's call signatures; all arithmetic
runs in hand-written HIP kernels of libvllm_musa_amd.so (C ABI declared in
include/vllm_musa_amd.h).  Importing the package does not require a GPU; the
first kernel call loads the library and raises if it has not been built.
"""
from __future__ import annotations

from . import _custom_ops  # noqa: F401
from ._lib import LIB_PATH, VmamdError, load  # noqa: F401
from .fp8_utils import per_token_group_quant_fp8, silu_mul_per_token_group_quant_fp8  # noqa: F401
from .router import fused_topk, grouped_topk, topk_sigmoid, topk_softmax  # noqa: F401
from .w4afp8_moe import w4afp8_moe  # noqa: F401

__all__ = [
    "LIB_PATH", "VmamdError", "load",
    "per_token_group_quant_fp8", "silu_mul_per_token_group_quant_fp8",
    "fused_topk", "grouped_topk", "topk_sigmoid", "topk_softmax", "w4afp8_moe",
]
