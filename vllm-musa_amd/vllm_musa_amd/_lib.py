"""ctypes binding of libvllm_musa_amd.so (the gfx950 C ABI in include/vllm_musa_amd.h).

The library is built in-tree by ``make -C vllm-musa_amd/csrc``.  There is no
fallback: if the shared object is missing or a call fails, this module raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libvllm_musa_amd.so")

DTYPE_F32 = 0
DTYPE_F16 = 1
DTYPE_BF16 = 2
DTYPE_E4M3 = 4  # fp8 operands of the GEMV ops

_TORCH_DTYPE = {torch.float32: DTYPE_F32, torch.float16: DTYPE_F16, torch.bfloat16: DTYPE_BF16}

_p = ctypes.c_void_p
_i32 = ctypes.c_int
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_sz = ctypes.c_size_t

# Signatures of every exported entry point (name -> argtypes); restype is int
# (a VMAMD status code) unless listed in _RESTYPES.
SIGNATURES: dict[str, list] = {
    "vmamd_last_error": [],
    "vmamd_abi_version": [],
    "vmamd_per_token_group_quant_fp8": [_p, _i32, _i64, _i64, _i64, _i32, _f32, _f32, _f32, _p, _p,
                                        _i64, _i64, _p],
    "vmamd_silu_and_mul": [_p, _i32, _i64, _i64, _p, _p],
    "vmamd_silu_and_mul_quant_fp8": [_p, _i32, _i64, _i64, _i32, _f32, _f32, _f32, _f32, _p, _p,
                                     _p],
    "vmamd_extend_topk_with_shared": [_p, _p, _i64, _i32, _p, _i32, _i32, _p, _p, _p],
    "vmamd_convert_scales": [_p, _i32, _i64, _p, _i32, _p, _p],
    "vmamd_router_gate_fp32": [_p, _i32, _i64, _i64, _p, _i64, _p, _p],
    "vmamd_topk_softmax_shared": [_p, _i32, _i64, _i32, _i32, _i32, _f32, _p, _p, _i32, _i32, _p, _p,
                                  _p],
    "vmamd_topk_sigmoid_shared": [_p, _i32, _i64, _i32, _i32, _i32, _p, _p, _i32, _i32, _p, _p, _p],
    "vmamd_topk_softmax": [_p, _i32, _i64, _i32, _i32, _i32, _f32, _p, _p, _p, _p, _p],
    "vmamd_topk_sigmoid": [_p, _i32, _i64, _i32, _i32, _i32, _p, _p, _p, _p, _p],
    "vmamd_grouped_topk": [_p, _i32, _i64, _i32, _i32, _i32, _i32, _i32, _i32, _f32, _p, _p, _p,
                           _p],
    "vmamd_moe_align_block_size": [_p, _i64, _i32, _i32, _p, _i64, _p, _i64, _p, _p, _p, _p, _p,
                                   _p, _p],
    "vmamd_moe_align_block_size_quant_fp8": [_p, _i64, _i32, _i32, _p, _i64, _p, _i64, _p, _p, _p,
                                             _p, _p, _p, _i64, _i64, _p, _p, _p],
    "vmamd_moe_sum": [_p, _i32, _i64, _i32, _i64, _p, _p, _i64, _p, _p],
    "vmamd_w8a8_block_fp8_matmul_workspace_size": [_i64, _i64, _i64],
    "vmamd_w8a8_block_fp8_matmul": [_p, _p, _i64, _i64, _p, _p, _p, _i64, _i64, _i64, _i32, _i32,
                                    _p, _sz, _p],
    "vmamd_w8a8_block_fp8_matmul_noalloc": [_p, _p, _i64, _i64, _p, _p, _p, _i64, _i64, _i64,
                                            _i32, _i32, _p],
    "vmamd_fused_moe_fp8_workspace_size": [_i64, _i32, _i32, _i64, _i64, _i32],
    "vmamd_fused_moe_fp8": [_p, _i32, _i64, _i64, _p, _p, _p, _p, _i32, _i64, _p, _p, _i32, _p,
                            _i64, _f32, _i32, _i32, _p, _p, _sz, _p],
    "vmamd_moe_fp8_stage_workspace_size": [_i64, _i32, _i32, _i64, _i64, _i32],
    "vmamd_moe_fp8_w13": [_p, _p, _i64, _i64, _i32, _p, _i64, _i32, _p, _p, _p, _p, _p, _p, _i32,
                          _i64, _f32, _p, _p, _p, _sz, _p],
    "vmamd_moe_fp8_w2": [_p, _p, _i64, _i32, _p, _i64, _i32, _p, _p, _p, _p, _p, _p, _i32, _i64,
                         _i64, _p, _p, _p, _i64, _p, _p, _sz, _p],
    "vmamd_fused_moe_bf16_workspace_size": [_i64, _i32, _i32, _i64, _i64, _i32],
    "vmamd_fused_moe_bf16": [_p, _i64, _i64, _p, _p, _i32, _i64, _p, _p, _i32, _p, _i64, _f32,
                             _i32, _i32, _p, _p, _sz, _p],
    "vmamd_moe_bf16_stage_workspace_size": [_i64, _i32, _i32, _i64, _i64, _i32],
    "vmamd_moe_bf16_w13": [_p, _i64, _i64, _i32, _p, _i64, _i32, _p, _p, _p, _p, _p, _i32, _i64,
                           _f32, _p, _p, _sz, _p],
    "vmamd_moe_bf16_w2": [_p, _i64, _i32, _p, _i64, _i32, _p, _p, _p, _p, _p, _i32, _i64, _i64,
                          _p, _p, _p, _i64, _p, _p, _sz, _p],
    "vmamd_per_token_quant_fp8": [_p, _i64, _i64, _i64, _f32, _f32, _f32, _p, _p, _p],
    "vmamd_moe_weighted_sum": [_p, _i32, _i64, _i32, _i64, _p, _p, _p, _i64, _p, _p],
    "vmamd_w4afp8_moe_workspace_size": [_i64, _i32, _i32, _i64, _i64, _i32],
    "vmamd_w4afp8_moe": [_p, _i64, _i64, _p, _p, _p, _p, _i32, _i64, _p, _p, _i32, _p, _i64, _f32,
                         _i32, _p, _p, _sz, _p],
    "vmamd_fused_gemv_moe_workspace_size": [_i64, _i32, _i32, _i64, _i64, _i32, _i32],
    "vmamd_fused_gemv_moe": [_p, _i32, _p, _i64, _i64, _p, _i32, _p, _i32, _i64, _p, _p, _i32, _i32,
                             _i32, _f32, _p, _p, _sz, _p],
    "vmamd_fused_gemv_workspace_size": [_i64, _i64, _i64, _i32, _i32],
    "vmamd_fused_gemv": [_p, _i32, _p, _i64, _i64, _p, _i32, _p, _i64, _i32, _p, _p, _sz, _p],
}
_RESTYPES = {"vmamd_last_error": ctypes.c_char_p,
             "vmamd_w4afp8_moe_workspace_size": ctypes.c_size_t,
             "vmamd_fused_moe_bf16_workspace_size": ctypes.c_size_t,
             "vmamd_moe_bf16_stage_workspace_size": ctypes.c_size_t,
             "vmamd_w8a8_block_fp8_matmul_workspace_size": ctypes.c_size_t,
             "vmamd_fused_moe_fp8_workspace_size": ctypes.c_size_t,
             "vmamd_moe_fp8_stage_workspace_size": ctypes.c_size_t,
             "vmamd_fused_gemv_moe_workspace_size": ctypes.c_size_t,
             "vmamd_fused_gemv_workspace_size": ctypes.c_size_t}

_lib = None
_lock = threading.Lock()


class VmamdError(RuntimeError):
    """A C-ABI call returned an error status."""


def load() -> ctypes.CDLL:
    """Load the shared library once; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise ImportError(
                    f"{LIB_PATH} is missing: build it with `make -C vllm-musa_amd/csrc` "
                    "(or __graft_entry__.build()); there is no non-native fallback")
            lib = ctypes.CDLL(LIB_PATH)
            for name, args in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.argtypes = args
                fn.restype = _RESTYPES.get(name, ctypes.c_int)
            _lib = lib
    return _lib


def call(name: str, *args) -> None:
    """Invoke an entry point and raise VmamdError on a non-zero status."""
    lib = load()
    status = getattr(lib, name)(*args)
    if status != 0:
        msg = lib.vmamd_last_error().decode(errors="replace")
        if status == 1:
            raise ValueError(f"{name}: {msg}")
        raise VmamdError(f"{name} failed ({status}): {msg}")


def ptr(t: torch.Tensor | None) -> int | None:
    """Device pointer of a tensor (None -> NULL)."""
    return None if t is None else t.data_ptr()


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _TORCH_DTYPE[dt]
    except KeyError:
        raise ValueError(f"unsupported activation dtype {dt}") from None


def stream_of(t: torch.Tensor) -> int:
    """hipStream_t of torch's current stream on the tensor's device."""
    if t.device.type != "cuda":
        raise ValueError(f"vllm_musa_amd kernels run on the GPU; got a tensor on {t.device}")
    return torch.cuda.current_stream(t.device).cuda_stream


def check_cuda(*tensors: torch.Tensor | None) -> None:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise ValueError(f"expected a GPU tensor, got one on {t.device}")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} and {t.device}")
