"""w4afp8 fused MoE with the reference's Python signature.

Reference: w4afp8_moe (vllm_musa/kernels/w4afp8_moe.py:164-362); argument
checks and messages follow its lines 177-221.  The whole layer is one C-ABI
call (vmamd_w4afp8_moe): per-row fp8 quantisation of x, moe_align_block_size,
the int4 x fp8 W13 GEMM with SiLU-and-mul, per-row quantisation of the
activation, the W2 GEMM and the weighted combine, all on the current stream.
"""
from __future__ import annotations

import torch

from . import _lib
from ._lib import call, ptr, stream_of

PATHS = {"auto": 0, "gemv": 1, "gemm": 2}


def w4afp8_moe(hidden_states: torch.Tensor, gateup_weight: torch.Tensor,
               down_weight: torch.Tensor, gateup_scale: torch.Tensor, down_scale: torch.Tensor,
               topk_weights: torch.Tensor, topk_ids: torch.Tensor,
               expert_map: torch.Tensor | None = None, *, swiglu_limit: float | None = None,
               path: str = "auto") -> torch.Tensor:
    """Routed W4AFP8 experts without expanding the packed int4 weights.

    hidden_states [T, H] bf16; gateup_weight [E, 2I, H/2] and down_weight
    [E, H, I/2] int8 (two signed int4 per byte, even index in the low nibble);
    gateup_scale [E, 2I, H/128] and down_scale [E, H, I/128] bf16;
    topk_weights / topk_ids [T, topk]; expert_map maps global to local ids
    (-1: not local)."""
    if hidden_states.ndim != 2 or gateup_weight.ndim != 3:
        raise ValueError("W4AFP8 expects hidden states [T,H] and weights [E,N,K/2]")
    tokens, hidden = hidden_states.shape
    experts, doubled_intermediate, packed_hidden = gateup_weight.shape
    intermediate = doubled_intermediate // 2
    if (topk_ids.ndim != 2 or topk_ids.shape[0] != tokens or topk_weights.shape != topk_ids.shape
            or topk_ids.shape[1] == 0):
        raise ValueError("W4AFP8 routing IDs and weights must have matching [T,topk] shapes")
    if topk_ids.dtype not in (torch.int32, torch.int64):
        raise ValueError("W4AFP8 routing IDs must be INT32 or INT64")
    if expert_map is not None and (expert_map.ndim != 1 or
                                   expert_map.dtype not in (torch.int32, torch.int64)):
        raise ValueError("W4AFP8 expert map must be a one-dimensional integer tensor")
    if (experts == 0 or hidden == 0 or intermediate == 0 or doubled_intermediate % 2
            or hidden != packed_hidden * 2 or hidden % 128 or intermediate % 128):
        raise ValueError("W4AFP8 requires packed INT4 K/2 and group128 dimensions")
    if hidden_states.dtype != torch.bfloat16:
        raise ValueError("W4AFP8 requires BF16 hidden states")
    if gateup_weight.dtype != torch.int8 or down_weight.dtype != torch.int8:
        raise ValueError("W4AFP8 weights must be signed INT4 packed into INT8")
    if down_weight.shape != (experts, hidden, intermediate // 2):
        raise ValueError("W4AFP8 Down weight shape does not match GateUp")
    for scale, expected in ((gateup_scale, (experts, doubled_intermediate, hidden // 128)),
                            (down_scale, (experts, hidden, intermediate // 128))):
        if tuple(scale.shape) != expected or scale.dtype != torch.bfloat16:
            raise ValueError("W4AFP8 weight scales must be BF16 [E,N,K/128]")
    if tokens == 0:
        return torch.empty_like(hidden_states)
    x = hidden_states.contiguous()
    ids = topk_ids.to(torch.int32).contiguous()
    wts = topk_weights.to(torch.float32).contiguous()
    emap = None if expert_map is None else expert_map.to(torch.int32).contiguous()
    w13, w2 = gateup_weight.contiguous(), down_weight.contiguous()
    s13, s2 = gateup_scale.contiguous(), down_scale.contiguous()
    # The grouped GEMMs read the bf16 scales in aligned 4-byte words.
    s13 = s13 if s13.data_ptr() % 4 == 0 else s13.clone()
    s2 = s2 if s2.data_ptr() % 4 == 0 else s2.clone()
    _lib.check_cuda(x, w13, w2, s13, s2, wts, ids, emap)
    topk = ids.shape[1]
    code = PATHS[path]
    limit = 0.0 if swiglu_limit is None else float(swiglu_limit)
    nbytes = _lib.load().vmamd_w4afp8_moe_workspace_size(tokens, topk, experts, hidden,
                                                          intermediate, code)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=x.device)
    out = torch.empty_like(x)
    call("vmamd_w4afp8_moe", ptr(x), tokens, hidden, ptr(w13), ptr(s13), ptr(w2), ptr(s2), experts,
         intermediate, ptr(wts), ptr(ids), topk, ptr(emap), 0 if emap is None else emap.numel(),
         limit, code, ptr(out), ptr(ws), nbytes, stream_of(x))
    return out
