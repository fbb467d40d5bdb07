"""The fp8 block MoE layer restated in PyTorch on the CPU (float32 contractions,
multi-threaded): the CPU baseline that bench.py times beside the GPU layer.

Test infrastructure, like the rest of oracle/: only tests/ and bench.py's
cpu_baseline import it.  Same rounding points as oracle/moe.py (reference:
fused_moe.py:1935-2184; activation then a2 quantisation, patches/series/
0144-...:62-78; block-scaled accumulate, 0081-...:64-108; routed weight in the
W2 epilogue, fused_moe.py:2164-2178; moe_sum in slot order, jit_kernel/csrc/
moe/moe_sum_reduce.mu:127-146), with the contractions in float32 on
dequantised operands, the reference's own fp32 oracle style
(benchmarks/fused_moe/benchmark_dispatch_crossover.py:660-707).  Its outputs
agree with oracle/moe.py within the path's tolerance
(tests/test_oracle_moe_torch.py).
"""
from __future__ import annotations

import torch

FP8 = torch.float8_e4m3fn


def group_quant_fp8(x: torch.Tensor, group: int = 128, eps: float = 1e-10):
    """x [M, K] float -> (e4m3 values as float32 [M, K], scales [M, K/group])."""
    m, k = x.shape
    g = x.float().reshape(m, k // group, group)
    s = g.abs().amax(dim=-1).clamp_min(eps) / 448.0
    q = (g / s[..., None]).clamp(-448.0, 448.0).to(FP8).float()
    return q.reshape(m, k), s


def _dequant(wq: torch.Tensor, ws: torch.Tensor, block: int = 128) -> torch.Tensor:
    """e4m3 codes (uint8 [N, K]) and [ceil(N/b), K/b] scales -> float32 [N, K]."""
    w = wq.view(FP8).float()
    n, k = w.shape
    s = ws.float().repeat_interleave(block, 0)[:n].repeat_interleave(block, 1)[:, :k]
    return w * s


def fused_experts_fp8(x, w13_q, w13_s, w2_q, w2_s, topk_weights, topk_ids, block: int = 128):
    """x [T, H] bf16-valued; w13_q [E, 2I, H] / w2_q [E, H, I] uint8 e4m3 codes with
    float32 block scales; topk_weights [T, K] float32, topk_ids [T, K] int
    (negative: no expert).  Returns the bf16-valued output [T, H] (float32)."""
    x = torch.as_tensor(x).float()
    ids = torch.as_tensor(topk_ids).long()
    w = torch.as_tensor(topk_weights).float()
    t, h = x.shape
    k = ids.shape[1]
    i = w13_q.shape[1] // 2
    xq, xs = group_quant_fp8(x, block)
    xd = xq * xs.repeat_interleave(block, 1)
    y = torch.zeros(t, k, h)
    for e in torch.unique(ids[ids >= 0]).tolist():
        tt, kk = torch.nonzero(ids == e, as_tuple=True)
        w1 = _dequant(torch.as_tensor(w13_q[e]), torch.as_tensor(w13_s[e]), block)
        hh = (xd[tt] @ w1.T).bfloat16().float()
        a = (torch.nn.functional.silu(hh[:, :i]) * hh[:, i:]).bfloat16().float()
        aq, a_s = group_quant_fp8(a, block)
        w2 = _dequant(torch.as_tensor(w2_q[e]), torch.as_tensor(w2_s[e]), block)
        acc = (aq * a_s.repeat_interleave(block, 1)) @ w2.T
        y[tt, kk] = (acc * w[tt, kk][:, None]).bfloat16().float()
    out = torch.zeros(t, h)
    for kk in range(k):
        out = out + y[:, kk]
    return out.bfloat16().float()
