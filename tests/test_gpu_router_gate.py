"""vmamd_router_gate_fp32 on the GPU: bitwise equal to the oracle's fixed
order (reference contract: tests/test_musa_router_gemm.py:131-167, bitwise
logits so the router's top-k cannot move), batch invariant, close to the
platform's own fp32 GEMM, and the guard decisions on device tensors
(tests/test_musa_router_gemm.py:62-128)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import router_gate as org

pytestmark = pytest.mark.gpu
DEV = "cuda"
HIDDEN, EXPERTS = 2688, 128
FOREIGN_GATE_SHAPES = ((128, 2048), (256, 4096), (256, 7168), (64, 2048))


def _bits(t):
    return t.detach().float().cpu().numpy().view(np.uint32)


def _inputs(m, x_dtype, weight_bf16, seed, k=HIDDEN, e=EXPERTS):
    g = torch.Generator().manual_seed(seed)
    w = torch.randn((e, k), generator=g, dtype=torch.float32)
    if weight_bf16:  # what a bf16 checkpoint gives
        w = w.to(torch.bfloat16).to(torch.float32)
    x = torch.randn((m, k), generator=g, dtype=torch.float32).to(x_dtype)
    return x, w


@pytest.mark.parametrize("m", [1, 2, 7, 64, 65, 115, 512])
@pytest.mark.parametrize("x_dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("weight_bf16", [True, False])
def test_bitwise_equal_to_oracle(m, x_dtype, weight_bf16):
    from vllm_musa_amd.router_gemm import router_gate_fp32
    x, w = _inputs(m, x_dtype, weight_bf16, 100037 + m)
    out = router_gate_fp32(x.to(DEV), w.to(DEV))
    assert out is not None and out.dtype == torch.float32 and tuple(out.shape) == (m, EXPERTS)
    rows = np.arange(m) if m <= 128 else np.unique(np.r_[0, 1, m - 1, np.arange(3, m, 37)])
    ref = org.router_gate_fp32(x.float().numpy()[rows], w.numpy())
    assert np.array_equal(_bits(out)[rows], ref.view(np.uint32))


def test_batch_invariant_and_deterministic():
    from vllm_musa_amd.router_gemm import router_gate_fp32
    x, w = _inputs(512, torch.bfloat16, True, 5)
    xd, wd = x.to(DEV), w.to(DEV)
    full = router_gate_fp32(xd, wd)
    assert torch.equal(full, router_gate_fp32(xd, wd))
    for lo, hi in ((0, 1), (5, 7), (100, 115), (64, 128), (511, 512)):
        assert torch.equal(router_gate_fp32(xd[lo:hi].contiguous(), wd), full[lo:hi])


@pytest.mark.parametrize("m", [1, 7, 115])
def test_close_to_platform_fp32_gemm_and_topk_stream(m):
    from vllm_musa_amd.router_gemm import router_gate_fp32
    g = torch.Generator().manual_seed(7000 + m)
    w = torch.randn((EXPERTS, HIDDEN), generator=g).to(torch.bfloat16)
    x = torch.randn((m, HIDDEN), generator=g).to(torch.bfloat16)
    out = router_gate_fp32(x.to(DEV), w.float().to(DEV))
    plat = x.to(DEV).float() @ w.to(DEV).float().t()
    exact = x.double() @ w.double().t()
    scale = (x.double().abs() @ w.double().abs().t())
    assert ((out.double().cpu() - exact).abs() <= (HIDDEN // 64 + 6) * 2.0 ** -24 * scale).all()
    assert (out - plat).abs().max().item() <= 1e-4 * plat.abs().max().item()
    assert torch.equal(out.topk(6, dim=-1).indices.cpu(), exact.topk(6, dim=-1).indices)


def test_guard_on_device_tensors():
    from vllm_musa_amd import router_gemm as rg
    x = torch.zeros((4, HIDDEN), device=DEV, dtype=torch.bfloat16)
    w = torch.zeros((EXPERTS, HIDDEN), device=DEV, dtype=torch.float32)
    for experts, hidden in FOREIGN_GATE_SHAPES:
        assert rg.router_gate_fp32(torch.zeros((4, hidden), device=DEV, dtype=torch.bfloat16),
                                   torch.zeros((experts, hidden), device=DEV)) is None
    assert rg.router_gate_fp32(x, w.to(torch.bfloat16)) is None
    assert rg.router_gate_fp32(x, w.to(torch.float16)) is None
    assert rg.router_gate_fp32(x.to(torch.float16), w) is None
    assert rg.router_gate_fp32(x[:, :1024].contiguous(), w) is None
    wide = torch.zeros((EXPERTS, 2 * HIDDEN), device=DEV, dtype=torch.float32)
    assert rg.router_gate_fp32(x, wide[:, ::2]) is None
    empty = rg.router_gate_fp32(x[:0], w)
    assert empty is not None and tuple(empty.shape) == (0, EXPERTS)
    before = rg.activation_count()
    assert rg.router_gate_fp32(x, w) is not None
    assert rg.activation_count() == before + 1
    declined = torch.zeros((7, 2048), device=DEV)
    assert rg.router_gate_fp32(declined, w[:, :2048].contiguous()) is None
    assert rg.activation_count() == before + 1


@pytest.mark.parametrize("m,k,e", [(5, 256, 3), (3, 128, 1), (70, 384, 6), (1, 7168, 256)])
def test_c_abi_general_shapes(m, k, e):
    from vllm_musa_amd import _custom_ops as ops
    x, w = _inputs(m, torch.float32, False, m * k + e, k=k, e=e)
    out = torch.full((m, e), float("nan"), device=DEV)
    ops.router_gate_fp32(x.to(DEV), w.to(DEV), out)
    assert np.array_equal(_bits(out), org.router_gate_fp32(x.numpy(), w.numpy()).view(np.uint32))


def test_c_abi_rejects_bad_arguments():
    from vllm_musa_amd import _custom_ops as ops
    w = torch.zeros((4, 200), device=DEV)
    with pytest.raises(ValueError, match="multiple of 128"):
        ops.router_gate_fp32(torch.zeros((2, 200), device=DEV), w, torch.zeros((2, 4), device=DEV))
    with pytest.raises(ValueError):
        ops.router_gate_fp32(torch.zeros((2, 256), device=DEV), torch.zeros((4, 256), device=DEV),
                             torch.zeros((2, 5), device=DEV))
    with pytest.raises(ValueError):
        ops.router_gate_fp32(torch.zeros((2, 256), device=DEV, dtype=torch.float16),
                             torch.zeros((4, 256), device=DEV), torch.zeros((2, 4), device=DEV))
