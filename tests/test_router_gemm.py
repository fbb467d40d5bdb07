"""Guard contract of the fp32 router gate (host side), after the reference's
tests/test_musa_router_gemm.py:52-120: CPU tensors and the kill switch are
declined, and meta tensors (how tracing presents the operands) are served by
the op's fake implementation for the supported gate only."""
from __future__ import annotations

import pytest
import torch

from vllm_musa_amd import router_gemm as rg

HIDDEN, EXPERTS = 2688, 128
FOREIGN_GATE_SHAPES = ((128, 2048), (256, 4096), (256, 7168), (64, 2048))


def test_guard_declines_cpu_tensors():
    x = torch.zeros((4, HIDDEN), dtype=torch.bfloat16)
    w = torch.zeros((EXPERTS, HIDDEN), dtype=torch.float32)
    assert rg.router_gate_fp32(x, w) is None


def test_guard_respects_env_kill_switch(monkeypatch):
    assert rg.router_gate_enabled()
    monkeypatch.setenv("VLLM_MUSA_ROUTER_GATE_FP32", "0")
    assert not rg.router_gate_enabled()
    x = torch.zeros((7, HIDDEN), dtype=torch.bfloat16, device="meta")
    w = torch.zeros((EXPERTS, HIDDEN), dtype=torch.float32, device="meta")
    assert rg.router_gate_fp32(x, w) is None


def test_guard_serves_meta_tensors_for_the_supported_gate_only():
    before = rg.activation_count()
    x = torch.zeros((7, HIDDEN), dtype=torch.bfloat16, device="meta")
    w = torch.zeros((EXPERTS, HIDDEN), dtype=torch.float32, device="meta")
    out = rg.router_gate_fp32(x, w)
    assert out is not None and tuple(out.shape) == (7, EXPERTS) and out.dtype == torch.float32
    assert rg.activation_count() == before  # the fake implementation launches nothing
    for experts, hidden in FOREIGN_GATE_SHAPES:
        xf = torch.zeros((7, hidden), dtype=torch.bfloat16, device="meta")
        wf = torch.zeros((experts, hidden), dtype=torch.float32, device="meta")
        assert rg.router_gate_fp32(xf, wf) is None
    assert rg.router_gate_fp32(x, w.to(torch.bfloat16)) is None
    assert rg.router_gate_fp32(x.to(torch.float16), w) is None
    wide = torch.zeros((EXPERTS, 2 * HIDDEN), dtype=torch.float32, device="meta")
    assert rg.router_gate_fp32(x, wide[:, ::2]) is None


def test_custom_op_is_registered():
    assert hasattr(torch.ops.vllm_musa_amd, "router_gate_fp32")
