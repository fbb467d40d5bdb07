"""CPU checks of the row-parallel forward_swiglu_clamp hook's gates (the
reference's conditions, vllm_musa/model_executor/layers/linear.py:58-74): every
unmet condition returns None before any GPU work, so the model runs its
ordinary activation and linear path."""
from __future__ import annotations

from types import SimpleNamespace

import pytest
import torch

from vllm_musa_amd.block_fp8 import Fp8BlockScaledMMKernel, silu_clamp_block_fp8_matmul
from vllm_musa_amd.linear import forward_swiglu_clamp


def _layer(**kw):
    base = dict(quant_method=SimpleNamespace(block_quant=True, fp8_linear=Fp8BlockScaledMMKernel()),
                input_is_parallel=True, bias=None, input_size_per_partition=256,
                output_size_per_partition=64, weight=None, weight_scale_inv=None,
                weight_block_size=(128, 128), reduce_results=True, tp_size=1)
    base.update(kw)
    return SimpleNamespace(**base)


GATE_UP = torch.zeros(3, 512, dtype=torch.bfloat16)


@pytest.mark.parametrize("kw,x,limit", [
    (dict(bias=torch.zeros(64)), GATE_UP, 10.0),
    (dict(input_is_parallel=False), GATE_UP, 10.0),
    (dict(quant_method=SimpleNamespace(block_quant=False, fp8_linear=Fp8BlockScaledMMKernel())), GATE_UP, 10.0),
    (dict(quant_method=SimpleNamespace(block_quant=True, fp8_linear=object())), GATE_UP, 10.0),
    (dict(quant_method=None), GATE_UP, 10.0),
    (dict(weight_block_size=(64, 64)), GATE_UP, 10.0),
    (dict(input_size_per_partition=128), GATE_UP, 10.0),
    ({}, GATE_UP.float(), 10.0),
    ({}, torch.zeros(512, 3, dtype=torch.bfloat16).t(), 10.0),
    ({}, torch.zeros(512, dtype=torch.bfloat16), 10.0),
    ({}, GATE_UP, 8.0),
])
def test_gates_return_none(kw, x, limit):
    assert forward_swiglu_clamp(_layer(**kw), x, limit) is None


def test_missing_weight_scale_returns_none():
    assert forward_swiglu_clamp(_layer(), GATE_UP, 10.0) is None


def test_batch_invariant_returns_none(monkeypatch):
    monkeypatch.setenv("VLLM_BATCH_INVARIANT", "1")
    layer = _layer(weight_scale_inv=torch.ones(1, 2))
    assert forward_swiglu_clamp(layer, GATE_UP, 10.0) is None


def test_ue8m0_scales_are_refused():
    with pytest.raises(NotImplementedError):
        silu_clamp_block_fp8_matmul(GATE_UP, torch.zeros(64, 256), torch.ones(1, 2), 128, True, 10.0)
