"""CPU checks of the shared-expert fold's weight handling
(Fp8MoEMethod.fold_shared_expert; reference quantization/fp8.py:118-185): the
shared projections become expert E of the stack in the routed layout, are
released afterwards, mismatched shapes or dtypes are refused, and a second
fold does nothing."""
from __future__ import annotations

from types import SimpleNamespace

import pytest
import torch

from vllm_musa_amd.quant_methods import Fp8MoEMethod

E, H, I = 4, 256, 128


def _layer():
    g = torch.Generator().manual_seed(0)
    f8 = lambda *s: torch.randn(*s, generator=g).to(torch.float8_e4m3fn)
    layer = SimpleNamespace(w13_weight=f8(E, 2 * I, H), w2_weight=f8(E, H, I),
                            w13_weight_scale_inv=torch.rand(E, 2 * I // 128, H // 128, generator=g),
                            w2_weight_scale_inv=torch.rand(E, H // 128, I // 128, generator=g),
                            expert_map=None)
    mlp = SimpleNamespace(gate_up_proj=SimpleNamespace(weight=f8(2 * I, H),
                                                       weight_scale_inv=torch.rand(2 * I // 128, H // 128)),
                          down_proj=SimpleNamespace(weight=f8(H, I),
                                                    weight_scale_inv=torch.rand(H // 128, I // 128)))
    return layer, mlp


def test_fold_appends_expert_e_and_releases_shared():
    layer, mlp = _layer()
    w13, s13 = layer.w13_weight.clone(), layer.w13_weight_scale_inv.clone()
    gu, gus = mlp.gate_up_proj.weight.clone(), mlp.gate_up_proj.weight_scale_inv.clone()
    dn = mlp.down_proj.weight.clone()
    Fp8MoEMethod().fold_shared_expert(layer, mlp)
    assert layer._musa_shared_folded and layer._musa_shared_expert_id == E
    assert layer.w13_weight.shape == (E + 1, 2 * I, H) and layer.w2_weight.shape == (E + 1, H, I)
    u8 = lambda t: t.view(torch.uint8)
    assert torch.equal(u8(layer.w13_weight[:E]), u8(w13)) and torch.equal(u8(layer.w13_weight[E]), u8(gu))
    assert torch.equal(u8(layer.w2_weight[E]), u8(dn))
    assert torch.equal(layer.w13_weight_scale_inv[:E], s13)
    assert torch.equal(layer.w13_weight_scale_inv[E], gus)
    assert layer.w13_weight.is_contiguous() and layer.w2_weight_scale_inv.is_contiguous()
    assert mlp.gate_up_proj.weight is None and mlp.down_proj.weight_scale_inv is None


def test_fold_is_done_once():
    layer, mlp = _layer()
    m = Fp8MoEMethod()
    m.fold_shared_expert(layer, mlp)
    m.fold_shared_expert(layer, mlp)  # already folded: nothing happens
    assert layer.w13_weight.shape[0] == E + 1


@pytest.mark.parametrize("what", ["shape", "dtype", "scale"])
def test_fold_refuses_mismatches(what):
    layer, mlp = _layer()
    if what == "shape":
        mlp.down_proj.weight = mlp.down_proj.weight[:, :64]
    elif what == "dtype":
        mlp.gate_up_proj.weight = mlp.gate_up_proj.weight.to(torch.bfloat16)
    else:
        mlp.down_proj.weight_scale_inv = torch.rand(1, 1)
    with pytest.raises(RuntimeError):
        Fp8MoEMethod().fold_shared_expert(layer, mlp)


def test_fold_refuses_expert_parallel():
    layer, mlp = _layer()
    layer.expert_map = torch.arange(E, dtype=torch.int32)
    with pytest.raises(RuntimeError):
        Fp8MoEMethod().fold_shared_expert(layer, mlp)
