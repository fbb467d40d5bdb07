"""Block-grid padding of the fp8 MoE intermediate partition (quant_methods:
Fp8MoEMethod.maybe_roundup_sizes / create_weights / load_expert), after the
reference's quantization/fp8.py:27-115.

The pin: zero-filled padding rows of W13 and columns of W2 contribute nothing,
so the oracle's layer on the padded stack equals the layer on the unpadded
one exactly (the padding's a2 group is all zeros: silu(0) * 0 = 0, its
quantised codes are 0, and it meets zero W2 columns).
"""
from __future__ import annotations

import types

import numpy as np
import pytest
import torch

from oracle import moe as omoe
from oracle.numerics import bf16_round
from vllm_musa_amd.quant_methods import Fp8MoEMethod


@pytest.fixture
def rng():
    return np.random.default_rng(2024)


@pytest.mark.parametrize("tp,i,want", [(1, 320, 320), (2, 320, 384), (8, 256, 256), (4, 200, 256),
                                       (2, 128, 128), (2, 129, 256)])
def test_roundup_sizes(tp, i, want):
    m = Fp8MoEMethod()
    cfg = types.SimpleNamespace(tp_size=tp)
    assert m.maybe_roundup_sizes(7168, i, torch.bfloat16, cfg) == (7168, want)


def test_roundup_needs_block_quant():
    m = Fp8MoEMethod(block_quant=False)
    assert m.maybe_roundup_sizes(1024, 320, torch.bfloat16, types.SimpleNamespace(tp_size=4)) == (1024, 320)


def test_roundup_uses_lcm_of_block_sides():
    m = Fp8MoEMethod(block_shape=(128, 64))
    assert m.maybe_roundup_sizes(512, 200, torch.bfloat16, types.SimpleNamespace(tp_size=2)) == (512, 256)


def test_create_weights_zero_fills_padding():
    layer = types.SimpleNamespace()
    Fp8MoEMethod().create_weights(layer, 3, 256, 384, intermediate_size_unpadded=256, device="cpu")
    assert layer.w13_weight.shape == (3, 768, 256) and layer.w13_weight.dtype == torch.float8_e4m3fn
    assert layer.w2_weight.shape == (3, 256, 384)
    assert layer.w13_weight_scale_inv.shape == (3, 6, 2) and layer.w2_weight_scale_inv.shape == (3, 2, 3)
    assert not layer.w13_weight.view(torch.uint8).any() and not layer.w2_weight.view(torch.uint8).any()


def _codes(rng, shape):
    c = rng.integers(0, 256, shape).astype(np.uint8)
    c[(c & 0x7F) == 0x7F] = 0x38  # no NaN codes
    return c


def test_padded_stack_gives_the_unpadded_layer(rng):
    e, h, i0, i, t, k = 3, 256, 256, 384, 6, 2
    w13 = _codes(rng, (e, 2 * i0, h))
    w2 = _codes(rng, (e, h, i0))
    s13 = rng.uniform(0.5, 2, (e, 2 * i0 // 128, h // 128)).astype(np.float32) / 448 / 64
    s2 = rng.uniform(0.5, 2, (e, h // 128, i0 // 128)).astype(np.float32) / 448 / 64
    x = bf16_round(rng.standard_normal((t, h)).astype(np.float32))
    ids = np.stack([rng.permutation(e)[:k] for _ in range(t)]).astype(np.int32)
    w = rng.uniform(0.1, 1.0, (t, k)).astype(np.float32)

    m = Fp8MoEMethod()
    layer = types.SimpleNamespace()
    m.create_weights(layer, e, h, i, intermediate_size_unpadded=i0, device="cpu")
    for ex in range(e):
        m.load_expert(layer, ex, torch.from_numpy(w13[ex]).view(torch.float8_e4m3fn),
                      torch.from_numpy(s13[ex]), torch.from_numpy(w2[ex]).view(torch.float8_e4m3fn),
                      torch.from_numpy(s2[ex]))
    u8 = lambda tt: tt.view(torch.uint8).numpy()
    padded = omoe.fused_experts_fp8(x, u8(layer.w13_weight), layer.w13_weight_scale_inv.numpy(),
                                    u8(layer.w2_weight), layer.w2_weight_scale_inv.numpy(), w, ids)
    plain = omoe.fused_experts_fp8(x, w13, s13, w2, s2, w, ids)
    np.testing.assert_array_equal(padded, plain)


def test_load_expert_rejects_off_grid_sizes():
    layer = types.SimpleNamespace()
    m = Fp8MoEMethod()
    m.create_weights(layer, 1, 256, 384, intermediate_size_unpadded=200, device="cpu")
    with pytest.raises(ValueError):
        m.load_expert(layer, 0, torch.zeros(400, 256, dtype=torch.float8_e4m3fn), torch.ones(4, 2),
                      torch.zeros(256, 200, dtype=torch.float8_e4m3fn), torch.ones(2, 2))
