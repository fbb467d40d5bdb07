"""Host-side W4AFP8 expert loading: allocation, tensor-parallel shards and the
size gate, mirroring the reference's tests/test_w4afp8_quantization.py
(test_tp8_unaligned_groups_fail_instead_of_silently_slicing_scales,
test_packed_weight_allocation_and_scale_conversion,
test_packed_weights_and_group128_scales_use_matching_loader_shards)."""
from __future__ import annotations

import pytest
import torch

from vllm_musa_amd.quant_methods import W4AFp8MoEMethod


def test_unaligned_groups_fail():
    m = W4AFp8MoEMethod()
    assert m.maybe_roundup_sizes(5120, 2304, torch.bfloat16, None) == (5120, 2304)
    with pytest.raises(ValueError, match="enable-expert-parallel"):
        m.maybe_roundup_sizes(5120, 288, torch.bfloat16, None)
    with pytest.raises(ValueError):
        m.maybe_roundup_sizes(5000, 256, torch.bfloat16, None)


def test_packed_weight_allocation():
    m = W4AFp8MoEMethod()
    layer = torch.nn.Module()
    loader = object()
    m.create_weights(layer, 2, 256, 384, torch.bfloat16, device="cpu", weight_loader=loader)
    assert layer.w13_weight.shape == (2, 768, 128)
    assert layer.w2_weight.shape == (2, 256, 192)
    assert layer.w13_weight_scale_inv.shape == (2, 768, 2)
    assert layer.w2_weight_scale_inv.shape == (2, 256, 3)
    assert layer.w13_weight.dtype == torch.int8
    assert layer.w13_weight_scale_inv.dtype == torch.float32
    assert layer.w13_input_scale.dtype == torch.bfloat16 and (layer.w2_input_scale == 1).all()
    assert layer.w13_weight.weight_loader is loader
    assert layer.w2_weight_scale_inv.quant_method == "group"
    assert not hasattr(layer.w13_weight, "quant_method")


@pytest.mark.parametrize("tp_size,tp_rank", [(1, 0), (2, 0), (2, 1), (4, 3)])
def test_packed_weights_and_group128_scales_use_matching_loader_shards(tp_size, tp_rank):
    m = W4AFp8MoEMethod()
    layer = torch.nn.Module()
    intermediate, hidden = 128 * 4, 128
    m.create_weights(layer, 1, hidden, intermediate // tp_size, torch.bfloat16, device="cpu")
    for shard_id, name, shape, dim, dtype in (
            ("w1", "w13_weight", (intermediate, hidden // 2), 0, torch.int8),
            ("w3", "w13_weight", (intermediate, hidden // 2), 0, torch.int8),
            ("w2", "w2_weight", (hidden, intermediate // 2), 1, torch.int8),
            ("w1", "w13_weight_scale_inv", (intermediate, hidden // 128), 0, torch.float32),
            ("w3", "w13_weight_scale_inv", (intermediate, hidden // 128), 0, torch.float32),
            ("w2", "w2_weight_scale_inv", (hidden, intermediate // 128), 1, torch.float32)):
        ckpt = torch.arange(shape[0] * shape[1]).reshape(shape).to(dtype)
        m.load_weight(layer, name, ckpt, 0, shard_id, tp_rank, tp_size)
        dest = getattr(layer, name).data[0]
        want = ckpt.chunk(tp_size, dim=dim)[tp_rank]
        if shard_id in ("w1", "w3"):
            dest = dest.chunk(2, dim=0)[shard_id == "w3"]
        torch.testing.assert_close(dest, want, rtol=0, atol=0)


def test_loader_rejects_mismatched_checkpoints():
    m = W4AFp8MoEMethod()
    layer = torch.nn.Module()
    m.create_weights(layer, 2, 256, 128, torch.bfloat16, device="cpu")
    with pytest.raises(ValueError, match="checkpoint shape"):
        m.load_weight(layer, "w13_weight", torch.zeros(256, 128, dtype=torch.int8), 0, "w1", 0, 1)
    with pytest.raises(ValueError, match="checkpoint shape"):
        m.load_weight(layer, "w2_weight", torch.zeros(256, 128, dtype=torch.int8), 1, "w2", 0, 1)
    with pytest.raises(ValueError, match="belongs to w13"):
        m.load_weight(layer, "w2_weight", torch.zeros(128, 128, dtype=torch.int8), 0, "w1", 0, 1)
    with pytest.raises(ValueError, match="shard id"):
        m.load_weight(layer, "w2_weight", torch.zeros(256, 64, dtype=torch.int8), 0, "w4", 0, 1)
    with pytest.raises(ValueError, match="tp_rank"):
        m.load_weight(layer, "w2_weight", torch.zeros(256, 64, dtype=torch.int8), 0, "w2", 2, 2)
    before = layer.w13_input_scale.clone()
    m.load_weight(layer, "w13_input_scale", torch.full((1,), 5.0), 0, "w1", 0, 1)
    assert torch.equal(layer.w13_input_scale, before)
