"""fused_experts_impl(path="auto") follows the dispatch on the GPU.  On the
fp8 shape E=256, N=256, H=2048, top-8 the reference runs its native GEMV up
to 13 tokens (its S5000 table), so auto computes those numerics there
(path 3); above, MI355X's own table picks the W8A8 decode kernels up to 64
tokens (path 1) and the grouped GEMMs beyond (path 2).  Each result is
bitwise the forced path's, the overrides map to the reference's backends,
and a captured call follows the capture entry."""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

E, N, I, H, TOPK = 256, 256, 128, 2048, 8


@pytest.fixture(scope="module")
def layer():
    from vllm_musa_amd import synthetic
    w13, s13, w2, s2 = synthetic.moe_fp8_weights(E, H, I, 21)
    return w13, s13, w2, s2


@pytest.fixture
def paths(monkeypatch):
    """Records the path code (1 = W8A8 decode kernels, 2 = grouped GEMMs,
    3 = native GEMV numerics) of every fused fp8 layer launched through the
    C ABI."""
    from vllm_musa_amd import fused_moe
    seen = []
    real = fused_moe.call

    def spy(name, *args):
        if name == "vmamd_fused_moe_fp8":
            seen.append(args[17])
        return real(name, *args)

    monkeypatch.setattr(fused_moe, "call", spy)
    return seen


def _run(layer, t, path="auto"):
    from vllm_musa_amd import synthetic
    from vllm_musa_amd.fused_moe import fused_experts_impl
    w13, s13, w2, s2 = layer
    x = synthetic.activations(t, H, 300 + t)
    g = torch.Generator().manual_seed(t)
    ids = torch.stack([torch.randperm(E, generator=g)[:TOPK] for _ in range(t)]).to(torch.int32)
    w = torch.softmax(torch.randn(t, TOPK, generator=g), -1)
    return fused_experts_impl(x, w13, w2, w.cuda(), ids.cuda(), use_fp8_w8a8=True, w1_scale=s13,
                              w2_scale=s2, block_shape=[128, 128], path=path)


def test_auto_follows_the_calibrated_threshold(layer, paths):
    from vllm_musa_amd import dispatch_policy as dp
    from vllm_musa_amd.dispatch_policy import shape_of_layer, thresholds_for_shape
    w13, s13, w2, s2 = layer
    x = torch.zeros(1, H, dtype=torch.bfloat16, device="cuda")
    th = thresholds_for_shape(shape_of_layer(x, w13, w2, s13, s2, TOPK, [128, 128], None, "eager"))
    assert th.gemv_max_tokens == 64, th  # the device really is the calibrated MI355X
    forced = {1: "gemv", 2: "gemm", 3: "native_gemv"}
    for t, code in ((1, 3), (13, 3), (14, 1), (64, 1), (65, 2), (300, 2)):
        paths.clear()
        out = _run(layer, t)
        assert paths == [code], (t, paths)
        assert torch.equal(out, _run(layer, t, forced[code]))
    assert dp.resolve_path(x, w13, w2, s13, s2, TOPK, [128, 128], None) == "gemv"


def test_override_forces_a_backend(layer, monkeypatch, paths):
    from vllm_musa_amd import dispatch_policy as dp
    monkeypatch.setenv(dp.MUSA_FUSED_MOE_DISPATCH_ENV, "grouped_gemm")
    _run(layer, 4)
    monkeypatch.setenv(dp.MUSA_FUSED_MOE_DISPATCH_ENV, "gemv")
    _run(layer, 100)
    monkeypatch.setenv(dp.MUSA_FUSED_MOE_DISPATCH_ENV, "upstream")
    _run(layer, 4)
    assert paths == [2, 3, 1]


def test_captured_call_uses_capture_entry(layer, paths):
    from vllm_musa_amd import synthetic
    from vllm_musa_amd.fused_moe import fused_experts_impl
    w13, s13, w2, s2 = layer
    t = 8
    x = synthetic.activations(t, H, 77)
    ids = (torch.arange(t * TOPK) % E).reshape(t, TOPK).to(torch.int32).cuda()
    w = torch.full((t, TOPK), 1.0 / TOPK, device="cuda")
    call = lambda path: fused_experts_impl(x, w13, w2, w, ids, use_fp8_w8a8=True, w1_scale=s13,
                                           w2_scale=s2, block_shape=[128, 128], path=path)
    eager = call("native_gemv")
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call("auto")
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    paths.clear()
    with torch.cuda.graph(graph):
        out = call("auto")
    assert paths == [3]
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
