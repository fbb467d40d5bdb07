"""GPU parity of the shared-expert fold: the routing column that
extend_topk_with_shared / the fused-shared top-k append, and the folded fp8 MoE
layer (Fp8MoEMethod.fold_shared_expert + apply) against the oracle.

Routing: ids bit-exact; the shared weight is sigmoid(logit) in fp32 rounded to
the logit dtype, compared with numpy's float32 sigmoid rounded the same way (at
most one bf16 ulp apart, from the exp of each side).  Layer: the oracle's
fused fp8 MoE over the E+1-expert stack with the extended routing, to the
path's bar (rel-L2 <= 1e-2, max-abs <= 2e-2 max|ref|); and, as a check that does
not go through the fold, the routed layer plus the shared expert run as its own
one-route MoE agree with the folded layer to two bf16 roundings."""
from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from oracle.numerics import bf16_round

from test_gpu_moe import _check, _case, _oracle, _run

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _sigmoid_bf16(x: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        return bf16_round((np.float32(1) / (np.float32(1) + np.exp(-x.astype(np.float32)))).astype(np.float32))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_extend_topk_with_shared(dtype):
    from vllm_musa_amd.router import extend_topk_with_shared
    g = torch.Generator().manual_seed(4)
    T, K, E = 300, 8, 256
    w = torch.rand(T, K, generator=g).to(DEV)
    ids = torch.randint(0, E, (T, K), generator=g, dtype=torch.int32).to(DEV)
    logits = (torch.randn(T, 1, generator=g) * 4).to(dtype).to(DEV)
    logits[0, 0] = -100.0
    logits[1, 0] = 100.0
    ow, oi = extend_topk_with_shared(w, ids, logits, E)
    assert ow.shape == (T, K + 1) and oi.shape == (T, K + 1)
    assert torch.equal(ow[:, :K], w) and torch.equal(oi[:, :K], ids)
    assert (oi[:, K] == E).all()
    lg = logits.float().cpu().numpy().reshape(-1)
    with np.errstate(over="ignore"):  # fp32 sigmoid: exp overflows to inf, the weight to 0
        ref32 = np.float32(1) / (np.float32(1) + np.exp(-lg.astype(np.float32)))
    ref = _sigmoid_bf16(lg) if dtype == torch.bfloat16 else ref32
    got = ow[:, K].cpu().numpy()
    np.testing.assert_allclose(got, ref, rtol=2 ** -8 if dtype == torch.bfloat16 else 1e-6, atol=0)
    assert got[0] == 0.0 and got[1] == 1.0


@pytest.mark.parametrize("scoring", ["softmax", "sigmoid"])
def test_topk_with_fused_shared_column(scoring):
    from vllm_musa_amd import _custom_ops as ops
    g = torch.Generator().manual_seed(5)
    T, E, K = 97, 128, 8
    gating = torch.randn(T, E, generator=g).to(DEV)
    shared = torch.randn(T, generator=g).to(torch.bfloat16).to(DEV)
    fn = ops.topk_softmax if scoring == "softmax" else ops.topk_sigmoid
    w0 = torch.empty(T, K, device=DEV)
    i0 = torch.empty(T, K, dtype=torch.int32, device=DEV)
    fn(w0, i0, gating, True)
    w1 = torch.empty(T, K + 1, device=DEV)
    i1 = torch.empty(T, K + 1, dtype=torch.int32, device=DEV)
    fn(w1, i1, gating, True, shared_expert_gate_output=shared, num_fused_shared_experts=1)
    assert torch.equal(w1[:, :K], w0) and torch.equal(i1[:, :K], i0)
    assert (i1[:, K] == E).all()
    np.testing.assert_allclose(w1[:, K].cpu().numpy(), _sigmoid_bf16(shared.float().cpu().numpy()),
                               rtol=2 ** -8)


def _fold_case(T, seed, E=16, H=512, I=256, K=4):
    from vllm_musa_amd import synthetic
    from vllm_musa_amd.quant_methods import Fp8MoEMethod
    x, w13, s13, w2, s2, w, ids = _case(T, E, H, I, K, seed)
    sw13, ss13, sw2, ss2 = synthetic.moe_fp8_weights(1, H, I, seed + 7)
    gate_w = (torch.randn(H, generator=torch.Generator().manual_seed(seed)) * 0.05).to(DEV)
    layer = SimpleNamespace(w13_weight=w13, w2_weight=w2, w13_weight_scale_inv=s13,
                            w2_weight_scale_inv=s2, expert_map=None, activation="silu",
                            apply_router_weight_on_input=False,
                            moe_config=SimpleNamespace(experts_per_token=K))
    mlp = SimpleNamespace(gate_up_proj=SimpleNamespace(weight=sw13[0], weight_scale_inv=ss13[0]),
                          down_proj=SimpleNamespace(weight=sw2[0], weight_scale_inv=ss2[0]))
    layer._musa_shared_gate = lambda h: ((h.float() @ gate_w).to(torch.bfloat16).view(-1, 1), None)
    method = Fp8MoEMethod()
    method.fold_shared_expert(layer, mlp)
    return method, layer, x, w, ids, (sw13, ss13, sw2, ss2), (w13, s13, w2, s2)


@pytest.mark.parametrize("T,path", [(1, "gemv"), (16, "gemv"), (300, "gemm")])
def test_folded_shared_expert_layer(T, path):
    from vllm_musa_amd import _custom_ops as ops
    method, layer, x, w, ids, shared, routed = _fold_case(T, 100 + T)
    E = routed[0].shape[0]
    assert layer._musa_shared_expert_id == E and layer.w13_weight.shape[0] == E + 1
    out = method.apply(layer, x, w, ids)
    logits, _ = layer._musa_shared_gate(x)
    we, ie = ops.extend_topk_with_shared(w, ids, logits.reshape(-1), E)
    ref = _oracle(x, layer.w13_weight, layer.w13_weight_scale_inv, layer.w2_weight,
                  layer.w2_weight_scale_inv, we, ie)
    _check(out, ref)
    # routed layer + the shared expert as a one-route MoE, without the fold
    routed_out = _run(x, *routed, w, ids, path).float()
    one = torch.zeros(T, 1, dtype=torch.int32, device=DEV)
    shared_out = _run(x, *shared, we[:, -1:].contiguous(), one, path).float()
    sep = (routed_out + shared_out).cpu().numpy().astype(np.float64)
    diff = out.float().cpu().numpy() - sep
    assert np.abs(diff).max() <= 2 ** -7 * np.abs(sep).max()


def test_folded_apply_accepts_router_with_shared_column():
    from vllm_musa_amd import _custom_ops as ops
    method, layer, x, w, ids, _, routed = _fold_case(8, 9)
    logits, _ = layer._musa_shared_gate(x)
    we, ie = ops.extend_topk_with_shared(w, ids, logits.reshape(-1), routed[0].shape[0])
    a = method.apply(layer, x, w, ids)
    b = method.apply(layer, x, we, ie)
    assert torch.equal(a, b)


@pytest.mark.parametrize("kind", ["softmax", "sigmoid"])
@pytest.mark.parametrize("gate_dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("experts,topk,tokens", [(256, 8, 37), (64, 6, 1), (128, 63, 5)])
def test_fused_shared_column_equals_two_launch_composition(kind, gate_dtype, experts, topk, tokens):
    from vllm_musa_amd import _custom_ops as ops
    g = torch.Generator().manual_seed(experts + topk + tokens)
    logits = torch.randn(tokens, experts, generator=g).to(gate_dtype).cuda()
    shared = (torch.randn(tokens, 1, generator=g) * 3).to(gate_dtype).cuda()
    fn = ops.topk_softmax if kind == "softmax" else ops.topk_sigmoid
    w1 = torch.full((tokens, topk + 1), float("nan"), device="cuda")
    i1 = torch.full((tokens, topk + 1), -1, dtype=torch.int32, device="cuda")
    fn(w1, i1, logits, True, shared_expert_gate_output=shared, num_fused_shared_experts=1)
    w0 = torch.empty(tokens, topk, device="cuda")
    i0 = torch.empty(tokens, topk, dtype=torch.int32, device="cuda")
    fn(w0, i0, logits, True)
    w2, i2 = ops.extend_topk_with_shared(w0, i0, shared.reshape(-1), experts)
    assert torch.equal(i1, i2) and torch.equal(w1, w2)
    assert (i1[:, topk] == experts).all()
