"""Pins of oracle/gemv.py (the reference's native GEMV ops, W8A16 numerics).

Each check would fail for a plausible slip: torch float64 matmuls on weights
dequantised through torch's own float8 cast (a transposed operand, a wrong
scale block, an activation that was quantised), torch's SiLU on hand-built
gate / up halves (the halves swapped, the routed weight applied after the
activation instead of before), the bf16 rounding of the clamp limit, power-of-
two linearity of the routed weight, dead routes, and the whole layer restated
token by token in torch."""
from __future__ import annotations

import numpy as np
import torch

from oracle import gemv as ogemv
from oracle import moe as omoe
from oracle.numerics import bf16_round, e4m3_encode


def _bf16(a) -> np.ndarray:
    return bf16_round(np.asarray(a, np.float32))


def _torch_dequant(codes: np.ndarray, scales: np.ndarray) -> torch.Tensor:
    """[N, K] e4m3 codes and [N/128, K/128] scales -> float64, via torch's cast."""
    w = torch.from_numpy(codes.copy()).view(torch.float8_e4m3fn).to(torch.float64)
    s = torch.from_numpy(np.asarray(scales, np.float64))
    s = s.repeat_interleave(128, 0)[: w.shape[0]].repeat_interleave(128, 1)[:, : w.shape[1]]
    return w * s


def _fp8_weights(rng, e, n, k):
    codes = e4m3_encode(np.clip(rng.standard_normal((e, n, k)) * 64, -448, 448).astype(np.float32))
    scales = rng.uniform(0.5, 2.0, (e, -(-n // 128), k // 128)).astype(np.float32) / 448.0
    return codes, scales


def _ulp_close(a: np.ndarray, b: np.ndarray, ulps: int = 1):
    """Equal within `ulps` bf16 units in the last place of the larger value."""
    tol = np.maximum(np.abs(a), np.abs(b)) * 2.0 ** -7 * ulps + 1e-30
    assert (np.abs(a - b) <= tol).all(), np.abs(a - b).max()


def test_one_expert_equals_torch_matmul_on_dequantised_weights(rng):
    codes, scales = _fp8_weights(rng, 1, 256, 384)
    x = _bf16(rng.standard_normal((5, 384)))
    got = ogemv.fused_gemv_moe(x, codes, np.ones((5, 1), np.float32), np.zeros((5, 1), np.int32),
                               False, 1, False, b_scale=scales)
    ref = torch.from_numpy(x.astype(np.float64)) @ _torch_dequant(codes[0], scales[0]).T
    _ulp_close(got, ref.to(torch.float32).to(torch.bfloat16).float().numpy())


def test_activations_are_not_quantised(rng):
    """A bf16 activation that no e4m3 code can hold (1 + 2^-7) enters at its
    own value: the product with a unit weight returns it exactly."""
    x = np.zeros((1, 128), np.float32)
    x[0, 3] = 1.0 + 2.0 ** -7
    codes = np.zeros((1, 16, 128), np.uint8)
    codes[0, :, 3] = e4m3_encode(np.ones(16, np.float32))
    out = ogemv.fused_gemv_moe(x, codes, np.ones((1, 1), np.float32), np.zeros((1, 1), np.int32),
                               False, 1, False, b_scale=np.ones((1, 1, 1), np.float32))
    assert (out == np.float32(1.0 + 2.0 ** -7)).all()


def test_bf16_weights_equal_torch_matmul(rng):
    w = _bf16(rng.standard_normal((3, 32, 128)) * 0.3)
    x = _bf16(rng.standard_normal((4, 128)))
    ids = np.array([[2], [0], [1], [2]], np.int32)
    got = ogemv.fused_gemv_moe(x, w, np.ones((4, 1), np.float32), ids, False, 1, False)
    for r in range(4):
        ref = torch.from_numpy(x[r].astype(np.float64)) @ torch.from_numpy(
            w[ids[r, 0]].astype(np.float64)).T
        _ulp_close(got[r], ref.to(torch.float32).to(torch.bfloat16).float().numpy())


def test_swiglu_gate_first_and_weight_before_the_activation():
    """Rows [0, N/2) are the gate: with a one-hot x, g = [3, -1] and u = [2, 5]
    come straight out of the weight columns; mul_routed_weight scales g and u
    before silu (silu(2g) * 2u, not 2 * silu(g) * u)."""
    n, k = 4, 128
    w = np.zeros((1, n, k), np.float32)
    w[0, :, 0] = [3.0, -1.0, 2.0, 5.0]
    x = np.zeros((1, k), np.float32)
    x[0, 0] = 1.0
    ids = np.zeros((1, 1), np.int32)
    one = ogemv.fused_gemv_moe(x, w, np.ones((1, 1), np.float32), ids, False, 1, True)
    g, u = torch.tensor([3.0, -1.0], dtype=torch.float64), torch.tensor([2.0, 5.0], dtype=torch.float64)
    want = (torch.nn.functional.silu(g) * u).float().to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(one[0], want)
    swapped = (torch.nn.functional.silu(u) * g).float().to(torch.bfloat16).float().numpy()
    assert not np.array_equal(one[0], swapped)
    two = ogemv.fused_gemv_moe(x, w, np.full((1, 1), 2.0, np.float32), ids, True, 1, True)
    want2 = (torch.nn.functional.silu(2 * g) * 2 * u).float().to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(two[0], want2)
    assert not np.array_equal(two[0], _bf16(2 * one[0]))


def test_limit_is_rounded_to_bf16_first():
    """7.03 rounds to 7.03125 in bf16: a gate of 7.1 is clamped to 7.03125.
    The two clamps differ by 1.8e-4 relative, below bf16's resolution, so the
    up value is picked (a scan over bf16 values) to put silu(gate) * up across
    a rounding boundary, where the two limits give different outputs."""
    lim = torch.tensor(7.03, dtype=torch.bfloat16).double()
    assert float(lim) == 7.03125
    unrounded = torch.tensor(7.03, dtype=torch.float64)

    def act(g, u):
        return (torch.nn.functional.silu(g) * u).float().to(torch.bfloat16).float().item()

    ups = [1.0 + j / 128 for j in range(128)]
    u = next(u for u in ups if act(lim, u) != act(unrounded, u))
    k = 128
    w = np.zeros((1, 2, k), np.float32)
    w[0, :, 0] = [7.1, u]
    x = np.zeros((1, k), np.float32)
    x[0, 0] = 1.0
    out = ogemv.fused_gemv_moe(x, w, np.ones((1, 1), np.float32), np.zeros((1, 1), np.int32),
                               False, 1, True, swiglu_limit=7.03)
    assert out[0, 0] == act(lim, u) != act(unrounded, u)


def test_routed_weight_linearity_and_dead_routes(rng):
    codes, scales = _fp8_weights(rng, 4, 128, 256)
    a = _bf16(rng.standard_normal((6, 256)))
    ids = np.array([0, 3, -1, 2, 4, 1], np.int32).reshape(6, 1)
    w = rng.uniform(0.1, 1.0, (6, 1)).astype(np.float32)
    one = ogemv.fused_gemv_moe(a, codes, w, ids, True, 1, False, b_scale=scales)
    two = ogemv.fused_gemv_moe(a, codes, 2 * w, ids, True, 1, False, b_scale=scales)
    np.testing.assert_array_equal(two, 2 * one)
    assert not one[2].any() and not one[4].any()   # id -1 and id == E
    assert one[[0, 1, 3, 5]].any(axis=1).all()


def test_dense_gemv_is_the_one_expert_case(rng):
    codes, scales = _fp8_weights(rng, 1, 256, 512)
    x = _bf16(rng.standard_normal((3, 512)))
    dense = ogemv.fused_gemv(x, codes[0], False, qweight_scale=scales[0])
    moe = ogemv.fused_gemv_moe(x, codes, np.ones((3, 1), np.float32), np.zeros((3, 1), np.int32),
                               False, 1, False, b_scale=scales)
    np.testing.assert_array_equal(dense, moe)


def test_fp8_activation_branch_carries_both_scales(rng):
    codes, scales = _fp8_weights(rng, 1, 128, 256)
    aq = e4m3_encode(np.clip(rng.standard_normal((2, 256)) * 100, -448, 448).astype(np.float32))
    asc = rng.uniform(0.001, 0.01, (2, 2)).astype(np.float32)
    got = ogemv.fused_gemv_moe(aq, codes, np.ones((2, 1), np.float32), np.zeros((2, 1), np.int32),
                               False, 1, False, a_scale=asc, b_scale=scales)
    a = torch.from_numpy(aq.copy()).view(torch.float8_e4m3fn).double() * torch.from_numpy(
        asc.astype(np.float64)).repeat_interleave(128, 1)
    ref = a @ _torch_dequant(codes[0], scales[0]).T
    _ulp_close(got, ref.float().to(torch.bfloat16).float().numpy())


def test_layer_restated_token_by_token_in_torch(rng):
    """fused_experts_w8a16 against the reference's driver written per token
    and slot with torch ops: cache2 = bf16(silu(g) * u) from fp32 sums,
    cache3 = bf16(W2 . cache2 * w), out = bf16(fp32 sum over slots)."""
    e, i, h, t, k = 6, 128, 256, 3, 2
    w13c, w13s = _fp8_weights(rng, e, 2 * i, h)
    w2c, w2s = _fp8_weights(rng, e, h, i)
    w13s *= 0.02
    w2s *= 0.02
    x = _bf16(rng.standard_normal((t, h)))
    ids = np.array([[0, 5], [2, 2], [4, -1]], np.int32)
    wts = rng.uniform(0.2, 0.8, (t, k)).astype(np.float32)
    got = ogemv.fused_experts_w8a16(x, w13c, w2c, wts, ids, w13s, w2s)
    out = torch.zeros(t, h, dtype=torch.float32)
    for tt in range(t):
        for kk in range(k):
            ex = int(ids[tt, kk])
            if ex < 0:
                continue
            hg = (_torch_dequant(w13c[ex], w13s[ex]) @ torch.from_numpy(x[tt].astype(np.float64))
                  ).float()
            a = (torch.nn.functional.silu(hg[:i].double()) * hg[i:].double()).float()
            a = a.to(torch.bfloat16).double()
            y = ((_torch_dequant(w2c[ex], w2s[ex]) @ a).float() * float(wts[tt, kk]))
            out[tt] += y.to(torch.bfloat16).float()
    _ulp_close(got, out.to(torch.bfloat16).float().numpy(), ulps=2)


def test_w8a16_and_w8a8_layers_differ_beyond_rounding(rng):
    """The reason the numerics are chosen per call: on a decode-shaped layer
    the W8A16 layer and the W8A8 layer (x and a2 quantised per 1x128 group)
    differ by far more than bf16 rounding."""
    e, i, h, t, k = 8, 256, 512, 4, 2
    w13c, w13s = _fp8_weights(rng, e, 2 * i, h)
    w2c, w2s = _fp8_weights(rng, e, h, i)
    w13s *= 0.01
    w2s *= 0.01
    x = _bf16(rng.standard_normal((t, h)))
    ids = np.stack([rng.permutation(e)[:k] for _ in range(t)]).astype(np.int32)
    wts = rng.uniform(0.2, 0.8, (t, k)).astype(np.float32)
    a16 = ogemv.fused_experts_w8a16(x, w13c, w2c, wts, ids, w13s, w2s)
    a8 = omoe.fused_experts_fp8(x, w13c, w13s, w2c, w2s, wts, ids)
    rel = np.linalg.norm(a16 - a8) / np.linalg.norm(a16)
    assert rel > 1e-2, rel
