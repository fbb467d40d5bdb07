"""Pins of the fused-experts oracle (oracle/moe.py) without re-typing it.

- one expert, top-1, weight 1 reduces to a dense gated MLP computed by torch
  (float64 matmuls, torch's SiLU);
- the routed weight enters once, after W2: scaling every routed weight by 2
  scales the output by exactly 2 (bf16 rounding commutes with x2); applied on
  the input instead, SiLU would break that;
- routes of non-local experts (expert_map -> -1) contribute nothing;
- moe_sum is one rounding of the fp32 slot-order sum;
- the fp8 layer equals the per-route composition of the separately pinned
  pieces (group quantiser, block-fp8 GEMM closed form, SiLU-and-mul).
"""
from __future__ import annotations

import numpy as np
import torch

from oracle import moe as omoe
from oracle import quant as oquant
from oracle.gemm import block_fp8_matmul_f64
from oracle.numerics import bf16_round, e4m3_encode


def _bf16(a):
    return bf16_round(np.asarray(a, np.float32))


def _mlp_case(rng, t=6, h=256, i=128, e=1):
    x = _bf16(rng.standard_normal((t, h)))
    w13 = _bf16(rng.standard_normal((e, 2 * i, h)) * 0.05)
    w2 = _bf16(rng.standard_normal((e, h, i)) * 0.05)
    return x, w13, w2


def test_single_expert_equals_dense_mlp(rng):
    x, w13, w2 = _mlp_case(rng)
    t = x.shape[0]
    ids = np.zeros((t, 1), np.int32)
    w = np.ones((t, 1), np.float32)
    got = omoe.fused_experts_bf16(x, w13, w2, w, ids)
    xt = torch.from_numpy(x).double()
    h = (xt @ torch.from_numpy(w13[0]).double().T).float().bfloat16().float()
    i = w13.shape[1] // 2
    a = (torch.nn.functional.silu(h[:, :i]) * h[:, i:]).bfloat16().float()
    y = (a.double() @ torch.from_numpy(w2[0]).double().T).float().bfloat16().float()
    np.testing.assert_array_equal(got, y.numpy())


def test_routed_weight_enters_after_w2_bf16(rng):
    x, w13, w2 = _mlp_case(rng, t=9, e=4)
    ids = np.stack([rng.permutation(4)[:2] for _ in range(9)]).astype(np.int32)
    w = rng.uniform(0.1, 1.0, (9, 2)).astype(np.float32)
    a = omoe.fused_experts_bf16(x, w13, w2, w, ids)
    b = omoe.fused_experts_bf16(x, w13, w2, 2 * w, ids)
    np.testing.assert_array_equal(b, 2 * a)


def _fp8_case(rng, t=7, h=256, i=256, e=4):
    from oracle.numerics import e4m3_decode
    w13 = rng.integers(0, 256, (e, 2 * i, h)).astype(np.uint8)
    w2 = rng.integers(0, 256, (e, h, i)).astype(np.uint8)
    # drop NaN codes (0x7f / 0xff)
    w13[(w13 & 0x7F) == 0x7F] = 0x38
    w2[(w2 & 0x7F) == 0x7F] = 0x38
    s13 = rng.uniform(0.5, 2, (e, 2 * i // 128, h // 128)).astype(np.float32) / 448 / 64
    s2 = rng.uniform(0.5, 2, (e, h // 128, i // 128)).astype(np.float32) / 448 / 64
    x = _bf16(rng.standard_normal((t, h)))
    assert np.isfinite(e4m3_decode(w13)).all()
    return x, w13, s13, w2, s2


def test_routed_weight_enters_after_w2_fp8(rng):
    x, w13, s13, w2, s2 = _fp8_case(rng)
    ids = np.stack([rng.permutation(4)[:3] for _ in range(7)]).astype(np.int32)
    w = rng.uniform(0.1, 1.0, (7, 3)).astype(np.float32)
    a = omoe.fused_experts_fp8(x, w13, s13, w2, s2, w, ids)
    b = omoe.fused_experts_fp8(x, w13, s13, w2, s2, 2 * w, ids)
    np.testing.assert_array_equal(b, 2 * a)


def test_expert_map_drops_non_local_routes(rng):
    x, w13, w2 = _mlp_case(rng, t=8, e=4)
    gids = np.stack([rng.permutation(8)[:3] for _ in range(8)]).astype(np.int32)
    w = rng.uniform(0.1, 1.0, (8, 3)).astype(np.float32)
    emap = np.array([-1, -1, -1, -1, 0, 1, 2, 3], np.int32)  # globals 4..7 are local 0..3
    got = omoe.fused_experts_bf16(x, w13, w2, w, gids, expert_map=emap)
    # same layer on local ids with the non-local routes' weights set to 0
    loc = np.where(gids >= 4, gids - 4, 0).astype(np.int32)
    w0 = np.where(gids >= 4, w, 0).astype(np.float32)
    np.testing.assert_array_equal(got, omoe.fused_experts_bf16(x, w13, w2, w0, loc))


def test_moe_sum_is_one_rounding(rng):
    # values k * 2^-8 with |k| < 2^12: fp32 sums of 8 of them are exact
    y = (rng.integers(-4096, 4096, (5, 8, 64)) / 256.0).astype(np.float32)
    exact = y.astype(np.float64).sum(axis=1)
    np.testing.assert_array_equal(omoe.moe_sum(y), _bf16(exact.astype(np.float32)))


def test_fp8_layer_is_the_composition_of_pinned_pieces(rng):
    x, w13, s13, w2, s2 = _fp8_case(rng, t=5)
    t, k = 5, 2
    ids = np.stack([rng.permutation(4)[:k] for _ in range(t)]).astype(np.int32)
    w = rng.uniform(0.1, 1.0, (t, k)).astype(np.float32)
    got = omoe.fused_experts_fp8(x, w13, s13, w2, s2, w, ids)
    xq, xs = oquant.group_quant_fp8(x)
    y = np.zeros((t, k, x.shape[1]), np.float32)
    for tt in range(t):
        for kk in range(k):
            e = ids[tt, kk]
            hh = _bf16(block_fp8_matmul_f64(xq[tt:tt + 1], xs[tt:tt + 1], w13[e], s13[e])
                       .astype(np.float32))
            a = oquant.silu_and_mul(hh, "bf16")
            aq, as_ = oquant.group_quant_fp8(a)
            acc = block_fp8_matmul_f64(aq, as_, w2[e], s2[e]).astype(np.float32)
            y[tt, kk] = _bf16(acc * w[tt, kk])[0]
    ref = omoe.moe_sum(y)
    # the two float64 contraction orders may differ in the last bits before
    # the bf16 rounding: allow a rare 1-ulp flip
    diff = np.abs(got - ref)
    ulp = np.abs(ref) * 2.0 ** -7 + 1e-30
    assert (diff <= ulp).all()
    assert (diff == 0).mean() > 0.99


def test_fp8_codes_used_by_the_oracle_are_exact(rng):
    # e4m3 encode of decoded codes is the identity (the layer's weights are codes)
    from oracle.numerics import e4m3_decode
    codes = np.array([c for c in range(256) if (c & 0x7F) != 0x7F], np.uint8)
    np.testing.assert_array_equal(e4m3_encode(e4m3_decode(codes)), codes)


def test_weight_on_input_equals_scaling_x_bf16(rng):
    """apply_router_weight_on_input with a power-of-two routed weight equals the
    default layer on x scaled by that weight with weight 1: the weight enters
    once, on the W13 side, before the SiLU.  On the W2 side instead (or twice)
    the SiLU would break the equality."""
    x, w13, w2 = _mlp_case(rng, t=9, e=4)
    ids = rng.integers(0, 4, (9, 1)).astype(np.int32)
    half = np.full((9, 1), 0.5, np.float32)
    got = omoe.fused_experts_bf16(x, w13, w2, half, ids, apply_router_weight_on_input=True)
    ref = omoe.fused_experts_bf16(x * np.float32(0.5), w13, w2, np.ones((9, 1), np.float32), ids)
    np.testing.assert_array_equal(got, ref)
    assert not np.array_equal(got, omoe.fused_experts_bf16(x, w13, w2, half, ids))


def test_weight_on_input_equals_scaling_x_fp8(rng):
    # halving x halves every 1x128 scale exactly and keeps the codes
    x, w13, s13, w2, s2 = _fp8_case(rng)
    ids = rng.integers(0, 4, (7, 1)).astype(np.int32)
    quarter = np.full((7, 1), 0.25, np.float32)
    got = omoe.fused_experts_fp8(x, w13, s13, w2, s2, quarter, ids,
                                 apply_router_weight_on_input=True)
    ref = omoe.fused_experts_fp8(x * np.float32(0.25), w13, s13, w2, s2,
                                 np.ones((7, 1), np.float32), ids)
    np.testing.assert_array_equal(got, ref)


def test_weight_on_input_unit_weights_match_default(rng):
    x, w13, s13, w2, s2 = _fp8_case(rng)
    ids = np.stack([rng.permutation(4)[:2] for _ in range(7)]).astype(np.int32)
    ones = np.ones((7, 2), np.float32)
    np.testing.assert_array_equal(
        omoe.fused_experts_fp8(x, w13, s13, w2, s2, ones, ids, apply_router_weight_on_input=True),
        omoe.fused_experts_fp8(x, w13, s13, w2, s2, ones, ids))
