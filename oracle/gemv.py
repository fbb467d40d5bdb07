"""The reference's native GEMV ops, W8A16 numerics (numpy, float64 contractions).

Restates ``musa_gemv_kernel`` and its two host entries
(vllm_musa csrc/musa/gemv.mu:249-514, 723-925, 927-1170) as the reference's
fused-MoE driver calls them (model_executor/layers/fused_moe/fused_moe.py:
2126-2184) and as its small-M dense path calls them
(model_executor/kernels/linear/scaled_mm/deep_gemm.py:512-536):

  route r = row * topk + k over A's rows (gemv.mu:293-296: grid z = rows,
  grid y = topk), expert e = topk_ids.flat[r]; an id outside [0, E) writes a
  zero output row (gemv.mu:297-311).

  acc[n] = sum_kb s_w[e, n // 128, kb] * sum_{k in kb} a[row, k] * w[e, n, k]
      bf16 activations against fp8 weights (the fused cast, gemv.mu:405-419):
      the activation is NOT quantised; the e4m3 weight value is exact in the
      product.  fp8 activations with A_scale multiply s_a[row, kb] in as well
      (gemv.mu:420-427); bf16 weights take no scales (gemv.mu:430-434).
  acc *= topk_weights.flat[r]            when mul_routed_weight (gemv.mu:472-475)
  SwiGLU (use_swigelu): rows [0, N/2) are the gate, [N/2, N) the up
      projection (gemv.mu:322-327); with L = swiglu_limit > 0 the gate is
      clamped to <= L and up to [-L, L]; out = g * sigmoid(g) * u, all in fp32
      from the fp32 sums (gemv.mu:477-487).  L is first rounded to the
      activation dtype (gemv.mu:946-951).
  out = bf16(value)                       (C is bf16, gemv.mu:487, 512)

The fused layer (fused_moe.py:2148-2184): W13 with mul_routed_weight =
apply_router_weight_on_input and SwiGLU into cache2 [T*K, I]; W2 with
topk = 1 over cache2's rows and mul_routed_weight = not
apply_router_weight_on_input into cache3 [T, K, H]; then moe_sum (fp32 sum in
slot order, one rounding).  T is processed in chunks of 16384 tokens
(fused_moe.py:2126-2128), which does not change any value.

The reference sums a K-block in its own thread order; float64 here is the
exact value up to the final fp32 products, well inside the path's tolerance.
"""
from __future__ import annotations

import numpy as np

from .moe import moe_sum
from .numerics import bf16_round, e4m3_decode


def _sigmoid(x: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        return 1.0 / (1.0 + np.exp(-x))


def round_limit(limit: float, act_dtype: str = "bf16") -> float:
    """swiglu_limit in the activation dtype (gemv.mu:946-951); fp8
    activations keep the float value."""
    if act_dtype == "bf16":
        return float(bf16_round(np.asarray([limit], np.float32))[0])
    return float(np.float32(limit))


def weight_values(b, b_scale=None, block: int = 128) -> np.ndarray:
    """Weights [..., N, K] as float64 values: e4m3 codes (uint8) times their
    [..., ceil(N/128), K/128] block scales, or bf16 values passed through."""
    b = np.asarray(b)
    if b.dtype == np.uint8:
        w = e4m3_decode(b).astype(np.float64)
        n, k = w.shape[-2:]
        s = np.asarray(b_scale, np.float64)
        s = np.repeat(np.repeat(s, block, axis=-2)[..., :n, :], block, axis=-1)[..., :k]
        return w * s
    if b_scale is not None:
        raise ValueError("bf16 weights take no scales")
    return b.astype(np.float64)


def act_values(a, a_scale=None, block: int = 128) -> tuple[np.ndarray, str]:
    """Activation rows as float64 values and their dtype tag: bf16 values as
    given, or e4m3 codes (uint8) times their [rows, K/128] group scales."""
    a = np.asarray(a)
    if a.dtype == np.uint8:
        v = e4m3_decode(a).astype(np.float64)
        return v * np.repeat(np.asarray(a_scale, np.float64), block, axis=-1)[:, :v.shape[1]], "fp8"
    return a.astype(np.float64), "bf16"


def fused_gemv_moe(a, b, topk_weights, topk_ids, mul_routed_weight: bool, topk: int,
                   use_swiglu: bool, swiglu_limit: float = 0.0, a_scale=None, b_scale=None
                   ) -> np.ndarray:
    """musa_fused_gemv_moe: A [rows, K], B [E, N, K] -> C [rows * topk, N or N/2]
    as bf16 values (float32).  topk_ids / topk_weights hold rows * topk entries
    (route r = row * topk + k).  One expert's weights are dequantised at a
    time."""
    av, adt = act_values(a, a_scale)
    b = np.asarray(b)
    rows, _ = av.shape
    e_cnt, n, _ = b.shape
    ids = np.asarray(topk_ids).reshape(-1).astype(np.int64)
    wts = np.asarray(topk_weights, np.float32).reshape(-1)
    if ids.size != rows * topk:
        raise ValueError("topk_ids must hold rows * topk entries")
    n_out = n // 2 if use_swiglu else n
    out = np.zeros((rows * topk, n_out), dtype=np.float32)
    lim = round_limit(swiglu_limit, adt) if swiglu_limit > 0 else 0.0
    live = (ids >= 0) & (ids < e_cnt)   # other ids leave a zero row
    for e in np.unique(ids[live]):
        routes = np.nonzero(ids == e)[0]
        we = weight_values(b[e], None if b_scale is None else np.asarray(b_scale)[e])
        acc = (av[routes // topk] @ we.T).astype(np.float32)
        if mul_routed_weight:
            acc = (acc * wts[routes][:, None]).astype(np.float32)
        if use_swiglu:
            g = acc[:, : n // 2].astype(np.float64)
            u = acc[:, n // 2:].astype(np.float64)
            if lim > 0:
                g = np.minimum(g, lim)
                u = np.clip(u, -lim, lim)
            v = (g * _sigmoid(g) * u).astype(np.float32)
        else:
            v = acc
        out[routes] = bf16_round(v)
    return out


def fused_gemv(x, qweight, use_swiglu: bool = False, x_scale=None, qweight_scale=None
               ) -> np.ndarray:
    """musa_fused_gemv (gemv.mu:723-925 with the fused-cast branch): one expert,
    every row its own route with weight 1: x [M, K], qweight [N, K] ->
    [M, N or N/2] bf16 values."""
    qw = np.asarray(qweight)[None]
    qs = None if qweight_scale is None else np.asarray(qweight_scale)[None]
    m = np.asarray(x).shape[0]
    ids = np.zeros((m, 1), np.int32)
    return fused_gemv_moe(x, qw, np.ones((m, 1), np.float32), ids, False, 1, use_swiglu,
                          a_scale=x_scale, b_scale=qs)


def fused_experts_w8a16(x, w13, w2, topk_weights, topk_ids, w13_scale=None, w2_scale=None,
                        apply_router_weight_on_input: bool = False, swiglu_limit: float = 0.0,
                        expert_map=None, return_y: bool = False):
    """The reference's GEMV-MoE layer (fused_moe.py:2126-2184): bf16 x [T, H];
    w13 [E, 2I, H] / w2 [E, H, I] as e4m3 codes with block scales, or bf16
    values without.  expert_map (global -> local, -1 = not here) is applied to
    the ids first; routes without a local expert contribute nothing."""
    t = np.asarray(x).shape[0]
    k = np.asarray(topk_ids).shape[1]
    ids = np.asarray(topk_ids).astype(np.int64)
    if expert_map is not None:
        em = np.asarray(expert_map).astype(np.int64)
        ids = np.where((ids >= 0) & (ids < em.size), em[np.clip(ids, 0, em.size - 1)], -1)
    cache2 = fused_gemv_moe(x, w13, topk_weights, ids, apply_router_weight_on_input, k, True,
                            swiglu_limit, b_scale=w13_scale)
    cache3 = fused_gemv_moe(cache2, w2, topk_weights, ids.reshape(-1, 1),
                            not apply_router_weight_on_input, 1, False, b_scale=w2_scale)
    y = cache3.reshape(t, k, -1)
    out = moe_sum(y)
    return (out, y) if return_y else out


__all__ = ["act_values", "fused_experts_w8a16", "fused_gemv", "fused_gemv_moe", "round_limit",
           "weight_values"]
