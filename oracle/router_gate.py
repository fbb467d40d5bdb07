"""fp32 router-gate GEMM with its fixed summation order (TEST INFRASTRUCTURE
ONLY: the checker of vmamd_router_gate_fp32).

The reference computes the Nemotron-H router logits x[M, 2688] . W[128, 2688]^T
in plain fp32 FMA arithmetic and requires them to be bitwise reproducible, so
the router's top-k cannot move
(vllm_musa/model_executor/layers/fused_moe/router/musa_router_gemm.py:140-185,
tests/test_musa_router_gemm.py:131-167).  The order restated here is the one
this package's kernel fixes for every logit:

  lane l in 0..63 owns k = 2l + 128 i + j for i = 0..K/128-1, j = 0, 1, and
  p_l = fma(x[k], w[k], p_l) over those k in that order, starting at +0;
  then p_l <- p_l + p_{l xor s} for s = 32, 16, 8, 4, 2, 1; the logit is p_0.

fmaf is emulated exactly: the float64 product of two float32 values is exact,
TwoSum gives the exact error of the float64 sum, the sum is rounded to odd at
53 bits and then to nearest-even at 24 bits, which is the correctly rounded
fused result (round-to-odd double rounding, Boldo & Melquiond 2008).  Pinned
in tests/test_oracle_router_gate.py against the C library's fmaf and a scalar
restatement, and against the exact (float64) dot product within its error
bound.
"""
from __future__ import annotations

import numpy as np

LANES = 64


def fmaf(a, b, c) -> np.ndarray:
    """Correctly rounded float32 a * b + c, element-wise."""
    a64 = np.asarray(a, np.float32).astype(np.float64)
    b64 = np.asarray(b, np.float32).astype(np.float64)
    c64 = np.asarray(c, np.float32).astype(np.float64)
    p = a64 * b64                                   # exact: 48 significant bits
    s = p + c64
    bp = s - c64
    err = (p - bp) + (c64 - (s - bp))               # s + err == p + c exactly
    inexact = err != 0
    # truncate toward zero, then force the last bit to 1 when inexact
    over = inexact & (np.signbit(err) != np.signbit(s))
    t = np.where(over, np.nextafter(s, 0.0), s)
    bits = t.view(np.uint64)
    bits = np.where(inexact, bits | np.uint64(1), bits)
    with np.errstate(over="ignore"):           # overflow to +-inf is IEEE's answer
        return bits.view(np.float64).astype(np.float32)


def lane_order(K: int) -> np.ndarray:
    """[64, K/64] k indices each lane visits, in chain order."""
    if K % 128:
        raise ValueError("K must be a multiple of 128")
    i = np.arange(K // 128)
    lane = np.arange(LANES)
    k = 2 * lane[:, None, None] + 128 * i[None, :, None] + np.arange(2)[None, None, :]
    return k.reshape(LANES, -1)


def router_gate_fp32(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    """x [M, K] (float32 values; bf16 inputs already widened), w [E, K] float32
    -> logits [M, E] float32 in the fixed order above."""
    x = np.asarray(x, np.float32)
    w = np.asarray(w, np.float32)
    M, K = x.shape
    E = w.shape[0]
    order = lane_order(K)                            # [64, S]
    acc = np.zeros((M, E, LANES), np.float32)
    for step in range(order.shape[1]):
        k = order[:, step]
        acc = fmaf(x[:, None, k], w[None, :, k], acc)
    lane = np.arange(LANES)
    for s in (32, 16, 8, 4, 2, 1):
        acc = (acc + acc[..., lane ^ s]).astype(np.float32)
    return acc[..., 0]


__all__ = ["fmaf", "lane_order", "router_gate_fp32", "LANES"]
