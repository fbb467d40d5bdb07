"""Pins oracle/router_gate.py: the exact fmaf emulation against the C
library's fmaf (random and cancellation-heavy cases), the summation order
against a scalar restatement built on that fmaf, and the logits against the
exact (float64) dot product within the fp32 error bound.  Two plausible slips
(an unfused chain, a reversed butterfly) change the bits on random data, so the
bit-exact GPU test would see them."""
from __future__ import annotations

import ctypes
import ctypes.util

import numpy as np
import pytest

from oracle import router_gate as org

_libm = ctypes.CDLL(ctypes.util.find_library("m") or "libm.so.6")
_libm.fmaf.restype = ctypes.c_float
_libm.fmaf.argtypes = [ctypes.c_float] * 3


def _c_fmaf(a, b, c) -> np.ndarray:
    return np.array([_libm.fmaf(float(x), float(y), float(z)) for x, y, z in zip(a, b, c)],
                    np.float32)


def _bits(v):
    return np.asarray(v, np.float32).view(np.uint32)


def test_fmaf_matches_libm_random():
    rng = np.random.default_rng(1)
    n = 30000
    a, b, c = (rng.standard_normal(n).astype(np.float32)
               * np.float32(2.0) ** rng.integers(-30, 30, n).astype(np.float32) for _ in range(3))
    assert np.array_equal(_bits(org.fmaf(a, b, c)), _bits(_c_fmaf(a, b, c)))


def test_fmaf_matches_libm_cancellation_and_signs():
    rng = np.random.default_rng(2)
    n = 20000
    a = rng.standard_normal(n).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    prod = (a * b).astype(np.float32)                       # rounded product
    jitter = rng.integers(-3, 4, n).astype(np.int32)
    c = -(prod.view(np.int32) + jitter).view(np.float32)    # c ~ -a*b: the result is the tiny error
    extra = np.array([0.0, -0.0, 1e-45, -1e-45, 3.4e38], np.float32)
    a = np.concatenate([a, extra, extra])
    b = np.concatenate([b, extra[::-1], -extra])
    c = np.concatenate([c, -extra, extra])
    got, ref = org.fmaf(a, b, c), _c_fmaf(a, b, c)
    assert np.array_equal(_bits(got), _bits(ref))
    # the non-fused result differs on these inputs (the test has power)
    with np.errstate(over="ignore"):
        unfused = (a * b).astype(np.float32) + c
    assert not np.array_equal(_bits(unfused), _bits(ref))


def _scalar_router(x, w):
    """The order restated with scalar C fmaf calls."""
    M, K = x.shape
    E = w.shape[0]
    out = np.zeros((M, E), np.float32)
    for m in range(M):
        for e in range(E):
            p = []
            for lane in range(64):
                acc = 0.0
                for i in range(K // 128):
                    for j in (0, 1):
                        k = 2 * lane + 128 * i + j
                        acc = _libm.fmaf(float(x[m, k]), float(w[e, k]), acc)
                p.append(np.float32(acc))
            for s in (32, 16, 8, 4, 2, 1):
                p = [np.float32(p[l] + p[l ^ s]) for l in range(64)]
            out[m, e] = p[0]
    return out


def test_order_matches_scalar_restatement():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((2, 256)).astype(np.float32)
    w = rng.standard_normal((3, 256)).astype(np.float32)
    assert np.array_equal(_bits(org.router_gate_fp32(x, w)), _bits(_scalar_router(x, w)))


@pytest.mark.parametrize("K", [128, 2688, 7168])
def test_logits_within_fp32_error_bound(K):
    rng = np.random.default_rng(K)
    x = rng.standard_normal((5, K)).astype(np.float32)
    w = rng.standard_normal((16, K)).astype(np.float32)
    got = org.router_gate_fp32(x, w).astype(np.float64)
    exact = x.astype(np.float64) @ w.T.astype(np.float64)
    depth = K // 64 + 6                       # chain length + butterfly levels
    bound = depth * 2.0 ** -24 * (np.abs(x).astype(np.float64) @ np.abs(w).T.astype(np.float64))
    assert (np.abs(got - exact) <= bound).all()


def test_lane_order_covers_k_once():
    order = org.lane_order(2688)
    assert order.shape == (64, 42)
    assert np.array_equal(np.sort(order.ravel()), np.arange(2688))
    assert (order[:, 1:] > order[:, :-1]).all()
    with pytest.raises(ValueError):
        org.lane_order(2700)


def test_plausible_slips_change_bits():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((3, 2688)).astype(np.float32)
    w = rng.standard_normal((8, 2688)).astype(np.float32)
    good = org.router_gate_fp32(x, w)
    # reversed butterfly
    order = org.lane_order(2688)
    acc = np.zeros((3, 8, 64), np.float32)
    for s in range(order.shape[1]):
        k = order[:, s]
        acc = org.fmaf(x[:, None, k], w[None, :, k], acc)
    lane = np.arange(64)
    rev = acc.copy()
    for s in (1, 2, 4, 8, 16, 32):
        rev = (rev + rev[..., lane ^ s]).astype(np.float32)
    assert not np.array_equal(_bits(rev[..., 0]), _bits(good))
    # unfused chain
    acc = np.zeros((3, 8, 64), np.float32)
    for s in range(order.shape[1]):
        k = order[:, s]
        acc = (acc + (x[:, None, k] * w[None, :, k]).astype(np.float32)).astype(np.float32)
    for s in (32, 16, 8, 4, 2, 1):
        acc = (acc + acc[..., lane ^ s]).astype(np.float32)
    assert not np.array_equal(_bits(acc[..., 0]), _bits(good))
