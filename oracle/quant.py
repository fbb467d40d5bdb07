"""1x128 activation quantisation and the SiLU-and-mul activation (numpy).

References:
  per_token_group_quant_8bit_vec  csrc/musa/quantization/per_token_group_quant_8bit_vec.cu:65-95
      absmax starts at eps (fmaxf ignores NaN), s = absmax / fp8_max,
      q = fp8(fminf(fmaxf(x / s, fp8_min), fp8_max)) with IEEE division.
  silu_and_mul(+quant)            csrc/musa/quantization/silu_and_mul_per_token_group_fp8_quant.cu:63-127
      value = round_T(silu(g) * u), silu(g) = g / (1 + exp(-g)); clamp variant
      rounds sigmoid, silu and product to T and sends NaN / -inf gates and NaN
      ups to fp8_min.
"""
from __future__ import annotations

import numpy as np

from .numerics import E4M3_MAX, bf16_round, e4m3_encode, f16_round

GROUP = 128


def group_quant_fp8(x: np.ndarray, group: int = GROUP, eps: float = 1e-10,
                    qmin: float = -E4M3_MAX, qmax: float = E4M3_MAX):
    """x [..., K] float32 -> (q uint8 [..., K], s float32 [..., K/group])."""
    x = np.asarray(x, dtype=np.float32)
    *lead, k = x.shape
    assert k % group == 0
    xg = x.reshape(*lead, k // group, group)
    amax = np.fmax.reduce(np.abs(xg), axis=-1, initial=np.float32(eps))  # NaN-ignoring
    amax = np.fmax(amax, np.float32(eps)).astype(np.float32)
    s = (amax / np.float32(qmax)).astype(np.float32)
    v = (xg / s[..., None]).astype(np.float32)
    v = np.fmin(np.fmax(v, np.float32(qmin)), np.float32(qmax))
    q = e4m3_encode(v).reshape(*lead, k)
    return q, s


def _round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "bf16":
        return bf16_round(x)
    if dtype == "f16":
        return f16_round(x)
    return np.asarray(x, dtype=np.float32)


def silu(g: np.ndarray) -> np.ndarray:
    g = np.asarray(g, dtype=np.float32)
    with np.errstate(over="ignore"):
        return (g / (np.float32(1.0) + np.exp(-g))).astype(np.float32)


def silu_and_mul(x: np.ndarray, dtype: str = "bf16") -> np.ndarray:
    """x [..., 2d] -> round_dtype(silu(x[..., :d]) * x[..., d:]) as float32."""
    x = np.asarray(x, dtype=np.float32)
    d = x.shape[-1] // 2
    return _round_to(silu(x[..., :d]) * x[..., d:], dtype)


def silu_and_mul_clamped(x: np.ndarray, limit: float, dtype: str = "bf16"):
    """Clamp variant: returns (values, to_min mask)."""
    x = np.asarray(x, dtype=np.float32)
    d = x.shape[-1] // 2
    g, u = x[..., :d].copy(), x[..., d:].copy()
    to_min = np.isnan(g) | (g == -np.inf) | np.isnan(u)
    lim = _round_to(np.float32(limit), dtype)
    with np.errstate(invalid="ignore"):
        g = np.where(g > lim, lim, g)
        u = np.where(u < -lim, -lim, np.where(u > lim, lim, u))
    with np.errstate(over="ignore"):
        sig = _round_to(np.float32(1.0) / (np.float32(1.0) + np.exp(-g)), dtype)
    with np.errstate(invalid="ignore"):
        s = _round_to(g * sig, dtype)
        return _round_to(s * u, dtype), to_min


def silu_and_mul_quant_fp8(x: np.ndarray, dtype: str = "bf16", limit: float | None = None,
                           eps: float = 1e-10):
    """SiLU-and-mul then the 1x128 quantiser -> (q, s)."""
    if limit is None:
        v = silu_and_mul(x, dtype)
        return group_quant_fp8(v, eps=eps)
    v, to_min = silu_and_mul_clamped(x, limit, dtype)
    # Poisoned entries are NaN here, so the NaN-ignoring absmax skips them and
    # fmax(NaN, fp8_min) sends them to fp8_min, as in the reference.
    q, s = group_quant_fp8(np.where(to_min, np.float32(np.nan), v), eps=eps)
    return q, s
