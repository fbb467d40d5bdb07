"""w4afp8 fused MoE (numpy, float64 contractions).

Reference: vllm_musa/kernels/w4afp8_moe.py:164-362 (w4afp8_moe) and its own
torch oracle tests/kernels/test_w4afp8_moe.py:18-56:

  int4 weights, two per byte, element 2j in the low nibble of byte j
  (_pack_int4, test file 18-22), signed 4-bit; W[n, k] = int4 * s[n, k // 128]
  with bf16 scales [E, N, K/128];
  activations quantised per row: s = max(absmax(row), 1e-4) / 448,
  q = e4m3(clamp(x / s, -448, 448)) (_scatter_quantized_rows 71-72,
  _dynamic_fp8 test 25-28);
  h = bf16(dequant(q) @ W13[e]^T); gate, up = h[:I], h[I:];
  a = bf16(silu(min(gate, L)) * clamp(up, -L, L)) (one rounding; no clamp
  without a limit; _swiglu_quantized_rows 110-126);
  y = bf16(dequant(q_row(a)) @ W2[e]^T);
  out[t] = bf16(sum_k y[t, k] * w[t, k]) with a float32 accumulator in slot
  order, one fused multiply-add per slot (_combine_expert_rows 145-161).
Routes whose expert maps to a negative local id contribute nothing.
"""
from __future__ import annotations

import numpy as np

from .numerics import E4M3_MAX, bf16_round, e4m3_decode, e4m3_encode
from .quant import silu

W4_EPS = 1e-4


def unpack_int4(packed: np.ndarray) -> np.ndarray:
    """int8 [..., K/2] -> int8 [..., K] signed values (even index = low nibble)."""
    b = np.asarray(packed).astype(np.uint8)
    lo = (b & 0xF).astype(np.int16)
    hi = (b >> 4).astype(np.int16)
    out = np.empty(b.shape[:-1] + (2 * b.shape[-1],), np.int8)
    out[..., 0::2] = np.where(lo >= 8, lo - 16, lo)
    out[..., 1::2] = np.where(hi >= 8, hi - 16, hi)
    return out


def pack_int4(values: np.ndarray) -> np.ndarray:
    """int values in [-8, 7] (last dim even) -> int8 with element 2j in the low nibble."""
    v = np.asarray(values).astype(np.int16)
    return ((v[..., 0::2] & 15) | ((v[..., 1::2] & 15) << 4)).astype(np.uint8).view(np.int8)


def dynamic_fp8_rows(x: np.ndarray, eps: float = W4_EPS):
    """x [rows, K] float32 -> (codes uint8 [rows, K], scales float32 [rows])."""
    x = np.asarray(x, np.float32)
    amax = np.fmax.reduce(np.abs(x), axis=-1, initial=np.float32(0.0))
    s = (np.fmax(amax, np.float32(eps)) / np.float32(E4M3_MAX)).astype(np.float32)
    v = (x / s[..., None]).astype(np.float32)
    v = np.fmin(np.fmax(v, np.float32(-E4M3_MAX)), np.float32(E4M3_MAX))
    return e4m3_encode(v), s


def dequant_w4(packed: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """[N, K/2] int8 + [N, K/128] scale values -> float64 [N, K]."""
    w = unpack_int4(packed).astype(np.float64)
    return w * np.repeat(np.asarray(scales, np.float64), 128, axis=-1)[..., :w.shape[-1]]


def swiglu_w4(h: np.ndarray, limit: float | None) -> np.ndarray:
    h = np.asarray(h, np.float32)
    i = h.shape[-1] // 2
    g, u = h[..., :i], h[..., i:]
    if limit is not None and limit > 0:
        g = np.fmin(g, np.float32(limit))
        u = np.fmax(np.fmin(u, np.float32(limit)), np.float32(-limit))
    return bf16_round((silu(g) * u).astype(np.float32))


def w4afp8_moe(x, w13, w2, w13_scale, w2_scale, topk_weights, topk_ids, expert_map=None,
               swiglu_limit=None, return_h=False):
    """x [T, H] (bf16 values); w13 [E, 2I, H/2] int8; w2 [E, H, I/2] int8;
    scales [E, 2I, H/128], [E, H, I/128] (bf16 values as float32)."""
    x = np.asarray(x, np.float32)
    t, h = x.shape
    e_cnt = w13.shape[0]
    ids = np.asarray(topk_ids).astype(np.int64)
    if expert_map is not None:
        em = np.asarray(expert_map).astype(np.int64)
        loc = np.where((ids >= 0) & (ids < em.size), em[np.clip(ids, 0, em.size - 1)], -1)
    else:
        loc = ids
    loc = np.where((loc >= 0) & (loc < e_cnt), loc, -1)
    w = np.asarray(topk_weights, np.float32)
    xq, xs = dynamic_fp8_rows(x)
    xd = e4m3_decode(xq).astype(np.float64) * xs.astype(np.float64)[:, None]
    y = np.zeros((t, ids.shape[1], h), np.float32)
    hs = {}
    for e in np.unique(loc[loc >= 0]):
        tt, kk = np.nonzero(loc == e)
        hh = bf16_round((xd[tt] @ dequant_w4(w13[e], w13_scale[e]).T).astype(np.float32))
        if return_h:
            hs[int(e)] = (tt, kk, hh)
        a = swiglu_w4(hh, swiglu_limit)
        aq, as_ = dynamic_fp8_rows(a)
        ad = e4m3_decode(aq).astype(np.float64) * as_.astype(np.float64)[:, None]
        y[tt, kk] = bf16_round((ad @ dequant_w4(w2[e], w2_scale[e]).T).astype(np.float32))
    out = bf16_round(weighted_sum_fma(y, w, loc >= 0))
    return (out, hs) if return_h else out


def weighted_sum_fma(y: np.ndarray, w: np.ndarray, live: np.ndarray | None = None) -> np.ndarray:
    """sum_k y[:, k] * w[:, k] in slot order, each step a float32 fused
    multiply-add (the combine's `acc += values * weight`, which compiles to an
    FMA): the float32 x float32 product is exact in float64, so adding in
    float64 and rounding once to float32 is the FMA (barring a float64 sum that
    lands exactly on a float32 halfway point)."""
    y = np.asarray(y, np.float32)
    w = np.asarray(w, np.float32)
    acc = np.zeros(y.shape[::2], np.float32)
    for k in range(y.shape[1]):
        prod = y[:, k].astype(np.float64) * w[:, k:k + 1].astype(np.float64)
        if live is not None:
            prod = np.where(live[:, k:k + 1], prod, 0.0)
        acc = (acc.astype(np.float64) + prod).astype(np.float32)
    return acc
