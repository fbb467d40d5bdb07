"""Fused experts and the top-k combine (numpy, float64 contractions).

Rounding points follow the reference's default (upstream Triton) path and its
DeepGEMM prefill path, which agree (Appendix of the path's numerics):
  fused_moe.py:1935-2184 (driver), patches/series/0144-…:62-78 (activation,
  then a2 quantisation), 0081-…:64-108 (block-scaled accumulate), fused_moe.py
  2164-2178 (routed weight applied in the W2 epilogue), moe_sum
  (jit_kernel/csrc/moe/moe_sum_reduce.mu:127-146: fp32 sum in slot order, one
  rounding):

  bf16 weights:   h = bf16(x @ W13[e]^T)
                  a = bf16(silu(h[:I]) * h[I:])
                  y = bf16((a @ W2[e]^T) * w)
  fp8 block:      xq, xs = quant1x128(x)
                  h = bf16(block_gemm(xq, W13[e]))
                  a = bf16(silu(h[:I]) * h[I:]);  aq, as = quant1x128(a)
                  y = bf16(block_gemm(aq, W2[e]) * w)
  combine:        out[t] = bf16(sum_k f32(y[t, k]))   (slot order)

Routes whose expert maps to a negative local id (expert_map) contribute
nothing.  With apply_router_weight_on_input the routed weight multiplies the
W13 output (gate and up, fp32) before its bf16 rounding and y is not weighted:
the reference's native GEMV-MoE driver passes mul_routed_weight =
apply_router_weight_on_input to its first GEMV and the negation to its second
(fused_moe.py:2148-2177; the multiply, csrc/musa/gemv.mu:472-475, precedes the
SwiGLU at 477-487), and upstream's Triton fused_moe_kernel does the same
through MUL_ROUTED_WEIGHT on the first GEMM:

  h = bf16(W13[e] . x * w);  y = bf16(W2[e] . q(act(h)))
"""
from __future__ import annotations

import numpy as np

from .gemm import dequant_block_weight
from .numerics import bf16_round, e4m3_decode
from .quant import group_quant_fp8, silu_and_mul


def local_experts(topk_ids: np.ndarray, expert_map: np.ndarray | None, num_experts: int):
    ids = np.asarray(topk_ids).astype(np.int64)
    if expert_map is None:
        loc = ids
    else:
        em = np.asarray(expert_map).astype(np.int64)
        loc = np.where((ids >= 0) & (ids < em.size), em[np.clip(ids, 0, em.size - 1)], -1)
    return np.where((loc >= 0) & (loc < num_experts), loc, -1)


def moe_sum(y: np.ndarray, dtype: str = "bf16") -> np.ndarray:
    """y [T, K, H] values -> round(sum_k y[:, k]) with a float32 accumulator in slot order."""
    y = np.asarray(y, dtype=np.float32)
    acc = np.zeros(y.shape[::2], dtype=np.float32)
    for k in range(y.shape[1]):
        acc = (acc + y[:, k]).astype(np.float32)
    return bf16_round(acc) if dtype == "bf16" else acc


def fused_experts_bf16(x, w13, w2, topk_weights, topk_ids, expert_map=None,
                       apply_router_weight_on_input=False, return_y=False):
    """x [T,H], w13 [E,2I,H], w2 [E,H,I] (bf16 values as float32)."""
    x = np.asarray(x, np.float32)
    t, h = x.shape
    e_cnt, n2, _ = w13.shape
    k = topk_ids.shape[1]
    loc = local_experts(topk_ids, expert_map, e_cnt)
    w = np.asarray(topk_weights, np.float32)
    y = np.zeros((t, k, h), dtype=np.float32)
    for e in np.unique(loc[loc >= 0]):
        tt, kk = np.nonzero(loc == e)
        hh = (x[tt].astype(np.float64) @ np.asarray(w13[e], np.float64).T).astype(np.float32)
        if apply_router_weight_on_input:
            hh = (hh * w[tt, kk][:, None]).astype(np.float32)
        hh = bf16_round(hh)
        a = silu_and_mul(hh, "bf16")
        acc = (a.astype(np.float64) @ np.asarray(w2[e], np.float64).T).astype(np.float32)
        if not apply_router_weight_on_input:
            acc = (acc * w[tt, kk][:, None]).astype(np.float32)
        y[tt, kk] = bf16_round(acc)
    out = moe_sum(y)
    return (out, y) if return_y else out


def fused_experts_fp8(x, w13_q, w13_s, w2_q, w2_s, topk_weights, topk_ids, expert_map=None,
                      block_shape=(128, 128), apply_router_weight_on_input=False,
                      return_y=False, experts_subset=None):
    """x [T,H] (bf16 values); w13_q [E,2I,H] e4m3 codes, w13_s [E,2I/bn,H/bk];
    w2_q [E,H,I], w2_s [E,H/bn,I/bk].  experts_subset (optional) restricts the
    work to those experts (used to time a bounded sample)."""
    bn, bk = block_shape
    x = np.asarray(x, np.float32)
    t, h = x.shape
    e_cnt = w13_q.shape[0]
    k = topk_ids.shape[1]
    loc = local_experts(topk_ids, expert_map, e_cnt)
    w = np.asarray(topk_weights, np.float32)
    xq, xs = group_quant_fp8(x)
    y = np.zeros((t, k, h), dtype=np.float32)
    experts = np.unique(loc[loc >= 0]) if experts_subset is None else experts_subset
    for e in experts:
        tt, kk = np.nonzero(loc == e)
        if tt.size == 0:
            continue
        aq_, as_ = xq[tt], xs[tt]
        a_deq = e4m3_decode(aq_).astype(np.float64) * np.repeat(as_.astype(np.float64), bk, axis=-1)
        w1 = _dequant64(w13_q[e], w13_s[e], bn, bk)
        hh = (a_deq @ w1.T).astype(np.float32)
        if apply_router_weight_on_input:
            hh = (hh * w[tt, kk][:, None]).astype(np.float32)
        hh = bf16_round(hh)
        a = silu_and_mul(hh, "bf16")
        a_q, a_s = group_quant_fp8(a)
        a2 = e4m3_decode(a_q).astype(np.float64) * np.repeat(a_s.astype(np.float64), bk, axis=-1)
        w2d = _dequant64(w2_q[e], w2_s[e], bn, bk)
        acc = (a2 @ w2d.T).astype(np.float32)
        if not apply_router_weight_on_input:
            acc = (acc * w[tt, kk][:, None]).astype(np.float32)
        y[tt, kk] = bf16_round(acc)
    out = moe_sum(y)
    return (out, y) if return_y else out


def _dequant64(q, s, bn, bk):
    wq = e4m3_decode(q).astype(np.float64)
    n, kk = wq.shape
    sc = np.repeat(np.repeat(np.asarray(s, np.float64), bn, axis=0)[:n], bk, axis=1)[:, :kk]
    return wq * sc


__all__ = ["fused_experts_bf16", "fused_experts_fp8", "moe_sum", "local_experts",
           "dequant_block_weight"]
