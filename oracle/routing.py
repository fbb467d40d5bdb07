"""Router top-k (numpy).

Selection order everywhere: descending score, ties to the lower expert id
(jit_kernel/csrc/topk/topk_gating.mu:29-39; selection loops 114-137, 481-504).
A stable argsort of the negated scores gives exactly that order.

Transcendental scores that take part in a selection together with a bias
(sigmoid scores, grouped softmax scores) are evaluated in float64 and rounded
once to float32, i.e. they are the correctly rounded float32 values; the GPU
kernels evaluate them the same way, so selections agree bit for bit.
"""
from __future__ import annotations

import numpy as np


def _stable_topk(sel: np.ndarray, k: int) -> np.ndarray:
    """Indices of the k largest entries per row, descending, ties -> lower index."""
    order = np.argsort(-sel, axis=-1, kind="stable")
    return order[..., :k]


def sigmoid_cr(x: np.ndarray) -> np.ndarray:
    """float32 logistic function, correctly rounded via float64."""
    x64 = np.asarray(x, dtype=np.float32).astype(np.float64)
    with np.errstate(over="ignore"):
        return (1.0 / (1.0 + np.exp(-x64))).astype(np.float32)


def softmax_cr(x: np.ndarray) -> np.ndarray:
    """float32 softmax over the last axis, evaluated in float64 and rounded once."""
    x64 = np.asarray(x, dtype=np.float32).astype(np.float64)
    m = x64.max(axis=-1, keepdims=True)
    e = np.exp(x64 - m)
    return (e / e.sum(axis=-1, keepdims=True)).astype(np.float32)


def topk_softmax(gating: np.ndarray, topk: int, renormalize: bool,
                 bias: np.ndarray | None = None, softcap: float = 0.0):
    """Reference: topk_softmax (jit_kernel/csrc/topk.py:211-242), torch ref
    tests/jit_kernel/test_csrc_jit_kernels.py:429-443 (select on the biased
    logits, weights from softmax of the biased logits).  Renormalised weights
    follow the fixed-K kernel topk_gating.mu:511-528: exp(l_k - l_0) / sum over
    the selection in slot order."""
    l = np.asarray(gating, dtype=np.float32)
    if bias is not None:
        l = (l + np.asarray(bias, dtype=np.float32)[None, :]).astype(np.float32)
    if softcap > 0:
        l = (np.tanh(l / np.float32(softcap)) * np.float32(softcap)).astype(np.float32)
    ids = _stable_topk(l, topk)
    sel = np.take_along_axis(l, ids, axis=-1)
    first = sel[:, :1]
    e_sel = np.exp((sel - first).astype(np.float32)).astype(np.float32)
    if renormalize:
        denom = np.zeros(l.shape[0], dtype=np.float32)
        for k in range(topk):  # slot order, float32
            denom = (denom + e_sel[:, k]).astype(np.float32)
    else:
        denom = np.exp((l - first).astype(np.float32)).astype(np.float32).sum(-1, dtype=np.float32)
    w = (e_sel / denom[:, None]).astype(np.float32)
    return w, ids.astype(np.int32)


def topk_sigmoid(gating: np.ndarray, topk: int, renormalize: bool,
                 bias: np.ndarray | None = None):
    """Reference: topk_sigmoid (jit_kernel/csrc/topk.py:245-275), torch ref
    tests/jit_kernel/test_csrc_jit_kernels.py:446-461: scores = sigmoid(l),
    select on scores + bias, weights = unbiased scores, optional renorm."""
    s = sigmoid_cr(gating)
    sel = s if bias is None else (s + np.asarray(bias, dtype=np.float32)[None, :]).astype(np.float32)
    ids = _stable_topk(sel, topk)
    w = np.take_along_axis(s, ids, axis=-1)
    if renormalize:
        denom = np.zeros(s.shape[0], dtype=np.float32)
        for k in range(topk):
            denom = (denom + w[:, k]).astype(np.float32)
        w = (w / denom[:, None]).astype(np.float32)
    return w.astype(np.float32), ids.astype(np.int32)


def grouped_topk(gating: np.ndarray, topk: int, renormalize: bool, num_expert_group: int,
                 topk_group: int, scoring_func: str = "softmax",
                 routed_scaling_factor: float = 1.0, bias: np.ndarray | None = None):
    """Reference: _grouped_topk_general
    (model_executor/layers/fused_moe/router/grouped_topk_router.py:257-357):
      scores = softmax|sigmoid(gating) (308-313); with a bias, selection
      scores = scores + bias and the group score is the sum of the group's
      top-2 (315-323), else the group max (324-327); keep topk_group groups
      (331-341); top-k over the kept experts (343-351); weights are the
      unbiased scores (346); renormalise (352-353); scale (355-356).
    """
    g32 = np.asarray(gating, dtype=np.float32)
    t, e = g32.shape
    if scoring_func == "softmax":
        scores = softmax_cr(g32)
    elif scoring_func == "sigmoid":
        scores = sigmoid_cr(g32)
    else:
        raise ValueError(scoring_func)
    sel = scores if bias is None else (scores + np.asarray(bias, np.float32)[None, :]).astype(np.float32)
    grp = sel.reshape(t, num_expert_group, e // num_expert_group)
    if bias is not None:
        top2 = -np.sort(-grp, axis=-1)[..., :2]
        gscore = (top2[..., 0] + top2[..., 1]).astype(np.float32)
    else:
        gscore = grp.max(axis=-1)
    gidx = _stable_topk(gscore, topk_group)
    keep = np.zeros((t, num_expert_group), dtype=bool)
    np.put_along_axis(keep, gidx, True, axis=-1)
    mask = np.repeat(keep, e // num_expert_group, axis=-1)
    masked = np.where(mask, sel, -np.inf).astype(np.float32)
    ids = _stable_topk(masked, topk)
    w = np.take_along_axis(scores, ids, axis=-1).astype(np.float32)
    if renormalize:
        denom = np.zeros(t, dtype=np.float32)
        for k in range(topk):
            denom = (denom + w[:, k]).astype(np.float32)
        w = (w / denom[:, None]).astype(np.float32)
    if routed_scaling_factor != 1.0:
        w = (w * np.float32(routed_scaling_factor)).astype(np.float32)
    return w, ids.astype(np.int32)
