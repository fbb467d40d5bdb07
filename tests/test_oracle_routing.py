"""Pins oracle/routing.py: brute-force selection on tiny inputs (with ties),
torch.topk / torch.softmax restatements (the reference's own test refs,
tests/jit_kernel/test_csrc_jit_kernels.py:429-461), closed-form special cases."""
from __future__ import annotations

import itertools

import numpy as np
import pytest
import torch

from oracle.routing import (grouped_topk, sigmoid_cr, softmax_cr, topk_sigmoid,
                            topk_softmax)


def _brute_ids(sel_row, k):
    return sorted(range(len(sel_row)), key=lambda e: (-float(sel_row[e]), e))[:k]


def test_topk_softmax_brute_force_with_ties(rng):
    g = rng.integers(-2, 3, size=(200, 6)).astype(np.float32)  # many exact ties
    for renorm in (False, True):
        w, ids = topk_softmax(g, 3, renorm)
        for r in range(g.shape[0]):
            assert list(ids[r]) == _brute_ids(g[r], 3)


@pytest.mark.parametrize("renorm", [False, True])
@pytest.mark.parametrize("with_bias", [False, True])
def test_topk_softmax_vs_torch_ref(rng, renorm, with_bias):
    # the reference test's construction: distinct values, then a bias
    base = rng.permutation(np.linspace(-4, 4, 128)).astype(np.float32)
    g = base[None, :] + np.arange(7, dtype=np.float32)[:, None] * 0.001
    bias = (rng.standard_normal(128) * 0.01).astype(np.float32) if with_bias else None
    w, ids = topk_softmax(g, 8, renorm, bias)
    logits = torch.from_numpy(g)
    if bias is not None:
        logits = logits + torch.from_numpy(bias)[None]
    scores = torch.softmax(logits.double(), -1)
    _, rid = torch.topk(logits, 8, dim=-1)
    vals = scores.gather(1, rid)
    if renorm:
        vals = vals / vals.sum(-1, keepdim=True)
    np.testing.assert_array_equal(ids, rid.int().numpy())
    np.testing.assert_allclose(w, vals.float().numpy(), rtol=2e-6, atol=1e-7)


def test_topk_softmax_k_equals_e(rng):
    g = rng.standard_normal((50, 16)).astype(np.float32)
    w, ids = topk_softmax(g, 16, True)
    assert np.all(np.sort(ids, axis=1) == np.arange(16))
    np.testing.assert_allclose(w.sum(1), 1.0, rtol=1e-6)
    w2, _ = topk_softmax(g, 16, False)
    np.testing.assert_allclose(w, w2, rtol=1e-5)  # full softmax == renormalised when K == E


def test_sigmoid_cr_is_correctly_rounded(rng):
    x = (rng.standard_normal(100_000) * 6).astype(np.float32)
    ref = torch.sigmoid(torch.from_numpy(x).double()).float().numpy()
    np.testing.assert_array_equal(sigmoid_cr(x), ref)
    s = softmax_cr(x.reshape(100, 1000))
    ref = torch.softmax(torch.from_numpy(x.reshape(100, 1000)).double(), -1).float().numpy()
    np.testing.assert_array_equal(s, ref)


def test_topk_sigmoid_brute_force(rng):
    g = rng.standard_normal((300, 8)).astype(np.float32)
    bias = rng.integers(-1, 2, 8).astype(np.float32) * 0.25
    w, ids = topk_sigmoid(g, 3, True, bias)
    s = sigmoid_cr(g)
    for r in range(g.shape[0]):
        exp_ids = _brute_ids(s[r] + bias, 3)
        assert list(ids[r]) == exp_ids
        ws = s[r, exp_ids]
        np.testing.assert_allclose(w[r], ws / ws.sum(), rtol=1e-6)


def _torch_grouped(g, topk, renorm, ng, tg, scoring, scale, bias):
    """torch restatement of _grouped_topk_general (grouped_topk_router.py:308-357)."""
    gating = torch.from_numpy(g).double()
    scores = torch.softmax(gating, -1) if scoring == "softmax" else gating.sigmoid()
    scores = scores.float()
    t = scores.shape[0]
    if bias is not None:
        original = scores
        scores = scores + torch.from_numpy(bias)[None]
        gs = scores.view(t, ng, -1).topk(2, dim=-1)[0].sum(-1)
    else:
        gs = scores.view(t, ng, -1).max(-1).values
    gidx = torch.topk(gs, tg, dim=-1, sorted=True)[1]
    mask = torch.zeros_like(gs).scatter_(1, gidx, 1)
    smask = mask.unsqueeze(-1).expand(t, ng, scores.shape[-1] // ng).reshape(t, -1)
    tmp = scores.masked_fill(~smask.bool(), float("-inf"))
    if bias is not None:
        ids = torch.topk(tmp, topk, dim=-1, sorted=True)[1]
        w = original.gather(1, ids)
    else:
        w, ids = torch.topk(tmp, topk, dim=-1, sorted=True)
    if renorm:
        w = w / w.sum(-1, keepdim=True)
    return (w * scale).float().numpy(), ids.int().numpy()


@pytest.mark.parametrize("scoring,with_bias", [("sigmoid", True), ("softmax", False),
                                                ("sigmoid", False)])
def test_grouped_topk_vs_torch_ref(rng, scoring, with_bias):
    g = rng.standard_normal((64, 256)).astype(np.float32)
    bias = (rng.standard_normal(256) * 0.1).astype(np.float32) if with_bias else None
    w, ids = grouped_topk(g, 8, True, 8, 4, scoring, 2.5, bias)
    wr, idr = _torch_grouped(g, 8, True, 8, 4, scoring, 2.5, bias)
    np.testing.assert_array_equal(ids, idr)
    np.testing.assert_allclose(w, wr, rtol=2e-6)


def test_grouped_topk_brute_force_groups(rng):
    # E=8 in 4 groups of 2, keep 2 groups, top-3: enumerate every group pair
    g = rng.integers(-3, 4, size=(200, 8)).astype(np.float32) * 0.5
    bias = rng.integers(-2, 3, 8).astype(np.float32) * 0.125
    w, ids = grouped_topk(g, 3, False, 4, 2, "sigmoid", 1.0, bias)
    s = sigmoid_cr(g)
    sel = s + bias
    for r in range(g.shape[0]):
        gsc = [float(np.float32(sorted(sel[r, 2 * j:2 * j + 2])[-1] + sorted(sel[r, 2 * j:2 * j + 2])[-2]))
               for j in range(4)]
        kept = sorted(range(4), key=lambda j: (-gsc[j], j))[:2]
        cand = [e for e in range(8) if e // 2 in kept]
        exp = sorted(cand, key=lambda e: (-float(sel[r, e]), e))[:3]
        assert list(ids[r]) == exp
        np.testing.assert_array_equal(w[r], s[r, exp])


def test_grouped_one_group_reduces_to_topk_sigmoid(rng):
    g = rng.standard_normal((100, 128)).astype(np.float32)
    bias = (rng.standard_normal(128) * 0.1).astype(np.float32)
    w1, i1 = grouped_topk(g, 8, True, 1, 1, "sigmoid", 1.0, bias)
    w2, i2 = topk_sigmoid(g, 8, True, bias)
    np.testing.assert_array_equal(i1, i2)
    np.testing.assert_array_equal(w1, w2)
