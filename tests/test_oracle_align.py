"""Pins oracle/align.py against a pure-Python construction and the invariants
of moe_align_block_size (every route once, padded segments, sentinel padding,
monotone expert ids, num_tokens_post_pad = sum ceil(cnt/bs)*bs)."""
from __future__ import annotations

import numpy as np
import pytest

from oracle.align import capacity_for, moe_align_block_size


def _python_align(ids, E, bs, emap=None):
    flat = [int(v) for v in np.asarray(ids).reshape(-1)]
    numel = len(flat)
    seg = {e: [] for e in range(E)}
    for r, e in enumerate(flat):
        if emap is not None:
            e = int(emap[e]) if 0 <= e < len(emap) else -1
        if 0 <= e < E:
            seg[e].append(r)
    out, eids = [], []
    for e in range(E):
        lst = seg[e]
        pad = -(-len(lst) // bs) * bs
        out += lst + [numel] * (pad - len(lst))
        eids += [e] * (pad // bs)
    return out, eids


@pytest.mark.parametrize("T,K,E,bs", [(1, 1, 4, 16), (7, 2, 8, 4), (33, 8, 64, 16),
                                      (100, 6, 256, 64), (0, 8, 16, 16), (5, 3, 3, 1)])
def test_align_matches_python(rng, T, K, E, bs):
    ids = np.stack([rng.permutation(E)[:K] for _ in range(T)]) if T else np.zeros((0, K), np.int64)
    s, eids, ntpp, offs, scat = moe_align_block_size(ids, E, bs)
    ref_s, ref_e = _python_align(ids, E, bs)
    n = len(ref_s)
    assert ntpp[0] == n
    assert list(s[:n]) == ref_s
    assert np.all(s[n:] == T * K)
    assert list(eids[: n // bs]) == ref_e
    assert np.all(eids[n // bs:] == -1)
    assert len(s) == capacity_for(T * K, E, bs)
    # scatter is the inverse map of the placement
    for r in range(T * K):
        assert s[scat[r]] == r
    assert offs[-1] == n and np.all(np.diff(offs) % bs == 0)


def test_align_invariants_hot_expert(rng):
    T, K, E, bs = 300, 4, 32, 16
    ids = np.stack([rng.permutation(E)[:K] for _ in range(T)])
    ids[:, 0] = 3  # every token hits expert 3
    s, eids, ntpp, offs, _ = moe_align_block_size(ids, E, bs)
    n = int(ntpp[0])
    routes = s[:n][s[:n] < T * K]
    assert sorted(routes.tolist()) == list(range(T * K))            # each route once
    assert n == sum(-(-np.sum(ids == e) // bs) * bs for e in range(E))
    used = eids[: n // bs]
    assert np.all(np.diff(used) >= 0)                                # monotone
    for b, e in enumerate(used):                                     # block membership
        blk = s[b * bs:(b + 1) * bs]
        real = blk[blk < T * K]
        assert np.all(ids.reshape(-1)[real] == e)
        assert np.all(np.diff(real) > 0)                             # ascending


def test_align_expert_map(rng):
    T, K, E_glob, E_loc, bs = 40, 4, 16, 8, 8
    ids = np.stack([rng.permutation(E_glob)[:K] for _ in range(T)])
    emap = np.full(E_glob, -1, np.int32)
    emap[8:] = np.arange(8)   # this rank owns global experts 8..15
    s, eids, ntpp, _, scat = moe_align_block_size(ids, E_loc, bs, expert_map=emap)
    ref_s, ref_e = _python_align(ids, E_loc, bs, emap)
    assert list(s[: len(ref_s)]) == ref_s and ntpp[0] == len(ref_s)
    assert np.all((scat >= 0) == (ids.reshape(-1) >= 8))
