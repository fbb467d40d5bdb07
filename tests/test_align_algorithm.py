"""CPU emulation of the GPU moe_align placement algorithm (1024-route steps,
16 waves of 64 lanes, bit-sliced ballot ranks, [wave][expert] count table,
running per-expert counters; large inputs split into chunks, one workgroup
each, whose counters start at the histogram of the routes before the chunk).
Checks that every write stays inside its expert's segment and that the result
equals the oracle, at the sizes the kernel runs at (including several steps,
several chunks, ragged chunk ends and skewed routing)."""
from __future__ import annotations

import numpy as np
import pytest

from oracle.align import moe_align_block_size

THREADS, WAVE = 1024, 64


def _chunk_for(numel):
    """Routes per workgroup, as the launcher picks it (1024-route steps, at
    most 256 workgroups)."""
    return THREADS * max(1, -(-numel // (THREADS * 256)))


def _emulate(ids, E, bs, chunk=None):
    flat = np.asarray(ids).reshape(-1).astype(np.int64)
    numel = flat.size
    chunk = chunk or max(numel, 1)
    cnt = np.bincount(flat, minlength=E)
    padded = (cnt + bs - 1) // bs * bs
    base = np.concatenate([[0], np.cumsum(padded)])
    cap = numel + E * (bs - 1)
    out = np.full(cap, numel, np.int64)
    for c_begin in range(0, max(numel, 1), chunk):
        c_end = min(numel, c_begin + chunk)
        run = np.bincount(flat[:c_begin], minlength=E).astype(np.int64)
        _place(flat, E, base, run, out, c_begin, c_end)
    return out


def _place(flat, E, base, run, out, c_begin, c_end):
    numel = flat.size
    nbits = max(1, int(np.ceil(np.log2(E))) if E > 1 else 1)
    lanes = np.arange(WAVE)
    for c0 in range(c_begin, c_end, THREADS):
        wcnt = np.zeros((THREADS // WAVE, E), np.int64)
        r = c0 + np.arange(THREADS)
        e = np.where(r < c_end, flat[np.minimum(r, numel - 1)], -1)
        ranks = np.zeros(THREADS, np.int64)
        for w in range(THREADS // WAVE):
            ew = e[w * WAVE:(w + 1) * WAVE]
            valid = ew >= 0
            same = np.tile(valid, (WAVE, 1))  # same[l] = mask of lanes equal to lane l
            for b in range(nbits):
                on = valid & (((ew >> b) & 1) == 1)
                mine = ((ew >> b) & 1) == 1
                same &= np.where(mine[:, None], on[None, :], ~on[None, :])
            rank = (same & (lanes[None, :] < lanes[:, None])).sum(1)
            ranks[w * WAVE:(w + 1) * WAVE] = rank
            for l in range(WAVE):
                if valid[l] and rank[l] == 0:
                    wcnt[w, ew[l]] = same[l].sum()
        for t in range(THREADS):
            if e[t] < 0:
                continue
            w = t // WAVE
            pos = base[e[t]] + run[e[t]] + wcnt[:w, e[t]].sum() + ranks[t]
            assert base[e[t]] <= pos < base[e[t] + 1]
            out[pos] = r[t]
        run += wcnt.sum(0)


@pytest.mark.parametrize("T,K,E,bs,skew", [(4096, 8, 256, 128, False), (300, 8, 64, 16, True),
                                           (129, 8, 1000, 4, False)])
def test_emulated_kernel_matches_oracle(T, K, E, bs, skew):
    g = np.random.Generator(np.random.PCG64(T + 17 * E + bs))
    ids = np.stack([g.permutation(E)[:K] for _ in range(T)]).astype(np.int32)
    if skew:
        ids[:, 0] = 5
    got = _emulate(ids, E, bs)
    ref = moe_align_block_size(ids, E, bs)[0]
    np.testing.assert_array_equal(got, ref)


@pytest.mark.parametrize("T,K,E,bs,chunk", [(4096, 8, 256, 128, None), (1251, 8, 64, 32, 1024),
                                            (700, 8, 128, 16, 2048), (1500, 1, 8, 4, 1024)])
def test_emulated_chunked_kernel_matches_oracle(T, K, E, bs, chunk):
    """Several workgroups, each placing one chunk (ragged last chunk, a hot
    expert spanning chunks): same sorted_token_ids as the oracle."""
    g = np.random.Generator(np.random.PCG64(3 * T + E))
    ids = np.stack([g.permutation(E)[:K] for _ in range(T)]).astype(np.int32)
    ids[::3, 0] = 1
    chunk = chunk or _chunk_for(T * K)
    assert chunk < T * K
    got = _emulate(ids, E, bs, chunk)
    ref = moe_align_block_size(ids, E, bs)[0]
    np.testing.assert_array_equal(got, ref)
