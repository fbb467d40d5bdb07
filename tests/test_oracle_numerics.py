"""Pins oracle/numerics.py: e4m3fn and bf16 encoders against closed forms,
brute-force nearest-value search and torch's CPU casts."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.numerics import (bf16_decode, bf16_encode, e4m3_decode, e4m3_decode_table,
                             e4m3_encode)


def test_e4m3_known_codes():
    t = e4m3_decode_table()
    assert t[0x00] == 0.0 and t[0x80] == 0.0 and np.signbit(t[0x80])
    assert t[0x01] == 2.0 ** -9            # smallest subnormal
    assert t[0x07] == 7 * 2.0 ** -9        # largest subnormal
    assert t[0x08] == 2.0 ** -6            # smallest normal
    assert t[0x38] == 1.0
    assert t[0x7E] == 448.0 and t[0xFE] == -448.0
    assert np.isnan(t[0x7F]) and np.isnan(t[0xFF])
    assert np.isnan(t).sum() == 2


def test_e4m3_decode_matches_torch():
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    ref = codes.view(torch.float8_e4m3fn).float().numpy()
    ours = e4m3_decode(np.arange(256, dtype=np.uint8))
    np.testing.assert_array_equal(np.isnan(ours), np.isnan(ref))
    m = ~np.isnan(ref)
    np.testing.assert_array_equal(ours[m], ref[m])


def _sample(rng, n=200_000):
    mag = rng.uniform(-1, 1, n) * np.exp2(rng.integers(-14, 10, n))
    x = np.clip(mag, -448, 448).astype(np.float32)
    t = e4m3_decode_table().astype(np.float64)
    fin = np.sort(np.unique(t[~np.isnan(t)]))
    mids = ((fin[:-1] + fin[1:]) / 2).astype(np.float32)  # exact ties
    return np.concatenate([x, mids, -mids, np.float32([0.0, -0.0, 448.0, -448.0, 464.0, -464.0])])


def test_e4m3_encode_matches_torch_cast(rng):
    x = _sample(rng)
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(e4m3_encode(x), ref)


def test_e4m3_encode_is_nearest_ties_even(rng):
    x = _sample(rng, 20_000)
    t = e4m3_decode_table().astype(np.float64)
    codes = np.array([c for c in range(256) if not np.isnan(t[c])])
    q = e4m3_encode(x)
    d = np.abs(t[codes][None, :] - x.astype(np.float64)[:, None])
    best = d.min(axis=1)
    np.testing.assert_array_equal(np.abs(t[q] - x), best)
    # at exact ties the chosen code has an even mantissa
    ties = (d == best[:, None]).sum(axis=1) > 1
    nonzero = x != 0
    assert np.all((q[ties & nonzero] & 1) == 0)
    # sign of zero results follows the input
    z = (t[q] == 0)
    np.testing.assert_array_equal(np.signbit(x[z]), (q[z] & 0x80) != 0)


def test_e4m3_overflow_is_nan():
    q = e4m3_encode(np.float32([480.0, -1000.0, np.nan]))
    assert np.all(np.isnan(e4m3_decode(q)))


def test_bf16_matches_torch(rng):
    x = (rng.standard_normal(100_000) * np.exp2(rng.integers(-30, 30, 100_000))).astype(np.float32)
    # exact ties and specials
    ties = (np.arange(1, 1000, dtype=np.uint32) << 16 | 0x8000).view(np.float32)
    x = np.concatenate([x, ties, -ties, np.float32([np.inf, -np.inf, 0.0, -0.0, 3.3895314e38])])
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(bf16_encode(x), ref)
    np.testing.assert_array_equal(bf16_decode(bf16_encode(x)),
                                  torch.from_numpy(x).to(torch.bfloat16).float().numpy())


def test_bf16_nan_canonical():
    assert bf16_encode(np.float32([np.nan]))[0] == 0x7FC0


@pytest.mark.parametrize("x", [1.0, -2.5, 3.0e-3])
def test_bf16_roundtrip_exact_values(x):
    v = np.float32(x)
    r = bf16_decode(bf16_encode(np.array([v])))[0]
    assert abs(r - v) <= abs(v) * 2 ** -8
