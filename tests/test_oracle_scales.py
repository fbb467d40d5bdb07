"""Pins oracle/scales.py: closed forms of the e8m0 upcast, torch's own
float8_e8m0fnu and bfloat16 casts (library cross-checks), and the invalid
scales of the reference's loader test (tests/test_w4afp8_quantization.py:207-224)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import scales as osc
from oracle.numerics import bf16_decode


def test_e8m0_closed_forms():
    b = np.array([0, 1, 126, 127, 128, 200, 254, 255], dtype=np.uint8)
    got = osc.upcast_e8m0_to_fp32(b)
    want = np.array([0.0, 2.0 ** -126, 0.5, 1.0, 2.0, 2.0 ** 73, 2.0 ** 127, np.inf], np.float32)
    assert np.array_equal(got, want)


@pytest.mark.skipif(getattr(torch, "float8_e8m0fnu", None) is None, reason="no e8m0 dtype")
def test_e8m0_matches_torch_on_normal_exponents():
    # torch decodes byte b as 2^(b-127); the reference's shift agrees on 1..254
    # and differs only at 0 (2^-127 vs +0.0) and 255 (NaN vs +inf).
    b = torch.arange(256, dtype=torch.uint8)
    t = b.view(torch.float8_e8m0fnu).float().numpy()
    o = osc.upcast_e8m0_to_fp32(b.numpy())
    assert np.array_equal(t[1:255], o[1:255])
    assert o[0] == 0.0 and t[0] == 2.0 ** -127
    assert np.isinf(o[255]) and np.isnan(t[255])


def _f32_cases(rng):
    specials = np.array([0.0, -0.0, 1.0, -1.0, np.inf, -np.inf, np.nan, 1e-42, -1e-42, 3.4e38,
                         3.3895314e38, np.finfo(np.float32).max, np.finfo(np.float32).tiny],
                        np.float32)
    # exact ties between two bf16 values, both parities of the kept bit
    ties = (np.array([0x3F808000, 0x3F818000, 0xBF808000, 0x7F7F8000, 0x00008000],
                     np.uint32)).view(np.float32)
    rand = rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(
        -30, 30, 20000).astype(np.float32)
    bits = rng.integers(0, 2 ** 32, 20000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    return np.concatenate([specials, ties, rand, bits])


def test_f32_to_bf16_matches_torch():
    x = _f32_cases(np.random.default_rng(7))
    h, _ = osc.convert_scales(x, "f32", "bf16")
    t = torch.from_numpy(x.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(h[~nan], t[~nan])
    assert (h[nan] == 0x7FC0).all()


def test_truncating_cast_would_be_caught():
    # a plausible slip (dropping the rounding) disagrees with torch on these inputs
    x = _f32_cases(np.random.default_rng(8))
    x = x[np.isfinite(x)]
    trunc = (x.view(np.uint32) >> 16).astype(np.uint16)
    t = torch.from_numpy(x.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert not np.array_equal(trunc, t)


@pytest.mark.parametrize("invalid", [float("nan"), float("inf"), -0.1, 0.0, 1.0e-42, 3.4e38])
def test_reference_invalid_scales_are_rejected(invalid):
    s = np.full((4, 3), 0.01, np.float32)
    s[1, 2] = invalid
    _, ok = osc.w4afp8_scales(s)
    assert not ok
    _, bad = osc.convert_scales(s, "f32", "bf16")
    assert bad == 1


def test_reference_valid_scales_cast_like_torch():
    s = torch.linspace(0.001, 0.013, 2 * 768 * 2).reshape(2, 768, 2)
    h, ok = osc.w4afp8_scales(s.numpy())
    assert ok
    t = s.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(h, t)


def test_invalid_count_counts_each_kind():
    v = np.array([1.0, 0.0, -0.0, -2.0, np.nan, np.inf, -np.inf, 1e-45, 2.0], np.float32)
    assert osc.invalid_count(v) == 6  # 1e-45 is a positive subnormal: valid in f32
    h, bad = osc.convert_scales(v, "f32", "bf16")
    assert bad == 7 and bf16_decode(h)[7] == 0.0  # ... but rounds to zero in bf16
