"""Pins oracle/gemm.py: exactness of the float64 block form, agreement with
dequantise-then-matmul, torch._scaled_mm (CPU) on a single block, linearity in
the scales, the sampled variant, and N not a multiple of the block."""
from __future__ import annotations

import numpy as np
import torch

from oracle.gemm import (block_fp8_matmul_f64, block_fp8_matmul_sampled, dequant_block_weight,
                         w8a8_block_fp8_matmul)
from oracle.numerics import e4m3_decode, e4m3_encode


def _case(rng, m, n, k):
    a_q = e4m3_encode(np.clip(rng.standard_normal((m, k)) * 100, -448, 448).astype(np.float32))
    b_q = e4m3_encode(np.clip(rng.standard_normal((n, k)) * 64, -448, 448).astype(np.float32))
    a_s = rng.uniform(0.001, 0.01, (m, k // 128)).astype(np.float32)
    b_s = (rng.uniform(0.5, 2, (-(-n // 128), k // 128)) / 448).astype(np.float32)
    return a_q, a_s, b_q, b_s


def test_unit_scales_equal_plain_matmul(rng):
    a_q, _, b_q, _ = _case(rng, 9, 256, 384)
    ones_a = np.ones((9, 3), np.float32)
    ones_b = np.ones((2, 3), np.float32)
    ref = e4m3_decode(a_q).astype(np.float64) @ e4m3_decode(b_q).astype(np.float64).T
    np.testing.assert_array_equal(block_fp8_matmul_f64(a_q, ones_a, b_q, ones_b), ref)


def test_matches_dequantised_matmul(rng):
    a_q, a_s, b_q, b_s = _case(rng, 17, 320, 512)  # N = 320: partial last weight block
    a = e4m3_decode(a_q).astype(np.float64) * np.repeat(a_s, 128, 1)
    w = e4m3_decode(b_q).astype(np.float64) * np.repeat(np.repeat(b_s, 128, 0)[:320], 128, 1)
    np.testing.assert_allclose(block_fp8_matmul_f64(a_q, a_s, b_q, b_s), a @ w.T, rtol=1e-12,
                               atol=1e-12)
    np.testing.assert_allclose(dequant_block_weight(b_q, b_s), w.astype(np.float32), rtol=1e-6)


def test_single_block_matches_torch_scaled_mm(rng):
    a_q, a_s, b_q, b_s = _case(rng, 16, 128, 128)
    a_s[:] = a_s[0, 0]  # per-tensor scales, which _scaled_mm takes on the CPU
    at = torch.from_numpy(a_q).view(torch.float8_e4m3fn)
    bt = torch.from_numpy(b_q).view(torch.float8_e4m3fn)
    ref = torch._scaled_mm(at, bt.t(), scale_a=torch.tensor(float(a_s[0, 0])),
                           scale_b=torch.tensor(float(b_s[0, 0])), out_dtype=torch.float32)
    ours = block_fp8_matmul_f64(a_q, a_s, b_q, b_s)
    np.testing.assert_allclose(ours, ref.double().numpy(), rtol=1e-5, atol=1e-6)


def test_linear_in_each_block_scale(rng):
    a_q, a_s, b_q, b_s = _case(rng, 5, 256, 256)
    base = block_fp8_matmul_f64(a_q, a_s, b_q, b_s)
    b2 = b_s.copy()
    b2[1, 0] *= 2.0  # weight block (rows 128..255, k-block 0)
    part = block_fp8_matmul_f64(a_q, a_s * np.array([[1, 0]], np.float32), b_q, b_s)
    d = block_fp8_matmul_f64(a_q, a_s, b_q, b2) - base
    np.testing.assert_allclose(d[:, :128], 0, atol=1e-12)
    np.testing.assert_allclose(d[:, 128:], part[:, 128:], rtol=1e-12)


def test_sampled_and_rounded(rng):
    a_q, a_s, b_q, b_s = _case(rng, 40, 384, 256)
    full = block_fp8_matmul_f64(a_q, a_s, b_q, b_s)
    rows, cols = np.array([0, 7, 39]), np.array([1, 200, 383])
    np.testing.assert_allclose(block_fp8_matmul_sampled(a_q, a_s, b_q, b_s, rows, cols),
                               full[np.ix_(rows, cols)], rtol=1e-14)
    r = w8a8_block_fp8_matmul(a_q, a_s, b_q, b_s)
    np.testing.assert_allclose(r, full, rtol=2 ** -8)
