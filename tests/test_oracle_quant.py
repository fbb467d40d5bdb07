"""Pins oracle/quant.py: the 1x128 quantiser and SiLU-and-mul against closed
forms, special cases and a torch (CPU) restatement."""
from __future__ import annotations

import numpy as np
import torch

from oracle.numerics import bf16_round, e4m3_decode
from oracle.quant import group_quant_fp8, silu_and_mul, silu_and_mul_quant_fp8


def _torch_quant(x: np.ndarray, eps=1e-10):
    """torch restatement: s = max(eps, absmax)/448, q = fp8(clamp(x / s))."""
    t = torch.from_numpy(x).float().view(x.shape[0], -1, 128)
    s = t.abs().amax(-1, keepdim=True).clamp_min(eps) / 448.0
    q = (t / s).clamp(-448, 448).to(torch.float8_e4m3fn)
    return q.view(torch.uint8).reshape(x.shape).numpy(), s.squeeze(-1).numpy()


def test_quant_matches_torch_restatement(rng):
    x = bf16_round((rng.standard_normal((64, 1024)) * rng.uniform(0.01, 50, (64, 1))).astype(np.float32))
    q, s = group_quant_fp8(x)
    q_ref, s_ref = _torch_quant(x)
    np.testing.assert_array_equal(s, s_ref)
    np.testing.assert_array_equal(q, q_ref)


def test_quant_closed_form_special_cases():
    x = np.zeros((4, 256), np.float32)
    x[1, :128] = np.linspace(-3, 3, 128)
    x[1, 5] = 7.0           # group max -> +448
    x[2, 128:] = -1.0       # constant group -> all -448
    x[3, 0] = np.nan        # NaN element -> -448, ignored by the absmax
    x[3, 1] = 2.0
    q, s = group_quant_fp8(x)
    assert s[0, 0] == np.float32(1e-10) / np.float32(448)           # all-zero group
    assert np.all(q[0] == 0)
    assert s[1, 0] == np.float32(7.0) / np.float32(448)
    assert q[1, 5] == 0x7E                                         # +448
    assert np.all(q[2, 128:] == 0xFE)                               # -448
    assert q[3, 0] == 0xFE and s[3, 0] == np.float32(2.0) / np.float32(448)
    assert q[3, 1] == 0x7E


def test_quant_dequant_error_bound(rng):
    x = rng.standard_normal((32, 512)).astype(np.float32)
    q, s = group_quant_fp8(x)
    deq = e4m3_decode(q).reshape(32, 4, 128) * s[..., None]
    err = np.abs(deq.reshape(32, 512) - x)
    # e4m3 has 3 mantissa bits: relative half-ulp 1/16 for normals, plus the
    # absolute subnormal step 2^-10 * s.
    bound = np.abs(x) / 16 + np.repeat(s, 128, axis=1) * 2.0 ** -10
    assert np.all(err <= bound * 1.0001)


def test_quant_uses_true_division():
    # x / s and x * (1/s) differ in float32 for these values; the oracle must
    # quantise the quotient, as the reference does.
    x = np.full((1, 128), 0.0, np.float32)
    x[0, 0] = np.float32(448.0 * 3)  # s = 3
    found = 0
    for v in np.linspace(0.1, 3 * 448, 20000, dtype=np.float32):
        s = np.float32(3.0)
        if np.float32(v / s) != np.float32(v * (np.float32(1) / s)):
            x[0, 1 + found] = v
            found += 1
            if found == 100:
                break
    q, sc = group_quant_fp8(x)
    q_ref, _ = _torch_quant(x)
    np.testing.assert_array_equal(q, q_ref)


def test_silu_and_mul_matches_torch(rng):
    x = bf16_round(rng.standard_normal((64, 512)).astype(np.float32) * 4)
    ours = silu_and_mul(x)
    t = torch.from_numpy(x)
    ref = (torch.nn.functional.silu(t[:, :256]) * t[:, 256:]).to(torch.bfloat16).float().numpy()
    diff = ours != ref
    # both are float32 silu then one bf16 rounding; exp may differ by an ulp
    assert diff.mean() < 1e-3
    np.testing.assert_allclose(ours, ref, rtol=2 ** -7, atol=1e-6)


def test_silu_quant_is_quant_of_silu(rng):
    x = bf16_round(rng.standard_normal((16, 512)).astype(np.float32) * 3)
    q, s = silu_and_mul_quant_fp8(x)
    q2, s2 = group_quant_fp8(silu_and_mul(x))
    np.testing.assert_array_equal(q, q2)
    np.testing.assert_array_equal(s, s2)


def test_silu_quant_clamp_nan_to_min():
    x = np.zeros((1, 256), np.float32)
    x[0, :128] = 1.0
    x[0, 128:] = 2.0
    x[0, 3] = np.nan         # gate NaN
    x[0, 4] = -np.inf        # gate -inf
    x[0, 128 + 5] = np.nan   # up NaN
    x[0, 6] = 50.0           # gate clamped to 10
    q, s = silu_and_mul_quant_fp8(x, limit=10.0)
    assert q[0, 3] == 0xFE and q[0, 4] == 0xFE and q[0, 5] == 0xFE
    # clamped gate: silu(10) * 2 is the group max -> +448
    assert q[0, 6] == 0x7E
