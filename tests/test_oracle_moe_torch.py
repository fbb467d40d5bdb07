"""The torch restatement of the fp8 MoE layer (oracle/moe_torch.py, the CPU
baseline bench.py times) against the float64 numpy oracle: its quantiser is
bit-exact, its layer output within the path's bf16/fp8 tolerance (float32
instead of float64 contractions move a few bf16 roundings by one ulp)."""
from __future__ import annotations

import numpy as np
import torch

from oracle import moe as omoe
from oracle import moe_torch as omt
from oracle import quant as oquant
from oracle.numerics import bf16_round


def test_group_quant_matches_oracle(rng):
    x = bf16_round((rng.standard_normal((9, 512)) * rng.uniform(0.01, 20, (9, 1))).astype(np.float32))
    x[0] = 0.0
    q_ref, s_ref = oquant.group_quant_fp8(x)
    q, s = omt.group_quant_fp8(torch.from_numpy(x))
    np.testing.assert_array_equal(s.numpy(), s_ref)
    np.testing.assert_array_equal(q.to(torch.float8_e4m3fn).view(torch.uint8).numpy(), q_ref)


def test_layer_matches_oracle(rng):
    t, h, i, e, k = 11, 256, 256, 4, 2
    w13 = rng.integers(0, 256, (e, 2 * i, h)).astype(np.uint8)
    w2 = rng.integers(0, 256, (e, h, i)).astype(np.uint8)
    w13[(w13 & 0x7F) == 0x7F] = 0x38
    w2[(w2 & 0x7F) == 0x7F] = 0x38
    s13 = rng.uniform(0.5, 2, (e, 2 * i // 128, h // 128)).astype(np.float32) / 448 / 64
    s2 = rng.uniform(0.5, 2, (e, h // 128, i // 128)).astype(np.float32) / 448 / 64
    x = bf16_round(rng.standard_normal((t, h)).astype(np.float32))
    ids = np.stack([rng.permutation(e)[:k] for _ in range(t)]).astype(np.int32)
    ids[3, 1] = -1
    w = rng.uniform(0.1, 1.0, (t, k)).astype(np.float32)
    ref = omoe.fused_experts_fp8(x, w13, s13, w2, s2, w, ids)
    got = omt.fused_experts_fp8(torch.from_numpy(x), torch.from_numpy(w13), torch.from_numpy(s13),
                                torch.from_numpy(w2), torch.from_numpy(s2), torch.from_numpy(w),
                                torch.from_numpy(ids)).numpy()
    err = got.astype(np.float64) - ref
    assert np.linalg.norm(err) / np.linalg.norm(ref) < 5e-3
    assert np.abs(err).max() <= 2e-2 * np.abs(ref).max()
