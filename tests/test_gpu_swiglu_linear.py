"""GPU parity of the clamp-aware SwiGLU + block-fp8 down projection
(silu_clamp_block_fp8_matmul, the reference's _musa_silu_clamp_deepgemm_fp8_op)
and of the row-parallel forward_swiglu_clamp hook.

The oracle composition is the clamped SiLU-and-mul with every step rounded to
bf16 (oracle.quant.silu_and_mul_clamped, pinned against torch), the 1x128
quantiser and the float64 closed form of the block GEMM.  Tolerance as for the
dense GEMM: rel-L2 <= 4e-3 and an elementwise bound of 2^-7 |ref| + 1e-3 max|ref|
(one bf16 rounding of an fp32 accumulation); the quantised activation bytes are
compared to the oracle's with at most 2e-3 of them one code apart (an ulp of
exp can flip a bf16 rounding of silu(g) * u)."""
from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from oracle.gemm import block_fp8_matmul_sampled
from oracle.quant import silu_and_mul_quant_fp8

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _check(out: np.ndarray, ref: np.ndarray):
    err = out.astype(np.float64) - ref
    rel_l2 = np.linalg.norm(err) / max(np.linalg.norm(ref), 1e-30)
    mref = np.abs(ref).max()
    assert rel_l2 <= 4e-3, rel_l2
    assert np.all(np.abs(err) <= 2 ** -7 * np.abs(ref) + 1e-3 * mref)


def _case(m, d, n, seed, boundary=True):
    from vllm_musa_amd import synthetic
    g = np.random.Generator(np.random.PCG64(seed))
    x = (g.standard_normal((m, 2 * d)) * 6).astype(np.float32)
    if boundary:
        edge = np.array([-np.inf, -20, -10, -0.0, 0.0, 10, 20, np.inf], np.float32)
        x[0, :8] = edge
        x[0, d:d + 8] = edge[::-1]
    gate_up = torch.from_numpy(x).to(torch.bfloat16).to(DEV)
    w, ws = synthetic.dense_fp8_weight(n, d, seed + 1)
    return gate_up, w, ws


def _oracle(gate_up, w, ws, rows, cols):
    xq, xs = silu_and_mul_quant_fp8(gate_up.float().cpu().numpy(), limit=10.0)
    return xq, xs, block_fp8_matmul_sampled(xq, xs, w.view(torch.uint8).cpu().numpy(),
                                            ws.cpu().numpy(), rows, cols)


@pytest.mark.parametrize("m", [1, 4, 64, 300])
def test_silu_clamp_block_fp8_matmul_matches_oracle(m):
    from vllm_musa_amd.block_fp8 import silu_clamp_block_fp8_matmul
    d, n = 2048, 384
    gate_up, w, ws = _case(m, d, n, 40 + m)
    out = silu_clamp_block_fp8_matmul(gate_up, w, ws, 128, False, 10.0)
    assert out.shape == (m, n) and out.dtype == torch.bfloat16
    rows = np.arange(m)
    xq, xs, ref = _oracle(gate_up, w, ws, rows, np.arange(n))
    got = out.float().cpu().numpy()
    # the boundary row holds infinities whose products are exceptional; its
    # quantised bytes are checked through the kernel tests, the rest here
    live = rows[1:] if m > 1 else rows
    if m > 1:
        _check(got[live], ref[live])
    assert np.isfinite(got[live]).all()


def test_silu_clamp_fallback_equals_fused_path():
    """A non-contiguous gate_up takes the reference's fallback (activation in
    torch, then the quantiser and the GEMM): same result as the fused path."""
    from vllm_musa_amd.block_fp8 import silu_clamp_block_fp8_matmul
    d, n, m = 1024, 256, 33
    gate_up, w, ws = _case(m, d, n, 7, boundary=False)
    wide = torch.zeros(m, 2 * d + 128, dtype=torch.bfloat16, device=DEV)
    wide[:, :2 * d] = gate_up
    view = wide[:, :2 * d]
    assert not view.is_contiguous()
    fused = silu_clamp_block_fp8_matmul(gate_up, w, ws, 128, False, 10.0).float()
    fallback = silu_clamp_block_fp8_matmul(view, w, ws, 128, False, 10.0).float()
    _check(fallback.cpu().numpy(), fused.double().cpu().numpy())


def test_forward_swiglu_clamp_hook():
    from vllm_musa_amd.block_fp8 import Fp8BlockScaledMMKernel, silu_clamp_block_fp8_matmul
    from vllm_musa_amd.linear import forward_swiglu_clamp
    d, n, m = 2048, 512, 5
    gate_up, w, ws = _case(m, d, n, 11, boundary=False)
    layer = SimpleNamespace(quant_method=SimpleNamespace(block_quant=True,
                                                         fp8_linear=Fp8BlockScaledMMKernel()),
                            input_is_parallel=True, bias=None, input_size_per_partition=d,
                            output_size_per_partition=n, weight=w, weight_scale_inv=ws,
                            weight_block_size=[128, 128], reduce_results=True, tp_size=1)
    out = forward_swiglu_clamp(layer, gate_up.view(1, m, 2 * d), 10.0)
    assert out is not None and out.shape == (1, m, n)
    ref = silu_clamp_block_fp8_matmul(gate_up, w, ws, 128, False, 10.0)
    assert torch.equal(out.view(m, n), ref)
    # the limit the fused path is confirmed for is 10; others fall back to the model
    assert forward_swiglu_clamp(layer, gate_up, 7.0) is None
