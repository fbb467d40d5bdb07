"""GPU parity of the dense w8a8 block-fp8 GEMM / split-K GEMV against the
float64 closed form of the oracle (sampled outputs for the big shapes).

Tolerance (the block-fp8 bar of the path): rel-L2 <= 1e-2 and
max-abs <= 2e-2 * max|ref|; the kernels accumulate in fp32 and round once to
bf16, so the test also asserts the tighter rel-L2 <= 4e-3 and an elementwise
bound of 2^-7 |ref| + 1e-3 max|ref|."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.gemm import block_fp8_matmul_sampled
from oracle.quant import group_quant_fp8

pytestmark = pytest.mark.gpu

SHAPES = [(24576, 1536), (7168, 18432), (2112, 7168), (7168, 2048)]


def _check(out: np.ndarray, ref: np.ndarray):
    err = out.astype(np.float64) - ref
    rel_l2 = np.linalg.norm(err) / max(np.linalg.norm(ref), 1e-30)
    mref = np.abs(ref).max()
    assert rel_l2 <= 4e-3, rel_l2
    assert np.abs(err).max() <= 2e-2 * mref
    assert np.all(np.abs(err) <= 2 ** -7 * np.abs(ref) + 1e-3 * mref)


def _run(M, N, K, seed, sample_rows=16, sample_cols=768):
    from vllm_musa_amd import synthetic
    from vllm_musa_amd.block_fp8 import apply_w8a8_block_fp8_linear
    from vllm_musa_amd.fp8_utils import per_token_group_quant_fp8
    w, ws = synthetic.dense_fp8_weight(N, K, seed)
    x = synthetic.activations(M, K, seed + 1)
    out = apply_w8a8_block_fp8_linear(x, w, ws).float().cpu().numpy()
    xq, xs = per_token_group_quant_fp8(x, 128)
    # activation quantisation is itself checked against the oracle
    q_ref, s_ref = group_quant_fp8(x.float().cpu().numpy())
    np.testing.assert_array_equal(xq.view(torch.uint8).cpu().numpy(), q_ref)
    g = np.random.Generator(np.random.PCG64(seed))
    rows = np.unique(np.concatenate([[0, M - 1], g.integers(0, M, min(M, sample_rows))]))
    cols = np.unique(np.concatenate([[0, N - 1], g.integers(0, N, min(N, sample_cols))]))
    ref = block_fp8_matmul_sampled(q_ref, s_ref, w.view(torch.uint8).cpu().numpy(),
                                   ws.cpu().numpy(), rows, cols)
    _check(out[np.ix_(rows, cols)], ref)


@pytest.mark.parametrize("N,K", SHAPES)
@pytest.mark.parametrize("M", [1, 4, 16, 64, 512])
def test_block_fp8_gemm_shapes(M, N, K):
    _run(M, N, K, seed=1000 + M + N // 16 + K // 128)


@pytest.mark.parametrize("N,K", SHAPES)
def test_block_fp8_gemm_m4096(N, K):
    """M = 4096 at every dense DeepSeek-V3 shape (the compute-bound point)."""
    _run(4096, N, K, seed=77, sample_rows=24, sample_cols=512)


@pytest.mark.parametrize("M", [3600, 4000])
def test_block_fp8_gemm_256_row_tiles_ragged(M):
    """M and N where the 256 x 256 GEMM is chosen (two rounds of 128 x 256
    tiles against one of 256 x 256), with the last row tile (M = 4000) and
    the last column tile (N = 2112) only partly inside the output."""
    _run(M, 2112, 1024, seed=31 + M, sample_rows=64, sample_cols=2112)


def test_block_fp8_gemm_256_row_tiles_column_major_scales():
    """The 256-row GEMM reads activation scales through their strides: the
    column-major layout gives the same bits as the row-major one."""
    from vllm_musa_amd import synthetic
    from vllm_musa_amd.block_fp8 import w8a8_block_fp8_matmul
    from vllm_musa_amd.fp8_utils import per_token_group_quant_fp8
    M, N, K = 4000, 2112, 1024
    w, ws = synthetic.dense_fp8_weight(N, K, 41)
    x = synthetic.activations(M, K, 42)
    xq, xs = per_token_group_quant_fp8(x, 128)
    xq2, xs2 = per_token_group_quant_fp8(x, 128, column_major_scales=True)
    assert xs2.stride(0) == 1
    a = w8a8_block_fp8_matmul(xq, w, xs, ws, [128, 128])
    b = w8a8_block_fp8_matmul(xq2, w, xs2, ws, [128, 128])
    assert torch.equal(a, b)


def test_block_fp8_gemm_256_row_tiles_unaligned_out():
    """The 256-row GEMM stages its bf16 tile through LDS and stores whole
    16-byte chunks when C is 16-byte aligned; an output 8 bytes off that
    alignment takes the per-fragment stores: the same bits."""
    from vllm_musa_amd import synthetic
    from vllm_musa_amd.block_fp8 import w8a8_block_fp8_matmul
    from vllm_musa_amd.fp8_utils import per_token_group_quant_fp8
    M, N, K = 4000, 2112, 1024
    w, ws = synthetic.dense_fp8_weight(N, K, 45)
    xq, xs = per_token_group_quant_fp8(synthetic.activations(M, K, 46), 128)
    a = w8a8_block_fp8_matmul(xq, w, xs, ws, [128, 128])
    assert a.data_ptr() % 16 == 0
    buf = torch.full((M * N + 4,), float("nan"), dtype=torch.bfloat16, device="cuda")
    out = buf[4:].view(M, N)
    assert out.data_ptr() % 16 == 8
    w8a8_block_fp8_matmul(xq, w, xs, ws, [128, 128], out=out)
    assert torch.equal(a, out)


@pytest.mark.parametrize("M", [512, 700])
def test_block_fp8_gemm_256_row_tiles_split_k(M):
    """Long rows at mid M (7168 x 16384): the 256 x 256 GEMM with K split over
    workgroups (fp32 partials added by the reduce); M = 700 leaves the last
    row tile mostly outside the output."""
    _run(M, 7168, 16384, seed=57 + M, sample_rows=48, sample_cols=1024)


def test_block_fp8_gemm_256_row_tiles_split_k_column_major_scales():
    """The split 256-row GEMM reads column-major activation scales through
    their strides: the same bits as row-major ones."""
    from vllm_musa_amd import synthetic
    from vllm_musa_amd.block_fp8 import w8a8_block_fp8_matmul
    from vllm_musa_amd.fp8_utils import per_token_group_quant_fp8
    M, N, K = 512, 7168, 16384
    w, ws = synthetic.dense_fp8_weight(N, K, 43)
    x = synthetic.activations(M, K, 44)
    xq, xs = per_token_group_quant_fp8(x, 128)
    xq2, xs2 = per_token_group_quant_fp8(x, 128, column_major_scales=True)
    a = w8a8_block_fp8_matmul(xq, w, xs, ws, [128, 128])
    b = w8a8_block_fp8_matmul(xq2, w, xs2, ws, [128, 128])
    assert torch.equal(a, b)


@pytest.mark.parametrize("M", [3, 17, 33, 65, 100, 130])
def test_block_fp8_gemm_ragged_m(M):
    _run(M, 2112, 1024, seed=5 + M, sample_rows=200, sample_cols=2112)


def test_block_fp8_matmul_full_small():
    """Every output element on a small case, through w8a8_block_fp8_matmul."""
    from vllm_musa_amd import synthetic
    from vllm_musa_amd.block_fp8 import w8a8_block_fp8_matmul
    from vllm_musa_amd.fp8_utils import per_token_group_quant_fp8
    M, N, K = 96, 400, 640
    w, ws = synthetic.dense_fp8_weight(N, K, 3)
    x = synthetic.activations(M, K, 4)
    xq, xs = per_token_group_quant_fp8(x, 128)
    out = w8a8_block_fp8_matmul(xq, w, xs, ws, [128, 128]).float().cpu().numpy()
    ref = block_fp8_matmul_sampled(xq.view(torch.uint8).cpu().numpy(), xs.cpu().numpy(),
                                   w.view(torch.uint8).cpu().numpy(), ws.cpu().numpy(),
                                   np.arange(M), np.arange(N))
    _check(out, ref)


@pytest.mark.parametrize("M", [1, 7, 40])
@pytest.mark.parametrize("K", [640, 1152])
def test_block_fp8_gemv_k_not_multiple_of_512(M, K):
    """Decode-sized M with K / 128 not a multiple of 4: the K-groups of the
    GEMV's waves end part-way through the last group (masked blocks), and the
    scales take the per-block load path.  Every output element is checked,
    and a second call must give identical bits (fixed summation order)."""
    from vllm_musa_amd import synthetic
    from vllm_musa_amd.block_fp8 import w8a8_block_fp8_matmul
    from vllm_musa_amd.fp8_utils import per_token_group_quant_fp8
    N = 400
    w, ws = synthetic.dense_fp8_weight(N, K, 11)
    x = synthetic.activations(M, K, 12 + M)
    xq, xs = per_token_group_quant_fp8(x, 128)
    out = w8a8_block_fp8_matmul(xq, w, xs, ws, [128, 128])
    again = w8a8_block_fp8_matmul(xq, w, xs, ws, [128, 128])
    assert torch.equal(out, again)
    ref = block_fp8_matmul_sampled(xq.view(torch.uint8).cpu().numpy(), xs.cpu().numpy(),
                                   w.view(torch.uint8).cpu().numpy(), ws.cpu().numpy(),
                                   np.arange(M), np.arange(N))
    _check(out.float().cpu().numpy(), ref)


def test_block_fp8_column_major_scales():
    from vllm_musa_amd import synthetic
    from vllm_musa_amd.block_fp8 import w8a8_block_fp8_matmul
    from vllm_musa_amd.fp8_utils import per_token_group_quant_fp8
    M, N, K = 8, 256, 512
    w, ws = synthetic.dense_fp8_weight(N, K, 9)
    x = synthetic.activations(M, K, 10)
    xq, xs = per_token_group_quant_fp8(x, 128)
    xq2, xs2 = per_token_group_quant_fp8(x, 128, column_major_scales=True)
    a = w8a8_block_fp8_matmul(xq, w, xs, ws, [128, 128])
    b = w8a8_block_fp8_matmul(xq2, w, xs2, ws, [128, 128])
    assert torch.equal(a, b)


@pytest.mark.parametrize("M", [1, 17, 33, 64])
def test_block_fp8_gemv_wide_weight_tiles(M):
    """N = 12288, K = 4096 with a workspace: M <= 32 runs the GEMV, whose
    waves hold two (M <= 16) or four (M > 16) 16-row weight tiles so every
    activation fragment is reused across them; M = 33 and 64 run the split-K
    GEMM (K >= 4096 from M = 33).  Sampled outputs against the oracle and a
    repeat call with identical bits."""
    from vllm_musa_amd import synthetic
    from vllm_musa_amd.block_fp8 import w8a8_block_fp8_matmul
    from vllm_musa_amd.fp8_utils import per_token_group_quant_fp8
    N, K = 12288, 4096
    w, ws = synthetic.dense_fp8_weight(N, K, 21)
    x = synthetic.activations(M, K, 22 + M)
    xq, xs = per_token_group_quant_fp8(x, 128)
    out = w8a8_block_fp8_matmul(xq, w, xs, ws, [128, 128])
    assert torch.equal(out, w8a8_block_fp8_matmul(xq, w, xs, ws, [128, 128]))
    g = np.random.Generator(np.random.PCG64(M))
    cols = np.unique(np.concatenate([[0, 63, 64, N - 1], g.integers(0, N, 1024)]))
    ref = block_fp8_matmul_sampled(xq.view(torch.uint8).cpu().numpy(), xs.cpu().numpy(),
                                   w.view(torch.uint8).cpu().numpy(), ws.cpu().numpy(),
                                   np.arange(M), cols)
    _check(out.float().cpu().numpy()[:, cols], ref)


@pytest.mark.parametrize("M", [1, 7, 40])
def test_block_fp8_gemv_wide_tiles_ragged_k(M):
    """N = 7168 (two weight tiles per wave, passes of 2 K-blocks) with
    K / 128 = 9: the last pass of a wave is half masked and the scales take
    the per-block path.  Every output element is checked."""
    from vllm_musa_amd import synthetic
    from vllm_musa_amd.block_fp8 import w8a8_block_fp8_matmul
    from vllm_musa_amd.fp8_utils import per_token_group_quant_fp8
    N, K = 7168, 1152
    w, ws = synthetic.dense_fp8_weight(N, K, 31)
    x = synthetic.activations(M, K, 32 + M)
    xq, xs = per_token_group_quant_fp8(x, 128)
    out = w8a8_block_fp8_matmul(xq, w, xs, ws, [128, 128])
    ref = block_fp8_matmul_sampled(xq.view(torch.uint8).cpu().numpy(), xs.cpu().numpy(),
                                   w.view(torch.uint8).cpu().numpy(), ws.cpu().numpy(),
                                   np.arange(M), np.arange(N))
    _check(out.float().cpu().numpy(), ref)


@pytest.mark.parametrize("M", [8, 24, 64])
def test_block_fp8_wide_tiles_column_major_scales(M):
    """N = 12288, K = 4096 (GEMV with wide weight tiles at M = 8 and 24, the
    split GEMM at M = 64): row-major and column-major activation scales take
    different scale loads but the same tiles and plan: identical bits."""
    from vllm_musa_amd import synthetic
    from vllm_musa_amd.block_fp8 import w8a8_block_fp8_matmul
    from vllm_musa_amd.fp8_utils import per_token_group_quant_fp8
    N, K = 12288, 4096
    w, ws = synthetic.dense_fp8_weight(N, K, 41)
    x = synthetic.activations(M, K, 42)
    xq, xs = per_token_group_quant_fp8(x, 128)
    xq2, xs2 = per_token_group_quant_fp8(x, 128, column_major_scales=True)
    a = w8a8_block_fp8_matmul(xq, w, xs, ws, [128, 128])
    b = w8a8_block_fp8_matmul(xq2, w, xs2, ws, [128, 128])
    assert torch.equal(a, b)


SPLIT_CASES = [(40, 2112, 7168), (65, 576, 7168), (130, 7168, 2048), (200, 2112, 7168), (512, 1536, 7168)]


@pytest.mark.parametrize("M,N,K", SPLIT_CASES)
def test_block_fp8_splitk_gemm(M, N, K):
    """Shapes whose 128 x 256 GEMM tiles are too few for the GPU: the GEMM
    splits K over workgroups into fp32 partials (the workspace) and adds them
    in split order.  M = 40 at K = 7168 takes the split GEMM instead of the
    GEMV.  Sampled outputs against the oracle; a repeat call gives identical
    bits."""
    from vllm_musa_amd import _lib, synthetic
    from vllm_musa_amd.block_fp8 import w8a8_block_fp8_matmul
    from vllm_musa_amd.fp8_utils import per_token_group_quant_fp8
    assert _lib.load().vmamd_w8a8_block_fp8_matmul_workspace_size(M, N, K) > 0
    w, ws = synthetic.dense_fp8_weight(N, K, 51)
    x = synthetic.activations(M, K, 52 + M)
    xq, xs = per_token_group_quant_fp8(x, 128)
    out = w8a8_block_fp8_matmul(xq, w, xs, ws, [128, 128])
    assert torch.equal(out, w8a8_block_fp8_matmul(xq, w, xs, ws, [128, 128]))
    g = np.random.Generator(np.random.PCG64(M + N))
    rows = np.unique(np.concatenate([[0, M - 1], g.integers(0, M, 48)]))
    cols = np.unique(np.concatenate([[0, N - 1], g.integers(0, N, 512)]))
    ref = block_fp8_matmul_sampled(xq.view(torch.uint8).cpu().numpy(), xs.cpu().numpy(),
                                   w.view(torch.uint8).cpu().numpy(), ws.cpu().numpy(), rows, cols)
    _check(out.float().cpu().numpy()[np.ix_(rows, cols)], ref)


def test_block_fp8_big_split_plan_on_128_row_tiles():
    """512 x 7168 x 16384 plans the 256 x 256 kernel split over K.  With the
    activation scales passed at a negative row stride (last row first),
    which only the 128 x 256 kernel takes, the call runs that kernel with the
    split its own model prices, within the workspace sized for the plan:
    sampled outputs against the oracle, and the usual call's values to the
    fp32 summation order."""
    from vllm_musa_amd import _lib, synthetic
    from vllm_musa_amd._lib import call, ptr, stream_of
    from vllm_musa_amd.block_fp8 import w8a8_block_fp8_matmul
    from vllm_musa_amd.fp8_utils import per_token_group_quant_fp8
    M, N, K = 512, 7168, 16384
    KB = K // 128
    nbytes = _lib.load().vmamd_w8a8_block_fp8_matmul_workspace_size(M, N, K)
    assert nbytes > 0
    w, ws = synthetic.dense_fp8_weight(N, K, 81)
    xq, xs = per_token_group_quant_fp8(synthetic.activations(M, K, 82), 128)
    usual = w8a8_block_fp8_matmul(xq, w, xs, ws, [128, 128])
    rev = xs.flip(0).contiguous()  # rev[j] = xs[M - 1 - j]
    work = torch.empty(nbytes, dtype=torch.uint8, device=xq.device)
    out = torch.empty(M, N, dtype=torch.bfloat16, device=xq.device)
    call("vmamd_w8a8_block_fp8_matmul", ptr(xq), rev.data_ptr() + (M - 1) * KB * 4, -KB, 1, ptr(w),
         ptr(ws), ptr(out), M, N, K, 128, 128, ptr(work), nbytes, stream_of(xq))
    g = np.random.Generator(np.random.PCG64(83))
    rows = np.unique(np.concatenate([[0, M - 1], g.integers(0, M, 32)]))
    cols = np.unique(np.concatenate([[0, N - 1], g.integers(0, N, 512)]))
    ref = block_fp8_matmul_sampled(xq.view(torch.uint8).cpu().numpy(), xs.cpu().numpy(),
                                   w.view(torch.uint8).cpu().numpy(), ws.cpu().numpy(), rows, cols)
    _check(out.float().cpu().numpy()[np.ix_(rows, cols)], ref)
    d = (out.float() - usual.float()).abs().max().item()
    assert d <= 2 ** -7 * usual.float().abs().max().item()


@pytest.mark.parametrize("M,N,K", [(128, 7168, 2048), (512, 7168, 2048), (128, 2112, 7168),
                                   (200, 2112, 7168), (128, 24576, 1536)])
def test_block_fp8_gemm_128_column_tiles(M, N, K):
    """Mid-size M on small N, where the time model takes 128 x 128 tiles
    (unsplit at 512 x 7168 x 2048 and 128 x 24576 x 1536, whose workspace
    query is 0; split over K elsewhere), including a last column tile half
    outside N = 2112 and a ragged M = 200: every output against the oracle,
    a repeat call bitwise equal, and the call without a workspace (unsplit)
    equal to the fp32 summation order."""
    from vllm_musa_amd import _lib, synthetic
    from vllm_musa_amd._lib import call, ptr, stream_of
    from vllm_musa_amd.block_fp8 import w8a8_block_fp8_matmul
    from vllm_musa_amd.fp8_utils import per_token_group_quant_fp8
    nbytes = _lib.load().vmamd_w8a8_block_fp8_matmul_workspace_size(M, N, K)
    if (M, N, K) in ((512, 7168, 2048), (128, 24576, 1536)):
        assert nbytes == 0
    w, ws = synthetic.dense_fp8_weight(N, K, 91)
    xq, xs = per_token_group_quant_fp8(synthetic.activations(M, K, 92 + M), 128)
    out = w8a8_block_fp8_matmul(xq, w, xs, ws, [128, 128])
    assert torch.equal(out, w8a8_block_fp8_matmul(xq, w, xs, ws, [128, 128]))
    ref = block_fp8_matmul_sampled(xq.view(torch.uint8).cpu().numpy(), xs.cpu().numpy(),
                                   w.view(torch.uint8).cpu().numpy(), ws.cpu().numpy(),
                                   np.arange(M), np.arange(N))
    _check(out.float().cpu().numpy(), ref)
    unsplit = torch.empty(M, N, dtype=torch.bfloat16, device=xq.device)
    call("vmamd_w8a8_block_fp8_matmul", ptr(xq), ptr(xs), xs.stride(0), xs.stride(1), ptr(w), ptr(ws),
         ptr(unsplit), M, N, K, 128, 128, None, 0, stream_of(xq))
    if nbytes == 0:
        assert torch.equal(unsplit, out)
    d = (unsplit.float() - out.float()).abs().max().item()
    assert d <= 2 ** -7 * out.float().abs().max().item()


@pytest.mark.parametrize("M,N,K", [(40, 2112, 7168), (200, 2112, 7168)])
def test_block_fp8_gemm_without_workspace(M, N, K):
    """Through the C ABI with a NULL workspace where the plan wants one: the
    call succeeds on the unsplit path (the GEMV at M <= 64) and matches the
    oracle; the split result agrees with it to the fp32 summation order."""
    from vllm_musa_amd import synthetic
    from vllm_musa_amd._lib import call, ptr, stream_of
    from vllm_musa_amd.block_fp8 import w8a8_block_fp8_matmul
    from vllm_musa_amd.fp8_utils import per_token_group_quant_fp8
    w, ws = synthetic.dense_fp8_weight(N, K, 61)
    x = synthetic.activations(M, K, 62)
    xq, xs = per_token_group_quant_fp8(x, 128)
    out = torch.empty(M, N, dtype=torch.bfloat16, device=xq.device)
    call("vmamd_w8a8_block_fp8_matmul", ptr(xq), ptr(xs), xs.stride(0), xs.stride(1), ptr(w), ptr(ws),
         ptr(out), M, N, K, 128, 128, None, 0, stream_of(xq))
    split = w8a8_block_fp8_matmul(xq, w, xs, ws, [128, 128])
    ref = block_fp8_matmul_sampled(xq.view(torch.uint8).cpu().numpy(), xs.cpu().numpy(),
                                   w.view(torch.uint8).cpu().numpy(), ws.cpu().numpy(),
                                   np.arange(M), np.arange(N))
    _check(out.float().cpu().numpy(), ref)
    _check(split.float().cpu().numpy(), ref)
    d = (out.float() - split.float()).abs().max().item()
    assert d <= 2 ** -7 * split.float().abs().max().item()


@pytest.mark.parametrize("M", [40, 200])
def test_block_fp8_splitk_column_major_scales(M):
    """Split-K plans (N = 2112, K = 7168) with column-major activation
    scales: each split starts its scale reads K-blocks into the strided
    layout; same plan and same values as row-major scales, so identical
    bits."""
    from vllm_musa_amd import synthetic
    from vllm_musa_amd.block_fp8 import w8a8_block_fp8_matmul
    from vllm_musa_amd.fp8_utils import per_token_group_quant_fp8
    N, K = 2112, 7168
    w, ws = synthetic.dense_fp8_weight(N, K, 71)
    x = synthetic.activations(M, K, 72)
    xq, xs = per_token_group_quant_fp8(x, 128)
    xq2, xs2 = per_token_group_quant_fp8(x, 128, column_major_scales=True)
    assert xs2.stride(0) == 1
    a = w8a8_block_fp8_matmul(xq, w, xs, ws, [128, 128])
    b = w8a8_block_fp8_matmul(xq2, w, xs2, ws, [128, 128])
    assert torch.equal(a, b)


@pytest.mark.parametrize("M,N,K", [(33, 12288, 4096), (48, 12288, 4096), (64, 12288, 4096)])
def test_block_fp8_gemv_fallback_without_workspace(M, N, K):
    """M = 33..64 on a weight the plan sends to the split GEMM, called through
    the C ABI with a NULL workspace: the call falls back to the GEMV with four
    16-row weight tiles per wave (gemv_fp8_bs_kernel<4, 4, 2>).  Every output
    element against the oracle, and a repeat call gives identical bits."""
    from vllm_musa_amd import _lib, synthetic
    from vllm_musa_amd._lib import call, ptr, stream_of
    from vllm_musa_amd.fp8_utils import per_token_group_quant_fp8
    assert _lib.load().vmamd_w8a8_block_fp8_matmul_workspace_size(M, N, K) > 0
    w, ws = synthetic.dense_fp8_weight(N, K, 81)
    x = synthetic.activations(M, K, 82 + M)
    xq, xs = per_token_group_quant_fp8(x, 128)
    outs = []
    for _ in range(2):
        out = torch.empty(M, N, dtype=torch.bfloat16, device=xq.device)
        call("vmamd_w8a8_block_fp8_matmul", ptr(xq), ptr(xs), xs.stride(0), xs.stride(1), ptr(w),
             ptr(ws), ptr(out), M, N, K, 128, 128, None, 0, stream_of(xq))
        outs.append(out)
    assert torch.equal(outs[0], outs[1])
    ref = block_fp8_matmul_sampled(xq.view(torch.uint8).cpu().numpy(), xs.cpu().numpy(),
                                   w.view(torch.uint8).cpu().numpy(), ws.cpu().numpy(),
                                   np.arange(M), np.arange(N))
    _check(outs[0].float().cpu().numpy(), ref)


def test_block_fp8_matmul_rejects_bad_out():
    from vllm_musa_amd import synthetic
    from vllm_musa_amd.block_fp8 import w8a8_block_fp8_matmul
    from vllm_musa_amd.fp8_utils import per_token_group_quant_fp8
    M, N, K = 8, 256, 512
    w, ws = synthetic.dense_fp8_weight(N, K, 9)
    xq, xs = per_token_group_quant_fp8(synthetic.activations(M, K, 10), 128)
    for bad in (torch.empty(M, N - 1, dtype=torch.bfloat16, device=xq.device),
                torch.empty(M, N, dtype=torch.float16, device=xq.device),
                torch.empty(N, M, dtype=torch.bfloat16, device=xq.device).t()):
        with pytest.raises(ValueError, match="out must be"):
            w8a8_block_fp8_matmul(xq, w, xs, ws, [128, 128], out=bad)
