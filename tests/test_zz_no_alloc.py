"""The allocation-free dense block-fp8 GEMM (vmamd_w8a8_block_fp8_matmul_noalloc)
against the workspace entry point through the C ABI: identical bits on two
calls in a row, the second on a smaller input (the fixed scratch keeps the
first call's partials), for split-K plans and for the unsplit GEMV / GEMM."""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


def _operands(M, N, K, seed):
    from vllm_musa_amd import synthetic
    from vllm_musa_amd.fp8_utils import per_token_group_quant_fp8
    w, ws = synthetic.dense_fp8_weight(N, K, seed)
    xq, xs = per_token_group_quant_fp8(synthetic.activations(M, K, seed + 1), 128)
    return xq, xs, w, ws


def _with_workspace(xq, xs, w, ws):
    from vllm_musa_amd import _lib
    from vllm_musa_amd._lib import call, ptr, stream_of
    M, K = xq.shape
    N = w.shape[0]
    nbytes = _lib.load().vmamd_w8a8_block_fp8_matmul_workspace_size(M, N, K)
    work = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=xq.device)
    out = torch.empty(M, N, dtype=torch.bfloat16, device=xq.device)
    call("vmamd_w8a8_block_fp8_matmul", ptr(xq), ptr(xs), xs.stride(0), xs.stride(1), ptr(w),
         ptr(ws), ptr(out), M, N, K, 128, 128, ptr(work) if nbytes else None, nbytes,
         stream_of(xq))
    return out


def _no_alloc(xq, xs, w, ws, out):
    from vllm_musa_amd._lib import call, ptr, stream_of
    M, K = xq.shape
    N = w.shape[0]
    call("vmamd_w8a8_block_fp8_matmul_noalloc", ptr(xq), ptr(xs), xs.stride(0), xs.stride(1),
         ptr(w), ptr(ws), ptr(out), M, N, K, 128, 128, stream_of(xq))
    return out


# (first call, second smaller call): split-K plans share the scratch; the
# last pair runs the GEMV / unsplit plans (no scratch) after a split plan.
# 512 x 7168 x 16384 is a 256 x 256 split plan (4 splits of 32 K steps,
# 58.7 MB of partials through the fixed scratch).
PAIRS = [((512, 2112, 7168), (200, 2112, 7168)),
         ((130, 7168, 2048), (65, 576, 7168)),
         ((512, 7168, 16384), (200, 2112, 7168)),
         ((200, 2112, 7168), (1, 2112, 7168))]


@pytest.mark.parametrize("first,second", PAIRS)
def test_no_alloc_matches_workspace_entry(first, second):
    from vllm_musa_amd import _lib
    lib = _lib.load()
    assert lib.vmamd_w8a8_block_fp8_matmul_workspace_size(*first) > 0
    for seed, (M, N, K) in ((901, first), (903, second)):
        ops = _operands(M, N, K, seed)
        ref = _with_workspace(*ops)
        out = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=ref.device)
        torch.cuda.synchronize()
        before = torch.cuda.memory_stats()["allocation.all.allocated"]
        _no_alloc(*ops, out)
        torch.cuda.synchronize()
        assert torch.cuda.memory_stats()["allocation.all.allocated"] == before
        assert torch.equal(out, ref), (M, N, K)


def test_no_alloc_rejects_plans_beyond_the_scratch():
    from vllm_musa_amd import _lib
    M, N, K = 384, 8192, 65536  # a split plan whose partials (96 MiB) exceed 64 MiB
    need = _lib.load().vmamd_w8a8_block_fp8_matmul_workspace_size(M, N, K)
    if need <= 64 << 20:
        pytest.skip(f"plan needs only {need} bytes here")
    ops = _operands(M, N, K, 905)
    out = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError, match="fixed scratch holds"):
        _no_alloc(*ops, out)
