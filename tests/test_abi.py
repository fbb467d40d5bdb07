"""The C-ABI library: it loads, exports every symbol include/vllm_musa_amd.h
declares, and its argument checks reject bad calls before touching a GPU."""
from __future__ import annotations

import ctypes
import os
import re

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "vllm_musa_amd.h")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[\w\s\*]+?\b(vmamd_\w+)\s*\(", text, re.M)))


def test_header_declares_entry_points():
    names = _declared()
    assert "vmamd_last_error" in names and len(names) >= 8


def test_library_exports_every_declared_symbol():
    from vllm_musa_amd import _lib
    lib = _lib.load()
    missing = [n for n in _declared() if not hasattr(lib, n)]
    assert not missing, missing
    # the Python binding describes every declared entry point
    assert set(_declared()) == set(_lib.SIGNATURES)


def test_abi_version():
    from vllm_musa_amd import _lib
    assert _lib.load().vmamd_abi_version() >= 1


def test_argument_errors_are_reported_without_a_gpu():
    from vllm_musa_amd import _lib
    with pytest.raises(ValueError, match="experts must be in"):
        _lib.call("vmamd_topk_softmax", None, 2, 4, 0, 1, 0, 0.0, None, None, None, None, None)
    with pytest.raises(ValueError, match="group_size must be 128"):
        _lib.call("vmamd_per_token_group_quant_fp8", None, 2, 1, 128, 128, 64, 1e-10, -448.0,
                  448.0, None, None, 1, 1, None)
    with pytest.raises(ValueError, match="capacity"):
        _lib.call("vmamd_moe_align_block_size", None, 100, 8, 16, None, 0, None, 10, None, None,
                  None, None, None, None, None)
    msg = _lib.load().vmamd_last_error().decode()
    assert "capacity" in msg
    # 320-route blocks are a bf16 tile: the fp8 stages refuse them
    with pytest.raises(ValueError, match="bf16 weights only"):
        _lib.call("vmamd_moe_fp8_w13", None, None, 1024, 512, 2, None, 1 << 20, 320, None, None, None,
                  None, None, None, 8, 256, 0.0, None, None, None, 0, None)


def test_bf16_large_block_rule():
    """The bf16 grouped GEMMs take 320-route blocks where the expected largest
    expert (mean + 3 sqrt(mean) routes) needs fewer of them than of 256-route
    blocks, each counted 1.25x: mean 256 -> one 320 block instead of two;
    mean 512 -> two instead of three; mean 1024 -> 256 (four 320 blocks
    cost as much as five); mean 128, 175 and 384 -> 256 (as many blocks
    either way)."""
    from vllm_musa_amd.fused_moe import _bf16_big_block
    assert _bf16_big_block(2048 * 8, 128) == 256       # mean 128
    assert _bf16_big_block(4096 * 8, 128) == 320       # mean 256
    assert _bf16_big_block(8192 * 8, 128) == 320       # mean 512
    assert _bf16_big_block(16384 * 8, 128) == 256      # mean 1024: 5 vs 4 * 1.25
    assert _bf16_big_block(6144 * 8, 128) == 256       # mean 384: 2 vs 2
    assert _bf16_big_block(700 * 2, 8) == 256          # mean 175
    assert _bf16_big_block(1024 * 2, 8) == 320


def test_dense_workspace_query():
    """vmamd_w8a8_block_fp8_matmul_workspace_size is host arithmetic (no GPU
    needed): nothing for the GEMV (M <= 16) or for a GEMM whose tiles fill
    the GPU; for a split plan, a whole number (2..16) of fp32 M x N partials
    within 256 MiB."""
    from vllm_musa_amd import _lib
    q = _lib.load().vmamd_w8a8_block_fp8_matmul_workspace_size
    for m, n, k in [(1, 2112, 7168), (16, 7168, 18432), (64, 7168, 2048), (4096, 7168, 18432),
                    (2048, 36864, 7168), (0, 7168, 2048)]:
        assert q(m, n, k) == 0, (m, n, k)
    for m, n, k in [(40, 2112, 7168), (65, 7168, 18432), (512, 2112, 7168), (130, 7168, 2048)]:
        b = q(m, n, k)
        assert b > 0 and b % (m * n * 4) == 0 and 2 <= b // (m * n * 4) <= 16 and b <= 256 << 20, (m, n, k, b)
