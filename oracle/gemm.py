"""w8a8 block-fp8 GEMM (numpy, float64 closed form).

Reference semantics (every kernel of the reference applies the scales per
K-block to a float accumulator): upstream fused_moe_kernel block-wise branch
vllm_musa/patches/series/0081-MUSA-fused_moe_kernel-even_Ks-scalar-b_scale-fast-pa.patch:64-108
(`acc += dot(a, b) * a_scale[:, None] * b_scale[None, :]`),
vllm_musa/kernels/fp8_block_gemm.py:17-75 and the DeepGEMM call
model_executor/kernels/linear/scaled_mm/deep_gemm.py:233-262:

    C[m, n] = sum_kb (sum_{k in kb} A[m,k] * B[n,k]) * As[m, kb] * Bs[n // bn, kb]

The inner sums are exact in float64 (products of two e4m3 values and sums of
at most 2^11 of them fit in 53 bits), so this is the exact value up to the
final scaling; outputs are rounded once to bf16.
"""
from __future__ import annotations

import numpy as np

from .numerics import bf16_round, e4m3_decode


def block_fp8_matmul_f64(a_q: np.ndarray, a_s: np.ndarray, b_q: np.ndarray, b_s: np.ndarray,
                         block_n: int = 128, block_k: int = 128) -> np.ndarray:
    """a_q [M,K] uint8, a_s [M, K/bk] f32, b_q [N,K] uint8, b_s [ceil(N/bn), K/bk] f32 -> [M,N] f64."""
    a = e4m3_decode(a_q).astype(np.float64)
    b = e4m3_decode(b_q).astype(np.float64)
    m, k = a.shape
    n = b.shape[0]
    kb = -(-k // block_k)
    out = np.zeros((m, n), dtype=np.float64)
    nb_idx = np.arange(n) // block_n
    for j in range(kb):
        sl = slice(j * block_k, min(k, (j + 1) * block_k))
        part = a[:, sl] @ b[:, sl].T
        out += part * np.asarray(a_s, np.float64)[:, j:j + 1] * np.asarray(b_s, np.float64)[nb_idx, j][None, :]
    return out


def w8a8_block_fp8_matmul(a_q, a_s, b_q, b_s, block_size=(128, 128)) -> np.ndarray:
    """bf16-rounded result (as float32 values)."""
    bn, bk = block_size
    return bf16_round(block_fp8_matmul_f64(a_q, a_s, b_q, b_s, bn, bk).astype(np.float32))


def dequant_block_weight(b_q: np.ndarray, b_s: np.ndarray, block_n: int = 128,
                         block_k: int = 128) -> np.ndarray:
    """fp8 [..., N, K] weight with [..., N/bn, K/bk] scales -> float32 values."""
    w = e4m3_decode(b_q).astype(np.float32)
    n, k = w.shape[-2:]
    s = np.repeat(np.repeat(np.asarray(b_s, np.float32), block_n, axis=-2)[..., :n, :], block_k,
                  axis=-1)[..., :k]
    return (w * s).astype(np.float32)


def block_fp8_matmul_sampled(a_q: np.ndarray, a_s: np.ndarray, b_q: np.ndarray, b_s: np.ndarray,
                             rows: np.ndarray, cols: np.ndarray, block_n: int = 128,
                             block_k: int = 128) -> np.ndarray:
    """The closed form restricted to output rows `rows` and columns `cols`
    (float64), for checking large GEMMs on a sample of their outputs."""
    a = e4m3_decode(a_q[rows]).astype(np.float64)
    b = e4m3_decode(b_q[cols]).astype(np.float64)
    sa = np.asarray(a_s, np.float64)[rows]
    sb = np.asarray(b_s, np.float64)[np.asarray(cols) // block_n]
    kb = a.shape[1] // block_k
    out = np.zeros((len(rows), len(cols)), dtype=np.float64)
    for j in range(kb):
        sl = slice(j * block_k, (j + 1) * block_k)
        out += (a[:, sl] @ b[:, sl].T) * sa[:, j:j + 1] * sb[:, j][None, :]
    return out
