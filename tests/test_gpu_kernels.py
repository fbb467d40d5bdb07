"""GPU parity of the routing, align, quantiser and combine kernels against the
CPU oracle on identical seeded inputs.  Integer outputs (ids, sorted ids,
expert ids, padding, fp8 bytes of the quantiser, combine bits) are compared
bit for bit; float outputs within the stated tolerances."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import align as oalign
from oracle import moe as omoe
from oracle import quant as oquant
from oracle import routing as oroute
from oracle.numerics import bf16_round

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _bf16(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(torch.bfloat16).to(DEV)


def _np(t: torch.Tensor) -> np.ndarray:
    return t.float().cpu().numpy()


# ----------------------------------------------------------------- quant --
@pytest.mark.parametrize("rows,cols", [(1, 128), (7, 1024), (33, 7168), (256, 2048), (4096, 1536)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_group_quant_bit_exact(rows, cols, dtype):
    from vllm_musa_amd import per_token_group_quant_fp8
    g = np.random.Generator(np.random.PCG64(rows * 131 + cols))
    x = (g.standard_normal((rows, cols)) * g.uniform(0.01, 30, (rows, 1))).astype(np.float32)
    x[0, :128] = 0.0  # all-zero group
    xt = torch.from_numpy(x).to(dtype).to(DEV)
    q, s = per_token_group_quant_fp8(xt, 128)
    q_ref, s_ref = oquant.group_quant_fp8(xt.float().cpu().numpy())
    np.testing.assert_array_equal(s.cpu().numpy(), s_ref)
    np.testing.assert_array_equal(q.view(torch.uint8).cpu().numpy(), q_ref)


def test_group_quant_column_major_and_strided():
    from vllm_musa_amd import per_token_group_quant_fp8
    g = np.random.Generator(np.random.PCG64(5))
    big = _bf16(g.standard_normal((64, 1024 + 256)).astype(np.float32))
    x = big[:, :1024]  # row stride 1280, not contiguous
    q, s = per_token_group_quant_fp8(x, 128, column_major_scales=True)
    assert s.stride(0) == 1
    q_ref, s_ref = oquant.group_quant_fp8(_np(x))
    np.testing.assert_array_equal(s.cpu().numpy(), s_ref)
    np.testing.assert_array_equal(q.view(torch.uint8).cpu().numpy(), q_ref)


def test_group_quant_nan_and_saturation():
    from vllm_musa_amd import per_token_group_quant_fp8
    x = torch.zeros(2, 256, device=DEV, dtype=torch.bfloat16)
    x[0, 0] = float("nan")
    x[0, 1] = 3.0
    x[1, 128:] = -5.0
    q, s = per_token_group_quant_fp8(x, 128)
    qb = q.view(torch.uint8).cpu()
    assert qb[0, 0] == 0xFE and qb[0, 1] == 0x7E
    assert torch.all(qb[1, 128:] == 0xFE)


def _e4m3_rounding_targets() -> np.ndarray:
    """Quotients where e4m3 rounding is decided: every midpoint between two
    e4m3 values from the subnormal range up to 432 (ties, which round to
    even), the e4m3 values themselves, and each of them moved by 1-3 fp32
    ulps either way; plus +-0 and values just below 2^-10."""
    mids = [(2 * i + 1) * 2.0 ** -10 for i in range(8)]                    # subnormal range
    vals = [i * 2.0 ** -9 for i in range(1, 8)]
    for e in range(-6, 9):
        for k in range(8):
            vals.append((1 + k / 8) * 2.0 ** e)
            mids.append((1 + (2 * k + 1) / 16) * 2.0 ** e)
    base = np.array([m for m in mids + vals if m <= 448.0], np.float32)
    out = [base]
    up, down = base.copy(), base.copy()
    for _ in range(3):
        up = np.nextafter(up, np.float32(np.inf))
        down = np.nextafter(down, np.float32(0))
        out += [up.copy(), down.copy()]
    tiny = np.nextafter(np.float32(2.0 ** -10), np.float32(0)) * np.ones(4, np.float32)
    t = np.concatenate(out + [tiny, np.float32([0.0])])
    t = t[t <= 448.0]
    return np.concatenate([t, -t, np.float32([-0.0])])


@pytest.mark.parametrize("scale", ["pow2_low", "pow2_one", "pow2_high", "random"])
def test_group_quant_at_e4m3_rounding_boundaries(scale):
    """Quotients x / s on and within 3 ulps of every e4m3 rounding boundary,
    fp32 inputs: the bytes equal the oracle's (IEEE division, then
    round-to-nearest-even), including the ties, the e4m3 subnormal range and
    signed zeros.  A power-of-two scale (group max 448 * 2^k) makes x / s the
    target exactly; a random scale puts it within an ulp or so of it."""
    from vllm_musa_amd import per_token_group_quant_fp8
    t = _e4m3_rounding_targets()
    g = np.random.Generator(np.random.PCG64(17))
    ngroups = -(-t.size // 127)
    pad = np.zeros(ngroups * 127 - t.size, np.float32)
    body = np.concatenate([t, pad])
    g.shuffle(body)
    if scale == "random":
        s = g.uniform(0.01, 20.0, ngroups).astype(np.float32) / np.float32(448.0)
    else:
        k = {"pow2_low": -20, "pow2_one": 0, "pow2_high": 7}[scale]
        s = np.full(ngroups, 2.0 ** k, np.float32)
    x = np.empty((ngroups, 128), np.float32)
    x[:, 0] = (np.float32(448.0) * s).astype(np.float32)          # the group's absolute maximum
    x[:, 1:] = (body.reshape(ngroups, 127).astype(np.float64) * s[:, None]).astype(np.float32)
    xt = torch.from_numpy(x.reshape(1, -1)).to(DEV)
    q, sc = per_token_group_quant_fp8(xt, 128)
    q_ref, s_ref = oquant.group_quant_fp8(x.reshape(1, -1))
    np.testing.assert_array_equal(sc.cpu().numpy(), s_ref)
    np.testing.assert_array_equal(q.view(torch.uint8).cpu().numpy(), q_ref)


def test_silu_and_mul_close():
    from vllm_musa_amd import _custom_ops as ops
    g = np.random.Generator(np.random.PCG64(11))
    x = _bf16(g.standard_normal((300, 2 * 768)).astype(np.float32) * 3)
    out = torch.empty(300, 768, dtype=torch.bfloat16, device=DEV)
    ops.silu_and_mul(out, x)
    ref = oquant.silu_and_mul(_np(x))
    got = _np(out)
    assert (got != ref).mean() < 1e-3  # expf may differ from numpy's by an ulp
    np.testing.assert_allclose(got, ref, rtol=2 ** -7, atol=1e-6)


@pytest.mark.parametrize("limit", [None, 10.0])
def test_silu_quant(limit):
    from vllm_musa_amd import silu_mul_per_token_group_quant_fp8
    g = np.random.Generator(np.random.PCG64(12))
    x = _bf16(g.standard_normal((257, 2 * 2048)).astype(np.float32) * 4)
    q, s = silu_mul_per_token_group_quant_fp8(x, 128, swiglu_limit=limit)
    q_ref, s_ref = oquant.silu_and_mul_quant_fp8(_np(x), limit=limit)
    qb = q.view(torch.uint8).cpu().numpy()
    # the quantiser is exact; the only source of difference is an ulp of exp
    # flipping a bf16 rounding of silu(g)*u
    assert (qb != q_ref).mean() < 2e-3
    np.testing.assert_allclose(s.cpu().numpy(), s_ref, rtol=2 ** -7)
    # and it is exactly the quantiser applied to the GPU's own silu_and_mul
    from vllm_musa_amd import _custom_ops as ops
    if limit is None:
        a = torch.empty(257, 2048, dtype=torch.bfloat16, device=DEV)
        ops.silu_and_mul(a, x)
        q2, s2 = oquant.group_quant_fp8(_np(a))
        np.testing.assert_array_equal(qb, q2)
        np.testing.assert_array_equal(s.cpu().numpy(), s2)


# --------------------------------------------------------------- routing --
@pytest.mark.parametrize("T,E,K", [(1, 8, 2), (32, 8, 2), (1000, 128, 8), (77, 256, 8), (5, 1024, 4),
                                   (9, 60, 6)])
@pytest.mark.parametrize("renorm", [True, False])
def test_topk_softmax(T, E, K, renorm):
    from vllm_musa_amd import fused_topk
    g = np.random.Generator(np.random.PCG64(T * 7 + E))
    logits = g.standard_normal((T, E)).astype(np.float32)
    logits[:, :4] = np.round(logits[:, :4])  # exact ties
    lt = torch.from_numpy(logits).to(DEV)
    w, ids, tei = fused_topk(lt, lt, K, renorm)
    w_ref, ids_ref = oroute.topk_softmax(logits, K, renorm)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_allclose(w.cpu().numpy(), w_ref, rtol=1e-5, atol=1e-7)
    # upstream fused_topk's third output: [t, k] = k * T + t
    np.testing.assert_array_equal(tei.cpu().numpy(), np.arange(K)[None, :] * T + np.arange(T)[:, None])
    _, _, tei_s = fused_topk(lt, lt, K, renorm, scoring_func="sigmoid")
    np.testing.assert_array_equal(tei_s.cpu().numpy(), tei.cpu().numpy())


def test_topk_softmax_bias_bf16():
    from vllm_musa_amd import _custom_ops as ops
    g = np.random.Generator(np.random.PCG64(3))
    logits = bf16_round(g.standard_normal((100, 128)).astype(np.float32))
    bias = (g.standard_normal(128) * 0.01).astype(np.float32)
    w = torch.empty(100, 8, device=DEV)
    ids = torch.empty(100, 8, dtype=torch.int32, device=DEV)
    ops.topk_softmax(w, ids, _bf16(logits), True, correction_bias=torch.from_numpy(bias).to(DEV))
    w_ref, ids_ref = oroute.topk_softmax(logits, 8, True, bias)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_allclose(w.cpu().numpy(), w_ref, rtol=1e-5)


@pytest.mark.parametrize("with_bias", [False, True])
def test_topk_sigmoid(with_bias):
    from vllm_musa_amd import _custom_ops as ops
    g = np.random.Generator(np.random.PCG64(4))
    logits = (g.standard_normal((513, 128)) * 3).astype(np.float32)
    logits[:, 100:] = 30.0  # sigmoid saturates to 1.0 -> exact ties in the scores
    bias = (g.standard_normal(128) * 0.1).astype(np.float32) if with_bias else None
    w = torch.empty(513, 8, device=DEV)
    ids = torch.empty(513, 8, dtype=torch.int32, device=DEV)
    ops.topk_sigmoid(w, ids, torch.from_numpy(logits).to(DEV), True,
                     correction_bias=None if bias is None else torch.from_numpy(bias).to(DEV))
    w_ref, ids_ref = oroute.topk_sigmoid(logits, 8, True, bias)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_allclose(w.cpu().numpy(), w_ref, rtol=1e-6)


@pytest.mark.parametrize("T", [1, 16, 256, 4096])
def test_grouped_topk_dsv3(T):
    from vllm_musa_amd import grouped_topk
    g = np.random.Generator(np.random.PCG64(3000 + T))
    logits = g.standard_normal((T, 256)).astype(np.float32)
    bias = (g.standard_normal(256) * 0.1).astype(np.float32)
    lt = torch.from_numpy(logits).to(DEV)
    w, ids = grouped_topk(lt, lt, 8, True, 8, 4, "sigmoid", 2.5, torch.from_numpy(bias).to(DEV))
    w_ref, ids_ref = oroute.grouped_topk(logits, 8, True, 8, 4, "sigmoid", 2.5, bias)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_allclose(w.cpu().numpy(), w_ref, rtol=1e-6)


def test_grouped_topk_softmax_no_bias():
    from vllm_musa_amd import grouped_topk
    g = np.random.Generator(np.random.PCG64(77))
    logits = bf16_round(g.standard_normal((200, 160)).astype(np.float32))
    lt = _bf16(logits)
    w, ids = grouped_topk(lt, lt, 6, False, 8, 3, "softmax", 1.0, None)
    w_ref, ids_ref = oroute.grouped_topk(logits, 6, False, 8, 3, "softmax", 1.0, None)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_allclose(w.cpu().numpy(), w_ref, rtol=1e-6)


# ----------------------------------------------------------------- align --
@pytest.mark.parametrize("T,K,E,bs", [(1, 8, 256, 16), (16, 8, 256, 16), (32, 2, 8, 64),
                                      (4096, 8, 256, 128), (8192, 8, 128, 64), (3, 6, 1000, 4),
                                      (0, 8, 64, 16), (1000, 1, 7, 1)])
def test_moe_align_bit_exact(T, K, E, bs):
    from vllm_musa_amd.fused_moe import moe_align_block_size
    g = np.random.Generator(np.random.PCG64(T + 17 * E + bs))
    ids = np.stack([g.permutation(E)[:K] for _ in range(T)]).astype(np.int32) if T else \
        np.zeros((0, K), np.int32)
    it = torch.from_numpy(ids).to(DEV)
    s, eids, ntpp = moe_align_block_size(it, bs, E)
    s_ref, e_ref, n_ref, _, _ = oalign.moe_align_block_size(ids, E, bs)
    np.testing.assert_array_equal(s.cpu().numpy(), s_ref)
    np.testing.assert_array_equal(eids.cpu().numpy(), e_ref)
    assert int(ntpp.item()) == int(n_ref[0])


def test_moe_align_skewed_expert_map_and_scatter():
    from vllm_musa_amd import _custom_ops as ops
    g = np.random.Generator(np.random.PCG64(9))
    T, K, Eg, E, bs = 2000, 8, 128, 64, 32
    ids = np.stack([g.permutation(Eg)[:K] for _ in range(T)]).astype(np.int32)
    ids[:, 0] = 70  # one hot expert
    emap = np.full(Eg, -1, np.int32)
    emap[64:] = np.arange(64)
    cap = oalign.capacity_for(T * K, E, bs)
    s = torch.empty(cap, dtype=torch.int32, device=DEV)
    eids = torch.empty(-(-cap // bs), dtype=torch.int32, device=DEV)
    ntpp = torch.empty(1, dtype=torch.int32, device=DEV)
    offs = torch.empty(E + 1, dtype=torch.int32, device=DEV)
    scat = torch.empty(T * K, dtype=torch.int32, device=DEV)
    ops.moe_align_block_size(torch.from_numpy(ids).to(DEV), E, bs, s, eids, ntpp,
                             torch.from_numpy(emap).to(DEV), scat, offs)
    r = oalign.moe_align_block_size(ids, E, bs, expert_map=emap)
    for got, ref in zip((s, eids, ntpp, offs, scat), r):
        np.testing.assert_array_equal(got.cpu().numpy(), ref)


@pytest.mark.parametrize("T,K,E,bs", [(2000, 8, 256, 128), (1537, 3, 40, 16), (4096, 8, 256, 16)])
def test_moe_align_multi_workgroup_all_outputs(T, K, E, bs):
    """Inputs above 1024 routes are placed by one workgroup per chunk: every
    output (sorted ids, expert ids, padded count, offsets, scatter index,
    active experts) equals the oracle's, with a hot expert spanning chunks."""
    from vllm_musa_amd import _custom_ops as ops
    g = np.random.Generator(np.random.PCG64(T * K + E))
    ids = np.stack([g.permutation(E)[:K] for _ in range(T)]).astype(np.int32)
    ids[::2, 0] = 3
    ids[T // 3, :] = np.arange(K)
    cap = oalign.capacity_for(T * K, E, bs)
    s = torch.empty(cap, dtype=torch.int32, device=DEV)
    eids = torch.empty(-(-cap // bs), dtype=torch.int32, device=DEV)
    ntpp = torch.empty(1, dtype=torch.int32, device=DEV)
    offs = torch.empty(E + 1, dtype=torch.int32, device=DEV)
    scat = torch.empty(T * K, dtype=torch.int32, device=DEV)
    act = torch.full((E,), -7, dtype=torch.int32, device=DEV)
    nact = torch.empty(1, dtype=torch.int32, device=DEV)
    ops.moe_align_block_size(torch.from_numpy(ids).to(DEV), E, bs, s, eids, ntpp, None, scat, offs,
                             act, nact)
    r = oalign.moe_align_block_size(ids, E, bs)
    for got, ref in zip((s, eids, ntpp, offs, scat), r):
        np.testing.assert_array_equal(got.cpu().numpy(), ref)
    used = np.flatnonzero(np.bincount(ids.reshape(-1), minlength=E))
    assert int(nact.item()) == used.size
    np.testing.assert_array_equal(act.cpu().numpy()[:used.size], used)


# --------------------------------------------------------------- combine --
@pytest.mark.parametrize("T,K,H", [(1, 8, 7168), (33, 2, 1024), (300, 8, 2048), (5, 3, 100)])
def test_moe_sum_bit_exact(T, K, H):
    from vllm_musa_amd import _custom_ops as ops
    g = np.random.Generator(np.random.PCG64(T + H))
    y = bf16_round(g.standard_normal((T, K, H)).astype(np.float32))
    out = torch.empty(T, H, dtype=torch.bfloat16, device=DEV)
    ops.moe_sum(_bf16(y), out)
    np.testing.assert_array_equal(_np(out), omoe.moe_sum(y))


def test_moe_sum_skips_padding_slots():
    from vllm_musa_amd import _custom_ops as ops
    g = np.random.Generator(np.random.PCG64(2))
    y = bf16_round(g.standard_normal((10, 4, 256)).astype(np.float32))
    ids = g.integers(0, 8, (10, 4)).astype(np.int32)
    ids[0, 1] = -1
    emap = np.array([0, 1, 2, 3, -1, -1, -1, -1], np.int32)
    out = torch.empty(10, 256, dtype=torch.bfloat16, device=DEV)
    ops.moe_sum(_bf16(y), out, torch.from_numpy(ids).to(DEV), torch.from_numpy(emap).to(DEV))
    live = (ids >= 0) & (emap[np.clip(ids, 0, 7)] >= 0)
    ref = omoe.moe_sum(np.where(live[..., None], y, 0.0).astype(np.float32))
    np.testing.assert_array_equal(_np(out), ref)
