"""GPU parity at the exact benchmark configurations of the path, each checked
against the oracle on identical seeded inputs:

  C0  bf16 fused MoE, T=32, H=1024, I=512, E=8, top-2 softmax-renorm, seed 0
      (every output, both kernel paths);
  C2  bf16 fused MoE, E=128, top-8 softmax-renorm, H=2048, I=768 at T=8192,
      uniform and skewed (+2.0 on 8 hot experts) logits (sampled tokens);
  C3  fp8 block MoE, DeepSeek-V3 shape (E=256, grouped sigmoid+bias top-8,
      H=7168, I=2048): the T=4096 step exactly as bench.py times it (grouped
      top-k + fused_experts_impl, path auto) and T=257 (sampled tokens);
  C4  w4afp8 fused MoE, E=128, top-8, H=4096, I=1536 at T=4096 (sampled tokens).

Tokens are independent of each other in every layer (per-token quantisation,
per-route GEMMs), so a sample of output rows is checked against the oracle run
on those rows alone, with only the experts they touch copied to the host.
Routing ids are compared bit for bit on every token.

Tolerance (the path's bar for bf16/fp8 outputs): rel-L2 <= 1e-2 and
max-abs <= 2e-2 * max|ref|."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import moe as omoe
from oracle import routing as oroute
from oracle import w4afp8 as ow4

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _check(out: torch.Tensor, ref: np.ndarray, rel_l2=1e-2, max_frac=2e-2):
    o = out.float().cpu().numpy().astype(np.float64)
    err = o - ref
    rl2 = np.linalg.norm(err) / max(np.linalg.norm(ref), 1e-30)
    assert np.isfinite(o).all()
    assert rl2 <= rel_l2, f"rel-L2 {rl2}"
    assert np.abs(err).max() <= max_frac * np.abs(ref).max(), f"max-abs {np.abs(err).max()}"
    return rl2


def _sample_rows(T, ids, n, seed):
    """n token rows: the first, the last, one routed to the most loaded
    expert, and random ones."""
    g = np.random.Generator(np.random.PCG64(seed))
    ids_np = ids.cpu().numpy()
    hot = np.bincount(ids_np.reshape(-1)[ids_np.reshape(-1) >= 0]).argmax()
    hot_row = int(np.nonzero((ids_np == hot).any(axis=1))[0][0])
    rows = {0, T - 1, hot_row}
    while len(rows) < min(n, T):
        rows.add(int(g.integers(0, T)))
    return np.array(sorted(rows))


def _compact(ids_rows, E):
    """Ids of the sampled rows remapped onto the compact stack of the experts
    they touch (returned as a device index)."""
    used = np.unique(ids_rows[ids_rows >= 0])
    remap = np.full(E, -1, np.int64)
    remap[used] = np.arange(used.size)
    cids = np.where(ids_rows >= 0, remap[np.maximum(ids_rows, 0)], -1).astype(np.int32)
    return cids, torch.from_numpy(used).to(DEV)


def _oracle_fp8_rows(x, w13, s13, w2, s2, w, ids, rows):
    cids, sel = _compact(ids.cpu().numpy()[rows], w13.shape[0])
    u8 = lambda t: t.view(torch.uint8).index_select(0, sel).cpu().numpy()
    f32 = lambda t: t.index_select(0, sel).cpu().numpy()
    return omoe.fused_experts_fp8(x.float().cpu().numpy()[rows], u8(w13), f32(s13), u8(w2),
                                  f32(s2), w.cpu().numpy()[rows], cids)


def _oracle_bf16_rows(x, w13, w2, w, ids, rows):
    cids, sel = _compact(ids.cpu().numpy()[rows], w13.shape[0])
    f32 = lambda t: t.index_select(0, sel).float().cpu().numpy()
    return omoe.fused_experts_bf16(x.float().cpu().numpy()[rows], f32(w13), f32(w2),
                                   w.cpu().numpy()[rows], cids)


# ------------------------------------------------------------------ C0 -----
@pytest.mark.parametrize("path", ["gemv", "gemm", "auto"])
def test_c0_bf16_layer_exact_config(path):
    """C0: T=32, H=1024, I=512, E=8, top-2 softmax then renormalise, seed 0;
    routing on the GPU kernel (ids bit-exact), every output row checked."""
    from vllm_musa_amd import fused_topk, synthetic
    from vllm_musa_amd.fused_moe import fused_experts_impl
    T, H, I, E, K = 32, 1024, 512, 8, 2
    w13, w2 = synthetic.moe_bf16_weights(E, H, I, seed=0)
    x = synthetic.activations(T, H, seed=1)
    logits = synthetic.router_logits(T, E, seed=2)
    w, ids, _ = fused_topk(x, logits, K, True)
    w_ref, ids_ref = oroute.topk_softmax(logits.cpu().numpy(), K, True)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_allclose(w.cpu().numpy(), w_ref, rtol=1e-6, atol=1e-7)
    out = fused_experts_impl(x, w13, w2, w, ids, path=path)
    ref = omoe.fused_experts_bf16(x.float().cpu().numpy(), w13.float().cpu().numpy(),
                                  w2.float().cpu().numpy(), w.cpu().numpy(), ids.cpu().numpy())
    _check(out, ref)


# ------------------------------------------------------------------ C2 -----
@pytest.mark.parametrize("hot", [0, 8])
def test_c2_bf16_qwen3_t8192(hot):
    """C2 at T=8192 (the bf16-MFMA-bound point), uniform and skewed logits."""
    from vllm_musa_amd import fused_topk, synthetic
    from vllm_musa_amd.fused_moe import fused_experts_impl
    T, E, H, I = 8192, 128, 2048, 768
    w13, w2 = synthetic.moe_bf16_weights(E, H, I, 4000)
    x = synthetic.activations(T, H, 4001 + T)
    logits = synthetic.router_logits(T, E, 4002 + T, hot=hot)
    w, ids, _ = fused_topk(x, logits, 8, True)
    _, ids_ref = oroute.topk_softmax(logits.cpu().numpy(), 8, True)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    out = fused_experts_impl(x, w13, w2, w, ids)
    rows = _sample_rows(T, ids, 8, seed=T + hot)
    _check(out[torch.from_numpy(rows).to(DEV)], _oracle_bf16_rows(x, w13, w2, w, ids, rows))


# ------------------------------------------------------------------ C3 -----
@pytest.fixture(scope="module")
def dsv3_stack():
    from vllm_musa_amd import synthetic
    stack = synthetic.moe_fp8_weights(256, 7168, 2048, seed=3000)
    yield stack
    del stack
    torch.cuda.empty_cache()


@pytest.mark.parametrize("T", [257, 4096])
def test_c3_dsv3_layer_as_benchmarked(dsv3_stack, T):
    """The DeepSeek-V3 step exactly as bench.py builds and times it: same
    seeds, grouped_topk on the GPU, fused_experts_impl with path auto (the
    grouped GEMMs at these T; at T=4096 32 align workgroups, hot experts over
    several 128-route blocks and the XCD tile split over ~200 experts)."""
    from vllm_musa_amd import grouped_topk, synthetic
    from vllm_musa_amd.fused_moe import fused_experts_impl
    E, H = 256, 7168
    w13, s13, w2, s2 = dsv3_stack
    x = synthetic.activations(T, H, 3000 + 10 * T + 1)
    logits = synthetic.router_logits(T, E, 3000 + 10 * T + 2)
    bias = synthetic.score_bias(E, 3000 + 3)
    w, ids = grouped_topk(x, logits, 8, True, 8, 4, "sigmoid", 2.5, bias)
    w_ref, ids_ref = oroute.grouped_topk(logits.cpu().numpy(), 8, True, 8, 4, "sigmoid", 2.5,
                                         bias.cpu().numpy())
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    out = fused_experts_impl(x, w13, w2, w, ids, use_fp8_w8a8=True, w1_scale=s13, w2_scale=s2,
                             block_shape=[128, 128])
    assert torch.equal(out, fused_experts_impl(x, w13, w2, w, ids, use_fp8_w8a8=True,
                                               w1_scale=s13, w2_scale=s2, block_shape=[128, 128]))
    rows = _sample_rows(T, ids, 6, seed=T)
    _check(out[torch.from_numpy(rows).to(DEV)],
           _oracle_fp8_rows(x, w13, s13, w2, s2, w, ids, rows))


# ------------------------------------------------------------------ C4 -----
def test_c4_w4afp8_t4096():
    """C4 at T=4096 (the fp8-MFMA-bound point of the w4afp8 layer)."""
    from vllm_musa_amd import fused_topk, synthetic, w4afp8_moe
    T, E, H, I = 4096, 128, 4096, 1536
    w13, w2, s13, s2 = synthetic.moe_w4a8_weights(E, H, I, 5000)
    x = synthetic.activations(T, H, 5001 + T)
    logits = synthetic.router_logits(T, E, 5002 + T)
    w, ids, _ = fused_topk(x, logits, 8, True)
    out = w4afp8_moe(x, w13, w2, s13, s2, w, ids)
    rows = _sample_rows(T, ids, 6, seed=T + 1)
    cids, sel = _compact(ids.cpu().numpy()[rows], E)
    ref = ow4.w4afp8_moe(x.float().cpu().numpy()[rows], w13.index_select(0, sel).cpu().numpy(),
                         w2.index_select(0, sel).cpu().numpy(),
                         s13.index_select(0, sel).float().cpu().numpy(),
                         s2.index_select(0, sel).float().cpu().numpy(), w.cpu().numpy()[rows], cids)
    _check(out[torch.from_numpy(rows).to(DEV)], ref)


# ------------------------------------------- reference top-k construction --
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("renormalize", [False, True])
def test_topk_reference_construction(dtype, renormalize):
    """The reference's own top-k test input (tests/jit_kernel/
    test_csrc_jit_kernels.py:463-513): a permuted linspace(-4, 4, 128) with
    0.001 * row offsets, a 0.01 * randn correction bias, top-8 over 7 rows, in
    f32 / f16 / bf16.  Ids bit-exact against the oracle (and against torch.topk,
    the reference's own check: the construction has no ties), weights against
    the oracle and within the reference's atol / rtol 3e-3 of its torch ref."""
    from vllm_musa_amd import topk_sigmoid, topk_softmax
    g = torch.Generator().manual_seed(789)
    rows, experts, k = 7, 128, 8
    values = torch.linspace(-4.0, 4.0, experts, dtype=torch.float32)
    perm = torch.randperm(experts, generator=g)
    base = torch.empty(experts, dtype=torch.float32)
    base[perm] = values
    offsets = torch.arange(rows, dtype=torch.float32).unsqueeze(1)
    gating = (base.unsqueeze(0) + offsets * 0.001).to(dtype)
    bias = torch.randn(experts, generator=g, dtype=torch.float32) * 0.01
    gf = gating.float().numpy()
    for fn, kind, use_bias in ((topk_softmax, "softmax", False), (topk_softmax, "softmax", True),
                               (topk_sigmoid, "sigmoid", True)):
        w = torch.empty(rows, k, dtype=torch.float32, device=DEV)
        ids = torch.empty(rows, k, dtype=torch.int32, device=DEV)
        b = bias.to(DEV) if use_bias else None
        fn(w, ids, gating.to(DEV), renormalize, correction_bias=b)
        if kind == "softmax":
            w_ref, ids_ref = oroute.topk_softmax(gf, k, renormalize,
                                                 bias.numpy() if use_bias else None)
            logits = gating.float() + (bias.unsqueeze(0) if use_bias else 0)
            scores = torch.softmax(logits, dim=-1)
            _, t_ids = torch.topk(logits, k, dim=-1)
        else:
            w_ref, ids_ref = oroute.topk_sigmoid(gf, k, renormalize, bias.numpy())
            scores = torch.sigmoid(gating.float())
            _, t_ids = torch.topk(scores + bias.unsqueeze(0), k, dim=-1)
        np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
        np.testing.assert_array_equal(ids.cpu().numpy(), t_ids.int().numpy())
        t_w = scores.gather(1, t_ids)
        if renormalize:
            t_w = t_w / t_w.sum(dim=-1, keepdim=True)
        np.testing.assert_allclose(w.cpu().numpy(), w_ref, rtol=1e-5, atol=1e-6)
        torch.testing.assert_close(w.cpu(), t_w.float(), atol=3e-3, rtol=3e-3)


# ------------------------------------------------ router weight on input --
def _fp8_case(T, E, H, I, K, seed):
    from vllm_musa_amd import synthetic
    w13, s13, w2, s2 = synthetic.moe_fp8_weights(E, H, I, seed)
    x = synthetic.activations(T, H, seed + 1)
    gen = torch.Generator().manual_seed(seed + 2)
    ids = torch.stack([torch.randperm(E, generator=gen)[:K] for _ in range(T)]).to(torch.int32)
    w = torch.rand(T, K, generator=gen) * 0.9 + 0.1
    return x, w13, s13, w2, s2, w.to(DEV), ids.to(DEV)


@pytest.mark.parametrize("path", ["gemv", "gemm"])
@pytest.mark.parametrize("T,topk", [(40, 1), (40, 4), (1, 4)])
def test_fp8_router_weight_on_input(path, T, topk):
    """apply_router_weight_on_input: the routed weight multiplies the W13
    output before the SiLU, y is unweighted (oracle restates the reference's
    mul_routed_weight on the first GEMV).  T=1 on the decode kernels takes
    the direct route slots."""
    from vllm_musa_amd.fused_moe import fused_experts_impl
    x, w13, s13, w2, s2, w, ids = _fp8_case(T, 16, 1024, 512, topk, seed=700 + topk + T)
    out = fused_experts_impl(x, w13, w2, w, ids, apply_router_weight_on_input=True,
                             use_fp8_w8a8=True, w1_scale=s13, w2_scale=s2, block_shape=[128, 128],
                             path=path)
    rows = np.arange(T)
    cids, sel = _compact(ids.cpu().numpy(), 16)
    u8 = lambda t: t.view(torch.uint8).index_select(0, sel).cpu().numpy()
    f32 = lambda t: t.index_select(0, sel).cpu().numpy()
    ref = omoe.fused_experts_fp8(x.float().cpu().numpy()[rows], u8(w13), f32(s13), u8(w2), f32(s2),
                                 w.cpu().numpy(), cids, apply_router_weight_on_input=True)
    _check(out, ref)
    default = fused_experts_impl(x, w13, w2, w, ids, use_fp8_w8a8=True, w1_scale=s13,
                                 w2_scale=s2, block_shape=[128, 128], path=path)
    assert not torch.equal(out, default)


@pytest.mark.parametrize("path", ["gemv", "gemm"])
@pytest.mark.parametrize("T", [33, 1])
def test_bf16_router_weight_on_input(path, T):
    from vllm_musa_amd import synthetic
    from vllm_musa_amd.fused_moe import fused_experts_impl
    E, H, I, K = 8, 512, 256, 2
    w13, w2 = synthetic.moe_bf16_weights(E, H, I, 710)
    x = synthetic.activations(T, H, 711)
    gen = torch.Generator().manual_seed(712)
    ids = torch.stack([torch.randperm(E, generator=gen)[:K] for _ in range(T)]).to(torch.int32)
    w = (torch.rand(T, K, generator=gen) * 0.9 + 0.1).to(DEV)
    out = fused_experts_impl(x, w13, w2, w, ids.to(DEV), apply_router_weight_on_input=True,
                             path=path)
    ref = omoe.fused_experts_bf16(x.float().cpu().numpy(), w13.float().cpu().numpy(),
                                  w2.float().cpu().numpy(), w.cpu().numpy(), ids.numpy(),
                                  apply_router_weight_on_input=True)
    _check(out, ref)


# ---------------------------------------- per-tensor / per-expert scales --
@pytest.mark.parametrize("layout", ["0d", "one", "E", "E1"])
@pytest.mark.parametrize("path", ["gemv", "gemm"])
def test_fp8_per_tensor_scales_expand(layout, path):
    """Per-tensor (0-d, [1]) and per-expert ([E], [E, 1]) weight scales with
    block_shape None: expanded to the 128x128 grid (the reference's
    _maybe_expand_fp8_moe_per_tensor_scale), the layer equals the block-scale
    layer on the expanded scales bit for bit and matches the oracle."""
    from vllm_musa_amd import synthetic
    from vllm_musa_amd.fused_moe import fp8_moe_scale_layout_is_supported, fused_experts_impl
    E, H, I, T = 8, 512, 256, 24
    gen = torch.Generator(device=DEV).manual_seed(720)
    w13 = (torch.randn(E, 2 * I, H, generator=gen, device=DEV) * 64).clamp(-448, 448).to(torch.float8_e4m3fn)
    w2 = (torch.randn(E, H, I, generator=gen, device=DEV) * 64).clamp(-448, 448).to(torch.float8_e4m3fn)
    per_e13 = torch.rand(E, generator=gen, device=DEV) * 1e-4 + 1e-4
    per_e2 = torch.rand(E, generator=gen, device=DEV) * 1e-4 + 1e-4
    if layout == "0d":
        a, b = per_e13[0].clone(), per_e2[0].clone()
        e13, e2 = per_e13[:1].expand(E), per_e2[:1].expand(E)
    elif layout == "one":
        a, b = per_e13[:1].clone(), per_e2[:1].clone()
        e13, e2 = per_e13[:1].expand(E), per_e2[:1].expand(E)
    elif layout == "E":
        a, b, e13, e2 = per_e13, per_e2, per_e13, per_e2
    else:
        a, b = per_e13[:, None].contiguous(), per_e2[:, None].contiguous()
        e13, e2 = per_e13, per_e2
    assert fp8_moe_scale_layout_is_supported(a, w13) and fp8_moe_scale_layout_is_supported(b, w2)
    s13 = e13.reshape(E, 1, 1).expand(E, 2 * I // 128, H // 128).contiguous()
    s2 = e2.reshape(E, 1, 1).expand(E, H // 128, I // 128).contiguous()
    x = synthetic.activations(T, H, 721)
    g = torch.Generator().manual_seed(722)
    ids = torch.stack([torch.randperm(E, generator=g)[:4] for _ in range(T)]).to(torch.int32).to(DEV)
    w = torch.softmax(torch.randn(T, 4, generator=g), -1).to(DEV)
    out = fused_experts_impl(x, w13, w2, w, ids, use_fp8_w8a8=True, w1_scale=a, w2_scale=b,
                             block_shape=None, path=path)
    blk = fused_experts_impl(x, w13, w2, w, ids, use_fp8_w8a8=True, w1_scale=s13, w2_scale=s2,
                             block_shape=[128, 128], path=path)
    assert torch.equal(out, blk)
    ref = omoe.fused_experts_fp8(x.float().cpu().numpy(), w13.view(torch.uint8).cpu().numpy(),
                                 s13.cpu().numpy(), w2.view(torch.uint8).cpu().numpy(),
                                 s2.cpu().numpy(), w.cpu().numpy(), ids.cpu().numpy())
    _check(out, ref)


def test_fp8_scale_layout_guard():
    from vllm_musa_amd.fused_moe import fp8_moe_scale_layout_is_supported
    w = torch.empty(4, 256, 512, dtype=torch.float8_e4m3fn, device=DEV)
    ok = [torch.ones((), device=DEV), torch.ones(1, device=DEV), torch.ones(4, device=DEV),
          torch.ones(4, 1, device=DEV), torch.ones(4, 2, 4, device=DEV)]
    bad = [None, torch.ones(4, 4, 8, device=DEV),  # 64-wide grid
           torch.ones(4, device=DEV, dtype=torch.float16), torch.ones(4, 4, 2, device=DEV)[:, :2, :],
           torch.ones(3, device=DEV)]
    assert all(fp8_moe_scale_layout_is_supported(s, w) for s in ok)
    assert not any(fp8_moe_scale_layout_is_supported(s, w) for s in bad)


# ------------------------------------------------------ out-of-range ids --
@pytest.mark.parametrize("path", ["gemv", "gemm"])
@pytest.mark.parametrize("mapped", [False, True])
def test_fp8_layer_drops_out_of_range_ids(path, mapped, monkeypatch):
    """A route whose (local) expert id is >= E is dropped by the alignment;
    the combine skips its slot too (its rows were never written: the
    workspace starts as NaN bytes here), so the layer equals the one with
    that route's id set to -1."""
    from vllm_musa_amd.fused_moe import fused_experts_impl
    x, w13, s13, w2, s2, w, ids = _fp8_case(20, 8, 512, 256, 4, seed=730)
    real_empty = torch.empty

    def poisoned(*args, **kwargs):
        t = real_empty(*args, **kwargs)
        if t.is_cuda:
            t.view(torch.uint8).fill_(0xFF)
        return t

    monkeypatch.setattr(torch, "empty", poisoned)
    bad = ids.clone()
    emap = None
    if mapped:  # global ids 0..9 -> local 0..7, globals 8 and 9 map past the stack
        emap = torch.arange(10, dtype=torch.int32, device=DEV)
        bad[3, 1] = 9
    else:
        bad[3, 1] = 8
    dropped = ids.clone()
    dropped[3, 1] = -1
    kw = dict(use_fp8_w8a8=True, w1_scale=s13, w2_scale=s2, block_shape=[128, 128], path=path)
    ref = fused_experts_impl(x, w13, w2, w, dropped, **kw)
    for _ in range(2):  # the second call sees the first call's workspace contents
        assert torch.equal(fused_experts_impl(x, w13, w2, w, bad, expert_map=emap, **kw), ref)
