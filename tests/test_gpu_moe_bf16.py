"""GPU parity of the bf16 fused MoE layer (decode GEMV and prefill grouped
GEMM on bf16 MFMA) against the oracle on identical seeded inputs, including
the Qwen3-30B-A3B-like shape (E=128, top-8 softmax renorm, H=2048, I=768) with
uniform and skewed (+2.0 on 8 hot experts) router logits.

Tolerance: rel-L2 <= 1e-2 and max-abs <= 2e-2 * max|ref|."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import moe as omoe
from oracle import routing as oroute

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


def _routing(T, E, K, seed):
    g = torch.Generator().manual_seed(seed)
    ids = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)]).to(torch.int32)
    w = torch.softmax(torch.randn(T, K, generator=g), dim=-1)
    return w.to(DEV), ids.to(DEV)


def _weights(E, H, I, seed):
    from vllm_musa_amd import synthetic
    return synthetic.moe_bf16_weights(E, H, I, seed)


def _oracle(x, w13, w2, w, ids, emap=None):
    ids_np = ids.cpu().numpy()
    loc = omoe.local_experts(ids_np, None if emap is None else emap.cpu().numpy(), w13.shape[0])
    used = np.unique(loc[loc >= 0])
    remap = np.full(w13.shape[0], -1, np.int64)
    remap[used] = np.arange(used.size)
    cids = np.where(loc >= 0, remap[np.maximum(loc, 0)], -1).astype(np.int32)
    sel = torch.from_numpy(used).to(w13.device)
    f32 = lambda t: t.index_select(0, sel).float().cpu().numpy()
    return omoe.fused_experts_bf16(x.float().cpu().numpy(), f32(w13), f32(w2), w.cpu().numpy(),
                                   cids)


def _run(x, w13, w2, w, ids, path, emap=None, limit=None):
    from vllm_musa_amd.fused_moe import fused_experts_impl
    return fused_experts_impl(x, w13, w2, w, ids, expert_map=emap, gemm1_clamp_limit=limit,
                              path=path)


@pytest.mark.parametrize("path", ["gemv", "gemm"])
@pytest.mark.parametrize("T", [1, 3, 16, 64, 257])
def test_bf16_moe_small_vs_oracle(T, path):
    from vllm_musa_amd import synthetic
    w13, w2 = _weights(16, 1024, 512, 200 + T)
    x = synthetic.activations(T, 1024, 201 + T)
    w, ids = _routing(T, 16, 4, 202 + T)
    _check(_run(x, w13, w2, w, ids, path), _oracle(x, w13, w2, w, ids))


@pytest.mark.parametrize("path", ["gemv", "gemm"])
@pytest.mark.parametrize("T,hot", [(5, 0), (300, 0), (300, 8)])
def test_bf16_moe_qwen3_shape(T, hot, path):
    """E=128, top-8 softmax-renorm routing on the GPU kernel, H=2048, I=768."""
    from vllm_musa_amd import fused_topk, synthetic
    E, H, I = 128, 2048, 768
    w13, w2 = _weights(E, H, I, 4000)
    x = synthetic.activations(T, H, 4001 + T)
    logits = synthetic.router_logits(T, E, 4002 + T, hot=hot)
    w, ids, _ = fused_topk(x, logits, 8, True)
    w_ref, ids_ref = oroute.topk_softmax(logits.cpu().numpy(), 8, True)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    _check(_run(x, w13, w2, w, ids, path), _oracle(x, w13, w2, w, ids))


@pytest.mark.parametrize("path", ["gemv", "gemm"])
def test_bf16_moe_expert_map(path):
    from vllm_musa_amd import synthetic
    w13, w2 = _weights(8, 512, 256, 13)
    x = synthetic.activations(40, 512, 14)
    g = torch.Generator().manual_seed(15)
    gids = torch.stack([torch.randperm(16, generator=g)[:4] for _ in range(40)]).to(torch.int32).to(DEV)
    w = torch.softmax(torch.randn(40, 4, generator=g), -1).to(DEV)
    emap = torch.full((16,), -1, dtype=torch.int32)
    emap[8:] = torch.arange(8, dtype=torch.int32)
    emap = emap.to(DEV)
    _check(_run(x, w13, w2, w, gids, path, emap=emap), _oracle(x, w13, w2, w, gids, emap=emap))


def test_bf16_moe_256_route_blocks_vs_oracle():
    """From 128 routes per expert the grouped GEMMs take 256-route blocks (1200
    routes on 8 experts); H = 640 leaves the last 256-row W2 tile half outside
    the output, I = 384 gives three 128-column W13 tiles."""
    from vllm_musa_amd import synthetic
    w13, w2 = _weights(8, 640, 384, 51)
    x = synthetic.activations(600, 640, 52)
    w, ids = _routing(600, 8, 2, 53)
    _check(_run(x, w13, w2, w, ids, "gemm"), _oracle(x, w13, w2, w, ids))


@pytest.mark.parametrize("variant", ["plain", "expert_map", "limit"])
def test_bf16_moe_256_route_blocks_match_128(variant):
    """256- and 128-route blocks give the same bits (each route's row sees the
    same K order and roundings in either tile)."""
    from vllm_musa_amd import synthetic
    from vllm_musa_amd.fused_moe import MoeStages
    w13, w2 = _weights(8, 512, 256, 61)
    x = synthetic.activations(700, 512, 62)
    w, ids = _routing(700, 8, 2, 63)
    emap, limit = None, None
    if variant == "expert_map":
        g = torch.Generator().manual_seed(64)
        ids = torch.stack([torch.randperm(12, generator=g)[:2] for _ in range(700)]).to(torch.int32).to(DEV)
        emap = torch.full((12,), -1, dtype=torch.int32)
        emap[4:] = torch.arange(8, dtype=torch.int32)
        emap = emap.to(DEV)
    if variant == "limit":
        limit = 7.0
    big = MoeStages(x, w13, None, w2, None, w, ids, path="gemm", expert_map=emap, swiglu_limit=limit)
    assert big.block_m == 256
    small = MoeStages(x, w13, None, w2, None, w, ids, path="gemm", expert_map=emap, swiglu_limit=limit,
                      block_m=128)
    a = big.run().clone()
    assert torch.equal(a, small.run())
    assert torch.equal(_run(x, w13, w2, w, ids, "gemm", emap=emap, limit=limit), a)


def test_bf16_moe_320_route_blocks_vs_oracle():
    """320-route blocks (bf16 only): 2048 routes on 8 experts (mean 256, so
    the fused call takes them); H = 640 leaves the last 256-row W2 tile half
    outside the output, I = 384 gives three 128-column W13 tiles."""
    from vllm_musa_amd import synthetic
    from vllm_musa_amd.fused_moe import MoeStages
    w13, w2 = _weights(8, 640, 384, 54)
    x = synthetic.activations(1024, 640, 55)
    w, ids = _routing(1024, 8, 2, 56)
    assert MoeStages(x, w13, None, w2, None, w, ids, path="gemm").block_m == 320
    _check(_run(x, w13, w2, w, ids, "gemm"), _oracle(x, w13, w2, w, ids))


@pytest.mark.parametrize("variant", ["plain", "hot", "expert_map", "limit"])
def test_bf16_moe_320_route_blocks_match_256_and_128(variant):
    """320-, 256- and 128-route blocks give the same bits.  A hot expert
    (half the routes: its blocks run full, the last one partly padding), an
    expert map with dropped routes, and the clamped SwiGLU."""
    from vllm_musa_amd import synthetic
    from vllm_musa_amd.fused_moe import MoeStages
    T, E = 1024, 8
    w13, w2 = _weights(E, 512, 256, 65)
    x = synthetic.activations(T, 512, 66)
    w, ids = _routing(T, E, 2, 67)
    emap, limit = None, None
    if variant == "hot":
        ids[: T // 2, 0] = 3
        ids[: T // 2, 1] = torch.where(ids[: T // 2, 1] == 3, 5, ids[: T // 2, 1])
    if variant == "expert_map":
        g = torch.Generator().manual_seed(68)
        ids = torch.stack([torch.randperm(12, generator=g)[:2] for _ in range(T)]).to(torch.int32).to(DEV)
        emap = torch.full((12,), -1, dtype=torch.int32)
        emap[4:] = torch.arange(8, dtype=torch.int32)
        emap = emap.to(DEV)
    if variant == "limit":
        limit = 7.0
    kw = dict(path="gemm", expert_map=emap, swiglu_limit=limit)
    outs = {}
    for bm in (320, 256, 128):
        st = MoeStages(x, w13, None, w2, None, w, ids, block_m=bm, **kw)
        outs[bm] = st.run().clone()
    assert torch.equal(outs[320], outs[256]) and torch.equal(outs[320], outs[128])
    assert torch.equal(_run(x, w13, w2, w, ids, "gemm", emap=emap, limit=limit), outs[320])


def test_fp8_stages_refuse_320_route_blocks():
    from vllm_musa_amd import synthetic
    from vllm_musa_amd.fused_moe import Fp8MoeStages
    w13, s13, w2, s2 = synthetic.moe_fp8_weights(8, 256, 128, 57)
    x = synthetic.activations(16, 256, 58)
    w, ids = _routing(16, 8, 2, 59)
    with pytest.raises(ValueError, match="block_m 320"):
        Fp8MoeStages(x, w13, s13, w2, s2, w, ids, path="gemm", block_m=320)


def test_bf16_moe_paths_agree_and_deterministic():
    from vllm_musa_amd import synthetic
    w13, w2 = _weights(32, 2048, 768, 21)
    x = synthetic.activations(48, 2048, 22)
    w, ids = _routing(48, 32, 8, 23)
    a = _run(x, w13, w2, w, ids, "gemv")
    b = _run(x, w13, w2, w, ids, "gemm")
    rl2 = (torch.linalg.norm(a.float() - b.float()) / torch.linalg.norm(b.float())).item()
    assert rl2 < 5e-3, rl2
    assert torch.equal(a, _run(x, w13, w2, w, ids, "gemv"))
    assert torch.equal(b, _run(x, w13, w2, w, ids, "gemm"))


@pytest.mark.parametrize("path", ["gemv", "gemm"])
def test_bf16_moe_stages_match_fused(path):
    from vllm_musa_amd import synthetic
    from vllm_musa_amd.fused_moe import MoeStages
    w13, w2 = _weights(16, 1024, 512, 31)
    x = synthetic.activations(70, 1024, 32)
    w, ids = _routing(70, 16, 4, 33)
    ref = _run(x, w13, w2, w, ids, path)
    st = MoeStages(x, w13, None, w2, None, w, ids, path=path)
    assert torch.equal(st.run(), ref)


@pytest.mark.parametrize("T,K,E,variant", [(1, 8, 16, "plain"), (1, 4, 16, "expert_map"),
                                           (1, 4, 16, "limit"), (1, 8, 64, "plain")])
def test_bf16_moe_direct_decode_matches_grouped(T, K, E, variant):
    """One token: the fused bf16 decode call gives every route its own GEMV
    slot and sums the top-k inside the W2 launch; bit for bit the grouped
    decode stages (alignment, GEMVs over the active experts, moe_sum)."""
    from vllm_musa_amd import synthetic
    from vllm_musa_amd.fused_moe import MoeStages
    w13, w2 = _weights(E, 1024, 512, 41 + T)
    x = synthetic.activations(T, 1024, 42 + T)
    w, ids = _routing(T, E, K, 43 + T)
    emap, limit = None, None
    if variant == "expert_map":  # global ids 0..23, local experts = global 8..23
        g = torch.Generator().manual_seed(44)
        ids = torch.stack([torch.randperm(24, generator=g)[:K] for _ in range(T)]).to(torch.int32).to(DEV)
        emap = torch.full((24,), -1, dtype=torch.int32)
        emap[8:] = torch.arange(16, dtype=torch.int32)
        emap = emap.to(DEV)
    if variant == "limit":
        limit = 7.0
    st = MoeStages(x, w13, None, w2, None, w, ids, path="gemv", expert_map=emap, swiglu_limit=limit)
    grouped = st.run().clone()
    direct = _run(x, w13, w2, w, ids, "gemv", emap=emap, limit=limit)
    assert torch.equal(direct, grouped)
    if limit is None:
        _check(direct, _oracle(x, w13, w2, w, ids, emap=emap))


def test_bf16_moe_rejects_scales():
    from vllm_musa_amd import synthetic
    from vllm_musa_amd.fused_moe import fused_experts_impl
    w13, w2 = _weights(4, 256, 128, 41)
    x = synthetic.activations(2, 256, 42)
    w, ids = _routing(2, 4, 2, 43)
    with pytest.raises(ValueError):
        fused_experts_impl(x, w13, w2, w, ids, w1_scale=torch.ones(1, device=DEV))


@pytest.mark.parametrize("H,I,K", [(2048, 256, 8), (1024, 512, 4)])
def test_bf16_direct_decode_fused_activation_split_counts(H, I, K):
    """One token: the W13 launch writes the bf16 activation itself, one
    workgroup per (route, 16 columns) holding 2 x splits waves (H=2048,
    I=256: 8 splits, 16 waves; H=1024, I=512: 4 splits), summed in split
    order in LDS.  H=1024, I=512, top-4 also splits the grouped W2 GEMV's K
    in two, which the one-token W2 + top-k sum follows at the split
    boundary.  Bit for bit the grouped decode stages, and the oracle."""
    from vllm_musa_amd import synthetic
    from vllm_musa_amd.fused_moe import MoeStages
    E = 16
    w13, w2 = _weights(E, H, I, 91 + H)
    x = synthetic.activations(1, H, 92)
    w, ids = _routing(1, E, K, 93)
    st = MoeStages(x, w13, None, w2, None, w, ids, path="gemv")
    grouped = st.run().clone()
    direct = _run(x, w13, w2, w, ids, "gemv")
    assert torch.equal(direct, grouped)
    _check(direct, _oracle(x, w13, w2, w, ids))


@pytest.mark.parametrize("variant", ["plain", "expert_map"])
def test_bf16_layer_two_launch_alignment_long_batch(variant):
    """The bf16 layer aligns its routes in two launches (chunk histograms in
    the workspace, then the placement); at 320,000 routes each workgroup
    places 2048 of them.  Bit for bit the stage-by-stage call, whose
    alignment is the one-launch standalone kernel; rows of the oracle."""
    from vllm_musa_amd import synthetic
    from vllm_musa_amd.fused_moe import MoeStages
    E, H, I, K, T = 16, 256, 128, 8, 40000
    w13, w2 = _weights(E, H, I, 94)
    x = synthetic.activations(T, H, 95)
    w, ids = _routing(T, E, K, 96)
    emap = None
    if variant == "expert_map":  # global ids 0..23, local experts = global 8..23; ids 0..7 dropped
        g = torch.Generator().manual_seed(97)
        ids = torch.stack([torch.randperm(24, generator=g)[:K] for _ in range(T)]).to(torch.int32).to(DEV)
        emap = torch.full((24,), -1, dtype=torch.int32)
        emap[8:] = torch.arange(16, dtype=torch.int32)
        emap = emap.to(DEV)
    from vllm_musa_amd.fused_moe import fused_experts_impl
    out = fused_experts_impl(x, w13, w2, w, ids, expert_map=emap, path="gemm", chunk_size=T)
    st = MoeStages(x, w13, None, w2, None, w, ids, path="gemm", expert_map=emap)
    assert torch.equal(out, st.run())
    rows = np.array([0, 1, 19999, 20000, T - 1])
    ref = _oracle(x[rows], w13, w2, w[rows], ids[rows], emap=emap)
    _check(out[rows], ref)
