"""GPU parity of the fused fp8 block MoE layer (decode GEMV path and prefill
grouped-GEMM path) against the oracle on identical seeded inputs.

Tolerance (the path's bar for bf16/fp8 outputs): rel-L2 <= 1e-2 and
max-abs <= 2e-2 * max|ref|."""
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


def _routing(T, E, K, seed, hot=None):
    g = torch.Generator().manual_seed(seed)
    if hot is None:
        ids = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)])
    else:  # every token takes the hot expert plus K-1 distinct others
        others = torch.tensor([e for e in range(E) if e != hot])
        ids = torch.stack([torch.cat([torch.tensor([hot]),
                                      others[torch.randperm(E - 1, generator=g)[:K - 1]]])
                           for _ in range(T)])
    ids = ids.to(torch.int32)
    w = torch.softmax(torch.randn(T, K, generator=g), dim=-1)
    return w, ids


def _case(T, E, H, I, K, seed, hot=None):
    from vllm_musa_amd import synthetic
    w13, s13, w2, s2 = synthetic.moe_fp8_weights(E, H, I, seed)
    x = synthetic.activations(T, H, seed + 1)
    w, ids = _routing(T, E, K, seed + 2, hot)
    return x, w13, s13, w2, s2, w.to(DEV), ids.to(DEV)


def _oracle(x, w13, s13, w2, s2, w, ids, emap=None):
    """Oracle on the experts the routing touches (only those weights are copied
    to the host); ids are remapped onto the compact expert stack."""
    ids_np = ids.cpu().numpy()
    loc = omoe.local_experts(ids_np, None if emap is None else emap.cpu().numpy(), w13.shape[0])
    used = np.unique(loc[loc >= 0])
    remap = np.full(w13.shape[0], -1, np.int64)
    remap[used] = np.arange(used.size)
    cids = np.where(loc >= 0, remap[np.maximum(loc, 0)], -1).astype(np.int32)
    sel = torch.from_numpy(used).to(w13.device)
    u8 = lambda t: t.view(torch.uint8).index_select(0, sel).cpu().numpy()
    f32 = lambda t: t.index_select(0, sel).cpu().numpy()
    return omoe.fused_experts_fp8(x.float().cpu().numpy(), u8(w13), f32(s13), u8(w2), f32(s2),
                                  w.cpu().numpy(), cids)


def _run(x, w13, s13, w2, s2, w, ids, path, emap=None, limit=None):
    from vllm_musa_amd.fused_moe import fused_experts_impl
    return fused_experts_impl(x, w13, w2, w, ids, use_fp8_w8a8=True, w1_scale=s13, w2_scale=s2,
                              block_shape=[128, 128], expert_map=emap, gemm1_clamp_limit=limit,
                              path=path)


@pytest.mark.parametrize("path", ["gemv", "gemm"])
@pytest.mark.parametrize("T", [1, 3, 16, 64, 257])
def test_fp8_moe_small_vs_oracle(T, path):
    case = _case(T, 16, 1024, 512, 4, seed=100 + T)
    out = _run(*case, path=path)
    _check(out, _oracle(*case))


@pytest.mark.parametrize("path", ["gemv", "gemm"])
def test_fp8_moe_hot_expert_multi_block(path):
    # 600 routes on one expert: several 16-route and 128-route blocks
    case = _case(600, 16, 1024, 256, 4, seed=7, hot=3)
    out = _run(*case, path=path)
    _check(out, _oracle(*case))


def test_fp8_moe_256_route_blocks_vs_oracle():
    """From 128 routes per expert the grouped GEMMs take 256-route blocks
    (here 1200 routes on 8 experts); H = 640 leaves the last 256-row W2 tile
    half outside the output and I = 384 gives three 128-column W13 tiles."""
    case = _case(600, 8, 640, 384, 2, seed=71)
    out = _run(*case, path="gemm")
    _check(out, _oracle(*case))


@pytest.mark.parametrize("variant", ["hot", "expert_map", "limit"])
def test_fp8_moe_256_route_blocks_match_128(variant):
    """256- and 128-route blocks give the same bits: every route's row sees the
    same K order and roundings whatever tile it lands in.  A hot expert (1000
    routes: four 256-route blocks), an expert map with dropped routes, and the
    clamped SwiGLU."""
    from vllm_musa_amd.fused_moe import Fp8MoeStages
    emap, limit = None, None
    if variant == "hot":
        x, w13, s13, w2, s2, w, ids = _case(1000, 8, 512, 256, 2, seed=81, hot=5)
    else:
        x, w13, s13, w2, s2, w, ids = _case(700, 8, 768, 256, 2, seed=82)
    if variant == "expert_map":
        g = torch.Generator().manual_seed(83)
        ids = torch.stack([torch.randperm(12, generator=g)[:2] for _ in range(700)]).to(torch.int32).to(DEV)
        emap = torch.full((12,), -1, dtype=torch.int32)
        emap[4:] = torch.arange(8, dtype=torch.int32)
        emap = emap.to(DEV)
    if variant == "limit":
        limit = 7.0
    big = Fp8MoeStages(x, w13, s13, w2, s2, w, ids, path="gemm", expert_map=emap, swiglu_limit=limit)
    assert big.block_m == 256
    small = Fp8MoeStages(x, w13, s13, w2, s2, w, ids, path="gemm", expert_map=emap, swiglu_limit=limit,
                         block_m=128)
    a = big.run().clone()
    b = small.run()
    assert torch.equal(a, b)
    assert torch.equal(_run(x, w13, s13, w2, s2, w, ids, "gemm", emap=emap, limit=limit), a)


@pytest.mark.parametrize("path", ["gemv", "gemm"])
def test_fp8_moe_expert_map(path):
    x, w13, s13, w2, s2, w, ids = _case(40, 8, 512, 256, 4, seed=11)
    # global ids 0..15; this rank owns global experts 8..15 as local 0..7
    g = torch.Generator().manual_seed(12)
    gids = torch.stack([torch.randperm(16, generator=g)[:4] for _ in range(40)]).to(torch.int32).to(DEV)
    emap = torch.full((16,), -1, dtype=torch.int32)
    emap[8:] = torch.arange(8, dtype=torch.int32)
    emap = emap.to(DEV)
    out = _run(x, w13, s13, w2, s2, w, gids, path, emap=emap)
    _check(out, _oracle(x, w13, s13, w2, s2, w, gids, emap=emap))


@pytest.mark.parametrize("T,K,variant", [(1, 4, "plain"), (1, 8, "plain"), (1, 8, "expert_map"),
                                         (1, 4, "limit"), (1, 8, "duplicate"), (1, 4, "h640"),
                                         (2, 8, "plain")])
def test_fp8_moe_direct_decode_matches_grouped(T, K, variant):
    """One token: the fused decode call gives every route its own GEMV slot
    (no alignment) and sums the top-k inside the W2 launch; its output equals
    the stage-by-stage grouped decode path (alignment, GEMVs over the active
    experts, moe_sum) bit for bit, and the oracle.  Variants: an expert map
    that drops routes, the clamped SwiGLU, a token that names one expert
    twice; H = 640 (five scale blocks per row: scales read one at a time, x
    quantised by its own launch); T=2 takes the grouped slots in both."""
    from vllm_musa_amd.fused_moe import Fp8MoeStages
    E = 16
    H = 640 if variant == "h640" else 1024
    x, w13, s13, w2, s2, w, ids = _case(T, E, H, 512, K, seed=131 + 10 * T + K)
    emap, limit = None, None
    if variant == "expert_map":  # global ids 0..23, local experts = global 8..23
        g = torch.Generator().manual_seed(137)
        ids = torch.stack([torch.randperm(24, generator=g)[:K] for _ in range(T)]).to(torch.int32).to(DEV)
        emap = torch.full((24,), -1, dtype=torch.int32)
        emap[8:] = torch.arange(16, dtype=torch.int32)
        emap = emap.to(DEV)
    if variant == "limit":
        limit = 7.0
    if variant == "duplicate":
        ids[0, 1] = ids[0, 0]
    st = Fp8MoeStages(x, w13, s13, w2, s2, w, ids, path="gemv", expert_map=emap, swiglu_limit=limit)
    assert st.block_m == 16
    grouped = st.run().clone()
    direct = _run(x, w13, s13, w2, s2, w, ids, "gemv", emap=emap, limit=limit)
    assert torch.equal(direct, grouped)
    if limit is None:
        _check(direct, _oracle(x, w13, s13, w2, s2, w, ids, emap=emap))


def test_fp8_moe_direct_decode_dsv3_t1():
    """The DeepSeek-V3 layer at T=1 (8 routes, grouped sigmoid routing): the
    direct decode call equals the grouped decode stages bit for bit."""
    from vllm_musa_amd import grouped_topk, synthetic
    from vllm_musa_amd.fused_moe import Fp8MoeStages
    E, H, I = 256, 7168, 2048
    w13, s13, w2, s2 = synthetic.moe_fp8_weights(E, H, I, seed=3000)
    x = synthetic.activations(1, H, 3101)
    logits = synthetic.router_logits(1, E, 3102)
    bias = synthetic.score_bias(E, 3003)
    w, ids = grouped_topk(x, logits, 8, True, 8, 4, "sigmoid", 2.5, bias)
    grouped = Fp8MoeStages(x, w13, s13, w2, s2, w, ids, path="gemv").run().clone()
    assert torch.equal(_run(x, w13, s13, w2, s2, w, ids, "auto"), grouped)


def test_fp8_moe_paths_agree():
    case = _case(48, 32, 2048, 768, 8, seed=21)
    a = _run(*case, path="gemv").float()
    b = _run(*case, path="gemm").float()
    rl2 = (torch.linalg.norm(a - b) / torch.linalg.norm(b)).item()
    assert rl2 < 5e-3, rl2


def test_fp8_moe_deterministic():
    case = _case(200, 16, 1024, 512, 4, seed=31)
    for path in ("gemv", "gemm"):
        a = _run(*case, path=path)
        b = _run(*case, path=path)
        assert torch.equal(a, b)


@pytest.mark.parametrize("path", ["gemv", "gemm"])
def test_fp8_moe_dsv3_shape(path):
    """DeepSeek-V3 layer shape (E=256, H=7168, I=2048, grouped sigmoid routing,
    top-8) at T=2, checked against the oracle on every output."""
    from vllm_musa_amd import grouped_topk, synthetic
    T, E, H, I = 2, 256, 7168, 2048
    w13, s13, w2, s2 = synthetic.moe_fp8_weights(E, H, I, seed=3000)
    x = synthetic.activations(T, H, 3001)
    logits = synthetic.router_logits(T, E, 3002)
    bias = synthetic.score_bias(E, 3003)
    w, ids = grouped_topk(x, logits, 8, True, 8, 4, "sigmoid", 2.5, bias)
    w_ref, ids_ref = oroute.grouped_topk(logits.cpu().numpy(), 8, True, 8, 4, "sigmoid", 2.5,
                                         bias.cpu().numpy())
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    out = _run(x, w13, s13, w2, s2, w, ids, path)
    _check(out, _oracle(x, w13, s13, w2, s2, w, ids))


def test_fp8_moe_empty_and_inplace():
    from vllm_musa_amd.fused_moe import fused_experts_impl
    x, w13, s13, w2, s2, w, ids = _case(5, 8, 512, 256, 2, seed=41)
    empty = fused_experts_impl(x[:0], w13, w2, w[:0], ids[:0], use_fp8_w8a8=True, w1_scale=s13,
                               w2_scale=s2, block_shape=[128, 128])
    assert empty.shape == (0, 512)
    ref = _run(x, w13, s13, w2, s2, w, ids, "auto")
    xi = x.clone()
    got = fused_experts_impl(xi, w13, w2, w, ids, use_fp8_w8a8=True, w1_scale=s13, w2_scale=s2,
                             block_shape=[128, 128], inplace=True)
    assert got.data_ptr() == xi.data_ptr() and torch.equal(got, ref)


@pytest.mark.parametrize("T", [33, 1])
def test_fp8_moe_poisoned_workspace(monkeypatch, T):
    """Workspace and outputs start as NaN bytes: every value the layer reads
    must have been written by it (T=1: the direct decode route slots, with an
    expert map that drops some routes, whose partials are never written)."""
    case = _case(T, 16, 1024, 512, 4, seed=51)
    emap = None
    if T == 1:  # global ids 0..23, local experts = global 8..23
        g = torch.Generator().manual_seed(52)
        ids = torch.stack([torch.randperm(24, generator=g)[:4] for _ in range(T)]).to(torch.int32).to(DEV)
        emap = torch.full((24,), -1, dtype=torch.int32)
        emap[8:] = torch.arange(16, dtype=torch.int32)
        emap = emap.to(DEV)
        case = case[:6] + (ids,)
    ref = _oracle(*case, emap=emap)
    real_empty = torch.empty

    def poisoned(*args, **kwargs):
        t = real_empty(*args, **kwargs)
        if t.is_cuda:
            t.view(torch.uint8).fill_(0xFF)
        return t

    monkeypatch.setattr(torch, "empty", poisoned)
    monkeypatch.setattr(torch, "empty_like", lambda t, **kw: poisoned(t.shape, dtype=t.dtype,
                                                                      device=t.device))
    for path in ("gemv", "gemm"):
        _check(_run(*case, path=path, emap=emap), ref)


@pytest.mark.parametrize("path", ["gemv", "gemm"])
def test_fp8_moe_stages_match_fused(path):
    """The stage-by-stage launches (quant, align, W13, W2, combine) give the
    fused call's output bit for bit."""
    from vllm_musa_amd.fused_moe import Fp8MoeStages
    case = _case(70, 16, 1024, 512, 4, seed=61)
    ref = _run(*case, path=path)
    x, w13, s13, w2, s2, w, ids = case
    st = Fp8MoeStages(x, w13, s13, w2, s2, w, ids, path=path)
    assert torch.equal(st.run(), ref)
    assert torch.equal(st.run(), ref)  # buffers reused on a second pass


@pytest.mark.parametrize("path,T", [("gemv", 24), ("gemm", 24), ("gemv", 1)])
def test_fp8_moe_graph_replay_matches_eager(path, T):
    """The layer captured in a HIP graph replays bit-identically to the eager
    call, across several replays with eager work and syncs in between and with
    the routing changed in place between replays (T=1: the direct decode route
    slots, x quantised inside the W13 launch, top-k sum inside the W2 launch)."""
    x, w13, s13, w2, s2, w, ids = _case(T, 16, 1024, 512, 4, seed=71)
    eager = _run(x, w13, s13, w2, s2, w, ids, path)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            _run(x, w13, s13, w2, s2, w, ids, path)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = _run(x, w13, s13, w2, s2, w, ids, path)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        _run(x, w13, s13, w2, s2, w, ids, path)  # eager work between replays
    ids2 = ids.flip(0).contiguous() if T > 1 else ids.flip(1).contiguous()
    ids.copy_(ids2)
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, _run(x, w13, s13, w2, s2, w, ids2, path))


@pytest.mark.parametrize("path", ["gemv", "gemm"])
def test_fp8_moe_padded_intermediate_is_exact(path):
    # The intermediate partition padded to the block grid with zero weights
    # (Fp8MoEMethod.create_weights / load_expert) gives the unpadded layer's
    # output bit for bit.
    import types
    from vllm_musa_amd.quant_methods import Fp8MoEMethod
    E, H, I0, I = 8, 512, 256, 384
    x, w13, s13, w2, s2, w, ids = _case(24, E, H, I0, 4, seed=91)
    m = Fp8MoEMethod()
    layer = types.SimpleNamespace()
    m.create_weights(layer, E, H, I, intermediate_size_unpadded=I0)
    for e in range(E):
        m.load_expert(layer, e, w13[e], s13[e], w2[e], s2[e])
    padded = _run(x, layer.w13_weight, layer.w13_weight_scale_inv, layer.w2_weight,
                  layer.w2_weight_scale_inv, w, ids, path)
    assert torch.equal(padded, _run(x, w13, s13, w2, s2, w, ids, path))
