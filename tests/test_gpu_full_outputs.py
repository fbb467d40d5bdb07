"""Every output at the benchmark sizes, not a sample.

Each large configuration is checked in full against an independent kernel
family of this package that computes the same value (bit for bit where the
two share the arithmetic, to the path's tolerance where they sum in another
order), and on a sample of rows against the oracle:

  C3  DeepSeek-V3 fp8 layer at T=4096 as benchmarked: 256-route blocks vs
      128-route blocks (bitwise, all 4096 rows); vs the decode GEMVs
      (tolerance, all rows); the CPU restatement on 32 rows, one from each
      256-route block of the most loaded expert.
  C1  dense block-fp8 GEMM at M=4096, all four shapes: the 256 x 256 tile vs
      the 128 x 256 tile (128-row calls without a workspace), bitwise, every
      output.
  C2  bf16 layer at T=8192: 256- vs 128-route blocks bitwise, grouped GEMMs
      vs decode GEMVs within tolerance, every row.
  C4  w4afp8 layer at T=4096: grouped GEMMs vs decode GEMVs, every row.
  align at block size 256 (what the 256-route kernels consume) and the fused
      align + 1x128 quantiser launch, on the benchmark's routing: bit-exact
      against the oracle, every output.
  apply_router_weight_on_input on the 256-route kernels (fp8 and bf16):
      against the oracle, and bitwise against the 128-route kernels.
  the fp8 256-route stages (x scales copied in route order by the W13 stage)
      bitwise against the fused call (x and a2 scales in route order), with
      an expert map, and against the oracle.

Tolerance (the path's bar for bf16/fp8 outputs): rel-L2 <= 1e-2 and
max-abs <= 2e-2 * max|ref|."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import align as oalign
from oracle import moe as omoe
from oracle import moe_torch as omt
from oracle import quant as oquant

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _close(a: torch.Tensor, b: torch.Tensor, rel_l2=1e-2, max_frac=2e-2):
    a64, b64 = a.double(), b.double()
    assert torch.isfinite(a64).all() and torch.isfinite(b64).all()
    err = a64 - b64
    rl2 = (err.norm() / b64.norm().clamp_min(1e-30)).item()
    assert rl2 <= rel_l2, f"rel-L2 {rl2}"
    assert err.abs().max().item() <= max_frac * b64.abs().max().item()
    return rl2


def _check_np(out: torch.Tensor, ref: np.ndarray):
    o = out.float().cpu().numpy().astype(np.float64)
    err = o - ref
    assert np.isfinite(o).all()
    assert np.linalg.norm(err) / np.linalg.norm(ref) <= 1e-2
    assert np.abs(err).max() <= 2e-2 * np.abs(ref).max()


# ------------------------------------------------------------------- C3 ---
@pytest.fixture(scope="module")
def dsv3():
    """The benchmark's DeepSeek-V3 layer at T=4096 (bench.py's seeds)."""
    from vllm_musa_amd import grouped_topk, synthetic
    T, E, H = 4096, 256, 7168
    w13, s13, w2, s2 = synthetic.moe_fp8_weights(E, H, 2048, seed=3000)
    x = synthetic.activations(T, H, 3000 + 10 * T + 1)
    logits = synthetic.router_logits(T, E, 3000 + 10 * T + 2)
    bias = synthetic.score_bias(E, 3000 + 3)
    w, ids = grouped_topk(x, logits, 8, True, 8, 4, "sigmoid", 2.5, bias)
    yield x, w13, s13, w2, s2, w, ids
    del w13, w2
    torch.cuda.empty_cache()


def test_c3_t4096_every_row(dsv3):
    from vllm_musa_amd.fused_moe import MoeStages, fused_experts_impl
    x, w13, s13, w2, s2, w, ids = dsv3
    kw = dict(use_fp8_w8a8=True, w1_scale=s13, w2_scale=s2, block_shape=[128, 128])
    out = fused_experts_impl(x, w13, w2, w, ids, **kw)            # 256-route blocks
    st = MoeStages(x, w13, s13, w2, s2, w, ids, path="gemm", block_m=128)
    assert torch.equal(out, st.run())                              # 128-route blocks
    gemv = fused_experts_impl(x, w13, w2, w, ids, path="gemv", **kw)
    _close(gemv, out)
    for t in range(0, 4096, 512):                                  # and per row block
        _close(gemv[t:t + 512], out[t:t + 512])
    # 32 rows on the CPU: one from each 256-route block of the hottest expert
    ids_np = ids.cpu().numpy()
    flat = ids_np.reshape(-1)
    hot = np.bincount(flat).argmax()
    routes = np.nonzero(flat == hot)[0]                            # route order = block order
    rows = {int(r) // 8 for r in routes[::256]} | {0, 4095}
    g = np.random.Generator(np.random.PCG64(4096))
    while len(rows) < 32:
        rows.add(int(g.integers(0, 4096)))
    rows = np.array(sorted(rows))
    assert len(routes) > 256
    used = np.unique(ids_np[rows])
    remap = np.full(256, -1, np.int64)
    remap[used] = np.arange(used.size)
    sel = torch.from_numpy(used).to(DEV)
    u8 = lambda t: t.index_select(0, sel).view(torch.uint8).cpu()
    ref = omt.fused_experts_fp8(x.float().cpu()[rows], u8(w13), s13.index_select(0, sel).cpu(),
                                u8(w2), s2.index_select(0, sel).cpu(), w.cpu()[rows],
                                torch.from_numpy(remap[ids_np[rows]]))
    _check_np(out[torch.from_numpy(rows).to(DEV)], ref.numpy().astype(np.float64))


def test_align_block_256_and_fused_quant_on_the_benchmark_routing(dsv3):
    """moe_align_block_size at block 256 (and 128, 16) on the T=4096 routing,
    and the fused align + 1x128 quantiser launch the fp8 layer runs: every
    output bit-exact against the oracle."""
    from vllm_musa_amd import _custom_ops as ops
    x, _, _, _, _, _, ids = dsv3
    ids_np = ids.cpu().numpy()
    E, numel = 256, ids.numel()
    q_ref, s_ref = oquant.group_quant_fp8(x.float().cpu().numpy())
    for bs in (256, 128, 16):
        cap = numel + E * (bs - 1)
        ref_sorted, ref_eids, ref_ntpp, ref_offs, _ = oalign.moe_align_block_size(ids_np, E, bs)
        for fused in (False, True):
            i32 = dict(dtype=torch.int32, device=DEV)
            srt = torch.full((cap,), -7, **i32)
            eids = torch.full((-(-cap // bs),), -7, **i32)
            ntpp = torch.empty(1, **i32)
            offs = torch.empty(E + 1, **i32)
            act = torch.empty(E, **i32)
            nact = torch.empty(1, **i32)
            if fused:
                xq = torch.empty_like(x, dtype=torch.float8_e4m3fn)
                xs = torch.empty(x.shape[0], x.shape[1] // 128, dtype=torch.float32, device=DEV)
                ops.moe_align_block_size_quant_fp8(ids, E, bs, srt, eids, ntpp, x, xq, xs,
                                                   expert_offsets=offs, active_experts=act,
                                                   num_active=nact)
                np.testing.assert_array_equal(xq.view(torch.uint8).cpu().numpy(), q_ref)
                np.testing.assert_array_equal(xs.cpu().numpy(), s_ref)
            else:
                ops.moe_align_block_size(ids, E, bs, srt, eids, ntpp, None, None, offs, act, nact)
            np.testing.assert_array_equal(srt.cpu().numpy(), ref_sorted)
            np.testing.assert_array_equal(eids.cpu().numpy(), ref_eids)
            assert int(ntpp.item()) == int(ref_ntpp[0])
            np.testing.assert_array_equal(offs.cpu().numpy(), ref_offs)
            live = np.unique(ids_np)
            assert int(nact.item()) == live.size
            np.testing.assert_array_equal(act.cpu().numpy()[:live.size], live)


# ------------------------------------------------------------------- C1 ---
@pytest.mark.parametrize("N,K", [(24576, 1536), (7168, 18432), (2112, 7168), (7168, 2048)])
def test_c1_m4096_big_tile_equals_128_row_tiles(N, K):
    """M = 4096 runs the 256 x 256 kernel; the same rows in 128-row calls
    without a workspace run the unsplit 128 x 256 kernel (the 256-row tile
    is not used below M = 512).  Both promote per 128-K block in the same
    order: every output bit for bit."""
    from vllm_musa_amd import synthetic
    from vllm_musa_amd._lib import call, ptr, stream_of
    from vllm_musa_amd.block_fp8 import w8a8_block_fp8_matmul
    from vllm_musa_amd.fp8_utils import per_token_group_quant_fp8
    M = 4096
    w, ws = synthetic.dense_fp8_weight(N, K, 77)
    xq, xs = per_token_group_quant_fp8(synthetic.activations(M, K, 78), 128)
    full = w8a8_block_fp8_matmul(xq, w, xs, ws, [128, 128])
    rows = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=DEV)
    for m0 in range(0, M, 128):
        a, s, c = xq[m0:m0 + 128], xs[m0:m0 + 128], rows[m0:m0 + 128]
        call("vmamd_w8a8_block_fp8_matmul", ptr(a), ptr(s), s.stride(0), s.stride(1), ptr(w), ptr(ws),
             ptr(c), 128, N, K, 128, 128, None, 0, stream_of(a))
    assert torch.equal(full, rows)


# ------------------------------------------------------------------- C2 ---
def test_c2_t8192_every_row():
    from vllm_musa_amd import fused_topk, synthetic
    from vllm_musa_amd.fused_moe import MoeStages, fused_experts_impl
    T, E, H, I = 8192, 128, 2048, 768
    w13, w2 = synthetic.moe_bf16_weights(E, H, I, 4000)
    x = synthetic.activations(T, H, 4001 + T)
    logits = synthetic.router_logits(T, E, 4002 + T)
    w, ids, _ = fused_topk(x, logits, 8, True)
    out = fused_experts_impl(x, w13, w2, w, ids)                   # 256-route blocks
    st = MoeStages(x, w13, None, w2, None, w, ids, path="gemm", block_m=128)
    assert torch.equal(out, st.run())
    gemv = fused_experts_impl(x, w13, w2, w, ids, path="gemv")
    _close(gemv, out)
    for t in range(0, T, 1024):
        _close(gemv[t:t + 1024], out[t:t + 1024])


# ------------------------------------------------------------------- C4 ---
def test_c4_t4096_every_row():
    from vllm_musa_amd import fused_topk, synthetic, w4afp8_moe
    T, E, H, I = 4096, 128, 4096, 1536
    w13, w2, s13, s2 = synthetic.moe_w4a8_weights(E, H, I, 5000)
    x = synthetic.activations(T, H, 5001 + T)
    logits = synthetic.router_logits(T, E, 5002 + T)
    w, ids, _ = fused_topk(x, logits, 8, True)
    out = w4afp8_moe(x, w13, w2, s13, s2, w, ids, path="gemm")
    gemv = w4afp8_moe(x, w13, w2, s13, s2, w, ids, path="gemv")
    _close(gemv, out)
    for t in range(0, T, 512):
        _close(gemv[t:t + 512], out[t:t + 512])


# ------------------------------------------- routed weight on the input ---
def _pad_experts(w13, w2, extra, s13=None, s2=None):
    """The stack with `extra` unused experts appended: the same routes then
    average fewer than 128 per expert, which selects the 128-route blocks."""
    pad = lambda t: torch.cat([t, torch.zeros((extra,) + tuple(t.shape[1:]), dtype=t.dtype,
                                              device=t.device)])
    return pad(w13), pad(w2), None if s13 is None else pad(s13), None if s2 is None else pad(s2)


def test_fp8_router_weight_on_input_256_route_blocks():
    """E = 8, top-2, T = 600: 1200 routes >= 128 * 8, so the grouped GEMMs take
    256-route blocks; with 8 more (unused) experts the same layer takes
    128-route blocks.  On-input routed weight: oracle, and equal bits."""
    from vllm_musa_amd import synthetic
    from vllm_musa_amd.fused_moe import fused_experts_impl
    E, H, I, T, K = 8, 1024, 256, 600, 2
    w13, s13, w2, s2 = synthetic.moe_fp8_weights(E, H, I, 800)
    x = synthetic.activations(T, H, 801)
    g = torch.Generator().manual_seed(802)
    ids = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)]).to(torch.int32).to(DEV)
    w = (torch.rand(T, K, generator=g) * 0.9 + 0.1).to(DEV)
    kw = dict(use_fp8_w8a8=True, block_shape=[128, 128], apply_router_weight_on_input=True, path="gemm")
    out = fused_experts_impl(x, w13, w2, w, ids, w1_scale=s13, w2_scale=s2, **kw)
    p13, p2, ps13, ps2 = _pad_experts(w13, w2, 8, s13, s2)
    assert torch.equal(out, fused_experts_impl(x, p13, p2, w, ids, w1_scale=ps13, w2_scale=ps2, **kw))
    ref = omoe.fused_experts_fp8(x.float().cpu().numpy(), w13.view(torch.uint8).cpu().numpy(),
                                 s13.cpu().numpy(), w2.view(torch.uint8).cpu().numpy(),
                                 s2.cpu().numpy(), w.cpu().numpy(), ids.cpu().numpy(),
                                 apply_router_weight_on_input=True)
    _check_np(out, ref)
    plain = fused_experts_impl(x, w13, w2, w, ids, w1_scale=s13, w2_scale=s2, use_fp8_w8a8=True,
                               block_shape=[128, 128], path="gemm")
    assert not torch.equal(out, plain)


def test_bf16_router_weight_on_input_256_route_blocks():
    from vllm_musa_amd import synthetic
    from vllm_musa_amd.fused_moe import fused_experts_impl
    E, H, I, T, K = 8, 512, 256, 600, 2
    w13, w2 = synthetic.moe_bf16_weights(E, H, I, 810)
    x = synthetic.activations(T, H, 811)
    g = torch.Generator().manual_seed(812)
    ids = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)]).to(torch.int32).to(DEV)
    w = (torch.rand(T, K, generator=g) * 0.9 + 0.1).to(DEV)
    out = fused_experts_impl(x, w13, w2, w, ids, apply_router_weight_on_input=True, path="gemm")
    p13, p2, _, _ = _pad_experts(w13, w2, 8)
    assert torch.equal(out, fused_experts_impl(x, p13, p2, w, ids, apply_router_weight_on_input=True,
                                               path="gemm"))
    ref = omoe.fused_experts_bf16(x.float().cpu().numpy(), w13.float().cpu().numpy(),
                                  w2.float().cpu().numpy(), w.cpu().numpy(), ids.cpu().numpy(),
                                  apply_router_weight_on_input=True)
    _check_np(out, ref)


# ----------------------------------------------------- chunked long batches --
def test_long_batch_runs_in_chunks():
    """T = 20000 > 16384 (the reference's chunk, fused_moe.py:2126-2128): the
    layer runs as a 16384-token chunk and a 3616-token one with one chunk's
    workspace; rows on both sides of the boundary against the oracle, and the
    whole output equal to running the two chunks as separate calls."""
    from vllm_musa_amd import synthetic
    from vllm_musa_amd.fused_moe import fused_experts_impl
    E, H, I, T, K = 8, 512, 256, 20000, 2
    w13, s13, w2, s2 = synthetic.moe_fp8_weights(E, H, I, 820)
    x = synthetic.activations(T, H, 821)
    g = torch.Generator().manual_seed(822)
    ids = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)]).to(torch.int32).to(DEV)
    w = torch.softmax(torch.randn(T, K, generator=g), -1).to(DEV)
    kw = dict(use_fp8_w8a8=True, w1_scale=s13, w2_scale=s2, block_shape=[128, 128])
    out = fused_experts_impl(x, w13, w2, w, ids, **kw)
    parts = torch.cat([fused_experts_impl(x[:16384], w13, w2, w[:16384], ids[:16384], **kw),
                       fused_experts_impl(x[16384:], w13, w2, w[16384:], ids[16384:], **kw)])
    assert torch.equal(out, parts)
    rows = np.array([0, 16382, 16383, 16384, 16385, T - 1])
    ref = omoe.fused_experts_fp8(x.float().cpu().numpy()[rows], w13.view(torch.uint8).cpu().numpy(),
                                 s13.cpu().numpy(), w2.view(torch.uint8).cpu().numpy(),
                                 s2.cpu().numpy(), w.cpu().numpy()[rows], ids.cpu().numpy()[rows])
    _check_np(out[torch.from_numpy(rows).to(DEV)], ref)
    small = fused_experts_impl(x, w13, w2, w, ids, chunk_size=5000, **kw)
    assert torch.equal(small, torch.cat([fused_experts_impl(x[c:c + 5000], w13, w2, w[c:c + 5000],
                                                            ids[c:c + 5000], **kw)
                                         for c in range(0, T, 5000)]))


def test_fp8_256_route_stages_equal_fused_with_expert_map():
    """The 256-route fp8 kernels read their activation scales in route order:
    the fused call copies the x scales (and has W13 write the a2 scales) so,
    the W13 stage entry point copies the x scales into its workspace and W2
    reads the a2 scales row by row.  Stages at block 256, the fused call and
    the oracle agree, with an expert map that drops a third of the routes and
    H / 128 = 12 scales per row."""
    from vllm_musa_amd import synthetic
    from vllm_musa_amd.fused_moe import MoeStages, fused_experts_impl
    E, H, I, T, K = 12, 1536, 256, 800, 2  # 1600 routes >= 128 * E: 256-route blocks
    w13, s13, w2, s2 = synthetic.moe_fp8_weights(E, H, I, 810)
    x = synthetic.activations(T, H, 811)
    g = torch.Generator().manual_seed(812)
    ids = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)]).to(torch.int32).to(DEV)
    w = (torch.rand(T, K, generator=g) * 0.9 + 0.1).to(DEV)
    emap = torch.tensor([i if i % 3 else -1 for i in range(E)], dtype=torch.int32, device=DEV)
    kw = dict(use_fp8_w8a8=True, block_shape=[128, 128], path="gemm", expert_map=emap)
    out = fused_experts_impl(x, w13, w2, w, ids, w1_scale=s13, w2_scale=s2, **kw)
    st = MoeStages(x, w13, s13, w2, s2, w, ids, path="gemm", expert_map=emap, block_m=256)
    assert st.block_m == 256
    assert torch.equal(out, st.run())
    ref = omoe.fused_experts_fp8(x.float().cpu().numpy(), w13.view(torch.uint8).cpu().numpy(),
                                 s13.cpu().numpy(), w2.view(torch.uint8).cpu().numpy(),
                                 s2.cpu().numpy(), w.cpu().numpy(), ids.cpu().numpy(),
                                 expert_map=emap.cpu().numpy())
    _check_np(out, ref)
