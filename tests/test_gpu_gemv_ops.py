"""GPU parity of the reference's native GEMV ops and the layer with their
numerics (W8A16: bf16 activations against dequantised fp8 weights, gate and
up in fp32 through the SwiGLU), against oracle/gemv.py on identical seeded
inputs.

Ops: musa_fused_gemv_moe / musa_fused_gemv with the reference's argument
order (vllm_musa/_custom_ops.py:28-158, csrc/musa/torch_bindings.cpp:11-21),
through the Python wrappers and through torch.ops._C_musa_ops.  Layer:
fused_experts_impl(path="native_gemv") and the dispatch that sends the
reference's calibrated decode shapes there.

Tolerance (the path's bar for bf16/fp8 outputs): rel-L2 <= 1e-2 and
max-abs <= 2e-2 * max|ref|; the reference's own bf16 GEMV test bar
(rtol = atol = 2e-2, tests/test_deepseek_v4_gemv_numeric.py:54) where its
case is mirrored."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import gemv as ogemv
from oracle import numerics as onum

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _check(out: torch.Tensor, ref: np.ndarray, rel_l2=1e-2, max_frac=2e-2):
    o = out.float().cpu().numpy().astype(np.float64).reshape(ref.shape)
    err = o - ref
    rl2 = np.linalg.norm(err) / max(np.linalg.norm(ref), 1e-30)
    assert np.isfinite(o).all()
    assert rl2 <= rel_l2, f"rel-L2 {rl2}"
    assert np.abs(err).max() <= max_frac * np.abs(ref).max(), f"max-abs {np.abs(err).max()}"
    return rl2


def _np(t: torch.Tensor) -> np.ndarray:
    """Host copy: e4m3 as its codes (uint8), bf16 / f32 as float32 values."""
    t = t.detach().cpu()
    if t.dtype == torch.float8_e4m3fn:
        return t.view(torch.uint8).numpy()
    return t.float().numpy()


def _routing(t, e, k, seed, dead=()):
    g = torch.Generator().manual_seed(seed)
    ids = torch.stack([torch.randperm(e, generator=g)[:k] for _ in range(t)]).to(torch.int32)
    for (r, c, v) in dead:
        ids[r, c] = v
    w = torch.softmax(torch.randn(t, k, generator=g), dim=-1)
    return w.to(DEV), ids.to(DEV)


def _compact(ids: torch.Tensor, e: int):
    """The experts a routing touches and the ids remapped onto that compact
    stack (dead ids stay dead), so the oracle copies only those weights."""
    flat = ids.cpu().numpy().reshape(-1).astype(np.int64)
    live = (flat >= 0) & (flat < e)
    used = np.unique(flat[live])
    remap = np.full(e, -1, np.int64)
    remap[used] = np.arange(used.size)
    cids = np.where(live, remap[np.clip(flat, 0, e - 1)], -1).reshape(ids.shape)
    return torch.from_numpy(used).to(DEV), cids


# ------------------------------------------------------------ musa_fused_gemv_moe --
@pytest.mark.parametrize("e,i,h,k,t", [(256, 128, 2048, 8, 1), (256, 128, 2048, 8, 8),
                                       (256, 128, 2048, 8, 13), (256, 2048, 7168, 8, 1),
                                       (256, 2048, 7168, 8, 3), (64, 1408, 2048, 6, 3)])
def test_gemv_moe_fp8_w13_w2_match_oracle(e, i, h, k, t):
    """The driver's two calls (fused_moe.py:2148-2177) at the reference's
    calibrated decode shapes: W13 over the tokens with SwiGLU, then W2 over
    cache2's rows with the routed weight; up to 16 routes run direct slots,
    more the expert-grouped slots."""
    from vllm_musa_amd import _custom_ops as ops
    from vllm_musa_amd import synthetic
    w13, s13, w2, s2 = synthetic.moe_fp8_weights(e, h, i, 40 + t)
    x = synthetic.activations(t, h, 41 + t)
    w, ids = _routing(t, e, k, 42 + t)
    cache2 = torch.empty(t * k, i, dtype=torch.bfloat16, device=DEV)
    cache3 = torch.empty(t, k, h, dtype=torch.bfloat16, device=DEV)
    ops.musa_fused_gemv_moe(x, w13, cache2, None, s13, w, ids, False, k, False, True)
    ops.musa_fused_gemv_moe(cache2, w2, cache3, None, s2, w, ids, True, 1, False, False)
    used, cids = _compact(ids, e)
    ref2 = ogemv.fused_gemv_moe(_np(x), _np(w13[used]), _np(w), cids, False, k, True,
                                b_scale=_np(s13[used]))
    _check(cache2, ref2)
    # W2 on the GPU's own cache2, so each stage is checked on its own inputs
    ref3 = ogemv.fused_gemv_moe(_np(cache2), _np(w2[used]), _np(w), cids.reshape(-1, 1), True, 1,
                                False, b_scale=_np(s2[used]))
    _check(cache3, ref3)


def test_gemv_moe_dead_routes_write_zero_rows():
    """Ids outside [0, E) (gemv.mu:297-311) give zero rows in both calls,
    whatever C held, on the direct and the grouped slots."""
    from vllm_musa_amd import _custom_ops as ops
    from vllm_musa_amd import synthetic
    e, i, h, k = 16, 128, 1024, 4
    w13, s13, w2, s2 = synthetic.moe_fp8_weights(e, h, i, 5)
    for t in (2, 9):  # 8 routes: direct slots; 36: grouped
        x = synthetic.activations(t, h, 6 + t)
        w, ids = _routing(t, e, k, 7 + t, dead=((0, 1, -1), (t - 1, 3, e), (t - 1, 0, 1000)))
        c2 = torch.full((t * k, i), 7.0, dtype=torch.bfloat16, device=DEV)
        c3 = torch.full((t * k, h), 7.0, dtype=torch.bfloat16, device=DEV)
        ops.musa_fused_gemv_moe(x, w13, c2, None, s13, w, ids, False, k, False, True)
        ops.musa_fused_gemv_moe(c2, w2, c3, None, s2, w, ids, True, 1, False, False)
        idn = ids.cpu().numpy().reshape(-1)
        dead = (idn < 0) | (idn >= e)
        assert dead.sum() == 3
        assert torch.count_nonzero(c2[torch.from_numpy(dead).to(DEV)]) == 0
        assert torch.count_nonzero(c3[torch.from_numpy(dead).to(DEV)]) == 0
        ref = ogemv.fused_gemv_moe(_np(x), _np(w13), _np(w), ids.cpu().numpy(), False, k, True,
                                   b_scale=_np(s13))
        _check(c2, ref)


def test_gemv_moe_weight_decode_is_exact_for_every_code():
    """One-hot bf16 activations pick single weights: with unit block scales,
    C[r, n] must be the e4m3 value of code B[0, n, r] exactly (every e4m3
    value is a bf16 value), so each of the 254 finite codes is decoded
    exactly by the in-register fp8 -> bf16 conversion.  Row n holds the codes
    (n + 2r) % 256, which covers every code, with the two NaN codes replaced
    by zero (one NaN would make its whole row NaN through 0 * NaN)."""
    from vllm_musa_amd import _custom_ops as ops
    n, kdim = 256, 128
    nn, rr = np.meshgrid(np.arange(n), np.arange(kdim), indexing="ij")
    codes = ((nn + 2 * rr) % 256).astype(np.uint8)
    codes[(codes == 0x7F) | (codes == 0xFF)] = 0
    assert len(np.unique(codes)) == 254
    b = torch.from_numpy(codes)[None].view(torch.float8_e4m3fn).to(DEV)
    s = torch.ones(1, n // 128, kdim // 128, device=DEV)
    a = torch.eye(kdim, dtype=torch.bfloat16, device=DEV)  # row r = one-hot at r
    c = torch.empty(kdim, n, dtype=torch.bfloat16, device=DEV)
    ids = torch.zeros(kdim, 1, dtype=torch.int32, device=DEV)
    ops.musa_fused_gemv_moe(a, b, c, None, s, torch.ones(kdim, 1, device=DEV), ids, False, 1, False,
                            False)
    np.testing.assert_array_equal(c.float().cpu().numpy(), onum.e4m3_decode(codes.T))


@pytest.mark.parametrize("rows", [1, 2, 3, 4, 5])
def test_gemv_moe_bf16_weights_reference_case(rows):
    """The reference's own bf16 case (tests/test_deepseek_v4_gemv_numeric.py:17-54):
    one expert [32, 128], a 16x8 tile request, every row its own route;
    against torch's matmul with its tolerance and against the oracle."""
    from vllm_musa_amd import _custom_ops as ops
    torch.manual_seed(60083 + rows)
    a = torch.randn((rows, 128), device=DEV, dtype=torch.bfloat16)
    b = torch.randn((1, 32, 128), device=DEV, dtype=torch.bfloat16)
    c = torch.empty((rows, 32), device=DEV, dtype=torch.bfloat16)
    w = torch.ones((rows, 1), device=DEV, dtype=torch.float32)
    ids = torch.zeros((rows, 1), device=DEV, dtype=torch.int32)
    ops.musa_fused_gemv_moe(a, b, c, None, None, w, ids, False, 1, False, False, block_n=16,
                            block_k=8)
    expected = torch.matmul(a.float(), b[0].float().transpose(0, 1)).to(torch.bfloat16)
    torch.testing.assert_close(c.float(), expected.float(), rtol=2e-2, atol=2e-2)
    _check(c, ogemv.fused_gemv_moe(_np(a), _np(b), _np(w), ids.cpu().numpy(), False, 1, False))


def test_gemv_moe_clamped_swiglu_and_input_weight():
    """mul_routed_weight on the SwiGLU call (apply_router_weight_on_input)
    scales gate and up before the activation, and the limit is rounded to bf16
    first (gemv.mu:946-951): 7.03 acts as 7.03125."""
    from vllm_musa_amd import _custom_ops as ops
    from vllm_musa_amd import synthetic
    e, i, h, k, t = 32, 256, 1024, 4, 5
    w13, s13, _, _ = synthetic.moe_fp8_weights(e, h, i, 9)
    x = synthetic.activations(t, h, 10, scale=40.0)  # gate sums well past the limit
    w, ids = _routing(t, e, k, 11)
    w = w * 3.0
    c2 = torch.empty(t * k, i, dtype=torch.bfloat16, device=DEV)
    ops.musa_fused_gemv_moe(x, w13, c2, None, s13, w, ids, True, k, False, True, swiglu_limit=7.03)
    ref = ogemv.fused_gemv_moe(_np(x), _np(w13), _np(w), ids.cpu().numpy(), True, k, True, 7.03,
                               b_scale=_np(s13))
    _check(c2, ref)
    hi = c2.float().abs().max().item()
    assert hi <= 7.03125 * 7.03125 * 1.01  # silu(g) * u with both at the limit


def test_gemv_moe_fp8_activations_with_scales():
    """The op's fp8-activation branch (gemv.mu:420-427): A e4m3 with 1x128
    scales, products carry both scales."""
    from vllm_musa_amd import _custom_ops as ops
    from vllm_musa_amd import synthetic
    from vllm_musa_amd.fp8_utils import per_token_group_quant_fp8
    e, i, h, k, t = 16, 256, 2048, 4, 6
    w13, s13, _, _ = synthetic.moe_fp8_weights(e, h, i, 12)
    x = synthetic.activations(t, h, 13)
    xq, xs = per_token_group_quant_fp8(x, 128)
    w, ids = _routing(t, e, k, 14)
    c2 = torch.empty(t * k, i, dtype=torch.bfloat16, device=DEV)
    ops.musa_fused_gemv_moe(xq, w13, c2, xs, s13, w, ids, False, k, False, True)
    ref = ogemv.fused_gemv_moe(_np(xq), _np(w13), _np(w), ids.cpu().numpy(), False, k, True,
                               a_scale=_np(xs), b_scale=_np(s13))
    _check(c2, ref)


def test_gemv_moe_argument_errors():
    from vllm_musa_amd import _custom_ops as ops
    a = torch.zeros(2, 128, dtype=torch.bfloat16, device=DEV)
    b = torch.zeros(1, 32, 128, dtype=torch.bfloat16, device=DEV)
    c = torch.empty(2, 32, dtype=torch.bfloat16, device=DEV)
    w = torch.ones(2, 1, device=DEV)
    ids = torch.zeros(2, 1, dtype=torch.int32, device=DEV)
    with pytest.raises(RuntimeError, match="both block_n and block_k"):
        ops.musa_fused_gemv_moe(a, b, c, None, None, w, ids, False, 1, False, False, block_n=16)
    with pytest.raises(RuntimeError, match="<= 512"):
        ops.musa_fused_gemv_moe(a, b, c, None, None, w, ids, False, 1, False, False, 64, 16)
    with pytest.raises(RuntimeError, match="is invalid for"):
        ops.musa_fused_gemv_moe(a, b, c, None, None, w, ids, False, 1, False, False, 64, 8)
    with pytest.raises(RuntimeError, match="A must be dim 2"):
        ops.musa_fused_gemv_moe(a[None], b, c, None, None, w, ids, False, 1, False, False)
    with pytest.raises(NotImplementedError):
        ops.musa_fused_gemv_moe(a, b, c, None, None, w, ids, False, 1, True, False)


def test_gemv_moe_graph_replay_with_a_tile_request():
    """As the reference's graph test (test_deepseek_v4_gemv_numeric.py:57-128):
    captured once, replayed on new inputs copied into the captured buffer."""
    from vllm_musa_amd import _custom_ops as ops
    rows, h, n = 1, 128, 32
    a = torch.zeros((rows, h), device=DEV, dtype=torch.bfloat16)
    torch.manual_seed(3)
    b = torch.randn((1, n, h), device=DEV, dtype=torch.bfloat16)
    c = torch.empty((rows, n), device=DEV, dtype=torch.bfloat16)
    w = torch.ones((rows, 1), device=DEV, dtype=torch.float32)
    ids = torch.zeros((rows, 1), device=DEV, dtype=torch.int32)
    run = lambda: torch.ops._C_musa_ops.musa_fused_gemv_moe(a, b, c, None, None, w, ids, False, 1,
                                                            False, False, block_n=16, block_k=8)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            run()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run()
    for seed in (11, 13, 17):
        torch.manual_seed(seed)
        nxt = torch.randn_like(a)
        expected = torch.matmul(nxt.float(), b[0].float().transpose(0, 1)).to(torch.bfloat16)
        a.copy_(nxt)
        graph.replay()
        torch.cuda.synchronize()
        torch.testing.assert_close(c.float(), expected.float(), rtol=2e-2, atol=2e-2)


# ------------------------------------------------------------------ musa_fused_gemv --
@pytest.mark.parametrize("m,n,k", [(1, 2112, 7168), (3, 7168, 2048), (16, 512, 4096),
                                   (40, 24576, 1536)])
def test_dense_gemv_matches_oracle(m, n, k):
    """musa_fused_gemv with fp8 weights and bf16 x (the small-M path of
    _musa_fp8_small_m_gemv_op, deep_gemm.py:512-536), both through the Python
    wrapper and through torch.ops._C_musa_ops in the op's own argument order."""
    from vllm_musa_amd import _custom_ops as ops
    from vllm_musa_amd import synthetic
    w, ws = synthetic.dense_fp8_weight(n, k, 50 + m)
    x = synthetic.activations(m, k, 51 + m)
    out = ops.musa_fused_gemv(x, w, None, ws)
    ref = ogemv.fused_gemv(_np(x), _np(w), qweight_scale=_np(ws))
    _check(out, ref)
    out2 = torch.empty(m, n, dtype=torch.bfloat16, device=DEV)
    torch.ops._C_musa_ops.musa_fused_gemv(x, w, out2, None, ws, False, False, False, None, 1e-6)
    assert torch.equal(out, out2)
    # a caller-owned output is written in place
    out3 = torch.full((m, n), 3.0, dtype=torch.bfloat16, device=DEV)
    assert ops.musa_fused_gemv(x, w, None, ws, output=out3) is out3
    assert torch.equal(out3, out)


def test_dense_gemv_swiglu_and_bf16_weights():
    from vllm_musa_amd import _custom_ops as ops
    from vllm_musa_amd import synthetic
    w, ws = synthetic.dense_fp8_weight(1024, 4096, 60)
    x = synthetic.activations(2, 4096, 61, scale=0.05)
    out = ops.musa_fused_gemv(x, w, None, ws, use_swigelu=True)
    assert out.shape == (2, 512)
    _check(out, ogemv.fused_gemv(_np(x), _np(w), True, qweight_scale=_np(ws)))
    wb = (torch.randn(256, 512, device=DEV) * 0.05).to(torch.bfloat16)
    xb = synthetic.activations(3, 512, 62)
    outb = ops.musa_fused_gemv(xb, wb)
    assert outb.dtype == torch.bfloat16 and outb.shape == (3, 256)
    _check(outb, ogemv.fused_gemv(_np(xb), _np(wb)))
    with pytest.raises(NotImplementedError):
        ops.musa_fused_gemv(x, w, None, ws, use_rms_norm=True, gamma=torch.ones(1024, device=DEV))


# --------------------------------------------------------------- the layer path --
def _layer_case(e, i, h, k, t, seed):
    from vllm_musa_amd import synthetic
    w13, s13, w2, s2 = synthetic.moe_fp8_weights(e, h, i, seed)
    x = synthetic.activations(t, h, seed + 1)
    w, ids = _routing(t, e, k, seed + 2)
    return x, w13, s13, w2, s2, w, ids


def _layer_oracle(x, w13, s13, w2, s2, w, ids, **kw):
    used, cids = _compact(ids, w13.shape[0])
    return ogemv.fused_experts_w8a16(_np(x), _np(w13[used]), _np(w2[used]), _np(w), cids,
                                     _np(s13[used]), _np(s2[used]), **kw)


@pytest.mark.parametrize("e,i,h,k,t", [(256, 128, 2048, 8, 1), (256, 128, 2048, 8, 8),
                                       (256, 128, 2048, 8, 13), (256, 2048, 7168, 8, 1),
                                       (256, 2048, 7168, 8, 4), (64, 1408, 2048, 6, 3)])
def test_native_gemv_layer_matches_oracle(e, i, h, k, t):
    from vllm_musa_amd.fused_moe import fused_experts_impl
    x, w13, s13, w2, s2, w, ids = _layer_case(e, i, h, k, t, 70 + t)
    out = fused_experts_impl(x, w13, w2, w, ids, use_fp8_w8a8=True, w1_scale=s13, w2_scale=s2,
                             block_shape=[128, 128], path="native_gemv")
    _check(out, _layer_oracle(x, w13, s13, w2, s2, w, ids))


@pytest.mark.parametrize("t", [6, 1])
def test_native_gemv_layer_input_weight_and_limit(t):
    """T=1 runs the direct route slots, whose W13 launch writes the
    activation itself."""
    from vllm_musa_amd.fused_moe import fused_experts_impl
    x, w13, s13, w2, s2, w, ids = _layer_case(64, 256, 1024, 4, t, 90)
    x = x * 30
    out = fused_experts_impl(x, w13, w2, w, ids, use_fp8_w8a8=True, w1_scale=s13, w2_scale=s2,
                             block_shape=[128, 128], apply_router_weight_on_input=True,
                             gemm1_clamp_limit=7.03, path="native_gemv")
    _check(out, _layer_oracle(x, w13, s13, w2, s2, w, ids, apply_router_weight_on_input=True,
                              swiglu_limit=7.03))


def test_native_gemv_layer_bf16_weights():
    """bf16 experts on the native path: gate and up kept fp32 through the
    SwiGLU (gemv.mu:430-434, 477-487)."""
    from vllm_musa_amd import synthetic
    from vllm_musa_amd.fused_moe import fused_experts_impl
    e, i, h, k = 256, 128, 2048, 8
    w13, w2 = synthetic.moe_bf16_weights(e, h, i, 95)
    for t in (1, 12):
        x = synthetic.activations(t, h, 96 + t)
        w, ids = _routing(t, e, k, 97 + t)
        out = fused_experts_impl(x, w13, w2, w, ids, path="native_gemv")
        used, cids = _compact(ids, e)
        ref = ogemv.fused_experts_w8a16(_np(x), _np(w13[used]), _np(w2[used]), _np(w), cids)
        _check(out, ref)


def test_reference_driver_loop_runs_unchanged_on_these_ops():
    """The reference's GEMV-MoE driver (fused_moe.py:2106-2184) written out
    against torch.ops._C_musa_ops: cache3 / cache2 as it allocates them, the
    two musa_fused_gemv_moe calls in its argument order over 16384-token
    chunks, moe_sum.  Matches the oracle and this package's native path."""
    from vllm_musa_amd import _custom_ops as ops
    from vllm_musa_amd.fused_moe import fused_experts_impl
    e, i, h, k, t = 256, 128, 2048, 8, 13
    x, w1, s1, w2, s2, topk_weights, topk_ids = _layer_case(e, i, h, k, t, 100)
    M, K, N = t, w2.size(1), w1.size(1)
    cache3 = torch.empty((M, k, K), device=DEV, dtype=x.dtype)
    cache2 = torch.empty((M * k, N // 2), device=DEV, dtype=x.dtype)
    out = torch.empty_like(x)
    chunk = 16384
    for c in range((t // chunk) + 1):
        b0, b1 = c * chunk, min((c + 1) * chunk, t)
        cur = x[b0:b1]
        n_tok = cur.size(0)
        if n_tok == 0:
            break
        c2, c3 = cache2[:n_tok * k], cache3[:n_tok]
        torch.ops._C_musa_ops.musa_fused_gemv_moe(cur, w1, c2, None, s1, topk_weights[b0:b1],
                                                  topk_ids[b0:b1], False, topk_ids.shape[1], False,
                                                  use_swigelu=True, block_n=0, block_k=0,
                                                  swiglu_limit=0.0)
        torch.ops._C_musa_ops.musa_fused_gemv_moe(c2, w2, c3, None, s2, topk_weights[b0:b1],
                                                  topk_ids[b0:b1], True, 1, False,
                                                  use_swigelu=False, block_n=0, block_k=0)
        ops.moe_sum(c3, out[b0:b1])
    ref = _layer_oracle(x, w1, s1, w2, s2, topk_weights, topk_ids)
    _check(out, ref)
    fused = fused_experts_impl(x, w1, w2, topk_weights, topk_ids, use_fp8_w8a8=True, w1_scale=s1,
                               w2_scale=s2, block_shape=[128, 128], path="native_gemv")
    _check(fused, ref)
    _check(fused, out.float().cpu().numpy().astype(np.float64))


@pytest.fixture
def paths(monkeypatch):
    """Path codes (0 auto, 1 W8A8 decode, 2 grouped GEMM, 3 native GEMV) of
    every fused layer launched through the C ABI."""
    from vllm_musa_amd import fused_moe
    seen = []
    real = fused_moe.call

    def spy(name, *args):
        if name == "vmamd_fused_moe_fp8":
            seen.append(args[17])
        elif name == "vmamd_fused_moe_bf16":
            seen.append(args[14])
        return real(name, *args)

    monkeypatch.setattr(fused_moe, "call", spy)
    return seen


def test_auto_computes_what_the_reference_computes(monkeypatch, paths):
    """On the reference's calibrated fp8 decode shape (E=256, N=256, H=2048,
    top-8: native GEMV up to 13 tokens on its S5000) auto takes the native
    numerics up to 13 tokens and W8A8 above; the gemv override forces the
    native numerics at any size, but not with an expert map (its gate
    declines, fused_moe.py:1336); the DeepSeek-V3 shape, which the reference
    never serves with its GEMV, stays W8A8."""
    from vllm_musa_amd import dispatch_policy as dp
    from vllm_musa_amd.fused_moe import fused_experts_impl
    e, i, h, k = 256, 128, 2048, 8
    from vllm_musa_amd import synthetic
    w13, s13, w2, s2 = synthetic.moe_fp8_weights(e, h, i, 110)

    def run(t, **kw):
        x = synthetic.activations(t, h, 111 + t)
        w, ids = _routing(t, e, k, 112 + t)
        out = fused_experts_impl(x, w13, w2, w, ids, use_fp8_w8a8=True, w1_scale=s13,
                                 w2_scale=s2, block_shape=[128, 128], **kw)
        return out, (x, w13, s13, w2, s2, w, ids)

    for t, code in ((1, 3), (13, 3), (14, 1), (100, 2)):
        paths.clear()
        out, case = run(t)
        assert paths == [code], (t, paths)
        if code == 3:
            _check(out, _layer_oracle(*case))
    monkeypatch.setenv(dp.MUSA_FUSED_MOE_DISPATCH_ENV, "gemv")
    paths.clear()
    out, case = run(40)
    assert paths == [3]
    _check(out, _layer_oracle(*case))
    paths.clear()
    run(4, expert_map=torch.arange(e, dtype=torch.int32, device=DEV))
    assert paths and paths[0] != 3
    monkeypatch.delenv(dp.MUSA_FUSED_MOE_DISPATCH_ENV)
    w13d, s13d, w2d, s2d = synthetic.moe_fp8_weights(256, 7168, 2048, 113)
    x = synthetic.activations(2, 7168, 114)
    w, ids = _routing(2, 256, 8, 115)
    paths.clear()
    fused_experts_impl(x, w13d, w2d, w, ids, use_fp8_w8a8=True, w1_scale=s13d, w2_scale=s2d,
                       block_shape=[128, 128])
    assert paths == [1]


def test_native_layer_graph_replay_matches_eager():
    from vllm_musa_amd.fused_moe import fused_experts_impl
    x, w13, s13, w2, s2, w, ids = _layer_case(256, 128, 2048, 8, 4, 120)
    call = lambda: fused_experts_impl(x, w13, w2, w, ids, use_fp8_w8a8=True, w1_scale=s13,
                                      w2_scale=s2, block_shape=[128, 128], path="native_gemv")
    eager = call()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = call()
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        assert torch.equal(call(), eager)
