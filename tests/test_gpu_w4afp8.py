"""GPU parity of the w4afp8 MoE layer, the per-row fp8 quantiser and the
weighted combine against the oracle.

Cases follow the reference's own tests (tests/kernels/test_w4afp8_moe.py:
tokens 1/8/16/17/65/257, routings local / mapped / all_remote / hot_expert,
NaN-poisoned allocations, non-contiguous hidden states), on both kernel paths,
plus the E=128 / top-8 / H=4096 / I=1536 shape.  Layer tolerance: rel-L2 <=
1e-2 and max-abs <= 2e-2 * max|ref|; the quantiser and the combine are
bit-exact."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import w4afp8 as ow4
from oracle.numerics import bf16_round

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _check(out: torch.Tensor, ref: np.ndarray, rel_l2=1e-2, max_frac=2e-2):
    o = out.float().cpu().numpy().astype(np.float64)
    err = o - ref
    rl2 = np.linalg.norm(err) / max(np.linalg.norm(ref), 1e-30)
    assert np.isfinite(o).all()
    assert rl2 <= rel_l2, f"rel-L2 {rl2}"
    assert np.abs(err).max() <= max_frac * max(np.abs(ref).max(), 1e-30), f"max-abs {np.abs(err).max()}"


def _case(tokens, routing, experts=4, hidden=256, inter=256, topk=2, seed=128):
    g = torch.Generator().manual_seed(seed + tokens)
    states = (torch.randn(tokens, hidden, generator=g) * 0.3).to(torch.bfloat16)
    gu = torch.randint(-8, 8, (experts, 2 * inter, hidden), generator=g, dtype=torch.int8)
    dn = torch.randint(-8, 8, (experts, hidden, inter), generator=g, dtype=torch.int8)
    gu_s = (torch.rand(experts, 2 * inter, hidden // 128, generator=g) * 0.01 + 0.002).to(torch.bfloat16)
    dn_s = (torch.rand(experts, hidden, inter // 128, generator=g) * 0.01 + 0.002).to(torch.bfloat16)
    mapped = routing in ("mapped", "all_remote")
    total = experts * 2 if mapped else experts
    ids = torch.stack([torch.randperm(total, generator=g)[:topk] for _ in range(tokens)]).to(torch.int32)
    if routing == "all_remote":
        ids.remainder_(experts)
    elif routing == "hot_expert":
        ids.zero_()
    w = torch.softmax(torch.randn(tokens, topk, generator=g), dim=-1)
    emap = (torch.cat((torch.full((experts,), -1), torch.arange(experts))).to(torch.int32)
            if mapped else None)
    args = dict(x=states, w13=ow4.pack_int4(gu.numpy()), w2=ow4.pack_int4(dn.numpy()),
                s13=gu_s, s2=dn_s, w=w, ids=ids, emap=emap)
    return args


def _oracle(a, limit=10.0):
    f = lambda t: t.float().numpy()
    return ow4.w4afp8_moe(f(a["x"]), a["w13"], a["w2"], f(a["s13"]), f(a["s2"]), a["w"].numpy(),
                          a["ids"].numpy(), None if a["emap"] is None else a["emap"].numpy(),
                          swiglu_limit=limit)


def _run(a, path, limit=10.0, x=None):
    from vllm_musa_amd import w4afp8_moe
    d = lambda t: None if t is None else (torch.from_numpy(t) if isinstance(t, np.ndarray) else t).to(DEV)
    return w4afp8_moe(d(a["x"]) if x is None else x, d(a["w13"]), d(a["w2"]), d(a["s13"]),
                      d(a["s2"]), d(a["w"]), d(a["ids"]), d(a["emap"]), swiglu_limit=limit, path=path)


@pytest.mark.parametrize("path", ["gemv", "gemm"])
@pytest.mark.parametrize("routing", ["local", "mapped", "all_remote", "hot_expert"])
@pytest.mark.parametrize("tokens", [1, 8, 16, 17, 65, 257])
def test_w4afp8_vs_oracle(tokens, routing, path):
    a = _case(tokens, routing)
    ref = _oracle(a)
    out = _run(a, path)
    _check(out, ref)
    # the reference test's own bar, against the same oracle
    torch.testing.assert_close(out.float().cpu(), torch.from_numpy(ref), rtol=0.04, atol=0.008)


@pytest.mark.parametrize("path", ["gemv", "gemm"])
def test_w4afp8_without_limit(path):
    a = _case(33, "local")
    _check(_run(a, path, limit=None), _oracle(a, limit=None))


@pytest.mark.parametrize("path", ["gemv", "gemm"])
def test_w4afp8_nan_poisoned_allocations(path, monkeypatch):
    a = _case(17, "mapped")
    ref = _oracle(a)
    real = torch.empty

    def poisoned(*args, **kwargs):
        t = real(*args, **kwargs)
        if t.is_cuda:
            t.view(torch.uint8).fill_(0xFF)
        return t

    monkeypatch.setattr(torch, "empty", poisoned)
    out = _run(a, path)
    assert torch.isfinite(out).all()
    _check(out, ref)


def test_w4afp8_noncontiguous_hidden_states():
    a = _case(65, "mapped")
    x = a["x"].to(DEV).T.contiguous().T
    assert not x.is_contiguous()
    out = _run(a, "auto", x=x)
    assert out.is_contiguous()
    _check(out, _oracle(a))


@pytest.mark.parametrize("path", ["gemv", "gemm"])
@pytest.mark.parametrize("T", [5, 300])
def test_w4afp8_large_shape(T, path):
    """E=128, top-8 softmax-renorm routing, H=4096, I=1536 (only the touched
    experts go to the oracle)."""
    from vllm_musa_amd import fused_topk, synthetic
    E, H, I = 128, 4096, 1536
    w13, w2, s13, s2 = synthetic.moe_w4a8_weights(E, H, I, 5000)
    x = synthetic.activations(T, H, 5001 + T)
    logits = synthetic.router_logits(T, E, 5002 + T)
    w, ids, _ = fused_topk(x, logits, 8, True)
    from vllm_musa_amd import w4afp8_moe
    out = w4afp8_moe(x, w13, w2, s13, s2, w, ids, swiglu_limit=10.0, path=path)
    # tokens are independent: check a sample of rows on the experts they touch
    rows = torch.tensor(sorted({0, 1, T // 2, T - 1}))
    ids_s = ids.cpu()[rows]
    used = torch.unique(ids_s)
    remap = torch.full((E,), -1, dtype=torch.int32)
    remap[used] = torch.arange(used.numel(), dtype=torch.int32)
    cids = remap[ids_s.long()].numpy()
    sel = used.to(DEV)
    ref = ow4.w4afp8_moe(x.float().cpu().numpy()[rows.numpy()],
                         w13.index_select(0, sel).cpu().numpy(),
                         w2.index_select(0, sel).cpu().numpy(),
                         s13.index_select(0, sel).float().cpu().numpy(),
                         s2.index_select(0, sel).float().cpu().numpy(), w.cpu().numpy()[rows.numpy()],
                         cids, swiglu_limit=10.0)
    _check(out[rows.to(DEV)], ref)


def test_w4afp8_paths_agree_and_deterministic():
    a = _case(48, "local", experts=8, topk=4)
    g = _run(a, "gemv")
    m = _run(a, "gemm")
    rl2 = (torch.linalg.norm(g.float() - m.float()) / torch.linalg.norm(m.float())).item()
    assert rl2 < 5e-3, rl2
    assert torch.equal(g, _run(a, "gemv")) and torch.equal(m, _run(a, "gemm"))


def test_w4afp8_rejects_bad_shapes():
    from vllm_musa_amd import w4afp8_moe
    a = _case(2, "local")
    d = lambda t: (torch.from_numpy(t) if isinstance(t, np.ndarray) else t).to(DEV)
    with pytest.raises(ValueError, match="group128"):
        w4afp8_moe(d(a["x"])[:, :200], d(a["w13"]), d(a["w2"]), d(a["s13"]), d(a["s2"]),
                   d(a["w"]), d(a["ids"]))
    with pytest.raises(ValueError, match="BF16"):
        w4afp8_moe(d(a["x"]), d(a["w13"]), d(a["w2"]), d(a["s13"]).float(), d(a["s2"]),
                   d(a["w"]), d(a["ids"]))
    assert w4afp8_moe(d(a["x"])[:0], d(a["w13"]), d(a["w2"]), d(a["s13"]), d(a["s2"]),
                      d(a["w"])[:0], d(a["ids"])[:0]).shape == (0, 256)


@pytest.mark.parametrize("rows,cols", [(1, 256), (33, 4096), (300, 1536), (7, 16384)])
def test_per_token_quant_bit_exact(rows, cols):
    from vllm_musa_amd._custom_ops import per_token_quant_fp8
    g = np.random.Generator(np.random.PCG64(rows + cols))
    x = (g.standard_normal((rows, cols)) * g.uniform(1e-3, 30, (rows, 1))).astype(np.float32)
    x[0] = 0.0
    xt = torch.from_numpy(x).to(torch.bfloat16).to(DEV)
    q, s = per_token_quant_fp8(xt)
    q_ref, s_ref = ow4.dynamic_fp8_rows(xt.float().cpu().numpy())
    np.testing.assert_array_equal(s.cpu().numpy(), s_ref)
    np.testing.assert_array_equal(q.view(torch.uint8).cpu().numpy(), q_ref)


def test_per_token_quant_at_e4m3_rounding_boundaries():
    """bf16 rows whose quotients x / s are exactly e4m3 midpoints (ties) or
    e4m3 values (a power-of-two scale: the row maximum is 448 * 2^k), both
    signs, zeros, and bf16 neighbours of each: bytes equal the oracle's."""
    from vllm_musa_amd._custom_ops import per_token_quant_fp8
    from oracle.numerics import bf16_round
    mids = [(2 * i + 1) * 2.0 ** -10 for i in range(8)]
    vals = [i * 2.0 ** -9 for i in range(8)]
    for e in range(-6, 9):
        for k in range(8):
            vals.append((1 + k / 8) * 2.0 ** e)
            mids.append((1 + (2 * k + 1) / 16) * 2.0 ** e)
    t = np.array([m for m in mids + vals if m <= 448.0], np.float32)
    t = np.concatenate([t, bf16_round(t * np.float32(1 + 2 ** -8)), bf16_round(t * np.float32(1 - 2 ** -8))])
    t = np.concatenate([t[t <= 448.0], -t[t <= 448.0], np.float32([-0.0])])
    rows = []
    for k in (-12, 0, 3):
        r = np.zeros(1536, np.float32)
        r[0] = 448.0 * 2.0 ** k
        r[1:1 + t.size] = t * np.float32(2.0 ** k)
        rows.append(r)
    x = np.stack(rows)
    assert np.array_equal(bf16_round(x), x)
    q, s = per_token_quant_fp8(torch.from_numpy(x).to(torch.bfloat16).to(DEV))
    q_ref, s_ref = ow4.dynamic_fp8_rows(x)
    np.testing.assert_array_equal(s.cpu().numpy(), s_ref)
    np.testing.assert_array_equal(q.view(torch.uint8).cpu().numpy(), q_ref)


def test_weighted_sum_bit_exact():
    from vllm_musa_amd._custom_ops import moe_weighted_sum
    g = np.random.Generator(np.random.PCG64(9))
    y = bf16_round(g.standard_normal((37, 8, 1024)).astype(np.float32))
    w = g.uniform(0, 1, (37, 8)).astype(np.float32)
    ids = g.integers(-1, 16, (37, 8)).astype(np.int32)
    acc = ow4.weighted_sum_fma(y, w, ids >= 0)
    out = torch.empty(37, 1024, dtype=torch.bfloat16, device=DEV)
    moe_weighted_sum(torch.from_numpy(y).to(torch.bfloat16).to(DEV), torch.from_numpy(w).to(DEV),
                     out, torch.from_numpy(ids).to(DEV))
    np.testing.assert_array_equal(out.float().cpu().numpy(), bf16_round(acc))


def test_quant_method_hooks():
    from types import SimpleNamespace

    from vllm_musa_amd.quant_methods import W4AFp8MoEMethod
    a = _case(9, "mapped")
    d = lambda t: (torch.from_numpy(t) if isinstance(t, np.ndarray) else t).to(DEV)
    layer = SimpleNamespace(w13_weight=d(a["w13"]), w2_weight=d(a["w2"]),
                            w13_weight_scale_inv=d(a["s13"]), w2_weight_scale_inv=d(a["s2"]),
                            expert_map=d(a["emap"]), apply_router_weight_on_input=False)
    out = W4AFp8MoEMethod(swiglu_limit=10.0).apply(layer, d(a["x"]), d(a["w"]), d(a["ids"]))
    _check(out, _oracle(a))
