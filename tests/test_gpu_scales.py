"""vmamd_convert_scales and the loaders built on it, on the GPU, against
oracle/scales.py (bit-exact), plus end-to-end properties of the loaded layers:
e8m0-scaled dense GEMMs equal the same GEMM on float32 scales, and a W4AFP8
layer split over two tensor-parallel ranks sums to the unsplit layer."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import scales as osc
from oracle import w4afp8 as ow4
from oracle.gemm import w8a8_block_fp8_matmul as oracle_gemm

pytestmark = pytest.mark.gpu
DEV = "cuda"
E8M0 = getattr(torch, "float8_e8m0fnu", None)
_TORCH = {"e8m0": torch.uint8, "f32": torch.float32, "bf16": torch.bfloat16}


def _source(kind: str, n: int, rng) -> np.ndarray:
    """Raw source encodings with every class of value in them."""
    if kind == "e8m0":
        return rng.integers(0, 256, n, dtype=np.uint16).astype(np.uint8)
    if kind == "bf16":
        return rng.integers(0, 2 ** 16, n, dtype=np.uint32).astype(np.uint16)
    x = (rng.standard_normal(n) * 0.02).astype(np.float32)
    pick = rng.integers(0, 16, n)
    x[pick == 0] = np.nan
    x[pick == 1] = -np.abs(x[pick == 1])
    x[pick == 2] = rng.integers(0, 2 ** 32, int((pick == 2).sum()), dtype=np.uint64
                                ).astype(np.uint32).view(np.float32)
    return x


def _to_dev(a: np.ndarray, kind: str, offset: int) -> torch.Tensor:
    """The source on the GPU, starting `offset` elements into its allocation (so
    offset 1 leaves it unaligned)."""
    raw = torch.from_numpy(a.view(np.int16) if kind == "bf16" else a)
    buf = torch.zeros(a.size + offset, dtype=raw.dtype, device=DEV)
    buf[offset:] = raw.to(DEV)
    t = buf[offset:]
    return t.view(torch.bfloat16) if kind == "bf16" else t


def _bits(t: torch.Tensor) -> np.ndarray:
    c = t.cpu()
    return (c.view(torch.int16).numpy().view(np.uint16) if c.dtype == torch.bfloat16
            else c.numpy().view(np.uint32))


@pytest.mark.parametrize("n", [1, 7, 8, 9, 1000, 4099, (1 << 20) + 3])
@pytest.mark.parametrize("src,dst", [("e8m0", "f32"), ("e8m0", "bf16"), ("f32", "f32"),
                                     ("f32", "bf16"), ("bf16", "f32"), ("bf16", "bf16")])
@pytest.mark.parametrize("offset", [0, 1])
def test_convert_scales_bit_exact(src, dst, n, offset):
    rng = np.random.default_rng(n * 7 + offset)
    a = _source(src, n, rng)
    want, want_bad = osc.convert_scales(a, src, dst)
    s = _to_dev(a, src, offset)
    doff = 1 - offset  # misalign the destination when the source is aligned
    dbuf = torch.full((n + doff,), 7, dtype=_TORCH[dst], device=DEV)
    d = dbuf[doff:]
    bad = torch.zeros(1, dtype=torch.int32, device=DEV)
    from vllm_musa_amd import _custom_ops as ops
    ops.convert_scales(s, d, bad)
    got = _bits(d)
    want_bits = want.view(np.uint32) if dst == "f32" else want
    assert np.array_equal(got, want_bits)
    assert int(bad.item()) == want_bad
    if doff:
        assert float(dbuf[0]) == 7.0  # nothing written before the destination


def test_convert_f32_to_bf16_every_rounding_class():
    """f32 -> bf16 on every upper half (sign, exponent, 7 kept mantissa bits)
    with the lower halves that decide the rounding: exact, just below, at
    and just above the tie, the largest, and random ones -- NaN payloads,
    infinities, subnormals and carries into the exponent included (the
    kernels' conversion instruction against the integer rounding rule)."""
    hi = np.arange(1 << 16, dtype=np.uint32) << 16
    rng = np.random.default_rng(5)
    lows = [0x0000, 0x7FFF, 0x8000, 0x8001, 0xFFFF, 0x0001]
    bits = np.concatenate([hi | np.uint32(lo) for lo in lows] +
                          [hi | rng.integers(0, 1 << 16, hi.size, dtype=np.uint32)])
    a = bits.view(np.float32)
    want, want_bad = osc.convert_scales(a, "f32", "bf16")
    d = torch.empty(a.size, dtype=torch.bfloat16, device=DEV)
    bad = torch.zeros(1, dtype=torch.int32, device=DEV)
    from vllm_musa_amd import _custom_ops as ops
    ops.convert_scales(torch.from_numpy(a).to(DEV), d, bad)
    assert np.array_equal(_bits(d), want)
    assert int(bad.item()) == want_bad


def test_convert_scales_aliasing_and_empty():
    from vllm_musa_amd import _custom_ops as ops
    x = torch.rand(1000, device=DEV) + 0.5
    ref = x.clone()
    ops.convert_scales(x, x)  # in place, same element size
    assert torch.equal(x, ref)
    with pytest.raises(ValueError, match="overlap"):
        ops.convert_scales(x[:500], x[10:510])
    with pytest.raises(ValueError, match="overlap"):
        ops.convert_scales(x[:500], x.view(torch.bfloat16)[:500])
    ops.convert_scales(torch.empty(0, device=DEV), torch.empty(0, dtype=torch.bfloat16, device=DEV))
    with pytest.raises(ValueError):
        ops.convert_scales(x, torch.empty(999, device=DEV))
    with pytest.raises(ValueError):
        ops.convert_scales(x, torch.empty(1000, dtype=torch.float16, device=DEV))


@pytest.mark.skipif(E8M0 is None, reason="no float8_e8m0fnu in this torch")
def test_deepgemm_post_process_upcasts_e8m0_only():
    from vllm_musa_amd.fp8_utils import deepgemm_post_process_fp8_weight_block
    rng = np.random.default_rng(3)
    bits = rng.integers(0, 256, (56, 144), dtype=np.uint16).astype(np.uint8)
    wq = torch.zeros(16, 16, dtype=torch.float8_e4m3fn, device=DEV)
    ws = torch.from_numpy(bits).to(DEV).view(E8M0)
    q, s = deepgemm_post_process_fp8_weight_block(wq, ws, (128, 128), use_e8m0=False)
    assert q is wq and s.dtype == torch.float32 and s.shape == ws.shape
    assert np.array_equal(_bits(s), osc.upcast_e8m0_to_fp32(bits).view(np.uint32))
    assert deepgemm_post_process_fp8_weight_block(wq, ws, (128, 128), use_e8m0=True)[1] is ws
    f = torch.ones(4, 4, device=DEV)
    assert deepgemm_post_process_fp8_weight_block(wq, f, (128, 128), use_e8m0=False)[1] is f


@pytest.mark.skipif(E8M0 is None, reason="no float8_e8m0fnu in this torch")
@pytest.mark.parametrize("m,n,k", [(1, 512, 1024), (40, 384, 768), (300, 1024, 512)])
def test_dense_layer_with_e8m0_checkpoint_scales(m, n, k):
    from vllm_musa_amd.block_fp8 import Fp8BlockScaledMMKernel
    g = torch.Generator().manual_seed(m + n + k)
    w = (torch.randn(n, k, generator=g) * 0.5).clamp(-448, 448).to(torch.float8_e4m3fn)
    bits = torch.randint(118, 124, ((n + 127) // 128, k // 128), generator=g, dtype=torch.uint8)
    x = (torch.randn(m, k, generator=g) * 0.5).to(torch.bfloat16)
    layer = torch.nn.Module()
    layer.weight = torch.nn.Parameter(w.to(DEV), requires_grad=False)
    layer.weight_scale_inv = torch.nn.Parameter(bits.to(DEV).view(E8M0), requires_grad=False)
    layer.weight_block_size = [128, 128]
    kern = Fp8BlockScaledMMKernel()
    kern.process_weights_after_loading(layer)
    s = layer.weight_scale_inv
    assert isinstance(s, torch.nn.Parameter) and s.dtype == torch.float32
    f32 = osc.upcast_e8m0_to_fp32(bits.numpy())
    assert np.array_equal(_bits(s), f32.view(np.uint32))
    out = kern.apply_block_scaled_mm(x.to(DEV), layer.weight, None, s)
    ref_scales = torch.from_numpy(f32).to(DEV)
    same = kern.apply_block_scaled_mm(x.to(DEV), layer.weight, None, ref_scales)
    assert torch.equal(out, same)
    # and the layer output against the oracle GEMM on the same quantised input
    from vllm_musa_amd.fp8_utils import per_token_group_quant_fp8
    q, qs = per_token_group_quant_fp8(x.to(DEV), 128)
    ref = oracle_gemm(q.cpu().view(torch.uint8).numpy(), qs.cpu().numpy(),
                      w.view(torch.uint8).numpy(), f32)
    o = out.float().cpu().numpy()
    err = np.linalg.norm(o - ref) / max(np.linalg.norm(ref), 1e-30)
    assert err <= 1e-2, err


@pytest.mark.parametrize("invalid", [float("nan"), float("inf"), -0.1, 0.0, 1.0e-42, 3.4e38])
@pytest.mark.parametrize("scale_name", ["w13_weight_scale_inv", "w2_weight_scale_inv"])
def test_w4afp8_invalid_loaded_scales_fail(invalid, scale_name):
    from vllm_musa_amd.quant_methods import W4AFp8MoEMethod
    m = W4AFp8MoEMethod()
    layer = torch.nn.Module()
    m.create_weights(layer, 1, 128, 128, torch.bfloat16, device=DEV, weight_loader=object())
    layer.w13_weight_scale_inv.data.fill_(0.01)
    layer.w2_weight_scale_inv.data.fill_(0.01)
    getattr(layer, scale_name).data[0, 5, 0] = invalid
    with pytest.raises(ValueError, match=f"Invalid W4AFP8 weight scale in {scale_name}"):
        m.process_weights_after_loading(layer)


def test_w4afp8_scales_cast_like_the_oracle():
    from vllm_musa_amd.quant_methods import W4AFp8MoEMethod
    m = W4AFp8MoEMethod()
    layer = torch.nn.Module()
    m.create_weights(layer, 2, 256, 384, torch.bfloat16, device=DEV)
    scales = torch.linspace(0.001, 0.013, layer.w13_weight_scale_inv.numel()).reshape(
        layer.w13_weight_scale_inv.shape)
    layer.w13_weight_scale_inv.data.copy_(scales)
    layer.w2_weight_scale_inv.data.fill_(0.007)
    m.process_weights_after_loading(layer)
    assert layer.w13_weight.dtype == torch.int8
    assert layer.w13_weight_scale_inv.dtype == torch.bfloat16
    want, ok = osc.w4afp8_scales(scales.numpy())
    assert ok and np.array_equal(_bits(layer.w13_weight_scale_inv), want)
    torch.testing.assert_close(layer.w13_weight_scale_inv.cpu(), scales.to(torch.bfloat16),
                               rtol=0, atol=0)


def _w4_checkpoint(experts, hidden, inter, seed):
    """Per-expert unsplit checkpoint tensors: w1 / w3 [I, H/2] and w2 [H, I/2]
    packed int4, float32 group-128 scales."""
    g = torch.Generator().manual_seed(seed)
    ck = []
    for _ in range(experts):
        gu = torch.randint(-8, 8, (2 * inter, hidden), generator=g, dtype=torch.int8).numpy()
        dn = torch.randint(-8, 8, (hidden, inter), generator=g, dtype=torch.int8).numpy()
        gu_s = torch.rand(2 * inter, hidden // 128, generator=g) * 0.01 + 0.002
        dn_s = torch.rand(hidden, inter // 128, generator=g) * 0.01 + 0.002
        p13 = torch.from_numpy(ow4.pack_int4(gu))
        ck.append(dict(w1=p13[:inter], w3=p13[inter:], w2=torch.from_numpy(ow4.pack_int4(dn)),
                       s1=gu_s[:inter], s3=gu_s[inter:], s2=dn_s))
    return ck


def _w4_layer(ck, hidden, inter, tp_rank, tp_size):
    from vllm_musa_amd.quant_methods import W4AFp8MoEMethod
    m = W4AFp8MoEMethod(swiglu_limit=10.0)
    part = m.maybe_roundup_sizes(hidden, inter // tp_size, torch.bfloat16, None)[1]
    layer = torch.nn.Module()
    m.create_weights(layer, len(ck), hidden, part, torch.bfloat16, device=DEV)
    for e, c in enumerate(ck):
        for sid in ("w1", "w3", "w2"):
            wname = "w13" if sid != "w2" else "w2"
            m.load_weight(layer, f"{wname}_weight", c[sid], e, sid, tp_rank, tp_size)
            m.load_weight(layer, f"{wname}_weight_scale_inv", c["s" + sid[1]], e, sid, tp_rank,
                          tp_size)
    m.process_weights_after_loading(layer)
    return m, layer


def _oracle_layer(layer, x, w, ids):
    f = lambda t: t.float().cpu().numpy()
    return ow4.w4afp8_moe(f(x), layer.w13_weight.cpu().numpy(), layer.w2_weight.cpu().numpy(),
                          f(layer.w13_weight_scale_inv), f(layer.w2_weight_scale_inv),
                          w.cpu().numpy(), ids.cpu().numpy(), None, swiglu_limit=10.0)


def _rel_l2(a, b):
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


@pytest.mark.parametrize("tokens", [16, 300])
def test_w4afp8_tensor_parallel_shards(tokens):
    experts, hidden, inter, topk, tp = 4, 256, 512, 2, 2
    part = inter // tp
    ck = _w4_checkpoint(experts, hidden, inter, seed=tokens)
    g = torch.Generator().manual_seed(1000 + tokens)
    x = (torch.randn(tokens, hidden, generator=g) * 0.3).to(torch.bfloat16).to(DEV)
    ids = torch.stack([torch.randperm(experts, generator=g)[:topk] for _ in range(tokens)]
                      ).to(torch.int32).to(DEV)
    w = torch.softmax(torch.randn(tokens, topk, generator=g), dim=-1).to(DEV)
    m1, full = _w4_layer(ck, hidden, inter, 0, 1)
    out = m1.apply(full, x, w, ids).float().cpu().numpy()
    assert _rel_l2(out, _oracle_layer(full, x, w, ids)) <= 1e-2
    total = np.zeros_like(out)
    for r in range(tp):
        mr, lr = _w4_layer(ck, hidden, inter, r, tp)
        # a rank holds exactly its slices of the unsplit layer (gate rows, up
        # rows, w2 columns; packed bytes and bf16 scales alike)
        rows = lambda t: torch.cat([t[:, r * part:(r + 1) * part],
                                    t[:, inter + r * part:inter + (r + 1) * part]], 1)
        assert torch.equal(lr.w13_weight, rows(full.w13_weight))
        assert torch.equal(lr.w13_weight_scale_inv, rows(full.w13_weight_scale_inv))
        assert torch.equal(lr.w2_weight, full.w2_weight[:, :, r * part // 2:(r + 1) * part // 2])
        assert torch.equal(lr.w2_weight_scale_inv,
                           full.w2_weight_scale_inv[:, :, r * part // 128:(r + 1) * part // 128])
        o = mr.apply(lr, x, w, ids).float().cpu().numpy()
        ref = _oracle_layer(lr, x, w, ids)
        assert _rel_l2(o, ref) <= 1e-2
        assert np.abs(o - ref).max() <= 2e-2 * np.abs(ref).max()
        total += o
    # The ranks' partial sums add up to the unsplit layer up to fp8 rounding:
    # the down projection's input is quantised per row, and a rank's row
    # maximum covers only its half of I, so the e4m3 codes (3 mantissa bits)
    # differ between a shard and the whole.
    assert _rel_l2(total, out) <= 5e-2
