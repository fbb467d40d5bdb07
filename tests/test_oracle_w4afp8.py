"""Pins of the w4afp8 oracle (oracle/w4afp8.py).

- nibble order and sign: known packed bytes, and pack/unpack as the
  reference test packs (tests/kernels/test_w4afp8_moe.py:18-22, restated with
  torch ops here);
- per-row quantiser: closed-form special cases and torch's float8 cast (the
  cast the reference's own oracle uses, test file 25-28);
- the W13 stage equals the independently pinned block-fp8 path when the
  int4 scales are constant on 128x128 blocks and every 128-group of a row has
  the row's absmax (then per-row and per-group quantisation coincide);
- the W2 scales enter linearly: doubling them doubles the layer exactly;
- one expert, top-1, weight 1: the output is the expert output y.
"""
from __future__ import annotations

import numpy as np
import torch

from oracle import w4afp8 as ow4
from oracle.gemm import block_fp8_matmul_f64
from oracle.numerics import bf16_round, e4m3_decode, e4m3_encode
from oracle.quant import group_quant_fp8


def test_unpack_known_bytes():
    packed = np.array([[0x8F, 0x70, 0x01]], np.uint8).view(np.int8)
    np.testing.assert_array_equal(ow4.unpack_int4(packed), [[-1, -8, 0, 7, 1, 0]])


def test_pack_matches_torch_packing(rng):
    v = rng.integers(-8, 8, (5, 64)).astype(np.int8)
    t = torch.from_numpy(v)
    ref = ((t[..., ::2].to(torch.int16) & 15) | ((t[..., 1::2].to(torch.int16) & 15) << 4)).to(torch.int8)
    np.testing.assert_array_equal(ow4.pack_int4(v), ref.numpy())
    np.testing.assert_array_equal(ow4.unpack_int4(ow4.pack_int4(v)), v)


def test_row_quant_special_cases():
    x = np.zeros((3, 256), np.float32)
    x[1, 7] = 2.0
    x[2, :] = np.linspace(-5, 5, 256, dtype=np.float32)
    q, s = ow4.dynamic_fp8_rows(x)
    assert s[0] == np.float32(1e-4) / np.float32(448)
    assert (q[0] == 0).all()
    assert s[1] == np.float32(2.0) / np.float32(448) and q[1, 7] == 0x7E  # 448
    assert q[2, 0] == 0xFE and q[2, -1] == 0x7E


def test_row_quant_matches_torch_cast(rng):
    x = (rng.standard_normal((17, 384)) * rng.uniform(1e-3, 30, (17, 1))).astype(np.float32)
    q, s = ow4.dynamic_fp8_rows(x)
    xt = torch.from_numpy(x)
    st = xt.abs().amax(dim=-1, keepdim=True).clamp_min(1e-4) / 448.0
    qt = (xt / st).clamp(-448, 448).to(torch.float8_e4m3fn)
    np.testing.assert_array_equal(s, st[:, 0].numpy())
    np.testing.assert_array_equal(q, qt.view(torch.uint8).numpy())


def _block_case(rng, t=6, h=256, i=128, e=2):
    # every 128-group of each row holds the row's absmax at one position
    x = (rng.standard_normal((t, h)) * 0.3).astype(np.float32)
    for g in range(h // 128):
        x[:, g * 128 + 5] = 3.0
    x = bf16_round(x)
    vals = rng.integers(-8, 8, (e, 2 * i, h)).astype(np.int8)
    blk = rng.uniform(0.002, 0.012, (e, 2 * i // 128, h // 128)).astype(np.float32)
    blk = bf16_round(blk)
    row_scale = np.repeat(blk, 128, axis=1)  # [E, 2I, H/128]: constant on 128x128 blocks
    w2v = rng.integers(-8, 8, (e, h, i)).astype(np.int8)
    s2 = bf16_round(rng.uniform(0.002, 0.012, (e, h, i // 128)).astype(np.float32))
    return x, vals, blk, row_scale, w2v, s2


def test_w13_stage_equals_block_fp8_path(rng):
    x, vals, blk, row_scale, w2v, s2 = _block_case(rng)
    t = x.shape[0]
    ids = np.zeros((t, 1), np.int32)
    ids[::2] = 1
    w = np.ones((t, 1), np.float32)
    _, hs = ow4.w4afp8_moe(x, ow4.pack_int4(vals), ow4.pack_int4(w2v), row_scale, s2, w, ids,
                           return_h=True)
    xq, xs = group_quant_fp8(x)  # per-group scales == the row scale in every group
    for e, (tt, kk, hh) in hs.items():
        codes = e4m3_encode(vals[e].astype(np.float32))  # int4 values are exact e4m3
        ref = bf16_round(block_fp8_matmul_f64(xq[tt], xs[tt], codes, blk[e]).astype(np.float32))
        np.testing.assert_array_equal(hh, ref)


def test_w2_scales_enter_linearly(rng):
    x, vals, blk, row_scale, w2v, s2 = _block_case(rng, t=5)
    ids = np.stack([rng.permutation(2) for _ in range(5)]).astype(np.int32)
    w = rng.uniform(0.1, 1, (5, 2)).astype(np.float32)
    a = ow4.w4afp8_moe(x, ow4.pack_int4(vals), ow4.pack_int4(w2v), row_scale, s2, w, ids,
                       swiglu_limit=10.0)
    b = ow4.w4afp8_moe(x, ow4.pack_int4(vals), ow4.pack_int4(w2v), row_scale, 2 * s2, w, ids,
                       swiglu_limit=10.0)
    np.testing.assert_array_equal(b, 2 * a)


def test_single_route_output_is_expert_output(rng):
    x, vals, blk, row_scale, w2v, s2 = _block_case(rng, t=3, e=1)
    ids = np.zeros((3, 1), np.int32)
    w = np.ones((3, 1), np.float32)
    out = ow4.w4afp8_moe(x, ow4.pack_int4(vals), ow4.pack_int4(w2v), row_scale, s2, w, ids)
    # the expert output computed directly with torch (reference test's formula, float64)
    xt = torch.from_numpy(x).double()
    sx = xt.abs().amax(-1, keepdim=True).clamp_min(1e-4) / 448.0
    xd = (xt.float() / sx.float()).clamp(-448, 448).to(torch.float8_e4m3fn).double() * sx.float().double()
    g13 = torch.from_numpy(vals[0]).double() * torch.from_numpy(row_scale[0]).double().repeat_interleave(128, -1)
    h = (xd @ g13.T).float().bfloat16().float()
    i = h.shape[-1] // 2
    a = (torch.nn.functional.silu(h[:, :i]) * h[:, i:]).bfloat16().float()
    sa = a.abs().amax(-1, keepdim=True).clamp_min(1e-4) / 448.0
    ad = (a / sa).clamp(-448, 448).to(torch.float8_e4m3fn).double() * sa.double()
    g2 = torch.from_numpy(w2v[0]).double() * torch.from_numpy(s2[0]).double().repeat_interleave(128, -1)
    y = (ad @ g2.T).float().bfloat16().float()
    np.testing.assert_array_equal(out, y.numpy())


def test_expert_map_drops_routes(rng):
    x, vals, blk, row_scale, w2v, s2 = _block_case(rng, t=4)
    gids = np.array([[0, 3], [2, 1], [3, 2], [1, 0]], np.int32)
    emap = np.array([-1, -1, 0, 1], np.int32)
    w = rng.uniform(0.1, 1, (4, 2)).astype(np.float32)
    got = ow4.w4afp8_moe(x, ow4.pack_int4(vals), ow4.pack_int4(w2v), row_scale, s2, w, gids,
                         expert_map=emap)
    loc = np.where(gids >= 2, gids - 2, 0).astype(np.int32)
    w0 = np.where(gids >= 2, w, 0).astype(np.float32)
    np.testing.assert_array_equal(
        got, ow4.w4afp8_moe(x, ow4.pack_int4(vals), ow4.pack_int4(w2v), row_scale, s2, w0, loc))


def test_e4m3_of_int4_values():
    v = np.arange(-8, 8, dtype=np.float32)
    np.testing.assert_array_equal(e4m3_decode(e4m3_encode(v)), v)


def _perm(s0: int, s1: int, sel: int) -> int:
    """v_perm_b32: byte i of the result from selector byte sel_i over the 8
    bytes of {s0:s1} (s1 low): 0..7 pick a byte; 8, 9, 10, 11 replicate bit 7
    of byte 1, 3, 5, 7; 12 gives 0x00 and 13..255 give 0xFF."""
    data = (s0 << 32) | s1
    out = 0
    for i in range(4):
        k = (sel >> (8 * i)) & 0xFF
        if k < 8:
            b = (data >> (8 * k)) & 0xFF
        elif k < 12:
            b = 0xFF * ((data >> (8 * (2 * (k - 8) + 1) + 7)) & 1)
        else:
            b = 0x00 if k == 12 else 0xFF
        out |= b << (8 * i)
    return out


def _int4x8_to_fp8(x: int) -> int:
    """Host restatement of the kernels' nibble -> e4m3 conversion (mfma_fp8.h):
    8 packed int4 in a dword -> 8 e4m3 codes (64 bits, element order)."""
    m32 = 0xFFFFFFFF
    se, so = x & 0x07070707, (x >> 4) & 0x07070707
    qe = (x << 4) & m32
    me = _perm((qe << 8) & m32, qe, 0x090B080A)
    mo = _perm((x << 8) & m32, x, 0x090B080A)
    ce = (_perm(0xB8C0C4C8, 0xCACCCED0, se) & me) | (_perm(0x4E4C4A48, 0x44403800, se) & ~me & m32)
    co = (_perm(0xB8C0C4C8, 0xCACCCED0, so) & mo) | (_perm(0x4E4C4A48, 0x44403800, so) & ~mo & m32)
    return _perm(co, ce, 0x05010400) | (_perm(co, ce, 0x07030602) << 32)


def test_perm_emulation_known_selectors():
    """The emulated v_perm_b32 on selectors whose results the ISA fixes."""
    assert _perm(0x07060504, 0x03020100, 0x07050301) == 0x07050301
    assert _perm(0, 0x00008000, 0x08080808) == 0xFFFFFFFF  # bit 15 -> selector 8
    assert _perm(0x80000000, 0, 0x0B0B0B0B) == 0xFFFFFFFF  # bit 63 -> selector 11
    assert _perm(0xFFFFFFFF, 0xFFFFFFFF, 0x0D0C0D0C) == 0xFF00FF00


def test_kernel_nibble_table_is_e4m3_of_the_int4_value():
    g = np.random.Generator(np.random.PCG64(5))
    words = list(range(0, 1 << 16, 7)) + [int(w) for w in g.integers(0, 1 << 32, 4000, dtype=np.uint64)]
    words += [0x88888888, 0x77777777, 0xF0F0F0F0, 0x0F0F0F0F, 0x80808080, 0x08080808]
    for t in words:  # every nibble value in every position, many combinations
        out = _int4x8_to_fp8(t)
        for i in range(8):
            v = (t >> (4 * i)) & 0xF
            v = v - 16 if v >= 8 else v
            assert (out >> (8 * i)) & 0xFF == int(e4m3_encode(np.float32(v))), (hex(t), i)
