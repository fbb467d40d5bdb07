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
- one expert, top-1, weight 1: the output is the expert output y;
- the kernels' int4 operand encoding (mfma_fp8.h w4_frag): restated
  bit-for-bit on the host, every code decodes (torch's float8_e4m3fn) to
  (x + 8) / 512, the accumulator-input correction recovers the int4 dot
  product exactly, and the byte planes follow the activations' w4 order.
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


def _bitop3(s0: int, s1: int, s2: int, table: int) -> int:
    """v_bitop3_b32: bit i of the result is bit (s0_i << 2 | s1_i << 1 | s2_i)
    of the 8-bit truth table (s0 -> 0xF0, s1 -> 0xCC, s2 -> 0xAA)."""
    out = 0
    for i in range(32):
        idx = (((s0 >> i) & 1) << 2) | (((s1 >> i) & 1) << 1) | ((s2 >> i) & 1)
        out |= ((table >> idx) & 1) << i
    return out


def _w4_frag_word(w: int) -> tuple[int, int]:
    """Host restatement of one word of the kernels' w4_frag (mfma_fp8.h):
    8 packed int4 -> (even-element plane, odd-element plane) of e4m3 codes."""
    even = _bitop3(w, 0x88888888, 0x0F0F0F0F, 0x28)
    odd = _bitop3(w >> 4, 0x88888888, 0x0F0F0F0F, 0x28)
    return even, odd


def test_bitop3_table_0x28_is_xor_then_and():
    g = np.random.Generator(np.random.PCG64(3))
    for a, b, c in g.integers(0, 1 << 32, (200, 3), dtype=np.uint64).tolist():
        assert _bitop3(a, b, c, 0x28) == (a ^ b) & c


W4_ORDER = [0, 2, 4, 6, 1, 3, 5, 7]  # element of each byte position within 8 K-elements


def test_w4_codes_are_the_int4_value_plus_8_times_2_pow_minus_9():
    """Every nibble in every position: the code w4_frag emits at the position
    the w4 order gives decodes (torch's float8_e4m3fn) to (x + 8) / 512 exactly."""
    g = np.random.Generator(np.random.PCG64(5))
    words = list(range(0, 1 << 16, 7)) + [int(w) for w in g.integers(0, 1 << 32, 2000, dtype=np.uint64)]
    words += [0x88888888, 0x77777777, 0xF0F0F0F0, 0x0F0F0F0F, 0x80808080, 0x08080808]
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(torch.float8_e4m3fn).float()
    for t in words:
        even, odd = _w4_frag_word(t)
        planes = (even | (odd << 32))
        for p in range(8):
            code = (planes >> (8 * p)) & 0xFF
            x = (t >> (4 * W4_ORDER[p])) & 0xF
            x = x - 16 if x >= 8 else x
            assert float(codes[code]) == (x + 8) / 512.0, (hex(t), p)


def test_offset_correction_recovers_the_int4_dot_product(rng):
    """sum_k a_k * code_k + c with c = -(sum_k a_k) / 64 equals 2^-9 sum_k a_k x_k
    exactly (float64 over e4m3-valued activations), for any K-permutation that
    both operands share -- the identity the kernels' MFMA accumulator input uses."""
    for _ in range(50):
        a = e4m3_decode(e4m3_encode(rng.standard_normal(128).astype(np.float32) * 100)).astype(np.float64)
        x = rng.integers(-8, 8, 128)
        perm = rng.permutation(128)
        lhs = np.sum(a[perm] * ((x[perm] + 8) / 512.0)) - np.sum(a) / 64.0
        assert lhs == np.sum(a * x) / 512.0


def test_w4_order_matches_the_fragment_planes():
    """A word of 8 consecutive elements expands to [e0, e2, e4, e6 | e1, e3, e5, e7]:
    the order the activation quantisers store each 8-element chunk in."""
    t = 0
    for i in range(8):
        t |= ((i - 4) & 0xF) << (4 * i)  # element i holds value i - 4
    even, odd = _w4_frag_word(t)
    got = [((even | (odd << 32)) >> (8 * p)) & 0xFF for p in range(8)]
    assert [c - 8 + 4 for c in got] == W4_ORDER
