"""Seeded synthetic workloads of the MoE / block-fp8 path (benchmarks and tests).

All tensors are drawn with a torch.Generator on the target device, so a
multi-GB expert stack is created in HBM without a host round trip; copying a
tensor to the CPU gives the identical bytes for a CPU check.

Distributions (per workload):
  dense block-fp8 : activations ~N(0,1) bf16; weights e4m3fn codes of
                    clip(N(0,1)*64, +-448); scales ~U(0.5, 2)/448 per 128x128 block
  bf16 MoE        : weights ~N(0, 0.02) bf16, activations ~N(0,1), logits ~N(0,1)
  fp8 block MoE   : weights ~N(0, 0.02) quantised per 128x128 block (s = absmax/448)
  w4afp8 MoE      : int4 values U[-8, 7] packed two per byte (even index = low
                    nibble), bf16 scales per (row, 128-K group) ~U(0.002, 0.012)
"""
from __future__ import annotations

import torch

FP8 = torch.float8_e4m3fn


def _gen(seed: int, device) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def dense_fp8_weight(n: int, k: int, seed: int, device="cuda"):
    g = _gen(seed, device)
    w = (torch.randn(n, k, generator=g, device=device) * 64).clamp_(-448, 448).to(FP8)
    ws = (torch.rand((n + 127) // 128, k // 128, generator=g, device=device) * 1.5 + 0.5) / 448.0
    return w, ws


def activations(m: int, k: int, seed: int, device="cuda", scale: float = 1.0):
    g = _gen(seed, device)
    return (torch.randn(m, k, generator=g, device=device) * scale).to(torch.bfloat16)


def quantize_weight_blocks(w: torch.Tensor, block: int = 128):
    """[..., N, K] float -> (e4m3fn [..., N, K], f32 scales [..., N/128, K/128]), s = absmax/448."""
    *lead, n, k = w.shape
    nb, kb = (n + block - 1) // block, k // block
    pad = nb * block - n
    wp = torch.nn.functional.pad(w, (0, 0, 0, pad)) if pad else w
    blk = wp.reshape(*lead, nb, block, kb, block).float()
    amax = blk.abs().amax(dim=(-3, -1)).clamp_min(1e-12)
    s = amax / 448.0
    q = (blk / s[..., :, None, :, None]).clamp_(-448, 448).to(FP8).reshape(*lead, nb * block, k)
    return q[..., :n, :].contiguous(), s.contiguous()


def moe_fp8_weights(e: int, h: int, i: int, seed: int, device="cuda", chunk: int = 16):
    """w13 [E, 2I, H], w2 [E, H, I] e4m3fn + block scales, built chunk by chunk
    of experts so the fp32 staging stays small."""
    g = _gen(seed, device)
    w13 = torch.empty(e, 2 * i, h, dtype=FP8, device=device)
    w13_s = torch.empty(e, (2 * i + 127) // 128, h // 128, dtype=torch.float32, device=device)
    w2 = torch.empty(e, h, i, dtype=FP8, device=device)
    w2_s = torch.empty(e, (h + 127) // 128, i // 128, dtype=torch.float32, device=device)
    for e0 in range(0, e, chunk):
        e1 = min(e, e0 + chunk)
        a = torch.randn(e1 - e0, 2 * i, h, generator=g, device=device) * 0.02
        w13[e0:e1], w13_s[e0:e1] = quantize_weight_blocks(a)
        b = torch.randn(e1 - e0, h, i, generator=g, device=device) * 0.02
        w2[e0:e1], w2_s[e0:e1] = quantize_weight_blocks(b)
        del a, b
    return w13, w13_s, w2, w2_s


def moe_bf16_weights(e: int, h: int, i: int, seed: int, device="cuda"):
    g = _gen(seed, device)
    w13 = (torch.randn(e, 2 * i, h, generator=g, device=device) * 0.02).to(torch.bfloat16)
    w2 = (torch.randn(e, h, i, generator=g, device=device) * 0.02).to(torch.bfloat16)
    return w13, w2


def pack_int4(v: torch.Tensor) -> torch.Tensor:
    """int values in [-8, 7], last dim even -> int8 with element 2j in the low nibble."""
    lo = v[..., 0::2].to(torch.int16) & 15
    hi = (v[..., 1::2].to(torch.int16) & 15) << 4
    return (lo | hi).to(torch.int8)


def moe_w4a8_weights(e: int, h: int, i: int, seed: int, device="cuda"):
    """gateup [E, 2I, H/2] int8 (packed int4), down [E, H, I/2], bf16 scales."""
    g = _gen(seed, device)
    gu = torch.randint(-8, 8, (e, 2 * i, h), generator=g, device=device, dtype=torch.int8)
    dn = torch.randint(-8, 8, (e, h, i), generator=g, device=device, dtype=torch.int8)
    gu_s = (torch.rand(e, 2 * i, h // 128, generator=g, device=device) * 0.01 + 0.002).to(torch.bfloat16)
    dn_s = (torch.rand(e, h, i // 128, generator=g, device=device) * 0.01 + 0.002).to(torch.bfloat16)
    return pack_int4(gu), pack_int4(dn), gu_s, dn_s


def router_logits(t: int, e: int, seed: int, device="cuda", hot: int = 0, hot_bias: float = 2.0):
    """~N(0,1) fp32 logits; `hot` > 0 adds hot_bias to experts 0..hot-1 (skewed routing)."""
    g = _gen(seed, device)
    logits = torch.randn(t, e, generator=g, device=device)
    if hot:
        logits[:, :hot] += hot_bias
    return logits


def score_bias(e: int, seed: int, device="cuda"):
    g = _gen(seed, device)
    return torch.randn(e, generator=g, device=device) * 0.1
