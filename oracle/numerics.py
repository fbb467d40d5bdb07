"""Bit-level number formats: OCP float8 e4m3fn and bfloat16 (numpy only).

e4m3fn (OCP FP8, as torch.float8_e4m3fn): 1 sign, 4 exponent (bias 7), 3
mantissa bits; no infinities; S.1111.111 is NaN; largest finite 448;
subnormals m * 2^-9.  Conversion from float32 rounds to nearest, ties to even;
finite values beyond 448 become NaN (torch's CPU cast does the same), but every
caller in this oracle clamps to [-448, 448] first, as the reference quantiser
does (csrc/musa/quantization/per_token_group_quant_8bit_vec.cu:90-93).
"""
from __future__ import annotations

import numpy as np

E4M3_MAX = 448.0


def e4m3_decode_table() -> np.ndarray:
    """float32 value of each of the 256 e4m3fn codes (closed form)."""
    codes = np.arange(256, dtype=np.int64)
    sign = np.where(codes & 0x80, -1.0, 1.0)
    exp = (codes >> 3) & 0xF
    man = codes & 0x7
    val = np.where(exp == 0, man * 2.0 ** -9, (1.0 + man / 8.0) * 2.0 ** (exp - 7.0))
    val = sign * val
    val[(exp == 15) & (man == 7)] = np.nan
    return val.astype(np.float32)


_DECODE = e4m3_decode_table()


def e4m3_decode(q: np.ndarray) -> np.ndarray:
    return _DECODE[np.asarray(q, dtype=np.uint8)]


def e4m3_encode(x: np.ndarray) -> np.ndarray:
    """float32 -> e4m3fn code (uint8), round to nearest even."""
    x = np.asarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.int64)
    sign = ((u >> 31) & 1).astype(np.int64) << 7
    a = np.abs(x).astype(np.float32)
    au = a.view(np.uint32).astype(np.int64)
    exp32 = (au >> 23) - 127
    man32 = au & 0x7FFFFF
    # Normal range (|x| >= 2^-6): keep 3 mantissa bits, RNE on the 20 dropped.
    m3 = (man32 + 0x7FFFF + ((man32 >> 20) & 1)) >> 20  # may carry into 8
    normal_code = ((exp32 + 7) << 3) + m3  # a carry bumps the exponent field
    # Subnormal range: value = m * 2^-9 with m = RNE(|x| * 2^9) (exact scaling).
    a_fin = np.where(a < np.float32(2.0 ** -6), a, np.float32(0.0))  # NaN/large -> 0 here
    sub_m = np.rint(a_fin.astype(np.float64) * 512.0).astype(np.int64)  # rint = half-even
    code = np.where(a < np.float32(2.0 ** -6), sub_m, normal_code)
    nan = np.isnan(x) | (code > 0x7E)
    code = np.where(nan, 0x7F, code) | sign
    return code.astype(np.uint8)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest bfloat16 (ties to even), returned as float32 values."""
    return bf16_decode(bf16_encode(x))


def bf16_encode(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(np.isnan(x), np.uint16(0x7FC0), r).astype(np.uint16)


def bf16_decode(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f16_round(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)
