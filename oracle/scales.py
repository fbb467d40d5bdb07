"""Checkpoint scale conversion (TEST INFRASTRUCTURE ONLY: the checker of
vmamd_convert_scales and of the loaders built on it).

  upcast_e8m0_to_fp32   e8m0 byte b -> float32 bits b << 23
                        (vllm_musa/model_executor/layers/quantization/utils/fp8_utils.py:13-15)
  convert_scales        {e8m0, f32, bf16} -> {f32, bf16}; f32 -> bf16 rounds
                        to nearest even (torch's .to(bfloat16)), plus the count
                        of results that are not finite and positive
  w4afp8_scales         the cast + check of MusaW4AFp8MoEMethod.process_weights_after_loading
                        (model_executor/layers/quantization/w4afp8.py:126-131)

Pinned in tests/test_oracle_scales.py against closed forms, torch's own
float8_e8m0fnu and bfloat16 casts, and the invalid values of the reference's
test_invalid_loaded_scales_fail_before_kernel_launch
(tests/test_w4afp8_quantization.py:207-224).
"""
from __future__ import annotations

import numpy as np

from .numerics import bf16_decode, bf16_encode

KINDS = ("e8m0", "f32", "bf16")


def upcast_e8m0_to_fp32(bits: np.ndarray) -> np.ndarray:
    """fp8_utils.py:13-15: (uint8 -> int32) << 23, viewed as float32."""
    return (np.asarray(bits, dtype=np.uint8).astype(np.uint32) << 23).view(np.float32)


def to_f32(src: np.ndarray, kind: str) -> np.ndarray:
    """Source encoding -> float32 values (bf16 given as its uint16 bit patterns)."""
    if kind == "e8m0":
        return upcast_e8m0_to_fp32(src)
    if kind == "bf16":
        return bf16_decode(src)
    if kind == "f32":
        return np.asarray(src, dtype=np.float32)
    raise ValueError(kind)


def invalid_count(values: np.ndarray) -> int:
    """Number of values that are not finite and positive (NaN, +-inf, <= 0)."""
    v = np.asarray(values, dtype=np.float32)
    return int(np.count_nonzero(~(np.isfinite(v) & (v > 0))))


def convert_scales(src: np.ndarray, src_kind: str, dst_kind: str) -> tuple[np.ndarray, int]:
    """Returns (destination in its storage encoding: float32 values or bf16
    uint16 bits, invalid count of the destination values)."""
    f = to_f32(src, src_kind)
    if dst_kind == "f32":
        return f, invalid_count(f)
    if dst_kind == "bf16":
        h = bf16_encode(f)
        return h, invalid_count(bf16_decode(h))
    raise ValueError(dst_kind)


def w4afp8_scales(scales_f32: np.ndarray) -> tuple[np.ndarray, bool]:
    """w4afp8.py:126-131: bf16 bits of the scales, and whether every one is
    finite and positive after the cast."""
    h, bad = convert_scales(scales_f32, "f32", "bf16")
    return h, bad == 0


__all__ = ["KINDS", "upcast_e8m0_to_fp32", "to_f32", "invalid_count", "convert_scales",
           "w4afp8_scales"]
