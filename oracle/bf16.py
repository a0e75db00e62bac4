"""bfloat16 in numpy: uint16 bit patterns, round-to-nearest-even packing. Test infrastructure only.

Round-to-nearest-even on the top 16 bits of the fp32 pattern is the conversion the reference's Metal kernels apply to
the z column and to bf16 outputs (metal_score.py:31-40, metal_attend.py:30-35); NaN stays NaN, infinities stay.
"""
from __future__ import annotations

import numpy as np


def to_f32(bits: np.ndarray) -> np.ndarray:
    """uint16 bf16 patterns -> float32 values."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def from_f32(x) -> np.ndarray:
    """float32 values -> uint16 bf16 patterns, round to nearest, ties to even."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    special = (u & 0x7F800000) == 0x7F800000
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    top = (u >> 16) & 0xFFFF
    nan = special & ((u & 0x007FFFFF) != 0)
    out = np.where(special, np.where(nan, top | 0x40, top), rounded)
    return out.astype(np.uint16)


def round_f32(x) -> np.ndarray:
    """float32 -> nearest bf16 value, as float32."""
    return to_f32(from_f32(x))


def from_torch(t) -> np.ndarray:
    """A torch bfloat16 tensor (any device) -> uint16 patterns."""
    import torch
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def values(t) -> np.ndarray:
    """A torch tensor (bf16/fp16/fp32, any device) -> float64 numpy values."""
    return t.detach().cpu().float().numpy().astype(np.float64)
