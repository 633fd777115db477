"""float32 -> bfloat16 rounding on bit patterns (test infrastructure only).

Restates c10::BFloat16's round-to-nearest-even conversion, which is what the
reference's ``tensor.to(torch.bfloat16)`` performs inside
``PagedKVPool.write`` (memforge_ml/runtime/kv_pool.py:134-149). Values are
carried as uint16 bit patterns so the oracle never depends on numpy having a
bfloat16 type.
"""

from __future__ import annotations

import numpy as np


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round float32 values to bfloat16, returning uint16 bit patterns."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    out = np.where(nan, 0x7FC0, rounded & 0xFFFF)
    return out.astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    """Widen bfloat16 bit patterns to float32 (exact)."""
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_to_bf16(x: np.ndarray) -> np.ndarray:
    """float32 values rounded through bfloat16 and back."""
    return bf16_bits_to_f32(f32_to_bf16_bits(x))
