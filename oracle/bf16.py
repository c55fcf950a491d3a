"""bf16 rounding in numpy, used to emulate torch's bf16 elementwise ops.

torch rounds a bf16 op's fp32 result to the nearest bf16, ties to even; NaN
stays NaN. Pinned in tests against torch's own ``.to(torch.bfloat16)`` on
random and boundary values (ties, overflow to inf, subnormals).
"""

from __future__ import annotations

import numpy as np


def round_bf16(x: np.ndarray) -> np.ndarray:
    """Round float32 values to the nearest bfloat16 (ties to even); return float32."""

    a = np.ascontiguousarray(x, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    nan = np.isnan(a)
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    out = (rounded << 16).astype(np.uint32).view(np.float32)
    out = np.where(nan, np.float32(np.nan), out)
    return out.reshape(a.shape)


def rounder(dtype: str):
    """Return the per-op rounding function of a storage dtype ("bf16" or "f32")."""

    if dtype == "bf16":
        return round_bf16
    if dtype == "f32":
        return lambda x: np.asarray(x, dtype=np.float32)
    raise ValueError(f"unknown dtype {dtype!r}")
