"""bf16 emulation in numpy (test infrastructure).

The reference rounds to bf16 at explicit points: torch bf16 tensors after every op (server.py:511-518,
neural/q80/expert_runtime.py:63-72) and Triton's ``_rb`` (fused_core.py:67-69).  Both are IEEE round-to-nearest-even
from fp32.  ``rb`` returns the rounded value widened back to fp32 so the oracle can keep computing in numpy floats.
"""
import numpy as np


def f32_to_bf16_bits(x) -> np.ndarray:
    """fp32 -> bf16 bit patterns (uint16), round to nearest even; NaN stays NaN (quiet)."""
    a = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = a.view(np.uint32).astype(np.uint64)
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    nan = np.isnan(a)
    out = rounded.astype(np.uint16)
    if nan.any():
        out = np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), out)
    return out


def bf16_bits_to_f32(b) -> np.ndarray:
    b = np.asarray(b, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


def rb(x) -> np.ndarray:
    """Round fp32 values to bf16 and return them as fp32 (torch's ``.to(bfloat16).float()``)."""
    return bf16_bits_to_f32(f32_to_bf16_bits(x))


def f32(x) -> np.ndarray:
    return np.asarray(x, dtype=np.float32)
