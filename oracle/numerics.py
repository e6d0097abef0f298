"""Round-to-nearest-even emulation of bf16 and fp16 storage in numpy.

Test infrastructure only (see ``oracle/__init__.py``).

The fused kernel of the reference rounds at three points
(``fused_attn.py:344-345`` Q_rot, ``:389-390`` K_rot, ``:413`` P before the
PV product) and at the store (``:423``).  These helpers reproduce those
roundings on fp32 arrays so that the diagnostic oracle can model them.
"""
import numpy as np


def round_bf16(x: np.ndarray) -> np.ndarray:
    """Round fp32 values to the nearest bf16 (ties to even); return fp32."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) >> 16) << 16
    out = r.astype(np.uint32).view(np.float32).copy()
    nan = np.isnan(x)
    if nan.any():
        out[nan] = np.nan
    return out


def round_f16(x: np.ndarray) -> np.ndarray:
    """Round fp32 values to the nearest fp16 (ties to even); return fp32."""
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    """Round to ``dtype`` in {"bf16", "f16", "f32"} and return fp32."""
    if dtype == "bf16":
        return round_bf16(x)
    if dtype == "f16":
        return round_f16(x)
    if dtype == "f32":
        return np.asarray(x, dtype=np.float32)
    raise ValueError(f"unknown dtype {dtype!r}")


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """bf16 bit patterns (uint16) of fp32 values after RNE rounding."""
    return (round_bf16(x).view(np.uint32) >> 16).astype(np.uint16)


def from_bf16_bits(b: np.ndarray) -> np.ndarray:
    """fp32 values of bf16 bit patterns."""
    return (np.asarray(b, dtype=np.uint32) << 16).view(np.float32)
