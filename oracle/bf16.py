"""bfloat16 helpers for the oracle (numpy has no bfloat16 dtype).

bfloat16 is the upper 16 bits of an IEEE float32.  Rounding float32 ->
bfloat16 is round-to-nearest-even on the dropped 16 bits; NaN stays NaN.
"""
import numpy as np


def round_bf16(x) -> np.ndarray:
    """Round to the nearest bfloat16 value (ties to even); result is float32."""
    f = np.ascontiguousarray(x, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) & 0xFFFF0000).astype(np.uint32)
    out = r.view(np.float32).copy()
    nan = np.isnan(f)
    if nan.any():
        out[nan] = np.nan
    return out.reshape(np.shape(x))


def to_bf16_bits(x) -> np.ndarray:
    """float32 -> uint16 bit patterns of the RNE-rounded bfloat16 value."""
    r = round_bf16(x)
    return (r.view(np.uint32) >> 16).astype(np.uint16)


def from_bf16_bits(bits) -> np.ndarray:
    """uint16 bfloat16 bit patterns -> float32 values (exact)."""
    b = np.ascontiguousarray(bits, dtype=np.uint16).astype(np.uint32) << 16
    return b.view(np.float32)
