"""bfloat16 rounding on numpy arrays, by bit arithmetic.

Round-to-nearest-even of the float32 value to its top 16 bits; NaN becomes the
canonical quiet NaN 0x7fc0 (torch's float -> bfloat16 conversion does the same).
Reference use: every `.to(torch.bfloat16)` boundary of the hot path, e.g.
slimkv/llama3/decode_kernels.py:44-51.
"""
import numpy as np


def to_bits(x):
    """float array -> uint16 bf16 bit patterns (round to nearest even)."""
    f = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = f.view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    rounded = np.where(nan, 0x7FC0, rounded)
    return rounded.astype(np.uint16)


def from_bits(bits):
    """uint16 bf16 bit patterns -> float32 values."""
    b = np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16
    return b.view(np.float32)


def round_bf16(x):
    """Values of x rounded to bf16, returned as float32 (float64 input is first
    rounded to float32, as torch does for a float64 -> bf16 cast via float)."""
    return from_bits(to_bits(x))
