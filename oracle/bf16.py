"""bfloat16 helpers on numpy arrays (oracle; test infrastructure only).

bf16 values are held as uint16 bit patterns or as the float32 values they represent.
Rounding is IEEE round-to-nearest-even, the rule of torch's float->bfloat16 conversion and of
gfx950's v_cvt_pk_bf16_f32.
"""

from __future__ import annotations

import numpy as np


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round float32 values to bfloat16 (RNE); returns uint16 bit patterns."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        rounded = rounded.copy()
        rounded[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)  # quiet NaN, sign kept
    return rounded


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest bfloat16 value, returned as float32."""
    return bf16_bits_to_f32(f32_to_bf16_bits(x))


def round_f64_to_bf16(x: np.ndarray) -> np.ndarray:
    """float64 -> nearest bfloat16 (single rounding, RNE), returned as float32.

    Candidates are the bf16 neighbours of the float32 truncation toward zero; the nearer one
    in float64 wins and exact ties go to the even significand.
    """
    x = np.asarray(x, dtype=np.float64)
    out = np.empty(x.shape, dtype=np.float32)
    finite = np.isfinite(x)
    f = x.astype(np.float32)  # may round up in magnitude; fixed below
    bits = f.view(np.uint32)
    # Truncate the float32 to bf16 (toward zero) and take the next bf16 away from zero.
    low_bits = (bits & 0xFFFF0000).astype(np.uint32)
    low = low_bits.view(np.float32).astype(np.float64)
    # If the float32 rounding went past x, step the truncation back by one bf16 ulp.
    over = np.abs(low) > np.abs(x)
    low_bits = np.where(over & finite, low_bits - 0x10000, low_bits).astype(np.uint32)
    low = low_bits.view(np.float32).astype(np.float64)
    high_bits = (low_bits + 0x10000).astype(np.uint32)
    high = high_bits.view(np.float32).astype(np.float64)
    d_low = np.abs(x - low)
    d_high = np.abs(high - x)
    even_low = ((low_bits >> 16) & 1) == 0
    choose_low = (d_low < d_high) | ((d_low == d_high) & even_low)
    chosen = np.where(choose_low, low_bits, high_bits).astype(np.uint32)
    out[...] = chosen.view(np.float32)
    zero = finite & (x == 0)
    out[zero] = x[zero].astype(np.float32)
    out[~finite] = x[~finite].astype(np.float32)
    return out


def random_bf16(rng: np.random.Generator, shape, scale: float = 1.0) -> np.ndarray:
    """bf16(N(0, scale^2)) as float32 values."""
    return round_f32_to_bf16((rng.standard_normal(shape) * scale).astype(np.float32))
