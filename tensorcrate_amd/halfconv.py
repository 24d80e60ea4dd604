"""Host-side f32 -> f16/bf16 conversion for staging inputs, vectorised.

The rounding is the one `half` 2.7.1 applies (`bf16::from_f32`,
`f16::from_f32`): to nearest, ties to even, NaNs quieted.  numpy's own
float16 cast is that rounding; bf16 has no numpy type, so its bits are
formed here and held as uint16.
"""

from __future__ import annotations

import numpy as np


def bf16_bits(values) -> np.ndarray:
    x = np.ascontiguousarray(values, np.float32).view(np.uint32)
    rounded = ((x.astype(np.uint64) + 0x7FFF + ((x >> 16) & 1)) >> 16).astype(np.uint16)
    nan = (x & 0x7FFFFFFF) > 0x7F800000
    if np.any(nan):
        rounded[nan] = ((x[nan] >> 16) | 0x40).astype(np.uint16)
    return rounded


def bf16_to_f32(bits) -> np.ndarray:
    return (np.ascontiguousarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def f16(values) -> np.ndarray:
    return np.ascontiguousarray(values, np.float32).astype(np.float16)
