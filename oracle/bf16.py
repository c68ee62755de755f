"""BF16 <-> FP32 at the bit level, in numpy (test infrastructure only).

BF16 is the top 16 bits of an IEEE binary32. Rounding FP32 to BF16 is
round-to-nearest-even on the low 16 bits; every NaN becomes the canonical quiet
NaN 0x7FC0. This is torch's c10::BFloat16 rule, which the reference relies on
every time it casts with ``.to(torch.bfloat16)`` or Triton's ``.to(tl.bfloat16)``
(engine/kernels/linear.py:1-6, engine/kernels/rmsnorm.py:35-46).
"""

import numpy as np

CANONICAL_NAN = np.uint16(0x7FC0)


def round_bits(values):
    """FP32 (or anything castable to it) -> BF16 bit patterns, uint16, RNE."""
    f = np.ascontiguousarray(np.asarray(values, dtype=np.float32))
    u = f.view(np.uint32).astype(np.uint64)
    bias = ((u >> 16) & 1) + 0x7FFF
    out = ((u + bias) >> 16).astype(np.uint16)
    nan = np.isnan(f)
    if nan.any():
        out = np.where(nan, CANONICAL_NAN, out).astype(np.uint16)
    return out


def to_f32(bits):
    """BF16 bit patterns (uint16) -> FP32 values (exact)."""
    b = np.ascontiguousarray(np.asarray(bits, dtype=np.uint16))
    return (b.astype(np.uint32) << 16).view(np.float32)


def round_f32(values):
    """FP32 -> nearest BF16 value, returned as FP32 (one rounding)."""
    return to_f32(round_bits(values))


def from_f64(values):
    """FP64 -> BF16 bits through FP32 (the FP32 rounding first, as a kernel's FP32 sum would be)."""
    return round_bits(np.asarray(values, dtype=np.float64).astype(np.float32))


def ulp(values):
    """One BF16 step at the magnitude of ``values`` (fp64), as agent/local_cpu/interp/run_numeric.py:59 measures it."""
    v = np.abs(np.asarray(values, dtype=np.float64))
    v = np.maximum(v, 1e-30)
    return np.exp2(np.floor(np.log2(v))) / 128.0
