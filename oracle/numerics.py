"""Rounding helpers that mirror torch's rounding points (test infrastructure only).

torch computes a bf16 reduction (``mean``, ``matmul``, ``+``) by accumulating
in fp32 and rounding the fp32 result to bf16 with round-to-nearest-even
(c10::BFloat16 ``round_to_nearest_even``). The oracle takes the *exact* value
of the reduction (float64; exact for the sizes used here, see ``exact_sum``),
rounds it to fp32 (RNE) and then to bf16 (RNE). That is torch's result with an
ideal accumulator; a real fp32 accumulator can differ from it only when the
exact value lies within a few fp32 ulps of a bf16 rounding midpoint.

Values are carried as float64 arrays holding dtype-representable numbers.
"""
import numpy as np

DTYPES = ("f32", "bf16", "f16")


def f32_to_bf16_bits(x):
    """fp32 -> bf16 bit pattern (uint16), round-to-nearest-even, NaN -> 0x7FC0."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = x.view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        rounded = np.where(nan, np.uint16(0x7FC0), rounded)
    return rounded


def bf16_bits_to_f32(b):
    b = np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16
    return b.view(np.float32)


def round_f32(x):
    """Round (float64) values to fp32, RNE; returned as float64."""
    return np.asarray(x, dtype=np.float64).astype(np.float32).astype(np.float64)


def round_bf16(x):
    """Round to bf16 through fp32 (torch: fp32 accumulator -> bf16); float64 out."""
    x32 = np.asarray(x, dtype=np.float64).astype(np.float32)
    return bf16_bits_to_f32(f32_to_bf16_bits(x32)).astype(np.float64)


def round_f16(x):
    x32 = np.asarray(x, dtype=np.float64).astype(np.float32)
    return x32.astype(np.float16).astype(np.float64)


def round_to(x, dtype):
    if dtype == "f32":
        return round_f32(x)
    if dtype == "bf16":
        return round_bf16(x)
    if dtype == "f16":
        return round_f16(x)
    raise ValueError(f"unknown dtype {dtype!r}")


def exact_sum(x, axis):
    """Sum in float64. Exact whenever the addends' exponent spread plus
    log2(count) stays under 53 - significand bits (bf16: 8, fp32: 24), which
    holds for the N(0,1)-derived inputs used by the tests; then the result does
    not depend on the summation order, so GPU kernels that accumulate in fp64
    in any order return the same value."""
    return np.sum(np.asarray(x, dtype=np.float64), axis=axis)


def torch_dtype_name(t):
    """Map a torch dtype to the oracle's dtype tag."""
    import torch
    return {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16"}[t]
