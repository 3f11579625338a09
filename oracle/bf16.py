"""fp32 -> bf16 bit rules per round mode (numpy, bit-exact).

Restates reference csrc/attention_kernel.hip:110-145 (``bf16_round_one``):

* RTNE: ``u + 0x7FFF + ((u >> 16) & 1)``, keep the top 16 bits
* RTNA: ``u + 0x8000``
* RTZ : ``u`` (truncate)

``canon=True`` maps every NaN to 0x7FFF in all three modes (the reference does
this for RTNE/RTNA under ``MaybeNaN``, :116-140; this build extends it to RTZ).
Without ``canon`` a NaN is still kept a NaN (quiet bit pattern 0x7FC0 | sign);
that matches what the kernels produce for NaNs that come from bf16 inputs.
"""
import numpy as np

RTNE, RTNA, RTZ = 0, 1, 2
MODES = {"rtne": RTNE, "rtna": RTNA, "rtz": RTZ}
CANON_NAN = np.uint16(0x7FFF)


def f32_bits(x):
    return np.ascontiguousarray(np.asarray(x, dtype=np.float32)).view(np.uint32)


def bits_to_f32(u32):
    return np.ascontiguousarray(np.asarray(u32, dtype=np.uint32)).view(np.float32)


def bf16_to_f32(b16):
    """bf16 bit patterns (uint16) -> float32 values."""
    return bits_to_f32(np.asarray(b16, dtype=np.uint16).astype(np.uint32) << np.uint32(16))


def round_bits(x, mode, canon=False):
    """float32 array -> uint16 bf16 bit patterns under ``mode``."""
    u = f32_bits(x).astype(np.uint64)  # widen: no wrap on the bias add
    if mode == RTNE:
        r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    elif mode == RTNA:
        r = (u + 0x8000) >> 16
    elif mode == RTZ:
        r = u >> 16
    else:
        raise ValueError(f"unknown round mode {mode}")
    r = (r & 0xFFFF).astype(np.uint16)
    nan = np.isnan(np.asarray(x, dtype=np.float32))
    if canon:
        r = np.where(nan, CANON_NAN, r)
    else:
        sign = ((f32_bits(x) >> np.uint32(16)) & np.uint32(0x8000)).astype(np.uint16)
        r = np.where(nan, np.uint16(0x7FC0) | sign, r)
    return r.astype(np.uint16)


def round_f32(x, mode, canon=False):
    """Round to bf16 and return the value as float32."""
    return bf16_to_f32(round_bits(x, mode, canon))


def ulp_bf16(mag):
    """bf16 unit in the last place at magnitude ``mag`` (float64 array).

    For |x| in [2^e, 2^(e+1)) the bf16 ULP is 2^(e-7); subnormal range uses
    the minimum normal exponent (2^-133).
    """
    mag = np.abs(np.asarray(mag, dtype=np.float64))
    e = np.floor(np.log2(np.maximum(mag, 2.0 ** -126)))
    return np.exp2(e - 7)
