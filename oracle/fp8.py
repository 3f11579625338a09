"""OCP 8-bit float E4M3 ("e4m3fn") decode, restated from the OCP 8-bit
Floating Point Specification (OFP8) v1.0: 1 sign bit, 4 exponent bits (bias 7),
3 mantissa bits; no infinities; S.1111.111 is NaN; max finite 448.

  exponent 0      : (-1)^s * m/8 * 2^-6        (subnormal, incl. signed zero)
  exponent 1..15  : (-1)^s * (1 + m/8) * 2^(e-7)

Every value is exactly representable in bf16 and fp32. The gfx950 build reads
this format (the reference's gfx942 kernels read e4m3fnuz, csrc/mla_decode_a16w8.hip:38).
"""
import numpy as np


def _table():
    t = np.empty(256, dtype=np.float64)
    for b in range(256):
        s = -1.0 if b & 0x80 else 1.0
        e = (b >> 3) & 0xF
        m = b & 0x7
        if e == 0xF and m == 0x7:
            t[b] = np.nan
        elif e == 0:
            t[b] = s * (m / 8.0) * 2.0 ** -6
        else:
            t[b] = s * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return t


DECODE = _table()


def decode(u8):
    """uint8 array of e4m3fn bit patterns -> float64 values."""
    return DECODE[np.asarray(u8, dtype=np.uint8)]
