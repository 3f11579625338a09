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


def encode(x_f32, saturate=False):
    """float32 array -> e4m3fn bits (uint8) with torch's float8_e4m3fn cast
    (round to nearest even; |x| > 464 -> NaN, NaN -> NaN). With ``saturate``
    every non-NaN value is first clamped to [-448, 448] (the OCP "satfinite"
    conversion)."""
    import torch

    x = torch.from_numpy(np.ascontiguousarray(np.asarray(x_f32, dtype=np.float32)))
    if saturate:
        x = torch.where(torch.isnan(x), x, x.clamp(-448.0, 448.0))
    return x.to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def quantize_rows(c_kv_f32, k_pe_f32, kv_scale, saturate=False):
    """The KV producer's rows: encode(fl32(x / kv_scale)) of [c_kv | k_pe]
    (fp32 division, as the reference's tests fill the cache,
    tests/test_mla_decode.py:34-38). Inputs [N, 512] / [N, 64] float32."""
    import torch

    x = torch.cat([torch.from_numpy(np.asarray(c_kv_f32, np.float32)),
                   torch.from_numpy(np.asarray(k_pe_f32, np.float32))], dim=1)
    return encode((x / np.float32(kv_scale)).numpy(), saturate)
