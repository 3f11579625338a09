"""CPU pinning of the fp8 decode and the MLA oracle (no GPU)."""
import math

import numpy as np
import pytest
import torch

from oracle import bf16 as ob
from oracle import fp8 as of8
from oracle import mla as om
from mla_inputs import KV_SCALE, QK, SCALE_576, fp8_bits, paged_pool, rand_kv_rows, rand_q


@pytest.mark.parametrize("code,value", [
    (0x00, 0.0), (0x80, -0.0), (0x38, 1.0), (0xB8, -1.0), (0x7E, 448.0), (0xFE, -448.0),
    (0x01, 2.0 ** -9), (0x08, 2.0 ** -6), (0x07, 7 * 2.0 ** -9), (0x39, 1.125), (0x40, 2.0),
])
def test_fp8_known_answers(code, value):
    got = of8.DECODE[code]
    assert got == value and math.copysign(1.0, got) == math.copysign(1.0, value)


def test_fp8_nan_codes():
    assert np.isnan(of8.DECODE[0x7F]) and np.isnan(of8.DECODE[0xFF])
    assert np.isnan(of8.DECODE).sum() == 2


def test_fp8_matches_torch_float8_e4m3fn():
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    t = codes.view(torch.float8_e4m3fn).float().numpy().astype(np.float64)
    nan = np.isnan(of8.DECODE)
    assert np.array_equal(np.isnan(t), nan)
    assert np.array_equal(t[~nan], of8.DECODE[~nan])


def test_fp8_values_exact_in_bf16():
    vals = of8.DECODE[~np.isnan(of8.DECODE)].astype(np.float32)
    assert np.array_equal(ob.round_f32(vals, ob.RTZ), vals)


def test_oracle_close_to_fp32_formula():
    B, S, H, q_len = 2, 700, 8, 3
    kv = rand_kv_rows(B * S, 3).view(B, S, QK)
    q_lat, q_pe = rand_q(B, q_len, H, 3)
    u8 = fp8_bits(kv)
    ql, qp = q_lat.float().numpy(), q_pe.float().numpy()
    _, pre, _ = om.decode(ql, qp, u8, [S] * B, SCALE_576, KV_SCALE, aux=True)
    ref = om.fp32_reference(ql, qp, u8, [S] * B, SCALE_576, KV_SCALE)
    rel = np.linalg.norm(pre - ref) / np.linalg.norm(ref)
    assert rel < 2e-3  # bf16 P rounding only


def test_window_is_end_aligned_bruteforce():
    """Position t sees exactly S - q_len + t + 1 tokens: changing token j moves
    position t iff j < S - q_len + t + 1."""
    B, S, H, q_len = 1, 40, 4, 3
    kv = rand_kv_rows(S, 5).view(1, S, QK)
    q_lat, q_pe = rand_q(B, q_len, H, 5)
    ql, qp = q_lat.float().numpy(), q_pe.float().numpy()
    base = om.decode(ql, qp, fp8_bits(kv), [S], SCALE_576, KV_SCALE)
    for j in (S - 3, S - 2, S - 1):
        kv2 = kv.clone()
        kv2[0, j] = rand_kv_rows(1, 100 + j)[0]
        out = om.decode(ql, qp, fp8_bits(kv2), [S], SCALE_576, KV_SCALE)
        for t in range(q_len):
            sees = j < S - q_len + t + 1
            assert (not np.array_equal(out[0, t], base[0, t])) == sees, (j, t)


def test_paged_equals_contiguous():
    lens = [130, 70]
    pool, idx, indptr = paged_pool(lens, 9)
    B, H, q_len = 2, 4, 2
    q_lat, q_pe = rand_q(B, q_len, H, 9)
    ql, qp = q_lat.float().numpy(), q_pe.float().numpy()
    pu8 = fp8_bits(pool).reshape(-1, QK)
    slab = np.zeros((B, max(lens), QK), dtype=np.uint8)
    for b in range(B):
        rows = idx[indptr[b]:indptr[b] + lens[b]].numpy()
        slab[b, :lens[b]] = pu8[rows]
    a = om.decode(ql, qp, pu8, lens, SCALE_576, KV_SCALE, kv_indices=idx.numpy(), kv_indptr=indptr.numpy())
    c = om.decode(ql, qp, slab, lens, SCALE_576, KV_SCALE)
    assert np.array_equal(a, c)


def test_rows_remap():
    lens = [50, 60, 70]
    pool, idx, indptr = paged_pool(lens, 13)
    q_lat, q_pe = rand_q(3, 1, 4, 13)
    ql, qp = q_lat.float().numpy(), q_pe.float().numpy()
    base = om.decode(ql, qp, fp8_bits(pool), lens, SCALE_576, KV_SCALE, kv_indices=idx.numpy(),
                     kv_indptr=indptr.numpy())
    rows = np.array([2, 1, 0])
    rev = om.decode(ql[::-1].copy(), qp[::-1].copy(), fp8_bits(pool), lens, SCALE_576, KV_SCALE,
                    kv_indices=idx.numpy(), kv_indptr=indptr.numpy(), rows=rows)
    assert np.array_equal(rev[::-1], base)


def test_torch_formula_cpu_matches_numpy_fp32_reference():
    """The bench's CPU baseline (torch, paged gather) against the numpy fp32
    formula of the reference test (tests/test_mla_decode.py:50-66)."""
    from mla_inputs import paged_pool, rand_q

    lens = [70, 129, 64]
    pool, idx, indptr = paged_pool(lens, 9)
    q_lat, q_pe = rand_q(3, 2, 4, 9)
    got = om.torch_formula_cpu(q_lat, q_pe, pool, torch.tensor(lens, dtype=torch.int32), idx, indptr,
                               SCALE_576, KV_SCALE).numpy()
    ref = om.fp32_reference(q_lat.float().numpy(), q_pe.float().numpy(), pool.view(torch.uint8).numpy(), lens,
                            SCALE_576, KV_SCALE, kv_indices=idx.numpy(), kv_indptr=indptr.numpy())
    assert np.allclose(got, ref, rtol=1e-4, atol=1e-5)


# fp32 value -> expected e4m3fn bits, derived by hand from the OCP spec:
# 1.0 = 0.0111.000; 448 = max finite 0.1111.110; 464 = halfway 448..480 -> even
# (448); above it no finite value is nearer -> NaN (torch's cast); 2^-6 =
# smallest normal 0.0001.000; 2^-9 = smallest subnormal; 2^-10 = halfway 0..2^-9
# -> even (0); 1.5 * 2^-10 -> 2^-9; 1.0625 = 1 + 1/16, halfway 1..1.125 -> 1.0;
# -3 = -1.5 * 2^1 = 1.1000.100, -2 = 1.1000.000;
# 1.1875 halfway 1.125..1.25 -> even mantissa (1.25 = 0.0111.010).
ENCODE_KAT = [
    (1.0, 0x38, 0x38), (448.0, 0x7E, 0x7E), (464.0, 0x7E, 0x7E), (465.0, 0x7F, 0x7E), (1e6, 0x7F, 0x7E),
    (-1e6, 0xFF, 0xFE), (np.inf, 0x7F, 0x7E), (-np.inf, 0xFF, 0xFE), (2.0 ** -6, 0x08, 0x08),
    (2.0 ** -9, 0x01, 0x01), (2.0 ** -10, 0x00, 0x00), (1.5 * 2.0 ** -10, 0x01, 0x01), (1.0625, 0x38, 0x38),
    (1.1875, 0x3A, 0x3A), (-0.0, 0x80, 0x80), (0.0, 0x00, 0x00), (-3.0, 0xC4, 0xC4), (-2.0, 0xC0, 0xC0),
]


@pytest.mark.parametrize("x,plain,sat", ENCODE_KAT)
def test_fp8_encode_known_answers(x, plain, sat):
    assert int(of8.encode(np.array([x]))[0]) == plain
    assert int(of8.encode(np.array([x]), saturate=True)[0]) == sat


def test_fp8_encode_nan_and_round_trip_of_every_code():
    assert (int(of8.encode(np.array([np.nan]))[0]) & 0x7F) == 0x7F
    codes = np.array([c for c in range(256) if (c & 0x7F) != 0x7F], np.uint8)
    assert np.array_equal(of8.encode(of8.decode(codes).astype(np.float32)), codes)


def test_quantize_rows_divides_in_fp32():
    """kv_scale 0.1 is not a power of two: the row is encode(fl32(x / 0.1)),
    which differs from encode(fl32(x * fl32(1/0.1))) on some inputs."""
    g = np.random.default_rng(4)
    c = g.standard_normal((64, 512)).astype(np.float32)
    r = g.standard_normal((64, 64)).astype(np.float32)
    got = of8.quantize_rows(c, r, 0.1)
    x = np.concatenate([c, r], axis=1)
    assert np.array_equal(got, of8.encode((x / np.float32(0.1)).astype(np.float32)))
    assert got.shape == (64, 576)
