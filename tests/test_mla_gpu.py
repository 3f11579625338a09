"""GPU parity of the gfx950 MLA decode against the CPU oracle.

Mirrors reference tests/test_mla_decode.py (peaked queries x3, KV = e4m3 of
N(0,1) at kv_scale 1/32, random slot permutation, end-aligned window poison
test, rows reversal bit-identity, domain rejections) with OCP e4m3fn KV and the
gfx950 domain (H up to 128, multi-query q_len 2..8).

Tolerance (stated for this path): the same rule as the attention forward
(helpers.compare_bf16: 1 bf16 ULP at max(|ref|, A/4) against the oracle that
applies the kernel's precision model -- bf16 P (RTNE), integer-grid max, fp8
dequant -- plus >= 99% bit-exact and >= 99.9% strictly within 1 ULP), and the
reference's own floor: rel-L2 < 3e-3 against its plain fp32 formula.
"""
import numpy as np
import pytest
import torch

import moonmath_attention as ma
from moonmath_attention import _lib
from oracle import fp8 as of8
from oracle import mla as om
from helpers import aggregate_stats, bits, check_fractions, compare_bf16, log_stats
from mla_inputs import (KV_SCALE, QK, SCALE_192, SCALE_576, fp8_bits, paged_pool, ragged_lens, rand_kv_rows,
                        rand_q)

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
REL_L2 = 3e-3


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    assert torch.cuda.is_available(), "GPU tests need an MI355X"


def _d(t):
    return None if t is None else t.to(DEV)


def _rel_l2(out, ref):
    return float(np.linalg.norm(out.astype(np.float64) - ref) / np.linalg.norm(ref))


def _check(o_lat, q_lat, q_pe, kv_u8, lens, scale, kv_indices=None, kv_indptr=None, rows=None, batches=None):
    got = bits(o_lat)
    if got.ndim == 3:
        got = got[:, None]
    ql = q_lat.float().numpy()
    qp = q_pe.float().numpy()
    if ql.ndim == 3:
        ql, qp = ql[:, None], qp[:, None]
    ref, _, A = om.decode(ql, qp, kv_u8, lens, scale, KV_SCALE, kv_indices=kv_indices, kv_indptr=kv_indptr,
                          rows=rows, batches=batches, aux=True)
    bsel = list(range(ql.shape[0])) if batches is None else list(batches)
    qsel = bsel if rows is None else [min(max(int(rows[b]), 0), ql.shape[0] - 1) for b in bsel]
    # One record per request (the ULP rule per element); the fraction bars on
    # all of them together, with the worst request named in the log.
    per = [compare_bf16(got[r], ref[r], A[r], fractions=False) for r in qsel]
    stats = aggregate_stats(per, names=[f"req{b}" for b in bsel])
    check_fractions(stats)
    if rows is None and kv_indices is None:
        f32 = om.fp32_reference(ql[bsel], qp[bsel], kv_u8[bsel], [lens[b] for b in bsel], scale, KV_SCALE)
        stats["rel_l2"] = _rel_l2(om._b.bf16_to_f32(got[bsel]), f32)
        assert stats["rel_l2"] < REL_L2, stats
    log_stats(None, stats)
    return stats


def test_fp8_hardware_convert_matches_ocp_decode():
    """v_cvt_scalef32_pk_bf16_fp8 (scale 1) on all 256 e4m3fn codes vs the OCP table."""
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8).to(DEV)
    out = torch.empty(256, dtype=torch.int16, device=DEV)
    assert _lib.lib.moonmath_fp8e4m3_to_bf16(_lib.ptr(codes), _lib.ptr(out), 256, _lib.stream_ptr(DEV)) == 0
    torch.cuda.synchronize()
    got = om._b.bf16_to_f32(out.cpu().numpy().view(np.uint16)).astype(np.float64)
    exp = of8.DECODE
    nan = np.isnan(exp)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan], exp[~nan])
    assert np.array_equal(np.signbit(got[~nan]), np.signbit(exp[~nan]))


@pytest.mark.parametrize("H", [12, 16, 128])
def test_single_query_contiguous(H):
    B, S = 2, 2048
    kv = rand_kv_rows(B * S, 11).view(B, S, QK)
    q_lat, q_pe = rand_q(B, 1, H, 11)
    q_lat, q_pe = q_lat[:, 0].contiguous(), q_pe[:, 0].contiguous()
    o = torch.zeros(B, H, 512, dtype=torch.bfloat16, device=DEV)
    ma.mla_decode_a16w8(_d(q_lat), _d(q_pe), _d(kv), o, SCALE_576, KV_SCALE)
    torch.cuda.synchronize()
    print(_check(o, q_lat, q_pe, fp8_bits(kv), [S] * B, SCALE_576))


@pytest.mark.parametrize("q_len", [2, 4, 5, 8])
@pytest.mark.parametrize("H", [16, 128])
def test_multiq_contiguous(q_len, H):
    B, S = 2, 1000
    kv = rand_kv_rows(B * S, 23).view(B, S, QK)
    q_lat, q_pe = rand_q(B, q_len, H, 23)
    o = torch.zeros(B, q_len, H, 512, dtype=torch.bfloat16, device=DEV)
    ma.mla_decode_a16w8_multiq(_d(q_lat), _d(q_pe), _d(kv), o, SCALE_576, KV_SCALE)
    torch.cuda.synchronize()
    _check(o, q_lat, q_pe, fp8_bits(kv), [S] * B, SCALE_576)


def test_multiq_causal_window_is_end_aligned():
    """Reference tests/test_mla_decode.py:122-138: poisoning the last q_len-1
    rows leaves position 0 bit-identical and moves the last position."""
    B, S, H, q_len = 1, 2048, 16, 4
    kv = rand_kv_rows(B * S, 31).view(B, S, QK)
    q_lat, q_pe = rand_q(B, q_len, H, 31)
    o = torch.zeros(B, q_len, H, 512, dtype=torch.bfloat16, device=DEV)
    kvd = _d(kv)
    ma.mla_decode_a16w8_multiq(_d(q_lat), _d(q_pe), kvd, o, SCALE_576, KV_SCALE)
    base = o.clone()
    kvd[:, S - q_len + 1:] = _d(rand_kv_rows(q_len - 1, 99)).view(1, q_len - 1, QK)
    ma.mla_decode_a16w8_multiq(_d(q_lat), _d(q_pe), kvd, o, SCALE_576, KV_SCALE)
    torch.cuda.synchronize()
    assert torch.equal(o[:, 0].view(torch.int16), base[:, 0].view(torch.int16)), "position 0 read past its limit"
    assert not torch.equal(o[:, -1], base[:, -1]), "last position missed the tail tokens"


@pytest.mark.parametrize("q_len", [1, 2, 4, 8])
def test_paged_ragged_matches_oracle(q_len):
    B, H = 3, 16
    lens = [2048, 2064, 1024]
    pool, idx, indptr = paged_pool(lens, 43)
    q_lat, q_pe = rand_q(B, q_len, H, 43)
    o = torch.zeros(B, q_len, H, 512, dtype=torch.bfloat16, device=DEV)
    lens_t = torch.tensor(lens, dtype=torch.int32)
    parts = ma.mla_decode_a16w8_plan_parts_q(B, max(lens), q_len, H)
    assert parts >= 1
    if q_len == 1:
        ma.mla_decode_a16w8_paged_dev(_d(q_lat[:, 0].contiguous()), _d(q_pe[:, 0].contiguous()), _d(pool),
                                      o[:, 0], _d(lens_t), None, _d(idx), _d(indptr), parts, SCALE_576, KV_SCALE)
    else:
        ma.mla_decode_a16w8_multiq_paged_dev(_d(q_lat), _d(q_pe), _d(pool), o, _d(lens_t), None, _d(idx),
                                             _d(indptr), parts, SCALE_576, KV_SCALE)
    torch.cuda.synchronize()
    _check(o, q_lat, q_pe, fp8_bits(pool), lens, SCALE_576, kv_indices=idx.numpy(), kv_indptr=indptr.numpy())


def _random_mla_cases(n, seed):
    """Seeded random decode configs across the three kernels (query rows per
    request H * q_len: <= 16, 17..95 or > 128, 96..128), ragged lengths from 1
    token, split budgets 1..5, both softmax scales."""
    rng = np.random.default_rng(seed)
    cases = []
    for _ in range(n):
        q_len = int(rng.choice([1, 1, 2, 3, 4, 8]))
        kind = rng.integers(0, 3)
        rows = int(rng.integers(1, 17)) if kind == 0 else (int(rng.integers(96, 129)) if kind == 1
                                                         else int(rng.integers(17, 257)))
        H = max(1, min(128, rows // q_len))
        B = int(rng.integers(1, 7))
        lens = tuple(int(x) for x in rng.integers(1, 2000, size=B))
        cases.append((H, q_len, int(rng.integers(1, 6)), bool(rng.integers(0, 2)), lens))
    return cases


@pytest.mark.parametrize("case", _random_mla_cases(12, 2026),
                         ids=lambda c: "h{}_q{}_p{}_s{}_b{}".format(c[0], c[1], c[2], 576 if c[3] else 192, len(c[4])))
def test_random_paged_configs_match_oracle(case):
    H, q_len, parts, s576, lens = case
    lens = list(lens)
    B = len(lens)
    scale = SCALE_576 if s576 else SCALE_192
    seed = 7 * H + q_len + sum(lens) % 997
    pool, idx, indptr = paged_pool(lens, seed)
    q_lat, q_pe = rand_q(B, q_len, H, seed)
    o = torch.zeros(B, q_len, H, 512, dtype=torch.bfloat16, device=DEV)
    lens_t = torch.tensor(lens, dtype=torch.int32)
    if q_len == 1:
        ma.mla_decode_a16w8_paged_dev(_d(q_lat[:, 0].contiguous()), _d(q_pe[:, 0].contiguous()), _d(pool),
                                      o[:, 0], _d(lens_t), None, _d(idx), _d(indptr), parts, scale, KV_SCALE)
    else:
        ma.mla_decode_a16w8_multiq_paged_dev(_d(q_lat), _d(q_pe), _d(pool), o, _d(lens_t), None, _d(idx),
                                             _d(indptr), parts, scale, KV_SCALE)
    torch.cuda.synchronize()
    _check(o, q_lat, q_pe, fp8_bits(pool), lens, scale, kv_indices=idx.numpy(), kv_indptr=indptr.numpy())


@pytest.mark.parametrize("parts", [1, 3, 7])
def test_split_parts_agree(parts):
    """Any parts >= 1 gives results within the tolerance rule of parts = 1."""
    B, H, q_len = 2, 32, 2
    lens = [1500, 700]
    pool, idx, indptr = paged_pool(lens, 47)
    q_lat, q_pe = rand_q(B, q_len, H, 47)
    o = torch.zeros(B, q_len, H, 512, dtype=torch.bfloat16, device=DEV)
    ma.mla_decode_a16w8_multiq_paged_dev(_d(q_lat), _d(q_pe), _d(pool), o, _d(torch.tensor(lens, dtype=torch.int32)),
                                         None, _d(idx), _d(indptr), parts, SCALE_192, KV_SCALE)
    torch.cuda.synchronize()
    _check(o, q_lat, q_pe, fp8_bits(pool), lens, SCALE_192, kv_indices=idx.numpy(), kv_indptr=indptr.numpy())


@pytest.mark.parametrize("q_len,parts", [(1, 1), (1, 2), (1, 4), (3, 3)])
def test_paged_large_ragged_batch_balanced_split(q_len, parts):
    """80 requests (more than one 64-lane chunk of the device-side split plan),
    lengths from 1 token to 1500 including tile-edge values; the plan cuts long
    requests into equal parts and dispatches them longest first."""
    B, H = 80, 8
    lens = [1, 5, 31, 32, 33, 63, 64, 65, 600, 1500] + ragged_lens(B - 10, 1, 1200, 61)
    pool, idx, indptr = paged_pool(lens, 61)
    q_lat, q_pe = rand_q(B, q_len, H, 61)
    o = torch.zeros(B, q_len, H, 512, dtype=torch.bfloat16, device=DEV)
    lens_t = torch.tensor(lens, dtype=torch.int32)
    if q_len == 1:
        ma.mla_decode_a16w8_paged_dev(_d(q_lat[:, 0].contiguous()), _d(q_pe[:, 0].contiguous()), _d(pool),
                                      o[:, 0], _d(lens_t), None, _d(idx), _d(indptr), parts, SCALE_576, KV_SCALE)
    else:
        ma.mla_decode_a16w8_multiq_paged_dev(_d(q_lat), _d(q_pe), _d(pool), o, _d(lens_t), None, _d(idx),
                                             _d(indptr), parts, SCALE_576, KV_SCALE)
    torch.cuda.synchronize()
    _check(o, q_lat, q_pe, fp8_bits(pool), lens, SCALE_576, kv_indices=idx.numpy(), kv_indptr=indptr.numpy())


@pytest.mark.parametrize("H,q_len,parts", [(128, 1, 1), (128, 1, 3), (100, 1, 2), (64, 3, 2), (16, 8, 1)])
def test_wide_block_ragged_tile_edges(H, q_len, parts):
    """Query blocks of >= 96 rows run the 128-row kernel: lengths at tile edges
    (1, 31..33, 63..65 tokens), partial row tiles (H=100, 3 x 64 rows) and split
    parts, paged over a permuted pool."""
    lens = [1, 5, 31, 32, 33, 63, 64, 65, 97, 600, 1500, 2100]
    B = len(lens)
    pool, idx, indptr = paged_pool(lens, 67)
    q_lat, q_pe = rand_q(B, q_len, H, 67)
    o = torch.zeros(B, q_len, H, 512, dtype=torch.bfloat16, device=DEV)
    lens_t = torch.tensor(lens, dtype=torch.int32)
    if q_len == 1:
        ma.mla_decode_a16w8_paged_dev(_d(q_lat[:, 0].contiguous()), _d(q_pe[:, 0].contiguous()), _d(pool),
                                      o[:, 0], _d(lens_t), None, _d(idx), _d(indptr), parts, SCALE_576, KV_SCALE)
    else:
        ma.mla_decode_a16w8_multiq_paged_dev(_d(q_lat), _d(q_pe), _d(pool), o, _d(lens_t), None, _d(idx),
                                             _d(indptr), parts, SCALE_576, KV_SCALE)
    torch.cuda.synchronize()
    _check(o, q_lat, q_pe, fp8_bits(pool), lens, SCALE_576, kv_indices=idx.numpy(), kv_indptr=indptr.numpy())


@pytest.mark.parametrize("H,q_len,parts", [(16, 1, 1), (16, 1, 3), (8, 2, 2), (5, 3, 1), (1, 1, 2)])
def test_small_block_ragged_tile_edges(H, q_len, parts):
    """Query blocks of <= 16 rows run the 16-row kernel (64-token tiles, 16
    tokens per wave): lengths at its tile and sub-tile edges, padded query
    columns (H * q_len < 16), split parts, paged over a permuted pool."""
    lens = [1, 5, 15, 16, 17, 31, 32, 33, 63, 64, 65, 97, 600, 1500, 2100]
    B = len(lens)
    pool, idx, indptr = paged_pool(lens, 69)
    q_lat, q_pe = rand_q(B, q_len, H, 69)
    o = torch.zeros(B, q_len, H, 512, dtype=torch.bfloat16, device=DEV)
    lens_t = torch.tensor(lens, dtype=torch.int32)
    if q_len == 1:
        ma.mla_decode_a16w8_paged_dev(_d(q_lat[:, 0].contiguous()), _d(q_pe[:, 0].contiguous()), _d(pool),
                                      o[:, 0], _d(lens_t), None, _d(idx), _d(indptr), parts, SCALE_576, KV_SCALE)
    else:
        ma.mla_decode_a16w8_multiq_paged_dev(_d(q_lat), _d(q_pe), _d(pool), o, _d(lens_t), None, _d(idx),
                                             _d(indptr), parts, SCALE_576, KV_SCALE)
    torch.cuda.synchronize()
    _check(o, q_lat, q_pe, fp8_bits(pool), lens, SCALE_576, kv_indices=idx.numpy(), kv_indptr=indptr.numpy())


@pytest.mark.parametrize("H,B", [(4, 300), (64, 140)])
def test_more_requests_than_one_round_of_ctas(H, B):
    """More requests than one round of CTAs holds (256 for the 16-row kernel,
    128 two-CTA units for the 32-row kernel at H=64): one part per request,
    dispatched longest first over several rounds."""
    lens = ragged_lens(B, 1, 300, 79)
    pool, idx, indptr = paged_pool(lens, 79)
    q_lat, q_pe = rand_q(B, 1, H, 79)
    o = torch.zeros(B, 1, H, 512, dtype=torch.bfloat16, device=DEV)
    parts = ma.mla_decode_a16w8_plan_parts_q(B, max(lens), 1, H)
    ma.mla_decode_a16w8_paged_dev(_d(q_lat[:, 0].contiguous()), _d(q_pe[:, 0].contiguous()), _d(pool), o[:, 0],
                                  _d(torch.tensor(lens, dtype=torch.int32)), None, _d(idx), _d(indptr), parts,
                                  SCALE_576, KV_SCALE)
    torch.cuda.synchronize()
    _check(o, q_lat, q_pe, fp8_bits(pool), lens, SCALE_576, kv_indices=idx.numpy(), kv_indptr=indptr.numpy())


def test_small_block_multi_segment_part():
    """A part longer than the 16-row kernel's 9216-token tile table: the
    second segment re-stages its slot indices and refills the ring."""
    lens = [33100, 100]
    B, H = len(lens), 16
    pool, idx, indptr = paged_pool(lens, 73)
    q_lat, q_pe = rand_q(B, 1, H, 73)
    o = torch.zeros(B, 1, H, 512, dtype=torch.bfloat16, device=DEV)
    ma.mla_decode_a16w8_paged_dev(_d(q_lat[:, 0].contiguous()), _d(q_pe[:, 0].contiguous()), _d(pool), o[:, 0],
                                  _d(torch.tensor(lens, dtype=torch.int32)), None, _d(idx), _d(indptr), 1, SCALE_576,
                                  KV_SCALE)
    torch.cuda.synchronize()
    _check(o, q_lat, q_pe, fp8_bits(pool), lens, SCALE_576, kv_indices=idx.numpy(), kv_indptr=indptr.numpy())


def test_small_block_bench_config_sampled():
    """The HBM-bound shape: B=64, H=16 (128 heads over 8 GPUs), ctx ~
    U[1024, 8192], 64-token pages; 4 sampled requests vs the oracle, and
    run-to-run determinism."""
    B, H = 64, 16
    lens = ragged_lens(B, 1024, 8192, seed=5)
    pool, idx, indptr = paged_pool(lens, 61)
    q_lat, q_pe = rand_q(B, 1, H, 61, peak=1.0)
    parts = ma.mla_decode_a16w8_plan_parts_q(B, 8192, 1, H)
    o1 = torch.zeros(B, 1, H, 512, dtype=torch.bfloat16, device=DEV)
    o2 = torch.zeros_like(o1)
    qd, pd, lens_t = _d(q_lat[:, 0].contiguous()), _d(q_pe[:, 0].contiguous()), _d(torch.tensor(lens, dtype=torch.int32))
    pool_d, idx_d, indptr_d = _d(pool), _d(idx), _d(indptr)
    for o in (o1, o2):
        ma.mla_decode_a16w8_paged_dev(qd, pd, pool_d, o[:, 0], lens_t, None, idx_d, indptr_d, parts, SCALE_192,
                                      KV_SCALE)
    torch.cuda.synchronize()
    assert torch.equal(o1.view(torch.int16), o2.view(torch.int16)), "not deterministic"
    print(_check(o1, q_lat, q_pe, fp8_bits(pool), lens, SCALE_192, kv_indices=idx.numpy(),
                 kv_indptr=indptr.numpy(), batches=[0, 17, 40, 63]))


@pytest.mark.parametrize("H,q_len,S,paged,parts", [
    (16, 1, 300, False, 0),     # 16-row kernel, one part
    (128, 1, 300, False, 0),    # 128-row kernel, one part
    (32, 1, 2048, False, 0),    # 32-row kernel, planned split
    (128, 2, 2048, True, 4),    # 32-row kernel (8 row groups), paged, split
    (16, 1, 4096, True, 4),     # 16-row kernel, paged, split
    (128, 1, 4096, True, 4),    # 128-row kernel, paged, split
])
def test_max_fallback_on_growing_scores(H, q_len, S, paged, parts):
    """Scores that rise more than 2^64 above a row's first tile send the CTA
    through the exact-max fallback (a max-only pass, then accumulation with
    the row max fixed); the result must still match the exact-max oracle, also
    when only some parts of a split request fall back before the merge."""
    # Only q dims 0..100 are non-zero. Tokens >= lo carry k = 448 in dims 0..99
    # and a random k in dim 100 with |k| >= 1/16, so their scores (up to 9e4,
    # times c: ~170 on the log2 grid, vs ~0 for the first tokens) are sums of
    # products on a 2^-7 grid below 2^17: exact in fp32 in any order. (Random
    # scores of that size would carry fp32 accumulation-order noise of ~1e-5 in
    # the exponent, which flips bf16(P) far more often than the exactness bar
    # allows, in any correct kernel.)
    B, lo = 2, 40
    g = torch.Generator().manual_seed(71)
    kv = rand_kv_rows(B * S, 71).view(B, S, QK)
    kv[:, lo:, :100] = torch.full((B, S - lo, 100), 448.0).to(torch.float8_e4m3fn)
    k100 = kv[:, lo:, 100].float()
    kv[:, lo:, 100] = torch.where(k100.abs() < 0.0625, torch.full_like(k100, 0.0625), k100).to(torch.float8_e4m3fn)
    q_lat = torch.zeros(B, q_len, H, 512)
    q_lat[..., :100] = torch.randint(1, 3, (B, q_len, H, 100), generator=g).float()  # 1 or 2
    q_lat[..., 100] = 2.0 ** torch.randint(-1, 2, (B, q_len, H), generator=g).float()  # 0.5, 1 or 2
    q_lat = q_lat.to(torch.bfloat16)
    q_pe = torch.zeros(B, q_len, H, 64, dtype=torch.bfloat16)
    o = torch.zeros(B, q_len, H, 512, dtype=torch.bfloat16, device=DEV)
    lens = [S, S - 13]
    if not paged:
        assert q_len == 1
        ma.mla_decode_a16w8(_d(q_lat[:, 0]), _d(q_pe[:, 0]), _d(kv), o[:, 0], SCALE_576, KV_SCALE)
        torch.cuda.synchronize()
        print(_check(o[:, 0], q_lat[:, 0], q_pe[:, 0], fp8_bits(kv), [S] * B, SCALE_576))
        return
    # Paged: the tokens of both requests scattered over a permuted pool.
    slots = torch.randperm(B * S, generator=g).to(torch.int32)
    pool = torch.empty(B * S, 1, QK, dtype=torch.float8_e4m3fn)
    pool.view(torch.uint8)[slots.long(), 0] = kv.reshape(B * S, QK).view(torch.uint8)
    idx = torch.cat([slots[b * S: b * S + lens[b]] for b in range(B)])
    indptr = torch.tensor([0, lens[0], lens[0] + lens[1]], dtype=torch.int32)
    lens_t = torch.tensor(lens, dtype=torch.int32)
    eff = _lib.lib.moonmath_mla_effective_parts(B, H, parts, q_len, 1)
    assert eff > 1, eff
    if q_len == 1:
        ma.mla_decode_a16w8_paged_dev(_d(q_lat[:, 0]), _d(q_pe[:, 0]), _d(pool), o[:, 0], _d(lens_t), None, _d(idx),
                                      _d(indptr), parts, SCALE_576, KV_SCALE)
    else:
        ma.mla_decode_a16w8_multiq_paged_dev(_d(q_lat), _d(q_pe), _d(pool), o, _d(lens_t), None, _d(idx),
                                             _d(indptr), parts, SCALE_576, KV_SCALE)
    torch.cuda.synchronize()
    print(_check(o, q_lat, q_pe, fp8_bits(pool), lens, SCALE_576, kv_indices=idx.numpy(), kv_indptr=indptr.numpy()))


@pytest.mark.parametrize("H,q_len", [(16, 4), (16, 1), (128, 1), (100, 1)])
def test_paged_rows_remaps_query_and_output(H, q_len):
    """Reference tests/test_mla_decode.py:164-188: reversing rows reverses the
    batch; on the 32-row, 16-row and 128-row kernels (each split, so the row
    map also reaches both merge kernels; H=100 leaves padding rows in the
    128-row kernel's records)."""
    B = 4
    lens = [2048] * B
    pool, idx, indptr = paged_pool(lens, 57)
    q_lat, q_pe = rand_q(B, q_len, H, 57)
    if q_len == 1:
        q_lat, q_pe = q_lat[:, 0].contiguous(), q_pe[:, 0].contiguous()
    lens_t = _d(torch.tensor(lens, dtype=torch.int32))
    parts = ma.mla_decode_a16w8_plan_parts_q(B, lens[0], q_len, H)
    assert parts > 1
    o = torch.zeros(*q_lat.shape[:-1], 512, dtype=torch.bfloat16, device=DEV)
    ma.mla_decode_a16w8_paged_dev(_d(q_lat), _d(q_pe), _d(pool), o, lens_t, None, _d(idx), _d(indptr),
                                  parts, SCALE_576, KV_SCALE)
    rows = _d(torch.arange(B - 1, -1, -1, dtype=torch.int32))
    o_rev = torch.zeros_like(o)
    ma.mla_decode_a16w8_paged_dev(_d(q_lat.flip(0).contiguous()), _d(q_pe.flip(0).contiguous()), _d(pool),
                                  o_rev, lens_t, rows, _d(idx), _d(indptr), parts, SCALE_576, KV_SCALE)
    torch.cuda.synchronize()
    assert torch.equal(o_rev.flip(0).view(torch.int16), o.view(torch.int16))


@pytest.mark.parametrize("H,q_len", [(128, 1), (128, 2), (16, 1)])
def test_deepseek_config_all_requests(H, q_len):
    """B=64, ctx ~ U[1024, 8192], 64-token pages over a permuted
    pool, scale 1/sqrt(192), at H=128 (q_len 1 and 2) and at the H=16 TP8
    share: every one of the 64 requests against the oracle, and run-to-run
    determinism."""
    B = 64
    lens = ragged_lens(B, 1024, 8192, seed=5)
    pool, idx, indptr = paged_pool(lens, 61)
    q_lat, q_pe = rand_q(B, q_len, H, 61 + H, peak=1.0)
    lens_t = _d(torch.tensor(lens, dtype=torch.int32))
    parts = ma.mla_decode_a16w8_plan_parts_q(B, 8192, q_len, H)
    o1 = torch.zeros(B, q_len, H, 512, dtype=torch.bfloat16, device=DEV)
    o2 = torch.zeros_like(o1)
    fn = ma.mla_decode_a16w8_multiq_paged_dev if q_len > 1 else ma.mla_decode_a16w8_paged_dev
    qd, pd = _d(q_lat), _d(q_pe)
    if q_len == 1:
        qd, pd = qd[:, 0].contiguous(), pd[:, 0].contiguous()
    for o in (o1, o2):
        oo = o[:, 0] if q_len == 1 else o
        fn(qd, pd, _d(pool), oo, lens_t, None, _d(idx), _d(indptr), parts, SCALE_192, KV_SCALE)
    torch.cuda.synchronize()
    assert torch.equal(o1.view(torch.int16), o2.view(torch.int16)), "not deterministic"
    print(_check(o1, q_lat, q_pe, fp8_bits(pool), lens, SCALE_192, kv_indices=idx.numpy(),
                 kv_indptr=indptr.numpy()))


# ---- supported domain (reference tests/test_mla_decode.py:194-220) -------------


@pytest.mark.parametrize("q_len", [1, 9])
def test_multiq_rejects_q_len_out_of_domain(q_len):
    B, S, H = 1, 256, 16
    kv = _d(rand_kv_rows(B * S, 71).view(B, S, QK))
    q_lat, q_pe = rand_q(B, q_len, H, 71)
    o = torch.zeros(B, q_len, H, 512, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError, match="q_len"):
        ma.mla_decode_a16w8_multiq(_d(q_lat), _d(q_pe), kv, o, SCALE_576, KV_SCALE)


def test_multiq_rejects_too_many_heads():
    B, S, q_len = 1, 256, 4
    kv = _d(rand_kv_rows(B * S, 73).view(B, S, QK))
    q_lat, q_pe = rand_q(B, q_len, 129, 73)
    o = torch.zeros(B, q_len, 129, 512, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError, match="H must be"):
        ma.mla_decode_a16w8_multiq(_d(q_lat), _d(q_pe), kv, o, SCALE_576, KV_SCALE)


def test_multiq_rejects_q_len_1_rank():
    B, S, H = 1, 256, 16
    kv = _d(rand_kv_rows(B * S, 79).view(B, S, QK))
    q_lat, q_pe = rand_q(B, 1, H, 79)
    o = torch.zeros(B, H, 512, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError, match=r"\[B,q_len,H,512\]"):
        ma.mla_decode_a16w8_multiq(_d(q_lat[:, 0].contiguous()), _d(q_pe[:, 0].contiguous()), kv, o, SCALE_576,
                                   KV_SCALE)
