"""The allocation-free MLA entry point, launch_mla_decode_a16w8_paged_dev_noalloc,
against the launcher it varies (launch_mla_decode_a16w8_paged_dev with a
caller workspace): bit-identical output on two calls in a row, the second
with a smaller input (so stale contents of the library's array from the first
call must not leak into it), its size limit, and its argument codes (those of
the workspace launcher, checked before the size limit). All calls go through
the C ABI."""
import pytest
import torch

from moonmath_attention import _lib
from mla_inputs import KV_SCALE, SCALE_192, paged_pool, ragged_lens, rand_q

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _inputs(B, H, q_len, lo, hi, seed):
    lens = ragged_lens(B, lo, hi, seed)
    pool, idx, indptr = paged_pool(lens, seed)
    q_lat, q_pe = rand_q(B, q_len, H, seed, peak=1.0)
    t = [x.to(DEV) for x in (q_lat, q_pe, pool, torch.tensor(lens, dtype=torch.int32), idx, indptr)]
    return t, lens


def _run(noalloc, t, B, H, q_len, parts):
    q_lat, q_pe, pool, lens, idx, indptr = t
    o = torch.full((B, q_len, H, 512), float("nan"), dtype=torch.bfloat16, device=DEV)
    p = _lib.ptr
    args = (p(q_lat), p(q_pe), p(pool), p(o), p(lens), None, p(idx), p(indptr), B, H, parts, 512, 64,
            SCALE_192, KV_SCALE, 1.0)
    st = _lib.stream_ptr(DEV)
    kv_bytes = idx.numel() * 576
    if noalloc:
        rc = _lib.lib.launch_mla_decode_a16w8_paged_dev_noalloc(*args, st, kv_bytes, q_len)
        ws = None
    else:
        ws = torch.empty(_lib.lib.mla_decode_a16w8_multiq_workspace_for(B, H, parts, q_len), dtype=torch.uint8,
                         device=DEV)
        rc = _lib.lib.launch_mla_decode_a16w8_paged_dev(*args, p(ws), st, kv_bytes, q_len)
    torch.cuda.synchronize()
    assert rc == 0, rc
    del ws
    return o


def test_noalloc_matches_workspace_launcher_two_calls():
    cases = [
        # B, H, q_len, parts, ctx range: the DeepSeek decode shape, all 32768 records in use
        (64, 128, 1, 4, 1024, 8192),
        # then a smaller batch, 16 heads, a draft window of 2, 3 parts
        (6, 16, 2, 3, 200, 3000),
    ]
    for i, (B, H, q_len, parts, lo, hi) in enumerate(cases):
        assert _lib.lib.moonmath_mla_effective_parts(B, H, parts, q_len, 1) == parts
        t, _ = _inputs(B, H, q_len, lo, hi, seed=300 + i)
        got = _run(True, t, B, H, q_len, parts)
        want = _run(False, t, B, H, q_len, parts)
        assert not torch.isnan(want.float()).any()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"call {i}: outputs differ"


def test_noalloc_unsplit_needs_no_records():
    """parts 1 uses no split records, whatever the size."""
    B, H, q_len = 64, 128, 2
    t, _ = _inputs(B, H, q_len, 100, 900, seed=320)
    got = _run(True, t, B, H, q_len, 1)
    want = _run(False, t, B, H, q_len, 1)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_noalloc_rejects_records_beyond_its_array():
    """64 x 4 parts x 128 heads x 2 positions = 65536 records > 32768: -9, and
    nothing is launched (the output keeps its fill)."""
    B, H, q_len, parts = 64, 128, 2, 4
    t, _ = _inputs(B, H, q_len, 100, 300, seed=330)
    q_lat, q_pe, pool, lens, idx, indptr = t
    o = torch.full((B, q_len, H, 512), 7.0, dtype=torch.bfloat16, device=DEV)
    p = _lib.ptr
    rc = _lib.lib.launch_mla_decode_a16w8_paged_dev_noalloc(
        p(q_lat), p(q_pe), p(pool), p(o), p(lens), None, p(idx), p(indptr), B, H, parts, 512, 64, SCALE_192,
        KV_SCALE, 1.0, _lib.stream_ptr(DEV), idx.numel() * 576, q_len)
    torch.cuda.synchronize()
    assert rc == -9
    assert torch.all(o == 7.0)


def test_noalloc_argument_codes_before_the_size_limit():
    """Bad H gives the workspace launcher's -3 (not the size code), also with
    parts whose records would not fit; bad dims -2; nothing is launched."""
    B, q_len, parts = 64, 2, 4
    t, _ = _inputs(B, 16, q_len, 100, 300, seed=340)
    q_lat, q_pe, pool, lens, idx, indptr = t
    o = torch.full((B, q_len, 16, 512), 7.0, dtype=torch.bfloat16, device=DEV)
    p = _lib.ptr
    st = _lib.stream_ptr(DEV)
    for H, lat, want in ((200, 512, -3), (0, 512, -3), (128, 256, -2)):
        rc = _lib.lib.launch_mla_decode_a16w8_paged_dev_noalloc(
            p(q_lat), p(q_pe), p(pool), p(o), p(lens), None, p(idx), p(indptr), B, H, parts, lat, 64, SCALE_192,
            KV_SCALE, 1.0, st, idx.numel() * 576, q_len)
        assert rc == want, (H, lat, rc)
    torch.cuda.synchronize()
    assert torch.all(o == 7.0)
