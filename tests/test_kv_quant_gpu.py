"""GPU tests of the fp8 KV producer (mla_kv_quantize / launch_mla_kv_quantize).

Written rows must equal the oracle byte for byte (torch's float8_e4m3fn cast
of fl32(x / kv_scale), oracle/fp8.py), for a power-of-two kv_scale (the
multiply path) and others (correctly rounded division), both overflow modes,
and every bf16 bit pattern; rows of padding tokens (slot -1) and of slots past
the pool stay untouched; a cache filled by the producer decodes like one
filled on the host.
"""
import numpy as np
import pytest
import torch

import moonmath_attention as ma
from moonmath_attention import _lib
from oracle import fp8 as of8
from oracle import mla as om
from helpers import bits, compare_bf16, log_stats
from mla_inputs import KV_SCALE, QK, SCALE_192, fp8_bits, rand_q

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    assert torch.cuda.is_available(), "GPU tests need an MI355X"


def _run(c_kv, k_pe, num_slots, slots, kv_scale, saturate, fill=0x5A):
    pool = torch.full((num_slots, 1, QK), fill, dtype=torch.uint8, device=DEV).view(torch.float8_e4m3fn)
    ma.mla_kv_quantize(c_kv.to(DEV), k_pe.to(DEV), pool, slots.to(DEV), kv_scale, saturate=saturate)
    torch.cuda.synchronize()
    return pool.view(torch.uint8).cpu().numpy().reshape(num_slots, QK)


@pytest.mark.parametrize("kv_scale", [1.0 / 32, 0.0371, 3.0, 2.0 ** -12])
@pytest.mark.parametrize("saturate", [False, True])
def test_rows_match_oracle(kv_scale, saturate):
    N, num_slots = 3000, 4000
    g = torch.Generator().manual_seed(int(kv_scale * 1e4) + saturate)
    # wide dynamic range so that overflow, subnormals and ties all occur
    c_kv = (torch.randn(N, 512, generator=g) * torch.exp2(torch.randint(-14, 6, (N, 1), generator=g).float()))
    k_pe = (torch.randn(N, 64, generator=g) * 4).to(torch.bfloat16)
    c_kv = c_kv.to(torch.bfloat16)
    slots = torch.randperm(num_slots, generator=g)[:N].to(torch.int32)
    slots[::97] = -1                        # padding tokens
    slots[5] = num_slots + 3                # past the pool: skipped
    got = _run(c_kv, k_pe, num_slots, slots, kv_scale, saturate)
    want = of8.quantize_rows(c_kv.float().numpy(), k_pe.float().numpy(), kv_scale, saturate)
    s = slots.numpy()
    live = (s >= 0) & (s < num_slots)
    assert np.array_equal(got[s[live]], want[live])
    untouched = np.setdiff1d(np.arange(num_slots), s[live])
    assert np.all(got[untouched] == 0x5A)
    if saturate:  # the inputs are finite: saturation leaves no NaN
        assert not ((want & 0x7F) == 0x7F).any()


@pytest.mark.parametrize("saturate", [False, True])
def test_every_bf16_bit_pattern(saturate):
    """All 65536 bf16 patterns (zeros, subnormals, normals, inf, NaN) through
    the latent and rope columns, at a non-power-of-two scale."""
    pat = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    N = 65536 // 512
    c_kv = pat.view(N, 512).contiguous()
    k_pe = pat[: N * 64].view(N, 64).contiguous()
    slots = torch.arange(N, dtype=torch.int32)
    got = _run(c_kv, k_pe, N, slots, 0.75, saturate)
    want = of8.quantize_rows(c_kv.float().numpy(), k_pe.float().numpy(), 0.75, saturate)
    # NaN: any 0x7F / 0xFF pattern (the sign of a NaN is not part of the contract)
    gn, wn = (got & 0x7F) == 0x7F, (want & 0x7F) == 0x7F
    assert np.array_equal(gn, wn)
    assert np.array_equal(got[~gn], want[~wn])


def test_produced_cache_decodes_like_host_filled_cache():
    """Producer -> decode: a paged cache written by the producer from bf16
    latent / rope gives the same decode output as the same rows quantised on
    the host, and matches the oracle."""
    B, H, lens = 3, 16, [700, 1290, 64]
    total = sum(lens)
    g = torch.Generator().manual_seed(21)
    c_kv = torch.randn(total, 512, generator=g).to(torch.bfloat16)
    k_pe = torch.randn(total, 64, generator=g).to(torch.bfloat16)
    num_slots = total + 100
    slots = torch.randperm(num_slots, generator=g)[:total].to(torch.int32)
    pool_gpu = _run(c_kv, k_pe, num_slots, slots, KV_SCALE, False)
    pool_host = np.zeros((num_slots, QK), np.uint8)
    pool_host[slots.numpy()] = of8.quantize_rows(c_kv.float().numpy(), k_pe.float().numpy(), KV_SCALE)
    assert np.array_equal(pool_gpu[slots.numpy()], pool_host[slots.numpy()])
    pool = torch.from_numpy(pool_gpu).view(num_slots, 1, QK).view(torch.float8_e4m3fn).to(DEV)
    indptr = torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int32)
    q_lat, q_pe = (t[:, 0].contiguous() for t in rand_q(B, 1, H, 22))
    o = torch.zeros(B, H, 512, dtype=torch.bfloat16, device=DEV)
    parts = ma.mla_decode_a16w8_plan_parts_q(B, max(lens), 1, H)
    ma.mla_decode_a16w8_paged_dev(q_lat.to(DEV), q_pe.to(DEV), pool, o, torch.tensor(lens, dtype=torch.int32).to(DEV),
                                  None, slots.to(DEV), indptr.to(DEV), parts, SCALE_192, KV_SCALE)
    torch.cuda.synchronize()
    ref, _, A = om.decode(q_lat.float().numpy()[:, None], q_pe.float().numpy()[:, None], pool_host[:, None], lens,
                          SCALE_192, KV_SCALE, kv_indices=slots.numpy(), kv_indptr=indptr.numpy(), aux=True)
    log_stats("kv_quant_then_decode_b3_h16", compare_bf16(bits(o)[:, None], ref, A))


def test_c_abi_rejects_bad_scale_and_sizes():
    z = torch.zeros(1, dtype=torch.int32, device=DEV)
    p = _lib.ptr
    st = _lib.stream_ptr(DEV)
    assert _lib.lib.launch_mla_kv_quantize(p(z), p(z), p(z), p(z), 1, 1, 0.0, 0, st) == -12
    assert _lib.lib.launch_mla_kv_quantize(p(z), p(z), p(z), p(z), 1, 1, float("nan"), 0, st) == -12
    assert _lib.lib.launch_mla_kv_quantize(p(z), p(z), p(z), p(z), -1, 1, 1.0, 0, st) == -4
    assert _lib.lib.launch_mla_kv_quantize(None, p(z), p(z), p(z), 1, 1, 1.0, 0, st) == -6
    assert _lib.lib.launch_mla_kv_quantize(p(z), p(z), p(z), p(z), 0, 1, 1.0, 0, st) == 0
