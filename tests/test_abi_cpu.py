"""CPU tests of the boundary (no GPU): the library loads, exports every symbol
include/moonmath_gfx950.h declares, the host planners agree with the oracle's
restatement, and the Python surface raises the reference's exception types and
messages before touching a device (reference moonmath_attention/_kernel.py:41-82,
csrc/attention_api.cpp:134-229, csrc/mla_decode_a16w8_api.cpp:41-62,
csrc/mla_decode_a16w8_multiq_api.cpp:42-62)."""
import ctypes
import pathlib
import re

import pytest
import torch

import moonmath_attention as ma
from moonmath_attention import _lib
from oracle import planner

ROOT = pathlib.Path(__file__).resolve().parents[1]


def _header_symbols():
    text = (ROOT / "include" / "moonmath_gfx950.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(?:int|size_t)\s+(\w+)\s*\(", text)))


def test_header_declares_symbols():
    assert len(_header_symbols()) >= 26


@pytest.mark.parametrize("name", _header_symbols())
def test_library_exports_header_symbol(name):
    dll = ctypes.CDLL(_lib.LIB_PATH)
    assert hasattr(dll, name), name
    assert name in _lib.SIGNATURES, f"{name} not bound in _lib.SIGNATURES"


def test_attention_geometry():
    """One 8-wave CTA of 256 q rows per CU, 64-row kv blocks, 256 CUs, 1024
    split parts (the workspace size follows from these)."""
    geo = _lib.geometry()
    assert geo == {"rows_per_cta": 256, "kv_block": 64, "slots": 256, "max_parts": 1024}
    assert _lib.lib.tail_workspace_bytes_rtne() == 1024 * 256 * (128 + 2) * 4


@pytest.mark.parametrize("B,H,S,Skv", [(2, 24, 8192, 8192), (2, 24, 4097, 512), (2, 8, 86016, 86016),
                                       (1, 32, 16384, 16384), (1, 2, 256, 256), (3, 7, 5000, 9000),
                                       (1, 1, 100000, 100000), (4, 3, 777, 8191), (2, 24, 4097, 1024),
                                       (2, 24, 4097, 2048), (2, 24, 4097, 960)])
def test_tail_planner_matches_oracle(B, H, S, Skv):
    geo = _lib.geometry()
    nqb = -(-S // geo["rows_per_cta"])
    nkb = -(-Skv // 64)
    want = planner.plan_tail(nqb, B * H, nkb, geo["slots"], geo["max_parts"])
    assert _lib.plan_tail(B, H, S, Skv) == want


def test_tail_planner_splits_the_4097_shape():
    """(2,24,4097,8192): 17 q-blocks x 48 heads = 816 CTAs, a 48-CTA tail over
    128 kv blocks. G = 5: 240 parts in one round of 26 blocks,
    (26 + 4) + 3 + 4 = 37, beats G = 16 (three rounds of 8: 51) and no split (132)."""
    assert _lib.plan_tail(2, 24, 4097, 8192) == (768, 48, 5, 240)


def test_tail_planner_splits_short_kv_tails():
    """Below the reference's 48-block threshold: (2,24,4097,2048) has 32 kv
    blocks, split 4 ways in one round; 960 keys (15 blocks) stay unsplit."""
    assert _lib.plan_tail(2, 24, 4097, 2048) == (768, 48, 4, 192)
    assert _lib.plan_tail(2, 24, 4097, 960) == (816, 0, 1, 0)


def test_tail_planner_disabled_and_forced():
    geo = _lib.geometry()
    wgs = -(-4173 // geo["rows_per_cta"]) * 4
    assert _lib.plan_tail(1, 4, 4173, 4173, enable=False) == (wgs, 0, 1, 0)
    pre, tail, g, parts = _lib.plan_tail(1, 4, 4173, 4173, True, 5)
    assert g == 5 and parts == tail * 5 and pre + tail == wgs


def test_attention_launcher_argument_codes():
    lib = _lib.lib
    nul = None
    assert lib.launch_attention_forward_rtne(nul, nul, nul, nul, 0, 1, 1, 1, 128, 0, nul, nul) == 1
    assert lib.launch_attention_forward_rtne(nul, nul, nul, nul, 1, 1, 0, 1, 128, 0, nul, nul) == 2
    assert lib.launch_attention_forward_rtne(nul, nul, nul, nul, 1, 1, 1, 1, 64, 0, nul, nul) == 3
    assert lib.launch_attention_forward_rtne(nul, nul, nul, nul, 1, 1, 1, 0, 128, 0, nul, nul) == 5
    assert lib.launch_attention_forward_rtne(nul, nul, nul, nul, 1, 1, 1, 1, 128, 2, nul, nul) == 7
    assert lib.launch_attention_forward_rtne(nul, nul, nul, nul, 1, 1, 1, 1, 128, 0, nul, nul) == 8
    assert lib.moonmath_attention_forward_ex(nul, nul, nul, nul, 1, 1, 1, 1, 128, 0, 9, nul, 0, nul) == 10


def test_mla_launcher_argument_codes():
    lib = _lib.lib
    nul = None
    args = (nul, nul, nul, nul, nul, nul, nul, nul)
    assert lib.launch_mla_decode_a16w8_paged_dev(*args, 1, 16, 1, 256, 64, 1.0, 1.0, 1.0, nul, nul, 0, 1) == -2
    assert lib.launch_mla_decode_a16w8_paged_dev(*args, 1, 129, 1, 512, 64, 1.0, 1.0, 1.0, nul, nul, 0, 1) == -3
    assert lib.launch_mla_decode_a16w8_paged_dev(*args, 1, 16, 1, 512, 64, 1.0, 1.0, 1.0, nul, nul, 0, 9) == -4
    assert lib.launch_mla_decode_a16w8_paged_dev(*args, 1, 16, 1, 512, 64, 1.0, 1.0, 1.0, nul, nul, 0, 1) == -6
    assert lib.mla_decode_a16w8_plan_parts_q(4, 1024, 9, 16) == -4


def test_mla_noalloc_argument_codes_match_the_workspace_launcher():
    """The allocation-free entry returns the workspace launcher's code for every
    argument error, checked before its own scratch limit (-9): bad dims -2,
    bad H -3, bad q_len or B -4, null pointers -6 -- also with a parts count
    whose records would not fit the scratch array."""
    lib = _lib.lib
    nul = None
    args = (nul, nul, nul, nul, nul, nul, nul, nul)
    for B, H, parts, lat, ql in ((1, 16, 1, 256, 1), (1, 129, 1, 512, 1), (1, 0, 1, 512, 1), (1, 16, 1, 512, 9),
                                 (0, 16, 1, 512, 1), (1, 16, 1, 512, 1), (64, 200, 4, 512, 2), (64, 128, 4, 256, 2),
                                 (64, 128, 4, 512, 2)):
        want = lib.launch_mla_decode_a16w8_paged_dev(*args, B, H, parts, lat, 64, 1.0, 1.0, 1.0, nul, nul, 0, ql)
        got = lib.launch_mla_decode_a16w8_paged_dev_noalloc(*args, B, H, parts, lat, 64, 1.0, 1.0, 1.0, nul, 0, ql)
        assert got == want != 0, (B, H, parts, lat, ql, got, want)
    assert lib.launch_mla_decode_a16w8_paged_dev_noalloc(*args, 1, 129, 1, 512, 64, 1.0, 1.0, 1.0, nul, 0, 1) == -3


def test_mla_planners():
    for B, H, S, ql in [(64, 128, 8192, 1), (64, 128, 8192, 2), (64, 16, 8192, 1), (2, 16, 2048, 4), (1, 1, 1, 1),
                        (8, 100, 4096, 1), (8, 48, 4096, 2)]:
        p = ma.mla_decode_a16w8_plan_parts_q(B, S, ql, H)
        assert 1 <= p <= max(1, -(-S // 32))
        eff = _lib.lib.moonmath_mla_effective_parts(B, H, p, ql, 1)
        assert eff == p  # planned parts always fit the workspace
        # O records of R rows (the 128-row kernel's whole 32-row tiles for 96..128
        # query rows), an (m, l) pair per query row and part, 8 bytes per request.
        qrows = H * ql
        R = 32 * -(-qrows // 32) if 96 <= qrows <= 128 else qrows
        assert _lib.lib.mla_decode_a16w8_multiq_workspace_for(B, H, p, ql) == B * p * (R * 512 + qrows * 2) * 4 + 8 * B
    assert _lib.lib.moonmath_mla_effective_parts(4, 16, 9, 1, 0) == 1  # no workspace -> no split


# ---- Python surface validation (raises before any device work) -------------------


def _bf16(*shape):
    return torch.zeros(*shape, dtype=torch.bfloat16)


def test_forward_type_errors():
    q = _bf16(1, 2, 8, 128)
    with pytest.raises(TypeError, match="q must be torch.Tensor"):
        ma.forward([1], q, q)
    with pytest.raises(TypeError, match="k must be torch.bfloat16"):
        ma.forward(q, q.float(), q)
    with pytest.raises(ValueError, match="v must be 4-D"):
        ma.forward(q, q, q[0])


def test_forward_cpu_device_mix():
    q = _bf16(1, 2, 8, 128)
    k = torch.empty(1, 2, 8, 128, dtype=torch.bfloat16, device="meta")
    with pytest.raises(ValueError, match="all must be on the same device"):
        ma.forward(q, k, q)


def test_forward_unsupported_device():
    q = torch.empty(1, 2, 8, 128, dtype=torch.bfloat16, device="meta")
    with pytest.raises(NotImplementedError):
        ma.forward(q, q, q)


def test_check_args_messages():
    from moonmath_attention._kernel import check_args

    class FakeCuda:
        """check_args only reads dtype/dim/shape/contiguity/device."""

        def __init__(self, shape, dtype=torch.bfloat16, contiguous=True):
            self.shape = torch.Size(shape)
            self.dtype = dtype
            self._c = contiguous
            self.device = torch.device("cuda", 0)

        def dim(self):
            return len(self.shape)

        def is_contiguous(self):
            return self._c

    q = FakeCuda((2, 4, 16, 128))
    with pytest.raises(ValueError, match="round_mode must be"):
        check_args(q, q, q, None, "rtnx", "bhsd")
    with pytest.raises(ValueError, match="layout must be"):
        check_args(q, q, q, None, "rtne", "bsdh")
    with pytest.raises(ValueError, match="head_dim must be 128"):
        d64 = FakeCuda((2, 4, 16, 64))
        check_args(d64, d64, d64, None, "rtne", "bhsd")
    with pytest.raises(ValueError, match="k shape mismatch"):
        check_args(q, FakeCuda((2, 5, 16, 128)), q, None, "rtne", "bhsd")
    with pytest.raises(ValueError, match="v shape mismatch"):
        check_args(q, q, FakeCuda((2, 4, 17, 128)), None, "rtne", "bhsd")
    with pytest.raises(ValueError, match="must be contiguous"):
        check_args(FakeCuda((2, 4, 16, 128), contiguous=False), q, q, None, "rtne", "bhsd")
    with pytest.raises(ValueError, match="out shape must match"):
        check_args(q, q, q, FakeCuda((2, 4, 15, 128)), "rtne", "bhsd")
    assert check_args(q, FakeCuda((2, 4, 40, 128)), FakeCuda((2, 4, 40, 128)), None, "rtz", "bhsd") == (2, 4, 16, 40, 0)
    qs = FakeCuda((2, 16, 4, 128))
    assert check_args(qs, qs, qs, None, "rtna", "bshd") == (2, 4, 16, 16, 1)


def test_mla_checks_without_device():
    from moonmath_attention.mla import _check_q

    q = _bf16(2, 16, 512)
    with pytest.raises(ValueError, match="tensors must be on a CUDA/HIP device"):
        _check_q(q, _bf16(2, 16, 64), _bf16(2, 16, 512), "x", multiq=False)
    with pytest.raises(ValueError, match=r"\[B,q_len,H,512\]"):
        _check_q(q, _bf16(2, 16, 64), _bf16(2, 16, 512), "x", multiq=True)
    with pytest.raises(ValueError, match="must be bfloat16"):
        _check_q(q.float(), _bf16(2, 16, 64), _bf16(2, 16, 512), "x", multiq=False)
    with pytest.raises(ValueError, match="same rank"):
        _check_q(q, _bf16(2, 1, 16, 64), _bf16(2, 16, 512), "x", multiq=False)


def _mla_units(lens, c):
    return sum(1 if L <= c else -(-L // c) for L in lens)


def _mla_search_chunk(lens, budget):
    """csrc/mla_common.hpp search_chunk: bisection between sumL / budget and the
    feasible sumL / (budget - B) (or max L) over multiples of 32, >= 512."""
    B, sumL, maxL = len(lens), sum(lens), max(lens)
    hi = 512 if maxL < 512 else -(-maxL // 32) * 32
    if budget <= B:
        return hi
    ok = -(-sumL // (budget - B))
    if ok < hi:
        hi = 512 if ok < 512 else -(-ok // 32) * 32
    lo = min(-(-sumL // budget), hi)
    lo = max(512, min(-(-lo // 32) * 32, hi))
    while lo < hi:
        mid = lo + ((hi - lo) // 64) * 32
        if _mla_units(lens, mid) <= budget:
            hi = mid
        else:
            lo = mid + 32
    return hi


def test_mla_split_plan_fits_workspace():
    """The device split plan (budget U = max(B, min(B * P, cap)) units; chunk C =
    the smallest multiple of 32, >= 512, with sum_b max(1, ceil(L_b / C)) <= U)
    never needs more than B * P records and is minimal, for random and
    adversarial length mixes and the kernels' caps (256 CUs / CTAs per unit)."""
    import numpy as np

    rng = np.random.default_rng(3)
    cases = [rng.integers(0, 9000, size=int(rng.integers(1, 200))).tolist() for _ in range(300)]
    cases += [[0] * 7, [1] * 64, [100000] + [1] * 63, [512] * 10, [513] * 10, [8192] * 64]
    for lens in cases:
        B = len(lens)
        for P in (1, 2, 3, 4, 8, 16):
            for cap in (256, 128, 32):
                budget = max(B, min(B * P, cap))
                c = _mla_search_chunk(lens, budget)
                total = _mla_units(lens, c)
                assert c % 32 == 0 and c >= 512, (lens, P, cap, c)
                assert total <= budget <= max(B, B * P), (lens, P, cap, total)
                # minimal: 32 tokens less no longer fits (or the 512 floor)
                assert c == 512 or _mla_units(lens, c - 32) > budget, (lens, P, cap, c)
