"""Seeded MLA decode inputs shared by the tests and the bench (reference test
pattern tests/test_mla_decode.py:34-47, 73-91, with OCP e4m3fn KV)."""
import math

import numpy as np
import torch

LAT, ROPE, QK = 512, 64, 576
KV_SCALE = 1.0 / 32.0
QPEAK = 3.0
SCALE_192 = 1.0 / math.sqrt(192.0)  # DeepSeek-V3 qk head dim 128 + 64
SCALE_576 = QK ** -0.5              # the reference test's scale


def rand_q(B, q_len, H, seed, peak=QPEAK):
    g = torch.Generator().manual_seed(seed + 1)
    q_lat = (torch.randn(B, q_len, H, LAT, generator=g) * peak).to(torch.bfloat16)
    q_pe = (torch.randn(B, q_len, H, ROPE, generator=g) * peak).to(torch.bfloat16)
    return q_lat, q_pe


def rand_kv_rows(n, seed):
    """n fused rows of fp8: N(0,1)*KV_SCALE quantised at KV_SCALE (-> e4m3fn of N(0,1))."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(n, QK, generator=g) * KV_SCALE
    return (x / KV_SCALE).to(torch.float8_e4m3fn)


def paged_pool(seq_lens, seed, page=64, slack=1.25):
    """Random 64-token block tables over a pool of pages, flattened to the
    flat-slot ABI: kv_indices[indptr[b] + j] = block[b][j // page] * page + j % page.
    Returns (pool [slots,1,576] fp8, kv_indices int32, kv_indptr int32)."""
    g = torch.Generator().manual_seed(seed + 2)
    pages_per = [-(-int(s) // page) for s in seq_lens]
    n_pages = int(math.ceil(sum(pages_per) * slack))
    perm = torch.randperm(n_pages, generator=g)
    pool = rand_kv_rows(n_pages * page, seed).view(n_pages * page, 1, QK)
    idx, indptr, off = [], [0], 0
    for b, s in enumerate(seq_lens):
        blocks = perm[off:off + pages_per[b]]
        off += pages_per[b]
        j = torch.arange(int(s))
        idx.append(blocks[j // page] * page + j % page)
        indptr.append(indptr[-1] + int(s))
    kv_indices = torch.cat(idx).to(torch.int32)
    return pool, kv_indices, torch.tensor(indptr, dtype=torch.int32)


def fp8_bits(t):
    return t.contiguous().view(torch.uint8).cpu().numpy()


def ragged_lens(B, lo, hi, seed):
    rng = np.random.default_rng(seed)
    return [int(x) for x in rng.integers(lo, hi + 1, size=B)]
