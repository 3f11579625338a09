"""Writes the small golden fixtures under tests/golden/ from the CPU oracle.

The reference repository holds no golden vectors for these paths (its tests
draw seeded random data and compare against an fp32 formula), so these
fixtures pin this build's oracle output for fixed inputs: a regression anchor
for the oracle (tests/test_golden.py, CPU) and for the kernels (GPU).

    python tests/golden/make_fixtures.py
"""
import pathlib
import sys

import numpy as np
import torch

HERE = pathlib.Path(__file__).resolve().parent
sys.path[:0] = [str(HERE.parents[1]), str(HERE.parent)]

from oracle import attention as oa  # noqa: E402
from oracle import mla as om  # noqa: E402
from mla_inputs import KV_SCALE, SCALE_192, fp8_bits, paged_pool, rand_q  # noqa: E402


def bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def attention_fixture():
    g = torch.Generator().manual_seed(42)
    q = torch.randn(1, 2, 80, 128, generator=g).to(torch.bfloat16)
    k = torch.randn(1, 2, 150, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(1, 2, 150, 128, generator=g).to(torch.bfloat16)
    out = {"q": bits(q), "k": bits(k), "v": bits(v)}
    for mode in ("rtne", "rtna", "rtz"):
        o, _, a, _ = oa.forward(q.float().numpy(), k.float().numpy(), v.float().numpy(), mode, aux=True)
        out[f"out_{mode}"] = o
        out[f"scale_{mode}"] = a.astype(np.float16)  # tolerance floor only; half precision suffices
    np.savez_compressed(HERE / "attention_bhsd_1x2x80x150.npz", **out)


def mla_fixture():
    lens = [100, 37]
    pool, idx, indptr = paged_pool(lens, 3)
    q_lat, q_pe = rand_q(2, 2, 8, 3)
    o, _, a = om.decode(q_lat.float().numpy(), q_pe.float().numpy(), fp8_bits(pool), lens, SCALE_192, KV_SCALE,
                        kv_indices=idx.numpy(), kv_indptr=indptr.numpy(), aux=True)
    np.savez_compressed(HERE / "mla_paged_b2_q2_h8.npz", q_lat=bits(q_lat), q_pe=bits(q_pe),
                        pool=fp8_bits(pool), kv_indices=idx.numpy(), kv_indptr=indptr.numpy(),
                        seq_lens=np.array(lens, dtype=np.int32), out=o, scale=a.astype(np.float16),
                        softmax_scale=np.float64(SCALE_192), kv_scale=np.float64(KV_SCALE))


if __name__ == "__main__":
    attention_fixture()
    mla_fixture()
    print("fixtures written to", HERE)
