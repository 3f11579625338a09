"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_fixtures.py):
the CPU oracle must reproduce them bit for bit; on the GPU the kernels must
match them under the tolerance rule."""
import pathlib

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import bf16 as ob
from oracle import mla as om
from helpers import compare_bf16

G = pathlib.Path(__file__).resolve().parent / "golden"


def _f32(u16):
    return ob.bf16_to_f32(u16)


def _bf16_tensor(u16):
    return torch.from_numpy(u16.view(np.int16).copy()).view(torch.bfloat16)


def test_attention_fixture_reproduced_by_oracle():
    z = np.load(G / "attention_bhsd_1x2x80x150.npz")
    for mode in ("rtne", "rtna", "rtz"):
        o = oa.forward(_f32(z["q"]), _f32(z["k"]), _f32(z["v"]), mode)
        assert np.array_equal(o, z[f"out_{mode}"]), mode


def test_mla_fixture_reproduced_by_oracle():
    z = np.load(G / "mla_paged_b2_q2_h8.npz")
    o = om.decode(_f32(z["q_lat"]), _f32(z["q_pe"]), z["pool"], z["seq_lens"], float(z["softmax_scale"]),
                  float(z["kv_scale"]), kv_indices=z["kv_indices"], kv_indptr=z["kv_indptr"])
    assert np.array_equal(o, z["out"])


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["rtne", "rtna", "rtz"])
def test_attention_kernel_matches_fixture(mode):
    import moonmath_attention as ma

    z = np.load(G / "attention_bhsd_1x2x80x150.npz")
    q, k, v = (_bf16_tensor(z[n]).to("cuda:0") for n in ("q", "k", "v"))
    out = ma.forward(q, k, v, round_mode=mode, layout="bhsd")
    torch.cuda.synchronize()
    got = out.cpu().view(torch.int16).numpy().view(np.uint16)
    for h in range(2):
        compare_bf16(got[0, h], z[f"out_{mode}"][0, h], z[f"scale_{mode}"][0, h].astype(np.float64))


@pytest.mark.gpu
def test_mla_kernel_matches_fixture():
    import moonmath_attention as ma

    z = np.load(G / "mla_paged_b2_q2_h8.npz")
    dev = "cuda:0"
    q_lat, q_pe = _bf16_tensor(z["q_lat"]).to(dev), _bf16_tensor(z["q_pe"]).to(dev)
    pool = torch.from_numpy(z["pool"].copy()).view(torch.float8_e4m3fn).to(dev)
    o = torch.zeros_like(q_lat)
    lens = torch.from_numpy(z["seq_lens"]).to(dev)
    idx = torch.from_numpy(z["kv_indices"]).to(dev)
    ptr = torch.from_numpy(z["kv_indptr"]).to(dev)
    parts = ma.mla_decode_a16w8_multiq_plan_parts_q(2, 100, 2, 8)
    ma.mla_decode_a16w8_multiq_paged_dev(q_lat, q_pe, pool, o, lens, None, idx, ptr, parts,
                                         float(z["softmax_scale"]), float(z["kv_scale"]))
    torch.cuda.synchronize()
    got = o.cpu().view(torch.int16).numpy().view(np.uint16)
    compare_bf16(got, z["out"], z["scale"].astype(np.float64))
