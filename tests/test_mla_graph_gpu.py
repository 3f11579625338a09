"""MLA paged decode as a serving stack drives it: 64-token block tables and
HIP-graph capture with the split count fixed (reference moonmath_attention/
mla.py:64-95: the paged ops are device-driven so a graph captured once can be
replayed while seq_lens / kv_indices / kv_indptr / rows change in place).

Each replay is checked bit-identical to an eager call on the same inputs,
with eager work and synchronisations between the replays; block-table calls
are checked bit-identical to the flat-slot op on the equivalent slots and, on
sampled requests, against the CPU oracle.
"""
import numpy as np
import pytest
import torch

import moonmath_attention as ma
from moonmath_attention import _lib
from oracle import mla as om
from helpers import bits, compare_bf16, log_stats
from mla_inputs import KV_SCALE, QK, SCALE_192, fp8_bits, rand_kv_rows, rand_q

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
PAGE = 64


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    assert torch.cuda.is_available(), "GPU tests need an MI355X"


def _block_table(lens, max_blocks, num_blocks, seed):
    """Random distinct pages per request; unused table entries point anywhere."""
    g = torch.Generator().manual_seed(seed)
    perm = torch.randperm(num_blocks, generator=g).to(torch.int32)
    bt = torch.randint(0, num_blocks, (len(lens), max_blocks), generator=g, dtype=torch.int32)
    off = 0
    for b, L in enumerate(lens):
        n = -(-L // PAGE)
        bt[b, :n] = perm[off:off + n]
        off += n
    return bt


def _flat_from_table(bt, lens):
    idx = torch.cat([bt[b, torch.arange(L) // PAGE] * PAGE + torch.arange(L) % PAGE for b, L in enumerate(lens)])
    indptr = torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int32)
    return idx.to(torch.int32), indptr


@pytest.mark.parametrize("H,q_len", [(16, 1), (128, 1), (16, 2), (128, 2)])
def test_paged_blocks_matches_flat_slots(H, q_len):
    B, max_blocks = 5, 40
    lens = [2500, 64, 1, 1300, 2560]
    num_blocks = int(sum(-(-L // PAGE) for L in lens) * 1.5)
    pool = rand_kv_rows(num_blocks * PAGE, 7).view(num_blocks, PAGE, QK)
    bt = _block_table(lens, max_blocks, num_blocks, 8)
    idx, indptr = _flat_from_table(bt, lens)
    q_lat, q_pe = rand_q(B, q_len, H, 9)
    if q_len == 1:
        q_lat, q_pe = q_lat[:, 0].contiguous(), q_pe[:, 0].contiguous()
    parts = ma.mla_decode_a16w8_plan_parts_q(B, max(lens), q_len, H)
    d = lambda t: t.to(DEV)
    lens_t = torch.tensor(lens, dtype=torch.int32)
    o_blk = torch.full(q_lat.shape, float("nan"), dtype=torch.bfloat16, device=DEV)
    o_flat = torch.full(q_lat.shape, float("nan"), dtype=torch.bfloat16, device=DEV)
    ma.mla_decode_a16w8_paged_blocks(d(q_lat), d(q_pe), d(pool), o_blk, d(lens_t), d(bt), parts, SCALE_192, KV_SCALE)
    flat_pool = d(pool.view(num_blocks * PAGE, 1, QK))
    if q_len == 1:
        ma.mla_decode_a16w8_paged_dev(d(q_lat), d(q_pe), flat_pool, o_flat, d(lens_t), None, d(idx), d(indptr),
                                      parts, SCALE_192, KV_SCALE)
    else:
        ma.mla_decode_a16w8_multiq_paged_dev(d(q_lat), d(q_pe), flat_pool, o_flat, d(lens_t), None, d(idx),
                                             d(indptr), parts, SCALE_192, KV_SCALE)
    torch.cuda.synchronize()
    assert torch.equal(o_blk.view(torch.int16), o_flat.view(torch.int16))
    got = bits(o_blk)
    ql, qp = q_lat.float().numpy(), q_pe.float().numpy()
    if q_len == 1:
        got, ql, qp = got[:, None], ql[:, None], qp[:, None]
    ref, _, A = om.decode(ql, qp, fp8_bits(pool.view(-1, 1, QK)), lens, SCALE_192, KV_SCALE,
                          kv_indices=idx.numpy(), kv_indptr=indptr.numpy(), batches=[0, 1, 2], aux=True)
    stats = compare_bf16(got[:3], ref[:3], A[:3])
    log_stats(f"mla_blocks_b5_h{H}_q{q_len}", stats)


def test_paged_blocks_rejects_bad_tables():
    q_lat, q_pe = (t[:, 0].contiguous().to(DEV) for t in rand_q(2, 1, 16, 3))
    o = torch.empty_like(q_lat)
    pool = rand_kv_rows(4 * PAGE, 3).view(4, PAGE, QK).to(DEV)
    lens = torch.tensor([10, 20], dtype=torch.int32, device=DEV)
    with pytest.raises(ValueError, match="block_table"):
        ma.mla_decode_a16w8_paged_blocks(q_lat, q_pe, pool, o, lens, torch.zeros(2, 3, device=DEV), 1, 0.1, 0.5)
    with pytest.raises(ValueError, match="block_table"):
        ma.mla_decode_a16w8_paged_blocks(q_lat, q_pe, pool, o, lens, torch.zeros(3, 3, dtype=torch.int32,
                                                                                      device=DEV), 1, 0.1, 0.5)
    with pytest.raises(ValueError, match="pages"):
        ma.mla_decode_a16w8_paged_blocks(q_lat, q_pe, pool.view(-1, QK)[:100].contiguous(), o, lens,
                                         torch.zeros(2, 3, dtype=torch.int32, device=DEV), 1, 0.1, 0.5)


class _State:
    """Static device buffers of a decode graph, refilled in place per replay."""

    def __init__(self, B, H, q_len, max_len, num_blocks, seed):
        self.B, self.H, self.q_len, self.max_len = B, H, q_len, max_len
        self.max_blocks = -(-max_len // PAGE)
        self.num_blocks = num_blocks
        self.pool = rand_kv_rows(num_blocks * PAGE, seed).view(num_blocks * PAGE, 1, QK).to(DEV)
        shape = (B, q_len, H) if q_len > 1 else (B, H)
        self.q_lat = torch.empty(*shape, 512, dtype=torch.bfloat16, device=DEV)
        self.q_pe = torch.empty(*shape, 64, dtype=torch.bfloat16, device=DEV)
        self.lens = torch.empty(B, dtype=torch.int32, device=DEV)
        self.idx = torch.empty(B * max_len, dtype=torch.int32, device=DEV)
        self.indptr = torch.empty(B + 1, dtype=torch.int32, device=DEV)
        self.rows = torch.empty(B, dtype=torch.int32, device=DEV)
        self.bt = torch.empty(B, self.max_blocks, dtype=torch.int32, device=DEV)
        self.out = torch.empty(*shape, 512, dtype=torch.bfloat16, device=DEV)

    def refill(self, seed):
        g = torch.Generator().manual_seed(seed)
        ql, qp = rand_q(self.B, self.q_len, self.H, seed)
        if self.q_len == 1:
            ql, qp = ql[:, 0], qp[:, 0]
        self.q_lat.copy_(ql)
        self.q_pe.copy_(qp)
        lens = torch.randint(1, self.max_len + 1, (self.B,), generator=g).tolist()
        bt = _block_table(lens, self.max_blocks, self.num_blocks, seed + 1)
        idx, indptr = _flat_from_table(bt, lens)
        self.lens.copy_(torch.tensor(lens, dtype=torch.int32))
        self.idx[:idx.numel()].copy_(idx)
        self.indptr.copy_(indptr)
        self.rows.copy_(torch.randperm(self.B, generator=g).to(torch.int32))
        self.bt.copy_(bt)


def _op(kind, st, parts, out):
    if kind == "paged":
        ma.mla_decode_a16w8_paged_dev(st.q_lat, st.q_pe, st.pool, out, st.lens, st.rows, st.idx, st.indptr, parts,
                                      SCALE_192, KV_SCALE)
    elif kind == "multiq":
        ma.mla_decode_a16w8_multiq_paged_dev(st.q_lat, st.q_pe, st.pool, out, st.lens, st.rows, st.idx,
                                             st.indptr, parts, SCALE_192, KV_SCALE)
    elif kind == "blocks":
        ma.mla_decode_a16w8_paged_blocks(st.q_lat, st.q_pe, st.pool, out, st.lens, st.bt, parts, SCALE_192,
                                         KV_SCALE, rows=st.rows)
    else:  # the allocation-free C entry point
        p = _lib.ptr
        rc = _lib.lib.launch_mla_decode_a16w8_paged_dev_noalloc(
            p(st.q_lat), p(st.q_pe), p(st.pool), p(out), p(st.lens), p(st.rows), p(st.idx), p(st.indptr), st.B,
            st.H, parts, 512, 64, SCALE_192, KV_SCALE, 1.0, _lib.stream_ptr(DEV), st.idx.numel() * QK, st.q_len)
        assert rc == 0, rc


@pytest.mark.parametrize("kind,H,q_len", [("paged", 16, 1), ("paged", 128, 1), ("multiq", 128, 2),
                                          ("blocks", 16, 2), ("noalloc", 128, 1)])
def test_graph_capture_replay_with_inputs_updated_in_place(kind, H, q_len):
    B, max_len = 12, 3000
    st = _State(B, H, q_len, max_len, num_blocks=B * (-(-max_len // PAGE)) + 7, seed=40)
    parts = ma.mla_decode_a16w8_plan_parts_q(B, max_len, q_len, H)
    assert _lib.lib.moonmath_mla_effective_parts(B, H, parts, q_len, 1) > 1  # the split path is captured
    st.refill(1)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up outside the capture
        _op(kind, st, parts, st.out)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _op(kind, st, parts, st.out)
    eager_out = torch.empty_like(st.out)
    noise = torch.randn(512, 512, device=DEV)
    for r in range(4):
        st.refill(100 + r)
        torch.cuda.synchronize()
        graph.replay()
        _ = noise @ noise  # the program's own eager work between replays
        torch.cuda.synchronize()
        _op(kind, st, parts, eager_out)
        torch.cuda.synchronize()
        assert torch.equal(st.out.view(torch.int16), eager_out.view(torch.int16)), f"replay {r} differs from eager"
    # and the last replay against the oracle on two requests (through rows)
    got = bits(st.out)
    ql, qp = st.q_lat.float().cpu().numpy(), st.q_pe.float().cpu().numpy()
    if q_len == 1:
        got, ql, qp = got[:, None], ql[:, None], qp[:, None]
    lens = st.lens.cpu().numpy()
    rows = st.rows.cpu().numpy()
    ref, _, A = om.decode(ql, qp, fp8_bits(st.pool), lens, SCALE_192, KV_SCALE,
                          kv_indices=st.idx.cpu().numpy(), kv_indptr=st.indptr.cpu().numpy(), rows=rows,
                          batches=[0, 5], aux=True)
    sel = [int(rows[0]), int(rows[5])]
    log_stats(f"mla_graph_{kind}_h{H}_q{q_len}", compare_bf16(got[sel], ref[sel], A[sel]))
