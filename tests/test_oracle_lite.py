"""CPU pinning of the LiteAttention oracle (no GPU).

Checks chosen so a plausible mistake fails: the compute-all seed decodes to
every block ascending; whatever the keep pattern, a written row decodes (in
the opposite phase, as the next step reads it) to exactly the kept blocks, so
emitter and cursor agree on markers, directions and range ends; must_do pins
blocks; the work count matches a hand case from the reference's own comment
and the reference test's direction-free count; the LPT order is a stable
heaviest-first permutation; a tile's output over all blocks is the dense
oracle's.
"""
import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import lite as ol


def _ref_kept_blocks(row):
    """The reference test's count of kept blocks (tests/test_attention.py:154-158)."""
    n = int(row[0])
    return sum(abs(int(row[i]) - int(row[i - 1])) for i in range(n, 1, -2))


@pytest.mark.parametrize("nkb", [1, 2, 5, 64])
def test_seed_decodes_to_every_block_ascending(nkb):
    blocks, ends = ol.decode(ol.seed_row(nkb), nkb, phase=1)
    assert blocks == list(range(nkb))
    assert ends == [False] * (nkb - 1) + [True]


@pytest.mark.parametrize("seed", range(6))
def test_written_row_decodes_to_kept_blocks_in_the_next_phase(seed):
    rng = np.random.default_rng(seed)
    nkb = int(rng.integers(1, 40))
    row = ol.seed_row(nkb)
    phase = 1
    kept_prev = list(range(nkb))
    for _ in range(4):
        blocks, ends = ol.decode(np.asarray(row), nkb, phase)
        assert sorted(blocks) == sorted(kept_prev)
        # blocks are walked monotonically in the phase's direction
        assert blocks == sorted(blocks, reverse=(phase == 0))
        keep = [True] + [bool(x) for x in rng.integers(0, 2, len(blocks) - 1)]
        nxt = ol.emit(blocks, ends, keep, phase, nkb)
        kept_prev = [b for b, k in zip(blocks, keep) if k]
        assert _ref_kept_blocks(nxt) == len(kept_prev) == ol.kept_count(nxt, nkb)
        assert nxt[0] <= nkb + 1
        row = np.array(nxt + [0] * (nkb + 2 - len(nxt)), dtype=np.int16)
        phase = 1 - phase


def test_emit_hand_case():
    """Phase 1 over one range 0..9 keeping 0-2 and 6-7: markers 0,3 and 6,8."""
    blocks, ends = ol.decode(ol.seed_row(10), 10, 1)
    keep = [b in (0, 1, 2, 6, 7) for b in blocks]
    assert ol.emit(blocks, ends, keep, 1, 10) == [4, 0, 3, 6, 8]
    # read back in phase 0: ranges from the back: (8, 6) -> 7, 6; then (3, 0) -> 2, 1, 0
    b2, e2 = ol.decode(np.array([4, 0, 3, 6, 8, 0, 0, 0, 0, 0, 0, 0], np.int16), 10, 0)
    assert b2 == [7, 6, 2, 1, 0] and e2 == [False, True, False, False, True]


def test_must_do_pins_blocks():
    blocks, ends = ol.decode(ol.seed_row(12), 12, 1)
    keep = [True] + [False] * 11
    row = ol.emit(blocks, ends, keep, 1, 12, must_do=np.array([2, 0, 12], np.int16))
    assert ol.decode(np.array(row + [0] * 12, np.int16), 12, 0)[0] == list(range(11, -1, -1))
    row = ol.emit(blocks, ends, keep, 1, 12, must_do=np.array([4, 5, 7, 9, 10], np.int16))
    got = sorted(ol.decode(np.array(row + [0] * 12, np.int16), 12, 0)[0])
    assert got == [0, 5, 6, 9]


def test_kept_count_reference_hand_case():
    """Reference comment (attention_kernel.hip:1314-1315): (lstep=+1)
    row=[4,9,5,20,18] -> 4 + 2 = kept 6."""
    assert ol.kept_count(np.array([4, 9, 5, 20, 18], np.int16), 30) == 6


def test_lpt_order_is_stable_heaviest_first():
    nkb = 63  # 64 buckets of one block each
    rows = []
    for kept in (3, 10, 3, 63, 0, 10):
        r = np.zeros(nkb + 2, np.int16)
        if kept:
            r[:3] = (2, kept - 1, -1)
        rows.append(r)
    assert ol.lpt_order(rows, nkb) == [3, 1, 5, 0, 2, 4]


def test_votes_keep_first_and_near_max_blocks():
    """Block scores 5 (first), 9 (raises the max), 8.5 (within 1), 2 (7 below)."""
    c = float(oa.SCALE_LOG2E)
    s = np.array([[5 / c] * 64 + [9 / c] * 64 + [8.5 / c] * 64 + [2 / c] * 64], np.float32)
    assert ol.votes(s, [0, 1, 2, 3], 256, threshold=-3.0) == [True, True, True, False]
    assert ol.votes(s, [3, 2, 1, 0], 256, threshold=-3.0) == [True, True, True, False]


# Block maxima 4 and 3.9375 (bf16-exact scores); threshold = fl(fl(3.9375 c) - fl(4 c)).
VOTE_EDGE = (4.0, 3.9375)


def vote_edge_threshold():
    c = np.float32(oa.SCALE_LOG2E)
    return np.float32(np.float32(VOTE_EDGE[1]) * c - np.float32(VOTE_EDGE[0]) * c)


def test_votes_round_the_product_and_the_difference_separately():
    """The vote is fl(fl(bm c) - run) > thr with both roundings. At a threshold
    equal to that difference the block is dropped, while a fused
    multiply-subtract (one rounding; fl(3.9375 c) rounds down here) would keep
    it: the planted fused vote below disagrees on exactly this case."""
    from fractions import Fraction
    c = np.float32(oa.SCALE_LOG2E)
    thr = vote_edge_threshold()
    s = np.array([[VOTE_EDGE[0]] * 64 + [VOTE_EDGE[1]] * 64], np.float32)
    assert ol.votes(s, [0, 1], 128, threshold=float(thr)) == [True, False]
    assert ol.votes(s, [0, 1], 128, threshold=float(np.nextafter(thr, np.float32(-1)))) == [True, True]
    run = np.float32(VOTE_EDGE[0]) * c
    fused = np.float32(float(Fraction(VOTE_EDGE[1]) * Fraction(float(c)) - Fraction(float(run))))
    assert fused > thr  # a fused vote keeps block 1


def test_forward_tile_compute_all_equals_dense_oracle():
    g = torch.Generator().manual_seed(3)
    q, k, v = (torch.randn(n, 128, generator=g).to(torch.bfloat16).float().numpy() for n in (40, 300, 300))
    blocks, _ = ol.decode(ol.seed_row(5), 5, 1)
    assert np.array_equal(ol.forward_tile(q, k, v, blocks, 1), oa.head_forward(q, k, v, 1)[0])
    # descending order, same keys: same result
    assert np.array_equal(ol.forward_tile(q, k, v, blocks[::-1], 1), oa.head_forward(q, k, v, 1)[0])


def test_forward_tile_subset_equals_dense_oracle_on_kept_keys():
    """A skip list computes attention over exactly the keys of its kept
    blocks: the same as the dense oracle on those keys alone (ragged last
    block included), in either processing order."""
    g = torch.Generator().manual_seed(5)
    skv = 300  # 5 blocks, the last one 44 keys
    q, k, v = (torch.randn(n, 128, generator=g).to(torch.bfloat16).float().numpy() for n in (40, skv, skv))
    for blocks in ([0, 2, 4], [4, 1], [3]):
        keys = np.concatenate([np.arange(64 * b, min(64 * b + 64, skv)) for b in sorted(blocks)])
        want = oa.head_forward(q, k[keys], v[keys], 1)[0]
        assert np.array_equal(ol.forward_tile(q, k, v, blocks, 1), want), blocks
    # a planted mistake (off-by-one block) does not match
    wrong = oa.head_forward(q, k[64:192], v[64:192], 1)[0]
    assert not np.array_equal(ol.forward_tile(q, k, v, [0, 2], 1), wrong)
