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


def _bf(x):
    return torch.as_tensor(x, dtype=torch.float32).to(torch.bfloat16).float().numpy()


def _two_wave_case():
    """64 valid rows (two waves), 2 blocks. Block 0 is hot for every row; block
    1 is hot only for rows 0..15 (score 32 on dim 0) and scores 0 for the rest,
    5 log2 units below their running max (fl(32 c) = 4.08, m = 5)."""
    q = np.zeros((64, 128), np.float32)
    q[:16, 0] = 1.0
    q[16:, 1] = 1.0
    k = np.zeros((128, 128), np.float32)
    k[:64, 0] = 32.0
    k[:64, 1] = 32.0
    k[64:, 0] = 32.0
    g = torch.Generator().manual_seed(11)
    v = _bf(torch.randn(128, 128, generator=g))
    return q, k, v


def test_soft_skip_is_per_wave_of_32_rows():
    """Wave 0 (rows 0..31) keeps block 1 because rows 0..15 are within the
    threshold, so rows 16..31 see it too; wave 1 (rows 32..63) drops it and its
    rows are attention over block 0 alone. The tile's vote keeps both blocks.
    Expected values are the dense oracle on the stated key sets; a per-row
    skip, 16- or 48-row waves, or no soft skip (the whole list for every row)
    each give a different output, so each such mistake fails."""
    q, k, v = _two_wave_case()
    row = ol.seed_row(2)
    out, nxt, blocks = ol.step_tile(q, k, v, row, 1, -3.0, 1)
    assert blocks == [0, 1]
    both = oa.head_forward(q, k, v, 1)[0]
    first = oa.head_forward(q, k[:64], v[:64], 1)[0]
    assert np.array_equal(out[:32], both[:32])
    assert np.array_equal(out[32:], first[32:])
    assert nxt == ol.emit(blocks, [False, True], [True, True], 1, 2)
    assert [kb for _, _, kb in ol.wave_blocks(q, k, row, 1, -3.0)] == [[0, 1], [0]]
    # The mistakes a grouping or skip error would make differ from the oracle.
    per_row = np.concatenate([both[:16], first[16:]])
    rows48 = np.concatenate([both[:48], first[48:]])
    assert not np.array_equal(out, per_row)  # also what 16-row waves give
    assert not np.array_equal(out, rows48)
    assert not np.array_equal(out, both)  # no soft skip


def test_soft_skip_keeps_the_running_max_of_kept_blocks_only():
    """At threshold 0 a block can be dropped while its max is above the
    running max (block max 4.08 after 4.09): the wave's running max must stay
    that of the kept blocks, so block 2 (4.085) is compared with 4.09, not
    with block 1's max. One row, scores in log2 units x / c."""
    c = float(oa.SCALE_LOG2E)
    s = np.array([[4.08 / c] * 64 + [4.09 / c] * 64 + [4.06 / c] * 64 + [4.085 / c] * 64], np.float32)
    # block 1 > block 0 (kept, run = 4.09); block 2 below (dropped); block 3 below run (dropped)
    assert ol.wave_keep(s, [0, 1, 2, 3], 256, 0.0) == [True, True, False, False]
    # order 1, 0, 3: block 0 and 3 are below 4.09 -> dropped
    assert ol.wave_keep(s, [1, 0, 3], 256, 0.0) == [True, False, False]
    # with threshold -0.1 everything within 0.1 of the running max is kept
    assert ol.wave_keep(s, [1, 0, 2, 3], 256, -0.1) == [True, True, True, True]


def test_very_negative_threshold_is_attention_over_the_listed_blocks():
    """No wave drops a listed block at threshold -1e30: each tile is the dense
    oracle over exactly the keys its read row names."""
    g = torch.Generator().manual_seed(9)
    skv = 300
    q, k, v = (_bf(torch.randn(n, 128, generator=g)) for n in (100, skv, skv))
    b0, e0 = ol.decode(ol.seed_row(5), 5, 1)
    row = np.array(ol.emit(b0, e0, [True, False, True, True, False], 1, 5) + [0] * 7, np.int16)[:7]
    blocks, _ = ol.decode(row, 5, 0)  # read back in phase 0: 3, 2, 0
    out, _, got_blocks = ol.step_tile(q, k, v, row, 0, -1e30, 0)
    keys = np.concatenate([np.arange(64 * b, min(64 * b + 64, skv)) for b in sorted(blocks)])
    assert got_blocks == blocks == [3, 2, 0]
    assert np.array_equal(out, oa.head_forward(q, k[keys], v[keys], 0)[0])


def _peaked_head(h, H=8, S=4096):
    """Reference _lite_qkv_peaked (tests/test_attention.py:107-127) for one
    head h: seed 7, K-blocks 0..h at scale 2, the rest at 0.05, bf16."""
    g = torch.Generator().manual_seed(7)
    q, k, v = (torch.randn(1, S, H, 128, generator=g) for _ in range(3))
    scale = torch.full((H, S), 0.05)
    for hh in range(H):
        scale[hh, : (hh + 1) * 64] = 2.0
    k = k * scale.t().view(1, S, H, 1)
    return tuple(t.to(torch.bfloat16).float().numpy()[0, :, h] for t in (q, k, v))


def test_peaked_head0_compute_all_is_attention_over_the_hot_block():
    """Reference peaked inputs, head 0, compute-all step: block 0 is hot (K at
    scale 2), blocks 1..63 cold (0.05). For a wave where every row's best cold
    score is more than 3 log2 units (plus a margin) below its block-0 maximum,
    the soft skip must drop every cold block, so the wave's rows are exactly
    dense attention over keys 0..63 -- while full attention differs there (the
    4032 cold keys carry most of the softmax mass). The margin test uses plain
    numpy maxima, independent of the vote code."""
    q, k, v = _peaked_head(0)
    c = float(oa.SCALE_LOG2E)
    nkb = 64
    hot = oa.head_forward(q[:512], k[:64], v[:64], 1)[0]
    checked = 0
    for t in range(2):  # tiles 0 and 1 (rows 0..511)
        qt = q[256 * t: 256 * t + 256]
        s = qt.astype(np.float64) @ k.astype(np.float64).T * c
        out, nxt, blocks = ol.step_tile(qt, k, v, ol.seed_row(nkb), 1, -3.0, 1)
        assert blocks == list(range(nkb))
        for r0 in range(0, 256, 32):
            gap = (s[r0:r0 + 32, 64:].max(axis=1) - s[r0:r0 + 32, :64].max(axis=1)).max()
            if gap < -3.01:
                checked += 1
                assert np.array_equal(out[r0:r0 + 32], hot[256 * t + r0: 256 * t + r0 + 32]), (t, r0)
        # the tile's next list keeps block 0 and (since some wave kept nothing else) is short
        assert ol.kept_count(nxt, nkb) < nkb
    assert checked >= 12
    full = oa.head_forward(q[:64], k, v, 1)[0]
    assert (full != hot[:64]).mean() > 0.5


def test_lpt_bucket_arithmetic_fits_int32_for_any_row():
    """The planning kernel sums |end - start| over at most (nkb + 1) / 2 pairs
    of int16 ids in int32 (< 2^28 for nkb <= 8192), clamps the count to nkb + 1
    and only then multiplies by the 64 buckets (< 2^20): no intermediate can
    overflow, and the clamp does not change the oracle's bucket (counts past
    nkb already land in the top bucket)."""
    for nkb in (2048, 8192):
        row = np.zeros(nkb + 2, np.int16)
        row[0] = nkb + 1
        row[1:] = np.where(np.arange(nkb + 1) % 2 == 0, 32767, -32768)
        kept = ol.kept_count(row, nkb)
        assert kept == (nkb // 2) * 65535 < 2 ** 28
        assert kept * ol.LPT_BUCKETS >= 2 ** 31  # the unclamped product would wrap
        assert (nkb + 1) * ol.LPT_BUCKETS < 2 ** 31
        for k in (nkb, nkb + 1, kept):
            assert min(k * ol.LPT_BUCKETS // (nkb + 1), 63) == min(min(k, nkb + 1) * ol.LPT_BUCKETS // (nkb + 1), 63)
