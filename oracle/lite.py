"""CPU oracle for LiteAttention -- test infrastructure (see the package docstring).

Restates, for one (b, h, q-tile), the reference's skip-list semantics:

* ``decode``: the K-blocks a read-list row names, in processing order, with the
  last block of each range flagged (reference cursor,
  csrc/attention_kernel.hip:629-668): ranges are taken from the back of the
  row; range (s, e) yields s+d, s+2d, ... while strictly before e+d and at
  least once, d = +1 in phase 1 and -1 in phase 0. Ids outside [0, nkb) are
  dropped (this build's guard; a writer never produces them).
* ``wave_keep`` / ``votes``: the per-wave soft skip and the tile's vote
  (reference softmax :983-1001 and pv_phase :891-898). The tile's q rows are
  taken in wave groups of ``WAVE_ROWS`` (this build's wave owns 32 rows; the
  reference's owns 48). A wave keeps processed block i when i == 0 or when
  some valid row of the wave has fl32(fl32(bm * c) - run) > ``threshold``,
  with bm the row's fp32 max over the block's valid keys and run the row's
  running max of fl32(bm * c) over the blocks THIS WAVE kept before i. A
  block the wave does not keep adds nothing to the wave's rows (no PV, no
  denominator, no max change). The tile's vote for the next list is the OR of
  its waves' keep flags.
* ``forward_tile`` / ``step_tile``: each wave's rows are attention over the
  keys of the blocks that wave kept.
* ``emit``: the next row (reference record(), :685-716): a marker at every
  change of the skip state, which restarts as "skip" after each range end; a
  kept range-end block also writes block + d; ``must_do`` ranges [s, e) force
  "kept".
* ``kept_count`` / ``lpt_order``: the work count of a row (sum of |hi - lo| over
  its pairs, reference plan_lite_order :1314-1326) and the heaviest-first CTA
  order over 64 buckets of kept / (nkb + 1), stable in CTA index.

``seed_row`` is the compute-all row LiteAttention starts from
(reference moonmath_attention/lite.py:141-147).
"""
import numpy as np

from . import attention as _att

KV_BLOCK = 64
Q_TILE = 256
MAX_BLOCKS = 8192
LPT_BUCKETS = 64
WAVE_ROWS = 32


def seed_row(nkb):
    row = np.zeros(nkb + 2, dtype=np.int16)
    row[:3] = (2, nkb - 1, -1)
    return row


def decode(row, nkb, phase):
    d = 1 if phase else -1
    n = int(row[0])
    n = 0 if n < 0 else min(n, nkb + 1)
    blocks, ends = [], []
    for idx in range(n, 1, -2):
        start, stop = int(row[idx]) + d, int(row[idx - 1]) + d
        cnt = max(1, (stop - start) * d)
        seq = [b for b in (start + j * d for j in range(cnt)) if 0 <= b < nkb]
        seq = seq[:MAX_BLOCKS - len(blocks)]
        if seq:
            blocks += seq
            ends += [False] * (len(seq) - 1) + [True]
    return blocks, ends


def block_max_log2(s32, blocks, skv):
    """[len(blocks), rows] fp32 max over each block's valid keys, times c in fp32."""
    c = np.float32(_att.SCALE_LOG2E)
    out = []
    for b in blocks:
        sb = s32[:, b * KV_BLOCK:min(skv, (b + 1) * KV_BLOCK)]
        bm = np.fmax.reduce(sb, axis=1, initial=-np.inf).astype(np.float32)
        with np.errstate(invalid="ignore", over="ignore"):
            out.append((bm.astype(np.float64) * np.float64(c)).astype(np.float32))
    return np.array(out, dtype=np.float32).reshape(len(blocks), s32.shape[0])


def wave_keep(s32_wave, blocks, skv, threshold):
    """Keep flags of one wave over the processed blocks. s32_wave: fp32 scores
    [valid rows of the wave, Skv] (no rows: only the first block is kept)."""
    bms = block_max_log2(s32_wave, blocks, skv)
    run = np.full(s32_wave.shape[0], -np.inf, dtype=np.float32)
    thr = np.float32(threshold)
    keep = []
    with np.errstate(invalid="ignore", over="ignore"):
        for i, bm in enumerate(bms):
            k = i == 0 or bool(((bm - run) > thr).any())
            if k:
                run = np.fmax(run, bm)
            keep.append(k)
    return keep


def wave_groups(nrows):
    """Row ranges [r0, r1) of the tile's waves that hold valid rows."""
    return [(r0, min(nrows, r0 + WAVE_ROWS)) for r0 in range(0, nrows, WAVE_ROWS)]


def wave_keeps(s32_valid, blocks, skv, threshold):
    """[(r0, r1, keep flags)] for every wave with valid rows."""
    return [(r0, r1, wave_keep(s32_valid[r0:r1], blocks, skv, threshold)) for r0, r1 in wave_groups(s32_valid.shape[0])]


def votes(s32_valid, blocks, skv, threshold):
    """The tile's vote: block i stays in the next list when some wave kept it.
    s32_valid: fp32 scores [valid rows of the tile, Skv]."""
    keep = [False] * len(blocks)
    for _, _, kw in wave_keeps(s32_valid, blocks, skv, threshold):
        keep = [a or b for a, b in zip(keep, kw)]
    return keep


def _must_do_ranges(must_do):
    if must_do is None:
        return []
    n = max(0, int(must_do[0]))
    return [(int(must_do[m]), int(must_do[m + 1])) for m in range(1, n, 2) if m + 1 <= n]


def emit(blocks, ends, keep, phase, nkb, must_do=None):
    d = 1 if phase else -1
    md = _must_do_ranges(must_do)
    out = []
    state = True
    for i, b in enumerate(blocks):
        skip = not (keep[i] or any(s <= b < e for s, e in md))
        if skip != state:
            out.append(b)
            state = skip
        if ends[i] or i == len(blocks) - 1:
            state = True
            if not skip:
                out.append(b + d)
    cap = nkb + 1
    n = len(out) if len(out) <= cap else cap & ~1
    return [n] + out[:n]


def kept_count(row, nkb):
    n = int(row[0])
    n = 0 if n < 0 else min(n, nkb + 1)
    return sum(abs(int(row[i]) - int(row[i - 1])) for i in range(n, 1, -2))


def lpt_order(rows, nkb):
    """rows: [nctas, nkb + 2] read-list rows in CTA order (b*H + h, q-tile)."""
    buckets = [min(kept_count(r, nkb) * LPT_BUCKETS // (nkb + 1), LPT_BUCKETS - 1) for r in rows]
    return sorted(range(len(rows)), key=lambda w: -buckets[w])


def scores(q_rows, k_head):
    """fp32 scores as the attention oracle forms them (exact dot, one rounding)."""
    return (q_rows.astype(np.float64) @ k_head.astype(np.float64).T).astype(np.float32)


def forward_tile(q_rows, k_head, v_head, blocks, mode, aux=False):
    """Rows' output over the keys of ``blocks`` (order irrelevant)."""
    skv = k_head.shape[0]
    idx = np.concatenate([np.arange(b * KV_BLOCK, min(skv, (b + 1) * KV_BLOCK)) for b in blocks]) \
        if blocks else np.zeros(0, dtype=np.int64)
    if idx.size == 0:
        z = np.zeros((q_rows.shape[0], 128), dtype=np.uint16)
        return (z, None, np.zeros(z.shape), np.zeros(z.shape)) if aux else z
    res = _att.head_forward(q_rows, k_head[idx], v_head[idx], mode, aux=aux)
    return res if aux else res[0]


def step_tile(q_rows_valid, k_head, v_head, row, phase, threshold, mode, must_do=None, aux=False, s32=None):
    """One lite step of one tile: (output bits, next row, processed blocks).
    The output (and, with ``aux``, pre / scale / tie) stacks the waves' rows,
    each wave over the blocks it kept. ``s32``: the tile's ``scores``, if the
    caller already has them."""
    nkb = -(-k_head.shape[0] // KV_BLOCK)
    blocks, ends = decode(row, nkb, phase)
    if not blocks:
        return forward_tile(q_rows_valid, k_head, v_head, [], mode, aux=aux), emit([], [], [], phase, nkb, must_do), []
    s32 = scores(q_rows_valid, k_head) if s32 is None else s32
    waves = wave_keeps(s32, blocks, k_head.shape[0], threshold)
    keep = [any(kw[i] for _, _, kw in waves) for i in range(len(blocks))]
    nxt = emit(blocks, ends, keep, phase, nkb, must_do)
    parts = [forward_tile(q_rows_valid[r0:r1], k_head, v_head, [b for b, k in zip(blocks, kw) if k], mode, aux=True)
             for r0, r1, kw in waves]
    out = np.concatenate([pt[0] for pt in parts])
    if not aux:
        return out, nxt, blocks
    res = (out, None) + tuple(np.concatenate([pt[j] for pt in parts]) for j in (2, 3))
    return res, nxt, blocks


def wave_blocks(q_rows_valid, k_head, row, phase, threshold, s32=None):
    """The blocks each wave of the tile kept: [(r0, r1, [block ids])]."""
    nkb = -(-k_head.shape[0] // KV_BLOCK)
    blocks, _ = decode(row, nkb, phase)
    if not blocks:
        return [(r0, r1, []) for r0, r1 in wave_groups(q_rows_valid.shape[0])]
    s32 = scores(q_rows_valid, k_head) if s32 is None else s32
    waves = wave_keeps(s32, blocks, k_head.shape[0], threshold)
    return [(r0, r1, [b for b, k in zip(blocks, kw) if k]) for r0, r1, kw in waves]
