"""CPU oracle for LiteAttention -- test infrastructure (see the package docstring).

Restates, for one (b, h, q-tile), the reference's skip-list semantics:

* ``decode``: the K-blocks a read-list row names, in processing order, with the
  last block of each range flagged (reference cursor,
  csrc/attention_kernel.hip:629-668): ranges are taken from the back of the
  row; range (s, e) yields s+d, s+2d, ... while strictly before e+d and at
  least once, d = +1 in phase 1 and -1 in phase 0. Ids outside [0, nkb) are
  dropped (this build's guard; a writer never produces them).
* ``votes``: keep flags (reference softmax :983-995): block i is kept when some
  valid row's fp32 block max times c, minus the row's running max of the same
  over the blocks before it, exceeds ``threshold``; the first block always.
* ``emit``: the next row (reference record(), :685-716): a marker at every
  change of the skip state, which restarts as "skip" after each range end; a
  kept range-end block also writes block + d; ``must_do`` ranges [s, e) force
  "kept".
* ``kept_count`` / ``lpt_order``: the work count of a row (sum of |hi - lo| over
  its pairs, reference plan_lite_order :1314-1326) and the heaviest-first CTA
  order over 64 buckets of kept / (nkb + 1), stable in CTA index.
* ``forward_tile``: the tile's output = the attention oracle over the keys of
  the processed blocks.

``seed_row`` is the compute-all row LiteAttention starts from
(reference moonmath_attention/lite.py:141-147).
"""
import numpy as np

from . import attention as _att

KV_BLOCK = 64
Q_TILE = 256
MAX_BLOCKS = 8192
LPT_BUCKETS = 64


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


def votes(s32_valid, blocks, skv, threshold):
    """s32_valid: fp32 scores [valid rows of the tile, Skv]."""
    bms = block_max_log2(s32_valid, blocks, skv)
    run = np.full(s32_valid.shape[0], -np.inf, dtype=np.float32)
    thr = np.float32(threshold)
    keep = []
    with np.errstate(invalid="ignore", over="ignore"):
        for i, bm in enumerate(bms):
            k = bool(((bm - run) > thr).any())
            run = np.fmax(run, bm)
            keep.append(i == 0 or k)
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
    """The tile's output over the keys of ``blocks`` (order irrelevant)."""
    skv = k_head.shape[0]
    idx = np.concatenate([np.arange(b * KV_BLOCK, min(skv, (b + 1) * KV_BLOCK)) for b in blocks]) \
        if blocks else np.zeros(0, dtype=np.int64)
    if idx.size == 0:
        z = np.zeros((q_rows.shape[0], 128), dtype=np.uint16)
        return (z, None, np.zeros(z.shape), np.zeros(z.shape)) if aux else z
    res = _att.head_forward(q_rows, k_head[idx], v_head[idx], mode, aux=aux)
    return res if aux else res[0]


def step_tile(q_rows_valid, k_head, v_head, row, phase, threshold, mode, must_do=None, aux=False):
    """One lite step of one tile: (output bits, next row, processed blocks)."""
    nkb = -(-k_head.shape[0] // KV_BLOCK)
    blocks, ends = decode(row, nkb, phase)
    keep = votes(scores(q_rows_valid, k_head), blocks, k_head.shape[0], threshold) if blocks else []
    nxt = emit(blocks, ends, keep, phase, nkb, must_do)
    return forward_tile(q_rows_valid, k_head, v_head, blocks, mode, aux=aux), nxt, blocks
