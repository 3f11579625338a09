"""Tail KV-split planners (test infrastructure: the CPU restatement the host
planner is checked against).

``plan_tail_reference`` restates the reference's planner, csrc/attention_kernel.hip
:1349-1393 (mirror: tools/tail_speedup.py:33-73): no split when the grid tiles
the slots evenly, when the last round is > 95% full, or below 48 kv blocks;
otherwise G minimises ceil(tail*G/slots) * ceil(nkb/G) + 3 over
G <= max_parts/tail with nkb/G >= 4, against nkb + 3 unsplit.

``plan_tail`` is this build's re-derivation for MI355X (``slots`` = 256 CUs x
1 CTA of 256 rows): the same search and limits, from 16 kv blocks, with the
cost of a CTA's prologue and epilogue (4 blocks) per round and of the parts'
fp32 records (one block per 64 parts):
unsplit nkb + 4; G parts rounds * (ceil(nkb/G) + 4) + 3 + ceil(tail*G/64).
"""

REFERENCE_MIN_KV_BLOCKS = 48
MIN_KV_BLOCKS = 16
MIN_BLOCKS_PER_PART = 4
MERGE_COST = 3
CTA_COST = 4
PARTS_PER_RECORD_BLOCK = 64


def _ceil(a, b):
    return -(-a // b)


def plan_tail_reference(nqb, nbh, nkb, slots, max_parts, enable=True):
    """The reference's planner. Returns (prefix_wgs, tail, G, parts)."""
    wgs = nqb * nbh
    none = (wgs, 0, 1, 0)
    if not enable:
        return none
    tail = wgs % slots
    if tail == 0 or tail > slots * 19 // 20 or nkb < REFERENCE_MIN_KV_BLOCKS:
        return none
    best_g, best = 1, nkb + MERGE_COST
    g = 2
    while g <= max_parts // tail and nkb // g >= MIN_BLOCKS_PER_PART:
        span = _ceil(tail * g, slots) * _ceil(nkb, g) + MERGE_COST
        if span < best:
            best, best_g = span, g
        g += 1
    if best_g == 1:
        return none
    return (wgs - tail, tail, best_g, tail * best_g)


def plan_tail(nqb, nbh, nkb, slots, max_parts, enable=True):
    """This build's planner. Returns (prefix_wgs, tail, G, parts)."""
    wgs = nqb * nbh
    none = (wgs, 0, 1, 0)
    if not enable:
        return none
    tail = wgs % slots
    if tail == 0 or tail > slots * 19 // 20 or nkb < MIN_KV_BLOCKS:
        return none
    best_g, best = 1, nkb + CTA_COST
    g = 2
    while g <= max_parts // tail and nkb // g >= MIN_BLOCKS_PER_PART:
        span = (_ceil(tail * g, slots) * (_ceil(nkb, g) + CTA_COST) + MERGE_COST
                + _ceil(tail * g, PARTS_PER_RECORD_BLOCK))
        if span < best:
            best, best_g = span, g
        g += 1
    if best_g == 1:
        return none
    return (wgs - tail, tail, best_g, tail * best_g)
