"""Tail KV-split planner, restated from reference
csrc/attention_kernel.hip:1349-1393 (mirror: tools/tail_speedup.py:33-73) with
the CU count re-derived for MI355X.

``slots`` = CUs x CTAs resident per CU (256 x 1 for this build's 256-row CTAs).
No split when the grid tiles the slots evenly, when the last round is > 95%
full, or when there are fewer than ``min_kv_blocks`` kv blocks (the reference
uses 48; this build 16, measured on MI355X). Otherwise G minimises
ceil(tail*G/slots) * ceil(nkb/G) + 3 over G <= max_parts/tail with
nkb/G >= 4.
"""

REFERENCE_MIN_KV_BLOCKS = 48
MIN_KV_BLOCKS = 16
MIN_BLOCKS_PER_PART = 4
MERGE_COST = 3


def plan_tail(nqb, nbh, nkb, slots, max_parts, enable=True, min_kv_blocks=MIN_KV_BLOCKS):
    """Returns (prefix_wgs, tail, G, parts)."""
    wgs = nqb * nbh
    none = (wgs, 0, 1, 0)
    if not enable:
        return none
    tail = wgs % slots
    if tail == 0 or tail > slots * 19 // 20 or nkb < min_kv_blocks:
        return none
    best_g, best = 1, nkb + MERGE_COST
    g = 2
    while g <= max_parts // tail and nkb // g >= MIN_BLOCKS_PER_PART:
        span = -(-tail * g // slots) * -(-nkb // g) + MERGE_COST
        if span < best:
            best, best_g = span, g
        g += 1
    if best_g == 1:
        return none
    return (wgs - tail, tail, best_g, tail * best_g)
