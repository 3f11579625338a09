"""Shared test helpers: seeded inputs and the bf16 tolerance rule."""
import json
import os

import numpy as np
import torch

from oracle import bf16 as ob

# Tolerance rule for the attention forward (bf16 out, fp32 accumulate), all
# three must hold on every compared tensor:
#  1. |got - ref| <= ulp_bf16(max(|ref|, FLOOR_REL * A)) + T, where ref is the
#     oracle's bf16 output under the same round mode,
#     A = sum_j P_j |v_jd| / sum_j p_j is the element's absolute scale and T
#     the oracle's near-tie allowance (sum over terms whose fp32 p_j lies
#     within the GPU's fp32 error of a bf16 rounding boundary of
#     ulp_bf16(P_j) |v_jd| / sum_j p_j).
#     Why a floor: the kernel's fp32 scores and v_exp_f32 differ from the
#     oracle's in the last fp32 bit, which flips the bf16 rounding of a P term
#     now and then (about 4e-4 of terms). One flip moves the element by up to
#     2^-7 * P_j |v_jd| / l -- far below one ULP of A, but unbounded in ULPs of
#     an element that cancels to near zero. FLOOR_REL = 1/4 covers a flip of
#     any term that carries <= 1/8 of the absolute mass; T covers a flip of a
#     term that carries more (peaked attention: growing keys, spikes, the
#     reference benchmark's log-normal key norms), which moves the element by
#     up to 1 ULP before the output rounding.
#  2. >= MIN_EXACT of the elements are bit-identical to the oracle;
#  3. >= MIN_STRICT of the elements are within 1 ULP of |ref| itself (no floor).
# 2 and 3 catch systematic deviations (a wrong P rounding mode, a biased
# rescale) that stay under rule 1.
FLOOR_REL = 0.25
MIN_EXACT = 0.99
MIN_STRICT = 0.999


def randn_bf16(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g, dtype=torch.float32)
    if scale != 1.0:
        x = x * scale
    return x.to(torch.bfloat16)


def realistic_bf16(B, S, H, seed, D=128, sigma=0.6):
    """The reference benchmark's "realistic" pattern (reference
    benchmark/runner.py:34-47), BSHD: Q, V ~ N(0, 1); K = uniform direction with
    magnitude exp(N(0, sigma)) * sqrt(D) (log-normal row norms). Drawn on the
    CPU from a seeded generator (the reference draws on the GPU from seed 42)."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, S, H, D, generator=g)
    k_dir = torch.randn(B, S, H, D, generator=g)
    k_dir = k_dir / k_dir.norm(dim=-1, keepdim=True)
    log_norm = torch.randn(B, S, H, 1, generator=g) * sigma
    k = k_dir * (torch.exp(log_norm) * D ** 0.5)
    v = torch.randn(B, S, H, D, generator=g)
    return q.to(torch.bfloat16), k.to(torch.bfloat16), v.to(torch.bfloat16)


def growth_log2(q_head, k_head, block=64):
    """Per row: integer-grid max over all keys minus the one over the first
    block (log2 units) -- how far a row's max grows past its first block."""
    from oracle import attention as oa

    s_all = (q_head.astype(np.float64) @ k_head.astype(np.float64).T).astype(np.float32)
    return oa.row_max_int(s_all) - oa.row_max_int(s_all[:, :block])


def log_stats(name, stats):
    """Append one parity record to $MOONMATH_PARITY_LOG (a JSON-lines file);
    name None = the running pytest case."""
    path = os.environ.get("MOONMATH_PARITY_LOG")
    if path:
        if name is None:
            name = os.environ.get("PYTEST_CURRENT_TEST", "?").split(" ")[0].split("::")[-1]
        with open(path, "a") as f:
            f.write(json.dumps({"case": name, **stats}) + "\n")


def bits(t):
    """bf16 tensor (any device) -> numpy uint16 bits."""
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def f32(t):
    return t.detach().cpu().float().numpy()


def to_bhsd(a, layout):
    return a.transpose(0, 2, 1, 3) if layout == "bshd" else a


def check_fractions(stats, min_exact=MIN_EXACT, min_strict=MIN_STRICT):
    """Rules 2 and 3 on a stats dict (statistical: applied to >= 1000 elements,
    over all the tensors of one case when they are compared piecewise)."""
    if stats["n"] >= 1000:
        assert stats["exact"] >= min_exact, f"too few bit-exact elements: {stats}"
        assert stats["strict_le1"] >= min_strict, f"too many elements beyond strict 1 ULP: {stats}"


def aggregate_stats(stats, names=None):
    """Element-weighted totals of several compare_bf16 stats dicts (one per
    head, request or tile), plus the worst unit's fractions and the names
    (or indices) of the units of >= 1000 elements below the per-case bars
    (exact 0.99, strict 0.999), so a unit that only passes in aggregate is
    named in the parity log."""
    n = sum(s["n"] for s in stats)
    names = [str(i) for i in range(len(stats))] if names is None else [str(x) for x in names]
    big = [(nm, s) for nm, s in zip(names, stats) if s["n"] >= 1000]
    agg = {
        "n": n,
        "exact": sum(s["exact"] * s["n"] for s in stats) / max(n, 1),
        "strict_le1": sum(s["strict_le1"] * s["n"] for s in stats) / max(n, 1),
        "strict_max": max(s["strict_max"] for s in stats),
        "units": len(stats),
        "unit_min_exact": min((s["exact"] for _, s in big), default=1.0),
        "unit_min_strict": min((s["strict_le1"] for _, s in big), default=1.0),
        "units_below": [nm for nm, s in big if s["exact"] < MIN_EXACT or s["strict_le1"] < MIN_STRICT],
    }
    if all("rule_max" in s for s in stats):
        agg["rule_max"] = max(s["rule_max"] for s in stats)
    if all("n_tie" in s for s in stats):
        agg["n_tie"] = sum(s["n_tie"] for s in stats)
    return agg


def compare_bf16(got, ref, scale=None, tie=None, floor_rel=FLOOR_REL, min_exact=MIN_EXACT,
                 min_strict=MIN_STRICT, fractions=True):
    """got/ref: uint16 bit arrays (same shape); scale = A, tie = T from the
    oracle. Returns stats dict; asserts NaN positions/bits, Inf identity and
    the ULP rule, and (``fractions``) rules 2 and 3."""
    g = ob.bf16_to_f32(got).astype(np.float64)
    r = ob.bf16_to_f32(ref).astype(np.float64)
    gn, rn = np.isnan(g), np.isnan(r)
    assert np.array_equal(gn, rn), f"NaN positions differ: {int((gn != rn).sum())} elements"
    assert np.all(got[gn] == 0x7FFF), "non-canonical NaN in output"
    gi, ri = np.isinf(g), np.isinf(r)
    assert np.array_equal(gi, ri) and np.array_equal(g[gi], r[ri]), "Inf mismatch"
    fin = ~(gn | gi)
    d = np.abs(g[fin] - r[fin])
    strict_u = ob.ulp_bf16(np.abs(r[fin]))
    strict = d / strict_u
    stats = {
        "n": int(fin.sum()),
        "exact": float((d == 0).mean()) if d.size else 1.0,
        "strict_le1": float((strict <= 1).mean()) if d.size else 1.0,
        "strict_max": float(strict.max()) if d.size else 0.0,
    }
    if scale is not None:
        mag = np.maximum(np.abs(r[fin]), floor_rel * scale[fin])
        u = ob.ulp_bf16(mag)
        if tie is not None:
            stats["n_tie"] = int((d > u).sum())  # elements within the rule only through T
            u = u + tie[fin]
        ratio = d / u
        stats["rule_max"] = float(ratio.max()) if d.size else 0.0
        bad = ratio > 1.0
        assert not bad.any(), (
            f"{int(bad.sum())} elements beyond 1 ULP (rule), worst {stats['rule_max']:.2f}; stats={stats}"
        )
    if fractions:
        check_fractions(stats, min_exact, min_strict)
    return stats


def reference_pattern(name, B, S, H, D=128):
    """The reference benchmark's synthetic patterns (benchmark/runner.py:48-75),
    BSHD bf16, the same in every (b, h): "ones" (all ones), "linear" (q = s/S +
    0.1 d/D, k = s/S, v = s/S + d/D) and "diag" (q = k = one-hot rows of the
    identity repeated along S, v = s/S in every dim)."""
    s_idx = (torch.arange(S, dtype=torch.float32) / S).view(S, 1)
    d_idx = (torch.arange(D, dtype=torch.float32) / D).view(1, D)
    if name == "ones":
        q = k = v = torch.ones(S, D)
    elif name == "linear":
        q, k, v = s_idx + 0.1 * d_idx, s_idx.expand(S, D), s_idx + d_idx
    elif name == "diag":
        q = k = torch.eye(D).repeat(S // D + 1, 1)[:S]
        v = s_idx.expand(S, D)
    else:
        raise ValueError(name)
    return tuple(t.to(torch.bfloat16).reshape(1, S, 1, D).expand(B, S, H, D).contiguous() for t in (q, k, v))


def ones_closed_form(mode):
    """Every score is 128, so every p is the same p1 = exp2(fl32(128 c) - 17)
    (m = ceil(fl32(128 c)) = 17) and every output element is
    mode(S bf16(p1) / (S p1)) = mode(bf16(p1) / p1): the mean of V (1) scaled
    by the reference's numerics (bf16 P in the numerator, fp32 p in the
    denominator, attention_kernel.hip:438-451). The quotient is kept away from
    a bf16 rounding boundary (asserted), so fp32 sums of S equal terms cannot
    change its rounding."""
    from oracle import attention as oa
    from oracle import bf16 as ob

    c = np.float32(oa.SCALE_LOG2E)
    x = np.float32(np.float64(128.0) * np.float64(c) - 17.0)
    assert np.ceil(np.float32(128.0) * c) == 17
    p1 = np.float32(np.exp2(np.float64(x)))
    mc = ob.MODES[mode]
    P1 = ob.round_f32(np.array([p1], np.float32), mc)[0]
    ratio = np.float64(P1) / np.float64(p1)
    lo = ob.bf16_to_f32(ob.round_bits(np.array([ratio], np.float32), ob.RTZ))[0]
    ulp = float(ob.ulp_bf16(np.array([ratio]))[0])
    frac = (ratio - lo) / ulp
    assert 0.05 < frac < 0.45 or 0.55 < frac < 0.95, frac
    return int(ob.round_bits(np.array([ratio], np.float32), mc, canon=True)[0])
