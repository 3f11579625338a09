"""Shared test helpers: seeded inputs and the bf16 tolerance rule."""
import numpy as np
import torch

from oracle import bf16 as ob

# Tolerance rule for the attention forward (bf16 out, fp32 accumulate), all
# three must hold on every compared tensor:
#  1. |got - ref| <= 1 bf16 ULP of max(|ref|, FLOOR_REL * A), where ref is the
#     oracle's bf16 output under the same round mode and
#     A = sum_j P_j |v_jd| / sum_j p_j is the element's absolute scale.
#     Why a floor: the kernel's fp32 scores and v_exp_f32 differ from the
#     oracle's in the last fp32 bit, which flips the bf16 rounding of a P term
#     now and then (about 4e-4 of terms). One flip moves the element by up to
#     2^-7 * P_j |v_jd| / l -- far below one ULP of A, but unbounded in ULPs of
#     an element that cancels to near zero. FLOOR_REL = 1/4 covers a flip of
#     any term that carries <= 1/8 of the absolute mass.
#  2. >= MIN_EXACT of the elements are bit-identical to the oracle;
#  3. >= MIN_STRICT of the elements are within 1 ULP of |ref| itself (no floor).
# 2 and 3 catch systematic deviations (a wrong P rounding mode, a biased
# rescale) that stay under rule 1.
FLOOR_REL = 0.25
MIN_EXACT = 0.98
MIN_STRICT = 0.995


def randn_bf16(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g, dtype=torch.float32)
    if scale != 1.0:
        x = x * scale
    return x.to(torch.bfloat16)


def bits(t):
    """bf16 tensor (any device) -> numpy uint16 bits."""
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def f32(t):
    return t.detach().cpu().float().numpy()


def to_bhsd(a, layout):
    return a.transpose(0, 2, 1, 3) if layout == "bshd" else a


def compare_bf16(got, ref, scale=None, floor_rel=FLOOR_REL):
    """got/ref: uint16 bit arrays (same shape). Returns stats dict; asserts
    NaN positions/bits, Inf identity and the ULP rule."""
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
        ratio = d / u
        stats["rule_max"] = float(ratio.max()) if d.size else 0.0
        bad = ratio > 1.0
        assert not bad.any(), (
            f"{int(bad.sum())} elements beyond 1 ULP (rule), worst {stats['rule_max']:.2f}; stats={stats}"
        )
    if d.size >= 1000:
        assert stats["exact"] >= MIN_EXACT, f"too few bit-exact elements: {stats}"
        assert stats["strict_le1"] >= MIN_STRICT, f"too many elements beyond strict 1 ULP: {stats}"
    return stats
