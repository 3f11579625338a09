"""CPU oracle for the bf16 attention forward (numpy, float64 arithmetic).

Computes ``O = softmax(Q K^T / sqrt(128)) V`` with the precision model of the
reference kernel (moonmath reference csrc/attention_kernel.hip):

* scores ``s`` are fp32 dot products of bf16 inputs (MFMA, :837-862); here the
  exact fp64 dot product rounded once to fp32;
* base-2 softmax: ``x = fma(s, log2e/sqrt(128), -m)`` rounded to fp32 and
  ``p = exp2(x)`` rounded to fp32 (:441-444);
* P is rounded to bf16 with the *output* round mode before the PV product
  (:448, ``pack4_bf16`` with the build's ``BF16_ROUND``); the denominator sums
  the unrounded fp32 ``p`` (:445-451);
* ``out = mode(num * (l == 0 ? 0 : 1/l))`` with every NaN -> 0x7FFF (:1114-1127);
* kv rows past Skv contribute nothing (:954-965).

Running-max policy (documented divergence, chosen for blocking invariance):
the max is kept on the integer grid, ``m = ceil(fl32(max_j s_j * c))`` with a
floor of -FLT_MAX and NaN ignored (``fmaxf``). Rescales are then exact powers
of two, so bf16(P) relative to any running max equals bf16(P) relative to the
final max scaled by a power of two: the result does not depend on the kernel's
KV blocking or split factor. The reference keeps the exact max (:398-436),
which makes P's rounding depend on its 64-row blocking.

Also returns, on request (``aux``), for the tests' tolerance rule:

* the fp64 pre-rounding value;
* the per-element absolute scale ``A = sum_j P_j |v_jd| / sum_j p_j``;
* the near-tie allowance ``T = sum_j u_j |v_jd| / sum_j p_j``, where
  ``u_j = ulp_bf16(P_j)`` for every term whose fp32 ``p_j`` lies within the
  fp32 error of a GPU evaluation (scores accumulated in fp32 by the MFMA, the
  exp2 argument formed under another integer max, hardware exp2) of a bf16
  rounding boundary, and 0 otherwise. Such a term may be rounded to either
  bf16 neighbour by any fp32 implementation; ``T`` bounds what those choices
  can move the output. It matters when a few terms carry most of a row's
  weight (peaked attention), where one such choice moves the output by up to
  one bf16 ULP before the output rounding.
"""
import math

import numpy as np

from . import bf16 as _b

LOG2E = 1.4426950408889634
SCALE_LOG2E = np.float32(LOG2E / math.sqrt(128.0))  # host value the kernel also uses
FLT_MAX = np.float32(3.4028234663852886e38)
D = 128


def _to_bhsd(x, layout):
    x = np.asarray(x, dtype=np.float32)
    if layout == "bshd":
        return x.transpose(0, 2, 1, 3)
    if layout == "bhsd":
        return x
    raise ValueError(layout)


def row_max_int(s32):
    """Integer-grid running max of fp32 scores per row: ceil(fl32(max(s) * c)),
    NaN ignored, floored at -FLT_MAX (the kernel's initial running max)."""
    bm = np.fmax.reduce(s32, axis=-1, initial=-np.inf).astype(np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        mb = np.ceil((bm * SCALE_LOG2E).astype(np.float32))
    return np.fmax(mb, -FLT_MAX).astype(np.float32)


def exp2_arg(s32, m):
    """x = fl32(s * c - m) (one rounding, as fma(s, c, -m)), m broadcast per row."""
    with np.errstate(invalid="ignore", over="ignore"):
        return (s32.astype(np.float64) * np.float64(SCALE_LOG2E) - m.astype(np.float64)[..., None]).astype(np.float32)


def softmax_p(s32, m):
    """p = fl32(exp2(fl32(s * c - m))) elementwise (m broadcast per row)."""
    with np.errstate(invalid="ignore", over="ignore"):
        return np.exp2(exp2_arg(s32, m).astype(np.float64)).astype(np.float32)


# Bound on the GPU's exp2 argument beyond the oracle's: the kernel may form
# x = s*c - m under an integer max up to this far below the final one (its
# p <= 2^20 growth limit), which coarsens x's fp32 rounding.
_X_SLACK = 21.0


def tie_terms(s32, x32, p, p_mode):
    """ulp_bf16(P_j) for terms whose p_j is within the GPU's fp32 error of a
    bf16 rounding boundary of ``p_mode`` (0 elsewhere). The error budget, kept
    2x generous: 2 fp32 ulps of the score s times c, one fp32 ulp of
    |x| + _X_SLACK (the argument's rounding), and 2^-22 relative for exp2."""
    with np.errstate(invalid="ignore", over="ignore"):
        dx = (2.0 * float(SCALE_LOG2E)) * np.spacing(np.abs(s32)).astype(np.float64)
        dx += np.spacing((np.abs(x32) + np.float32(_X_SLACK)).astype(np.float32)).astype(np.float64)
        eps = 2.0 * (math.log(2.0) * dx + 2.0 ** -22) * p.astype(np.float64)
        lo_bits = p.view(np.uint32) & np.uint32(0xFFFF0000)
        lo = lo_bits.view(np.float32).astype(np.float64)
        hi = (lo_bits + np.uint32(0x10000)).view(np.float32).astype(np.float64)
        p64 = p.astype(np.float64)
        if p_mode == _b.RTZ:
            dist = np.minimum(p64 - lo, hi - p64)
        else:
            dist = np.abs(p64 - 0.5 * (lo + hi))
        return np.where(dist <= eps, hi - lo, 0.0)


def head_forward(Q, K, V, mode, p_round=True, aux=False, chunk=None, p_mode=None):
    """One head: Q [Sq,128], K/V [Skv,128] float32 (bf16-valued).

    ``p_mode`` overrides the rounding of P (tests use it to plant a mistake).
    """
    p_mode = mode if p_mode is None else p_mode
    Sq, Skv = Q.shape[0], K.shape[0]
    K64 = K.astype(np.float64)
    V64 = V.astype(np.float64)
    absV = np.abs(V64)
    out = np.empty((Sq, D), dtype=np.uint16)
    pre = np.empty((Sq, D), dtype=np.float64) if aux else None
    scl = np.empty((Sq, D), dtype=np.float64) if aux else None
    tie = np.empty((Sq, D), dtype=np.float64) if aux else None
    if chunk is None:
        chunk = max(1, min(Sq, (1 << 25) // max(Skv, 1)))
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        for r0 in range(0, Sq, chunk):
            r1 = min(Sq, r0 + chunk)
            s32 = (Q[r0:r1].astype(np.float64) @ K64.T).astype(np.float32)
            m = row_max_int(s32)
            x32 = exp2_arg(s32, m)
            p = np.exp2(x32.astype(np.float64)).astype(np.float32)
            P = _b.round_f32(p, p_mode) if p_round else p
            P64 = P.astype(np.float64)
            num = P64 @ V64
            den = p.astype(np.float64).sum(axis=1)
            inv = np.where(den == 0.0, 0.0, 1.0 / np.where(den == 0.0, 1.0, den))
            val = num * inv[:, None]
            out[r0:r1] = _b.round_bits(val.astype(np.float32), mode, canon=True)
            if aux:
                pre[r0:r1] = val
                scl[r0:r1] = (P64 @ absV) * inv[:, None]
                tie[r0:r1] = (tie_terms(s32, x32, p, p_mode) @ absV) * inv[:, None]
    return (out, pre, scl, tie) if aux else (out, None, None)


def forward(q, k, v, mode, layout="bhsd", heads=None, p_round=True, aux=False, p_mode=None):
    """Full forward. q/k/v float32 arrays of bf16 values in ``layout``.

    ``heads``: optional list of (b, h) to compute (others left 0 / NaN scale).
    Returns uint16 bits in BHSD order [B,H,Sq,128] (and pre / scale / tie if aux).
    """
    if isinstance(mode, str):
        mode = _b.MODES[mode]
    if isinstance(p_mode, str):
        p_mode = _b.MODES[p_mode]
    qh, kh, vh = _to_bhsd(q, layout), _to_bhsd(k, layout), _to_bhsd(v, layout)
    B, H, Sq, _ = qh.shape
    out = np.zeros((B, H, Sq, D), dtype=np.uint16)
    pre = np.full((B, H, Sq, D), np.nan) if aux else None
    scl = np.full((B, H, Sq, D), np.nan) if aux else None
    tie = np.full((B, H, Sq, D), np.nan) if aux else None
    todo = heads if heads is not None else [(b, h) for b in range(B) for h in range(H)]
    for b, h in todo:
        res = head_forward(qh[b, h], kh[b, h], vh[b, h], mode, p_round=p_round, aux=aux, p_mode=p_mode)
        out[b, h] = res[0]
        if aux:
            pre[b, h], scl[b, h], tie[b, h] = res[1], res[2], res[3]
    return (out, pre, scl, tie) if aux else out


def forward_rows(q, k, v, mode, layout, heads, rows, aux=False):
    """Selected query rows of selected heads against ALL keys: rows are
    independent in the forward, so this equals ``forward(...)[b, h, rows]``
    without the cost of the other rows (used for the long configs).

    Returns uint16 bits [len(heads), len(rows), 128] (and pre / scale / tie if aux).
    """
    if isinstance(mode, str):
        mode = _b.MODES[mode]
    qh, kh, vh = _to_bhsd(q, layout), _to_bhsd(k, layout), _to_bhsd(v, layout)
    rows = np.asarray(rows)
    out = np.zeros((len(heads), len(rows), D), dtype=np.uint16)
    pre = np.zeros(out.shape) if aux else None
    scl = np.zeros(out.shape) if aux else None
    tie = np.zeros(out.shape) if aux else None
    for i, (b, h) in enumerate(heads):
        res = head_forward(qh[b, h][rows], kh[b, h], vh[b, h], mode, aux=aux)
        out[i] = res[0]
        if aux:
            pre[i], scl[i], tie[i] = res[1], res[2], res[3]
    return (out, pre, scl, tie) if aux else out


def nan_rows(q_head, k_head):
    """Rows of one head whose output is NaN under the integer-grid max policy:
    row i is NaN iff some score s_ij is NaN or +inf (a NaN p enters both sums;
    a +inf score makes m = +inf and its own p = exp2(inf - inf) = NaN). Scores
    of keys with no non-finite element are finite and cannot do either, so only
    those keys are evaluated. q_head [Sq,128], k_head [Skv,128] float32."""
    bad = ~np.isfinite(k_head).all(axis=1)
    if not bad.any():
        return np.zeros(q_head.shape[0], dtype=bool)
    if np.isnan(k_head[bad]).any():
        return np.ones(q_head.shape[0], dtype=bool)
    with np.errstate(invalid="ignore", over="ignore"):
        s = q_head.astype(np.float64) @ k_head[bad].astype(np.float64).T
    return (np.isnan(s) | (s == np.inf)).any(axis=1)


def head_forward_blocked(Q, K, V, mode, kv_block=64, split_ways=1):
    """Kernel-shaped restatement for pinning blocking invariance: KV walked in
    ``kv_block`` rows inside ``split_ways`` contiguous parts, integer running max
    updated per block with exact power-of-two rescales, parts merged with
    weights 2^(m_p - M) (reference merge :1239-1279). fp64 accumulation."""
    Sq, Skv = Q.shape[0], K.shape[0]
    nkb = -(-Skv // kv_block)
    parts = []
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        for j in range(split_ways):
            kb0, kb1 = nkb * j // split_ways, nkb * (j + 1) // split_ways
            m = np.full(Sq, -FLT_MAX, dtype=np.float32)
            o = np.zeros((Sq, D))
            l = np.zeros(Sq)
            for kb in range(kb0, kb1):
                r0, r1 = kb * kv_block, min(Skv, (kb + 1) * kv_block)
                s32 = (Q.astype(np.float64) @ K[r0:r1].astype(np.float64).T).astype(np.float32)
                m_new = np.fmax(m, row_max_int(s32))
                grew = m_new > m
                sc = np.where(grew, np.exp2(np.where(grew, m - m_new, 0.0).astype(np.float64)), 1.0)
                o *= sc[:, None]
                l *= sc
                m = m_new
                p = softmax_p(s32, m)
                o += _b.round_f32(p, mode).astype(np.float64) @ V[r0:r1].astype(np.float64)
                l += p.astype(np.float64).sum(axis=1)
            parts.append((m, o, l))
        M = np.fmax.reduce(np.stack([pm for pm, _, _ in parts]), axis=0)
        num = np.zeros((Sq, D))
        den = np.zeros(Sq)
        for pm, po, pl in parts:
            w = np.where(pm == M, 1.0, np.exp2((pm.astype(np.float64) - M)))
            num += w[:, None] * po
            den += w * pl
        inv = np.where(den == 0.0, 0.0, 1.0 / np.where(den == 0.0, 1.0, den))
        return _b.round_bits((num * inv[:, None]).astype(np.float32), mode, canon=True)


def torch_formula_cpu(q, k, v):
    """The reference repo's own CPU oracle formula (examples/basic.py:16-17):
    softmax(q.float() @ k.float().T / sqrt(D)) @ v.float(), torch fp32, BHSD."""
    import torch

    qf, kf, vf = q.float(), k.float(), v.float()
    return torch.softmax(qf @ kf.transpose(-1, -2) / (qf.shape[-1] ** 0.5), dim=-1) @ vf
