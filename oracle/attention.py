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

Also returns, on request, the fp64 pre-rounding value and the per-element
absolute scale ``A = sum_j P_j |v_jd| / sum_j p_j`` used by the tests'
tolerance rule.
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


def softmax_p(s32, m):
    """p = fl32(exp2(fl32(s * c - m))) elementwise (m broadcast per row)."""
    with np.errstate(invalid="ignore", over="ignore"):
        x = (s32.astype(np.float64) * np.float64(SCALE_LOG2E) - m.astype(np.float64)[..., None]).astype(np.float32)
        return np.exp2(x.astype(np.float64)).astype(np.float32)


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
    if chunk is None:
        chunk = max(1, min(Sq, (1 << 25) // max(Skv, 1)))
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        for r0 in range(0, Sq, chunk):
            r1 = min(Sq, r0 + chunk)
            s32 = (Q[r0:r1].astype(np.float64) @ K64.T).astype(np.float32)
            m = row_max_int(s32)
            p = softmax_p(s32, m)
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
    return out, pre, scl


def forward(q, k, v, mode, layout="bhsd", heads=None, p_round=True, aux=False, p_mode=None):
    """Full forward. q/k/v float32 arrays of bf16 values in ``layout``.

    ``heads``: optional list of (b, h) to compute (others left 0 / NaN scale).
    Returns uint16 bits in BHSD order [B,H,Sq,128] (and pre / scale if aux).
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
    todo = heads if heads is not None else [(b, h) for b in range(B) for h in range(H)]
    for b, h in todo:
        o, pr, sc = head_forward(qh[b, h], kh[b, h], vh[b, h], mode, p_round=p_round, aux=aux, p_mode=p_mode)
        out[b, h] = o
        if aux:
            pre[b, h] = pr
            scl[b, h] = sc
    return (out, pre, scl) if aux else out


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
