"""CPU oracle for the fp8-KV absorbed-MLA decode (numpy, float64 arithmetic).

Semantics (moonmath reference csrc/mla_decode_a16w8.hip:1-24, :213-217 and
tests/test_mla_decode.py:50-66): for request b, draft position t of q_len and
head h,

    score[j] = (q_lat . c[j, :512] + q_pe . c[j, 512:]) * scale * kv_scale
    o_lat    = sum_j softmax(score)[j] * c[j, :512] * kv_scale,

over tokens j in [0, S_b - (q_len - 1 - t)) (end-aligned causal window), with
c the OCP e4m3fn decode of the 576-byte fused row.

Precision model (the kernel's; the reference folds kv_scale the same way,
mla_decode_a16w8.hip:278 and :600):
* s = fp32 of the exact dot product of bf16 q with the decoded c;
* x = fl32(s * C - m), C = fl32(scale * kv_scale * log2 e); p = fl32(2^x);
* m on the integer grid: ceil(fl32(max_j s_j * C)), NaN ignored, floor -FLT_MAX;
* P = bf16 RTNE of p (reference :146-155); numerator sum P * c (exact here),
  denominator sum of fp32 p;
* out = bf16 RTNE(fl32(num * kv_scale / den)), 0 when den == 0, NaN -> 0x7FFF.

``fp32_reference`` is the reference test's plain fp32 formula
(tests/test_mla_decode.py:50-66) for the rel-L2 floor check.
"""
import math

import numpy as np

from . import bf16 as _b
from . import fp8 as _f8

LAT, ROPE, QK = 512, 64, 576
LOG2E = 1.4426950408889634
FLT_MAX = np.float32(3.4028234663852886e38)


def score_c(scale, kv_scale):
    return np.float32(float(scale) * float(kv_scale) * LOG2E)


def request_rows(kv_u8, seq_lens, b, kv_indices=None, kv_indptr=None):
    """Decoded fp8 rows [S_b, 576] (float64) of request b, contiguous or paged."""
    S = int(seq_lens[b])
    if kv_indices is None:
        rows = kv_u8[b, :S]
    else:
        start = int(kv_indptr[b])
        rows = kv_u8.reshape(-1, QK)[np.asarray(kv_indices[start:start + S], dtype=np.int64)]
    return _f8.decode(rows)


def decode_one(q_lat, q_pe, c, scale, kv_scale, aux=False):
    """One query row set: q_lat [R,512], q_pe [R,64] float32 (bf16-valued),
    c [S,576] float64 decoded KV, per-row token limits handled by the caller.
    Returns bits [R,512] (and pre, A if aux)."""
    C = score_c(scale, kv_scale)
    q = np.concatenate([q_lat, q_pe], axis=1).astype(np.float64)
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        s32 = (q @ c.T).astype(np.float32)
        bm = np.fmax.reduce(s32, axis=1, initial=-np.inf).astype(np.float32)
        m = np.fmax(np.ceil((bm * C).astype(np.float32)), -FLT_MAX).astype(np.float32)
        x = (s32.astype(np.float64) * np.float64(C) - m.astype(np.float64)[:, None]).astype(np.float32)
        p = np.exp2(x.astype(np.float64)).astype(np.float32)
        P = _b.round_f32(p, _b.RTNE).astype(np.float64)
        lat = c[:, :LAT]
        num = P @ lat
        den = p.astype(np.float64).sum(axis=1)
        inv = np.where(den == 0.0, 0.0, float(kv_scale) / np.where(den == 0.0, 1.0, den))
        val = num * inv[:, None]
        bits = _b.round_bits(val.astype(np.float32), _b.RTNE, canon=True)
        if not aux:
            return bits
        A = (P @ np.abs(lat)) * inv[:, None]
        return bits, val, A


def decode(q_lat, q_pe, kv_u8, seq_lens, scale, kv_scale, kv_indices=None, kv_indptr=None, rows=None,
           batches=None, aux=False):
    """Full decode. q_lat [B,q_len,H,512] / q_pe [B,q_len,H,64] float32 arrays;
    kv_u8 uint8 fp8 bits ([B,S,576] contiguous or [slots,576] pool).
    rows[b] = q/out batch row served by request b (None = identity).
    Returns bits [B,q_len,H,512] (+ pre, A)."""
    B, q_len, H, _ = q_lat.shape
    out = np.zeros((B, q_len, H, LAT), dtype=np.uint16)
    pre = np.full((B, q_len, H, LAT), np.nan) if aux else None
    scl = np.full((B, q_len, H, LAT), np.nan) if aux else None
    todo = range(B) if batches is None else batches
    for b in todo:
        qb = b if rows is None else min(max(int(rows[b]), 0), B - 1)
        c = request_rows(kv_u8, seq_lens, b, kv_indices, kv_indptr)
        S = c.shape[0]
        for t in range(q_len):
            end = S - (q_len - 1 - t)
            r = decode_one(q_lat[qb, t], q_pe[qb, t], c[:max(end, 0)], scale, kv_scale, aux=aux)
            if aux:
                out[qb, t], pre[qb, t], scl[qb, t] = r
            else:
                out[qb, t] = r
    return (out, pre, scl) if aux else out


def fp32_reference(q_lat, q_pe, kv_u8, seq_lens, scale, kv_scale, kv_indices=None, kv_indptr=None):
    """Reference test's fp32 formula (tests/test_mla_decode.py:50-66): dequantise
    k = fp8 * kv_scale, softmax(q . k * scale) @ k_lat, all float32, no P rounding."""
    B, q_len, H, _ = q_lat.shape
    out = np.zeros((B, q_len, H, LAT), dtype=np.float32)
    for b in range(B):
        k = (request_rows(kv_u8, seq_lens, b, kv_indices, kv_indptr) * kv_scale).astype(np.float32)
        S = k.shape[0]
        for t in range(q_len):
            end = S - q_len + t + 1
            sc = (q_lat[b, t].astype(np.float32) @ k[:end, :LAT].T
                  + q_pe[b, t].astype(np.float32) @ k[:end, LAT:].T) * np.float32(scale)
            sc = sc - sc.max(axis=1, keepdims=True)
            e = np.exp(sc)
            out[b, t] = (e / e.sum(axis=1, keepdims=True)) @ k[:end, :LAT]
    return out


def torch_formula_cpu(q_lat, q_pe, pool, seq_lens, kv_indices, kv_indptr, scale, kv_scale):
    """The reference test's fp32 loop (tests/test_mla_decode.py:50-66) in CPU
    torch over a paged pool: per request, gather its rows by kv_indices,
    dequantise (OCP e4m3fn -> fp32, * kv_scale), then per draft position t
    softmax((q_lat . k_lat + q_pe . k_pe) * scale) @ k_lat over the end-aligned
    window. q_lat [B,q_len,H,512], q_pe [B,q_len,H,64] bf16; pool [slots,1,576]
    float8_e4m3fn; seq_lens / kv_indices / kv_indptr int32. Returns fp32
    [B,q_len,H,512]. (The CPU baseline the bench times.)"""
    import torch

    B, q_len, H, _ = q_lat.shape
    flat = pool.view(-1, QK)
    out = torch.empty(B, q_len, H, LAT, dtype=torch.float32)
    for b in range(B):
        S = int(seq_lens[b])
        start = int(kv_indptr[b])
        k = flat.index_select(0, kv_indices[start:start + S].long()).float() * kv_scale
        k_lat, k_pe = k[:, :LAT], k[:, LAT:]
        for t in range(q_len):
            end = S - q_len + t + 1
            score = (q_lat[b, t].float() @ k_lat[:end].T + q_pe[b, t].float() @ k_pe[:end].T) * scale
            out[b, t] = torch.softmax(score, dim=-1) @ k_lat[:end]
    return out


def smoke_check(ma, torch):
    """Tiny paged MLA decode on cuda:0 vs the oracle (used by __graft_entry__.smoke)."""
    g = torch.Generator().manual_seed(11)
    B, H, q_len, S = 2, 16, 1, 300
    kv = (torch.randn(B * S, 1, QK, generator=g)).to(torch.float8_e4m3fn)
    q_lat = (torch.randn(B, q_len, H, LAT, generator=g) * 3).to(torch.bfloat16)
    q_pe = (torch.randn(B, q_len, H, ROPE, generator=g) * 3).to(torch.bfloat16)
    perm = torch.randperm(B * S, generator=g).to(torch.int32)
    lens = torch.tensor([S, S - 17], dtype=torch.int32)
    indptr = torch.tensor([0, S, 2 * S - 17], dtype=torch.int32)
    o = torch.zeros(B, q_len, H, LAT, dtype=torch.bfloat16, device="cuda:0")
    dev = lambda t: t.to("cuda:0")
    parts = ma.mla_decode_a16w8_plan_parts_q(B, S, q_len, H)
    scale, kv_scale = 1.0 / math.sqrt(192.0), 0.5
    ma.mla_decode_a16w8_paged_dev(dev(q_lat), dev(q_pe), dev(kv), o, dev(lens), None, dev(perm), dev(indptr),
                                  parts, scale, kv_scale)
    torch.cuda.synchronize()
    got = o.cpu().view(torch.int16).numpy().view(np.uint16)
    ref, _, A = decode(q_lat.float().numpy(), q_pe.float().numpy(), kv.view(torch.uint8).numpy(), lens.numpy(),
                       scale, kv_scale, kv_indices=perm.numpy(), kv_indptr=indptr.numpy(), aux=True)
    gv = _b.bf16_to_f32(got).astype(np.float64)
    rv = _b.bf16_to_f32(ref).astype(np.float64)
    ulp = _b.ulp_bf16(np.maximum(np.abs(rv), 0.25 * A))
    worst = float((np.abs(gv - rv) / ulp).max())
    assert worst <= 1.0, f"mla smoke: {worst:.2f} ULP"
    print(f"smoke mla paged B=2 H=16 S=300: max {worst:.2f} ULP, exact {(gv == rv).mean():.4f}")
