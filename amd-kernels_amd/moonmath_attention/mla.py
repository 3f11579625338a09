"""Absorbed-MLA decode ops (DeepSeek-V3 style) on MI355X: bf16 Q against fp8 KV.

Mirrors the reference surface (moonmath reference moonmath_attention/mla.py:41-186)
and the checks of its pybind layer (csrc/mla_decode_a16w8_api.cpp:41-148,
csrc/mla_decode_a16w8_multiq_api.cpp:42-167). Divergences, by design of the
gfx950 build:

* KV is OCP ``torch.float8_e4m3fn`` (gfx950 native) instead of e4m3fnuz;
* H (query heads) may be 1..128 instead of 1..16;
* the multi-query ops accept q_len 2..8 (the reference: 4..8);
* one kernel serves both op families (queries of a draft window share each KV
  tile load; the window is end-aligned causal: position t of q_len sees tokens
  [0, S - q_len + t + 1)).

KV rows are fused 576-wide ([..., :512] latent, [512:576] rope) at one
per-tensor ``kv_scale``; ``o_lat`` is written in place on the caller's current
stream with no host synchronisation. ``scale_p`` is accepted for ABI symmetry
and unused, as in the reference.
"""
import torch

from . import _lib

__all__ = [
    "mla_decode_a16w8",
    "mla_decode_a16w8_paged_dev",
    "mla_decode_a16w8_paged_blocks",
    "mla_decode_a16w8_plan_parts",
    "mla_decode_a16w8_plan_parts_capped",
    "mla_decode_a16w8_plan_parts_q",
    "mla_decode_a16w8_multiq",
    "mla_decode_a16w8_multiq_paged_dev",
    "mla_decode_a16w8_multiq_plan_parts_q",
    "mla_kv_quantize",
]

_LAT = 512
_ROPE = 64
_QK = _LAT + _ROPE  # 576
_MAX_H = 128
_FP8 = torch.float8_e4m3fn


def _check_q(q_lat, q_pe, o_lat, who, multiq):
    """Query checks (reference mla_decode_a16w8_api.cpp:41-62 and
    mla_decode_a16w8_multiq_api.cpp:42-62). Returns (B, H, q_len)."""
    for name, t in (("q_lat", q_lat), ("q_pe", q_pe), ("o_lat", o_lat)):
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"{who}: {name} must be torch.Tensor; got {type(t).__name__}")
    D = q_lat.dim()
    if multiq:
        if D != 4:
            raise ValueError(f"{who}: q_lat must be [B,q_len,H,512] (q_len 2..8)")
    elif D not in (3, 4):
        raise ValueError(f"{who}: q_lat must be [B,H,512] or [B,q_len,H,512]")
    if q_pe.dim() != D or o_lat.dim() != D:
        raise ValueError(f"{who}: q_lat/q_pe/o_lat must have the same rank")
    if q_lat.dtype != torch.bfloat16 or q_pe.dtype != torch.bfloat16 or o_lat.dtype != torch.bfloat16:
        raise ValueError(f"{who}: q_lat/q_pe/o_lat must be bfloat16")
    if q_lat.device.type != "cuda":
        raise ValueError(f"{who}: tensors must be on a CUDA/HIP device")
    if q_pe.device != q_lat.device or o_lat.device != q_lat.device:
        raise ValueError(f"{who}: q_lat/q_pe/o_lat must be on the same device")
    if q_lat.shape[-1] != _LAT or q_pe.shape[-1] != _ROPE or o_lat.shape[-1] != _LAT:
        raise ValueError(f"{who}: expected q_lat[...,512], q_pe[...,64], o_lat[...,512]")
    if q_pe.shape[:-1] != q_lat.shape[:-1] or o_lat.shape != q_lat.shape:
        raise ValueError(f"{who}: q_pe/o_lat leading dims must match q_lat")
    H = q_lat.shape[-2]
    if H < 1 or H > _MAX_H:
        raise ValueError(f"{who}: H must be in [1,{_MAX_H}]")
    q_len = q_lat.shape[1] if D == 4 else 1
    lo = 2 if multiq else 1
    if q_len < lo or q_len > 8:
        raise ValueError(f"{who}: q_len must be in [{lo},8]")
    if not (q_lat.is_contiguous() and q_pe.is_contiguous() and o_lat.is_contiguous()):
        raise ValueError(f"{who}: q_lat/q_pe/o_lat must be contiguous")
    return q_lat.shape[0], H, q_len


def _check_slab(kv, B, who):
    if not isinstance(kv, torch.Tensor) or kv.dtype != _FP8:
        raise ValueError(f"{who}: kv must be float8_e4m3fn")
    if kv.dim() != 3 or kv.shape[2] != _QK:
        raise ValueError(
            f"{who}: kv must be the FUSED [B,S,576] slab ([...,:512]=latent, [512:576]=rope), "
            "not the split c_kv/k_pe pair"
        )
    if kv.shape[0] != B:
        raise ValueError(f"{who}: kv batch must match q_lat batch")
    if not kv.is_contiguous():
        raise ValueError(f"{who}: kv must be contiguous")
    if kv.shape[1] < 1:
        raise ValueError(f"{who}: kv must hold at least one token")


def _check_paged(kv_pool, seq_lens, rows, kv_indices, kv_indptr, parts, B, who):
    if not isinstance(kv_pool, torch.Tensor) or kv_pool.dtype != _FP8:
        raise ValueError(f"{who}: kv_pool must be float8_e4m3fn")
    if kv_pool.shape[-1] != _QK:
        raise ValueError(f"{who}: kv_pool rows must be 576 wide ([...,:512]=c_KV, [512:576]=k_pe)")
    if not kv_pool.is_contiguous():
        raise ValueError(f"{who}: kv_pool must be contiguous")
    for name, t in (("seq_lens", seq_lens), ("kv_indices", kv_indices), ("kv_indptr", kv_indptr)):
        if not isinstance(t, torch.Tensor) or t.dtype != torch.int32:
            raise ValueError(f"{who}: seq_lens/kv_indices/kv_indptr must be int32")
        if t.device != kv_pool.device:
            raise ValueError(f"{who}: {name} must be on the device")
    if seq_lens.numel() < B or not seq_lens.is_contiguous():
        raise ValueError(f"{who}: seq_lens must be contiguous with >= B entries")
    if kv_indptr.numel() < B + 1 or not kv_indptr.is_contiguous():
        raise ValueError(f"{who}: kv_indptr must be contiguous with >= B+1 entries")
    if not kv_indices.is_contiguous():
        raise ValueError(f"{who}: kv_indices must be contiguous")
    if rows is not None:
        if not isinstance(rows, torch.Tensor) or rows.dtype != torch.int32:
            raise ValueError(f"{who}: rows must be int32")
        if rows.numel() < B or not rows.is_contiguous():
            raise ValueError(f"{who}: rows must be contiguous with >= B entries")
        if rows.device != kv_pool.device:
            raise ValueError(f"{who}: rows must be on the device")
    if int(parts) > (1 << 20):
        raise ValueError(f"{who}: parts is absurd (> 2^20)")


def _workspace(B, H, parts, q_len, device):
    lib = _lib.lib
    eff = lib.moonmath_mla_effective_parts(B, H, int(parts), q_len, 1)
    if eff <= 1:
        return None
    nbytes = lib.mla_decode_a16w8_multiq_workspace_for(B, H, eff, q_len)
    return torch.empty(nbytes, dtype=torch.uint8, device=device)


def _run(fn_name, *args):
    rc = getattr(_lib.lib, fn_name)(*args)
    if rc != 0:
        raise RuntimeError(f"{fn_name} returned error code {rc}")


def mla_decode_a16w8(q_lat, q_pe, kv, o_lat, scale, kv_scale, scale_p=1.0) -> None:
    """Absorbed-decode MLA, q_len = 1, contiguous KV.

    q_lat [B,H,512] bf16, q_pe [B,H,64] bf16, kv [B,S,576] float8_e4m3fn,
    o_lat [B,H,512] bf16 (written in place). scale = softmax scale,
    kv_scale = per-tensor fp8 KV descale. (Reference mla.py:41-61.)
    """
    who = "mla_decode_a16w8"
    B, H, q_len = _check_q(q_lat, q_pe, o_lat, who, multiq=False)
    if q_len != 1:
        raise ValueError(
            f"{who}: the contiguous entry point is q_len==1 only; use mla_decode_a16w8_paged_dev for a draft window"
        )
    _check_slab(kv, B, who)
    S = kv.shape[1]
    dev = q_lat.device
    with torch.cuda.device(dev):
        parts = _lib.lib.mla_decode_a16w8_plan_parts(B, H, S, _LAT)
        ws = _workspace(B, H, parts, 1, dev)
        _run("launch_mla_decode_a16w8", _lib.ptr(q_lat), _lib.ptr(q_pe), _lib.ptr(kv), None, _lib.ptr(o_lat),
             B, H, S, _LAT, _ROPE, float(scale), float(kv_scale), float(scale_p), _lib.ptr(ws), _lib.stream_ptr(dev))


def mla_decode_a16w8_paged_dev(q_lat, q_pe, kv_pool, o_lat, seq_lens, rows, kv_indices, kv_indptr, parts,
                               scale, kv_scale, scale_p=1.0) -> None:
    """Absorbed-decode MLA over a paged pool, device-driven (graph capturable).

    q_lat/q_pe: [B,H,*] (q_len 1) or [B,q_len,H,*] (draft window, q_len <= 8);
    kv_pool [num_slots,1,576] (or [num_slots,576]) float8_e4m3fn; request b owns
    flat slots kv_indices[kv_indptr[b] : kv_indptr[b] + seq_lens[b]]; rows [B]
    int32 maps request -> q/out batch row (None = identity); parts is fixed by
    the caller (plan_parts*). (Reference mla.py:64-95.)
    """
    who = "mla_decode_a16w8_paged_dev"
    B, H, q_len = _check_q(q_lat, q_pe, o_lat, who, multiq=False)
    _check_paged(kv_pool, seq_lens, rows, kv_indices, kv_indptr, parts, B, who)
    dev = q_lat.device
    with torch.cuda.device(dev):
        ws = _workspace(B, H, parts, q_len, dev)
        _run("launch_mla_decode_a16w8_paged_dev", _lib.ptr(q_lat), _lib.ptr(q_pe), _lib.ptr(kv_pool),
             _lib.ptr(o_lat), _lib.ptr(seq_lens), _lib.ptr(rows), _lib.ptr(kv_indices), _lib.ptr(kv_indptr),
             B, H, int(parts), _LAT, _ROPE, float(scale), float(kv_scale), float(scale_p), _lib.ptr(ws),
             _lib.stream_ptr(dev), kv_indices.numel() * _QK, q_len)


_PAGE = 64


def mla_decode_a16w8_paged_blocks(q_lat, q_pe, kv_pool, o_lat, seq_lens, block_table, parts, scale, kv_scale,
                                  scale_p=1.0, rows=None) -> None:
    """Absorbed decode over a paged pool addressed by 64-token block tables (the
    form a serving stack's paged KV cache keeps; no counterpart in the
    reference, whose ops take flat per-token slots).

    kv_pool: float8_e4m3fn pages of 64 fused rows, [num_blocks, 64, 576] (or
    any contiguous shape of num_blocks * 64 rows of 576); block_table: int32
    [B, max_blocks], request b's token t is row t % 64 of page
    block_table[b, t // 64]; q_lat [B,H,512] (q_len 1) or [B,q_len,H,512]
    (q_len <= 8), draft window end-aligned; rows as in the paged ops. Device
    driven and graph capturable with ``parts`` fixed: the table is expanded to
    per-token slots on the GPU (page ids clamped to the pool, lengths to the
    table) and the flat-slot decode runs on the same stream.
    """
    who = "mla_decode_a16w8_paged_blocks"
    B, H, q_len = _check_q(q_lat, q_pe, o_lat, who, multiq=False)
    if not isinstance(kv_pool, torch.Tensor) or kv_pool.dtype != _FP8:
        raise ValueError(f"{who}: kv_pool must be float8_e4m3fn")
    if kv_pool.shape[-1] != _QK or kv_pool.numel() % (_PAGE * _QK) != 0 or not kv_pool.is_contiguous():
        raise ValueError(f"{who}: kv_pool must be contiguous pages of 64 rows of 576 ([num_blocks,64,576])")
    if not isinstance(block_table, torch.Tensor) or block_table.dtype != torch.int32 or block_table.dim() != 2:
        raise ValueError(f"{who}: block_table must be int32 [B, max_blocks]")
    if block_table.shape[0] != B or not block_table.is_contiguous() or block_table.shape[1] < 1:
        raise ValueError(f"{who}: block_table must be contiguous [B, max_blocks] with B = q_lat's batch")
    if not isinstance(seq_lens, torch.Tensor) or seq_lens.dtype != torch.int32 or not seq_lens.is_contiguous():
        raise ValueError(f"{who}: seq_lens must be contiguous int32")
    if seq_lens.numel() < B:
        raise ValueError(f"{who}: seq_lens must have >= B entries")
    for name, t in (("kv_pool", kv_pool), ("block_table", block_table), ("seq_lens", seq_lens)):
        if t.device != q_lat.device:
            raise ValueError(f"{who}: {name} must be on q_lat's device")
    if rows is not None:
        if not isinstance(rows, torch.Tensor) or rows.dtype != torch.int32 or rows.numel() < B:
            raise ValueError(f"{who}: rows must be int32 with >= B entries")
        if rows.device != q_lat.device or not rows.is_contiguous():
            raise ValueError(f"{who}: rows must be contiguous on q_lat's device")
    if int(parts) > (1 << 20):
        raise ValueError(f"{who}: parts is absurd (> 2^20)")
    num_blocks = kv_pool.numel() // (_PAGE * _QK)
    max_blocks = block_table.shape[1]
    dev = q_lat.device
    lib = _lib.lib
    with torch.cuda.device(dev):
        ws = _workspace(B, H, parts, q_len, dev)
        idx_ws = torch.empty(lib.mla_decode_a16w8_blocks_index_bytes(B, max_blocks), dtype=torch.uint8, device=dev)
        _run("launch_mla_decode_a16w8_paged_blocks_dev", _lib.ptr(q_lat), _lib.ptr(q_pe), _lib.ptr(kv_pool),
             _lib.ptr(o_lat), _lib.ptr(seq_lens), _lib.ptr(rows), _lib.ptr(block_table), max_blocks, num_blocks,
             B, H, int(parts), q_len, _LAT, _ROPE, float(scale), float(kv_scale), float(scale_p), _lib.ptr(ws),
             _lib.ptr(idx_ws), _lib.stream_ptr(dev))


def mla_decode_a16w8_plan_parts(B: int, H: int, max_seq_len: int, lat_dim: int = 512) -> int:
    """Fixed KV-split count for a graph captured at (B, H, max_seq_len)."""
    return int(_lib.lib.mla_decode_a16w8_plan_parts(int(B), int(H), int(max_seq_len), int(lat_dim)))


def mla_decode_a16w8_plan_parts_capped(B: int, H: int, max_seq_len: int, lat_dim: int = 512) -> int:
    """As plan_parts, clamped to the split workspace."""
    return int(_lib.lib.mla_decode_a16w8_plan_parts_capped(int(B), int(H), int(max_seq_len), int(lat_dim)))


def mla_decode_a16w8_plan_parts_q(B: int, max_seq_len: int, q_len: int = 1, H: int = 16) -> int:
    """q_len-aware fixed KV-split count for a graph captured at (B, max_seq_len, q_len)."""
    return int(_lib.lib.mla_decode_a16w8_plan_parts_q(int(B), int(max_seq_len), int(q_len), int(H)))


def mla_decode_a16w8_multiq(q_lat, q_pe, kv, o_lat, scale, kv_scale, scale_p=1.0) -> None:
    """Multi-query (draft window) absorbed decode, contiguous KV.

    q_lat [B,q_len,H,512], q_pe [B,q_len,H,64] bf16, q_len 2..8; kv [B,S,576]
    float8_e4m3fn; o_lat like q_lat. Position t attends kv[:, : S - q_len + t + 1].
    (Reference mla.py:122-145.)
    """
    who = "mla_decode_a16w8_multiq"
    B, H, q_len = _check_q(q_lat, q_pe, o_lat, who, multiq=True)
    _check_slab(kv, B, who)
    S = kv.shape[1]
    dev = q_lat.device
    with torch.cuda.device(dev):
        parts = _lib.lib.mla_decode_a16w8_multiq_plan_parts_q(B, S, q_len, H)
        ws = _workspace(B, H, parts, q_len, dev)
        _run("launch_mla_decode_a16w8_multiq", _lib.ptr(q_lat), _lib.ptr(q_pe), _lib.ptr(kv), _lib.ptr(o_lat),
             B, H, S, q_len, _LAT, _ROPE, float(scale), float(kv_scale), _lib.ptr(ws), _lib.stream_ptr(dev))


def mla_decode_a16w8_multiq_paged_dev(q_lat, q_pe, kv_pool, o_lat, seq_lens, rows, kv_indices, kv_indptr, parts,
                                      scale, kv_scale, scale_p=1.0) -> None:
    """Multi-query decode over a paged pool, device-driven (graph capturable).
    (Reference mla.py:148-176.)"""
    who = "mla_decode_a16w8_multiq_paged_dev"
    B, H, q_len = _check_q(q_lat, q_pe, o_lat, who, multiq=True)
    _check_paged(kv_pool, seq_lens, rows, kv_indices, kv_indptr, parts, B, who)
    dev = q_lat.device
    with torch.cuda.device(dev):
        ws = _workspace(B, H, parts, q_len, dev)
        _run("launch_mla_decode_a16w8_multiq_paged_dev", _lib.ptr(q_lat), _lib.ptr(q_pe), _lib.ptr(kv_pool),
             _lib.ptr(o_lat), _lib.ptr(seq_lens), _lib.ptr(rows), _lib.ptr(kv_indices), _lib.ptr(kv_indptr),
             B, H, int(parts), q_len, _LAT, _ROPE, float(scale), float(kv_scale), _lib.ptr(ws),
             _lib.stream_ptr(dev), kv_indices.numel() * _QK)


def mla_decode_a16w8_multiq_plan_parts_q(B: int, max_seq_len: int, q_len: int = 4, H: int = 16) -> int:
    """Fixed KV-split count for a multi-query graph captured at (B, max_seq_len, q_len, H)."""
    return int(_lib.lib.mla_decode_a16w8_multiq_plan_parts_q(int(B), int(max_seq_len), int(q_len), int(H)))


def mla_kv_quantize(c_kv, k_pe, kv_pool, slots, kv_scale, saturate=False) -> None:
    """Write new tokens into the fp8 KV cache the decode ops read.

    c_kv [N, 512] and k_pe [N, 64] bf16 (latent and roped key of N tokens);
    kv_pool float8_e4m3fn with rows of 576 ([num_slots, 576], [num_slots, 1,
    576] or [num_blocks, 64, 576]); slots int32 [N]: token i goes to row
    slots[i] (negative = padding token, skipped). Each row becomes
    e4m3fn(x / kv_scale) of [c_kv | k_pe], round to nearest even, |x / kv_scale|
    > 464 -> NaN as torch's float8_e4m3fn cast, or clamped to +-448 with
    ``saturate``. Written in place on the current stream (graph capturable).
    The reference has no producer; this is the cache format its ops take
    (moonmath_attention/mla.py:17-20) filled the way its tests fill it
    (tests/test_mla_decode.py:34-38).
    """
    who = "mla_kv_quantize"
    for name, t, w in (("c_kv", c_kv, _LAT), ("k_pe", k_pe, _ROPE)):
        if not isinstance(t, torch.Tensor) or t.dtype != torch.bfloat16:
            raise ValueError(f"{who}: {name} must be a bfloat16 tensor")
        if t.dim() < 1 or t.shape[-1] != w or not t.is_contiguous():
            raise ValueError(f"{who}: {name} must be contiguous [..., {w}]")
    N = c_kv.numel() // _LAT
    if k_pe.numel() // _ROPE != N:
        raise ValueError(f"{who}: c_kv and k_pe must hold the same number of tokens")
    if not isinstance(kv_pool, torch.Tensor) or kv_pool.dtype != _FP8:
        raise ValueError(f"{who}: kv_pool must be float8_e4m3fn")
    if kv_pool.shape[-1] != _QK or not kv_pool.is_contiguous():
        raise ValueError(f"{who}: kv_pool must be contiguous rows of 576")
    if not isinstance(slots, torch.Tensor) or slots.dtype != torch.int32 or not slots.is_contiguous():
        raise ValueError(f"{who}: slots must be contiguous int32")
    if slots.numel() != N:
        raise ValueError(f"{who}: slots must have one entry per token ({N}), got {slots.numel()}")
    for name, t in (("k_pe", k_pe), ("kv_pool", kv_pool), ("slots", slots)):
        if t.device != c_kv.device:
            raise ValueError(f"{who}: {name} must be on c_kv's device")
    if c_kv.device.type != "cuda":
        raise ValueError(f"{who}: tensors must be on a CUDA/HIP device")
    if not (float(kv_scale) > 0.0) or float(kv_scale) == float("inf"):
        raise ValueError(f"{who}: kv_scale must be a positive finite number")
    dev = c_kv.device
    with torch.cuda.device(dev):
        _run("launch_mla_kv_quantize", _lib.ptr(c_kv), _lib.ptr(k_pe), _lib.ptr(kv_pool), _lib.ptr(slots), N,
             kv_pool.numel() // _QK, float(kv_scale), int(bool(saturate)), _lib.stream_ptr(dev))
