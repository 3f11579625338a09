"""``forward``: bf16 flash-attention forward on MI355X through the C ABI.

Mirrors the reference surface (moonmath reference moonmath_attention/_kernel.py:14-82)
and the checks of its pybind layer (csrc/attention_api.cpp:134-283): same
argument names, defaults, exception types and messages. ``std::invalid_argument``
in the reference surfaces as ``ValueError`` through pybind; here the checks are
raised directly in Python before anything touches the GPU.
"""
import os

import torch

from . import _lib

_MODES = {"rtne": 0, "rtna": 1, "rtz": 2}


def forward(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    out: torch.Tensor | None = None,
    round_mode: str = "rtna",
    layout: str = "bhsd",
) -> torch.Tensor:
    """Fused forward attention: O = softmax(Q K^T / sqrt(D)) V on MI355X (gfx950).

    Args:
        q, k, v: torch.bfloat16 tensors of shape (batch, heads, seq_len, head_dim)
            ("bhsd") or (batch, seq_len, heads, head_dim) ("bshd"). Contiguous,
            head_dim = 128, any Sq / Skv >= 1. CPU tensors are moved to cuda:0
            and the result is returned on the CPU.
        out: optional preallocated output (q's shape, bf16, contiguous, same device).
        round_mode: "rtna" (default), "rtne" or "rtz" -- the bf16 rounding of P
            and of the output.
        layout: "bhsd" (default) or "bshd".

    Returns:
        torch.bfloat16 tensor of q's shape on q's device.
    """
    for name, t in (("q", q), ("k", k), ("v", v)):
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"{name} must be torch.Tensor; got {type(t).__name__}")
        if t.dtype != torch.bfloat16:
            raise TypeError(f"{name} must be torch.bfloat16; got dtype={t.dtype}")
        if t.dim() != 4:
            raise ValueError(f"{name} must be 4-D ({layout.upper()}); got shape={tuple(t.shape)}")

    if q.device.type == "cpu":
        if k.device.type != "cpu" or v.device.type != "cpu":
            raise ValueError("q is on CPU but k or v is not; all must be on the same device")
        device = torch.device("cuda:0")
        out_gpu = out.to(device) if out is not None else None
        res = _forward_device(q.to(device), k.to(device), v.to(device), out_gpu, round_mode, layout)
        return res.cpu()
    elif q.device.type in ("cuda", "hip"):
        if k.device != q.device or v.device != q.device:
            raise ValueError(
                f"q/k/v must be on the same device; got q={q.device}, k={k.device}, v={v.device}"
            )
        return _forward_device(q, k, v, out, round_mode, layout)
    else:
        raise NotImplementedError(f"Unsupported device {q.device!r}; expected 'cpu' or 'cuda'/'hip'")


def _check_tensor(t, name):
    # reference csrc/attention_api.cpp:134-150
    if t is None:
        raise ValueError(f"{name} must be a valid tensor")
    if t.dtype != torch.bfloat16:
        raise ValueError(f"{name} must be bfloat16, got {t.dtype}")
    if t.dim() != 4:
        raise ValueError(f"{name} must be 4-D, got {t.dim()}-D")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be on a CUDA/HIP device (GPU-only), got device={t.device}")


def check_args(q, k, v, out, round_mode, layout):
    """Validation of reference csrc/attention_api.cpp:160-229. Returns
    (B, H, Sq, Skv, layout_int)."""
    _check_tensor(q, "q")
    _check_tensor(k, "k")
    _check_tensor(v, "v")
    if round_mode not in _MODES:
        raise ValueError(f"round_mode must be 'rtna', 'rtne', or 'rtz', got '{round_mode}'")
    bshd = layout == "bshd"
    if not bshd and layout != "bhsd":
        raise ValueError(f"layout must be 'bhsd' or 'bshd', got '{layout}'")
    sax, hax = (1, 2) if bshd else (2, 1)
    B, H, Sq, D = q.shape[0], q.shape[hax], q.shape[sax], q.shape[3]
    Skv = k.shape[sax]
    if D != 128:
        raise ValueError(f"head_dim must be 128, got {D}")
    if k.shape[0] != B or k.shape[hax] != H or k.shape[3] != D:
        raise ValueError(
            f"k shape mismatch: expected batch={B}, heads={H}, head_dim={D}, got k.shape={list(k.shape)}"
        )
    if v.shape[0] != B or v.shape[hax] != H or v.shape[sax] != Skv or v.shape[3] != D:
        raise ValueError(f"v shape mismatch: must match k.shape, got v.shape={list(v.shape)}, k.shape={list(k.shape)}")
    if Sq <= 0 or Skv <= 0:
        raise ValueError(f"seq_len must be positive, got Sq={Sq}, Skv={Skv}")
    if q.device != k.device or q.device != v.device:
        raise ValueError("q, k, v must be on the same device")
    if out is not None:
        _check_tensor(out, "out")
        if out.shape != q.shape:
            raise ValueError(f"out shape must match q.shape, got out.shape={list(out.shape)}, q.shape={list(q.shape)}")
        if out.device != q.device:
            raise ValueError("out must be on the same device as q")
    return B, H, Sq, Skv, int(bshd)


def _forward_device(q, k, v, out, round_mode, layout):
    B, H, Sq, Skv, lay = check_args(q, k, v, out, round_mode, layout)
    if out is None:
        out = torch.empty_like(q)
    dev = q.device
    lib = _lib.lib
    with torch.cuda.device(dev):
        stream = _lib.stream_ptr(dev)
        vt = torch.empty(lib.moonmath_attention_vt_bytes(B, H, Skv) // 2, dtype=torch.bfloat16, device=dev)
        # Tail KV-split workspace, allocated only when the planner splits.
        # MOONMATH_NO_TAIL disables the split (reference csrc/attention_api.cpp:258-267);
        # MOONMATH_FORCE_SPLIT=G forces G parts on the last round (test hook).
        force = int(os.environ.get("MOONMATH_FORCE_SPLIT", "0") or 0)
        enable = os.environ.get("MOONMATH_NO_TAIL") is None
        ws = None
        if enable:
            plan = _lib.plan_tail(B, H, Sq, Skv, True, force)
            if plan[3] > 0:
                ws = torch.empty(lib.tail_workspace_bytes_rtne(), dtype=torch.uint8, device=dev)
        rc = getattr(lib, f"launch_v_transpose_{round_mode}")(
            _lib.ptr(v), _lib.ptr(vt), B * H * Skv, Skv, H, lay, stream
        )
        if rc != 0:
            raise RuntimeError(f"launch_v_transpose returned error code {rc}")
        rc = lib.moonmath_attention_forward_ex(
            _lib.ptr(q), _lib.ptr(k), _lib.ptr(vt), _lib.ptr(out), B, H, Sq, Skv, 128, lay,
            _MODES[round_mode], _lib.ptr(ws), force, stream,
        )
        if rc != 0:
            raise RuntimeError(f"launch_attention_forward returned error code {rc}")
    return out


def _check_list(t, name, q, min_numel):
    # reference csrc/attention_api.cpp:322-336; the size check is this build's
    # (the kernel reads and writes whole rows of [B,H,qtiles,ktiles+2]).
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be torch.Tensor; got {type(t).__name__}")
    if t.dtype != torch.int16:
        raise ValueError(f"{name} must be int16, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if t.device != q.device:
        raise ValueError(f"{name} must be on the same device as q")
    if t.numel() < min_numel:
        raise ValueError(f"{name} must hold at least {min_numel} int16 ([B,H,qtiles,ktiles+2]), got {t.numel()}")


def forward_lite(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    read_list: torch.Tensor,
    write_list: torch.Tensor,
    *,
    threshold: float,
    phase: int,
    must_do_list: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
    round_mode: str = "rtna",
    layout: str = "bhsd",
) -> torch.Tensor:
    """LiteAttention forward: only the K-blocks the skip list names are computed.

    Mirrors reference moonmath_attention/_kernel.py:85-134 and
    csrc/attention_api.cpp:283-440 (GPU tensors only). ``read_list`` /
    ``write_list`` are int16 [B, H, qtiles, ktiles+2] run-length rows (qtiles =
    ceil(Sq/256), ktiles = ceil(Skv/64)): ``read_list`` names the blocks this
    step loads, the kernel writes the next step's list into ``write_list``.
    Each wave of 32 q rows keeps a listed block for its rows when some valid
    row's block max came within ``threshold`` (log2) of the row's running max
    over the blocks the wave kept before (the first processed block always);
    a block the wave drops adds nothing to its rows. A block stays in the next
    list when some wave kept it. ``phase`` 1 walks ranges ascending, 0
    descending. ``must_do_list`` (int16 [len, s0, e0, ...], end exclusive)
    pins processed blocks as kept in the next list.
    MOONMATH_LITE_PLAIN=1 disables the LPT (heaviest-first) CTA order.
    """
    for name, t in (("q", q), ("k", k), ("v", v)):
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"{name} must be torch.Tensor; got {type(t).__name__}")
    B, H, Sq, Skv, lay = check_args(q, k, v, out, round_mode, layout)
    nqb = -(-Sq // 256)
    nkb = -(-Skv // 64)
    need = B * H * nqb * (nkb + 2)
    _check_list(read_list, "read_list", q, need)
    _check_list(write_list, "write_list", q, need)
    if must_do_list is not None:
        _check_list(must_do_list, "must_do_list", q, 1)
        # The kernel reads must_do_list[0] entries after the first: they must
        # exist (one host sync, only when a list is given).
        n_md = int(must_do_list[0].item())
        if n_md < 0 or n_md > must_do_list.numel() - 1:
            raise ValueError(f"must_do_list[0] = {n_md} but the list holds {must_do_list.numel() - 1} entries after it")
    if out is None:
        out = torch.empty_like(q)
    dev = q.device
    lib = _lib.lib
    with torch.cuda.device(dev):
        stream = _lib.stream_ptr(dev)
        vt = torch.empty(lib.moonmath_attention_vt_bytes(B, H, Skv) // 2, dtype=torch.bfloat16, device=dev)
        ws = None
        if os.environ.get("MOONMATH_LITE_PLAIN") is None:
            ws = torch.empty(getattr(lib, f"lite_workspace_bytes_{round_mode}")(B, H, Sq), dtype=torch.uint8,
                             device=dev)
        rc = getattr(lib, f"launch_v_transpose_{round_mode}")(
            _lib.ptr(v), _lib.ptr(vt), B * H * Skv, Skv, H, lay, stream
        )
        if rc != 0:
            raise RuntimeError(f"launch_v_transpose returned error code {rc}")
        rc = getattr(lib, f"launch_attention_forward_lite_{round_mode}")(
            _lib.ptr(q), _lib.ptr(k), _lib.ptr(vt), _lib.ptr(out), B, H, Sq, Skv, 128,
            _lib.ptr(read_list), _lib.ptr(write_list), _lib.ptr(must_do_list), float(threshold), int(phase), lay,
            _lib.ptr(ws), stream,
        )
        if rc != 0:
            raise RuntimeError(f"launch_attention_forward_lite returned error code {rc}")
    return out
