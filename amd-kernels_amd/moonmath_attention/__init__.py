"""MI355X (gfx950) bf16 flash-attention forward and fp8-KV absorbed-MLA decode.

Drop-in for the reference package's hot paths (moonmath reference
moonmath_attention/__init__.py:11-31), backed by hand-written gfx950 HIP
kernels in ``libmoonmath_gfx950.so`` called through ctypes.

>>> import torch, moonmath_attention as ma
>>> q = torch.randn(1, 4, 1024, 128, dtype=torch.bfloat16, device="cuda")
>>> out = ma.forward(q, q, q)          # bf16, same shape
"""

from ._kernel import forward, forward_lite
from .lite import LiteAttention
from .mla import (
    mla_decode_a16w8,
    mla_decode_a16w8_multiq,
    mla_decode_a16w8_multiq_paged_dev,
    mla_decode_a16w8_multiq_plan_parts_q,
    mla_decode_a16w8_paged_blocks,
    mla_decode_a16w8_paged_dev,
    mla_decode_a16w8_plan_parts,
    mla_decode_a16w8_plan_parts_capped,
    mla_decode_a16w8_plan_parts_q,
    mla_kv_quantize,
)

__all__ = [
    "forward", "forward_lite", "LiteAttention",
    "mla_decode_a16w8", "mla_decode_a16w8_paged_dev", "mla_decode_a16w8_paged_blocks",
    "mla_decode_a16w8_plan_parts", "mla_decode_a16w8_plan_parts_capped",
    "mla_decode_a16w8_plan_parts_q",
    "mla_decode_a16w8_multiq", "mla_decode_a16w8_multiq_paged_dev",
    "mla_decode_a16w8_multiq_plan_parts_q", "mla_kv_quantize",
]
