"""CPU oracle for the moonmath gfx950 hot paths -- TEST INFRASTRUCTURE ONLY.

This package is the checker, never the product: only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
it. The shipped path (``amd-kernels_amd/moonmath_attention``) never imports it
and fails loudly when its HIP library is missing.

Modules
-------
bf16       per-mode fp32 -> bf16 bit rules (reference csrc/attention_kernel.hip:110-145)
attention  softmax(Q K^T / sqrt(128)) V with the reference's per-mode P and
           output rounding (reference :390-452, :946-1016, :1088-1127) under the
           integer-grid running-max policy
vt_layout  the V_t operand permutation and a 32x32x16 MFMA lane-layout emulator
planner    tail KV-split planner (reference :1349-1393)
fp8        OCP e4m3fn decode (OCP 8-bit floating point spec, v1.0)
mla        absorbed-MLA paged decode (reference csrc/mla_decode_a16w8.hip:1-24,
           tests/test_mla_decode.py:50-66)
lite       LiteAttention skip lists: read-row cursor, vote, write-row emitter,
           LPT order (reference csrc/attention_kernel.hip:629-716, :983-995,
           :1296-1347)

Pinning: every function is checked in ``tests/test_oracle_*.py`` against
hand-derived known answers, closed forms or library routines (torch's RTNE
bf16 cast, torch's float8_e4m3fn decode, fp64 softmax), not against itself.
"""
