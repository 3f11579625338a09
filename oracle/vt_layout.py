"""V_t operand order and a wave64 MFMA lane-layout emulator (numpy).

The reference pre-transposes V for its 16x16x16 MFMA (csrc/attention_kernel.hip
:1130-1136, :1137-1217). This build re-derives the order for the gfx950
``v_mfma_f32_32x32x16_bf16`` with scores computed transposed (S^T = K Q^T):

* 32x32 accumulator: lane l, register i holds row ``8*(i//4) + 4*(l//32) + i%4``,
  column ``l % 32``.
* A/B operands: lane l holds 8 contraction elements ``8*(l//32) + e`` of
  row/column ``l % 32`` (any permutation of the 16 contraction slots that A and
  B share gives the same product).

For a 64-row kv block, V_t fragment ``f = (t*2 + s)*4 + dt`` (t = 32-row kv
tile, s = 16-row PV step, dt = 32-wide d tile), lane l, element e holds
``V[32t + 16s + 8(e//4) + 4(l//32) + e%4, 32dt + l%32]``; rows >= Skv are 0.
"""
import numpy as np

KV_BLOCK = 64
D = 128


def vt_source_index():
    """(kv, d) source of every V_t slot of one block: arrays [16, 64, 8]."""
    f = np.arange(16)[:, None, None]
    lane = np.arange(64)[None, :, None]
    e = np.arange(8)[None, None, :]
    t, s, dt = f // 8, (f // 4) % 2, f % 4
    kv = 32 * t + 16 * s + 8 * (e // 4) + 4 * (lane // 32) + e % 4
    d = 32 * dt + lane % 32
    return np.broadcast_to(kv, (16, 64, 8)), np.broadcast_to(d, (16, 64, 8))


def v_transpose(V, Skv=None):
    """One head: V [Skv, 128] (any dtype) -> V_t [nkb, 16, 64, 8], zero padded."""
    Skv = V.shape[0] if Skv is None else Skv
    nkb = -(-Skv // KV_BLOCK)
    pad = np.zeros((nkb * KV_BLOCK, D), dtype=V.dtype)
    pad[:Skv] = V[:Skv]
    kv, d = vt_source_index()
    out = np.empty((nkb, 16, 64, 8), dtype=V.dtype)
    for kb in range(nkb):
        out[kb] = pad[kb * KV_BLOCK + kv, d]
    return out


# ---- MFMA 32x32x16 emulator ---------------------------------------------------

def acc_row_col():
    """Accumulator ownership: rows[l, i], cols[l, i] for lane l, register i."""
    lane = np.arange(64)[:, None]
    i = np.arange(16)[None, :]
    rows = 8 * (i // 4) + 4 * (lane // 32) + i % 4
    cols = np.broadcast_to(lane % 32, (64, 16))
    return np.broadcast_to(rows, (64, 16)), cols


def mfma_32x32x16(a, b, c):
    """a, b: [64 lanes, 8] operand registers; c: [64, 16] accumulator registers.

    A[m, k] lives at lane (m + 32*(k//8)), element k%8; B[k, n] at lane
    (n + 32*(k//8)), element k%8. Returns c + A @ B in accumulator layout.
    """
    A = np.zeros((32, 16))
    B = np.zeros((16, 32))
    for lane in range(64):
        for e in range(8):
            k = 8 * (lane // 32) + e
            A[lane % 32, k] = a[lane, e]
            B[k, lane % 32] = b[lane, e]
    Dm = A @ B
    rows, cols = acc_row_col()
    return c + Dm[rows, cols]


def pv_block_emulated(P_T_acc, vt_block):
    """O^T (128 x 32) for one 64-row kv block from the S^T accumulators.

    P_T_acc: [2 (t), 64, 16] accumulator registers holding P^T (kv x q) for the
    two 32-row kv tiles. vt_block: [16, 64, 8]. Returns [4 (dt), 64, 16].
    """
    o = np.zeros((4, 64, 16))
    for dt in range(4):
        for t in range(2):
            for s in range(2):
                b = P_T_acc[t][:, 8 * s:8 * s + 8]  # B operand straight from registers
                a = vt_block[(t * 2 + s) * 4 + dt]
                o[dt] = mfma_32x32x16(a, b, o[dt])
    return o
