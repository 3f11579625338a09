"""LiteAttention: reuse of one diffusion step's attention sparsity in the next.

Same public surface as the reference class (moonmath reference
moonmath_attention/lite.py:44-185). Consecutive denoising steps attend to
nearly the same keys. Each call therefore hands the kernel two int16 lists per
(batch, head, q-tile): the one the previous call produced, which says which
64-row K blocks to load and compute at all, and an output list that the kernel
fills with the blocks this call found worth keeping. Inside a call, each wave
of 32 q rows also drops, for its own rows, a listed block whose scores all sit
more than |threshold| (log2 units) below the wave's running maxima. A block
stays in the next list when some wave kept it, or when ``must_do_list`` pins it.
The first call starts from a list that names every block.

Geometry of this build: q-tiles of 256 rows (8 waves x 32 rows) and 64-row K
blocks, reported by ``get_MN()`` (the reference's gfx942 kernel uses 384-row
tiles, so the two builds' lists are not interchangeable).

Typical use in a sampler loop::

    attn = moonmath_attention.LiteAttention(threshold=-6.0, layout="bshd")
    for step in range(steps):
        out = attn(q, k, v)
    attn.reset_skip_state()   # before a new prompt or another shape
"""
import torch

from . import _kernel

KBLOCK_M = 256
KBLOCK_N = 64


def _ceil_div(a, b):
    return (a + b - 1) // b


def _list_shape(q, k, layout):
    """(B, H, q-tiles, K-blocks) of the lists for these inputs."""
    if layout == "bshd":
        B, Sq, H = q.shape[0], q.shape[1], q.shape[2]
        Skv = k.shape[1]
    else:
        B, H, Sq = q.shape[0], q.shape[1], q.shape[2]
        Skv = k.shape[2]
    return B, H, _ceil_div(Sq, KBLOCK_M), _ceil_div(Skv, KBLOCK_N)


class LiteAttention:
    """Holds the pair of int16 lists ``[2, B, H, qtiles, ktiles + 2]``; the two
    halves swap roles (read / write) on every call.

    Args:
        threshold: negative log2 margin (default -6). A block is dropped for a
            wave when, for every row of the wave, its best score is more than
            |threshold| below that row's running max; a value further below
            zero drops fewer blocks.
        enable_skipping: when False, every call runs the dense forward.
        round_mode: bf16 output rounding, "rtna" (default), "rtne" or "rtz".
        layout: "bhsd" for [B,H,S,D] tensors, "bshd" for [B,S,H,D].
    """

    def __init__(self, threshold: float = -6.0, *, enable_skipping: bool = True, round_mode: str = "rtna",
                 layout: str = "bhsd"):
        if threshold >= 0:
            raise ValueError(f"threshold must be negative (log2 units); got {threshold}")
        if layout not in ("bhsd", "bshd"):
            raise ValueError(f"layout must be 'bhsd' or 'bshd' (got {layout!r})")
        self.threshold = float(threshold)
        self.enable_skipping = bool(enable_skipping)
        self.round_mode = round_mode
        self.layout = layout
        self._skip = None     # the list pair, allocated on first use
        self._phase = 0       # index of the half the next call reads
        self._key = None      # (list shape, device) the pair was made for

    @staticmethod
    def get_MN(head_dim=128, dtype=torch.bfloat16, v_colmajor=False):
        """(q rows per tile, K rows per block) that the lists index."""
        return KBLOCK_M, KBLOCK_N

    def reset_skip_state(self):
        """Forget the learned lists: the next call computes every block again."""
        self._skip = None
        self._phase = 0
        self._key = None

    def set_threshold(self, threshold: float):
        if threshold >= 0:
            raise ValueError("threshold must be negative (log2 units)")
        self.threshold = float(threshold)

    def enable_skip_optimization(self, enable: bool = True):
        self.enable_skipping = bool(enable)

    @property
    def read_list(self):
        """The half the next call will read (written by the last call)."""
        return None if self._skip is None else self._skip[self._phase]

    @property
    def write_list(self):
        """The half the next call will overwrite (read by the last call)."""
        return None if self._skip is None else self._skip[1 - self._phase]

    def _lists_for(self, q, k):
        key = (_list_shape(q, k, self.layout), q.device)
        if self._skip is None or self._key != key:
            B, H, qtiles, ktiles = key[0]
            pair = torch.zeros(2, B, H, qtiles, ktiles + 2, dtype=torch.int16, device=q.device)
            # Half 0 starts as one range covering blocks 0..ktiles-1, walked
            # ascending: the run-length row [2, ktiles - 1, -1].
            pair[0, ..., :3] = torch.tensor([2, ktiles - 1, -1], dtype=torch.int16)
            self._skip, self._phase, self._key = pair, 0, key
        return self._skip

    def __call__(self, q, k, v, *, out=None, must_do_list=None):
        return self.forward(q, k, v, out=out, must_do_list=must_do_list)

    def forward(self, q, k, v, *, out=None, must_do_list=None):
        """One denoising step. ``must_do_list``: optional int16
        ``[len, s0, e0, s1, e1, ...]`` of K-block ranges [s, e) that the next
        list keeps whatever the vote (attention sinks, for example)."""
        if not self.enable_skipping:
            return _kernel.forward(q, k, v, out=out, round_mode=self.round_mode, layout=self.layout)
        pair = self._lists_for(q, k)
        src = self._phase
        # The kernel walks the read list ascending in phase 1 and descending in
        # phase 0; the half just read becomes the next write target.
        self._phase = 1 - src
        return _kernel.forward_lite(q, k, v, pair[src], pair[1 - src], threshold=self.threshold, phase=self._phase,
                                    must_do_list=must_do_list, out=out, round_mode=self.round_mode,
                                    layout=self.layout)
