"""GPU tests of LiteAttention (forward_lite + LiteAttention + LPT order).

The reference's contracts (tests/test_attention.py:88-214), on this build's
256-row tiles and 32-row waves: the compute-all seed step on well-spread
inputs equals the dense forward (bit-identical here, once the oracle confirms
no wave drops a block; the reference checks against SDPA); the LPT order is
bit-identical to the plain order; a must_do list pinning every block
reproduces the compute-all step; the learned list keeps exactly the hot
blocks of each head. Beyond them: five LiteAttention steps on the reference's
peaked inputs, where the per-wave soft skip drops the cold blocks inside
every step, against the oracle at every step in two modes; single steps over
non-trivial read lists in both phases (output under the tolerance rule,
written rows exactly); and the LPT permutation against the oracle's,
including rows whose counts are far past the block count.
"""
import numpy as np
import pytest
import torch

import moonmath_attention as ma
from moonmath_attention import _lib
from oracle import attention as oa
from oracle import lite as ol
from helpers import aggregate_stats, bits, check_fractions, compare_bf16, f32, log_stats, randn_bf16, to_bhsd

pytestmark = pytest.mark.gpu
DEV = "cuda:0"

# Reference LITE_SHAPE (B=1, H=8, S=Skv=4096, D=128), 5 steps, threshold -3.
B, H, S = 1, 8, 4096
STEPS = 5
THR = -3.0


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    assert torch.cuda.is_available(), "GPU tests need an MI355X"


def _uniform(layout):
    q, k, v = (randn_bf16((B, S, H, 128), 7 + i) for i in range(3))
    if layout == "bhsd":
        q, k, v = (t.transpose(1, 2).contiguous() for t in (q, k, v))
    return q.to(DEV), k.to(DEV), v.to(DEV)


def _peaked():
    """Reference _lite_qkv_peaked: head h keeps K-blocks 0..h at scale 2, the
    rest damped to 0.05, so the vote drops the cold blocks per head."""
    g = torch.Generator().manual_seed(7)
    q, k, v = (torch.randn(B, S, H, 128, generator=g) for _ in range(3))
    scale = torch.full((H, S), 0.05)
    for h in range(H):
        scale[h, : (h + 1) * 64] = 2.0
    k = k * scale.t().view(1, S, H, 1)
    return tuple(t.to(torch.bfloat16).to(DEV) for t in (q, k, v))


def _run_lite(q, k, v, layout, steps, must_do=None):
    attn = ma.LiteAttention(threshold=THR, round_mode="rtna", layout=layout)
    out = None
    for _ in range(steps):
        out = attn(q, k, v, must_do_list=must_do)
    torch.cuda.synchronize()
    return out, attn


@pytest.mark.parametrize("layout", ["bhsd", "bshd"])
def test_lite_compute_all_equals_dense_forward(layout, monkeypatch):
    """The seed step is the dense forward without the tail KV-split (which
    lite never uses, as in the reference): bit-identical, and within the
    tolerance rule of the oracle (2 sampled heads)."""
    q, k, v = _uniform(layout)
    attn = ma.LiteAttention(threshold=THR, round_mode="rtna", layout=layout)
    lite = attn(q, k, v)
    monkeypatch.setenv("MOONMATH_NO_TAIL", "1")
    dense = ma.forward(q, k, v, round_mode="rtna", layout=layout)
    torch.cuda.synchronize()
    assert torch.equal(lite.view(torch.int16), dense.view(torch.int16))
    got = to_bhsd(bits(lite), layout)
    qb_, kb_ = (to_bhsd(f32(t), layout) for t in (q, k))
    nkb = S // 64
    for b, h in ((0, 0), (0, 5)):
        for t in range(S // 256):
            waves = ol.wave_blocks(qb_[b, h, 256 * t:256 * t + 256], kb_[b, h], ol.seed_row(nkb), 1, THR)
            assert all(kb == list(range(nkb)) for _, _, kb in waves), (b, h, t)
    stats = []
    for b, h in ((0, 0), (0, 5)):
        ref, _, scl, tie = oa.forward(f32(q), f32(k), f32(v), "rtna", layout=layout, heads=[(b, h)], aux=True)
        stats.append(compare_bf16(got[b, h], ref[b, h], scl[b, h], tie[b, h], fractions=False))
    agg = aggregate_stats(stats)
    log_stats(f"lite_compute_all_1x8x4096_{layout}_rtna", agg)
    check_fractions(agg)


@pytest.mark.parametrize("mode", ["rtna", "rtz"])
def test_lite_peaked_steps_match_oracle(mode):
    """Five LiteAttention steps on the reference's peaked inputs (head h: K
    blocks 0..h hot, the rest damped), phases 1, 0, 1, 0, 1. In the first
    (compute-all) step every wave drops the cold blocks it reaches after the
    hot ones, which carry most of the softmax mass, so the output is far from
    full attention; in descending steps the cold blocks walked before the hot
    ones are kept. At every step: every tile's output under the tolerance
    rule against the oracle's per-wave computation, and every written row
    exactly."""
    q, k, v = _peaked()
    nkb, nqb = S // 64, S // 256
    mcode = {"rtne": 0, "rtna": 1, "rtz": 2}[mode]
    qf, kf, vf = (to_bhsd(f32(t), "bshd") for t in (q, k, v))
    s32 = {(h, t): ol.scores(qf[0, h, 256 * t:256 * t + 256], kf[0, h]) for h in range(H) for t in range(nqb)}
    attn = ma.LiteAttention(threshold=THR, round_mode=mode, layout="bshd")
    rows = np.tile(ol.seed_row(nkb), (H, nqb, 1))
    dropped_in_step0 = 0
    for step in range(STEPS):
        phase = 1 - attn._phase
        out = attn(q, k, v)
        torch.cuda.synchronize()
        got = to_bhsd(bits(out), "bshd")
        written = attn.read_list.cpu().numpy()[0]
        stats = []
        for h in range(H):
            for t in range(nqb):
                r0 = 256 * t
                o, nxt, blocks = ol.step_tile(qf[0, h, r0:r0 + 256], kf[0, h], vf[0, h], rows[h, t], phase, THR, mcode,
                                              aux=True, s32=s32[h, t])
                assert list(written[h, t, :1 + nxt[0]]) == nxt, (step, h, t)
                ref, _, scl, tie = o
                stats.append(compare_bf16(got[0, h, r0:r0 + 256], ref, scl, tie, fractions=False))
                if step == 0:
                    waves = ol.wave_blocks(qf[0, h, r0:r0 + 256], kf[0, h], rows[h, t], phase, THR, s32=s32[h, t])
                    dropped_in_step0 += sum(len(kb) < nkb for _, _, kb in waves)
        agg = aggregate_stats(stats, names=[f"h{h}t{t}" for h in range(H) for t in range(nqb)])
        log_stats(f"lite_peaked_1x8x4096_step{step}_phase{phase}_{mode}", agg)
        check_fractions(agg)
        rows = written.copy()
    assert dropped_in_step0 == H * nqb * 8  # every wave dropped blocks inside the compute-all step


def test_lite_lpt_matches_plain_bitexact(monkeypatch):
    q, k, v = _peaked()
    monkeypatch.delenv("MOONMATH_LITE_PLAIN", raising=False)
    lpt, a1 = _run_lite(q, k, v, "bshd", STEPS)
    monkeypatch.setenv("MOONMATH_LITE_PLAIN", "1")
    plain, a2 = _run_lite(q, k, v, "bshd", STEPS)
    assert torch.equal(lpt.view(torch.int16), plain.view(torch.int16)), "LPT order changed the output"
    assert torch.equal(a1.read_list, a2.read_list)


def test_lite_lpt_full_rounds_match_plain_bitexact(monkeypatch):
    """800 CTAs (1 x 25 heads x 32 q-tiles): three full rounds of 256 grid
    slots, whose LPT positions are dealt to the XCDs in runs of 32 (reversed
    in odd rounds), and a partial fourth; four steps on inputs whose heads
    keep different numbers of blocks, so the order is not the plain one."""
    Bf, Hf, Sf = 1, 25, 8192
    g = torch.Generator().manual_seed(60)
    q, k, v = (torch.randn(Bf, Sf, Hf, 128, generator=g) for _ in range(3))
    scale = torch.full((Hf, Sf), 0.05)
    for h in range(Hf):  # head h: the first 4h + 1 K-blocks hot, the rest cold
        scale[h, : (4 * h + 1) * 64] = 2.0
    k = k * scale.t().view(1, Sf, Hf, 1)
    q, k, v = (t.to(torch.bfloat16).to(DEV) for t in (q, k, v))
    outs, lists = [], []
    for plain in (False, True):
        if plain:
            monkeypatch.setenv("MOONMATH_LITE_PLAIN", "1")
        else:
            monkeypatch.delenv("MOONMATH_LITE_PLAIN", raising=False)
        attn = ma.LiteAttention(threshold=-3.0, round_mode="rtne", layout="bshd")
        for _ in range(4):
            out = attn(q, k, v)
        torch.cuda.synchronize()
        outs.append(out)
        lists.append(attn.read_list.clone())
    kept = [ol.kept_count(r, Sf // 64) for r in lists[0].cpu().numpy().reshape(-1, Sf // 64 + 2)]
    assert len(set(kept)) > 8, "the order should not be trivial"
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16)), "LPT order changed the output"
    assert torch.equal(lists[0], lists[1])


def test_lite_must_do_all_equals_compute_all():
    q, k, v = _peaked()
    ktiles = S // 64
    must_do_all = torch.tensor([2, 0, ktiles], dtype=torch.int16, device=DEV)
    ref = ma.LiteAttention(threshold=THR, round_mode="rtna", layout="bshd")(q, k, v)
    forced, attn = _run_lite(q, k, v, "bshd", STEPS, must_do=must_do_all)
    assert torch.equal(forced.view(torch.int16), ref.view(torch.int16))
    kept = [ol.kept_count(attn.read_list[0, h, t].cpu().numpy(), ktiles) for h in range(H) for t in range(S // 256)]
    assert kept == [ktiles] * len(kept)


def test_lite_skip_list_develops():
    q, k, v = _peaked()
    ktiles = S // 64
    attn = ma.LiteAttention(threshold=THR, round_mode="rtna", layout="bshd")
    attn(q, k, v)
    torch.cuda.synchronize()
    assert ol.kept_count(attn.write_list[0, 0, 0].cpu().numpy(), ktiles) == ktiles  # the seed it read
    assert ol.kept_count(attn.read_list[0, 0, 0].cpu().numpy(), ktiles) < ktiles
    for _ in range(STEPS - 1):
        attn(q, k, v)
    torch.cuda.synchronize()
    kept_by_head = [ol.kept_count(attn.read_list[0, h, 0].cpu().numpy(), ktiles) for h in range(H)]
    assert kept_by_head == list(range(1, H + 1)), kept_by_head


def _random_rows(nrows, nkb, phase, seed):
    """Valid read rows as a writer in the other phase would produce them:
    random kept subsets (first block of the previous walk always kept)."""
    rng = np.random.default_rng(seed)
    rows = np.zeros((nrows, nkb + 2), np.int16)
    prev_phase = 1 - phase
    for i in range(nrows):
        blocks, ends = ol.decode(ol.seed_row(nkb), nkb, 1)
        if prev_phase == 0:
            blocks, ends = blocks[::-1], ends[::-1]
            ends = [False] * (nkb - 1) + [True]
        keep = [True] + [bool(x) for x in rng.random(nkb - 1) < rng.uniform(0.1, 0.9)]
        row = ol.emit(blocks, ends, keep, prev_phase, nkb)
        rows[i, :len(row)] = row
    return rows


def _lite_step_check(Bq, Hq, Sq, Skv, phase, mode, threshold, seed, row_seed, name):
    """One step over random valid read rows (BSHD): every tile's output under
    the tolerance rule, and every written row exactly. Returns the read rows."""
    nqb, nkb = -(-Sq // 256), -(-Skv // 64)
    q, k, v = (randn_bf16((Bq, s, Hq, 128), seed + i) for i, s in enumerate((Sq, Skv, Skv)))
    rows = _random_rows(Bq * Hq * nqb, nkb, phase, seed=row_seed)
    read = torch.from_numpy(rows).view(Bq, Hq, nqb, nkb + 2).to(DEV)
    write = torch.full_like(read, -7)
    out = ma.forward_lite(q.to(DEV), k.to(DEV), v.to(DEV), read, write, threshold=threshold, phase=phase,
                          round_mode=mode, layout="bshd")
    torch.cuda.synchronize()
    got_rows = write.cpu().numpy().reshape(-1, nkb + 2)
    got = to_bhsd(bits(out), "bshd")
    qf, kf, vf = (to_bhsd(f32(t), "bshd") for t in (q, k, v))
    stats = []
    for w in range(Bq * Hq * nqb):
        bh, t = divmod(w, nqb)
        b, h = divmod(bh, Hq)
        r0, r1 = t * 256, min(Sq, (t + 1) * 256)
        o, nxt, blocks = ol.step_tile(qf[b, h, r0:r1], kf[b, h], vf[b, h], rows[w], phase, threshold,
                                      {"rtne": 0, "rtna": 1, "rtz": 2}[mode], aux=True)
        assert list(got_rows[w, :1 + nxt[0]]) == nxt, (w, blocks)
        ref, _, scl, tie = o
        stats.append(compare_bf16(got[b, h, r0:r1], ref, scl, tie, fractions=False))
    agg = aggregate_stats(stats, names=[f"b{w // nqb // Hq}h{w // nqb % Hq}t{w % nqb}" for w in range(Bq * Hq * nqb)])
    log_stats(name, agg)
    check_fractions(agg)
    return rows, nkb


@pytest.mark.parametrize("phase", [1, 0])
@pytest.mark.parametrize("mode", ["rtna", "rtz"])
def test_lite_step_matches_oracle(phase, mode):
    """One step over random valid read rows (ragged Sq / Skv, BSHD): output of
    every tile under the tolerance rule, and every written row exactly."""
    rows, nkb = _lite_step_check(2, 3, 700, 1500, phase, mode, -6.0, 90, phase * 10 + len(mode),
                                 f"lite_step_2x3_sq700_skv1500_phase{phase}_{mode}")
    assert any(len(ol.decode(r, nkb, phase)[0]) < nkb for r in rows)


def _random_lite_cases(n, seed):
    rng = np.random.default_rng(seed)
    return [(int(rng.integers(1, 3)), int(rng.integers(1, 3)), int(rng.integers(8, 900)), int(rng.integers(1, 2500)),
             int(rng.integers(0, 2)), str(rng.choice(["rtne", "rtna", "rtz"])), float(rng.choice([-8.0, -3.0, 0.0])))
            for _ in range(n)]


@pytest.mark.parametrize("case", _random_lite_cases(6, 2026), ids=lambda c: "b{}h{}_sq{}_skv{}_ph{}_{}_t{}".format(*c))
def test_lite_random_shapes_match_oracle(case):
    """Seeded random shapes, phases, round modes and thresholds for one step."""
    Bq, Hq, Sq, Skv, phase, mode, thr = case
    _lite_step_check(Bq, Hq, Sq, Skv, phase, mode, thr, Sq + Skv, Sq * 3 + Skv,
                     "lite_random_{}x{}_sq{}_skv{}_ph{}_{}_t{}".format(*case))


def _lpt_rows(kind, nrows, nkb):
    rng = np.random.default_rng(5)
    if kind == "mixed":
        # Written rows of many ranges (up to nkb + 1 entries), plus rows whose
        # length is negative, odd, or past nkb + 1 (clamped).
        rows = _random_rows(nrows, nkb, 1, seed=11)
        rows[0, 0] = -3
        rows[1, :] = rng.integers(-1, nkb, nkb + 2)
        rows[1, 0] = nkb + 5
        rows[2, :8] = (7, 40, 3, 9, 1, 30, 12, 20)
        rows[3, :] = rng.integers(-1, nkb, nkb + 2)
        rows[3, 0] = 20
        return rows
    rows = np.zeros((nrows, nkb + 2), np.int16)
    for i in range(nrows):
        kept = int(rng.integers(1, nkb + 1))
        rows[i, :3] = (2, kept - 1, -1)
    return rows


def _extreme_rows(nrows, nkb):
    """Rows whose pair sums are far past nkb (alternating int16 extremes over
    the whole row: a count near 2^28), next to ordinary and empty rows."""
    rows = np.zeros((nrows, nkb + 2), np.int16)
    rows[0, 0] = nkb + 1
    rows[0, 1:] = np.where(np.arange(nkb + 1) % 2 == 0, 32767, -32768)
    rows[1, :3] = (2, 9, -1)
    rows[2, :3] = (2, nkb - 1, -1)
    rows[3, 0] = -5
    for i in range(4, nrows):
        rows[i] = rows[i % 4]
    return rows


@pytest.mark.parametrize("kind", ["counts", "mixed", "extreme2048", "extreme8192"])
def test_lite_lpt_order_matches_oracle(kind):
    """The planning kernel's CTA permutation (through the C ABI) against the
    oracle's stable heaviest-first order, on rows of very different weights
    (one range each, or many ranges and out-of-range lengths, or counts of
    ~2^28 at 2048 and 8192 blocks, whose bucket product would overflow int32
    without the clamp)."""
    Bq, Hq, Sq, Skv = 1, 6, 1024, 4096
    if kind.startswith("extreme"):
        Hq, Skv = 1, 64 * int(kind[len("extreme"):])
    nqb, nkb = Sq // 256, Skv // 64
    rows = _extreme_rows(Bq * Hq * nqb, nkb) if kind.startswith("extreme") else _lpt_rows(kind, Bq * Hq * nqb, nkb)
    assert kind == "counts" or max(int(r[0]) for r in rows) > 9
    q, k, v = (randn_bf16((Bq, s, Hq, 128), 50 + i).to(DEV) for i, s in enumerate((Sq, Skv, Skv)))
    vt = torch.empty(_lib.lib.moonmath_attention_vt_bytes(Bq, Hq, Skv) // 2, dtype=torch.bfloat16, device=DEV)
    st = _lib.stream_ptr(DEV)
    assert _lib.lib.launch_v_transpose_rtne(_lib.ptr(v), _lib.ptr(vt), Bq * Hq * Skv, Skv, Hq, 1, st) == 0
    read = torch.from_numpy(rows).to(DEV)
    write = torch.zeros_like(read)
    out = torch.empty_like(q)
    ws = torch.full((_lib.lib.lite_workspace_bytes_rtne(Bq, Hq, Sq) // 4,), -1, dtype=torch.int32, device=DEV)
    rc = _lib.lib.launch_attention_forward_lite_rtne(
        _lib.ptr(q), _lib.ptr(k), _lib.ptr(vt), _lib.ptr(out), Bq, Hq, Sq, Skv, 128, _lib.ptr(read),
        _lib.ptr(write), None, -6.0, 1, 1, _lib.ptr(ws), st)
    torch.cuda.synchronize()
    assert rc == 0
    assert ws.cpu().tolist()[:Bq * Hq * nqb] == ol.lpt_order(rows, nkb)


@pytest.mark.parametrize("layout", ["bhsd", "bshd"])
def test_lite_vote_rounds_product_and_difference_separately(layout):
    """Every row's block maxima are 4 (block 0) and 3.9375 (block 1); at
    threshold fl(fl(3.9375 c) - fl(4 c)) the oracle drops block 1, where a
    fused multiply-subtract would keep it. One ulp lower, block 1 is kept."""
    c = np.float32(oa.SCALE_LOG2E)
    thr = np.float32(np.float32(3.9375) * c - np.float32(4.0) * c)
    Sq, Skv = 256, 128
    q = torch.zeros(1, Sq, 1, 128)
    q[..., 0] = 1.0
    k = torch.zeros(1, Skv, 1, 128)
    k[:, :64, :, 0] = 4.0
    k[:, 64:, :, 0] = 3.9375
    v = randn_bf16((1, Skv, 1, 128), 31).float()
    if layout == "bhsd":
        q, k, v = (t.transpose(1, 2).contiguous() for t in (q, k, v))
    q, k, v = (t.to(torch.bfloat16).to(DEV) for t in (q, k, v))
    s = np.array([[4.0] * 64 + [3.9375] * 64] * Sq, np.float32)
    for t, expect in ((thr, [True, False]), (np.nextafter(thr, np.float32(-1)), [True, True])):
        assert ol.votes(s, [0, 1], Skv, float(t)) == expect
        read = torch.from_numpy(ol.seed_row(2)).view(1, 1, 1, 4).to(DEV)
        write = torch.full_like(read, -7)
        ma.forward_lite(q, k, v, read, write, threshold=float(t), phase=1, round_mode="rtna", layout=layout)
        torch.cuda.synchronize()
        want = ol.emit([0, 1], [False, True], expect, 1, 2)
        assert write.cpu().view(-1).tolist()[:1 + want[0]] == want, (float(t), expect)


def test_forward_lite_rejects_bad_lists():
    q, k, v = _uniform("bhsd")
    nqb, nkb = S // 256, S // 64
    good = torch.zeros(B, H, nqb, nkb + 2, dtype=torch.int16, device=DEV)
    with pytest.raises(ValueError, match="int16"):
        ma.forward_lite(q, k, v, good.int(), good, threshold=-3.0, phase=1)
    with pytest.raises(ValueError, match="at least"):
        ma.forward_lite(q, k, v, good[..., :-1].contiguous(), good, threshold=-3.0, phase=1)
    with pytest.raises(ValueError, match="same device"):
        ma.forward_lite(q, k, v, good, good.cpu(), threshold=-3.0, phase=1)
    short = torch.tensor([4, 0, 5], dtype=torch.int16, device=DEV)
    with pytest.raises(ValueError, match="must_do_list"):
        ma.forward_lite(q, k, v, good, good.clone(), threshold=-3.0, phase=1, must_do_list=short)
