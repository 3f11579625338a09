"""Benchmark: bf16 attention forward (headline) and fp8-KV MLA decode on one MI355X.

Prints ONE JSON line. ``value`` is the attention forward throughput in TFLOP/s
(4*B*H*Sq*Skv*D per call, the reference's formula benchmark/runner.py:7,174)
at configs[1]: BSHD (B=2, S=8192, H=24, D=128), round mode RTNE, inputs resident
in HBM; one step = one ``moonmath_attention.forward`` call (V transpose +
forward kernel, as the reference times it, benchmark/runner.py:176-181).

``roofline`` is for the dominant kernel (the attention forward kernel alone,
timed with HIP events on the stream it is launched on); its ``traffic`` (HBM
bytes per launch) comes from two rocprofv3 counter passes (FETCH_SIZE, then
WRITE_SIZE, each scaled by what the counter reads for a 1 GiB device copy)
that bench.py runs over this same build in child processes (``traffic_pass``
says how; ``--no-traffic`` skips them and falls back to the committed profile
figure). ``passes`` keys give the median of 5 further timing passes beside the
mean (the reference reports medians of 5 passes, benchmark/bench_table.py:50-55).
``cpu_baseline`` times
the reference repo's CPU oracle formula (examples/basic.py:16-17) over the
whole headline workload on this host's cores (median of 3). Extra keys:
``attention`` (the configs[0] tiny case, every round mode, the reference
benchmark's "realistic" inputs, the configs[3] long shapes, a shape whose tail
KV-split fires, with and without the split, the configs[2] cross-attention
shapes; each leg other than the headline's modes carries a ``cpu`` figure of
the same formula on its own input bits, the whole leg or a stated subset of
heads and rows; and the reference's other published shapes, README.md:96-124,
as RTNE legs beside its MI300X times), ``lite`` and ``mla`` (configs[4] decode
lines with their own CPU baseline, the reference test's fp32 formula).
"""
import argparse
import glob
import json
import os
import pathlib
import shutil
import signal
import subprocess
import sys
import tempfile
import time

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "amd-kernels_amd"))

PEAK_BF16_TFLOPS = 2516.6  # MI355X dense bf16 MFMA (256 CU x 2.4 GHz x 4096 flop/clk)
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E


def _log(msg):
    print(msg, file=sys.stderr, flush=True)


def attention_flops(B, H, Sq, Skv, D=128):
    return 4.0 * B * H * Sq * Skv * D


# Seconds of back-to-back work before each timed region, so clocks have settled
# (measured on MI355X: after only a few ms of warmup the MLA decode timed 10-15%
# slower than in steady state).
WARM_S = 0.25


def _warm(torch, fn, calls):
    """Run fn(i) at least `calls` times and until WARM_S seconds have passed."""
    t0 = time.perf_counter()
    i = 0
    while i < calls or time.perf_counter() - t0 < WARM_S:
        fn(i)
        i += 1
        if i % 16 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()


def _time(torch, fn, steps, warmup):
    """Mean ms per call of fn(i) over `steps` calls after warmup, HIP events on
    torch's current stream (the stream every launcher here is given)."""
    _warm(torch, fn, warmup)
    st = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for i in range(steps):
        fn(i)
    e1.record(st)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def _passes(torch, fn, iters, passes=5):
    """Per-pass mean ms of `passes` further timing passes of `iters` calls each
    (no warmup between them: the caller has just timed fn), and their median."""
    ms = sorted(_time(torch, fn, iters, 0) for _ in range(passes))
    return {"median_ms": round(ms[len(ms) // 2], 4), "passes": len(ms), "iters": iters,
            "min_ms": round(ms[0], 4), "max_ms": round(ms[-1], 4)}


def _headline_inputs(torch):
    """configs[1] inputs, N(0,1) bf16 drawn on the CPU from seed 42 (the CPU
    baseline runs on the same bits)."""
    B, S, H = 2, 8192, 24
    g = torch.Generator().manual_seed(42)
    return tuple(torch.randn(B, S, H, 128, generator=g).to(torch.bfloat16) for _ in range(3))


def bench_attention(args, torch, ma, _lib, qkv_cpu):
    B, S, H = 2, 8192, 24
    mode = args.mode
    q, k, v = (t.to("cuda:0") for t in qkv_cpu)
    out = torch.empty_like(q)
    flops = attention_flops(B, H, S, S)
    t0 = time.perf_counter()
    ms = _time(torch, lambda i: ma.forward(q, k, v, out=out, round_mode=mode, layout="bshd"), args.steps,
               args.warmup)
    wall = time.perf_counter() - t0
    med = _passes(torch, lambda i: ma.forward(q, k, v, out=out, round_mode=mode, layout="bshd"), args.steps)

    # Dominant kernel alone: forward kernel over a pre-transposed V_t, events on
    # the launch stream (torch's current stream, passed to the C ABI).
    vt = torch.empty(_lib.lib.moonmath_attention_vt_bytes(B, H, S) // 2, dtype=torch.bfloat16, device="cuda:0")
    sp = _lib.stream_ptr(q.device)
    rc = getattr(_lib.lib, f"launch_v_transpose_{mode}")(_lib.ptr(v), _lib.ptr(vt), B * H * S, S, H, 1, sp)
    assert rc == 0, rc
    fwd = getattr(_lib.lib, f"launch_attention_forward_{mode}")
    rcs = []
    kms = _time(torch, lambda i: rcs.append(fwd(_lib.ptr(q), _lib.ptr(k), _lib.ptr(vt), _lib.ptr(out), B, H, S, S,
                                                128, 1, None, sp)), max(args.steps, 5), 2)
    assert set(rcs) == {0}, set(rcs)
    achieved = flops / (kms * 1e-3) / 1e12
    # No nested counter passes from a leg run or from inside a profiler.
    under_prof = any(k.startswith("ROCPROF") for k in os.environ)
    tpass = None if (args.no_traffic or args.only or under_prof) else measure_traffic(mode)
    traffic = tpass.get("hbm_bytes_per_launch") if tpass else None
    if traffic is None:
        tfile = ROOT / "profiles" / "attn_fwd_traffic.json"
        if tfile.exists():
            traffic = json.loads(tfile.read_text()).get("hbm_bytes_per_launch")
            tpass = dict(tpass or {}, source=str(tfile.relative_to(ROOT)), measured=False)
    return {
        "ms": ms,
        "value": flops / (ms * 1e-3) / 1e12,
        "wall_s": wall,
        "passes": med,
        "traffic_pass": tpass,
        "kernel_ms": kms,
        "roofline": {
            "bound": "mfma",
            "achieved": round(achieved, 2),
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
            "traffic": traffic,
        },
    }


def run_traffic_workload(torch, _lib, mode):
    """The workload of a counter pass (``--only traffic``): three 1 GiB device
    copies (the counters' calibration: 1048576 KiB read and written each), then
    four launches of the headline forward kernel over a pre-transposed V_t."""
    n = 1 << 30
    src = torch.ones(n, dtype=torch.uint8, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    B, S, H = 2, 8192, 24
    q, k, v = (t.to("cuda:0") for t in _headline_inputs(torch))
    out = torch.empty_like(q)
    vt = torch.empty(_lib.lib.moonmath_attention_vt_bytes(B, H, S) // 2, dtype=torch.bfloat16, device="cuda:0")
    sp = _lib.stream_ptr(q.device)
    assert getattr(_lib.lib, f"launch_v_transpose_{mode}")(_lib.ptr(v), _lib.ptr(vt), B * H * S, S, H, 1, sp) == 0
    fwd = getattr(_lib.lib, f"launch_attention_forward_{mode}")
    for _ in range(4):
        assert fwd(_lib.ptr(q), _lib.ptr(k), _lib.ptr(vt), _lib.ptr(out), B, H, S, S, 128, 1, None, sp) == 0
    torch.cuda.synchronize()
    _log("bench: traffic workload done")


def _counter_pass(counter, mode, timeout_s=180):
    """Per-dispatch values of `counter` (KiB) for the copy kernel and the
    attention forward kernel, from one rocprofv3 pass over ``--only traffic``;
    the first dispatch of each kernel is dropped. None when rocprofv3 is absent
    or the pass fails."""
    rp = shutil.which("rocprofv3") or "/opt/rocm/bin/rocprofv3"
    if not os.path.exists(rp):
        return None, "rocprofv3 not found"
    out = tempfile.mkdtemp(prefix="mm_traffic_")
    cmd = [rp, "--kernel-trace", "--pmc", counter, "--output-format", "csv", "-d", out, "-o", "c", "--",
           sys.executable, str(pathlib.Path(__file__).resolve()), "--only", "traffic", "--mode", mode]
    env = dict(os.environ, TMPDIR=os.environ.get("TMPDIR", "/tmp"))
    try:
        proc = subprocess.Popen(cmd, stdout=subprocess.DEVNULL, stderr=subprocess.PIPE, env=env,
                                start_new_session=True)
        try:
            _, err = proc.communicate(timeout=timeout_s)
        except subprocess.TimeoutExpired:
            os.killpg(proc.pid, signal.SIGKILL)
            proc.communicate()
            return None, f"{counter} pass timed out after {timeout_s} s"
        files = glob.glob(os.path.join(out, "**", "*counter_collection.csv"), recursive=True)
        if not files:
            tail = err.decode(errors="replace").strip().splitlines()[-3:]
            return None, f"{counter} pass wrote no counters (rc {proc.returncode}): {' | '.join(tail)}"
        import csv

        vals = {}
        with open(files[0]) as f:
            for row in csv.DictReader(f):
                if row["Counter_Name"] != counter:
                    continue
                name = row["Kernel_Name"]
                key = "copy" if "copyBuffer" in name else ("attn" if "attn_fwd_kernel" in name else None)
                if key:
                    vals.setdefault(key, []).append(float(row["Counter_Value"]))
        if "copy" not in vals or "attn" not in vals:
            return None, f"{counter} pass: kernels missing from the counters ({sorted(vals)})"
        avg = {k: sum(v[1:]) / len(v[1:]) if len(v) > 1 else v[0] for k, v in vals.items()}
        avg["dispatches"] = {k: len(v) for k, v in vals.items()}
        return avg, None
    finally:
        shutil.rmtree(out, ignore_errors=True)


def measure_traffic(mode):
    """HBM bytes per launch of the headline forward kernel, measured now on
    this build: FETCH_SIZE and WRITE_SIZE (KiB per dispatch), each times its
    scale, 1048576 KiB over what the counter reads for the 1 GiB copy (FETCH
    2.000, WRITE 1.000 on MI355X)."""
    res = {"measured": True, "counters": "rocprofv3 --kernel-trace --pmc FETCH_SIZE | WRITE_SIZE, one pass each",
           "workload": "bench.py --only traffic (3 x 1 GiB copy, 4 x forward kernel)"}
    got = {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        avg, err = _counter_pass(counter, mode)
        if avg is None:
            _log(f"bench: traffic pass unavailable: {err}")
            return {"measured": False, "error": err}
        factor = avg["copy"] / 1048576.0
        got[counter] = {"kib_per_dispatch": round(avg["attn"], 1), "copy_kib": round(avg["copy"], 1),
                        "scale": round(1.0 / factor, 4), "bytes": avg["attn"] * 1024.0 / factor,
                        "dispatches": avg["dispatches"]}
    total = got["FETCH_SIZE"]["bytes"] + got["WRITE_SIZE"]["bytes"]
    alg = 4 * 2 * 8192 * 24 * 128 * 2  # Q, K, V_t read + O written, bf16
    res.update(fetch=got["FETCH_SIZE"], write=got["WRITE_SIZE"], hbm_bytes_per_launch=int(round(total)),
               algorithmic_bytes=alg, ratio=round(total / alg, 4))
    _log(f"bench: traffic {total / 2**20:.1f} MiB per launch ({total / alg:.3f}x algorithmic)")
    return res


# The reference's published MI300X times (README.md:96-124), other hardware:
# context for the extra legs, not a baseline of this metric.
REF_MI300X_MS = {
    ("headline", "rtne"): 3.083, ("headline", "rtna"): 3.022, ("headline", "rtz"): 2.983,
    ("1x32x16384", "rtne"): 8.013, ("2x8x86016", "rtne"): 101.071,
    ("2x24x16384", "rtne"): 11.670, ("4x16x16384", "rtne"): 15.591, ("1x64x16384", "rtne"): 15.528,
    ("2x24x32768", "rtne"): 46.002, ("2x16x65536", "rtne"): 117.612, ("1x16x131072", "rtne"): 232.517,
}
# Shapes (B, H, S) of the reference's table not benched elsewhere in this file.
PUBLISHED_SHAPES = ((2, 24, 16384), (4, 16, 16384), (1, 64, 16384), (2, 24, 32768), (2, 16, 65536),
                    (1, 16, 131072))


def _leg(name, B, H, Sq, Skv, ms, **extra):
    tf = attention_flops(B, H, Sq, Skv) / (ms * 1e-3) / 1e12
    rec = {"shape_bshd": [B, Sq, H, 128], "skv": Skv, "ms": round(ms, 4), "tflops": round(tf, 1),
           "pct_bf16_peak": round(100 * tf / PEAK_BF16_TFLOPS, 2)}
    rec.update(extra)
    _log(f"bench: attention {name}: {ms:.3f} ms, {tf:.0f} TFLOP/s")
    return rec


def bench_attention_extra(args, torch, ma, qkv_cpu):
    """Other round modes, the reference benchmark's input pattern, the long
    configs, the tail KV-split and the cross-attention configs (one `forward`
    call per step, as the headline)."""
    sys.path.insert(0, str(ROOT / "tests"))
    from helpers import realistic_bf16

    res = {}
    cpu = not args.no_cpu_baseline
    # the tiny BHSD case (1, 2, 256, 128), RTNE.
    g0 = torch.Generator().manual_seed(42)
    tq, tk, tv = (torch.randn(1, 2, 256, 128, generator=g0).to(torch.bfloat16) for _ in range(3))
    gq, gk, gv = (t.to("cuda:0") for t in (tq, tk, tv))
    ms = _time(torch, lambda i: ma.forward(gq, gk, gv, round_mode="rtne", layout="bhsd"), args.steps, args.warmup)
    res["tiny_1x2x256_bhsd_rtne"] = _leg("tiny 1x2x256 bhsd", 1, 2, 256, 256, ms, round_mode="rtne", layout="bhsd")
    if cpu:
        res["tiny_1x2x256_bhsd_rtne"]["cpu"] = cpu_attention(
            torch, tq.transpose(1, 2), tk.transpose(1, 2), tv.transpose(1, 2))
    del gq, gk, gv
    q, k, v = (t.to("cuda:0") for t in qkv_cpu)
    out = torch.empty_like(q)
    for mode in ("rtne", "rtna", "rtz"):
        fn = (lambda i: ma.forward(q, k, v, out=out, round_mode=mode, layout="bshd"))
        ms = _time(torch, fn, args.steps, args.warmup)
        res[f"headline_{mode}"] = _leg(f"headline {mode}", 2, 24, 8192, 8192, ms, round_mode=mode,
                                       ref_mi300x_ms=REF_MI300X_MS[("headline", mode)],
                                       median5=_passes(torch, fn, args.steps))
    qr, kr, vr = (t.to("cuda:0") for t in realistic_bf16(2, 8192, 24, seed=42))
    ms = _time(torch, lambda i: ma.forward(qr, kr, vr, out=out, round_mode="rtne", layout="bshd"), args.steps,
               args.warmup)
    res["headline_realistic_rtne"] = _leg("headline realistic rtne", 2, 24, 8192, 8192, ms, round_mode="rtne",
                                          inputs="log-normal K row norms (reference benchmark/runner.py:34-47)")
    del q, k, v, qr, kr, vr, out
    g = torch.Generator(device="cuda:0")
    for B, H, S, steps in ((1, 32, 16384, args.steps), (2, 8, 86016, max(3, args.steps // 6))):
        g.manual_seed(61)
        q, k, v = (torch.randn(B, S, H, 128, generator=g, device="cuda:0").to(torch.bfloat16) for _ in range(3))
        o = torch.empty_like(q)
        ms = _time(torch, lambda i: ma.forward(q, k, v, out=o, round_mode="rtne", layout="bshd"), steps, 2)
        key = f"{B}x{H}x{S}"
        res[f"long_{key}_rtne"] = _leg(f"long {key} rtne", B, H, S, S, ms, round_mode="rtne",
                                       ref_mi300x_ms=REF_MI300X_MS[(key, "rtne")])
        if cpu:
            # One head; for the 86016-token shape its first 8192 q rows.
            rows = S if S <= 16384 else 8192
            res[f"long_{key}_rtne"]["cpu"] = cpu_attention(
                torch, q[:1, :rows, :1].cpu(), k[:1, :, :1].cpu(), v[:1, :, :1].cpu())
            res[f"long_{key}_rtne"]["cpu"]["sample"] = f"1 of {B * H} heads x {rows} of {S} q rows"
        del q, k, v, o
    # The reference's other published shapes (README.md:96-124), RTNE: the mean
    # of a timed region, then the median of 5 passes (about 0.3 s each) as the
    # reference reports; CPU on one head's first 2048 q rows.
    for B, H, S in PUBLISHED_SHAPES:
        g.manual_seed(71)
        q, k, v = (torch.randn(B, S, H, 128, generator=g, device="cuda:0").to(torch.bfloat16) for _ in range(3))
        o = torch.empty_like(q)
        fn = (lambda i: ma.forward(q, k, v, out=o, round_mode="rtne", layout="bshd"))
        est_ms = attention_flops(B, H, S, S) / 1.1e12 * 1e3
        iters = max(2, min(args.steps, int(300 / est_ms)))
        ms = _time(torch, fn, iters, 2)
        key = f"{B}x{H}x{S}"
        res[f"published_{key}_rtne"] = _leg(f"published {key} rtne", B, H, S, S, ms, round_mode="rtne",
                                            ref_mi300x_ms=REF_MI300X_MS[(key, "rtne")],
                                            median5=_passes(torch, fn, iters))
        if cpu:
            res[f"published_{key}_rtne"]["cpu"] = cpu_attention(
                torch, q[:1, :2048, :1].cpu(), k[:1, :, :1].cpu(), v[:1, :, :1].cpu())
            res[f"published_{key}_rtne"]["cpu"]["sample"] = f"1 of {B * H} heads x 2048 of {S} q rows"
        del q, k, v, o
    # A shape whose last round of CTAs the tail planner splits: 17 q-blocks x 48
    # heads = 816 CTAs = 3 rounds of 256 + a 48-CTA tail.
    B, H, Sq, Skv = 2, 24, 4097, 8192
    g.manual_seed(17)
    q = torch.randn(B, Sq, H, 128, generator=g, device="cuda:0").to(torch.bfloat16)
    k, v = (torch.randn(B, Skv, H, 128, generator=g, device="cuda:0").to(torch.bfloat16) for _ in range(2))
    o = torch.empty_like(q)
    for label, env in (("split", None), ("no_split", "1")):
        if env:
            os.environ["MOONMATH_NO_TAIL"] = env
        try:
            ms = _time(torch, lambda i: ma.forward(q, k, v, out=o, round_mode="rtne", layout="bshd"), args.steps,
                       args.warmup)
        finally:
            os.environ.pop("MOONMATH_NO_TAIL", None)
        res[f"tail_{label}_2x24_sq4097_skv8192_rtne"] = _leg(f"tail {label}", B, H, Sq, Skv, ms, round_mode="rtne")
    if cpu:
        res["tail_split_2x24_sq4097_skv8192_rtne"]["cpu"] = cpu_attention(
            torch, q.cpu(), k.cpu(), v.cpu(), heads=[(0, h) for h in range(8)])
    del q, k, v, o
    # cross-attention, Q ~ N(0,1), K/V ~ 0.5 N(0,1). Short KV ranges
    # make these shapes partly HBM-bound (Q in, O out), so the leg also reports
    # the algorithmic bytes (q, k, v, out once) per second.
    for Sq, Skv in ((8192, 512), (8192, 77), (4097, 512)):
        g.manual_seed(23)
        q = torch.randn(2, Sq, 24, 128, generator=g, device="cuda:0").to(torch.bfloat16)
        k, v = ((0.5 * torch.randn(2, Skv, 24, 128, generator=g, device="cuda:0")).to(torch.bfloat16) for _ in range(2))
        o = torch.empty_like(q)
        ms = _time(torch, lambda i: ma.forward(q, k, v, out=o, round_mode="rtne", layout="bshd"), args.steps,
                   args.warmup)
        nbytes = 2 * 24 * 128 * 2 * (2 * Sq + 2 * Skv)
        res[f"cross_2x24_sq{Sq}_skv{Skv}_rtne"] = _leg(
            f"cross sq{Sq} skv{Skv}", 2, 24, Sq, Skv, ms, round_mode="rtne", hbm_bytes=nbytes,
            hbm_GBs=round(nbytes / (ms * 1e-3) / 1e9, 1))
        if cpu:
            res[f"cross_2x24_sq{Sq}_skv{Skv}_rtne"]["cpu"] = cpu_attention(torch, q.cpu(), k.cpu(), v.cpu())
        del q, k, v, o
    return res


def bench_lite(args, torch, ma, qkv_cpu):
    """LiteAttention steps at the headline shape (RTNA, the class default):
    the compute-all seed list, and read lists keeping the first block and a
    seeded 25% of the others per 256-row tile (heaviest-first CTA order).
    One step = one forward_lite call (V transpose + lite kernel + LPT plan)."""
    import numpy as np

    B, S, H = 2, 8192, 24
    q, k, v = (t.to("cuda:0") for t in qkv_cpu)
    out = torch.empty_like(q)
    nqb, nkb = S // 256, S // 64
    res = {}
    rng = np.random.default_rng(9)
    for label, frac in (("compute_all", 1.0), ("keep_25pct", 0.25)):
        rows = np.zeros((B * H * nqb, nkb + 2), np.int16)
        kept_total = 0
        for i in range(len(rows)):
            keep = np.concatenate([[True], rng.random(nkb - 1) < frac]) if frac < 1 else np.ones(nkb, bool)
            # runs of kept blocks written as a phase-0 list, read ascending in phase 1
            runs, b0 = [], None
            for b in range(nkb):
                if keep[b] and b0 is None:
                    b0 = b
                if (not keep[b] or b == nkb - 1) and b0 is not None:
                    runs.append((b0, b if not keep[b] else nkb))
                    b0 = None
            vals = []
            for lo, hi in reversed(runs):
                vals += [hi - 1, lo - 1]
            rows[i, 0] = len(vals)
            rows[i, 1:1 + len(vals)] = vals
            kept_total += int(keep.sum())
        read = torch.from_numpy(rows).to("cuda:0")
        write = torch.empty_like(read)
        ms = _time(torch, lambda i: ma.forward_lite(q, k, v, read, write, threshold=-6.0, phase=1, out=out,
                                                    round_mode="rtna", layout="bshd"), args.steps, args.warmup)
        frac_kept = kept_total / (B * H * nqb * nkb)
        eff = attention_flops(B, H, S, S) * frac_kept / (ms * 1e-3) / 1e12
        res[label] = {"ms": round(ms, 4), "kept_fraction": round(frac_kept, 4),
                      "tflops_on_kept_blocks": round(eff, 1)}
        _log(f"bench: lite {label}: {ms:.3f} ms, kept {frac_kept:.3f}, {eff:.0f} TFLOP/s on kept blocks")
    return res


def bench_mla(torch, ma, steps, warmup, configs=((128, 1), (128, 2), (16, 1)), cpu=True):
    """B=64 absorbed-MLA paged decode, ctx ~ U[1024, 8192], 64-token
    pages over a randomly permuted pool, OCP e4m3fn KV, scale 1/sqrt(192).
    Three independent (Q, pool, table) sets rotate so the ~640 MB working set
    exceeds the 256 MB Infinity Cache: each timed call streams its KV from HBM.
    With ``cpu``, each config also times the reference test's fp32 formula over
    the same 64 requests on the host (median of 3)."""
    sys.path.insert(0, str(ROOT / "tests"))
    from mla_inputs import KV_SCALE, SCALE_192, paged_pool, ragged_lens, rand_q

    B = 64
    lens = ragged_lens(B, 1024, 8192, seed=5)
    sum_l = sum(lens)
    n_blocks = sum(-(-l // 64) for l in lens)
    results = []
    sets, cpu_sets = [], []
    for r in range(3):
        pool, idx, indptr = paged_pool(lens, 100 + r)
        cpu_sets.append((pool, idx, indptr))
        sets.append((pool.to("cuda:0"), idx.to("cuda:0"), indptr.to("cuda:0")))
    lens_t = torch.tensor(lens, dtype=torch.int32, device="cuda:0")
    for H, q_len in configs:
        qs, qs_cpu = [], []
        for r in range(3):
            q_lat, q_pe = rand_q(B, q_len, H, 200 + r, peak=1.0)
            qs_cpu.append((q_lat, q_pe))
            o = torch.empty(B, q_len, H, 512, dtype=torch.bfloat16, device="cuda:0")
            qs.append((q_lat.to("cuda:0"), q_pe.to("cuda:0"), o))
        parts = ma.mla_decode_a16w8_plan_parts_q(B, 8192, q_len, H)

        def call(r):
            pool, idx, indptr = sets[r % 3]
            q_lat, q_pe, o = qs[r % 3]
            ma.mla_decode_a16w8_multiq_paged_dev(q_lat, q_pe, pool, o, lens_t, None, idx, indptr, parts,
                                                 SCALE_192, KV_SCALE) if q_len > 1 else \
                ma.mla_decode_a16w8_paged_dev(q_lat[:, 0], q_pe[:, 0], pool, o[:, 0], lens_t, None, idx, indptr,
                                              parts, SCALE_192, KV_SCALE)

        us = _time(torch, call, steps, warmup) * 1e3
        med = _passes(torch, call, steps)
        # Algorithmic bytes: KV once + Q in + O out + block tables and lengths.
        nbytes = sum_l * 576 + B * q_len * H * (576 + 512) * 2 + 4 * (n_blocks + B)
        flops = 2.0 * (576 + 512) * H * q_len * sum_l
        gbs = nbytes / (us * 1e-6) / 1e9
        tfs = flops / (us * 1e-6) / 1e12
        rec = {
            "B": B, "H": H, "q_len": q_len, "parts": parts, "us": round(us, 2),
            "hbm_GBs": round(gbs, 1), "pct_hbm_peak": round(100 * gbs / PEAK_HBM_GBS, 2),
            "mfma_TFLOPs": round(tfs, 1), "pct_bf16_peak": round(100 * tfs / PEAK_BF16_TFLOPS, 2),
            "bytes": nbytes, "median5_us": round(med["median_ms"] * 1e3, 2),
        }
        _log(f"bench: mla H={H} q_len={q_len}: {us:.1f} us (median of 5 passes {med['median_ms'] * 1e3:.1f}), "
             f"{gbs:.0f} GB/s, {tfs:.0f} TFLOP/s")
        if cpu:
            rec["cpu_baseline"] = mla_cpu_baseline(torch, qs_cpu[0], cpu_sets[0], lens, nbytes, flops)
        results.append(rec)
    # The fp8 KV producer filling the whole batch's cache: every token of the
    # 64 requests quantised from bf16 latent / rope into its pool slot
    # (HBM-bound: 1152 B read + 576 B written + 4 B of slot per token).
    g = torch.Generator(device="cuda:0").manual_seed(6)
    c_kv = torch.randn(sum_l, 512, generator=g, device="cuda:0").to(torch.bfloat16)
    k_pe = torch.randn(sum_l, 64, generator=g, device="cuda:0").to(torch.bfloat16)
    pool, idx, _ = sets[0]
    us = _time(torch, lambda i: ma.mla_kv_quantize(c_kv, k_pe, pool, idx, KV_SCALE), steps, warmup) * 1e3
    qbytes = sum_l * (1152 + 576 + 4)
    qgbs = qbytes / (us * 1e-6) / 1e9
    producer = {"tokens": sum_l, "us": round(us, 2), "bytes": qbytes, "hbm_GBs": round(qgbs, 1),
                "pct_hbm_peak": round(100 * qgbs / PEAK_HBM_GBS, 2), "kv_scale": KV_SCALE}
    _log(f"bench: mla kv producer {sum_l} tokens: {us:.1f} us, {qgbs:.0f} GB/s")
    return {
        "metric": "MLA decode HBM GB/s (% peak)",
        "workload": "B=64 ctx~U[1024,8192] (seed 5) 64-token pages, fp8 e4m3fn KV, 3 rotating pools",
        "sum_ctx": sum_l,
        "configs": results,
        "kv_producer": producer,
    }


def _cpu_threads():
    """Host threads for the CPU baselines: every core of this process's
    affinity, within the CPU share the GPU box gives one GPU's jobs
    (OMP_NUM_THREADS there)."""
    aff = len(os.sched_getaffinity(0))
    share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    return (min(aff, share) if share > 0 else aff), aff


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _median3(fn):
    ts = []
    for _ in range(3):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return sorted(ts)[1]


def mla_cpu_baseline(torch, q_cpu, set_cpu, lens, nbytes, flops):
    """The reference test's fp32 decode formula (tests/test_mla_decode.py:50-66)
    with OCP e4m3fn dequant, over all 64 requests of one (Q, pool) set."""
    from oracle.mla import torch_formula_cpu
    from mla_inputs import KV_SCALE, SCALE_192

    threads, aff = _cpu_threads()
    torch.set_num_threads(threads)
    q_lat, q_pe = q_cpu
    pool, idx, indptr = set_cpu
    lens_t = torch.tensor(lens, dtype=torch.int32)
    t = _median3(lambda: torch_formula_cpu(q_lat, q_pe, pool, lens_t, idx, indptr, SCALE_192, KV_SCALE))
    return {"value": round(nbytes / t / 1e9, 2), "unit": "GB/s", "tflops": round(flops / t / 1e12, 4),
            "ms": round(t * 1e3, 1), "cores": threads, "kind": "port",
            "sample": "all 64 requests, one (Q, pool) set, median of 3 runs"}


def cpu_attention(torch, q, k, v, heads=None, rows=None):
    """The same CPU formula as cpu_baseline on a leg's own input bits (BSHD CPU
    tensors): every (b, h) head and q row by default, or a stated subset
    (`heads` (b, h) pairs, the first `rows` q rows), whose rate stands for the
    whole leg (heads and rows are independent); median of 3 runs."""
    threads, aff = _cpu_threads()
    torch.set_num_threads(threads)
    from oracle.attention import torch_formula_cpu

    B, Sq, H, _ = q.shape
    Skv = k.shape[1]
    hs = heads if heads is not None else [(b, h) for b in range(B) for h in range(H)]
    r = rows if rows is not None else Sq

    def run():
        for b, h in hs:
            torch_formula_cpu(q[b:b + 1, :r, h].unsqueeze(1), k[b:b + 1, :, h].unsqueeze(1),
                              v[b:b + 1, :, h].unsqueeze(1))

    t = _median3(run)
    flops = 4.0 * len(hs) * r * Skv * 128
    whole = len(hs) == B * H and r == Sq
    return {"value": round(flops / t / 1e12, 4), "unit": "TFLOP/s", "ms": round(t * 1e3, 2), "cores": threads,
            "kind": "port",
            "sample": "whole leg" if whole else f"{len(hs)} of {B * H} heads x {r} of {Sq} q rows ({flops:.3g} flop)"}


def cpu_baseline(torch, qkv_cpu):
    """The reference's CPU oracle formula (examples/basic.py:16-17), fp32 torch on
    this host, over the whole headline workload (48 (b, h) heads, one at a time
    to bound memory), on the same input bits as the GPU run; median of 3 runs."""
    threads, aff = _cpu_threads()
    torch.set_num_threads(threads)
    from oracle.attention import torch_formula_cpu

    q, k, v = qkv_cpu
    B, S, H, _ = q.shape

    def run():
        for b in range(B):
            for h in range(H):
                torch_formula_cpu(q[b:b + 1, :, h].unsqueeze(1), k[b:b + 1, :, h].unsqueeze(1),
                                  v[b:b + 1, :, h].unsqueeze(1))

    t = _median3(run)
    flops = attention_flops(B, H, S, S)
    return {
        "value": round(flops / t / 1e12, 4),
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "cpu_model": _cpu_model(),
        "sample": f"the whole (2,24,8192,128) headline workload, fp32 torch softmax(q@k^T/sqrt(128))@v one (b,h) "
                  f"head at a time, median of 3 runs ({t:.2f} s each); {threads} threads "
                  f"(this process's affinity: {aff} cores)",
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--mode", default="rtne", choices=["rtne", "rtna", "rtz"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-mla", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="skip the extra attention legs")
    ap.add_argument("--no-traffic", action="store_true",
                    help="skip the rocprofv3 counter passes behind roofline.traffic")
    ap.add_argument("--only", choices=["attention", "mla", "copy", "traffic"], default=None,
                    help="run one leg only (for rocprofv3 counter passes); 'copy' runs a plain "
                         "1 GiB device copy used to calibrate FETCH_SIZE / WRITE_SIZE; 'traffic' "
                         "the workload of bench.py's own counter passes")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)

    import torch

    import moonmath_attention as ma
    from moonmath_attention import _lib

    assert torch.cuda.is_available(), "bench.py needs the GPU"
    if args.only == "copy":
        n = 1 << 30
        src = torch.ones(n, dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        _log(f"bench: copied {n} bytes x3 (calibration)")
        return
    if args.only == "traffic":
        run_traffic_workload(torch, _lib, args.mode)
        return
    if args.only == "mla":
        print(json.dumps(bench_mla(torch, ma, args.steps, args.warmup, cpu=False)), flush=True)
        return
    _log("bench: attention headline (2,8192,24,128) bshd")
    qkv_cpu = _headline_inputs(torch)
    att = bench_attention(args, torch, ma, _lib, qkv_cpu)
    _log(f"bench: attention {att['value']:.1f} TFLOP/s, kernel {att['kernel_ms']:.3f} ms")
    if args.only == "attention":
        print(json.dumps({"attention_tflops": att["value"], "kernel_ms": att["kernel_ms"],
                          "traffic": att["roofline"]["traffic"]}), flush=True)
        return
    extra = None if args.no_extra else bench_attention_extra(args, torch, ma, qkv_cpu)
    lite = None if args.no_extra else bench_lite(args, torch, ma, qkv_cpu)
    mla = None
    if not args.no_mla:
        _log("bench: mla decode")
        mla = bench_mla(torch, ma, args.steps, args.warmup, cpu=not args.no_cpu_baseline)
    cpu = None
    if not args.no_cpu_baseline:
        _log("bench: cpu baseline")
        cpu = cpu_baseline(torch, qkv_cpu)
    line = {
        "metric": "attn fwd TFLOP/s (% bf16 MFMA peak); MLA decode HBM GB/s (% peak)",
        "value": round(att["value"], 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(att["ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "attention forward BSHD B=2 S=8192 H=24 D=128 (configs[1])",
            "round_mode": args.mode,
            "pct_bf16_peak": round(100 * att["value"] / PEAK_BF16_TFLOPS, 2),
        },
        "roofline": att["roofline"],
        "cpu_baseline": cpu,
        "passes": att["passes"],
        "traffic_pass": att["traffic_pass"],
    }
    if extra is not None:
        line["attention"] = extra
    if lite is not None:
        line["lite"] = lite
    if mla is not None:
        line["mla"] = mla
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
