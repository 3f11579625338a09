"""Benchmark: bf16 attention forward (headline) and fp8-KV MLA decode on one MI355X.

Prints ONE JSON line. ``value`` is the attention forward throughput in TFLOP/s
(4*B*H*Sq*Skv*D per call, the reference's formula benchmark/runner.py:7,174)
at configs[1]: BSHD (B=2, S=8192, H=24, D=128), round mode RTNE, inputs resident
in HBM; one step = one ``moonmath_attention.forward`` call (V transpose +
forward kernel, as the reference times it, benchmark/runner.py:176-181).

``roofline`` is for the dominant kernel (the attention forward kernel alone,
timed with HIP events on the stream it is launched on). ``cpu_baseline`` times
the reference repo's CPU oracle formula (examples/basic.py:16-17) on a bounded
sample of heads on this host's cores. ``mla`` carries the MLA decode line
(HBM GB/s) when the MLA kernel is built.
"""
import argparse
import json
import os
import pathlib
import sys
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


def bench_attention(args, torch, ma, _lib):
    B, S, H = 2, 8192, 24
    mode = args.mode
    g = torch.Generator().manual_seed(42)
    q, k, v = (torch.randn(B, S, H, 128, generator=g).to(torch.bfloat16).to("cuda:0") for _ in range(3))
    out = torch.empty_like(q)
    _warm(torch, lambda i: ma.forward(q, k, v, out=out, round_mode=mode, layout="bshd"), args.warmup)
    st = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(st)
    for _ in range(args.steps):
        ma.forward(q, k, v, out=out, round_mode=mode, layout="bshd")
    e1.record(st)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_time(e1) / args.steps
    flops = attention_flops(B, H, S, S)

    # Dominant kernel alone: forward kernel over a pre-transposed V_t, events on
    # the launch stream (torch's current stream, passed to the C ABI).
    vt = torch.empty(_lib.lib.moonmath_attention_vt_bytes(B, H, S) // 2, dtype=torch.bfloat16, device="cuda:0")
    sp = _lib.stream_ptr(q.device)
    rc = getattr(_lib.lib, f"launch_v_transpose_{mode}")(_lib.ptr(v), _lib.ptr(vt), B * H * S, S, H, 1, sp)
    assert rc == 0, rc
    fwd = getattr(_lib.lib, f"launch_attention_forward_{mode}")
    reps = max(args.steps, 5)
    for _ in range(2):
        fwd(_lib.ptr(q), _lib.ptr(k), _lib.ptr(vt), _lib.ptr(out), B, H, S, S, 128, 1, None, sp)
    k0, k1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    k0.record(st)
    for _ in range(reps):
        rc = fwd(_lib.ptr(q), _lib.ptr(k), _lib.ptr(vt), _lib.ptr(out), B, H, S, S, 128, 1, None, sp)
    k1.record(st)
    torch.cuda.synchronize()
    assert rc == 0, rc
    kms = k0.elapsed_time(k1) / reps
    achieved = flops / (kms * 1e-3) / 1e12
    traffic = None
    tfile = ROOT / "profiles" / "attn_fwd_traffic.json"
    if tfile.exists():
        traffic = json.loads(tfile.read_text()).get("hbm_bytes_per_launch")
    return {
        "ms": ms,
        "value": flops / (ms * 1e-3) / 1e12,
        "wall_s": wall,
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


def bench_mla(torch, ma, steps, warmup, configs=((128, 1), (128, 2), (16, 1))):
    """B=64 absorbed-MLA paged decode, ctx ~ U[1024, 8192], 64-token
    pages over a randomly permuted pool, OCP e4m3fn KV, scale 1/sqrt(192).
    Three independent (Q, pool, table) sets rotate so the ~640 MB working set
    exceeds the 256 MB Infinity Cache: each timed call streams its KV from HBM."""
    sys.path.insert(0, str(ROOT / "tests"))
    from mla_inputs import KV_SCALE, SCALE_192, paged_pool, ragged_lens, rand_q

    B = 64
    lens = ragged_lens(B, 1024, 8192, seed=5)
    sum_l = sum(lens)
    n_blocks = sum(-(-l // 64) for l in lens)
    results = []
    sets = []
    for r in range(3):
        pool, idx, indptr = paged_pool(lens, 100 + r)
        sets.append((pool.to("cuda:0"), idx.to("cuda:0"), indptr.to("cuda:0")))
    lens_t = torch.tensor(lens, dtype=torch.int32, device="cuda:0")
    for H, q_len in configs:
        qs = []
        for r in range(3):
            q_lat, q_pe = rand_q(B, q_len, H, 200 + r, peak=1.0)
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

        _warm(torch, call, warmup)
        st = torch.cuda.current_stream()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(st)
        for r in range(steps):
            call(r)
        e1.record(st)
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / steps
        # Algorithmic bytes: KV once + Q in + O out + block tables and lengths.
        nbytes = sum_l * 576 + B * q_len * H * (576 + 512) * 2 + 4 * (n_blocks + B)
        flops = 2.0 * (576 + 512) * H * q_len * sum_l
        gbs = nbytes / (us * 1e-6) / 1e9
        tfs = flops / (us * 1e-6) / 1e12
        results.append({
            "B": B, "H": H, "q_len": q_len, "parts": parts, "us": round(us, 2),
            "hbm_GBs": round(gbs, 1), "pct_hbm_peak": round(100 * gbs / PEAK_HBM_GBS, 2),
            "mfma_TFLOPs": round(tfs, 1), "pct_bf16_peak": round(100 * tfs / PEAK_BF16_TFLOPS, 2),
            "bytes": nbytes,
        })
        _log(f"bench: mla H={H} q_len={q_len}: {us:.1f} us, {gbs:.0f} GB/s, {tfs:.0f} TFLOP/s")
    return {
        "metric": "MLA decode HBM GB/s (% peak)",
        "workload": "B=64 ctx~U[1024,8192] (seed 5) 64-token pages, fp8 e4m3fn KV, 3 rotating pools",
        "sum_ctx": sum_l,
        "configs": results,
    }


def cpu_baseline(torch, budget_s):
    """The reference's CPU oracle formula, fp32 torch on this host, one head at a
    time of the headline shape (S=8192), until ~budget_s seconds have elapsed."""
    cores = min(len(os.sched_getaffinity(0)), 16)
    torch.set_num_threads(cores)
    from oracle.attention import torch_formula_cpu

    g = torch.Generator().manual_seed(42)
    S = 8192
    done, t_total = 0, 0.0
    while t_total < budget_s and done < 480:
        q, k, v = (torch.randn(1, 1, S, 128, generator=g).to(torch.bfloat16) for _ in range(3))
        t0 = time.perf_counter()
        torch_formula_cpu(q, k, v)
        t_total += time.perf_counter() - t0
        done += 1
    flops = attention_flops(1, done, S, S)
    return {
        "value": round(flops / t_total / 1e12, 4),
        "unit": "TFLOP/s",
        "cores": cores,
        "kind": "port",
        "sample": f"{done} heads (each one (b,h) slice) of the (2,24,8192,128) headline shape, fp32 torch "
                  f"softmax(q@k^T/sqrt(128))@v per head, {t_total:.1f} s",
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--mode", default="rtne", choices=["rtne", "rtna", "rtz"])
    ap.add_argument("--cpu-budget", type=float, default=12.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-mla", action="store_true")
    ap.add_argument("--only", choices=["attention", "mla", "copy"], default=None,
                    help="run one leg only (for rocprofv3 counter passes); 'copy' runs a plain "
                         "1 GiB device copy used to calibrate FETCH_SIZE / WRITE_SIZE")
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
    if args.only == "mla":
        print(json.dumps(bench_mla(torch, ma, args.steps, args.warmup)), flush=True)
        return
    _log("bench: attention headline (2,8192,24,128) bshd")
    att = bench_attention(args, torch, ma, _lib)
    _log(f"bench: attention {att['value']:.1f} TFLOP/s, kernel {att['kernel_ms']:.3f} ms")
    if args.only == "attention":
        print(json.dumps({"attention_tflops": att["value"], "kernel_ms": att["kernel_ms"]}), flush=True)
        return
    mla = None
    if not args.no_mla:
        _log("bench: mla decode")
        mla = bench_mla(torch, ma, args.steps, args.warmup)
    cpu = None
    if not args.no_cpu_baseline:
        _log("bench: cpu baseline")
        cpu = cpu_baseline(torch, args.cpu_budget)
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
    }
    if mla is not None:
        line["mla"] = mla
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
