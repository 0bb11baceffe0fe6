"""Benchmark of the MI355X dense-contraction provider (one GPU).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-sweep]

A step is one Gemm launch of the headline workload, config 2's largest shape
(M, K, N) = (4096, 4096, 11008) in f16 with a row bias, operands resident in
HBM.  Before the W warm-up steps the same launch runs back to back for
--settle-ms (100 ms) of wall time: an idle GPU needs that long under load to
leave its idle clock, and the timed steps are meant to see the settled one.  The JSON line reports whole-job TFLOP/s for that step, the roofline of
the kernel (its average duration measured with HIP events on the stream it is
launched on), the reference-algorithm CPU baseline on a bounded row sample,
and a sweep over every configured workload (configs 1-3 of BASELINE.json).
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "conv/GEMM TFLOP/s & int8 TOPS (% MFMA peak); end-to-end ms/forward"
PEAK_TFLOPS = {"f16": 2500.0, "bf16": 2500.0, "f32": 157.3, "int8": 5000.0}
HBM_GBPS = 8000.0
HEADLINE = (4096, 4096, 11008)
# host threads this process may run on (the CPU baselines state how many they used)
HOST_CORES = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
GEMM_SWEEP = [(1, 25088, 512), (128, 768, 3072), (2048, 4096, 4096), (4096, 4096, 11008)]


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=100)
    p.add_argument("--warmup", type=int, default=30)
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--no-sweep", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=20.0)
    p.add_argument("--settle-ms", type=float, default=100.0,
                   help="GPU time of headline launches run before the warm-up steps, so that the timed "
                        "steps see the clock the GPU settles at under this load, not its idle ramp")
    p.add_argument("--e2e-fused-only", action="store_true",
                   help="end-to-end items: skip the reference-fusions-only forwards (a kernel trace then holds "
                        "only the provider's fused graph)")
    p.add_argument("--only", default="", help="run one item (for profiling): 'headline', 'copy', "
                   "'conv_f32_cfg1', 'int8_ffn', 'matmul_integer_i32', or a sweep item such as "
                   "'gemm_f16_2048x4096x4096'")
    p.add_argument("--trace-stats", default="", metavar="CSV",
                   help="summarise a rocprofv3 kernel_trace.csv or counter_collection.csv per (kernel, grid) "
                        "instead of benchmarking")
    p.add_argument("--trace-last", type=int, default=0,
                   help="with --trace-stats: also average each group's last N dispatches (the timed steps)")
    p.add_argument("--trace-forward", default="", metavar="MARK",
                   help="with --trace-stats on a kernel trace: a markdown table of kernel time per forward over "
                        "the last --trace-last forwards, a forward being the dispatches between two launches of "
                        "the kernel whose name contains MARK (one launch per forward)")
    return p.parse_args()


def trace_stats(path, last):
    """Per (full kernel name, grid size): dispatch count and average duration
    (kernel traces), or the average of each counter (counter collections)."""
    import csv
    import re
    rows = list(csv.DictReader(open(path)))
    groups = {}
    for r in rows:
        name = re.sub(r"\s+", " ", r["Kernel_Name"])
        grid = r.get("Grid_Size") or r.get("Grid_Size_X") or ""
        groups.setdefault((name, grid), []).append(r)
    for (name, grid), rs in groups.items():
        if "Counter_Name" in rs[0]:
            ctr = {}
            for r in rs:
                ctr.setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
            print(f"kernel {name}\n  grid {grid}")
            for c, v in ctr.items():
                print(f"  {c:36s} dispatches {len(v):4d}  avg {sum(v) / len(v):.6g}")
            continue
        rs.sort(key=lambda r: int(r["Start_Timestamp"]))
        d = [(int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3 for r in rs]
        line = f"dispatches {len(d):5d}  avg {sum(d) / len(d):9.2f} us  min {min(d):9.2f} us"
        if last and len(d) >= last:
            line += f"  last {last}: avg {sum(d[-last:]) / last:9.2f} us"
        print(f"kernel {name}\n  grid {grid}  {line}")


def trace_forward(path, mark, last):
    """Kernel time per forward over the last `last` forwards of a kernel
    trace: the dispatches after the (F - last)-th launch of the marker
    kernel up to and including the last one, F = the marker's launches."""
    import csv
    import re
    rows = sorted(csv.DictReader(open(path)), key=lambda r: int(r["Start_Timestamp"]))
    names = [re.sub(r"\s+", " ", r["Kernel_Name"]) for r in rows]
    idx = [i for i, n in enumerate(names) if mark in n]
    last = min(last or len(idx) - 1, len(idx) - 1)
    if last < 1:
        raise SystemExit(f"--trace-forward: fewer than two launches of a kernel matching {mark!r}")
    per = {}
    for i in range(idx[-last - 1] + 1, idx[-1] + 1):
        d = (int(rows[i]["End_Timestamp"]) - int(rows[i]["Start_Timestamp"])) / 1e3
        key = (names[i], rows[i].get("Grid_Size") or rows[i].get("Grid_Size_X") or "")
        per.setdefault(key, []).append(d)
    total = sum(sum(v) for v in per.values()) / last
    print(f"forwards in the trace: {len(idx)}; the last {last}: {total:.1f} us of kernel time per forward\n")
    print("| kernel | grid | calls per forward | us per call | us per forward | % |")
    print("|---|---|---|---|---|---|")
    for (name, grid), v in sorted(per.items(), key=lambda kv: -sum(kv[1])):
        pf = sum(v) / last
        print(f"| `{name}` | {grid} | {len(v) / last:.1f} | {sum(v) / len(v):.2f} | {pf:.1f} | {100 * pf / total:.1f} |")


def settle_clock(torch, fn, ms):
    """Runs fn back to back until `ms` of wall time have passed (an idle
    MI355X takes some 10-20 ms of load to leave its idle clock); returns the
    wall ms spent.  Not part of the timed region."""
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < ms:
        for _ in range(4):
            fn()
        torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3


def time_launches(torch, stream, fn, iters, warmup):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(iters):
        fn()
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / iters  # ms per launch


def time_graph(torch, ctx, L, fn, launches=20, reps=10):
    """ms per launch of fn replayed from a HIP graph of `launches` launches
    (launch overhead out of the figure).  fn runs once eagerly first, so its
    workspace comes from the context's pool during the capture."""
    import ctypes
    lib = L.lib()
    fn()
    torch.cuda.synchronize()
    L.check(lib.ohip_graph_begin(ctx.h))
    for _ in range(launches):
        fn()
    g = ctypes.c_void_p()
    L.check(lib.ohip_graph_end(ctx.h, ctypes.byref(g)))
    try:
        for _ in range(3):
            L.check(lib.ohip_graph_launch(g))
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            L.check(lib.ohip_graph_launch(g))
        L.check(lib.ohip_sync(ctx.h))
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3 / (reps * launches)
    finally:
        lib.ohip_graph_destroy(g)


def gemm_setup(torch, ctx, L, m, k, n, dtype, rng):
    a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    b = rng.normal(0, 1 / np.sqrt(k), (k, n)).astype(np.float32)
    c = rng.normal(0, 0.01, n).astype(np.float32)
    tdt = {L.F32: torch.float32, L.F16: torch.float16, L.BF16: torch.bfloat16}[dtype]
    w = ctx.weight_gemm(b, dtype=dtype, name=f"B_{m}_{k}_{n}_{dtype}", label="Gemm.B")
    at = torch.from_numpy(a).cuda().to(tdt)
    ct = torch.from_numpy(c).cuda().to(tdt)
    y = torch.empty((m, n), dtype=tdt, device="cuda")
    return a, b, c, w, at, ct, y


def load_traffic(name):
    """HBM bytes per launch from a committed rocprofv3 --pmc summary, if any."""
    path = os.path.join(ROOT, "profiles", f"{name}_pmc.txt")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch:"):
            return float(line.split(":", 1)[1])
    return None


def cpu_baseline_f16(seconds):
    """The reference's f16 Gemm algorithm (math_typed.rs:589-634, restated in C
    with the same per-element order) on a bounded row sample of the headline
    shape, single-threaded like the reference."""
    from oracle import oracle as O
    m, k, n = HEADLINE
    rng = np.random.default_rng(7)
    b = O.f32_to_half_bits(rng.normal(0, 1 / np.sqrt(k), (k, n)).astype(np.float32))
    c = O.f32_to_half_bits(rng.normal(0, 0.01, n).astype(np.float32))
    # per-row and per-call costs from a 1-row and a 4-row call (each call
    # also converts the operands: a fixed cost)
    a4 = O.f32_to_half_bits(rng.uniform(-1, 1, (4, k)).astype(np.float32))
    O.gemm_half(a4, b, c, rows=(0, 1))   # first call: library load, page faults
    t0 = time.perf_counter()
    O.gemm_half(a4, b, c, rows=(0, 1))
    t1 = time.perf_counter() - t0
    t0 = time.perf_counter()
    O.gemm_half(a4, b, c, rows=(0, 4))
    t4 = time.perf_counter() - t0
    per_row = max((t4 - t1) / 3, 1e-6)
    seconds = max(seconds - (t1 - per_row), per_row)
    # as many rows as fill the requested CPU time (the sample is a row band)
    rows = int(max(1, min(m, seconds / max(per_row, 1e-6))))
    a = O.f32_to_half_bits(rng.uniform(-1, 1, (rows, k)).astype(np.float32))
    t0 = time.perf_counter()
    O.gemm_half(a, b, c, rows=(0, rows))
    dt = time.perf_counter() - t0
    flops = 2.0 * rows * k * n
    return {"value": flops / dt / 1e12, "unit": "TFLOP/s", "cores": 1, "host_cores": HOST_CORES, "kind": "port",
            "sample": f"{rows} of {m} output rows of the f16 Gemm ({rows}x{k}x{n}), {dt:.2f} s; "
                      f"full forward extrapolates to {dt * m / rows:.0f} s; the restatement runs the "
                      f"reference's per-element order (ascending k, f32 accumulate, no FMA) as an i-p-j "
                      f"loop over contiguous B rows, faster than the reference's i-j-k loop that strides "
                      f"B by n (math_typed.rs:612-629), so this baseline flatters the CPU"}


def main():
    args = parse()
    if args.trace_stats:
        if args.trace_forward:
            trace_forward(args.trace_stats, args.trace_forward, args.trace_last)
        else:
            trace_stats(args.trace_stats, args.trace_last)
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; how the path would shard across GPUs "
                                   "is a design note, not a measured path", "n_gpus": args.gpus}))
        sys.exit(2)
    import torch
    from oxionnx_amd import _lib as L
    from oxionnx_amd.device import HipContext

    torch.cuda.set_device(0)
    if args.only == "copy":
        # calibration for the FETCH_SIZE / WRITE_SIZE counters: a plain device
        # copy of 256 MiB (reads 256 MiB, writes 256 MiB), five times
        src = torch.empty(64 * 1024 * 1024, dtype=torch.float32, device="cuda").fill_(1.0)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": src.numel() * 4, "launches": 5}))
        return
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        ctx = HipContext(0)   # adopts `stream`: events below are recorded on it
    rng = np.random.default_rng(2024)
    extras = {}

    with torch.cuda.stream(stream):
        m, k, n = HEADLINE
        _, _, _, w, at, ct, y = gemm_setup(torch, ctx, L, m, k, n, L.F16, rng)
        step = lambda: ctx.gemm(at, w, ct, out=y)
        steps = args.steps if args.only in ("", "headline") else 0   # profiling another item
        settled = settle_clock(torch, step, args.settle_ms) if steps else 0.0
        for _ in range(args.warmup if steps else 0):
            step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev0.record(stream)
        for _ in range(steps):
            step()
        ev1.record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        ms = ev0.elapsed_time(ev1) / max(steps, 1) if steps else float("nan")
        flops = 2.0 * m * k * n
        tflops = flops / (ms * 1e-3) / 1e12
        alg_bytes = 2 * (m * k + k * n + m * n) + 2 * n
        traffic = load_traffic("gemm_f16_4096x4096x11008")

        if not args.no_sweep and args.only != "headline":
            sweep = []
            for (mm, kk, nn) in GEMM_SWEEP:
                for dt, name in ((L.F32, "f32"), (L.F16, "f16")):
                    if args.only and args.only != f"gemm_{name}_{mm}x{kk}x{nn}":
                        continue
                    _, _, _, ww, aa, cc, yy = gemm_setup(torch, ctx, L, mm, kk, nn, dt, rng)
                    iters = 200 if mm * kk * nn < 1e9 else 30
                    fn = lambda: ctx.gemm(aa, ww, cc, out=yy)   # noqa: E731
                    if mm * kk * nn >= 1e10:
                        settle_clock(torch, fn, 50.0)   # the large shapes at the settled clock, as the headline
                    t = time_launches(torch, stream, fn, iters, 3)
                    eb = 4 if dt == L.F32 else 2
                    fl = 2.0 * mm * kk * nn
                    by = eb * (mm * kk + kk * nn + mm * nn + nn)
                    entry = {"shape": [mm, kk, nn], "dtype": name, "ms": round(t, 5),
                             "tflops": round(fl / t / 1e9, 2),
                             "frac_mfma": round(fl / t / 1e9 / PEAK_TFLOPS[name], 4),
                             "gbps": round(by / t / 1e6, 1),
                             "frac_hbm": round(by / t / 1e6 / HBM_GBPS, 4)}
                    if mm * kk * nn < 1e9:
                        # the launch-bound shapes also replayed from a HIP graph
                        tg = time_graph(torch, ctx, L, fn)
                        entry.update({"ms_graph": round(tg, 5), "gbps_graph": round(by / tg / 1e6, 1),
                                      "frac_hbm_graph": round(by / tg / 1e6 / HBM_GBPS, 4)})
                    sweep.append(entry)
                    del ww, aa, cc, yy
            extras["gemm_sweep"] = sweep
            extras.update(bench_conv(torch, ctx, L, stream, rng, args.only))
            extras.update(bench_int8(torch, ctx, L, stream, rng, args.only))
            extras.update(bench_large(torch, ctx, L, stream, rng, args.only))
            extras.update(bench_widened(torch, ctx, L, stream, rng, args.only))
            extras.update(bench_e2e(torch, ctx, stream, args.only, args.no_cpu, args.e2e_fused_only))
            extras.update(bench_gate(torch, ctx, L, args.only))

    line = {
        "metric": METRIC, "value": round(tflops, 2), "unit": "TFLOP/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f16",
        "data": "synthetic (seeded numpy; A~U(-1,1), B~N(0,1/sqrt(K)) initializer, bias~N(0,0.01))",
        "config": {"workload": "config 2: Gemm f16 (M,K,N)=(4096,4096,11008) + row bias, B resident",
                   "M": m, "K": k, "N": n, "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": PEAK_TFLOPS["f16"],
                     "unit": "TFLOP/s", "frac": round(tflops / PEAK_TFLOPS["f16"], 4),
                     "traffic": traffic, "algorithmic_bytes": alg_bytes,
                     "kernel": "mfma_gemm_kernel<Op::F16, Tile<256,256,2,4,2,8,3>, DenseRowsWhole, DenseRowsWhole, FloatEpi<_Float16>, false, false>"},
        "wall_s_timed_region": round(wall, 3),
        "settle_ms_before_warmup": round(settled, 1),
        "clock_note": "value is measured at the settled clock: the same launch runs back to back for "
                      "settle_ms_before_warmup before the warm-up steps (an idle MI355X needs 10-20 ms of load "
                      "to leave its idle clock); the sweep's large shapes settle 50 ms each the same way",
    }
    if not args.no_cpu and not args.only:
        line["cpu_baseline"] = cpu_baseline_f16(args.cpu_seconds)
    line.update(extras)
    print(json.dumps(line))
    ctx.close()


def bench_conv(torch, ctx, L, stream, rng, only):
    """Config 1: single Conv f32 NCHW [1,64,128,128] * [64,64,3,3] + bias + fused Relu."""
    if only and only != "conv_f32_cfg1":
        return {}
    x = rng.uniform(-1, 1, (1, 64, 128, 128)).astype(np.float32)
    wgt = rng.normal(0, 0.05, (64, 64, 3, 3)).astype(np.float32)
    b = rng.normal(0, 0.01, 64).astype(np.float32)
    w = ctx.weight_conv(wgt, name="conv1.W", label="Conv.W")
    xt = torch.from_numpy(x).cuda()
    bt = torch.from_numpy(b).cuda()
    y = torch.empty((1, 64, 128, 128), dtype=torch.float32, device="cuda")
    fc = lambda: ctx.conv2d(xt, w, bt, pads=(1, 1, 1, 1), act=L.ACT_RELU, out=y)   # noqa: E731
    settle_clock(torch, fc, 50.0)
    t = time_launches(torch, stream, fc, 100, 5)
    fl = 2.0 * 64 * 128 * 128 * 64 * 9
    return {"conv_cfg1_f32": {"ms": round(t, 5), "tflops": round(fl / t / 1e9, 2),
                              "frac_mfma": round(fl / t / 1e9 / PEAK_TFLOPS["f32"], 4),
                              "note": "NCHW input and output as the ONNX node has them (no layout staging is needed on this path)"}}


def bench_int8(torch, ctx, L, stream, rng, only):
    """Config 3: QLinearMatMul BERT-base FFN pair + MatMulInteger, each after
    50 ms of its own load (the settled clock)."""
    if only and only not in ("int8_ffn", "matmul_integer_i32"):
        return {}
    out = {}
    a = rng.integers(0, 256, (4096, 768)).astype(np.uint8)
    b1 = rng.integers(-127, 128, (768, 3072)).astype(np.int8)
    b2 = rng.integers(-127, 128, (3072, 768)).astype(np.int8)
    s1 = rng.uniform(0.001, 0.01, 3072).astype(np.float32)
    s2 = rng.uniform(0.001, 0.01, 768).astype(np.float32)
    w1 = ctx.weight_qgemm(b1, zp=0, scale=s1, name="ffn1.B")
    w2 = ctx.weight_qgemm(b2, zp=0, scale=s2, name="ffn2.B")
    at = torch.from_numpy(a).cuda()
    h = torch.empty((4096, 3072), dtype=torch.uint8, device="cuda")
    y = torch.empty((4096, 768), dtype=torch.uint8, device="cuda")
    yi = torch.empty((4096, 3072), dtype=torch.int32, device="cuda")

    def pair():
        ctx.qgemm(at, w1, a_zp=128, a_scale=0.02, y_scale=0.05, y_zp=128, out=h)
        ctx.qgemm(h, w2, a_zp=128, a_scale=0.05, y_scale=0.05, y_zp=128, out=y)

    ops = 2 * 2.0 * 4096 * 768 * 3072
    if only != "matmul_integer_i32":
        settle_clock(torch, pair, 50.0)
        t = time_launches(torch, stream, pair, 100, 5)
        out["int8_ffn_pair"] = {"ms": round(t, 5), "tops": round(ops / t / 1e9, 2),
                                "frac_mfma": round(ops / t / 1e9 / PEAK_TFLOPS["int8"], 4)}
    if only == "int8_ffn":
        return out
    fm = lambda: ctx.qgemm(at, w1, a_zp=128, out_kind=L.QOUT_I32, out=yi)   # noqa: E731
    settle_clock(torch, fm, 50.0)
    t = time_launches(torch, stream, fm, 100, 5)
    by = 4096 * 768 + 768 * 3072 + 4 * 4096 * 3072
    out["matmul_integer_i32"] = {"ms": round(t, 5), "tops": round(ops / 2 / t / 1e9, 2),
                                 "gbps": round(by / t / 1e6, 1), "frac_hbm": round(by / t / 1e6 / HBM_GBPS, 4)}
    return out


def bench_large(torch, ctx, L, stream, rng, only):
    """The same kernels at a large square shape, (M,K,N) = 8192^3: f16 Gemm
    (B resident, row bias) and int8 QLinearMatMul (u8 out), where the tile
    count fills the chip several times and the fixed per-launch costs vanish.
    Each runs back to back for 100 ms first (the clock settles under the
    dtype's own load, as for the headline), then 20 timed launches."""
    keys = ("large_gemm_f16", "large_qlinear_matmul_i8")
    if only and only not in keys:
        return {}
    out = {}
    m = k = n = 8192
    fl = 2.0 * m * k * n
    if not only or only == keys[0]:
        _, _, _, w, at, ct, y = gemm_setup(torch, ctx, L, m, k, n, L.F16, rng)
        fg = lambda: ctx.gemm(at, w, ct, out=y)   # noqa: E731
        settle_clock(torch, fg, 100.0)
        t = time_launches(torch, stream, fg, 20, 2)
        out[keys[0]] = {"shape": [m, k, n], "ms": round(t, 5), "tflops": round(fl / t / 1e9, 2),
                        "frac_mfma": round(fl / t / 1e9 / PEAK_TFLOPS["f16"], 4)}
        del w, at, ct, y
    if not only or only == keys[1]:
        a = torch.from_numpy(rng.integers(0, 256, (m, k)).astype(np.uint8)).cuda()
        wq = ctx.weight_qgemm(rng.integers(-127, 128, (k, n)).astype(np.int8), zp=0,
                              scale=rng.uniform(0.001, 0.01, n).astype(np.float32), name="large.B")
        yq = torch.empty((m, n), dtype=torch.uint8, device="cuda")
        fq = lambda: ctx.qgemm(a, wq, a_zp=128, a_scale=0.02, y_scale=0.05, y_zp=128, out=yq)   # noqa: E731
        settle_clock(torch, fq, 100.0)
        t = time_launches(torch, stream, fq, 20, 2)
        out[keys[1]] = {"shape": [m, k, n], "ms": round(t, 5), "tops": round(fl / t / 1e9, 2),
                        "frac_mfma": round(fl / t / 1e9 / PEAK_TFLOPS["int8"], 4)}
    return out


def bench_widened(torch, ctx, L, stream, rng, only):
    """The convolution forms beyond plain Conv, at decoder / mobile-net shapes,
    f16 NCHW, operands resident:
    * depthwise 3x3 [1,256,56,56] (the depthwise band kernel; memory-bound:
      GB/s of input + output + filter against HBM);
    * grouped 3x3 [1,256,56,56], 8 groups of 32 channels (one MFMA launch,
      the group on the grid z);
    * ConvTranspose 4x4 stride 2 [1,512,32,32] -> [1,256,64,64] (four
      sub-pixel phases on the MFMA engine);
    * config 4's residual conv, 3x3 512 -> 512 at 32x32 (input staging,
      split-K slices and their reduction included).
    Each is timed after 50 ms of its own launches (the settled clock).  ms:
    eager launches back to back (host dispatch included); ms_graph: the same
    launches replayed from a HIP graph."""
    keys = ("depthwise_conv_f16", "grouped_conv_f16", "conv_transpose_f16", "conv_res_f16")
    if only and only not in keys:
        return {}
    out = {}
    x = torch.from_numpy(rng.uniform(-1, 1, (1, 256, 56, 56)).astype(np.float32)).cuda().half()
    if not only or only == keys[0]:
        wt = ctx.weight_conv(rng.normal(0, 0.2, (256, 1, 3, 3)).astype(np.float32), dtype=L.F16)
        y = torch.empty((1, 256, 56, 56), dtype=torch.float16, device="cuda")
        f = lambda: ctx.conv2d(x, wt, None, pads=(1, 1, 1, 1), group=256, out=y)
        settle_clock(torch, f, 50.0)
        t = time_launches(torch, stream, f, 100, 5)
        tg = time_graph(torch, ctx, L, f)
        by = 2 * (2 * 256 * 56 * 56 + 256 * 9)
        fl = 2.0 * 256 * 56 * 56 * 9
        out[keys[0]] = {"ms": round(t, 5), "gbps": round(by / t / 1e6, 1),
                        "frac_hbm": round(by / t / 1e6 / HBM_GBPS, 4), "tflops": round(fl / t / 1e9, 2),
                        "ms_graph": round(tg, 5), "gbps_graph": round(by / tg / 1e6, 1)}
    if not only or only == keys[1]:
        wt = ctx.weight_conv(rng.normal(0, 0.05, (256, 32, 3, 3)).astype(np.float32), dtype=L.F16)
        y = torch.empty((1, 256, 56, 56), dtype=torch.float16, device="cuda")
        f = lambda: ctx.conv2d(x, wt, None, pads=(1, 1, 1, 1), group=8, out=y)
        settle_clock(torch, f, 50.0)
        t = time_launches(torch, stream, f, 100, 5)
        tg = time_graph(torch, ctx, L, f)
        fl = 2.0 * 256 * 56 * 56 * 32 * 9
        out[keys[1]] = {"ms": round(t, 5), "tflops": round(fl / t / 1e9, 2),
                        "frac_mfma": round(fl / t / 1e9 / PEAK_TFLOPS["f16"], 4), "ms_graph": round(tg, 5),
                        "tflops_graph": round(fl / tg / 1e9, 2)}
    if not only or only == keys[2]:
        xt = torch.from_numpy(rng.uniform(-1, 1, (1, 512, 32, 32)).astype(np.float32)).cuda().half()
        wt = ctx.weight_conv_transpose(rng.normal(0, 0.02, (512, 256, 4, 4)).astype(np.float32), dtype=L.F16,
                                       strides=(2, 2), pads=(1, 1, 1, 1))
        y = torch.empty((1, 256, 64, 64), dtype=torch.float16, device="cuda")
        f = lambda: ctx.conv_transpose2d(xt, wt, None, strides=(2, 2), pads=(1, 1, 1, 1), out=y)
        settle_clock(torch, f, 50.0)
        t = time_launches(torch, stream, f, 20, 2)
        fl = 2.0 * 512 * 32 * 32 * 256 * 16   # every input scatters a 4x4 tap into the output
        out[keys[2]] = {"ms": round(t, 5), "tflops": round(fl / t / 1e9, 2),
                        "frac_mfma": round(fl / t / 1e9 / PEAK_TFLOPS["f16"], 4)}
    if not only or only == keys[3]:
        xr = torch.from_numpy(rng.uniform(-1, 1, (1, 512, 32, 32)).astype(np.float32)).cuda().half()
        wt = ctx.weight_conv(rng.normal(0, 0.02, (512, 512, 3, 3)).astype(np.float32), dtype=L.F16)
        y = torch.empty((1, 512, 32, 32), dtype=torch.float16, device="cuda")
        f = lambda: ctx.conv2d(xr, wt, None, pads=(1, 1, 1, 1), out=y)
        settle_clock(torch, f, 50.0)
        t = time_launches(torch, stream, f, 100, 0)
        fl = 2.0 * 1024 * 512 * 4608
        out[keys[3]] = {"ms": round(t, 5), "tflops": round(fl / t / 1e9, 2),
                        "frac_mfma": round(fl / t / 1e9 / PEAK_TFLOPS["f16"], 4)}
    return out


GATE_M = [1, 2, 4, 8, 12, 16, 24, 32, 48, 64, 96, 128, 256]
GATE_KN = [(128, 128), (256, 256), (512, 512), (1024, 1024), (2048, 2048), (4096, 4096), (25088, 512)]
GATE_CONV = [(c, hw) for c in (8, 16, 32, 64, 128) for hw in (8, 16, 32, 64)]


def _best_ms(fn, reps):
    fn()
    best = float("inf")
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        best = min(best, (time.perf_counter() - t0) * 1e3)
    return best


def bench_gate(torch, ctx, L, only):
    """--only gate: the GPU / CPU crossover table the MI355X dispatch gate is
    set from, in the reference's method (tuning.rs:60-83): per shape, the
    best wall time of the provider's Gemm node with host operands in and the
    host result out (B uploaded every call, or B resident in the weight
    cache after its first call), against the reference's CPU algorithm on
    this host (2-D Gemm: single-threaded packed sgemm, math_typed.rs:45-79;
    Conv: im2col + sgemm over every host thread, conv2d.rs:246-547).  Not
    part of the default run."""
    if only != "gate":
        return {}
    import ctypes
    from oracle import oracle as O
    from oxionnx_amd import ep
    t = L.Tuning()
    L.lib().ohip_tuning_for_class(L.CLASS_PARITY, ctypes.byref(t))
    ctx.set_tuning(t)   # time every shape on the device, however small
    rng = np.random.default_rng(77)
    gemm = []
    node = ep.Node("Gemm", ["a", "b"], ["y"])
    for kk, nn in GATE_KN:
        b = rng.normal(0, 1 / np.sqrt(kk), (kk, nn)).astype(np.float32)
        for mm in GATE_M:
            a = rng.uniform(-1, 1, (mm, kk)).astype(np.float32)
            reps = 15 if mm * kk * nn < 2e8 else 5
            cpu = _best_ms(lambda: O.gemm(a, b, nthreads=1), reps)
            up = _best_ms(lambda: ep.try_hip_dispatch(node, {}, {"a": a, "b": b}, ctx), reps)
            wname = f"gate.B.{kk}.{nn}"
            cnode = ep.Node("Gemm", ["a", wname], ["y"])
            cached = _best_ms(lambda: ep.try_hip_dispatch(cnode, {wname: b}, {"a": a}, ctx), reps)
            gemm.append({"m": mm, "k": kk, "n": nn, "cpu_ms": round(cpu, 4), "gpu_upload_ms": round(up, 4),
                         "gpu_cached_ms": round(cached, 4), "ratio_upload": round(up / cpu, 3),
                         "ratio_cached": round(cached / cpu, 3)})
    conv = []
    for c, hw in GATE_CONV:
        x = rng.uniform(-1, 1, (1, c, hw, hw)).astype(np.float32)
        w = rng.normal(0, 0.05, (c, c, 3, 3)).astype(np.float32)
        wname = f"gate.W.{c}.{hw}"
        cn = ep.Node("Conv", ["x", wname], ["y"], ep.Attributes(int_lists={"pads": [1, 1, 1, 1]}))
        reps = 15 if c * c * 9 * hw * hw < 2e8 else 5
        cpu = _best_ms(lambda: O.conv(x, w, pads=[1, 1, 1, 1], nthreads=HOST_CORES), reps)
        gpu = _best_ms(lambda: ep.try_hip_dispatch(cn, {wname: w}, {"x": x}, ctx), reps)
        conv.append({"cout": c, "cin": c, "kernel": 3, "hw": hw, "implied_mac": c * c * 9 * hw * hw,
                     "cpu_ms": round(cpu, 4), "gpu_ms": round(gpu, 4), "ratio": round(gpu / cpu, 3)})
    return {"gate": {"host_cores": HOST_CORES, "gemm": gemm, "conv": conv,
                     "note": "ratio = GPU / CPU wall time; > 1 means the GPU lost"}}


def _time_forwards(torch, stream, fwd, n=10):
    """(median wall ms, median stream ms) of n forwards after two untimed ones."""
    for _ in range(2):
        fwd()
    walls, gpus = [], []
    for _ in range(n):
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record(stream)
        fwd()
        e1.record(stream)
        walls.append((time.perf_counter() - t0) * 1e3)
        torch.cuda.synchronize()
        gpus.append(e0.elapsed_time(e1))
    return round(float(np.median(walls)), 3), round(float(np.median(gpus)), 3)


def bench_e2e(torch, ctx, stream, only, no_cpu, fused_only=False):
    """Configs 4 and 5 end to end, median of 10 forwards each:
    * the session run loop (graph inputs uploaded, every node dispatched
      through ohip_try_dispatch, outputs downloaded);
    * the same forward captured once into a HIP graph and replayed (inputs
      uploaded, graph launched, outputs downloaded) -- ms_per_forward;
    * events on the context's stream around both;
    * the CPU graph oracle's time for one forward (the reference's algorithms
      restated: multi-threaded im2col + sgemm convolution like its rayon
      path, single-threaded integer convolution like its integer_conv)."""
    from oxionnx_amd import workloads
    from oxionnx_amd.session import Session
    names = {"e2e_face_swap_f32": lambda: workloads.face_swap_generator(dtype="f32"),
             "e2e_face_swap_f16": lambda: workloads.face_swap_generator(dtype="f16"),
             "e2e_yolo_backbone_int8": lambda: workloads.yolo_backbone_int8(size=640)}
    threads = max(1, min(16, int(os.environ.get("OMP_NUM_THREADS", "16"))))
    out = {}
    for key, make in names.items():
        if only and only != key:
            continue
        g, feeds = make()
        sess = Session(g, ctx)
        loop = _time_forwards(torch, stream, lambda: sess.run(feeds))
        cap = sess.capture(feeds)
        graph = _time_forwards(torch, stream, lambda: cap.replay(feeds))
        resident = _time_forwards(torch, stream, lambda: cap.replay(None, download=False))
        cap.close()
        # the same graph with only the fusion the reference's optimizer makes
        # (Conv + Relu): every other node runs as its own device kernel
        rec = {"ms_per_forward": graph[0], "ms_per_forward_run_loop": loop[0],
               "stream_ms_graph": graph[1], "stream_ms_run_loop": loop[1],
               "stream_ms_graph_io_resident": resident[1]}
        if not fused_only:
            rsess = Session(g, ctx, optimize="reference")
            rloop = _time_forwards(torch, stream, lambda: rsess.run(feeds))
            rcap = rsess.capture(feeds)
            rgraph = _time_forwards(torch, stream, lambda: rcap.replay(feeds))
            rcap.close()
            rec["reference_fusions_only"] = {"ms_per_forward": rgraph[0], "ms_per_forward_run_loop": rloop[0],
                                             "stream_ms_graph": rgraph[1], "nodes": len(rsess.graph.nodes)}
        rec.update({
               "nodes": len(g.nodes), "nodes_after_fusion": len(sess.graph.nodes),
               "conv_gmac": round(g.notes["conv_gmac"], 3),
               "note": "ms_per_forward: wall clock of one forward replayed from its captured HIP graph, incl. "
                       "input upload and output download (PCIe); stream_ms_graph_io_resident: the replay alone, its input "
                       "already on the device and its outputs left there; ms_per_forward_run_loop: the same forward "
                       "dispatched node by node through the Python run loop; reference_fusions_only: the "
                       "graph with only the reference optimizer's Conv+Relu fusion (no provider-side "
                       "rewrites)"})
        if not no_cpu and not only:
            from oracle import graph_ref
            t0 = time.perf_counter()
            graph_ref.run_graph(g, feeds, half=key.endswith("f16"), nthreads=threads)
            cpu = (time.perf_counter() - t0) * 1e3
            int8 = "int8" in key
            rec["cpu_baseline"] = {
                "ms_per_forward": round(cpu, 1), "kind": "port", "cores": 1 if int8 else threads,
                "host_cores": HOST_CORES,
                "sample": "one full forward of the same graph and inputs" + (
                    "; integer convolution single-threaded like the reference's integer_conv" if int8 else
                    "; float convolution as im2col + a packed Goto/BLIS sgemm (AVX2/FMA 6x16 "
                    "microkernel, rows split over the threads; oracle/oracle_sgemm.c: a stand-in for "
                    "matrixmultiply's packed 8x8 microkernel, not that kernel)")}
            rec["speedup_vs_cpu"] = round(cpu / rec["ms_per_forward"], 1)
            rec["speedup_vs_cpu_run_loop"] = round(cpu / rec["ms_per_forward_run_loop"], 1)
            if not fused_only:
                rec["speedup_vs_cpu_reference_fusions_only"] = round(cpu / rgraph[0], 1)
        out[key] = rec
    return out


if __name__ == "__main__":
    main()
