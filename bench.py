#!/usr/bin/env python3
"""Headline benchmark: fused fp32 relu(A @ B + bias) at M = N = K = 2048 on one
MI355X, through libtforge_hip (the gfx950 staged MFMA kernel).

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--options "..."]
                  [--no-cpu-baseline] [--no-autotune-compare]
  python bench.py --cpu-table results/cpu/cpu_baseline_host.csv   (CPU rows only)

A step is one launch of the compiled program over device-resident inputs:
the reference's seeded draws (numpy default_rng(1234), uniform[-1,1] in the
order A, B, bias; python/tforge_cpu.py:89-100), made on the host and uploaded
before any timing.  Order of work:

  1. pre-warm (disclosed in the line): launches in chunks of 20 until at least
     0.3 s have passed and the last three chunks' per-launch times agree within
     1% (at most 3 s) -- the GPU leaves its idle clock only under load, and a
     few milliseconds of warm-up would time the ramp;
  2. W untimed warm-up launches, then exactly K launches timed between two
     synchronisations with one HIP event pair on the launch stream (`value`);
  3. the shader clock measured on the device right after the window
     (tf_clock_probe: s_memtime cycles against the 100 MHz wall clock, one
     workgroup per XCD);
  4. K more launches, each bracketed by its own event pair on the same stream;
     their average and median (the reference runner reports medians,
     runners/gpu/tforge-gpu-bench.cu:345-363) go into the line beside the
     window's.  `roofline.achieved` uses the window: the average launch
     duration over the timed region.  A launch alone between its own events
     also pays its dispatch and completion latency (3-12 us more, varying
     between machines), which back-to-back launches overlap.

TFLOP/s = 2*M*N*K / time (the reference's convention, bench/gpu_bench.py:57);
the peak is MI355X's published FP32 matrix figure, 157.3 TFLOP/s.  The
autotune comparison times the selected and the cost-model default
configurations in alternating rounds and checks both outputs.  The CPU baseline
is the oracle's port of the reference's best CPU kernel (6x16x4 register tile,
FMA), one thread pinned to the first allowed core, with the default scalar
pipeline and NumPy beside it.
"""

import argparse
import json
import os
import pathlib
import statistics
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "fp32 TFLOP/s, fused relu(A@B+b) at 2048^3, and % of MI355X FP32 MFMA peak"
M = N = K = 2048
PEAK_TFLOPS = 157.3
PEAK_FLOP_PER_CLK = 256 * 256  # 256 CUs x 256 FP32 matrix FLOP per clock
TUNED = ROOT / "tensorforge_amd" / "tuned_configs.json"
PROFILED = ROOT / "profiles" / "traffic.json"

# Every configuration BASELINE.json names, for the CPU table: (label, workload, M, N, K).
CPU_CONFIGS = [
    ("examples/mbr.mlir", "mbr", 256, 256, 128),
    ("headline", "mbr", 2048, 2048, 2048),
    ("matmul 512", "matmul", 512, 512, 512),
    ("matmul 1024", "matmul", 1024, 1024, 1024),
    ("matmul 2048", "matmul", 2048, 2048, 2048),
    ("matmul 4096", "matmul", 4096, 4096, 4096),
    ("matmul 8192", "matmul", 8192, 8192, 8192),
    ("layer 8192x1024x4096", "mbr", 8192, 1024, 4096),
    ("layer 1024x8192x4096", "mbr", 1024, 8192, 4096),
    ("skinny 64x4096x4096", "mbr", 64, 4096, 4096),
    ("short-K 4096x4096x256", "mbr", 4096, 4096, 256),
    ("residual block layer 1", "mbr", 4096, 8192, 2048),
    ("residual block layer 2 (+x)", "mbr+add", 4096, 2048, 8192),
]


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def default_options():
    from tensorforge_amd import costmodel
    return costmodel.options(costmodel.default_config(M, N, K))


def tuned_options():
    if TUNED.exists():
        t = json.loads(TUNED.read_text()).get(f"mbr/{M}x{N}x{K}")
        if t:
            return t["options"]
    return None


class Launcher:
    """Launches one compiled program on fixed device buffers and times it with
    HIP events on the stream it launches on."""

    def __init__(self, kern, ptrs, stream, torch):
        self.kern, self.ptrs, self.stream, self.torch = kern, ptrs, stream, torch

    def event(self):
        return self.torch.cuda.Event(enable_timing=True)

    def launch(self, count=1):
        for _ in range(count):
            self.kern.launch(self.ptrs, self.stream.cuda_stream)

    def window(self, count):
        """ms per launch over `count` back-to-back launches (one event pair)."""
        a, b = self.event(), self.event()
        a.record(self.stream)
        self.launch(count)
        b.record(self.stream)
        b.synchronize()
        return a.elapsed_time(b) / count

    def per_launch(self, count):
        """Event-pair duration (ms) of each of `count` launches."""
        evs = [(self.event(), self.event()) for _ in range(count)]
        for a, b in evs:
            a.record(self.stream)
            self.launch()
            b.record(self.stream)
        evs[-1][1].synchronize()
        return [a.elapsed_time(b) for a, b in evs]

    def prewarm(self, min_s=0.3, max_s=3.0, chunk=20, tol=0.01):
        t0, chunks = time.perf_counter(), []
        while True:
            chunks.append(self.window(chunk))
            spent = time.perf_counter() - t0
            last = chunks[-3:]
            settled = len(last) == 3 and (max(last) - min(last)) <= tol * min(last)
            if (spent >= min_s and settled) or spent >= max_s:
                return {"launches": chunk * len(chunks), "seconds": round(spent, 3), "settled": settled,
                        "last_chunk_us": round(chunks[-1] * 1e3, 2)}


# err/bound of the reference's own kernels on the same inputs (ref:results/gpu/stage8.csv:86).
REFERENCE_ERR_OVER_BOUND = 0.00232


def parity_sample(torch, A, B, bias, C, rows=M):
    """err/bound of the reference check (python/tforge_gpu.py:134-145) with
    the ReLU mask rule, in float64 on the GPU, over `rows` evenly spaced output
    rows (all of them by default)."""
    idx = torch.linspace(0, M - 1, rows, device=A.device).long()
    a64, b64, c64 = A[idx].double(), B.double(), bias.double()
    z = a64 @ b64 + c64
    ref = torch.clamp_min(z, 0.0)
    mag = a64.abs() @ b64.abs() + c64.abs()
    u = 2.0 ** -24
    gamma = (K + 1) * u / (1 - (K + 1) * u)
    bound = gamma * mag + torch.finfo(torch.float32).tiny
    out = C[idx].double()
    eob = float(((out - ref).abs() / bound).max())
    decided = z.abs() > bound
    masks = int((decided & ((out == 0) != (z <= 0))).sum())
    return {"rows_checked": rows, "err_over_bound": eob, "mask_mismatches": masks,
            "reference_kernels_err_over_bound": REFERENCE_ERR_OVER_BOUND,
            "pass": eob <= 1.0 and masks == 0 and not bool(torch.isnan(out).any())}


# The reference's Stage 8 headline tiles (ref:results/gpu/stage8.csv:86; ref:bench/stage8_gpu.sh).
REFERENCE_TILES = "block-tile=128,64 thread-tile=8,4 tile-k=16 promote=1 vectorize=1"


def interleaved(launchers, rounds=6, steps=50, warm=10):
    """Median ms per launch of each launcher over `rounds` alternating rounds
    (the first launcher leads in even rounds, the last in odd ones), each
    round `warm` untimed launches then a `steps`-launch window."""
    names = list(launchers)
    times = {n: [] for n in names}
    for r in range(rounds):
        for n in (names if r % 2 == 0 else names[::-1]):
            launchers[n].launch(warm)
            times[n].append(launchers[n].window(steps))
    return {n: statistics.median(v) for n, v in times.items()}, times


def host_cpu():
    """CPU identity from /proc/cpuinfo and the cores this process may use."""
    info = {}
    try:
        for line in open("/proc/cpuinfo"):
            key, _, val = line.partition(":")
            key = key.strip()
            if key in ("model name", "cpu family", "model", "stepping") and key not in info:
                info[key] = val.strip()
    except OSError:
        pass
    allowed = sorted(os.sched_getaffinity(0))
    return {"model_name": info.get("model name", ""), "family": info.get("cpu family", ""),
            "model": info.get("model", ""), "stepping": info.get("stepping", ""),
            "allowed_cores": len(allowed), "pinned_cpu": allowed[0]}


def cpu_baseline(configs, call_budget_s=2.0):
    """Times the CPU baselines of each (label, workload, m, n, k) on one core
    pinned to the first allowed CPU, with 64-byte-aligned buffers
    (runners/cpu/tforge-cpu-bench.cpp:65-77, 174-186):

      vec6x16  the oracle's port of the reference's best CPU pipeline
               (fuse-elementwise=1 reg-tile=6,16,4 vectorize=1: 6x16 AVX2 FMA
               tiles, fused bias + relu), bitwise = its arithmetic
      scalar   the default pipeline's loop (one output at a time, k innermost,
               no FMA) plus its separate epilogue
      numpy    matmul, add, maximum with out=, 1 BLAS thread
               (bench/cpu_bench.py:54-77)

    Reps follow the reference: 10 warm-up + 100 timed calls where that fits
    in about 6 s, else 1 + 3.  A call estimated above `call_budget_s` runs on
    the first rows of A only (every row costs the same: each strip of rows
    streams all of B), and the sample says so.  Returns (rows, host)."""
    import numpy as np
    from threadpoolctl import threadpool_limits
    from oracle import oracle as o

    host = host_cpu()
    saved = os.sched_getaffinity(0)
    os.sched_setaffinity(0, {host["pinned_cpu"]})
    rate_guess = {"vec6x16": 40e9, "scalar": 0.4e9, "numpy": 150e9}
    rows_out = []
    try:
        for label, workload, m, n, k in configs:
            rng = np.random.default_rng(1234)
            a = o.aligned_copy(rng.uniform(-1, 1, (m, k)).astype(np.float32))
            b = o.aligned_copy(rng.uniform(-1, 1, (k, n)).astype(np.float32))
            fused = workload != "matmul"
            bias = o.aligned_copy(rng.uniform(-1, 1, n).astype(np.float32)) if fused else None
            for variant in ("vec6x16", "scalar", "numpy"):
                per_row = 2.0 * n * k / rate_guess[variant]
                rows = m
                if per_row * m > call_budget_s and variant != "numpy":
                    step = 6 if variant == "vec6x16" else 1
                    rows = max(step, int(call_budget_s / per_row) // step * step)
                warmup, reps = (10, 100) if per_row * rows * 110 <= 6.0 else (1, 3)
                a_s = a if rows == m else o.aligned_copy(a[:rows])
                t0 = time.perf_counter()
                if variant == "vec6x16":
                    ns = o.time_vec6x16(a_s, b, bias, warmup, reps, relu=fused)
                elif variant == "scalar":
                    ns = o.time_scalar(a_s, b, bias, warmup, reps, relu=fused)
                else:
                    out = o.aligned_empty((rows, n))
                    ts = []
                    with threadpool_limits(limits=1):
                        for i in range(warmup + reps):
                            s = time.perf_counter_ns()
                            np.matmul(a_s, b, out=out)
                            if fused:
                                np.add(out, bias, out=out)
                                np.maximum(out, np.float32(0), out=out)
                            ts.append(time.perf_counter_ns() - s)
                    ns = float(np.median(ts[warmup:]))
                rows_out.append({
                    "label": label, "workload": workload, "shape": f"{m}x{n}x{k}", "variant": variant,
                    "gflops": 2.0 * rows * n * k / ns, "median_ms": ns * 1e-6, "warmup": warmup, "reps": reps,
                    "sample": "full problem" if rows == m else f"first {rows} of {m} rows of A",
                    "seconds": round(time.perf_counter() - t0, 2)})
                log(f"cpu {label} {variant}: {rows_out[-1]['gflops']:.2f} GFLOP/s ({rows_out[-1]['sample']}, "
                    f"{warmup}+{reps} reps)")
    finally:
        os.sched_setaffinity(0, saved)
    host["avx2_fma"] = bool(o.lib().tfo_have_avx2())
    return rows_out, host


def cpu_line(rows, host):
    by = {r["variant"]: r for r in rows}
    v = by["vec6x16"]
    return {"value": v["gflops"] / 1e3, "unit": "TFLOP/s", "cores": 1, "kind": "port",
            "sample": (f"{v['shape']} fused mbr, {v['sample']}: the oracle's 6x16x4 AVX2-FMA port of the "
                       f"reference's best CPU pipeline (reg-tile=6,16,4 vectorize=1), 1 thread pinned to CPU "
                       f"{host['pinned_cpu']}, median of {v['reps']} reps after {v['warmup']}"),
            "gflops": v["gflops"], "scalar_default_pipeline_gflops": by["scalar"]["gflops"],
            "scalar_sample": by["scalar"]["sample"], "numpy_1thread_gflops": by["numpy"]["gflops"],
            "host": host, "seconds": round(sum(r["seconds"] for r in rows), 2)}


def write_cpu_table(path, rows, host):
    from tensorforge_amd import provenance
    table = provenance.ResultsTable(path)
    names = {"vec6x16": "cpu-port-vec-r6x16x4 (fuse-elementwise=1 reg-tile=6,16,4 vectorize=1)",
             "scalar": "cpu-port-scalar (tforge-cpu-pipeline defaults)",
             "numpy": "numpy matmul + add + maximum, 1 BLAS thread"}
    for r in rows:
        table.add(device=f"{host['model_name']} (family {host['family']} model {host['model']} stepping "
                         f"{host['stepping']}; {host['allowed_cores']} allowed cores)",
                  workload=r["workload"], shape=r["shape"], dtype="f32", pipeline=names[r["variant"]],
                  params=f"{r['label']}; {r['sample']}", threads=1, warmup=r["warmup"], reps=r["reps"],
                  median_ms=r["median_ms"], metric="GFLOP/s", metric_value=r["gflops"],
                  notes=(f"pinned to CPU {host['pinned_cpu']}; 64-byte-aligned buffers; avx2+fma "
                         f"{host['avx2_fma']}" + ("; the final +x of the block is not timed"
                                                  if r["workload"] == "mbr+add" else "")))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=50, help="untimed launches after the pre-warm")
    ap.add_argument("--options", default=None, help="pipeline options (default: autotuned, else cost model)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-autotune-compare", action="store_true")
    ap.add_argument("--cpu-table", metavar="CSV", help="time the CPU baselines of every configuration into CSV "
                                                       "and exit (no GPU work)")
    args = ap.parse_args()
    if args.cpu_table:
        rows, host = cpu_baseline(CPU_CONFIGS)
        write_cpu_table(args.cpu_table, rows, host)
        print(json.dumps({"cpu_rows": len(rows), "host": host, "csv": args.cpu_table}))
        return 0
    if args.gpus != 1:
        print(json.dumps({"error": "this backend runs on one GPU; multi-GPU runs are not part of this build",
                          "n_gpus": args.gpus}))
        return 2

    import torch
    from tensorforge_amd import _lib
    from tensorforge_amd import tforge_cpu as tc

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    host = tc.make_inputs("mbr", M, N, K, seed=1234)
    A, B, bias = (torch.from_numpy(host[s]).to(dev) for s in ("a", "b", "bias"))
    C = torch.empty((M, N), device=dev, dtype=torch.float32)
    ptrs = [A.data_ptr(), B.data_ptr(), bias.data_ptr(), C.data_ptr()]
    stream = torch.cuda.current_stream()
    program = tc.gen_mlir("mbr", M, N, K)

    dflt = default_options()
    opts = args.options or tuned_options() or dflt
    log(f"options: {opts}")
    kern = _lib.Kernel(program, opts, "bench.mlir")
    launch = kern.launches()[0]
    run = Launcher(kern, ptrs, stream, torch)
    prewarm = run.prewarm()
    log(f"pre-warm: {prewarm}")
    run.launch(args.warmup)
    torch.cuda.synchronize()
    window_ms = run.window(args.steps)
    clock_mhz = _lib.clock_probe(stream.cuda_stream)
    per_launch = run.per_launch(min(args.steps, 20))  # few, so the trace's kernel average stays the window's
    clock_after_mhz = _lib.clock_probe(stream.cuda_stream)
    parity = parity_sample(torch, A, B, bias, C)
    flops = 2.0 * M * N * K
    value = flops / (window_ms * 1e-3) / 1e12
    avg_ms = statistics.fmean(per_launch)
    med_ms = statistics.median(per_launch)
    achieved = flops / (window_ms * 1e-3) / 1e12
    log(f"{launch['kernel']}: {window_ms * 1e3:.1f} us/step, {value:.2f} TFLOP/s, per-launch avg "
        f"{avg_ms * 1e3:.1f} / median {med_ms * 1e3:.1f} us, clock {clock_mhz[0]:.0f} MHz, parity {parity}")

    autotune = None
    if not args.no_autotune_compare:
        # The autotuned configuration against the cost model's pick, and both
        # against the reference's own Stage 8 tiles (ref:results/gpu/stage8.csv:86,
        # full-128x64-t8x4-k16) run on this backend, in alternating rounds.
        others = {"default": dflt, "reference_tiles": REFERENCE_TILES}
        others = {k: v for k, v in others.items() if v != opts}
        if "default" in others and others.get("reference_tiles") == dflt:
            del others["reference_tiles"]
        launchers = {"selected": run}
        launchers.update({k: Launcher(_lib.Kernel(program, v, "bench.mlir"), ptrs, stream, torch) for k, v in others.items()})
        med, _ = interleaved(launchers)
        tf = {k: flops / (ms * 1e-3) / 1e12 for k, ms in med.items()}
        default_parity = parity
        if "default" in others:
            Launcher(_lib.Kernel(program, dflt, "bench.mlir"), ptrs, stream, torch).launch(1)
            torch.cuda.synchronize()
            default_parity = parity_sample(torch, A, B, bias, C)  # C holds the default's output now
        autotune = {"default_options": dflt, "selected_options": opts, "reference_tiles_options": REFERENCE_TILES,
                    "selected_tflops": tf["selected"],
                    "default_tflops": tf.get("default", tf["selected"]),
                    "speedup_over_default": med.get("default", med["selected"]) / med["selected"],
                    "reference_tiles_tflops": tf.get("reference_tiles", tf.get("default", tf["selected"])),
                    "speedup_over_reference_tiles": med.get("reference_tiles", med.get("default", med["selected"]))
                    / med["selected"],
                    "protocol": "6 alternating rounds of 10 warm-up + 50 timed launches each; medians",
                    "default_parity": default_parity}
        if opts == dflt:
            autotune["note"] = ("the cost model's pick is the autotuned configuration "
                                "(tensorforge_amd/tuned_configs.json), so the speedup over it is 1")
        log(f"autotune: {autotune}")

    traffic = None
    if PROFILED.exists():
        rec = json.loads(PROFILED.read_text()).get(launch["kernel"])
        if rec and rec.get("workload") == f"mbr/{M}x{N}x{K}":
            traffic = rec.get("hbm_bytes_per_launch")

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_line(*cpu_baseline([("headline", "mbr", M, N, K)]))
    peak_at_clock = PEAK_FLOP_PER_CLK * clock_mhz[0] * 1e6 / 1e12
    line = {
        "metric": METRIC, "value": round(value, 3), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": window_ms, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic: A, B, bias uniform[-1,1], the reference's draws "
                                                   "(numpy default_rng(1234), python/tforge_cpu.py:89-100)",
        "config": {"workload": f"fused mbr relu(A@B+bias) fp32 M=N=K={M}, row-major", "options": opts,
                   "kernel": launch["kernel"], "grid": launch["grid"], "block": launch["block"],
                   "parallelism": "single GPU"},
        "pct_of_fp32_mfma_peak": round(100.0 * value / PEAK_TFLOPS, 2),
        "pct_of_peak_at_measured_clock": round(100.0 * value / peak_at_clock, 2),
        "prewarm": prewarm,
        "clock": {"after_window_mhz": round(clock_mhz[0], 1), "xcd_min_mhz": round(clock_mhz[1], 1),
                  "xcd_max_mhz": round(clock_mhz[2], 1), "after_per_launch_mhz": round(clock_after_mhz[0], 1),
                  "method": "device probe: s_memtime cycles over the 100 MHz wall clock, one workgroup per XCD"},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 3), "peak": PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_TFLOPS, 4), "traffic": traffic,
                     "traffic_source": "profiles/traffic.json (rocprofv3 FETCH_SIZE + WRITE_SIZE, calibrated)"
                     if traffic else None,
                     "window_ms_per_launch": window_ms, "flop_per_launch": flops,
                     "per_launch_events": {"avg_ms": avg_ms, "median_ms": med_ms,
                                           "note": "20 launches, each between its own event pair, after the window"}},
        "parity": parity, "autotune": autotune, "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0 if parity["pass"] and (autotune is None or autotune["default_parity"]["pass"]) else 1


if __name__ == "__main__":
    sys.exit(main())
