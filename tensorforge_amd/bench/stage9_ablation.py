#!/usr/bin/env python3
"""Stage 9 ablation ladder for relu(A @ B + bias) on MI355X.

The reference's ladder (bench/stage9_ablation.py:1-13, 23-28), same steps,
shapes, CSV rows and checks, run on the gfx950 kernels:

  baseline     unfused: three direct kernels (matmul, bias_add, relu), one
               output per thread, 16x16 blocks; time = sum of the three
               medians, each kernel checked on its own (matmul against the
               FP64 bound, bias_add and relu bit-exact)
  +fusion      one direct fused kernel
  +tiling      128x64 blocks, 8x4 per thread, K step 16: FP32 MFMA on
               fragments read straight from global memory (no LDS, 32-bit)
  +promotion   + A/B slabs staged in LDS (double-buffered)
  +vectorize   + 128-bit global and LDS accesses (the reference's default)

and two MI355X rungs after them:

  +autotuned   the configuration the autotuner recorded for the shape (or the
               cost model's pick), split-K included
  +mask-edges  (shapes that are not tile multiples) the autotuned kernel on
               the true shape, edges masked in-kernel instead of padded copies

  python -m tensorforge_amd.bench.stage9_ablation --csv results/gpu/stage9_ablation.csv
"""

import argparse
import sys

from tensorforge_amd import costmodel as cm
from tensorforge_amd import provenance
from tensorforge_amd import tforge_gpu as tg

SHAPES = [(1024, 1024, 1024), (2048, 2048, 2048), (4096, 4096, 4096), (777, 1111, 333)]
NAIVE = "block-tile=16,16 thread-tile=1,1"
TILED = "block-tile=128,64 thread-tile=8,4 tile-k=16"
STEPS = [("+fusion", NAIVE), ("+tiling", TILED + " promote=0 vectorize=0"),
         ("+promotion", TILED + " promote=1 vectorize=0"), ("+vectorize", TILED + " promote=1 vectorize=1")]


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--csv", default="results/gpu/stage9_ablation.csv")
    ap.add_argument("--shapes", default="")
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--reps", type=int, default=100)
    args = ap.parse_args(argv)
    shapes = SHAPES
    if args.shapes:
        shapes = [tuple(int(v) for v in s.split("x")) for s in args.shapes.split(",")]
    base = provenance.common()
    out = provenance.CsvWriter(args.csv)
    failures = 0

    def record(step, workload, m, n, k, opts, r, chk, note=""):
        gf = 2.0 * m * n * k / (r["median_ms"] * 1e-3) / 1e9
        clk = r["sm_clock_median_mhz"]
        pct = 100.0 * gf / tg.fp32_peak_gflops(clk if clk > 0 else tg.PEAK_CLOCK_MHZ)
        out.row(**base, device=r["gpu"], workload=workload, shape=f"{m}x{n}x{k}", dtype="f32",
                pipeline=f"tforge-gpu-pipeline{{{opts}}}",
                params=f"{step}; grid={r['grid']} block={r['block']}; regs={r['regs']} smem={r['static_smem']}",
                threads="", warmup=r["warmup"], reps=r["reps"], median_ms=r["median_ms"], min_ms=r["min_ms"],
                std_ms=r["std_ms"], metric="GFLOP/s (of the full mbr)", metric_value=gf,
                sm_clock_median_mhz=clk,
                clock_adjusted_metric=f"{pct:.2f}% of FP32 matrix peak at median clock", alloc_bytes_per_call="",
                correctness=f"err/bound={chk['err_over_bound']:.3g}", notes=note)
        return gf, pct

    def rung(step, m, n, k, opts, note=""):
        nonlocal failures
        d, launch = tg.compile_kernel("mbr", m, n, k, opts, tag=f"stage9abl/{step[1:]}")
        chk, _ = tg.check("mbr", m, n, k, d, launch)
        if not chk["pass"]:
            failures += 1
            print(f"[FAIL] {step} {m}x{n}x{k}", flush=True)
            return
        r = tg.bench("mbr", m, n, k, d, launch, warmup=args.warmup, reps=args.reps)
        gf, pct = record(step, "mbr", m, n, k, opts, r, chk, note)
        print(f"{step:>12} {m}x{n}x{k}: {r['median_ms']:.4f} ms {gf:9.0f} GFLOP/s {pct:5.1f}%  [{opts}]", flush=True)

    for m, n, k in shapes:
        parts, total_ms, clocks, ok = [], 0.0, [], True
        for wl, kk in (("matmul", k), ("bias_add", None), ("relu", None)):
            d, launch = tg.compile_kernel(wl, m, n, kk, NAIVE, tag="stage9abl/baseline")
            chk, _ = tg.check(wl, m, n, kk, d, launch)
            ok &= chk["pass"]
            r = tg.bench(wl, m, n, kk, d, launch, warmup=args.warmup, reps=args.reps)
            parts.append((wl, r, chk))
            total_ms += r["median_ms"]
            clocks.append(r["sm_clock_median_mhz"])
        if not ok:
            failures += 1
            print(f"[FAIL] baseline {m}x{n}x{k}", flush=True)
        for wl, r, chk in parts:
            record(f"baseline part: {wl}", wl, m, n, k, NAIVE, r, chk,
                   note="one of three unfused kernels; metric uses the mbr FLOP count")
        gf = 2.0 * m * n * k / (total_ms * 1e-3) / 1e9
        clk = sorted(clocks)[1]
        pct = 100.0 * gf / tg.fp32_peak_gflops(clk if clk > 0 else tg.PEAK_CLOCK_MHZ)
        r0 = parts[0][1]
        out.row(**base, device=r0["gpu"], workload="mbr", shape=f"{m}x{n}x{k}", dtype="f32",
                pipeline=f"tforge-gpu-pipeline{{{NAIVE}}} x3 kernels (matmul, bias_add, relu)",
                params="baseline (unfused); sum of three kernel medians", threads="", warmup=args.warmup,
                reps=args.reps, median_ms=total_ms, min_ms=sum(p[1]["min_ms"] for p in parts), std_ms="",
                metric="GFLOP/s", metric_value=gf, sm_clock_median_mhz=clk,
                clock_adjusted_metric=f"{pct:.2f}% of FP32 matrix peak at median clock (median of 3 kernel clocks)",
                alloc_bytes_per_call="", correctness="each kernel checked; see baseline part rows",
                notes="time excludes launch gaps between the three kernels")
        print(f"{'baseline':>12} {m}x{n}x{k}: {total_ms:.4f} ms {gf:9.0f} GFLOP/s {pct:5.1f}%", flush=True)
        for step, opts in STEPS:
            rung(step, m, n, k, opts)
        tuned = cm.tuned_options("mbr", m, n, k)
        rung("+autotuned", m, n, k, tuned, note="MI355X rung: autotuned (or cost-model) configuration")
        if tg.padded_shape(m, n, k, tuned) != (m, n, k):
            rung("+mask-edges", m, n, k, tuned + " mask-edges=1",
                 note="MI355X rung: true shape, edges masked in-kernel, no pad copies")
    print(f"failures: {failures}")
    return 1 if failures else 0


if __name__ == "__main__":
    sys.exit(main())
