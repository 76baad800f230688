#!/usr/bin/env python3
"""What each optimisation buys for relu(A @ B + bias) on MI355X: an ablation
ladder from three unfused naive kernels to the autotuned fused kernel.

Rungs (the first five are the reference's, by name and meaning --
bench/stage9_ablation.py -- so the two tables line up row by row):

  baseline    matmul, bias_add and relu as three direct kernels (16x16 blocks,
              one output per thread); time = the sum of the three medians,
              each kernel checked on its own
  +fusion     one direct kernel with the epilogue fused
  +tiling     the reference's default tiles, 128x64 blocks, 8x4 per thread,
              K step 16, as FP32 MFMA on fragments read from global memory
  +promotion  ... with the A and B slabs staged through LDS
  +vectorize  ... with 128-bit global and LDS accesses
  +autotuned  (MI355X) the configuration recorded for the shape by the
              autotuner (else the cost model's pick), split-K included
  +mask-edges (MI355X, shapes that are not tile multiples) the autotuned kernel
              on the true shape, edges masked in-kernel instead of padded

Rows use the results columns of the other drivers; the rate of every rung,
the baseline's parts included, is GFLOP/s of the whole mbr (2*M*N*K).

  python -m tensorforge_amd.bench.stage9_ablation --csv results/gpu/stage9_ablation.csv
"""

import argparse
import sys

from tensorforge_amd import costmodel as cm
from tensorforge_amd import provenance
from tensorforge_amd import tforge_gpu as tg
from tensorforge_amd.bench import harness

DEFAULT_SHAPES = [(1024, 1024, 1024), (2048, 2048, 2048), (4096, 4096, 4096), (777, 1111, 333)]
NAIVE = "block-tile=16,16 thread-tile=1,1"
REFERENCE_TILES = "block-tile=128,64 thread-tile=8,4 tile-k=16"  # the reference's default configuration


def rungs(m, n, k):
    """(rung, options, note) of the fused rungs, in ladder order."""
    yield "+fusion", NAIVE, ""
    for rung, promote, vectorize in (("+tiling", 0, 0), ("+promotion", 1, 0), ("+vectorize", 1, 1)):
        yield rung, f"{REFERENCE_TILES} promote={promote} vectorize={vectorize}", ""
    tuned = cm.tuned_options("mbr", m, n, k)
    yield "+autotuned", tuned, "MI355X rung: autotuned (or cost-model) configuration"
    if tg.padded_shape(m, n, k, tuned) != (m, n, k):
        yield "+mask-edges", tuned + " mask-edges=1", "MI355X rung: true shape, edges masked in-kernel, no pad copies"


def mbr_rate(m, n, k, ms):
    return 2.0 * m * n * k / (ms * 1e-3) / 1e9


def unfused_baseline(m, n, k, warmup, reps, table):
    """The three unfused kernels; returns (passed, total median ms)."""
    parts = [harness.measure(harness.Job(wl, m, n, kk, f"baseline-{wl}", NAIVE), warmup=warmup, reps=reps,
                             tag="stage9abl")
             for wl, kk in (("matmul", k), ("bias_add", 0), ("relu", 0))]
    if not all(p.passed for p in parts):
        return False, None
    total = sum(p.timing["median_ms"] for p in parts)
    for p in parts:
        table.add(**p.row(workload=p.job.workload, shape=f"{m}x{n}x{k}", params=f"baseline part: {p.job.workload}; "
                          f"{p.describe()}", metric="GFLOP/s (of the full mbr)",
                          metric_value=mbr_rate(m, n, k, p.timing["median_ms"]),
                          notes="one of three unfused kernels; metric uses the mbr FLOP count"))
    clocks = sorted(p.timing["sm_clock_median_mhz"] for p in parts)
    gf = mbr_rate(m, n, k, total)
    table.add(device=harness.device_label(), workload="mbr", shape=f"{m}x{n}x{k}", dtype="f32",
              pipeline=f"tforge-gpu-pipeline{{{NAIVE}}} x3 kernels (matmul, bias_add, relu)",
              params="baseline (unfused); sum of three kernel medians", warmup=warmup, reps=reps, median_ms=total,
              min_ms=sum(p.timing["min_ms"] for p in parts), metric="GFLOP/s", metric_value=gf,
              sm_clock_median_mhz=clocks[1],
              clock_adjusted_metric=f"{100.0 * gf / tg.fp32_peak_gflops(clocks[1]):.2f}% of FP32 matrix peak at the "
                                    "median of the three kernels' clocks",
              correctness="each kernel checked; see the baseline part rows",
              notes="time excludes launch gaps between the three kernels")
    return True, total


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--csv", default="results/gpu/stage9_ablation.csv")
    ap.add_argument("--shapes", default="")
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--reps", type=int, default=100)
    args = ap.parse_args(argv)
    table = provenance.ResultsTable(args.csv)
    failed = 0
    for m, n, k in harness.parse_shapes(args.shapes, DEFAULT_SHAPES):
        ok, total = unfused_baseline(m, n, k, args.warmup, args.reps, table)
        if not ok:
            failed += 1
            print(f"[FAIL] baseline {m}x{n}x{k}", flush=True)
        else:
            print(f"{'baseline':>12} {m}x{n}x{k}: {total:.4f} ms {mbr_rate(m, n, k, total):9.0f} GFLOP/s", flush=True)
        problem = harness.Problem("mbr", m, n, k)
        for rung, opts, note in rungs(m, n, k):
            res = harness.measure(harness.Job("mbr", m, n, k, rung, opts), problem, args.warmup, args.reps,
                                  tag="stage9abl")
            if not res.passed:
                failed += 1
                print(f"[FAIL] {rung} {m}x{n}x{k}", flush=True)
                continue
            table.add(**res.row(params=f"{rung}; {res.describe()}", metric="GFLOP/s (of the full mbr)", notes=note))
            nominal, at_clock = res.shares()
            print(f"{rung:>12} {m}x{n}x{k}: {res.timing['median_ms']:.4f} ms {res.rate()[1]:9.0f} GFLOP/s "
                  f"{at_clock:5.1f}%  [{opts}]", flush=True)
    print(f"failures: {failed}")
    return 1 if failed else 0


if __name__ == "__main__":
    sys.exit(main())
