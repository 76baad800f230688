#!/usr/bin/env python3
"""GPU correctness + timing driver for TensorForge kernels on MI355X (and rocBLAS).

Same command line, shapes and CSV rows as the reference's bench/gpu_bench.py
(bench/gpu_bench.py:1-103).  Every (variant, workload, shape) is compiled and
checked before timing:
  - pass/fail: FP64 reference with the gamma_{K+1} bound (and exact ReLU masks)
  - reported: max |kernel - rocBLAS| on the same inputs
Timing: 10 warm-up + 100 reps (HIP events), median; GPU clock sampled per rep
through amdsmi; clock-adjusted metric = % of the FP32 matrix peak at the median
clock (256 CUs x 256 FLOP/clk); element-op workloads (add, bias_add, relu)
report GB/s of compulsory traffic and % of the 8 TB/s HBM peak.  --cublas (alias --rocblas) also times rocBLAS
sgemm plus a separate epilogue kernel, the counterpart of the reference's
cuBLAS row.

  python -m tensorforge_amd.bench.gpu_bench --csv results/gpu/stage8.csv --tag stage8 \\
      --variant full-128x128-t8x8-k32="block-tile=128,128 thread-tile=8,8 tile-k=32 promote=1 vectorize=1" \\
      --cublas

A variant's options may be @tuned (per shape: the autotuned options, else the cost model's pick) or
@tuned-masked (the same, with mask-edges where the shape is not a tile multiple).
"""

import argparse
import sys

import numpy as np

from tensorforge_amd import costmodel as cm
from tensorforge_amd import provenance
from tensorforge_amd import tforge_cpu as tc
from tensorforge_amd import tforge_gpu as tg

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, AMD's published figure

SHAPES = [(256, 256, 256), (512, 512, 512), (1024, 1024, 1024), (2048, 2048, 2048),
          (4096, 4096, 4096), (1000, 1000, 1000), (777, 1111, 333)]


def shape_str(m, n, k):
    return f"{m}x{n}x{k}"


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--csv", required=True)
    ap.add_argument("--tag", required=True)
    ap.add_argument("--variant", action="append", default=[])
    ap.add_argument("--workloads", default="matmul,mbr")
    ap.add_argument("--shapes", default="")
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--reps", type=int, default=100)
    ap.add_argument("--flush", action="store_true")
    ap.add_argument("--cublas", "--rocblas", dest="blas", action="store_true",
                    help="also time rocBLAS (+ separate epilogue)")
    ap.add_argument("--check-only", action="store_true")
    args = ap.parse_args(argv)

    variants = [v.split("=", 1) for v in args.variant]
    shapes = SHAPES
    if args.shapes:
        # MxNxK, or MxN for element-op workloads (K = 0, as the CSV rows write it)
        shapes = [tuple(int(x) for x in s.split("x")) for s in args.shapes.split(",")]
        bad = [s for s in shapes if len(s) not in (2, 3)]
        if bad:
            ap.error(f"--shapes takes MxNxK or MxN, got {args.shapes}")
        shapes = [s if len(s) == 3 else s + (0,) for s in shapes]
    base = provenance.common()
    out = None if args.check_only else provenance.CsvWriter(args.csv)
    failures = 0

    for workload in args.workloads.split(","):
        for m, n, k in shapes:
            unit, work = tc.flops_or_bytes(workload, m, n, k)
            elementwise = unit == "GB/s"
            ref_blas = None
            if workload in ("matmul", "mbr"):
                _, ref_blas = tg.check(workload, m, n, k, mode="rocblas")
            rows = []
            for name, opts in variants:
                # @tuned: the autotuned (else cost-model) options of this shape; @tuned-masked: the same
                # with mask-edges on shapes that are not tile multiples.
                if opts in ("@tuned", "@tuned-masked") and workload in ("matmul", "mbr"):
                    t = cm.tuned_options(workload, m, n, k)
                    if opts == "@tuned-masked" and tg.padded_shape(m, n, k, t) != (m, n, k):
                        t += " mask-edges=1"
                    opts = t
                rows.append((name, opts, "kernel"))
            if args.blas and workload in ("matmul", "mbr"):
                rows.append(("rocblas", "", "rocblas"))
            for name, opts, mode in rows:
                kdir = launch = None
                res_info = {}
                if mode == "kernel":
                    kdir, launch = tg.compile_kernel(workload, m, n, k, opts, tag=f"{args.tag}/{name}")
                    res_info = tg.ptxas_resources(kdir)
                chk, got = tg.check(workload, m, n, k, kdir, launch, mode)
                diff = float(np.nanmax(np.abs(got.astype(np.float64) - ref_blas))) if ref_blas is not None else 0.0
                status = "PASS" if chk["pass"] else "FAIL"
                print(f"[{status}] {name:>22} {workload:>6} {shape_str(m, n, k):>16} "
                      f"err/bound={chk['err_over_bound']:.3g} max|x-rocblas|={diff:.3g}", flush=True)
                if not chk["pass"]:
                    failures += 1
                    continue
                if out is None:
                    continue
                r = tg.bench(workload, m, n, k, kdir, launch, mode, args.warmup, args.reps, args.flush)
                gflops = work / (r["median_ms"] * 1e-3) / 1e9  # GFLOP/s, or GB/s for element ops
                clk = r["sm_clock_median_mhz"]
                if elementwise:
                    pct = pct_nominal = 100.0 * gflops / HBM_PEAK_GBS
                else:
                    pct = 100.0 * gflops / tg.fp32_peak_gflops(clk) if clk > 0 else float("nan")
                    pct_nominal = 100.0 * gflops / tg.fp32_peak_gflops(tg.PEAK_CLOCK_MHZ)
                launch_str = f"grid={r['grid']} block={r['block']} padded={r['padded']}"
                res = (f"regs={r['regs']} local={r['local_bytes']} smem={r['static_smem']} "
                       f"blocks/SM={r['blocks_per_sm']} occ={r['theo_occupancy']}")
                if res_info:
                    res += (f" spill_st={res_info['spill_stores']} spill_ld={res_info['spill_loads']} "
                            f"agprs={res_info['agprs']}")
                pipeline = (f"tforge-gpu-pipeline{{{opts}}}" if mode == "kernel" else
                            "rocblas_sgemm FP32" + (" + epilogue kernel" if workload == "mbr" else ""))
                out.row(**base, device=r["gpu"], workload=workload, shape=shape_str(m, n, k),
                        dtype="f32", pipeline=pipeline, params=f"{name}; {launch_str}; {res}",
                        threads="", warmup=r["warmup"], reps=r["reps"], median_ms=r["median_ms"],
                        min_ms=r["min_ms"], std_ms=r["std_ms"], metric=unit,
                        metric_value=gflops, sm_clock_median_mhz=clk,
                        clock_adjusted_metric=(f"{pct:.2f}% of 8 TB/s HBM (compulsory bytes)" if elementwise else
                                               f"{pct:.2f}% of FP32 matrix peak at median clock; "
                                               f"{pct_nominal:.2f}% of 157.3 TFLOP/s"),
                        alloc_bytes_per_call="",
                        correctness=f"err/bound={chk['err_over_bound']:.3g}; max|x-rocblas|={diff:.3g}",
                        notes=(f"l2_flush={r['l2_flush']}; gfx clock {r['sm_clock_min_mhz']}-"
                               f"{r['sm_clock_max_mhz']} MHz; power {r['power_median_w']} W; "
                               f"hip driver {r['hip_driver']}"))
                print(f"        median {r['median_ms']:.4f} ms  {gflops:.1f} {unit}  "
                      f"{pct_nominal:.1f}% of peak ({pct:.1f}% @ {clk:.0f} MHz)  {res}", flush=True)
    print(f"failures: {failures}")
    return 1 if failures else 0


if __name__ == "__main__":
    sys.exit(main())
