#!/usr/bin/env python3
"""Correctness-then-timing table of TensorForge kernels on MI355X, with rocBLAS
beside them.

Command line and CSV columns are the reference driver's (bench/gpu_bench.py:
--csv --tag --variant NAME=OPTIONS --workloads --shapes --warmup --reps --flush
--cublas --check-only; the provenance columns of python/provenance.py:11-16),
so existing scripts and result readers work unchanged; --rocblas is an alias
of --cublas.

For every workload x shape the driver first runs rocBLAS once on the seeded
inputs (the column `max|x-rocblas|` compares each variant with it), then for
each variant: compile, one checked run (FP64 bound with exact ReLU masks for
matmul / mbr, bit-exact for element ops), and -- only if it passed -- timing
with tf_bench (10 warm-up + 100 reps, one HIP event pair per rep, median; the
shader clock measured on the device after each rep).  A variant's options may
be `@tuned` or `@tuned-masked` (see harness.resolve_options).  Products report
GFLOP/s and % of the FP32 matrix peak (nominal and at the measured clock);
element ops report GB/s of compulsory traffic and % of 8 TB/s.

  python -m tensorforge_amd.bench.gpu_bench --csv results/gpu/stage8_mi355x.csv --tag stage8 \\
      --variant tuned=@tuned-masked --cublas
"""

import argparse
import sys

import numpy as np

from tensorforge_amd import provenance
from tensorforge_amd.bench import harness

# The reference's default shape list (bench/gpu_bench.py), kept so tables line up.
DEFAULT_SHAPES = [(256, 256, 256), (512, 512, 512), (1024, 1024, 1024), (2048, 2048, 2048),
                  (4096, 4096, 4096), (1000, 1000, 1000), (777, 1111, 333)]


def cli():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--csv", required=True)
    ap.add_argument("--tag", required=True, help="artifact subdirectory of this run")
    ap.add_argument("--variant", action="append", default=[], metavar="NAME=OPTIONS")
    ap.add_argument("--workloads", default="matmul,mbr")
    ap.add_argument("--shapes", default="", help="MxNxK,... (MxN for element ops)")
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--reps", type=int, default=100)
    ap.add_argument("--flush", action="store_true", help="512 MiB L2/MALL flush before every rep")
    ap.add_argument("--cublas", "--rocblas", dest="blas", action="store_true",
                    help="also time rocBLAS sgemm (+ a separate epilogue kernel for mbr)")
    ap.add_argument("--check-only", action="store_true")
    return ap


def plan(workload, shape, variants, with_blas):
    """The jobs of one workload x shape, in table order."""
    m, n, k = shape
    for name, spec in variants:
        yield harness.Job(workload, m, n, k, name, harness.resolve_options(spec, workload, m, n, k))
    if with_blas and workload in harness.GEMM_WORKLOADS:
        yield harness.Job(workload, m, n, k, "rocblas", mode="rocblas")


def main(argv=None):
    args = cli().parse_args(argv)
    variants = harness.parse_variants(args.variant)
    table = None if args.check_only else provenance.ResultsTable(args.csv)
    failed = 0
    for workload in args.workloads.split(","):
        for shape in harness.parse_shapes(args.shapes, DEFAULT_SHAPES):
            problem = harness.Problem(workload, *shape)
            vendor = None
            if workload in harness.GEMM_WORKLOADS:
                vendor = harness.measure(harness.Job(workload, *shape, "rocblas", mode="rocblas"), problem,
                                         timed=False).output.astype(np.float64)
            for job in plan(workload, shape, variants, args.blas):
                res = harness.measure(job, problem, args.warmup, args.reps, args.flush, timed=table is not None,
                                      tag=args.tag)
                gap = "" if vendor is None else f"max|x-rocblas|={np.nanmax(np.abs(res.output - vendor)):.3g}"
                print(harness.status_line(res, gap), flush=True)
                if not res.passed:
                    failed += 1
                    continue
                if table is None:
                    continue
                table.add(**res.row(correctness=f"err/bound={res.verdict['err_over_bound']:.3g}; {gap}".rstrip("; ")))
                print(harness.timing_line(res), flush=True)
    print(f"failures: {failed}")
    return 1 if failed else 0


if __name__ == "__main__":
    sys.exit(main())
