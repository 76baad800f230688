#!/usr/bin/env python3
"""Numerics of every kernel variant on MI355X: how far each output is from
FP64, and which variants change the float32 bits.

For relu(A @ B + bias) and plain matmul on the reference's E1 shapes and
seeded inputs, each variant's output is compared with the FP64 reference and
with two float32 anchors.  Columns and variant names are the reference's E1
table (bench/e1_numerics.py, results/numerics/e1.csv), so the tables line up
row by row:

  max_abs_err, rms_err, max_err_over_bound   |x - x64| against the FP64
        reference; bound = gamma_{K(+1)} (|A||B| (+ |bias|)) + FLT_MIN, valid
        for any summation order
  bitwise_diff_vs_cpu_scalar (+ fraction)    outputs whose bits differ from the
        CPU scalar form: k in order from +0.0, each product rounded to float32
        before its add (the reference CPU pipeline's default arithmetic)
  bitwise_diff_vs_gpu_naive                  ... from the direct kernel (one FMA
        per k in order: the reference GPU kernels' arithmetic)

Variants here: cpu-scalar and numpy-openblas (1 thread) on the host; the
direct kernel (gpu-naive); the reference's staged configurations
(gpu-staged-bk8/16/32, FP32 MFMA here); the autotuned configuration; split-K
and mask-edges (backend options); rocBLAS (+ the epilogue kernel).  The
reference's CPU fused / tiled / vectorized pipeline rows are not rebuilt: the
CPU pipeline is not part of this backend.

  python -m tensorforge_amd.bench.e1_numerics --csv results/numerics/e1_mi355x.csv
"""

import argparse
import csv
import os
import pathlib
import sys

os.environ.setdefault("OPENBLAS_NUM_THREADS", "1")
import numpy as np  # noqa: E402

from tensorforge_amd import costmodel as cm  # noqa: E402
from tensorforge_amd import provenance  # noqa: E402
from tensorforge_amd.bench import harness  # noqa: E402

DEFAULT_SHAPES = [(256, 256, 256), (1000, 1000, 1000), (777, 1111, 333), (512, 512, 4096)]
COLUMNS = ["commit", "llvm_version", "hip_version", "job_id", "date", "device", "workload",
           "shape", "dtype", "variant", "pipeline", "max_abs_err", "rms_err", "max_err_over_bound",
           "bitwise_diff_vs_cpu_scalar", "bitwise_diff_fraction", "max_abs_diff_vs_cpu_scalar",
           "bitwise_diff_vs_gpu_naive"]
REF_STAGED = "block-tile=128,64 thread-tile=8,4 tile-k={} promote=1 vectorize=1"


def scalar_form(workload, ins):
    """The CPU scalar arithmetic in float32: acc = +0; for k in order:
    acc += fl(a[:, k] * b[k, :]); then + bias and IEEE maximum with +0."""
    a, b = ins["a"], ins["b"]
    acc = np.zeros((a.shape[0], b.shape[1]), np.float32)
    prod = np.empty_like(acc)
    for kk in range(a.shape[1]):
        np.multiply(a[:, kk, None], b[None, kk, :], out=prod)
        np.add(acc, prod, out=acc)
    if workload == "mbr":
        np.add(acc, ins["bias"], out=acc)
        acc = np.where(np.isnan(acc) | (acc > 0), acc, np.float32(0)).astype(np.float32)
    return acc


def numpy_form(workload, ins):
    out = np.matmul(ins["a"], ins["b"])
    if workload == "mbr":
        np.add(out, ins["bias"], out=out)
        np.maximum(out, np.float32(0), out=out)
    return out


def gpu_variants(workload, m, n, k):
    """(variant, options or None for rocBLAS) in table order."""
    yield "gpu-naive", "block-tile=16,16 thread-tile=1,1"
    for bk in (8, 16, 32):
        yield f"gpu-staged-bk{bk}", REF_STAGED.format(bk)
    yield "gpu-autotuned", cm.tuned_options(workload, m, n, k)
    yield "gpu-split-k4", REF_STAGED.format(16) + " split-k=4"
    yield "gpu-mask-edges", REF_STAGED.format(16) + " mask-edges=1"
    yield "rocblas", None


def statistics(out, ref, bound, scalar, naive):
    err = np.abs(out.astype(np.float64) - ref)
    bits = out.view(np.uint32)
    diff = int(np.count_nonzero(bits != scalar.view(np.uint32)))
    return {"max_abs_err": f"{err.max():.4g}", "rms_err": f"{np.sqrt(np.mean(err * err)):.4g}",
            "max_err_over_bound": f"{(err / bound).max():.4g}", "bitwise_diff_vs_cpu_scalar": diff,
            "bitwise_diff_fraction": f"{diff / out.size:.4f}",
            "max_abs_diff_vs_cpu_scalar": f"{np.abs(out.astype(np.float64) - scalar).max():.4g}",
            "bitwise_diff_vs_gpu_naive": int(np.count_nonzero(bits != naive.view(np.uint32)))}


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--csv", default="results/numerics/e1_mi355x.csv")
    ap.add_argument("--shapes", default="")
    args = ap.parse_args(argv)
    base = provenance.common()
    shared = {"commit": base["commit"], "llvm_version": base["mlir_llvm_version"], "hip_version": base["cuda_version"],
              "job_id": base["job_id"], "date": base["date"], "dtype": "f32"}
    path = pathlib.Path(args.csv)
    path.parent.mkdir(parents=True, exist_ok=True)
    host = provenance.cpu_model()
    failed = 0
    with open(path, "w", newline="") as fh:
        table = csv.DictWriter(fh, fieldnames=COLUMNS)
        table.writeheader()
        for workload in ("mbr", "matmul"):
            for m, n, k in harness.parse_shapes(args.shapes, DEFAULT_SHAPES):
                problem = harness.Problem(workload, m, n, k)
                ref, bound, _ = problem.reference()
                outputs = [("cpu-scalar", "tforge-cpu-pipeline{} arithmetic (NumPy float32)", host,
                            scalar_form(workload, problem.ins)),
                           ("numpy-openblas", "numpy matmul (+ add, maximum), 1 thread", host,
                            numpy_form(workload, problem.ins))]
                for variant, opts in gpu_variants(workload, m, n, k):
                    job = (harness.Job(workload, m, n, k, variant, opts) if opts is not None else
                           harness.Job(workload, m, n, k, variant, mode="rocblas"))
                    res = harness.measure(job, problem, timed=False, tag="e1")
                    failed += not res.passed
                    outputs.append((variant, job.pipeline, harness.device_label(), res.output))
                scalar = outputs[0][3]
                naive = next(out for name, _, _, out in outputs if name == "gpu-naive")
                for variant, pipeline, device, out in outputs:
                    row = statistics(out, ref, bound, scalar, naive)
                    table.writerow({**shared, "device": device, "workload": workload, "shape": f"{m}x{n}x{k}",
                                    "variant": variant, "pipeline": pipeline, **row})
                    print(f"{workload} {m}x{n}x{k} {variant:>16}: max_err={row['max_abs_err']} "
                          f"err/bound={row['max_err_over_bound']} bitwise-diff={row['bitwise_diff_fraction']} "
                          f"vs-naive={row['bitwise_diff_vs_gpu_naive']}", flush=True)
                fh.flush()
    print(f"failures: {failed}")
    return 1 if failed else 0


if __name__ == "__main__":
    sys.exit(main())
