#!/usr/bin/env python3
"""E1 on MI355X: which kernel variants change floating-point results, and by how much.

The reference's E1 (bench/e1_numerics.py:1-15, 93-104), same shapes, inputs
and columns.  For relu(A @ B + bias) and plain matmul, every variant runs on
the same inputs; reported per variant: max |x - x64|, RMS |x - x64|,
max |x - x64| / bound against the FP64 reference (bound = gamma_{K+1}
(|A||B| + |bias|), valid for any summation order), and the number and
fraction of outputs that differ bitwise from the CPU scalar form (sequential
k, product rounded before the add) and from the GPU naive kernel.

Variants:
  cpu-scalar       the reference CPU default pipeline's arithmetic, evaluated
                   here in NumPy float32 (one rounded multiply and one rounded
                   add per k, in k order; IEEE maximum) -- the bitwise anchor
  numpy-openblas   NumPy matmul (+ add, maximum), 1 BLAS thread
  gpu-naive        the direct kernel (tile-k=0): one FMA per k in k order, the
                   reference's naive kernel arithmetic, so its row should
                   equal the reference's gpu-naive row
  gpu-staged-bk8/16/32   the reference's staged configurations, here FP32 MFMA
  gpu-autotuned    the recorded autotuned configuration (split-K included)
  gpu-split-k4     the bk16 configuration with split-k=4
  gpu-mask-edges   the bk16 configuration on the true shape, edges masked
  rocblas          rocBLAS sgemm (+ the separate epilogue kernel)
The reference's CPU fused/tiled/vectorized pipeline rows are not rebuilt
(the CPU pipeline is not part of this backend).

  python -m tensorforge_amd.bench.e1_numerics --csv results/numerics/e1_mi355x.csv
"""

import argparse
import csv
import os
import pathlib
import sys

os.environ.setdefault("OPENBLAS_NUM_THREADS", "1")
import numpy as np  # noqa: E402

from tensorforge_amd import _lib  # noqa: E402
from tensorforge_amd import costmodel as cm  # noqa: E402
from tensorforge_amd import provenance  # noqa: E402
from tensorforge_amd import tforge_cpu as tc  # noqa: E402
from tensorforge_amd import tforge_gpu as tg  # noqa: E402

SHAPES = [(256, 256, 256), (1000, 1000, 1000), (777, 1111, 333), (512, 512, 4096)]
STAGED = "block-tile=128,64 thread-tile=8,4 tile-k={} promote=1 vectorize=1"
GPU = [("gpu-naive", "block-tile=16,16 thread-tile=1,1"),
       ("gpu-staged-bk8", STAGED.format(8)), ("gpu-staged-bk16", STAGED.format(16)),
       ("gpu-staged-bk32", STAGED.format(32))]


def relu_ieee(x):
    return np.where((x > 0) | np.isnan(x), x, np.float32(0))


def cpu_scalar(workload, ins):
    """Sequential k, float32 product then float32 add, from +0.0."""
    a, b = ins["a"], ins["b"]
    c = np.zeros((a.shape[0], b.shape[1]), np.float32)
    for kk in range(a.shape[1]):
        c = c + a[:, kk:kk + 1] * b[kk:kk + 1, :]
    if workload == "mbr":
        c = relu_ieee(c + ins["bias"])
    return c


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--csv", default="results/numerics/e1_mi355x.csv")
    ap.add_argument("--shapes", default="")
    args = ap.parse_args(argv)
    shapes = SHAPES
    if args.shapes:
        shapes = [tuple(int(v) for v in s.split("x")) for s in args.shapes.split(",")]
    base = provenance.common()
    path = pathlib.Path(args.csv)
    path.parent.mkdir(parents=True, exist_ok=True)
    f = open(path, "w", newline="")
    w = csv.writer(f)
    w.writerow(["commit", "llvm_version", "hip_version", "job_id", "date", "device", "workload",
                "shape", "dtype", "variant", "pipeline", "max_abs_err", "rms_err", "max_err_over_bound",
                "bitwise_diff_vs_cpu_scalar", "bitwise_diff_fraction", "max_abs_diff_vs_cpu_scalar",
                "bitwise_diff_vs_gpu_naive"])
    cpu_dev = provenance.cpu_model()
    dev = _lib.device_info()
    gpu_dev = dev["name"] or dev["arch"]
    failures = 0
    for workload in ("mbr", "matmul"):
        for m, n, k in shapes:
            ins = tc.make_inputs(workload, m, n, k)
            a64, b64 = ins["a"].astype(np.float64), ins["b"].astype(np.float64)
            ref, mag, steps = a64 @ b64, np.abs(a64) @ np.abs(b64), k
            if workload == "mbr":
                bias64 = ins["bias"].astype(np.float64)
                ref, mag, steps = np.maximum(ref + bias64, 0), mag + np.abs(bias64), k + 1
            bound = steps * tc.F32_EPS / (1 - steps * tc.F32_EPS) * mag + np.finfo(np.float32).tiny
            outs = [("cpu-scalar", "tforge-cpu-pipeline{} arithmetic (NumPy float32)", cpu_dev,
                     cpu_scalar(workload, ins))]
            npo = ins["a"] @ ins["b"]
            if workload == "mbr":
                npo = np.maximum(npo + ins["bias"], np.float32(0))
            outs.append(("numpy-openblas", "numpy matmul (+ add, maximum), 1 thread", cpu_dev, npo))
            gpu = list(GPU) + [("gpu-autotuned", cm.tuned_options(workload, m, n, k)),
                               ("gpu-split-k4", STAGED.format(16) + " split-k=4"),
                               ("gpu-mask-edges", STAGED.format(16) + " mask-edges=1")]
            for name, opts in gpu:
                d, launch = tg.compile_kernel(workload, m, n, k, opts, tag=f"e1/{name}")
                res, o = tg.check(workload, m, n, k, d, launch)
                failures += not res["pass"]
                outs.append((name, f"tforge-gpu-pipeline{{{opts}}}", gpu_dev, o))
            res, o = tg.check(workload, m, n, k, mode="cublas")
            failures += not res["pass"]
            outs.append(("rocblas", "rocblas_sgemm FP32" + (" + bias_relu kernel" if workload == "mbr" else ""),
                         gpu_dev, o))
            scalar = outs[0][3]
            naive = next(o for nm, _, _, o in outs if nm == "gpu-naive")
            for name, pipe, devname, o in outs:
                err = np.abs(o.astype(np.float64) - ref)
                diff = int(np.count_nonzero(o.view(np.uint32) != scalar.view(np.uint32)))
                diff_naive = int(np.count_nonzero(o.view(np.uint32) != naive.view(np.uint32)))
                w.writerow([base["commit"], base["mlir_llvm_version"], base["cuda_version"], base["job_id"],
                            base["date"], devname, workload, f"{m}x{n}x{k}", "f32", name, pipe,
                            f"{err.max():.4g}", f"{np.sqrt((err ** 2).mean()):.4g}",
                            f"{(err / bound).max():.4g}", diff, f"{diff / o.size:.4f}",
                            f"{np.abs(o.astype(np.float64) - scalar).max():.4g}", diff_naive])
                print(f"{workload} {m}x{n}x{k} {name:>16}: max_err={err.max():.3g} "
                      f"err/bound={(err / bound).max():.3g} bitwise-diff={diff / o.size:.3f} "
                      f"vs-naive={diff_naive / o.size:.3f}", flush=True)
            f.flush()
    print(f"failures: {failures}")
    return 1 if failures else 0


if __name__ == "__main__":
    sys.exit(main())
