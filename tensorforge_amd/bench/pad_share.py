#!/usr/bin/env python3
"""The padding share at shapes that are not tile multiples, and in-kernel masking.

The reference compiles staged kernels for the padded problem and pads on the
device inside the timed region (python/tforge_gpu.py:54-63;
runners/gpu/tforge-gpu-bench.cu:214-232, 292-302); it never measured the
copies' share (docs/stage8.md:117; docs/report.md:93).  For each shape and
configuration this times, on the same inputs:

  pad_path      the reference's path: pad copies + padded kernel + unpad copy,
                one event pair around all of it (tf_bench with a logical shape)
  padded_kernel the padded kernel alone on resident padded buffers
  masked        the kernel on the true shape with mask-edges=1 (no copies)

and reports pad_share = 1 - padded_kernel / pad_path and the masked kernel's
speedup over the pad path.  Every variant is checked against the FP64 bound
first, and the masked output must equal the pad path's bit for bit.

  python -m tensorforge_amd.bench.pad_share --csv results/gpu/pad_share.csv
"""

import argparse
import sys

import numpy as np

from tensorforge_amd import _lib
from tensorforge_amd import costmodel as cm
from tensorforge_amd import provenance
from tensorforge_amd import tforge_cpu as tc
from tensorforge_amd import tforge_gpu as tg
from tensorforge_amd.bench import harness

SHAPES = [(1000, 1000, 1000), (777, 1111, 333), (3000, 2000, 1000), (4095, 4097, 1023)]
REFERENCE = "block-tile=128,64 thread-tile=8,4 tile-k=16 promote=1 vectorize=1"  # docs/stage8.md:107


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--csv", default="results/gpu/pad_share.csv")
    ap.add_argument("--shapes", default="")
    ap.add_argument("--workload", default="mbr", choices=("mbr", "matmul"))
    ap.add_argument("--variant", action="append", default=[], help="NAME=OPTIONS (default: reference, tuned)")
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--reps", type=int, default=100)
    args = ap.parse_args(argv)
    shapes = SHAPES
    if args.shapes:
        shapes = [tuple(int(v) for v in s.split("x")) for s in args.shapes.split(",")]
    out = provenance.ResultsTable(args.csv, device=harness.device_label(), dtype="f32", threads="",
                                  alloc_bytes_per_call="", clock_adjusted_metric="")
    wl = args.workload
    failures = 0
    for m, n, k in shapes:
        variants = [v.split("=", 1) for v in args.variant] or [
            ("reference-128x64", REFERENCE), ("tuned", cm.tuned_options(wl, m, n, k))]
        ins = tc.make_inputs(wl, m, n, k)
        arrays = [np.ascontiguousarray(v) for v in ins.values()]
        flops = 2.0 * m * n * k
        for name, opts in variants:
            # the pad path is the reference's: no mask-edges, whatever the tuned options say
            opts = " ".join(t for t in opts.split() if not t.startswith("mask-edges"))
            pm, pn, pk = tg.padded_shape(m, n, k, opts)
            padded = _lib.Kernel(tc.gen_mlir(wl, pm, pn, pk), opts, "pad.mlir")
            masked = _lib.Kernel(tc.gen_mlir(wl, m, n, k), opts + " mask-edges=1", "mask.mlir")
            o_pad = np.empty((m, n), np.float32)
            o_mask = np.empty((m, n), np.float32)
            logical = None if (pm, pn, pk) == (m, n, k) else (m, n, k)
            padded.run(arrays, o_pad, logical=logical)
            masked.run(arrays, o_mask)
            chk = tg._bound_check(wl, ins, o_mask, k)
            same = int(np.count_nonzero(o_pad.view(np.uint32) != o_mask.view(np.uint32)))
            ok = chk["pass"] and tg._bound_check(wl, ins, o_pad, k)["pass"] and same == 0
            failures += not ok
            t_path = padded.bench(logical=logical, warmup=args.warmup, reps=args.reps)
            t_kern = padded.bench(warmup=args.warmup, reps=args.reps)
            t_mask = masked.bench(warmup=args.warmup, reps=args.reps)
            share = 1.0 - t_kern.median_ms / t_path.median_ms
            for label, r, pipe in (("pad_path", t_path, opts), ("padded_kernel", t_kern, opts),
                                   ("masked", t_mask, opts + " mask-edges=1")):
                gf = flops / (r.median_ms * 1e-3) / 1e9
                out.add(workload=wl, shape=f"{m}x{n}x{k}", pipeline=f"tforge-gpu-pipeline{{{pipe}}}",
                        params=f"{name}; {label}; padded={pm}x{pn}x{pk}", warmup=args.warmup,
                        reps=args.reps, median_ms=r.median_ms, min_ms=r.min_ms, std_ms=r.std_ms,
                        metric="GFLOP/s (logical shape)", metric_value=gf, sm_clock_median_mhz=r.clock_median_mhz,
                        correctness=f"err/bound={chk['err_over_bound']:.3g}; masked vs pad path bitwise diffs={same}",
                        notes=(f"pad_share={share:.3f}; masked speedup over pad path="
                               f"{t_path.median_ms / t_mask.median_ms:.3f}"))
            print(f"{m}x{n}x{k} {name:>18}: pad path {t_path.median_ms * 1e3:8.1f} us, padded kernel "
                  f"{t_kern.median_ms * 1e3:8.1f} us (pad share {100 * share:4.1f}%), masked "
                  f"{t_mask.median_ms * 1e3:8.1f} us ({flops / t_mask.median_ms / 1e9:6.1f} TFLOP/s, "
                  f"{t_path.median_ms / t_mask.median_ms:.2f}x), bitwise diffs {same}, "
                  f"err/bound {chk['err_over_bound']:.3g}", flush=True)
    print(f"failures: {failures}")
    return 1 if failures else 0


if __name__ == "__main__":
    sys.exit(main())
