#!/usr/bin/env python3
"""This backend's GEMM kernels against the vendor library's fp32 GEMM, back to
back, in one process on one GPU.

Four variants on the same device-resident inputs (the reference's seeded
draws, python/tforge_cpu.py:89-100):

  ours_fused        the fused relu(A @ B + bias) program, autotuned options
  ours_matmul       the plain matmul program, autotuned options
  torch_mm          torch.mm (hipBLASLt's fp32 GEMM on ROCm), TF32 off
  torch_addmm_relu  torch.addmm(bias, A, B) then relu_: the vendor's fused-
                    bias GEMM plus a separate ReLU kernel

After one second of untimed launches of all four, `--rounds` rounds alternate
the variants (reversed every other round); in each round a variant runs 20
untimed launches and then a `--steps`-launch window between two events on the
launch stream.  The median window per variant is reported, as bench.py times
its value.  Under rocprofv3 --kernel-trace the kernel names and durations of
both libraries come out of the same run.  Each variant's output is then
checked with the reference's FP64 bound (python/tforge_gpu.py:134-145, the
ReLU masks exact for the fused variants) on up to 256 evenly spaced rows,
and with --csv every variant becomes a row of a results table in the
reference's schema (python/provenance.py:11-16).

  python -m tensorforge_amd.bench.vendor_compare --shape 2048x2048x2048
  python -m tensorforge_amd.bench.vendor_compare --shape 1024x1024x1024,4096x4096x256 \
      --csv results/gpu/vendor_compare.csv
"""

import argparse
import json
import statistics
import sys
import time

VARIANTS = {  # name: (workload, pipeline column for the vendor's rows)
    "ours_fused": ("mbr", None),
    "ours_matmul": ("matmul", None),
    "torch_mm": ("matmul", "torch.mm fp32 (hipBLASLt), TF32 off"),
    "torch_addmm_relu": ("mbr", "torch.addmm fp32 (hipBLASLt, bias in the GEMM) + relu_ kernel, TF32 off"),
}


def bound_check(torch, a, b, bias, out, relu, rows=256):
    """err/bound of the reference check (python/tforge_gpu.py:134-145) on up
    to `rows` evenly spaced output rows, in float64 on the GPU, with the ReLU
    mask rule where `relu`."""
    m, k = a.shape
    idx = torch.linspace(0, m - 1, min(rows, m), device=a.device).long()
    a64, b64 = a[idx].double(), b.double()
    z, mag, steps = a64 @ b64, a64.abs() @ b64.abs(), k
    if relu:
        z, mag, steps = z + bias.double(), mag + bias.double().abs(), k + 1
    ref = torch.clamp_min(z, 0.0) if relu else z
    u = 2.0 ** -24
    bound = steps * u / (1 - steps * u) * mag + torch.finfo(torch.float32).tiny
    got = out[idx].double()
    eob = float(((got - ref).abs() / bound).max())
    masks = int(((z.abs() > bound) & ((got == 0) != (z <= 0))).sum()) if relu else 0
    ok = eob <= 1.0 and masks == 0 and not bool(torch.isnan(got).any())
    return ok, f"err/bound={eob:.3g} mask_mismatches={masks} rows={len(idx)}"


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--shape", default="2048x2048x2048", help="MxNxK, or several separated by commas")
    ap.add_argument("--rounds", type=int, default=8)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--csv", default=None, help="append one results row per variant and shape")
    args = ap.parse_args(argv)

    import torch
    from tensorforge_amd import provenance

    table = provenance.ResultsTable(args.csv) if args.csv else None
    rc = 0
    for shape in args.shape.split(","):
        rc |= compare(torch, args, shape, table)
    return rc


def compare(torch, args, shape, table):
    from tensorforge_amd import _lib
    from tensorforge_amd import costmodel as cm
    from tensorforge_amd import provenance
    from tensorforge_amd import tforge_cpu as tc

    m, n, k = (int(v) for v in shape.split("x"))
    dev = torch.device("cuda:0")
    torch.backends.cuda.matmul.allow_tf32 = False
    host = tc.make_inputs("mbr", m, n, k)
    a, b, bias = (torch.from_numpy(host[s]).to(dev) for s in ("a", "b", "bias"))
    c = torch.empty((m, n), device=dev)
    stream = torch.cuda.current_stream()
    fused = _lib.Kernel(tc.gen_mlir("mbr", m, n, k), cm.tuned_options("mbr", m, n, k))
    plain = _lib.Kernel(tc.gen_mlir("matmul", m, n, k), cm.tuned_options("matmul", m, n, k))
    pf = [a.data_ptr(), b.data_ptr(), bias.data_ptr(), c.data_ptr()]
    pm = [a.data_ptr(), b.data_ptr(), c.data_ptr()]
    variants = {
        "ours_fused": lambda: fused.launch(pf, stream.cuda_stream),
        "ours_matmul": lambda: plain.launch(pm, stream.cuda_stream),
        "torch_mm": lambda: torch.mm(a, b, out=c),
        "torch_addmm_relu": lambda: torch.addmm(bias, a, b, out=c).relu_(),
    }

    def window(fn, count):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(count):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / count

    t0 = time.time()
    while time.time() - t0 < 1.0:
        for fn in variants.values():
            fn()
    torch.cuda.synchronize()
    times = {name: [] for name in variants}
    names = list(variants)
    for r in range(args.rounds):
        for name in (names if r % 2 == 0 else names[::-1]):
            window(variants[name], 20)
            times[name].append(window(variants[name], args.steps))
        print(f"round {r}: " + ", ".join(f"{nm} {times[nm][-1] * 1e3:.2f} us" for nm in names), flush=True)
    clock = _lib.clock_probe(stream.cuda_stream)
    flops = 2.0 * m * n * k
    out = {"shape": shape, "options": {"ours_fused": fused.options, "ours_matmul": plain.options},
           "clock_mhz": clock}
    rc = 0
    for name, v in times.items():
        med = statistics.median(v)
        c.fill_(float("nan"))
        variants[name]()
        torch.cuda.synchronize()
        ok, verdict = bound_check(torch, a, b, bias, c, VARIANTS[name][0] == "mbr")
        rc |= 0 if ok else 1
        out[name] = {"us_per_launch": med * 1e3, "tflops": flops / (med * 1e-3) / 1e12, "check": verdict}
        if table is not None:
            workload, vendor = VARIANTS[name]
            opts = fused.options if name == "ours_fused" else plain.options
            table.add(device=provenance.device_label(_lib.device_info()), workload=workload, shape=shape,
                      dtype="f32", pipeline=vendor or f"tforge-gpu-pipeline{{{opts}}}", params=name, threads="",
                      warmup=20, reps=args.steps, median_ms=med, min_ms=min(v), std_ms=statistics.pstdev(v),
                      metric="GFLOP/s", metric_value=flops / (med * 1e-3) / 1e9, sm_clock_median_mhz=clock[0],
                      correctness=("PASS " if ok else "FAIL ") + verdict,
                      notes=f"back to back: median of {args.rounds} alternating windows of {args.steps} launches "
                            "after 20 untimed, one process with the other variants")
    print(json.dumps(out), flush=True)
    return rc


if __name__ == "__main__":
    sys.exit(main())
