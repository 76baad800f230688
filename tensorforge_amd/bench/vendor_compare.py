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
both libraries come out of the same run.

  python -m tensorforge_amd.bench.vendor_compare --shape 2048x2048x2048
"""

import argparse
import json
import statistics
import sys
import time


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--shape", default="2048x2048x2048")
    ap.add_argument("--rounds", type=int, default=8)
    ap.add_argument("--steps", type=int, default=200)
    args = ap.parse_args(argv)
    m, n, k = (int(v) for v in args.shape.split("x"))

    import torch
    from tensorforge_amd import _lib
    from tensorforge_amd import costmodel as cm
    from tensorforge_amd import tforge_cpu as tc

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
    flops = 2.0 * m * n * k
    out = {"shape": args.shape, "options": {"ours_fused": fused.options, "ours_matmul": plain.options},
           "clock_mhz": _lib.clock_probe(stream.cuda_stream)}
    for name, v in times.items():
        med = statistics.median(v)
        out[name] = {"us_per_launch": med * 1e3, "tflops": flops / (med * 1e-3) / 1e12}
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
