#!/usr/bin/env python3
"""A device-to-device copy of known size, for calibrating HBM byte counters.

rocprofv3 --pmc FETCH_SIZE (or WRITE_SIZE) over this program reports the
counter for a kernel whose algorithmic traffic is exactly `--mib` MiB read and
`--mib` MiB written; the ratio counter / known bytes is the scale factor
applied to the same counter on the GEMM kernel.

  rocprofv3 --pmc FETCH_SIZE -d out -o copy -- python3 tensorforge_amd/bench/copy_calibration.py --mib 256
"""

import argparse

import torch


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--mib", type=int, default=256)
    ap.add_argument("--reps", type=int, default=5)
    a = ap.parse_args()
    n = a.mib * (1 << 20) // 4
    src = torch.ones(n, device="cuda:0", dtype=torch.float32)
    dst = torch.empty_like(src)
    for _ in range(a.reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(f"copied {a.mib} MiB x {a.reps}", flush=True)


if __name__ == "__main__":
    main()
