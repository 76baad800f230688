#!/usr/bin/env python3
"""A device-to-device copy of known size, for calibrating HBM byte counters.

rocprofv3 --pmc FETCH_SIZE (or WRITE_SIZE) over this program reports the
counter for a kernel whose algorithmic traffic is exactly `--mib` MiB read and
`--mib` MiB written; the ratio counter / known bytes is the scale factor
applied to the same counter on the GEMM kernel.

  rocprofv3 --pmc FETCH_SIZE -d out -o copy -- python3 tensorforge_amd/bench/copy_calibration.py --mib 256

With --write-rate it instead times a store-only stream (torch's fill kernel)
of --mib MiB, the HBM write rate one round of a GEMM's C tiles can reach.
"""

import argparse

import torch


def write_rate(mib, reps):
    """HBM write rate of a store-only stream of `mib` MiB (torch's fill
    kernel): median per launch between its own event pair, and back to back
    over `reps` launches.  The size of one round of C tiles of a GEMM shows
    what its epilogue's store burst can reach."""
    import statistics
    buf = torch.empty(mib * (1 << 20) // 4, device="cuda:0", dtype=torch.float32)
    for _ in range(50):
        buf.fill_(1.0)
    ev = lambda: torch.cuda.Event(enable_timing=True)
    single = []
    for _ in range(reps):
        a, b = ev(), ev()
        a.record()
        buf.fill_(2.0)
        b.record()
        b.synchronize()
        single.append(a.elapsed_time(b))
    a, b = ev(), ev()
    a.record()
    for _ in range(reps):
        buf.fill_(3.0)
    b.record()
    b.synchronize()
    bytes_ = mib * (1 << 20)
    med, b2b = statistics.median(single), a.elapsed_time(b) / reps
    print(f"write {mib} MiB: per launch {med * 1e3:.2f} us ({bytes_ / (med * 1e-3) / 1e12:.2f} TB/s), "
          f"back to back {b2b * 1e3:.2f} us ({bytes_ / (b2b * 1e-3) / 1e12:.2f} TB/s)", flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--mib", type=int, default=256)
    ap.add_argument("--reps", type=int, default=5)
    ap.add_argument("--write-rate", action="store_true", help="time a store-only stream of --mib MiB instead")
    a = ap.parse_args()
    if a.write_rate:
        write_rate(a.mib, max(a.reps, 20))
        return
    n = a.mib * (1 << 20) // 4
    src = torch.ones(n, device="cuda:0", dtype=torch.float32)
    dst = torch.empty_like(src)
    for _ in range(a.reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(f"copied {a.mib} MiB x {a.reps}", flush=True)


if __name__ == "__main__":
    main()
