"""Provenance fields shared by every results CSV row (python/provenance.py:1-70).

The column set is unchanged so CSVs stay comparable with the reference's.  On
this backend "mlir_llvm_version" holds the LLVM version of hipcc (there is no
MLIR in the tool chain) and "cuda_version" holds the HIP version.
"""

import csv
import datetime
import os
import pathlib
import subprocess

ROOT = pathlib.Path(__file__).resolve().parent.parent

FIELDS = [
    "commit", "mlir_llvm_version", "cuda_version", "device", "job_id", "date",
    "workload", "shape", "dtype", "pipeline", "params", "threads", "warmup", "reps",
    "median_ms", "min_ms", "std_ms", "metric", "metric_value", "sm_clock_median_mhz",
    "clock_adjusted_metric", "alloc_bytes_per_call", "correctness", "notes",
]


def _sh(cmd):
    try:
        return subprocess.run(cmd, shell=True, capture_output=True, text=True, timeout=60).stdout.strip()
    except (OSError, subprocess.SubprocessError):
        return ""


def common():
    dirty = _sh(f"git -C {ROOT} status --porcelain --untracked-files=no")
    commit = _sh(f"git -C {ROOT} rev-parse --short HEAD") + ("-dirty" if dirty else "")
    llvm = _sh("/opt/rocm/bin/hipcc --version 2>/dev/null | grep -o 'clang version [0-9.a-z]*'").replace(
        "clang version ", "")
    hip = _sh("/opt/rocm/bin/hipcc --version 2>/dev/null | grep -o 'HIP version: [0-9.]*'").replace(
        "HIP version: ", "")
    return {
        "commit": commit,
        "mlir_llvm_version": llvm,
        "cuda_version": hip,
        "job_id": os.environ.get("SLURM_JOB_ID", os.environ.get("GRAFT_JOB_ID", "none")),
        "date": datetime.datetime.now().astimezone().isoformat(timespec="seconds"),
    }


def cpu_model():
    return _sh("lscpu | grep -m1 'Model name' | sed 's/Model name:[ ]*//'")


def save_lscpu(outdir):
    outdir = pathlib.Path(outdir)
    outdir.mkdir(parents=True, exist_ok=True)
    job = os.environ.get("SLURM_JOB_ID", "none")
    p = outdir / f"lscpu_{job}.txt"
    p.write_text(_sh("hostname") + "\n" + _sh("lscpu") + "\n")
    return p


class CsvWriter:
    """Appends rows to a CSV, writing the header only for a new file."""

    def __init__(self, path):
        self.path = pathlib.Path(path)
        self.path.parent.mkdir(parents=True, exist_ok=True)
        new = not self.path.exists()
        self.f = open(self.path, "a", newline="")
        self.w = csv.DictWriter(self.f, fieldnames=FIELDS)
        if new:
            self.w.writeheader()

    def row(self, **kw):
        missing = set(kw) - set(FIELDS)
        if missing:
            raise KeyError(missing)
        self.w.writerow(kw)
        self.f.flush()
