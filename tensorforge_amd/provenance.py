"""Provenance fields shared by every results CSV row (python/provenance.py:1-70).

The column set is unchanged so CSVs stay comparable with the reference's.  On
this backend "mlir_llvm_version" holds the version of ROCm's LLVM (there is no
MLIR in the tool chain) and "cuda_version" holds the HIP version.

Everything is read from files (the git refs, the ROCm headers, /proc/cpuinfo)
rather than from tools run in a shell: these rows are written from processes
that hold the GPU, sometimes under a profiler whose preloaded library sets up
the GPU in every child, and a tool that replaces itself with another program
(exec) from such a process is not allowed.  The commit therefore carries no
"-dirty" mark.
"""

import csv
import datetime
import os
import pathlib
import re
import socket
import subprocess

ROOT = pathlib.Path(__file__).resolve().parent.parent
ROCM = pathlib.Path(os.environ.get("ROCM_PATH", "/opt/rocm"))

FIELDS = [
    "commit", "mlir_llvm_version", "cuda_version", "device", "job_id", "date",
    "workload", "shape", "dtype", "pipeline", "params", "threads", "warmup", "reps",
    "median_ms", "min_ms", "std_ms", "metric", "metric_value", "sm_clock_median_mhz",
    "clock_adjusted_metric", "alloc_bytes_per_call", "correctness", "notes",
]


def _read(path):
    try:
        return pathlib.Path(path).read_text()
    except OSError:
        return ""


def _commit():
    """Short hash of HEAD from .git (empty where the tree has no .git)."""
    git = ROOT / ".git"
    head = _read(git / "HEAD").strip()
    if not head.startswith("ref: "):
        return head[:7]
    name = head[5:]
    sha = _read(git / name).strip()
    if not sha:
        for line in _read(git / "packed-refs").splitlines():
            if line.endswith(" " + name):
                sha = line.split()[0]
    return sha[:7]


def _define(text, name):
    m = re.search(rf"#define\s+{name}\s+\"?([^\s\"]+)", text)
    return m.group(1) if m else ""


def common():
    hipv = _read(ROCM / "include/hip/hip_version.h")
    hip = ".".join(_define(hipv, f"HIP_VERSION_{p}") for p in ("MAJOR", "MINOR", "PATCH")).strip(".")
    llvm = _define(_read(ROCM / "lib/llvm/include/flang/Version.inc"), "FLANG_VERSION_STRING")
    return {
        "commit": _commit(),
        "mlir_llvm_version": llvm,
        "cuda_version": hip,
        "job_id": os.environ.get("SLURM_JOB_ID", os.environ.get("GRAFT_JOB_ID", "none")),
        "date": datetime.datetime.now().astimezone().isoformat(timespec="seconds"),
    }


def cpu_model():
    for line in _read("/proc/cpuinfo").splitlines():
        if line.startswith("model name"):
            return line.split(":", 1)[1].strip()
    return ""


def save_lscpu(outdir):
    """hostname and lscpu's report (lscpu run directly as a child process)."""
    outdir = pathlib.Path(outdir)
    outdir.mkdir(parents=True, exist_ok=True)
    job = os.environ.get("SLURM_JOB_ID", "none")
    p = outdir / f"lscpu_{job}.txt"
    try:
        report = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=60).stdout
    except (OSError, subprocess.SubprocessError):
        report = ""
    p.write_text(socket.gethostname() + "\n" + report + "\n")
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
