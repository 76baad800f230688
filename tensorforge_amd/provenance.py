"""Provenance of every results row: which code, tool chain, device and time
produced it.  The column set is the reference's results schema
(python/provenance.py:11-16) so that MI355X tables line up with its tables; on
this backend "mlir_llvm_version" holds ROCm's LLVM version (there is no MLIR in
the tool chain) and "cuda_version" holds the HIP version.

The commit comes from BUILD_INFO.json, which `tensorforge_amd.build` writes
next to the library it links (HEAD and whether the tree differed from it), so
rows written on a machine that received the built tree without its .git still
name the code; a tree without that file falls back to reading .git.  Nothing
here runs a tool in a child process except save_lscpu: rows are written from
processes that hold the GPU, sometimes under a profiler, where replacing a
process image is not allowed.
"""

import csv
import datetime
import json
import os
import pathlib
import re
import socket
import subprocess

PKG = pathlib.Path(__file__).resolve().parent
ROOT = PKG.parent
ROCM = pathlib.Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
BUILD_INFO = PKG / "BUILD_INFO.json"

FIELDS = [
    "commit", "mlir_llvm_version", "cuda_version", "device", "job_id", "date",
    "workload", "shape", "dtype", "pipeline", "params", "threads", "warmup", "reps",
    "median_ms", "min_ms", "std_ms", "metric", "metric_value", "sm_clock_median_mhz",
    "clock_adjusted_metric", "alloc_bytes_per_call", "correctness", "notes",
]


def _text(path):
    try:
        return pathlib.Path(path).read_text()
    except OSError:
        return ""


def git_head(root=ROOT):
    """Full hash of HEAD read from the .git files ("" without a .git)."""
    git = pathlib.Path(root) / ".git"
    head = _text(git / "HEAD").strip()
    if not head.startswith("ref: "):
        return head
    ref = head[5:]
    sha = _text(git / ref).strip()
    if not sha:
        packed = dict(reversed(line.split(" ", 1)) for line in _text(git / "packed-refs").splitlines()
                      if line and not line.startswith(("#", "^")))
        sha = packed.get(ref, "")
    return sha


def commit_label():
    """`<short hash>[-dirty]` of the code that was built, as the build recorded it."""
    try:
        info = json.loads(BUILD_INFO.read_text())
        return info["commit"][:12] + ("-dirty" if info.get("dirty") else "")
    except (OSError, ValueError, KeyError):
        return git_head()[:12]


def write_build_info(path=BUILD_INFO):
    """Called by the build (on the machine that has the .git): record HEAD and
    whether tracked or untracked files differed from it."""
    sha = git_head()
    try:
        status = subprocess.run(["git", "-C", str(ROOT), "status", "--porcelain", "--untracked-files=no"],
                                capture_output=True, text=True, timeout=60).stdout
        dirty = bool(status.strip())
    except (OSError, subprocess.SubprocessError):
        dirty = None
    info = {"commit": sha, "dirty": dirty, "built": datetime.datetime.now().astimezone().isoformat(timespec="seconds")}
    pathlib.Path(path).write_text(json.dumps(info, indent=1) + "\n")
    return info


def _hip_version():
    text = _text(ROCM / "include/hip/hip_version.h")
    parts = [re.search(rf"#define\s+HIP_VERSION_{p}\s+(\d+)", text) for p in ("MAJOR", "MINOR", "PATCH")]
    return ".".join(m.group(1) for m in parts if m)


def _llvm_version():
    m = re.search(r'#define\s+FLANG_VERSION_STRING\s+"([^"]+)"', _text(ROCM / "lib/llvm/include/flang/Version.inc"))
    return m.group(1) if m else ""


def common():
    """The columns every row shares within one run."""
    return {"commit": commit_label(), "mlir_llvm_version": _llvm_version(), "cuda_version": _hip_version(),
            "job_id": os.environ.get("SLURM_JOB_ID", os.environ.get("GRAFT_JOB_ID", "none")),
            "date": datetime.datetime.now().astimezone().isoformat(timespec="seconds")}


def device_label(dev):
    """GPU description for the `device` column, from _lib.device_info(): the
    marketing name where the driver knows it, always the ISA and CU count."""
    name = dev.get("name") or "AMD GPU"
    return f"{name} [{dev.get('arch', '')}, {dev.get('compute_units', 0)} CUs]"


def cpu_model():
    for line in _text("/proc/cpuinfo").splitlines():
        if line.startswith("model name"):
            return line.split(":", 1)[1].strip()
    return ""


def save_lscpu(outdir):
    """hostname and lscpu's report (lscpu run directly as a child process)."""
    outdir = pathlib.Path(outdir)
    outdir.mkdir(parents=True, exist_ok=True)
    p = outdir / f"lscpu_{os.environ.get('SLURM_JOB_ID', 'none')}.txt"
    try:
        report = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=60).stdout
    except (OSError, subprocess.SubprocessError):
        report = ""
    p.write_text(socket.gethostname() + "\n" + report + "\n")
    return p


class ResultsTable:
    """A results CSV in the schema above, opened for appending.  Each row
    starts from the run's shared provenance (`common()`, taken once when the
    table is opened) and `defaults`; `add` overrides them per row and refuses
    a column the schema does not have.  Rows are flushed as they are added, so
    a run that dies keeps what it measured."""

    def __init__(self, path, **defaults):
        unknown = set(defaults) - set(FIELDS)
        if unknown:
            raise KeyError(f"not a results column: {sorted(unknown)}")
        self.path = pathlib.Path(path)
        self.path.parent.mkdir(parents=True, exist_ok=True)
        self.base = {**common(), **defaults}
        fresh = not self.path.exists() or self.path.stat().st_size == 0
        self._file = open(self.path, "a", newline="")
        self._csv = csv.DictWriter(self._file, fieldnames=FIELDS, restval="")
        if fresh:
            self._csv.writeheader()
        self.count = 0

    def add(self, **cols):
        unknown = set(cols) - set(FIELDS)
        if unknown:
            raise KeyError(f"not a results column: {sorted(unknown)}")
        self._csv.writerow({**self.base, **cols})
        self._file.flush()
        self.count += 1

    def close(self):
        self._file.close()
