"""Shared machinery of the MI355X measurement drivers (gpu_bench, stage9_ablation,
stage9_costmodel, e1_numerics, pad_share).

A driver describes its work as `Job`s -- a workload, a shape, a label and the
pipeline options (or the vendor-library mode) -- and hands each one to
`measure` together with the `Problem` it runs on.  `measure` compiles the
program, runs it once on the problem's seeded inputs, has the problem judge
the output (the FP64 bound with exact ReLU masks for products, bit-exactness
for element ops) and, when asked and only when the output passed, times it
with tf_bench.  The `Result` it returns knows its rate, its share of the
MI355X peak and the results-table row it becomes, so that every driver writes
the same columns in the same way and computes each FP64 reference once per
shape, however many variants it compares there.
"""

import dataclasses

import numpy as np

from tensorforge_amd import _lib
from tensorforge_amd import costmodel as cm
from tensorforge_amd import provenance
from tensorforge_amd import tforge_cpu as tc
from tensorforge_amd import tforge_gpu as tg

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, AMD's published figure
GEMM_WORKLOADS = ("matmul", "mbr")

_device = None


def device_label():
    global _device
    if _device is None:
        _device = provenance.device_label(_lib.device_info())
    return _device


def parse_shapes(text, default):
    """`MxNxK,...` (or `MxN` for element ops, stored with K = 0) -> tuples."""
    if not text:
        return list(default)
    shapes = []
    for item in text.split(","):
        dims = tuple(int(v) for v in item.lower().split("x"))
        if len(dims) not in (2, 3):
            raise ValueError(f"a shape is MxNxK or MxN, got {item!r}")
        shapes.append(dims if len(dims) == 3 else dims + (0,))
    return shapes


def parse_variants(items):
    """`NAME=OPTIONS` command-line items -> [(name, options)]."""
    out = []
    for item in items:
        name, sep, opts = item.partition("=")
        if not sep or not name:
            raise ValueError(f"a variant is NAME=OPTIONS, got {item!r}")
        out.append((name, opts))
    return out


def resolve_options(spec, workload, m, n, k):
    """Pipeline options for a variant spec: literal options, or `@tuned` (the
    autotuned configuration of this shape, else the cost model's pick) and
    `@tuned-masked` (the same, with mask-edges where the shape is not a tile
    multiple)."""
    if spec not in ("@tuned", "@tuned-masked") or workload not in GEMM_WORKLOADS:
        return spec
    opts = cm.tuned_options(workload, m, n, k)
    if spec == "@tuned-masked" and tg.padded_shape(m, n, k, opts) != (m, n, k):
        opts += " mask-edges=1"
    return opts


def without_option(options, key):
    return " ".join(t for t in options.split() if t.split("=", 1)[0] != key)


@dataclasses.dataclass(frozen=True)
class Job:
    workload: str
    m: int
    n: int
    k: int
    label: str
    options: str = ""
    mode: str = "kernel"  # "kernel" (the compiled program) or "rocblas" (sgemm + epilogue kernel)

    @property
    def shape(self):
        return f"{self.m}x{self.n}x{self.k}"

    @property
    def pipeline(self):
        if self.mode == "kernel":
            return f"tforge-gpu-pipeline{{{self.options}}}"
        return "rocblas_sgemm FP32" + ("" if self.workload == "matmul" else " + epilogue kernel")


class Problem:
    """Seeded inputs of one (workload, shape) (python/tforge_cpu.py:89-100) and,
    computed on first use and kept, the FP64 reference they imply."""

    def __init__(self, workload, m, n, k, seed=1234):
        self.workload, self.m, self.n, self.k = workload, m, n, k
        self.ins = tc.make_inputs(workload, m, n, k, seed)
        self.arrays = [np.ascontiguousarray(v) for v in self.ins.values()]
        self._ref = None

    def reference(self):
        if self._ref is None:
            self._ref = tg.reference64(self.workload, self.ins)
        return self._ref

    def judge(self, out):
        if self.workload in GEMM_WORKLOADS:
            return tg.bound_verdict(out, *self.reference())
        return tg.verdict(self.workload, self.ins, out)


@dataclasses.dataclass
class Result:
    job: Job
    verdict: dict
    output: np.ndarray
    timing: dict = None     # tg.bench's runner dict, None when untimed or failed
    compiled: dict = None   # compiler resource remarks of the selected instantiation

    @property
    def passed(self):
        return bool(self.verdict["pass"])

    def rate(self, median_ms=None):
        """(unit, GFLOP/s or GB/s) at the timed median (or a given time)."""
        unit, work = tc.flops_or_bytes(self.job.workload, self.job.m, self.job.n, self.job.k)
        ms = median_ms if median_ms is not None else self.timing["median_ms"]
        return unit, work / (ms * 1e-3) / 1e9

    def shares(self):
        """(% of the nominal peak, % of the peak at the measured clock): FP32
        matrix peak for products, 8 TB/s for element ops (compulsory bytes)."""
        unit, rate = self.rate()
        if unit == "GB/s":
            pct = 100.0 * rate / HBM_PEAK_GBS
            return pct, pct
        clk = self.timing["sm_clock_median_mhz"]
        at_clock = 100.0 * rate / tg.fp32_peak_gflops(clk) if clk > 0 else float("nan")
        return 100.0 * rate / tg.fp32_peak_gflops(tg.PEAK_CLOCK_MHZ), at_clock

    def share_text(self):
        nominal, at_clock = self.shares()
        if self.rate()[0] == "GB/s":
            return f"{nominal:.2f}% of 8 TB/s HBM (compulsory bytes)"
        return f"{at_clock:.2f}% of FP32 matrix peak at median clock; {nominal:.2f}% of 157.3 TFLOP/s"

    def describe(self):
        """Launch geometry and resources, for the params column."""
        t = self.timing
        text = (f"grid={t['grid']} block={t['block']} padded={t['padded']}; regs={t['regs']} "
                f"local={t['local_bytes']} smem={t['static_smem']} blocks/SM={t['blocks_per_sm']} "
                f"occ={t['theo_occupancy']}")
        if self.compiled:
            text += (f" spill_st={self.compiled['spill_stores']} spill_ld={self.compiled['spill_loads']} "
                     f"agprs={self.compiled['agprs']}")
        return text

    def row(self, **cols):
        """Results-table columns of this timed result; keyword arguments replace
        any default (params, correctness, notes, metric, ...)."""
        t = self.timing
        unit, rate = self.rate()
        base = {"device": device_label(), "workload": self.job.workload, "shape": self.job.shape, "dtype": "f32",
                "pipeline": self.job.pipeline, "params": f"{self.job.label}; {self.describe()}",
                "warmup": t["warmup"], "reps": t["reps"], "median_ms": t["median_ms"], "min_ms": t["min_ms"],
                "std_ms": t["std_ms"], "metric": unit, "metric_value": rate,
                "sm_clock_median_mhz": t["sm_clock_median_mhz"], "clock_adjusted_metric": self.share_text(),
                "correctness": f"err/bound={self.verdict['err_over_bound']:.3g}",
                "notes": (f"l2_flush={t['l2_flush']}; shader clock {t['sm_clock_min_mhz']:.0f}-"
                          f"{t['sm_clock_max_mhz']:.0f} MHz (device probe after each rep); power "
                          f"{t['power_median_w']} W; hip driver {t['hip_driver']}")}
        base.update(cols)
        return base


def measure(job, problem=None, warmup=10, reps=100, flush=False, timed=True, tag="bench"):
    """Compile, run once, judge and (if timed and passed) time one job."""
    problem = problem or Problem(job.workload, job.m, job.n, job.k)
    kdir = launch = compiled = None
    if job.mode == "kernel":
        kdir, launch = tg.compile_kernel(job.workload, job.m, job.n, job.k, job.options, tag=f"{tag}/{job.label}")
        compiled = tg.ptxas_resources(kdir)
    out = tg.execute(job.workload, job.m, job.n, job.k, problem.arrays, kdir, launch, job.mode)
    res = Result(job, problem.judge(out), out, compiled=compiled)
    if timed and res.passed:
        res.timing = tg.bench(job.workload, job.m, job.n, job.k, kdir, launch, job.mode, warmup, reps, flush)
    return res


def status_line(res, extra=""):
    j = res.job
    return (f"[{'PASS' if res.passed else 'FAIL'}] {j.label:>22} {j.workload:>8} {j.shape:>16} "
            f"err/bound={res.verdict['err_over_bound']:.3g} {extra}").rstrip()


def timing_line(res):
    unit, rate = res.rate()
    nominal, at_clock = res.shares()
    return (f"        median {res.timing['median_ms']:.4f} ms  {rate:.1f} {unit}  {nominal:.1f}% of peak "
            f"({at_clock:.1f}% at {res.timing['sm_clock_median_mhz']:.0f} MHz)")
