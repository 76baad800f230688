"""Workload programs, seeded inputs and shared constants of the TensorForge
drivers (the parts of the reference's python/tforge_cpu.py that the GPU path
uses: python/tforge_cpu.py:26, 29-53, 89-100, 154-159).

Workloads and their entry signatures (tensors, row-major f32):
  add      entry(a: MxN, b: MxN) -> MxN
  relu     entry(a: MxN) -> MxN
  matmul   entry(a: MxK, b: KxN) -> MxN
  mbr      entry(a: MxK, b: KxN, bias: N) -> MxN      relu(a @ b + bias)
  bias_add entry(a: MxN, bias: N) -> MxN
  resmlp   entry(x: MxN, w1: NxK, b1: K, w2: KxN, b2: N) -> MxN
           relu(relu(x @ w1 + b1) @ w2 + b2) + x   (two-layer residual block;
           an extension: the reference has no such workload)

The reference's CPU pipeline itself (tensorforge-opt --tforge-cpu-pipeline)
needs MLIR and is not part of this package; the CPU baselines live with the
test oracle.
"""

import pathlib

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parent.parent
BUILD = ROOT / "build"
ART = BUILD / "artifacts"

F32_EPS = 2.0 ** -24  # unit roundoff for f32, round to nearest

WORKLOADS = ("add", "relu", "matmul", "mbr", "bias_add", "resmlp")


def _t(*d):
    return "tensor<" + "x".join(str(x) for x in d) + "xf32>"


def gen_mlir(workload, m, n, k=None):
    t = _t
    if workload == "add":
        return (f"func.func @entry(%a: {t(m, n)}, %b: {t(m, n)}) -> {t(m, n)} {{\n"
                f"  %0 = tforge.add %a, %b : {t(m, n)}, {t(m, n)} -> {t(m, n)}\n"
                f"  return %0 : {t(m, n)}\n}}\n")
    if workload == "bias_add":
        return (f"func.func @entry(%a: {t(m, n)}, %bias: {t(n)}) -> {t(m, n)} {{\n"
                f"  %0 = tforge.bias_add %a, %bias : {t(m, n)}, {t(n)} -> {t(m, n)}\n"
                f"  return %0 : {t(m, n)}\n}}\n")
    if workload == "relu":
        return (f"func.func @entry(%a: {t(m, n)}) -> {t(m, n)} {{\n"
                f"  %0 = tforge.relu %a : {t(m, n)} -> {t(m, n)}\n"
                f"  return %0 : {t(m, n)}\n}}\n")
    if workload == "matmul":
        return (f"func.func @entry(%a: {t(m, k)}, %b: {t(k, n)}) -> {t(m, n)} {{\n"
                f"  %0 = tforge.matmul %a, %b : {t(m, k)}, {t(k, n)} -> {t(m, n)}\n"
                f"  return %0 : {t(m, n)}\n}}\n")
    if workload == "mbr":
        return (f"func.func @entry(%a: {t(m, k)}, %b: {t(k, n)}, %bias: {t(n)}) -> {t(m, n)} {{\n"
                f"  %0 = tforge.matmul %a, %b : {t(m, k)}, {t(k, n)} -> {t(m, n)}\n"
                f"  %1 = tforge.bias_add %0, %bias : {t(m, n)}, {t(n)} -> {t(m, n)}\n"
                f"  %2 = tforge.relu %1 : {t(m, n)} -> {t(m, n)}\n"
                f"  return %2 : {t(m, n)}\n}}\n")
    if workload == "resmlp":
        return (f"func.func @entry(%x: {t(m, n)}, %w1: {t(n, k)}, %b1: {t(k)}, %w2: {t(k, n)}, "
                f"%b2: {t(n)}) -> {t(m, n)} {{\n"
                f"  %0 = tforge.matmul %x, %w1 : {t(m, n)}, {t(n, k)} -> {t(m, k)}\n"
                f"  %1 = tforge.bias_add %0, %b1 : {t(m, k)}, {t(k)} -> {t(m, k)}\n"
                f"  %2 = tforge.relu %1 : {t(m, k)} -> {t(m, k)}\n"
                f"  %3 = tforge.matmul %2, %w2 : {t(m, k)}, {t(k, n)} -> {t(m, n)}\n"
                f"  %4 = tforge.bias_add %3, %b2 : {t(m, n)}, {t(n)} -> {t(m, n)}\n"
                f"  %5 = tforge.relu %4 : {t(m, n)} -> {t(m, n)}\n"
                f"  %6 = tforge.add %5, %x : {t(m, n)}, {t(m, n)} -> {t(m, n)}\n"
                f"  return %6 : {t(m, n)}\n}}\n")
    raise ValueError(workload)


def make_inputs(workload, m, n, k, seed=1234):
    """Seeded inputs in entry-argument order (python/tforge_cpu.py:89-100).

    resmlp: x ~ N(0, 1); w1, w2 ~ N(0, sigma = 1/sqrt(fan_in)); b1, b2 ~
    N(0, sigma = 0.02); drawn in the order x, w1, b1, w2, b2.
    """
    rng = np.random.default_rng(seed)
    u = lambda *s: rng.uniform(-1.0, 1.0, size=s).astype(np.float32)
    if workload == "add":
        return {"a": u(m, n), "b": u(m, n)}
    if workload == "relu":
        return {"a": u(m, n)}
    if workload == "bias_add":
        return {"a": u(m, n), "bias": u(n)}
    if workload == "matmul":
        return {"a": u(m, k), "b": u(k, n)}
    if workload == "mbr":
        return {"a": u(m, k), "b": u(k, n), "bias": u(n)}
    if workload == "resmlp":
        g = lambda sigma, *s: (rng.standard_normal(size=s) * sigma).astype(np.float32)
        x = g(1.0, m, n)
        w1 = g(1.0 / np.sqrt(n), n, k)
        b1 = g(0.02, k)
        w2 = g(1.0 / np.sqrt(k), k, n)
        b2 = g(0.02, n)
        return {"x": x, "w1": w1, "b1": b1, "w2": w2, "b2": b2}
    raise ValueError(workload)


# Work per call that the rate metrics divide by: FP32 FLOPs of the matrix
# products (2 per multiply-add; the epilogue's adds and maxima are not counted,
# as in the reference's tables), or the compulsory bytes an element op moves
# (every input read once, the output written once).
_WORK = {
    "matmul": ("GFLOP/s", lambda m, n, k: 2.0 * m * n * k),
    "mbr": ("GFLOP/s", lambda m, n, k: 2.0 * m * n * k),
    "resmlp": ("GFLOP/s", lambda m, n, k: 2 * (2.0 * m * n * k)),  # two products of m*n*k each
    "add": ("GB/s", lambda m, n, k: 4.0 * 3 * m * n),
    "relu": ("GB/s", lambda m, n, k: 4.0 * 2 * m * n),
    "bias_add": ("GB/s", lambda m, n, k: 4.0 * 2 * m * n),
}


def flops_or_bytes(workload, m, n, k):
    """(rate unit, work per call) of a workload (python/tforge_cpu.py:154-159
    defines the same pair for the reference's four workloads)."""
    unit, work = _WORK[workload]
    return unit, work(m, n, k or 0)
