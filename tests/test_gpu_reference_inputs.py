"""Every benchmark configuration on the reference's own seeded inputs, with
both configurations the benchmarks run: the autotuned one
(costmodel.tuned_options) and the cost model's pick (costmodel.default_config).

Inputs are numpy default_rng(1234) uniform[-1, 1] draws in the order a, b,
bias (python/tforge_cpu.py:89-100), made on the host and uploaded.  Bars
(python/tforge_gpu.py:112-145, plus the north star's ReLU-mask rule):

  * up to 2048^3 the whole output against the FP64 reference: err/bound <= 1
    with the reference's gamma_{K(+1)} bound, no NaN (the output is
    NaN-prefilled), and exact ReLU masks wherever |z| exceeds the bound;
  * above 2048^3, 64 sampled rows against the same reference, exact masks
    included, and the whole output free of NaN.

The 2048^3 headline's err/bound is printed beside the reference's own figure
on its FMA kernels, 0.00232 (results/gpu/stage8.csv:86).  The residual block
runs on its own seeded draws in test_gpu_fullsize.py.
"""

import re

import numpy as np
import pytest

from oracle import oracle as o
from tensorforge_amd import _lib
from tensorforge_amd import costmodel as cm
from tensorforge_amd import tforge_cpu as tc

pytestmark = pytest.mark.gpu

# BASELINE configurations: examples/mbr.mlir, the headline, plain matmul
# 512..8192^3, the four rectangular MLP layers.
CASES = [("mbr", 256, 256, 128), ("mbr", 2048, 2048, 2048),
         ("matmul", 512, 512, 512), ("matmul", 1024, 1024, 1024), ("matmul", 2048, 2048, 2048),
         ("matmul", 4096, 4096, 4096), ("matmul", 8192, 8192, 8192),
         ("mbr", 8192, 1024, 4096), ("mbr", 1024, 8192, 4096), ("mbr", 64, 4096, 4096), ("mbr", 4096, 4096, 256)]
FULL_LIMIT = 2048 ** 3
REFERENCE_EOB_2048 = 0.00232  # results/gpu/stage8.csv:86 (mbr 2048^3, the reference's FMA kernels)


def _torch():
    import torch
    return torch, torch.device("cuda:0")


def _compiled_shape(options, m, n, k):
    """The shape to compile at: the true one, or the padded one when the
    options' tiles do not divide it and mask-edges is off (the reference pads:
    python/tforge_gpu.py:54-63)."""
    if "mask-edges" in options or "tile-k" not in options:
        return m, n, k
    bm, bn = (int(x) for x in re.search(r"block-tile=(\d+),(\d+)", options).groups())
    bk = int(re.search(r"tile-k=(\d+)", options).group(1))
    up = lambda x, t: -(-x // t) * t
    return up(m, bm), up(n, bn), up(k, bk)


def _run_on_reference_inputs(workload, m, n, k, options, ins):
    """Upload the host draws, run the program once through tf_launch on a
    NaN-prefilled output (zero-padded copies when the tiles need padding),
    return the m x n output on the host."""
    torch, dev = _torch()
    pm, pn, pk = _compiled_shape(options, m, n, k)
    kern = _lib.Kernel(tc.gen_mlir(workload, pm, pn, pk), options, "t.mlir")
    a = torch.zeros((pm, pk), device=dev)
    a[:m, :k] = torch.from_numpy(ins["a"]).to(dev)
    b = torch.zeros((pk, pn), device=dev)
    b[:k, :n] = torch.from_numpy(ins["b"]).to(dev)
    args = [a, b]
    if workload == "mbr":
        bias = torch.zeros(pn, device=dev)
        bias[:n] = torch.from_numpy(ins["bias"]).to(dev)
        args.append(bias)
    out = torch.full((pm, pn), float("nan"), device=dev)
    stream = torch.cuda.current_stream().cuda_stream
    kern.launch([t.data_ptr() for t in args] + [out.data_ptr()], stream)
    torch.cuda.synchronize()
    got = out[:m, :n]
    assert not torch.isnan(got).any(), "unwritten (NaN-prefilled) outputs"
    return kern.launches()[0]["kernel"], got.cpu().numpy()


def _configurations(workload, m, n, k):
    tuned = cm.tuned_options(workload, m, n, k)
    default = cm.options(cm.default_config(m, n, k))
    return [("tuned", tuned)] + ([("default", default)] if default != tuned else [])


@pytest.mark.parametrize("workload,m,n,k", CASES)
def test_reference_inputs_tuned_and_default(workload, m, n, k):
    ins = o.make_inputs(workload, m, n, k, seed=1234)
    full = m * n * k <= FULL_LIMIT
    if full:
        sub = ins
        rows = slice(None)
    else:
        rows = np.sort(np.random.default_rng(7).choice(m, size=min(64, m), replace=False))
        sub = dict(ins, a=ins["a"][rows])
    ref, bound = o.fp64_reference(workload, sub)
    z = o.preactivation64(sub) if workload == "mbr" else None
    for which, options in _configurations(workload, m, n, k):
        print(f"{workload} {m}x{n}x{k} {which}: {options}", flush=True)
        kernel, out = _run_on_reference_inputs(workload, m, n, k, options, ins)
        got = out[rows]
        eob = o.e1_metrics(got, ref, bound)["max_err_over_bound"]
        masks = o.mask_mismatches(got, z, bound) if z is not None else 0
        scope = "full output" if full else f"{len(rows)} sampled rows"
        note = f" (reference FMA kernels: {REFERENCE_EOB_2048})" if (workload, m, n, k) == ("mbr", 2048, 2048, 2048) else ""
        print(f"  {kernel}: err/bound {eob:.5f} over the {scope}{note}, ReLU mask mismatches {masks}", flush=True)
        assert eob <= 1.0, (which, options, eob)
        assert masks == 0, (which, options, masks)

