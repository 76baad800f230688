"""The vendor comparison's output check (tensorforge_amd/bench/vendor_compare.py)
is the reference's bound (python/tforge_gpu.py:134-145): it passes a
correctly rounded float32 result and fails a planted error or a flipped
ReLU mask.  Runs on the CPU (torch CPU tensors)."""

import numpy as np
import torch

from oracle import oracle as o
from tensorforge_amd.bench import vendor_compare as vc


def _inputs(m=48, n=40, k=96):
    ins = o.make_inputs("mbr", m, n, k, seed=1234)
    return ins, [torch.from_numpy(ins[s]) for s in ("a", "b", "bias")]


def test_correct_results_pass():
    ins, (a, b, bias) = _inputs()
    mbr = torch.from_numpy(o.mbr_fma(ins["a"], ins["b"], ins["bias"]))
    ok, verdict = vc.bound_check(torch, a, b, bias, mbr, relu=True)
    assert ok and "mask_mismatches=0" in verdict
    mm = torch.from_numpy(o.matmul_fma(ins["a"], ins["b"]))
    assert vc.bound_check(torch, a, b, bias, mm, relu=False)[0]


def test_planted_errors_fail():
    ins, (a, b, bias) = _inputs()
    good = o.mbr_fma(ins["a"], ins["b"], ins["bias"])
    bad = good.copy()
    r, c = np.argwhere(good > 0.5)[0]
    bad[r, c] *= 1.001  # far beyond the bound of a K = 96 sum
    assert not vc.bound_check(torch, a, b, bias, torch.from_numpy(bad), relu=True)[0]
    z = o.preactivation64(ins)
    _, bound = o.fp64_reference("mbr", ins)
    neg = np.argwhere((z < 0) & (np.abs(z) > bound))[0]
    flipped = good.copy()
    flipped[tuple(neg)] = 1e-30  # a zero the ReLU decides turned positive (tiny: within the error bound)
    ok, verdict = vc.bound_check(torch, a, b, bias, torch.from_numpy(flipped), relu=True)
    assert not ok and "mask_mismatches=1" in verdict
    nan = good.copy()
    nan[0, 0] = np.nan
    assert not vc.bound_check(torch, a, b, bias, torch.from_numpy(nan), relu=True)[0]
