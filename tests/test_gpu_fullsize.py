"""Every benchmark configuration at its full size, through tf_launch, with the
options the benchmarks use (autotuned, else the cost model's pick).

A full FP64 reference of the largest problems costs minutes on the host, so
these tests check properties that hold for any summation order and are
therefore exact at any size, plus the reference's bound on sampled rows:

  * scaling: doubling A and the bias (and x, b1, b2 of the residual block)
    doubles every output bit for bit -- products and sums scale exactly by a
    power of two, relu(2z) = 2 relu(z);
  * row permutation: permuting the rows of A (of x) permutes the output rows
    bit for bit -- each output row's arithmetic does not depend on its tile;
  * column permutation: permuting the columns of B together with the bias
    permutes the output columns bit for bit;
  * 32 sampled rows against the FP64 reference with the reference's bound
    (python/tforge_gpu.py:134-145) and exact ReLU masks, or the composed
    bound of the residual block.

Inputs are the reference's seeded draws (numpy default_rng(1234) uniform[-1, 1]
in the order a, b, bias: python/tforge_cpu.py:89-100; the residual block's
standard-normal draws from tforge_cpu.make_inputs), made on the host and
uploaded.
"""

import numpy as np
import pytest

from oracle import oracle as o
from tensorforge_amd import _lib
from tensorforge_amd import costmodel as cm
from tensorforge_amd import tforge_cpu as tc
from tensorforge_amd import tforge_gpu as tg

pytestmark = pytest.mark.gpu

# The benchmark configurations: examples/mbr.mlir, the 2048^3 headline, plain matmul
# 512..8192^3, the rectangular MLP layers (skinny and short-K included).
CASES = [("mbr", 256, 256, 128), ("mbr", 2048, 2048, 2048),
         ("matmul", 512, 512, 512), ("matmul", 1024, 1024, 1024), ("matmul", 2048, 2048, 2048),
         ("matmul", 4096, 4096, 4096), ("matmul", 8192, 8192, 8192),
         ("mbr", 8192, 1024, 4096), ("mbr", 1024, 8192, 4096), ("mbr", 64, 4096, 4096), ("mbr", 4096, 4096, 256)]


def _torch():
    import torch
    return torch, torch.device("cuda:0")


def _bits(t):
    torch, _ = _torch()
    return t.contiguous().view(torch.int32)


@pytest.mark.parametrize("workload,m,n,k", CASES)
def test_full_size_properties(workload, m, n, k):
    torch, dev = _torch()
    opts = cm.tuned_options(workload, m, n, k)
    kern = _lib.Kernel(tc.gen_mlir(workload, m, n, k), opts, "t.mlir")
    stream = torch.cuda.current_stream().cuda_stream
    # The reference's seeded draws (numpy default_rng(1234), python/tforge_cpu.py:89-100).
    host = o.make_inputs("mbr", m, n, k, seed=1234)
    a, b, bias = (torch.from_numpy(host[s]).to(dev) for s in ("a", "b", "bias"))
    g = torch.Generator(device=dev).manual_seed(1234)
    mbr = workload == "mbr"

    def run(a_, b_, bias_):
        out = torch.full((m, n), float("nan"), device=dev)
        ins = [a_.contiguous(), b_.contiguous()] + ([bias_.contiguous()] if mbr else [])
        kern.launch([t.data_ptr() for t in ins] + [out.data_ptr()], stream)
        torch.cuda.synchronize()
        return out

    out = run(a, b, bias)
    assert not torch.isnan(out).any()
    assert torch.equal(_bits(run(2 * a, b, 2 * bias)), _bits(2 * out))
    rp = torch.randperm(m, device=dev, generator=g)
    assert torch.equal(_bits(run(a[rp], b, bias)), _bits(out[rp]))
    cp = torch.randperm(n, device=dev, generator=g)
    assert torch.equal(_bits(run(a, b[:, cp], bias[cp])), _bits(out[:, cp]))

    rows = np.sort(np.random.default_rng(7).choice(m, size=min(32, m), replace=False))
    ins = {"a": host["a"][rows], "b": host["b"]}
    if mbr:
        ins["bias"] = host["bias"]
    got = out[rows].cpu().numpy()
    ref, bound = o.fp64_reference(workload, ins)
    assert o.e1_metrics(got, ref, bound)["max_err_over_bound"] <= 1.0
    if mbr:
        assert o.mask_mismatches(got, o.preactivation64(ins), bound) == 0


# The residual block's measured best tiles (results/gpu/resmlp.csv) and the earlier pick.
RESMLP_OPTS = ["block-tile=128,128 thread-tile=8,8 tile-k=16 promote=1 vectorize=1",
               "block-tile=128,256 thread-tile=8,4 tile-k=32 promote=1 vectorize=1"]


@pytest.mark.parametrize("opts", RESMLP_OPTS)
def test_full_size_residual_block(opts):
    """The residual block at its benchmark size (x 4096x2048, W1 2048x8192,
    W2 8192x2048)."""
    torch, dev = _torch()
    m, n, k = 4096, 2048, 8192
    kern = _lib.Kernel(tc.gen_mlir("resmlp", m, n, k), opts, "t.mlir")
    stream = torch.cuda.current_stream().cuda_stream
    host = tc.make_inputs("resmlp", m, n, k)
    x, w1, b1, w2, b2 = (torch.from_numpy(np.ascontiguousarray(host[s])).to(dev) for s in ("x", "w1", "b1", "w2", "b2"))

    def run(x_, b1_, b2_):
        y = torch.full((m, n), float("nan"), device=dev)
        kern.launch([t.contiguous().data_ptr() for t in (x_, w1, b1_, w2, b2_)] + [y.data_ptr()], stream)
        torch.cuda.synchronize()
        return y

    y = run(x, b1, b2)
    assert not torch.isnan(y).any()
    assert torch.equal(_bits(run(2 * x, 2 * b1, 2 * b2)), _bits(2 * y))
    g = torch.Generator(device=dev).manual_seed(5)
    rp = torch.randperm(m, device=dev, generator=g)
    xp = x[rp].contiguous()
    assert torch.equal(_bits(run(xp, b1, b2)), _bits(y[rp]))

    rows = np.sort(np.random.default_rng(7).choice(m, size=32, replace=False))
    sub = dict(host)
    sub["x"] = host["x"][rows]
    assert tg._resmlp_check(sub, y[rows].cpu().numpy())["pass"]


# Layer 2 of the residual block as a program of its own: relu(h @ w2 + b2) + x.
LAYER2 = """func.func @entry(%h: {h}, %w2: {w2}, %b2: {b2}, %x: {y}) -> {y} {{
  %0 = tforge.matmul %h, %w2 : {h}, {w2} -> {y}
  %1 = tforge.bias_add %0, %b2 : {y}, {b2} -> {y}
  %2 = tforge.relu %1 : {y} -> {y}
  %3 = tforge.add %2, %x : {y}, {y} -> {y}
  return %3 : {y}
}}
"""


def test_full_size_residual_layers_against_the_oracle():
    """The residual block at its benchmark size, one layer at a time against
    the oracle.  Layer 1, relu(x @ w1 + b1), runs as its own program with the
    block's configuration and meets the reference bound with exact ReLU masks
    on sampled rows.  Layer 2 on the kernel's own float32 h meets the reference
    bound widened by the final add's one rounding, u (|relu(z) + x| + bound),
    and where the ReLU decides zero the output is x itself, bit for bit.  The
    block equals the two programs run one after the other, bit for bit, so
    the two checks cover it."""
    torch, dev = _torch()
    m, n, k = 4096, 2048, 8192
    opts = RESMLP_OPTS[0]
    stream = torch.cuda.current_stream().cuda_stream
    host = tc.make_inputs("resmlp", m, n, k)
    x, w1, b1, w2, b2 = (torch.from_numpy(np.ascontiguousarray(host[s])).to(dev) for s in ("x", "w1", "b1", "w2", "b2"))

    def run(program, args, shape):
        out = torch.full(shape, float("nan"), device=dev)
        _lib.Kernel(program, opts, "t.mlir").launch([a.data_ptr() for a in args] + [out.data_ptr()], stream)
        torch.cuda.synchronize()
        return out

    t = lambda *s: "tensor<" + "x".join(map(str, s)) + "xf32>"
    h = run(tc.gen_mlir("mbr", m, k, n), [x, w1, b1], (m, k))
    y2 = run(LAYER2.format(h=t(m, k), w2=t(k, n), b2=t(n), y=t(m, n)), [h, w2, b2, x], (m, n))
    y = run(tc.gen_mlir("resmlp", m, n, k), [x, w1, b1, w2, b2], (m, n))
    assert torch.equal(_bits(y), _bits(y2))

    rows = np.sort(np.random.default_rng(11).choice(m, size=32, replace=False))
    layer1 = {"a": host["x"][rows], "b": host["w1"], "bias": host["b1"]}
    ref1, bound1 = o.fp64_reference("mbr", layer1)
    h_rows = h[rows].cpu().numpy()
    assert o.e1_metrics(h_rows, ref1, bound1)["max_err_over_bound"] <= 1.0
    assert o.mask_mismatches(h_rows, o.preactivation64(layer1), bound1) == 0

    layer2 = {"a": h_rows, "b": host["w2"], "bias": host["b2"]}
    ref2, bound2 = o.fp64_reference("mbr", layer2)
    x_rows = host["x"][rows]
    y_ref = ref2 + x_rows.astype(np.float64)
    y_rows = y[rows].cpu().numpy()
    assert o.e1_metrics(y_rows, y_ref, bound2 + o.F32_EPS * (np.abs(y_ref) + bound2))["max_err_over_bound"] <= 1.0
    z2 = o.preactivation64(layer2)
    zero = (z2 <= 0) & (np.abs(z2) > bound2)
    assert zero.sum() > 1000
    assert o.bitwise_diff(y_rows[zero], x_rows[zero]) == 0
