"""The streamed (persistent) kernel: one workgroup per compute unit streams K
slabs over its output tiles and writes each finished tile's C during the next
tile's matrix work.  Its per-output arithmetic is the staged kernel's with the
same configuration, so every result must equal that kernel's bit for bit,
including the cases the stream makes special: the fewest slabs per tile (a tile
boundary comes every 4 slabs), workgroups with different tile counts, a
single tile per workgroup, 16x16 MFMA blocks, and residual adds.  One case
also meets the reference's FP64 bound against the oracle."""

import numpy as np
import pytest

from oracle import oracle as o
from tensorforge_amd import _lib
from tensorforge_amd import tforge_cpu as tc

STAGED = "block-tile={},{} thread-tile={},{} tile-k={} promote=1 vectorize=1"

CASES = [  # (workload, (m, n, k), (bm, bn, tm, tn, bk))
    ("mbr", (4096, 4096, 256), (128, 128, 8, 4, 32)),    # 1024 tiles: 4 per workgroup, 8 slabs each
    ("mbr", (4096, 4096, 256), (128, 128, 8, 4, 16)),    # 16 slabs per tile
    ("mbr", (2048, 4096, 64), (128, 128, 8, 4, 16)),     # the fewest slabs per tile (4): C drained in 4 slabs
    ("matmul", (2048, 4096, 128), (128, 128, 8, 4, 32)),
    ("mbr", (2176, 2048, 192), (128, 128, 4, 4, 32)),    # 272 tiles: 16 workgroups take two, the rest one
    ("mbr", (1024, 1024, 512), (128, 128, 8, 8, 32)),    # 64 tiles: one per workgroup
    ("mbr", (2048, 2048, 512), (64, 64, 4, 2, 64)),      # 16x16 MFMA blocks, 1024 tiles
    ("matmul", (2048, 1024, 256), (64, 64, 2, 2, 64)),
    ("mbr", (1024, 2048, 256), (64, 128, 4, 4, 32)),
    ("mbr", (2048, 1024, 128), (128, 64, 4, 4, 32)),
    ("mbr", (1024, 1024, 256), (64, 64, 4, 4, 32)),
    ("mbr", (1024, 2048, 512), (64, 128, 4, 4, 64)),
]

pytestmark = pytest.mark.gpu


def _run(workload, shape, opts, ins):
    m, n, k = shape
    kern = _lib.Kernel(tc.gen_mlir(workload, m, n, k), opts, "t.mlir")
    out = np.empty((m, n), np.float32)
    kern.run([np.ascontiguousarray(v) for v in ins.values()], out)
    return kern, out


@pytest.mark.parametrize("workload,shape,cfg", CASES, ids=[f"{c[0]}-{'x'.join(map(str, c[1]))}-"
                                                           f"b{c[2][0]}x{c[2][1]}-t{c[2][2]}x{c[2][3]}-k{c[2][4]}"
                                                           for c in CASES])
def test_streamed_equals_staged_bits(workload, shape, cfg):
    print(f"streamed {workload} {shape} {cfg}", flush=True)
    opts = STAGED.format(*cfg)
    ins = o.make_inputs(workload, *shape)
    kern, got = _run(workload, shape, opts + " persistent=1", ins)
    launch = kern.launches()[0]
    assert launch["family"] == "streamed" and launch["kernel"].startswith("tf_streamed_")
    m, n, _ = shape
    assert launch["grid"] == [min(256, (m // cfg[0]) * (n // cfg[1])), 1, 1]
    _, want = _run(workload, shape, opts, ins)
    assert not np.isnan(got).any()
    assert o.bitwise_diff(got, want) == 0


def test_streamed_meets_the_reference_bound():
    m, n, k = 2048, 4096, 128
    ins = o.make_inputs("mbr", m, n, k)
    _, out = _run("mbr", (m, n, k), STAGED.format(128, 128, 8, 4, 32) + " persistent=1", ins)
    ref, bound = o.fp64_reference("mbr", ins)
    assert o.e1_metrics(out, ref, bound)["max_err_over_bound"] <= 1.0
    assert o.mask_mismatches(out, o.preactivation64(ins), bound) == 0


def test_streamed_residual_block_equals_staged_bits():
    """Two GEMM stages (the second adds the residual x in its epilogue)."""
    m, n, k = 1024, 512, 2048
    ins = tc.make_inputs("resmlp", m, n, k)
    opts = STAGED.format(128, 128, 8, 4, 32)
    _, got = _run("resmlp", (m, n, k), opts + " persistent=1", ins)
    _, want = _run("resmlp", (m, n, k), opts, ins)
    assert o.bitwise_diff(got, want) == 0


def test_streamed_repeat_launches_are_deterministic():
    import torch
    m, n, k = 4096, 4096, 256
    dev = torch.device("cuda:0")
    ins = o.make_inputs("mbr", m, n, k)
    bufs = [torch.from_numpy(v).to(dev) for v in ins.values()]
    out = torch.empty((m, n), device=dev)
    kern = _lib.Kernel(tc.gen_mlir("mbr", m, n, k), STAGED.format(128, 128, 8, 4, 32) + " persistent=1", "t.mlir")
    ptrs = [b.data_ptr() for b in bufs] + [out.data_ptr()]
    stream = torch.cuda.current_stream().cuda_stream
    kern.launch(ptrs, stream)
    torch.cuda.synchronize()
    first = out.cpu().numpy().copy()
    for _ in range(20):
        kern.launch(ptrs, stream)
    torch.cuda.synchronize()
    assert o.bitwise_diff(out.cpu().numpy(), first) == 0
