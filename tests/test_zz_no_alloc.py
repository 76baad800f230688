"""tf_launch_noalloc -- the allocation-free variant of tf_launch (no
counterpart in the reference; for callers that cannot allocate device memory).
It must give tf_launch's bits on the same inputs, including on a second call
with a smaller program after a larger one left the shared scratch array full
of its data, and refuse programs whose scratch exceeds the array."""

import ctypes

import numpy as np
import pytest

from oracle import oracle as o
from tensorforge_amd import _lib
from tensorforge_amd import tforge_cpu as tc

STAGED = "block-tile=64,64 thread-tile=4,2 tile-k=64 promote=1 vectorize=1"

# (workload, (m, n, k), options), large first: the split-K workspaces and the
# residual block's intermediate h are what the scratch array holds.
CALLS = [
    ("mbr", (256, 2048, 4096), STAGED + " split-k=8"),     # 16 MiB workspace
    ("resmlp", (256, 512, 2048), STAGED + " split-k=2"),   # 4 MiB workspace + 2 MiB h
    ("mbr", (64, 512, 1024), STAGED + " split-k=4"),       # smaller: 512 KiB workspace
    ("resmlp", (128, 128, 256), STAGED),                   # smaller: 128 KiB h, no workspace
]


def _run(kern, bufs, out, noalloc, torch):
    out.fill_(float("nan"))
    ptrs = [b.data_ptr() for b in bufs] + [out.data_ptr()]
    stream = torch.cuda.current_stream().cuda_stream
    (kern.launch_noalloc if noalloc else kern.launch)(ptrs, stream)
    torch.cuda.synchronize()
    return out.cpu().numpy().copy()


@pytest.mark.gpu
def test_noalloc_first_call_under_graph_capture():
    """tf_launch_noalloc's first call in the process happens inside a HIP graph
    capture (torch.cuda.graph), so the scratch array's address is looked up
    there: a split-K mbr and the residual block (split-K workspace plus the
    intermediate h), each graph replayed four times with eager work and a
    synchronisation between replays, give tf_launch's eager bits every time.
    (Runs first in this module: later tests have resolved the address.)"""
    import torch
    dev = torch.device("cuda:0")
    for workload, (m, n, k), opts in [("mbr", (256, 1024, 2048), STAGED + " split-k=4"),
                                      ("resmlp", (256, 512, 1024), STAGED + " split-k=2")]:
        print(f"noalloc under capture {workload} {m}x{n}x{k} [{opts}]", flush=True)
        ins = tc.make_inputs(workload, m, n, k)
        bufs = [torch.from_numpy(np.ascontiguousarray(v)).to(dev) for v in ins.values()]
        out = torch.empty((m, n), device=dev, dtype=torch.float32)
        kern = _lib.Kernel(tc.gen_mlir(workload, m, n, k), opts, "noalloc.mlir")
        want = _run(kern, bufs, out, False, torch)
        ptrs = [b.data_ptr() for b in bufs] + [out.data_ptr()]
        graph = torch.cuda.CUDAGraph()
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        with torch.cuda.graph(graph):
            kern.launch_noalloc(ptrs, torch.cuda.current_stream().cuda_stream)
        for replay in range(4):
            out.fill_(float("nan"))
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            got = out.cpu().numpy()
            assert not np.isnan(got).any(), (workload, replay)
            assert o.bitwise_diff(got, want) == 0, (workload, replay)
        del graph


@pytest.mark.gpu
def test_noalloc_matches_tf_launch_on_consecutive_calls():
    import torch
    dev = torch.device("cuda:0")
    for workload, (m, n, k), opts in CALLS:
        print(f"noalloc {workload} {m}x{n}x{k} [{opts}]", flush=True)
        ins = tc.make_inputs(workload, m, n, k)
        bufs = [torch.from_numpy(np.ascontiguousarray(v)).to(dev) for v in ins.values()]
        out = torch.empty((m, n), device=dev, dtype=torch.float32)
        kern = _lib.Kernel(tc.gen_mlir(workload, m, n, k), opts, "noalloc.mlir")
        got = _run(kern, bufs, out, True, torch)
        want = _run(kern, bufs, out, False, torch)
        assert not np.isnan(got).any()
        assert o.bitwise_diff(got, want) == 0, (workload, m, n, k)
        if workload == "mbr":
            ref, bound = o.fp64_reference("mbr", ins)
            assert o.e1_metrics(got, ref, bound)["max_err_over_bound"] <= 1.0
            assert o.mask_mismatches(got, o.preactivation64(ins), bound) == 0


def test_noalloc_refuses_programs_beyond_the_scratch_array():
    """The residual block at its benchmark size keeps a 128 MiB intermediate:
    more than the 32 MiB array, so the call fails before any device work
    (which is why this runs without a GPU)."""
    kern = _lib.Kernel(tc.gen_mlir("resmlp", 4096, 2048, 8192), STAGED, "noalloc.mlir")
    arr = (ctypes.c_void_p * 6)(*([256] * 6))
    assert _lib.lib().tf_launch_noalloc(kern.h, arr, None) == -4
    msg = _lib.lib().tf_last_error().decode()
    assert "needs 134217728 bytes of scratch" in msg and "has 33554432" in msg, msg
    with pytest.raises(RuntimeError, match="use tf_launch, which allocates them"):
        kern.launch_noalloc([256] * 6)
