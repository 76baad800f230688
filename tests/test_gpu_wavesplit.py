"""The wave-split kernel (wave-split-k=1): the waves of a workgroup each reduce
their own range of K slabs for the workgroup's whole output tile and add the
partial tiles in LDS in wave order.  Its bar is the staged kernels': the
reference's FP64 bound with exact ReLU masks and no unwritten (NaN-prefilled)
output, on every instantiation and on the cases its K split makes special:
fewer slabs than waves (idle waves, leading zero slabs), uneven slab ranges,
K = 0, split-K across workgroups on top, a padded ragged problem, the
residual block's add epilogue, and the skinny layer 64 x 4096 x 4096 it is
built for.  Its results are deterministic (fixed summation order)."""

import numpy as np
import pytest

from oracle import oracle as o
from tensorforge_amd import _lib
from tensorforge_amd import costmodel as cm
from tensorforge_amd import tforge_cpu as tc
from tensorforge_amd import tforge_gpu as tg

pytestmark = pytest.mark.gpu

WAVE = "block-tile={},{} thread-tile={},{} tile-k={} promote=1 vectorize=1 wave-split-k=1"


def _run(workload, shape, opts, ins, logical=None):
    m, n, k = shape
    pm, pn, pk = logical or shape
    kern = _lib.Kernel(tc.gen_mlir(workload, pm, pn, pk), opts, "t.mlir")
    out = np.empty((m, n), np.float32)
    kern.run([np.ascontiguousarray(v) for v in ins.values()], out,
             logical=None if logical is None or tuple(logical) == tuple(shape) else shape)
    return kern, out


def _bound(workload, ins, out):
    ref, bound = o.fp64_reference(workload, ins)
    assert not np.isnan(out).any(), "unwritten (NaN-prefilled) outputs"
    eob = o.e1_metrics(out, ref, bound)["max_err_over_bound"]
    assert eob <= 1.0, eob
    if workload == "mbr":
        assert o.mask_mismatches(out, o.preactivation64(ins), bound) == 0
    return eob


def test_every_wave_split_instantiation():
    """Each instantiation (every thread tile of it) on a 2x2-tile problem whose
    K gives the waves uneven slab ranges (2W + 1 slabs over W waves)."""
    failures = []
    for e in _lib.registry():
        if e["family"] != "wavek":
            continue
        bm, bn, tm, tn, bk = e["cfg"][:5]
        w = (bm // tm) * (bn // tn) // 64
        m, n, k = 2 * bm, 2 * bn, (2 * w + 1) * bk
        print(f"instantiation {e['name']} at {m}x{n}x{k}", flush=True)
        ins = o.make_inputs("mbr", m, n, k)
        _, out = _run("mbr", (m, n, k), WAVE.format(bm, bn, tm, tn, bk), ins)
        ref, bound = o.fp64_reference("mbr", ins)
        eob = o.e1_metrics(out, ref, bound)["max_err_over_bound"]
        masks = o.mask_mismatches(out, o.preactivation64(ins), bound)
        if np.isnan(out).any() or eob > 1.0 or masks:
            failures.append((e["name"], eob, masks))
    assert not failures, failures


@pytest.mark.parametrize("workload", ["mbr", "matmul"])
@pytest.mark.parametrize("cfg,shape", [
    ((32, 32, 1, 1, 32), (64, 1024, 512)),    # one slab per wave (16 waves, 16 slabs)
    ((32, 32, 1, 1, 32), (64, 512, 160)),     # 5 slabs for 16 waves: 11 idle waves
    ((32, 32, 1, 1, 32), (32, 32, 32)),       # one slab in all
    ((32, 32, 2, 1, 64), (96, 160, 1216)),    # 19 slabs over 8 waves (leading zero slabs)
    ((16, 64, 1, 1, 16), (48, 320, 784)),     # 16x16 blocks, B staged through LDS
    ((64, 64, 2, 4, 16), (128, 128, 2048)),   # 64 accumulators per lane
])
def test_wave_split_bound(workload, cfg, shape):
    ins = o.make_inputs(workload, *shape)
    _, out = _run(workload, shape, WAVE.format(*cfg), ins)
    _bound(workload, ins, out)


@pytest.mark.parametrize("workload", ["mbr", "matmul"])
def test_wave_split_skinny_layer(workload):
    """The configuration the tuner records for 64 x 4096 x 4096, full size."""
    m, n, k = 64, 4096, 4096
    opts = cm.tuned_options(workload, m, n, k)
    if "wave-split-k=1" not in opts:
        opts = WAVE.format(32, 32, 1, 1, 32)
    ins = o.make_inputs(workload, m, n, k)
    kern, out = _run(workload, (m, n, k), opts, ins)
    assert kern.launches()[0]["family"] == "wavek"
    _bound(workload, ins, out)


@pytest.mark.parametrize("splits,shape", [(2, (64, 1024, 1024)), (3, (64, 512, 2080)), (4, (128, 256, 512))])
def test_wave_split_with_split_k_bound(splits, shape):
    ins = o.make_inputs("mbr", *shape)
    kern, out = _run("mbr", shape, WAVE.format(32, 32, 2, 1, 32) + f" split-k={splits}", ins)
    assert kern.launches()[0]["grid"][2] == splits
    _bound("mbr", ins, out)


@pytest.mark.parametrize("workload", ["mbr", "matmul"])
def test_wave_split_padded_ragged(workload):
    """A ragged problem compiled at its padded shape: the library pads and unpads."""
    m, n, k = 77, 111, 333
    cfg = (32, 32, 1, 1, 32)
    ins = o.make_inputs(workload, m, n, k)
    _, out = _run(workload, (m, n, k), WAVE.format(*cfg), ins, logical=cm.padded(cfg, m, n, k))
    _bound(workload, ins, out)


def test_wave_split_empty_k():
    """K = 0 is an empty sum: every wave adds nothing, the output is relu(bias)."""
    m, n = 64, 96
    ins = o.make_inputs("mbr", m, n, 0)
    _, out = _run("mbr", (m, n, 0), WAVE.format(32, 32, 1, 1, 32), ins)
    want = np.broadcast_to(o.relu(ins["bias"]), (m, n))
    assert o.bitwise_diff(out, want) == 0


def test_wave_split_resmlp():
    """The residual block: two wave-split stages, the second adding x."""
    m, n, k = 128, 128, 512
    d, launch = tg.compile_kernel("resmlp", m, n, k, WAVE.format(32, 32, 1, 1, 32), tag="test")
    assert [L["family"] for L in launch["launches"]] == ["wavek", "wavek"]
    res, _ = tg.check("resmlp", m, n, k, d, launch)
    assert res["pass"], res


def test_wave_split_is_deterministic():
    """Fixed slab ranges and a fixed partial-sum order: 30 more launches on
    the handle and a fresh handle give the first run's bits."""
    m, n, k = 64, 1024, 4096
    opts = WAVE.format(32, 32, 1, 1, 32)
    ins = o.make_inputs("mbr", m, n, k)
    arrays = [np.ascontiguousarray(v) for v in ins.values()]
    kern, first = _run("mbr", (m, n, k), opts, ins)
    kern.bench(arrays, warmup=10, reps=20)
    again = np.empty((m, n), np.float32)
    kern.run(arrays, again)
    _, fresh = _run("mbr", (m, n, k), opts, ins)
    assert o.bitwise_diff(first, again) == 0 and o.bitwise_diff(first, fresh) == 0


def test_wave_split_replays_from_a_hip_graph():
    """Captured after one eager launch, replayed five times with eager work and
    synchronisation in between: every replay gives the eager bits."""
    import torch
    m, n, k = 64, 2048, 2048
    dev = torch.device("cuda:0")
    ins = o.make_inputs("mbr", m, n, k)
    bufs = [torch.from_numpy(np.ascontiguousarray(v)).to(dev) for v in ins.values()]
    kern = _lib.Kernel(tc.gen_mlir("mbr", m, n, k), WAVE.format(32, 32, 1, 1, 32), "t.mlir")
    out = torch.full((m, n), float("nan"), device=dev)
    ptrs = [b.data_ptr() for b in bufs] + [out.data_ptr()]
    kern.launch(ptrs, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    want = out.cpu().numpy().copy()
    _bound("mbr", ins, want)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        kern.launch(ptrs, torch.cuda.current_stream().cuda_stream)
    for rep in range(5):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert o.bitwise_diff(out.cpu().numpy(), want) == 0, rep
