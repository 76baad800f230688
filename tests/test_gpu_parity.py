"""GPU parity: libtforge_hip's kernels on cuda:0 against the CPU oracle.

Bars (python/tforge_gpu.py:112-145, plus exact ReLU masks):
  * staged MFMA kernels: err/bound <= 1 against the FP64 reference with the
    reference's gamma_{K+1} bound, no NaN (outputs are NaN-prefilled), and
    exact ReLU masks wherever |pre-activation| exceeds the bound;
  * direct kernels: bit-identical to the sequential-FMA closed form (the
    reference's naive kernel arithmetic);
  * element-op programs: bit-exact against the oracle's IEEE ops.
Every call goes through the C ABI (tf_compile / tf_run / tf_launch).
"""

import numpy as np
import pytest

from oracle import oracle as o
from tensorforge_amd import _lib
from tensorforge_amd import costmodel as cm
from tensorforge_amd import tforge_cpu as tc
from tensorforge_amd import tforge_gpu as tg

pytestmark = pytest.mark.gpu

STAGED = "block-tile={},{} thread-tile={},{} tile-k={} promote=1 vectorize=1"


def run_prog(workload, m, n, k, options, ins=None, logical=None):
    pm, pn, pk = (m, n, k) if logical is None else logical
    ins = ins or o.make_inputs(workload, m, n, k)
    kern = _lib.Kernel(tc.gen_mlir(workload, pm, pn, pk if k else None), options, "t.mlir")
    out = np.empty((m, n), np.float32)
    lg = None if logical is None or tuple(logical) == (m, n, k) else (m, n, k)
    kern.run([np.ascontiguousarray(v) for v in ins.values()], out, logical=lg)
    return ins, out


def assert_bound(workload, ins, out):
    ref, bound = o.fp64_reference(workload, ins)
    assert not np.isnan(out).any(), "unwritten (NaN-prefilled) outputs"
    eob = o.e1_metrics(out, ref, bound)["max_err_over_bound"]
    assert eob <= 1.0, eob
    if workload == "mbr":
        assert o.mask_mismatches(out, o.preactivation64(ins), bound) == 0
    return eob


@pytest.mark.parametrize("workload", ["mbr", "matmul"])
@pytest.mark.parametrize("shape", [(256, 256, 128), (67, 17, 33), (777, 1111, 333), (1, 1, 1), (64, 300, 5)])
@pytest.mark.parametrize("tt", [(1, 1), (2, 2), (4, 4), (8, 4)])
def test_direct_bitwise_fma(workload, shape, tt):
    m, n, k = shape
    tm, tn = tt
    opts = f"block-tile={16 * tm},{16 * tn} thread-tile={tm},{tn}"
    ins, out = run_prog(workload, m, n, k, opts)
    want = o.matmul_fma(ins["a"], ins["b"])
    if workload == "mbr":
        want = o.epilogue(want, ins["bias"], relu=True)
    assert o.bitwise_diff(out, want) == 0


@pytest.mark.parametrize("workload", ["mbr", "matmul"])
@pytest.mark.parametrize("cfg", [(128, 128, 8, 8, 32), (128, 64, 8, 4, 16), (64, 64, 4, 4, 16), (32, 32, 4, 4, 8),
                                 (256, 128, 8, 8, 32), (64, 128, 8, 4, 32), (128, 128, 4, 4, 64)])
@pytest.mark.parametrize("shape", [(256, 256, 128), (512, 256, 1024)])
def test_staged_bound(workload, cfg, shape):
    m, n, k = shape
    pm, pn, pk = cm.padded(cfg, m, n, k)
    ins, out = run_prog(workload, m, n, k, STAGED.format(*cfg), logical=(pm, pn, pk))
    assert_bound(workload, ins, out)


@pytest.mark.parametrize("workload", ["mbr", "matmul"])
def test_staged_padded_ragged(workload):
    """777x1111x333 compiled at the padded 896x1152x336 (reference
    docs/stage8.md:107); the library pads and unpads."""
    m, n, k = 777, 1111, 333
    cfg = (128, 64, 8, 4, 16)
    ins, out = run_prog(workload, m, n, k, STAGED.format(*cfg), logical=cm.padded(cfg, m, n, k))
    assert_bound(workload, ins, out)


def test_every_staged_instantiation():
    """Each ahead-of-time instantiation (all promote / vectorize variants) on
    a small problem padded to its tiles; each masked twin on a problem that
    is ragged in M, N and K."""
    ins_cache = {}
    failures = []
    for e in _lib.registry():
        if e["family"] != "staged":
            continue
        bm, bn, tm, tn, bk, p, v = e["cfg"]
        m, n, k = 2 * bm, 2 * bn, 2 * bk if bk >= 32 else 64
        masked = e["name"].endswith("_masked")
        if masked:
            m, n, k = m - 3, n - 5, k - 7
        key = (m, n, k)
        if key not in ins_cache:
            ins = o.make_inputs("mbr", m, n, k)
            ins_cache[key] = (ins,) + o.fp64_reference("mbr", ins)
        ins, ref, bound = ins_cache[key]
        opts = f"block-tile={bm},{bn} thread-tile={tm},{tn} tile-k={bk} promote={p} vectorize={v}"
        if masked:
            opts += " mask-edges=1"
        print(f"instantiation {e['name']} at {m}x{n}x{k}", flush=True)
        _, out = run_prog("mbr", m, n, k, opts, ins=ins)
        eob = o.e1_metrics(out, ref, bound)["max_err_over_bound"]
        if np.isnan(out).any() or eob > 1.0:
            failures.append((e["name"], eob))
    assert not failures, failures


def test_reference_space_stand_in_layouts():
    """The 30 configurations of the reference's Stage 9 grid whose own wave
    tile cannot tile the block (python/costmodel.py:49-60) run on their
    stand-in wave layout: each meets the reference bound with exact ReLU
    masks on a padded problem and a ragged masked one, and equals, bit for
    bit, the same problem run with the stand-in's own thread tile."""
    shapes = {}
    for cfg in cm.reference_space():
        bm, bn, tm, tn, bk = cfg
        ktm, ktn = cm.kernel_tile(cfg)
        if (ktm, ktn) == (tm, tn):
            continue
        for masked in (False, True):
            if masked and cfg in ((32, 128, 8, 8, 32), (128, 32, 8, 8, 32)):
                continue  # no masked twin (20 staging vectors per thread)
            m, n, k = (2 * bm - 3, 2 * bn - 5, 4 * bk - 7) if masked else (2 * bm, 2 * bn, 4 * bk)
            if (m, n, k) not in shapes:
                ins = o.make_inputs("mbr", m, n, k)
                shapes[(m, n, k)] = (ins,) + o.fp64_reference("mbr", ins) + (o.preactivation64(ins),)
            ins, ref, bound, z = shapes[(m, n, k)]
            extra = " mask-edges=1" if masked else ""
            print(f"stand-in {cfg} -> thread-tile {ktm},{ktn} at {m}x{n}x{k}{extra}", flush=True)
            _, out = run_prog("mbr", m, n, k, cm.options(cfg) + extra, ins=ins)
            assert not np.isnan(out).any()
            assert o.e1_metrics(out, ref, bound)["max_err_over_bound"] <= 1.0, cfg
            assert o.mask_mismatches(out, z, bound) == 0, cfg
            _, own = run_prog("mbr", m, n, k, STAGED.format(bm, bn, ktm, ktn, bk) + extra, ins=ins)
            assert o.bitwise_diff(out, own) == 0, cfg


@pytest.mark.parametrize("which", ["naive", "tuned", "default"])
def test_headline_2048(which):
    """The headline shape through the product's check() (reference bound) with
    the reference's default naive options, the autotuned configuration and the
    cost model's pick, and 64 sampled rows of the same output against the
    oracle: the reference bound and the ReLU-mask gate."""
    opts = {"naive": "block-tile=16,16 thread-tile=1,1",
            "tuned": cm.tuned_options("mbr", 2048, 2048, 2048),
            "default": cm.options(cm.default_config(2048, 2048, 2048))}[which]
    d, launch = tg.compile_kernel("mbr", 2048, 2048, 2048, opts, tag="test")
    res, out = tg.check("mbr", 2048, 2048, 2048, d, launch)
    print(f"headline {which} {launch['kernel']}: err/bound {res['err_over_bound']:.5f} "
          "(reference FMA kernels 0.00232, results/gpu/stage8.csv:86)", flush=True)
    assert res["pass"], res
    assert res["err_over_bound"] < 0.05
    ins = o.make_inputs("mbr", 2048, 2048, 2048)
    rows = np.sort(np.random.default_rng(3).choice(2048, size=64, replace=False))
    sub = {"a": ins["a"][rows], "b": ins["b"], "bias": ins["bias"]}
    ref, bound = o.fp64_reference("mbr", sub)
    assert o.e1_metrics(out[rows], ref, bound)["max_err_over_bound"] <= 1.0
    assert o.mask_mismatches(out[rows], o.preactivation64(sub), bound) == 0


@pytest.mark.parametrize("workload,shape", [("relu", (999, 1001)), ("bias_add", (33, 17)), ("add", (1024, 1024)),
                                            ("bias_add", (300, 1024)), ("relu", (64, 36))])
@pytest.mark.parametrize("opts", ["block-tile=16,16 thread-tile=1,1", "block-tile=4,256 thread-tile=1,4",
                                  "block-tile=8,512 thread-tile=2,8"])
def test_elementwise_bit_exact(workload, shape, opts):
    """Scalar and 128-bit paths (thread tiles 4k wide on aligned rows; ragged
    and unaligned widths fall back per element) are bit-exact."""
    m, n = shape
    d, launch = tg.compile_kernel(workload, m, n, None, opts, tag="test")
    res, out = tg.check(workload, m, n, None, d, launch)
    assert res["pass"], res
    assert o.bitwise_diff(out, o.elementwise(workload, o.make_inputs(workload, m, n, None))) == 0


@pytest.mark.parametrize("workload", ["relu", "bias_add", "add"])
@pytest.mark.parametrize("opts,shape", [
    ("block-tile=16,16 thread-tile=1,1", (37, 512)),     # the reference default, 32-bit path
    ("block-tile=16,16 thread-tile=2,2", (20, 1024)),    # 2 x 2 per thread, 32-bit path
    ("block-tile=4,256 thread-tile=1,4", (5, 2048)),     # one 128-bit vector per thread
    ("block-tile=8,512 thread-tile=2,8", (9, 4096)),     # 4 vectors per thread
])
def test_elementwise_row_chunks_bit_exact(workload, opts, shape):
    """N a multiple of a workgroup's BM*BN elements and M not a multiple of
    the block tile (the grid's last row of workgroups is partly past M), on
    the 32-bit and 128-bit paths, 1 to 4 vectors per thread."""
    m, n = shape
    d, launch = tg.compile_kernel(workload, m, n, None, opts, tag="test")
    res, out = tg.check(workload, m, n, None, d, launch)
    assert res["pass"], res
    assert o.bitwise_diff(out, o.elementwise(workload, o.make_inputs(workload, m, n, None))) == 0


@pytest.mark.parametrize("workload", ["relu", "bias_add", "add"])
def test_elementwise_misaligned_buffers(workload):
    """tf_launch on buffers 4 bytes past a 16-byte boundary (torch views one
    float into an allocation): the element-op kernel drops to its 32-bit path
    (and loads the bias in the epilogue) and stays bit-exact; N = 1024 would
    otherwise take the 128-bit path."""
    import torch
    dev = torch.device("cuda:0")
    m, n = 37, 1024
    opts = "block-tile=4,256 thread-tile=1,4"
    ins = o.make_inputs(workload, m, n, None)
    views = []
    for v in ins.values():
        flat = np.ascontiguousarray(v).ravel()
        base = torch.zeros(flat.size + 1, device=dev)
        base[1:] = torch.from_numpy(flat).to(dev)
        views.append(base[1:].view(v.shape))
    out_base = torch.full((m * n + 1,), float("nan"), device=dev)
    out = out_base[1:].view(m, n)
    assert all(t.data_ptr() % 16 == 4 for t in views + [out])
    kern = _lib.Kernel(tc.gen_mlir(workload, m, n, None), opts, "t.mlir")
    kern.launch([t.data_ptr() for t in views] + [out.data_ptr()], torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert o.bitwise_diff(out.cpu().numpy(), o.elementwise(workload, ins)) == 0


def test_launch_abi_matches_run():
    """tf_launch on caller-owned device buffers (torch) gives the same bits as tf_run."""
    import torch
    m = n = k = 512
    opts = STAGED.format(128, 128, 8, 8, 32)
    ins, out = run_prog("mbr", m, n, k, opts)
    dev = torch.device("cuda:0")
    bufs = [torch.from_numpy(v).to(dev) for v in ins.values()]
    c = torch.full((m, n), float("nan"), device=dev)
    kern = _lib.Kernel(tc.gen_mlir("mbr", m, n, k), opts, "t.mlir")
    stream = torch.cuda.current_stream()
    kern.launch([b.data_ptr() for b in bufs] + [c.data_ptr()], stream.cuda_stream)
    torch.cuda.synchronize()
    assert o.bitwise_diff(c.cpu().numpy(), out) == 0


def test_concurrent_streams_with_separate_handles():
    """Handles launched concurrently on their own streams (tf_launch's
    contract: one handle per concurrent stream) give the bits each gives alone:
    a plain staged kernel, a split-K kernel (private partial-sum workspace) and
    the residual block (private intermediate h), two handles of each, 20
    rounds on 6 streams."""
    import torch
    dev = torch.device("cuda:0")
    cases = [("mbr", (512, 512, 512), STAGED.format(128, 128, 8, 4, 32)),
             ("mbr", (512, 512, 512), STAGED.format(64, 128, 4, 4, 32) + " split-k=4"),
             ("resmlp", (256, 128, 512), STAGED.format(64, 64, 4, 4, 32))]
    jobs = []
    for wl, (m, n, k), opts in cases:
        ins = tc.make_inputs(wl, m, n, k)
        bufs = [torch.from_numpy(np.ascontiguousarray(v)).to(dev) for v in ins.values()]
        for _ in range(2):
            kern = _lib.Kernel(tc.gen_mlir(wl, m, n, k), opts, "t.mlir")
            out = torch.full((m, n), float("nan"), device=dev)
            jobs.append((kern, [b.data_ptr() for b in bufs] + [out.data_ptr()], out, bufs))
    cur = torch.cuda.current_stream()
    for kern, ptrs, out, _ in jobs:
        kern.launch(ptrs, cur.cuda_stream)
    torch.cuda.synchronize()
    alone = [out.cpu().numpy().copy() for _, _, out, _ in jobs]
    for _, _, out, _ in jobs:
        out.fill_(float("nan"))
    streams = [torch.cuda.Stream() for _ in jobs]
    torch.cuda.synchronize()
    for _ in range(20):
        for (kern, ptrs, _, _), s in zip(jobs, streams):
            kern.launch(ptrs, s.cuda_stream)
    torch.cuda.synchronize()
    for (_, _, out, _), want in zip(jobs, alone):
        assert not np.isnan(want).any()
        assert o.bitwise_diff(out.cpu().numpy(), want) == 0


def test_launch_replays_from_a_hip_graph():
    """tf_launch enqueues only kernel launches on the caller's stream (no
    memsets; a handle allocates its workspace and intermediates on its first
    launch), so after one eager launch it can be captured into a HIP graph:
    a plain staged kernel, split-K (GEMM + reduction) and the residual block
    (two layers and an intermediate) replay the eager bits five times, with
    eager work and synchronisation between the replays."""
    import torch
    dev = torch.device("cuda:0")
    cases = [("mbr", (512, 512, 512), STAGED.format(128, 128, 8, 4, 32)),
             ("mbr", (512, 512, 512), STAGED.format(64, 128, 4, 4, 32) + " split-k=4"),
             ("resmlp", (256, 128, 512), STAGED.format(64, 64, 4, 4, 32))]
    for wl, (m, n, k), opts in cases:
        ins = tc.make_inputs(wl, m, n, k)
        bufs = [torch.from_numpy(np.ascontiguousarray(v)).to(dev) for v in ins.values()]
        kern = _lib.Kernel(tc.gen_mlir(wl, m, n, k), opts, "t.mlir")
        out = torch.full((m, n), float("nan"), device=dev)
        ptrs = [b.data_ptr() for b in bufs] + [out.data_ptr()]
        kern.launch(ptrs, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        want = out.cpu().numpy().copy()
        assert not np.isnan(want).any()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            kern.launch(ptrs, torch.cuda.current_stream().cuda_stream)
        for rep in range(5):
            out.fill_(float("nan"))
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert o.bitwise_diff(out.cpu().numpy(), want) == 0, (wl, opts, rep)


@pytest.mark.parametrize("workload,shape,opts", [
    ("mbr", (0, 4, 4), "block-tile=16,16 thread-tile=1,1"),
    ("mbr", (4, 0, 4), "block-tile=16,16 thread-tile=1,1"),
    ("mbr", (5, 4, 0), "block-tile=16,16 thread-tile=1,1"),
    ("matmul", (8, 8, 0), "block-tile=16,16 thread-tile=1,1"),
    ("mbr", (0, 64, 64), STAGED.format(64, 64, 4, 4, 32)),
    ("mbr", (64, 64, 0), STAGED.format(64, 64, 4, 4, 32)),
    ("mbr", (65, 70, 0), STAGED.format(64, 64, 4, 4, 32) + " mask-edges=1"),
    ("matmul", (64, 128, 0), STAGED.format(64, 64, 2, 2, 64)),
])
def test_empty_dimensions(workload, shape, opts):
    """Zero-sized M or N launch nothing; K = 0 is an empty sum, +0.0, so the
    output is the epilogue of zero: relu(0 + bias) for mbr, +0.0 for matmul."""
    m, n, k = shape
    ins = o.make_inputs(workload, m, n, k)
    kern = _lib.Kernel(tc.gen_mlir(workload, m, n, k), opts, "t.mlir")
    out = np.full((m, n), np.nan, np.float32)
    kern.run([np.ascontiguousarray(v) for v in ins.values()], out)
    if m and n:
        want = np.zeros((m, n), np.float32)
        if workload == "mbr":
            want = o.epilogue(want, ins["bias"], relu=True)
        assert o.bitwise_diff(out, want) == 0


@pytest.mark.parametrize("shape", [(0, 8), (8, 0)])
def test_empty_element_op(shape):
    m, n = shape
    d, launch = tg.compile_kernel("relu", m, n, None, "block-tile=4,256 thread-tile=1,4", tag="test")
    res, out = tg.check("relu", m, n, None, d, launch)
    assert res["pass"] and out.shape == (m, n)


def test_deterministic():
    opts = STAGED.format(128, 64, 8, 4, 16)
    _, a = run_prog("mbr", 512, 512, 512, opts)
    _, b = run_prog("mbr", 512, 512, 512, opts)
    assert o.bitwise_diff(a, b) == 0


def test_unfused_program_matches_fused_bits():
    """fuse-elementwise=0 runs matmul, bias_add and relu as three launches;
    with the direct kernel both are the same FMA chain + IEEE ops."""
    m, n, k = 300, 200, 100
    ins = o.make_inputs("mbr", m, n, k)
    _, fused = run_prog("mbr", m, n, k, "block-tile=16,16 thread-tile=1,1", ins=ins)
    _, unfused = run_prog("mbr", m, n, k, "block-tile=16,16 thread-tile=1,1 fuse-elementwise=0", ins=ins)
    assert o.bitwise_diff(fused, unfused) == 0


def test_blas_mode_bound():
    res, out = tg.check("mbr", 1000, 1000, 1000, mode="cublas")
    assert res["pass"], res


def test_resmlp_small():
    m, n, k = 256, 128, 512
    d, launch = tg.compile_kernel("resmlp", m, n, k, STAGED.format(128, 128, 8, 8, 32), tag="test")
    assert len(launch["launches"]) == 2
    res, out = tg.check("resmlp", m, n, k, d, launch)
    assert res["pass"], res


@pytest.mark.parametrize("workload", ["mbr", "matmul"])
@pytest.mark.parametrize("cfg,splits,shape", [
    ((64, 64, 4, 4, 32), 8, (64, 4096, 4096)),     # the skinny measured shape
    ((128, 128, 4, 4, 32), 3, (256, 256, 1024)),   # uneven slab ranges: 32 slabs over 3
    ((64, 64, 4, 4, 16), 5, (128, 192, 80)),       # one slab per split
    ((128, 64, 8, 4, 16), 2, (777, 1111, 333)),    # padded ragged problem
])
def test_split_k_bound(workload, cfg, splits, shape):
    m, n, k = shape
    opts = STAGED.format(*cfg) + f" split-k={splits}"
    ins, out = run_prog(workload, m, n, k, opts, logical=cm.padded(cfg, m, n, k))
    assert_bound(workload, ins, out)


def test_split_k_handle_reuse_is_deterministic():
    """The partial-sum workspace is reused across launches: after 30 launches
    on one handle, a correctness run on it gives the bits of a fresh handle
    (the slices are added in a fixed order)."""
    m, n, k = 128, 512, 2048
    opts = STAGED.format(64, 64, 4, 4, 32) + " split-k=7"
    ins = o.make_inputs("mbr", m, n, k)
    arrays = [np.ascontiguousarray(v) for v in ins.values()]
    kern = _lib.Kernel(tc.gen_mlir("mbr", m, n, k), opts, "t.mlir")
    first = np.empty((m, n), np.float32)
    kern.run(arrays, first)
    kern.bench(arrays, warmup=10, reps=20)
    again = np.empty((m, n), np.float32)
    kern.run(arrays, again)
    _, fresh = run_prog("mbr", m, n, k, opts, ins=ins)
    assert o.bitwise_diff(first, again) == 0 and o.bitwise_diff(first, fresh) == 0
    assert_bound("mbr", ins, first)


def test_split_k_resmlp():
    m, n, k = 256, 128, 512
    d, launch = tg.compile_kernel("resmlp", m, n, k, STAGED.format(128, 128, 4, 4, 32) + " split-k=4", tag="test")
    assert [L["grid"][2] for L in launch["launches"]] == [4, 4]
    res, out = tg.check("resmlp", m, n, k, d, launch)
    assert res["pass"], res


MASKED_SHAPES = [(777, 1111, 333), (1000, 1000, 1000), (67, 17, 33), (1, 1, 1), (130, 258, 1031), (64, 4095, 4097)]


@pytest.mark.parametrize("workload", ["mbr", "matmul"])
@pytest.mark.parametrize("shape", MASKED_SHAPES)
@pytest.mark.parametrize("cfg,extra", [((128, 64, 8, 4, 16), ""), ((128, 128, 4, 4, 32), ""),
                                       ((64, 64, 4, 4, 32), " split-k=3"),
                                       ((64, 64, 4, 4, 32), " vectorize=0")])
def test_masked_edges_equal_pad_path_bits(workload, shape, cfg, extra):
    """mask-edges=1 on the true shape gives the bits of the reference's pad
    path (zero-padded copies, padded kernel, unpad): the same tiles see the
    same zeros.  Both pass the FP64 bound."""
    m, n, k = shape
    opts = STAGED.format(*cfg) + extra
    if "vectorize=0" in extra:
        opts = opts.replace("vectorize=1 vectorize=0", "vectorize=0")
    slabs = cm.padded(cfg, m, n, k)[2] // cfg[4]
    if "split-k" in extra and slabs < 3:
        # fewer K slabs than splits: the library refuses, naming both counts
        with pytest.raises(RuntimeError, match=f"split-k 3 exceeds the {slabs} K slabs of this matmul"):
            _lib.Kernel(tc.gen_mlir(workload, m, n, k), opts + " mask-edges=1", "t.mlir")
        return
    ins = o.make_inputs(workload, m, n, k)
    _, masked = run_prog(workload, m, n, k, opts + " mask-edges=1", ins=ins)
    _, padded = run_prog(workload, m, n, k, opts, ins=ins, logical=cm.padded(cfg, m, n, k))
    assert o.bitwise_diff(masked, padded) == 0
    assert_bound(workload, ins, masked)


@pytest.mark.parametrize("workload", ["mbr", "matmul"])
@pytest.mark.parametrize("shape", [(130, 70, 91), (200, 300, 1010), (97, 130, 313), (65, 66, 109), (64, 64, 96)])
@pytest.mark.parametrize("cfg", [(64, 64, 4, 4, 16), (128, 64, 8, 4, 16), (128, 128, 8, 8, 64)])
def test_masked_k_tail_equals_pad_path_bits(workload, shape, cfg):
    """The end of the K loop of masked kernels: the slab holding row K - 1 is
    loaded element by element DEPTH slabs before it is stored with the zero
    fill, after a steady loop of an even number of slabs.  Tile-k 16 (two
    staging sets): K = 91, 1010, 313, 96, 109 give 6, 64, 20, 6, 7 slabs (an
    even and an odd count after the steady loop); tile-k 64 (the 128 x 128
    configuration, one staging set): 5, 16 and 2 slabs.  The pad path's bits
    and the bound."""
    m, n, k = shape
    opts = STAGED.format(*cfg)
    ins = o.make_inputs(workload, m, n, k)
    _, masked = run_prog(workload, m, n, k, opts + " mask-edges=1", ins=ins)
    _, padded = run_prog(workload, m, n, k, opts, ins=ins, logical=cm.padded(cfg, m, n, k))
    assert o.bitwise_diff(masked, padded) == 0
    assert_bound(workload, ins, masked)


NARROW_SHAPES = [(5, 2, 3), (33, 3, 70), (70, 6, 9), (65, 7, 2), (2, 130, 5), (129, 1, 257)]


@pytest.mark.parametrize("workload", ["mbr", "matmul"])
@pytest.mark.parametrize("shape", NARROW_SHAPES)
@pytest.mark.parametrize("cfg", [(64, 64, 2, 2, 64), (64, 64, 4, 4, 32)])
def test_masked_narrow_shapes_equal_pad_path_bits(workload, shape, cfg):
    """Rows narrower than one 16-byte vector (N < 4: every slab guarded),
    unaligned rows (N % 4 != 0), K below one k-chunk, on 16x16 and 32x32
    MFMA blocks: the pad path's bits and the bound."""
    m, n, k = shape
    opts = STAGED.format(*cfg)
    ins = o.make_inputs(workload, m, n, k)
    _, masked = run_prog(workload, m, n, k, opts + " mask-edges=1", ins=ins)
    _, padded = run_prog(workload, m, n, k, opts, ins=ins, logical=cm.padded(cfg, m, n, k))
    assert o.bitwise_diff(masked, padded) == 0
    assert_bound(workload, ins, masked)


def test_masked_resmlp_ragged():
    """Residual block at a shape that is not a multiple of the tiles."""
    m, n, k = 200, 72, 136
    ins = tc.make_inputs("resmlp", m, n, k)
    opts = STAGED.format(64, 64, 4, 4, 32) + " mask-edges=1"
    kern = _lib.Kernel(tc.gen_mlir("resmlp", m, n, k), opts, "t.mlir")
    y = np.empty((m, n), np.float32)
    kern.run([np.ascontiguousarray(v) for v in ins.values()], y)
    assert tg._resmlp_check(ins, y)["pass"]


@pytest.mark.parametrize("shape", [(77, 45, 53), (130, 258, 97), (9, 6, 3)])
@pytest.mark.parametrize("cfg", [(64, 64, 4, 4, 32), (64, 64, 2, 2, 64)])
def test_masked_resmlp_unaligned_rows_equal_unfused_bits(shape, cfg):
    """Residual block with mask-edges at shapes whose rows are not 16-byte
    aligned (n, k not multiples of 4): the fused epilogue (bias, relu, add of
    the row-indexed residual) writes the bits of the unfused program, where
    each element op is its own launch on the same GEMM output."""
    m, n, k = shape
    ins = tc.make_inputs("resmlp", m, n, k)
    arrays = [np.ascontiguousarray(v) for v in ins.values()]
    outs = []
    for extra in ("", " fuse-elementwise=0"):
        kern = _lib.Kernel(tc.gen_mlir("resmlp", m, n, k), STAGED.format(*cfg) + " mask-edges=1" + extra, "t.mlir")
        y = np.empty((m, n), np.float32)
        kern.run(arrays, y)
        outs.append(y)
    assert o.bitwise_diff(outs[0], outs[1]) == 0
    assert tg._resmlp_check(ins, outs[0])["pass"]


def test_info_and_bench_keys():
    d, launch = tg.compile_kernel("mbr", 1024, 1024, 1024, STAGED.format(128, 128, 8, 8, 32), tag="test")
    inf = tg.info("mbr", 1024, 1024, 1024, d, launch)
    assert inf["threads"] == 256 and inf["blocks_per_sm"] >= 1
    r = tg.bench("mbr", 1024, 1024, 1024, d, launch, warmup=2, reps=5)
    for key in ("gpu", "median_ms", "min_ms", "std_ms", "sm_clock_median_mhz", "padded", "grid", "block"):
        assert key in r
    assert r["median_ms"] > 0


def test_bench_with_l2_flush_is_not_faster():
    """--flush (ref:runners/gpu/tforge-gpu-bench.cu:337-350): a 512 MiB fill
    before every rep evicts A and B from L2 and the MALL, so the flushed
    median cannot beat the warm one (small tolerance for clock noise)."""
    m = n = k = 1024
    d, launch = tg.compile_kernel("mbr", m, n, k, STAGED.format(64, 64, 4, 2, 64), tag="test")
    warm = tg.bench("mbr", m, n, k, d, launch, warmup=20, reps=50)
    cold = tg.bench("mbr", m, n, k, d, launch, warmup=20, reps=50, flush=True)
    assert cold["l2_flush"] == 1 and warm["l2_flush"] == 0
    assert cold["median_ms"] >= 0.97 * warm["median_ms"], (cold["median_ms"], warm["median_ms"])


def test_clock_probe_reads_the_shader_clock():
    """The device probe reads a plausible MI355X shader clock on every XCD,
    and tf_bench reports one sample per rep from it."""
    mean, lo, hi = _lib.clock_probe()
    assert 100.0 <= lo <= mean <= hi <= 3000.0, (mean, lo, hi)
    d, launch = tg.compile_kernel("mbr", 512, 512, 512, STAGED.format(64, 64, 4, 2, 64), tag="test")
    r = tg.bench("mbr", 512, 512, 512, d, launch, warmup=5, reps=20)
    assert 100.0 <= r["sm_clock_min_mhz"] <= r["sm_clock_median_mhz"] <= r["sm_clock_max_mhz"] <= 3000.0, r
