"""A seeded random sweep over the staged path's option space, through tf_run.

144 draws (seed 2026): workload mbr or matmul; each of M, N, K uniform in
1..700; a configuration from the 224-entry CDNA4 space; a split-K factor from
1, 2, 3, 5, 8 (at most the problem's K slabs); mask-edges on or off (on only
for configurations that have a masked twin).  Every draw meets the reference's
bar: no NaN in the NaN-prefilled output, max err/bound <= 1 against the FP64
reference (python/tforge_gpu.py:134-145), exact ReLU masks.  A masked draw
also equals the pad path (zero-padded copies through the unmasked kernel,
the reference runner's method) bit for bit, and a masked mbr draw run unfused
(fuse-elementwise=0: the matmul, bias_add and relu as three launches) equals
the fused kernel bit for bit (the fused epilogue performs the same IEEE
operations in registers).

48 more draws of the same kind come from the reference's own 105-configuration
Stage 9 grid, whose 30 configurations without a whole-wave tile of their own
run on a stand-in wave layout.

A third GEMM family draws 64 cases from the promote=0 / vectorize=0
instantiations (the ablation rungs, masked twins included) and from
promote=1 vectorize=1 ones with xcd-swizzle=0, at random shapes up to 400 and
split factors up to 3.

A fourth draws 72 wave-split configurations (wave-split-k=1; every entry of
the cost model's wave-split space is eligible) at random shapes up to 700,
compiled at the padded shape, with split factors 1, 2 or 3.

Two more families: 64 element-op programs (relu, bias_add, add; shapes up to
3000 x 8192, half of them with rows of whole workgroup chunks; every thread tile 1..8 x 1..8 that compiles) bit-exact against
NumPy float32 (python/tforge_gpu.py:116-126), and 32 residual blocks at ragged
shapes with masked tiles against the two-layer composed bound.
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


def _draws(count=144, seed=2026):
    rng = np.random.default_rng(seed)
    space = list(cm.config_space())
    twins = {tuple(e["cfg"][:5]) for e in _lib.registry() if e["family"] == "staged" and e["name"].endswith("_masked")}
    out = []
    while len(out) < count:
        wl = ("mbr", "matmul")[rng.integers(2)]
        m, n, k = (int(v) for v in rng.integers(1, 701, size=3))
        cfg = tuple(int(v) for v in space[rng.integers(len(space))])
        masked = bool(rng.integers(2)) and cfg in twins
        kk = k if masked else cm.padded(cfg, m, n, k)[2]
        slabs = -(-kk // cfg[4])
        split = int(rng.choice([1, 2, 3, 5, 8]))
        if split > slabs:
            split = 1
        out.append((wl, (m, n, k), cfg, split, masked))
    return out


def _reference_draws(count=48, seed=2031):
    """Draws from the reference's own Stage 9 grid (python/costmodel.py:49-60),
    stand-in wave layouts included, in the same form as _draws."""
    rng = np.random.default_rng(seed)
    space = cm.reference_space()
    twins = {tuple(e["cfg"][:5]) for e in _lib.registry() if e["family"] == "staged" and e["name"].endswith("_masked")}
    out = []
    while len(out) < count:
        wl = ("mbr", "matmul")[rng.integers(2)]
        m, n, k = (int(v) for v in rng.integers(1, 701, size=3))
        cfg = tuple(int(v) for v in space[rng.integers(len(space))])
        masked = bool(rng.integers(2)) and (cfg[:2] + cm.kernel_tile(cfg) + cfg[4:5]) in twins
        kk = k if masked else cm.padded(cfg, m, n, k)[2]
        split = int(rng.choice([1, 2, 3]))
        if split > -(-kk // cfg[4]):
            split = 1
        out.append((wl, (m, n, k), cfg, split, masked))
    return out


def _elt_draws(count=64, seed=2027):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < count:
        wl = ("relu", "bias_add", "add")[rng.integers(3)]
        m, n = (int(v) for v in rng.integers(1, 3001, size=2))
        tm, tn = (int(v) for v in rng.choice([1, 2, 4, 8], size=2))
        bm, bn = tm * int(rng.choice([1, 2, 4, 8, 16])), tn * int(rng.choice([4, 8, 16, 32, 64]))
        opts = f"block-tile={bm},{bn} thread-tile={tm},{tn}"
        if rng.random() < 0.5 and bm * bn <= 4096:  # rows of whole workgroup chunks
            n = bm * bn * int(rng.integers(1, max(2, 8192 // (bm * bn) + 1)))
        try:
            _lib.Kernel(tc.gen_mlir(wl, m, n, None), opts, "t.mlir")
        except RuntimeError:
            continue  # e.g. not a whole number of waves: tf_compile refuses it
        out.append((wl, (m, n), opts))
    return out


def _resmlp_draws(count=32, seed=2028):
    rng = np.random.default_rng(seed)
    space = [tuple(e["cfg"][:5]) for e in _lib.registry() if e["family"] == "staged" and e["name"].endswith("_masked")
             and e["cfg"][5] == 1 and e["cfg"][6] == 1]
    out = []
    while len(out) < count:
        m, n, k = (int(v) for v in rng.integers(1, 301, size=3))
        out.append(((m, n, k), space[rng.integers(len(space))]))
    return out


def _variant_draws(count=64, seed=2029):
    """The promote=0 / vectorize=0 instantiations (the ablation rungs) and
    promote=1 vectorize=1 ones with the XCD tile order switched off."""
    rng = np.random.default_rng(seed)
    reg = [e for e in _lib.registry() if e["family"] == "staged"]
    rungs = [e for e in reg if (e["cfg"][5], e["cfg"][6]) != (1, 1)]
    plain = [e for e in reg if (e["cfg"][5], e["cfg"][6]) == (1, 1) and not e["name"].endswith("_masked")]
    out = []
    while len(out) < count:
        e = rungs[rng.integers(len(rungs))] if rng.random() < 0.7 else plain[rng.integers(len(plain))]
        bm, bn, tm, tn, bk, pr, vec = e["cfg"]
        masked = e["name"].endswith("_masked")
        m, n, k = (int(v) for v in rng.integers(1, 401, size=3))
        opts = f"block-tile={bm},{bn} thread-tile={tm},{tn} tile-k={bk} promote={pr} vectorize={vec}"
        kk = k if masked else cm.padded((bm, bn, tm, tn, bk), m, n, k)[2]
        split = int(rng.choice([1, 1, 2, 3]))
        if split > 1 and -(-kk // bk) >= split:
            opts += f" split-k={split}"
        if (pr, vec) == (1, 1) or rng.random() < 0.5:
            opts += " xcd-swizzle=0"
        out.append((("mbr", "matmul")[rng.integers(2)], (m, n, k), (bm, bn, tm, tn, bk), opts, masked))
    return out


def _wave_draws(count=72, seed=2030):
    rng = np.random.default_rng(seed)
    space = cm.wave_split_space()
    out = []
    while len(out) < count:
        cfg = space[rng.integers(len(space))]
        m, n, k = (int(v) for v in rng.integers(1, 701, size=3))
        slabs = cm.padded(cfg, m, n, k)[2] // cfg[4]
        split = int(rng.choice([1, 1, 2, 3]))
        out.append((("mbr", "matmul")[rng.integers(2)], (m, n, k), tuple(cfg[:5]), split if split <= slabs else 1))
    return out


DRAWS = _draws() + _reference_draws()
VARIANT_DRAWS = _variant_draws()
WAVE_DRAWS = _wave_draws()
ELT_DRAWS = _elt_draws()
RESMLP_DRAWS = _resmlp_draws()


def _run(workload, m, n, k, options, ins, logical=None):
    pm, pn, pk = logical or (m, n, k)
    kern = _lib.Kernel(tc.gen_mlir(workload, pm, pn, pk), options, "t.mlir")
    out = np.empty((m, n), np.float32)
    kern.run([np.ascontiguousarray(v) for v in ins.values()], out,
             logical=None if logical is None or tuple(logical) == (m, n, k) else (m, n, k))
    return out


@pytest.mark.parametrize("workload,shape,cfg,split,masked", DRAWS,
                         ids=[f"{d[0]}-{'x'.join(map(str, d[1]))}-b{d[2][0]}x{d[2][1]}-t{d[2][2]}x{d[2][3]}"
                              f"-k{d[2][4]}-s{d[3]}{'-masked' if d[4] else ''}" for d in DRAWS])
def test_random_draw(workload, shape, cfg, split, masked):
    m, n, k = shape
    opts = STAGED.format(*cfg) + (f" split-k={split}" if split > 1 else "")
    ins = o.make_inputs(workload, m, n, k)
    print(f"draw {workload} {shape} {opts} masked={masked}", flush=True)
    padded = _run(workload, m, n, k, opts, ins, logical=cm.padded(cfg, m, n, k))
    ref, bound = o.fp64_reference(workload, ins)
    for out in ([padded, _run(workload, m, n, k, opts + " mask-edges=1", ins)] if masked else [padded]):
        assert not np.isnan(out).any()
        eob = o.e1_metrics(out, ref, bound)["max_err_over_bound"]
        assert eob <= 1.0, eob
        if workload == "mbr":
            assert o.mask_mismatches(out, o.preactivation64(ins), bound) == 0
        assert o.bitwise_diff(out, padded) == 0
    if workload == "mbr" and masked:  # the pad path takes single-launch programs only
        unfused = _run(workload, m, n, k, opts + " mask-edges=1 fuse-elementwise=0", ins)
        assert o.bitwise_diff(unfused, padded) == 0


@pytest.mark.parametrize("workload,shape,cfg,opts,masked", VARIANT_DRAWS,
                         ids=[f"{d[0]}-{'x'.join(map(str, d[1]))}-{d[3].replace(' ', '-')}{'-masked' if d[4] else ''}"
                              for d in VARIANT_DRAWS])
def test_random_variant(workload, shape, cfg, opts, masked):
    m, n, k = shape
    ins = o.make_inputs(workload, m, n, k)
    print(f"draw {workload} {shape} {opts} masked={masked}", flush=True)
    padded = _run(workload, m, n, k, opts, ins, logical=cm.padded(cfg, m, n, k))
    outs = [padded, _run(workload, m, n, k, opts + " mask-edges=1", ins)] if masked else [padded]
    ref, bound = o.fp64_reference(workload, ins)
    for out in outs:
        assert not np.isnan(out).any()
        assert o.e1_metrics(out, ref, bound)["max_err_over_bound"] <= 1.0
        if workload == "mbr":
            assert o.mask_mismatches(out, o.preactivation64(ins), bound) == 0
        assert o.bitwise_diff(out, padded) == 0


@pytest.mark.parametrize("workload,shape,cfg,split", WAVE_DRAWS,
                         ids=[f"{d[0]}-{'x'.join(map(str, d[1]))}-b{d[2][0]}x{d[2][1]}-t{d[2][2]}x{d[2][3]}"
                              f"-k{d[2][4]}-s{d[3]}" for d in WAVE_DRAWS])
def test_random_wave_split(workload, shape, cfg, split):
    m, n, k = shape
    opts = STAGED.format(*cfg) + " wave-split-k=1" + (f" split-k={split}" if split > 1 else "")
    ins = o.make_inputs(workload, m, n, k)
    print(f"draw {workload} {shape} {opts}", flush=True)
    out = _run(workload, m, n, k, opts, ins, logical=cm.padded(cfg, m, n, k))
    ref, bound = o.fp64_reference(workload, ins)
    assert not np.isnan(out).any()
    assert o.e1_metrics(out, ref, bound)["max_err_over_bound"] <= 1.0
    if workload == "mbr":
        assert o.mask_mismatches(out, o.preactivation64(ins), bound) == 0


@pytest.mark.parametrize("workload,shape,opts", ELT_DRAWS,
                         ids=[f"{d[0]}-{d[1][0]}x{d[1][1]}-{d[2].replace(' ', '-')}" for d in ELT_DRAWS])
def test_random_element_op(workload, shape, opts):
    m, n = shape
    print(f"draw {workload} {shape} {opts}", flush=True)
    d, launch = tg.compile_kernel(workload, m, n, None, opts, tag="test")
    res, out = tg.check(workload, m, n, None, d, launch)
    assert res["pass"], res
    assert o.bitwise_diff(out, o.elementwise(workload, o.make_inputs(workload, m, n, None))) == 0


@pytest.mark.parametrize("shape,cfg", RESMLP_DRAWS,
                         ids=[f"{'x'.join(map(str, d[0]))}-b{d[1][0]}x{d[1][1]}-t{d[1][2]}x{d[1][3]}-k{d[1][4]}"
                              for d in RESMLP_DRAWS])
def test_random_residual_block(shape, cfg):
    m, n, k = shape
    print(f"draw resmlp {shape} {cfg}", flush=True)
    ins = tc.make_inputs("resmlp", m, n, k)
    kern = _lib.Kernel(tc.gen_mlir("resmlp", m, n, k), STAGED.format(*cfg) + " mask-edges=1", "t.mlir")
    y = np.empty((m, n), np.float32)
    kern.run([np.ascontiguousarray(v) for v in ins.values()], y)
    assert tg._resmlp_check(ins, y)["pass"]
