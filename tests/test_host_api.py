"""Host-side API of the Python mirror (python/tforge_gpu.py, python/tforge_cpu.py,
python/provenance.py) on the CPU: programs, seeded inputs, padding, the FP64
bound check and its failure modes, artifacts, CSV schema."""

import json

import numpy as np
import pytest

from oracle import oracle as o
from tensorforge_amd import provenance
from tensorforge_amd import tforge_cpu as tc
from tensorforge_amd import tforge_gpu as tg


@pytest.mark.parametrize("workload", ["add", "relu", "bias_add", "matmul", "mbr"])
def test_make_inputs_match_oracle(workload):
    a = tc.make_inputs(workload, 33, 17, 9)
    b = o.make_inputs(workload, 33, 17, 9)
    assert list(a) == list(b)
    for k in a:
        assert a[k].dtype == np.float32 and np.array_equal(a[k], b[k])


def test_resmlp_inputs_distribution():
    ins = tc.make_inputs("resmlp", 512, 256, 1024)
    assert list(ins) == ["x", "w1", "b1", "w2", "b2"]
    assert abs(ins["x"].std() - 1.0) < 0.02
    assert abs(ins["w1"].std() - 1 / 16) < 0.002 and abs(ins["w2"].std() - 1 / 32) < 0.001
    assert abs(ins["b1"].std() - 0.02) < 0.003


def test_padded_shape():
    opts = "block-tile=128,64 thread-tile=8,4 tile-k=16 promote=1 vectorize=1"
    assert tg.padded_shape(777, 1111, 333, opts) == (896, 1152, 336)  # docs/stage8.md:107
    assert tg.padded_shape(777, 1111, 333, "block-tile=16,16 thread-tile=1,1") == (777, 1111, 333)


def test_peak():
    assert abs(tg.FP32_PEAK_TFLOPS - 157.3) < 0.05


def test_bound_check_passes_fma_closed_form_with_reference_value():
    ins = tc.make_inputs("mbr", 256, 256, 256)
    out = o.mbr_fma(ins["a"], ins["b"], ins["bias"])
    res = tg._bound_check("mbr", ins, out, 256)
    assert res["pass"] and f"{res['err_over_bound']:.3g}" == "0.0129"  # results/numerics/e1.csv:7
    assert res["mask_mismatches"] == 0


def test_bound_check_failure_modes():
    ins = tc.make_inputs("mbr", 64, 64, 64)
    good = o.mbr_fma(ins["a"], ins["b"], ins["bias"])
    bad = good.copy()
    bad[3, 5] = np.nextafter(bad[3, 5], np.float32(np.inf)) + 1e-3  # one element beyond the bound
    assert not tg._bound_check("mbr", ins, bad, 64)["pass"]
    nan = good.copy()
    nan[0, 0] = np.nan  # an unwritten (NaN-prefilled) output
    r = tg._bound_check("mbr", ins, nan, 64)
    assert not r["pass"] and r["nan_count"] == 1
    z = o.preactivation64(ins)
    i, j = np.unravel_index(np.argmax(z), z.shape)
    masked = good.copy()
    masked[i, j] = 0.0  # a clearly positive pre-activation reported as zero
    r = tg._bound_check("mbr", ins, masked, 64)
    assert not r["pass"] and r["mask_mismatches"] == 1


def test_resmlp_bound_accepts_f32_emulation_and_rejects_errors():
    m, n, k = 64, 32, 128
    ins = tc.make_inputs("resmlp", m, n, k)
    h = o.epilogue(o.matmul_fma(ins["x"], ins["w1"]), ins["b1"], relu=True)
    y = o.epilogue(o.matmul_fma(h, ins["w2"]), ins["b2"], relu=True, resid=ins["x"])
    r = tg._resmlp_check(ins, y)
    assert r["pass"], r
    y_nofma = o.epilogue(o.epilogue(o.matmul_nofma(o.epilogue(o.matmul_nofma(ins["x"], ins["w1"]), ins["b1"], relu=True),
                                                   ins["w2"]), ins["b2"], relu=True), resid=ins["x"])
    assert tg._resmlp_check(ins, y_nofma)["pass"]
    wrong = o.epilogue(o.matmul_fma(h, ins["w2"]), ins["b2"], relu=True)  # residual add dropped
    assert not tg._resmlp_check(ins, wrong)["pass"]


def test_compile_kernel_writes_artifacts(tmp_path, monkeypatch):
    monkeypatch.setattr(tg, "ART", tmp_path)
    d, launch = tg.compile_kernel("mbr", 777, 1111, 333,
                                  "block-tile=128,64 thread-tile=8,4 tile-k=16 promote=1 vectorize=1", tag="t")
    assert (d / "input.mlir").read_text() == tc.gen_mlir("mbr", 896, 1152, 336)
    assert tg.parse_launch(d) == launch == json.loads((d / "launch.json").read_text())
    assert launch["grid"] == [18, 7, 1] and launch["padded"] == [896, 1152, 336]
    res = tg.ptxas_resources(d)
    assert res["regs"] > 0 and res["spill_stores"] == 0 and res["smem"] > 0


def test_compile_kernel_error_is_runtime_error(tmp_path, monkeypatch):
    monkeypatch.setattr(tg, "ART", tmp_path)
    with pytest.raises(RuntimeError, match="block-tile and thread-tile need 2 values"):
        tg.compile_kernel("mbr", 64, 64, 64, "block-tile=64")


def test_provenance_fields_are_the_reference_schema(tmp_path):
    assert provenance.FIELDS == [
        "commit", "mlir_llvm_version", "cuda_version", "device", "job_id", "date",
        "workload", "shape", "dtype", "pipeline", "params", "threads", "warmup", "reps",
        "median_ms", "min_ms", "std_ms", "metric", "metric_value", "sm_clock_median_mhz",
        "clock_adjusted_metric", "alloc_bytes_per_call", "correctness", "notes"]
    t = provenance.ResultsTable(tmp_path / "x.csv", device="dev")
    t.add(workload="mbr", shape="1x2x3")
    t.add(workload="relu", device="other")
    with pytest.raises(KeyError):
        t.add(bogus=1)
    with pytest.raises(KeyError):
        provenance.ResultsTable(tmp_path / "y.csv", bogus=1)
    t.close()
    import csv
    rows = list(csv.DictReader(open(tmp_path / "x.csv")))
    assert [r["workload"] for r in rows] == ["mbr", "relu"] and [r["device"] for r in rows] == ["dev", "other"]
    assert rows[0]["commit"] == provenance.commit_label() and rows[0]["shape"] == "1x2x3"
    provenance.ResultsTable(tmp_path / "x.csv").add(workload="add")  # appends, no second header
    assert len(list(csv.DictReader(open(tmp_path / "x.csv")))) == 3


def test_build_info_names_the_commit(tmp_path, monkeypatch):
    """The build records HEAD (and whether the tree differed from it) next to
    the library; rows read it there, so a copy without .git still names it."""
    info = provenance.write_build_info(tmp_path / "BUILD_INFO.json")
    assert len(info["commit"]) == 40 and info["commit"] == provenance.git_head()
    monkeypatch.setattr(provenance, "BUILD_INFO", tmp_path / "BUILD_INFO.json")
    monkeypatch.setattr(provenance, "ROOT", tmp_path)  # no .git here: only the file can answer
    assert provenance.commit_label().startswith(info["commit"][:12])
    assert provenance.commit_label().endswith("-dirty") == bool(info["dirty"])
    assert provenance.device_label({"name": "AMD Instinct MI355X", "arch": "gfx950:sramecc+:xnack-",
                                    "compute_units": 256}) == "AMD Instinct MI355X [gfx950:sramecc+:xnack-, 256 CUs]"


def test_flops_convention():
    assert tc.flops_or_bytes("mbr", 2048, 2048, 2048) == ("GFLOP/s", 2.0 * 2048 ** 3)
    assert tc.flops_or_bytes("resmlp", 4096, 2048, 8192)[1] == 4.0 * 4096 * 2048 * 8192


def test_host_arrays_and_pointer_counts_are_validated():
    """tf_run copies whole buffers from and to host pointers and tf_launch
    reads one device pointer per buffer, so the Python mirror checks counts,
    dtype, layout and element counts before calling (no GPU needed: every
    case raises first)."""
    import numpy as np
    import pytest
    from tensorforge_amd import _lib, tforge_cpu as tc
    k = _lib.Kernel(tc.gen_mlir("mbr", 64, 32, 16), "")
    a, b, bias, c = (np.zeros(s, np.float32) for s in ((64, 16), (16, 32), (32,), (64, 32)))
    with pytest.raises(ValueError, match="takes 3 input arrays, got 1"):
        k.run([a], c)
    with pytest.raises(TypeError, match="input 2 must be a C-contiguous float32"):
        k.run([a, b, bias.astype(np.float64)], c)
    with pytest.raises(TypeError, match="input 1 must be a C-contiguous float32"):
        k.run([a, np.zeros((32, 16), np.float32).T, bias], c)
    with pytest.raises(ValueError, match="input 2 has 31 elements, the program needs 32"):
        k.run([a, b, bias[:31]], c)
    with pytest.raises(ValueError, match="output has 1984 elements, the program needs 2048"):
        k.run([a, b, bias], np.zeros((64, 31), np.float32))
    with pytest.raises(ValueError, match="takes 4 device buffers"):
        k.launch([1, 2, 3])
    # logical (unpadded) sizes of a padded single-matmul program: A m x k, B k x n, bias n, C m x n
    kp = _lib.Kernel(tc.gen_mlir("mbr", 128, 64, 32), "block-tile=128,64 thread-tile=8,4 tile-k=16 promote=1")
    with pytest.raises(ValueError, match="input 0 has 1600 elements, the program needs 1500"):
        kp.run([np.zeros((100, 16), np.float32), np.zeros((15, 50), np.float32), np.zeros(50, np.float32)],
               np.zeros((100, 50), np.float32), logical=(100, 50, 15))


def _prog(args, body, ret):
    """A tforge program from (name, dims) arguments, op lines and the result type."""
    t = lambda *d: "tensor<" + "x".join(str(x) for x in d) + "xf32>"
    head = ", ".join(f"%{n}: {t(*d)}" for n, d in args)
    return f"func.func @entry({head}) -> {t(*ret)} {{\n" + "".join(f"  {l}\n" for l in body) + \
        f"  return %{len(body) - 1} : {t(*ret)}\n}}\n"


STAGED_16 = "block-tile=64,64 thread-tile=4,4 tile-k=16 promote=1 vectorize=1"


def test_host_shapes_follow_roles_not_positions():
    """The library reports each buffer's host shape from its role in the chain,
    and the Python mirror checks arrays against that report: an add residual is
    m x n (not a bias), and reordered arguments keep their own roles."""
    from tensorforge_amd import _lib
    t = "tensor<64x32xf32>, tensor<32x64xf32> -> tensor<64x64xf32>"
    resid = _prog([("a", (64, 32)), ("b", (32, 64)), ("r", (64, 64))],
                  [f"%0 = tforge.matmul %a, %b : {t}",
                   "%1 = tforge.add %0, %r : tensor<64x64xf32>, tensor<64x64xf32> -> tensor<64x64xf32>"], (64, 64))
    k = _lib.Kernel(resid, STAGED_16)
    assert k.host_shapes() == [(64, 32), (32, 64), (64, 64), (64, 64)]
    assert k.host_shapes((50, 50, 20)) == [(50, 20), (20, 50), (50, 50), (50, 50)]
    with pytest.raises(ValueError, match="input 2 has 50 elements, the program needs 2500"):
        k.run([np.zeros((50, 20), np.float32), np.zeros((20, 50), np.float32), np.zeros(50, np.float32)],
              np.zeros((50, 50), np.float32), logical=(50, 50, 20))
    swapped = _prog([("b", (32, 64)), ("a", (64, 32))], [f"%0 = tforge.matmul %a, %b : {t}"], (64, 64))
    k = _lib.Kernel(swapped, STAGED_16)
    assert k.host_shapes((50, 40, 20)) == [(20, 40), (50, 20), (50, 40)]
    with pytest.raises(ValueError, match="input 0 has 1000 elements, the program needs 800"):
        k.run([np.zeros((50, 20), np.float32), np.zeros((20, 40), np.float32)], np.zeros((50, 40), np.float32),
              logical=(50, 40, 20))


def test_buffer_in_two_roles_refuses_inconsistent_logical_sizes():
    """A reused as the residual (K == N when compiled): logical sizes with
    k != n would need two different pads of one buffer, so the library refuses
    them; with k == n the two roles agree and the sizes are accepted."""
    from tensorforge_amd import _lib
    t = "tensor<64x64xf32>"
    prog = _prog([("a", (64, 64)), ("b", (64, 64))],
                 [f"%0 = tforge.matmul %a, %b : {t}, {t} -> {t}", f"%1 = tforge.add %0, %a : {t}, {t} -> {t}"],
                 (64, 64))
    k = _lib.Kernel(prog, STAGED_16)
    with pytest.raises(RuntimeError, match=r"buffer 0 \(%a\) is both the matmul lhs and the add operand"):
        k.host_shapes((50, 50, 20))
    assert k.host_shapes((50, 40, 40)) == [(50, 40), (40, 40), (50, 40)]
    with pytest.raises(RuntimeError, match="single-matmul programs only"):
        _lib.Kernel(tc.gen_mlir("resmlp", 64, 64, 64), STAGED_16).host_shapes((60, 60, 60))
    with pytest.raises(RuntimeError, match="padded sizes must be >= M, N, K"):
        k.host_shapes((65, 64, 64))


def test_null_device_pointer_is_refused_before_any_launch():
    """A null buffer would fault the GPU; the library refuses it before it
    touches the device (so this runs without one), and so does the mirror."""
    import ctypes
    from tensorforge_amd import _lib
    k = _lib.Kernel(tc.gen_mlir("mbr", 64, 64, 64), STAGED_16)
    with pytest.raises(ValueError, match=r"device buffer 2 \(%bias\) is a null pointer"):
        k.launch([16, 32, 0, 48])
    L = _lib.lib()
    arr = (ctypes.c_void_p * 4)(16, 32, None, 48)
    assert L.tf_launch(k.h, arr, None) == -4
    assert b"buffer 2 (%bias) is a null pointer" in L.tf_last_error()
    ins = (ctypes.POINTER(ctypes.c_float) * 3)()
    out = np.zeros((64, 64), np.float32)
    assert L.tf_run(k.h, 0, None, ins, out.ctypes.data_as(ctypes.POINTER(ctypes.c_float))) == -4
    assert b"host input 0 is a null pointer" in L.tf_last_error()


def test_persistent_option_is_gone():
    """The persistent (streamed) option was measured slower than the staged
    kernel everywhere and removed; the option parser now refuses it like any
    unknown option."""
    from tensorforge_amd import _lib
    with pytest.raises(RuntimeError, match="no such option persistent"):
        _lib.Kernel(tc.gen_mlir("mbr", 1024, 1024, 256), STAGED_16 + " persistent=1")


@pytest.mark.parametrize("shape,options,message", [
    ((1000, 1024, 256), "block-tile=32,32 thread-tile=1,1 tile-k=32 promote=1 vectorize=1 mask-edges=1 "
     "wave-split-k=1", "wave-split-k needs M, N and K to be multiples"),
    ((1024, 1024, 256), "block-tile=16,16 thread-tile=1,1 wave-split-k=1", "wave-split-k needs tile-k"),
    ((1024, 1024, 256), "block-tile=32,32 thread-tile=1,1 tile-k=32 promote=1 vectorize=0 wave-split-k=1",
     "wave-split-k needs promote=1 vectorize=1"),
    ((1024, 1024, 256), "block-tile=32,32 thread-tile=1,1 tile-k=32 promote=0 vectorize=1 wave-split-k=1",
     "wave-split-k needs promote=1 vectorize=1"),
    ((1024, 1024, 256), "block-tile=128,128 thread-tile=8,4 tile-k=32 promote=1 vectorize=1 wave-split-k=1",
     "wave-split-k has no instantiation of this configuration"),
    ((64, 65536, 16384), "block-tile=32,32 thread-tile=1,1 tile-k=32 promote=1 vectorize=1 wave-split-k=1",
     "wave-split-k supports"),
])
def test_wave_split_option_refusals(shape, options, message):
    """The wave-split option's limits are compile-time errors with the reason."""
    from tensorforge_amd import _lib
    with pytest.raises(RuntimeError, match=message):
        _lib.Kernel(tc.gen_mlir("mbr", *shape), options)


def test_wave_split_launch_geometry():
    """The reference's geometry: grid (N/BN, M/BM[, split-k]), block (BN/TN,
    BM/TM); the block's waves are the K ranges."""
    from tensorforge_amd import _lib
    opts = "block-tile=32,32 thread-tile=1,1 tile-k=32 promote=1 vectorize=1 wave-split-k=1"
    one = _lib.Kernel(tc.gen_mlir("mbr", 64, 4096, 4096), opts).launches()[0]
    assert one["family"] == "wavek" and one["kernel"] == "tf_wavek_b32x32_t1x1_k32"
    assert one["grid"] == [128, 2, 1] and one["block"] == [32, 32, 1]
    two = _lib.Kernel(tc.gen_mlir("mbr", 64, 4096, 4096), opts + " split-k=2").launches()[0]
    assert two["grid"] == [128, 2, 2]


def test_wave_split_configurations_in_the_cost_model():
    """Every wave-split registry entry is in the cost model's space with the
    same name, and its options compile to it."""
    from tensorforge_amd import _lib
    from tensorforge_amd import costmodel as cm
    names = {e["name"] for e in _lib.registry() if e["family"] == "wavek"}
    space = cm.wave_split_space()
    assert {cm.kernel_name(c) for c in space} == names
    for cfg in space[::7]:
        launch = _lib.Kernel(tc.gen_mlir("mbr", 2 * cfg[0], 2 * cfg[1], 4 * cfg[4]), cm.options(cfg)).launches()[0]
        assert launch["kernel"] == cm.kernel_name(cfg)


def test_reference_stage9_space_compiles():
    """Every configuration of the reference's Stage 9 grid (105:
    python/costmodel.py:49-60) compiles.  The 75 whose (8 TM) x (8 TN) wave
    tile tiles the block run their own instantiation with the reference's
    block (BN/TN, BM/TM); the other 30 run the stand-in wave layout and report
    the block actually launched: one 64-lane wave over the whole block for
    the 32-thread configurations, else the same thread count."""
    from tensorforge_amd import _lib
    from tensorforge_amd import costmodel as cm
    ref = cm.reference_space()
    assert len(ref) == 105
    mapped = 0
    for cfg in ref:
        bm, bn, tm, tn, bk = cfg
        for masked in (False, True):
            if masked and cfg in ((32, 128, 8, 8, 32), (128, 32, 8, 8, 32)):
                continue  # a 64-thread block staging 20 vectors per thread: no masked twin
            shape = (2 * bm - 3, 2 * bn - 5, 4 * bk - 7) if masked else (2 * bm, 2 * bn, 4 * bk)
            opts = cm.options(cfg) + (" mask-edges=1" if masked else "")
            launch = _lib.Kernel(tc.gen_mlir("mbr", *shape), opts).launches()[0]
            ktm, ktn = cm.kernel_tile(cfg)
            assert launch["kernel"] == cm.kernel_name(cfg) + ("_masked" if masked else ""), (cfg, launch["kernel"])
            assert launch["block"] == [bn // ktn, bm // ktm, 1]
            assert launch["grid"][:2] == [-(-shape[1] // bn), -(-shape[0] // bm)]
            threads = (bm // tm) * (bn // tn)
            if (ktm, ktn) != (tm, tn):
                mapped += not masked
                assert (bn // ktn) * (bm // ktm) == max(threads, 64)
                assert 8 * tm > bm or 8 * tn > bn or threads < 64
    assert mapped == 30
    with pytest.raises(RuntimeError, match="no masked twin|stage 20 vectors per slab"):
        _lib.Kernel(tc.gen_mlir("mbr", 61, 251, 121), cm.options((32, 128, 8, 8, 32)) + " mask-edges=1")
