"""Pins the CPU oracle to known answers the reference itself holds.

results/numerics/e1.csv gives, per workload and shape, the error statistics of
the reference's two arithmetic orders (no-FMA scalar pipeline, sequential-FMA
GPU kernels) against FP64 and the number of outputs on which they differ
bitwise.  Reproducing every printed digit pins, together, the seeded input
generator, the FP64 reference and bound formula, and both closed forms.
results/gpu/stage8.csv / stage7.csv give err/bound of the FMA kernels at more
shapes.  The planted-mistake tests show that plausible slips in the oracle
(wrong order, dropped bias, transposed operand, wrong gamma) fail these pins.
"""

import json
import pathlib

import numpy as np
import pytest

from oracle import oracle as o

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"
E1 = json.loads((GOLDEN / "e1_known_answers.json").read_text())
STAGE8 = json.loads((GOLDEN / "stage8_err_bound.json").read_text())
CPU = json.loads((GOLDEN / "cpu_err_bound.json").read_text())

_cache = {}


def forms(workload, m, n, k):
    """(inputs, fma output, no-fma output, ref, bound) at a shape."""
    key = (workload, m, n, k)
    if key not in _cache:
        ins = o.make_inputs(workload, m, n, k)
        fma = o.matmul_fma(ins["a"], ins["b"])
        nofma = o.matmul_nofma(ins["a"], ins["b"])
        if workload == "mbr":
            fma = o.epilogue(fma, ins["bias"], relu=True)
            nofma = o.epilogue(nofma, ins["bias"], relu=True)
        ref, bound = o.fp64_reference(workload, ins)
        _cache[key] = (ins, fma, nofma, ref, bound)
    return _cache[key]


def sig(x, digits=4):
    return float(f"{float(x):.{digits}g}")


def shape_of(key):
    wl, shape = key.split("/")
    return (wl,) + tuple(int(v) for v in shape.split("x"))


@pytest.mark.parametrize("key", sorted(E1))
def test_e1_known_answers(key):
    wl, m, n, k = shape_of(key)
    ins, fma, nofma, ref, bound = forms(wl, m, n, k)
    for form, out in (("fma", fma), ("nofma", nofma)):
        want = E1[key][form]
        got = o.e1_metrics(out, ref, bound)
        for stat in ("max_abs_err", "rms_err", "max_err_over_bound"):
            digits = len(want[stat].replace(".", "").replace("-", "").split("e")[0].lstrip("0"))
            assert sig(got[stat], digits) == float(want[stat]), (key, form, stat, got[stat], want[stat])
    assert o.bitwise_diff(fma, nofma) == E1[key]["fma"]["bitwise_diff_vs_nofma"]


@pytest.mark.parametrize("key", sorted(k for k in STAGE8 if max(shape_of(k)[1:]) <= 2048))
def test_stage8_err_over_bound(key):
    wl, m, n, k = shape_of(key)
    ins = o.make_inputs(wl, m, n, k)
    out = o.matmul_fma(ins["a"], ins["b"])
    if wl == "mbr":
        out = o.epilogue(out, ins["bias"], relu=True)
    ref, bound = o.fp64_reference(wl, ins)
    want = STAGE8[key]["err_over_bound"]
    digits = len(want.replace(".", "").split("e")[0].lstrip("0"))
    assert sig(o.e1_metrics(out, ref, bound)["max_err_over_bound"], digits) == float(want)


@pytest.mark.slow
@pytest.mark.parametrize("key", sorted(k for k in STAGE8 if max(shape_of(k)[1:]) > 2048))
def test_stage8_err_over_bound_4096(key):
    """The 4096^3 rows of the same column (results/gpu/stage8.csv): the FMA
    closed form on all host cores (its bits do not depend on the thread
    count), FP64 reference from NumPy."""
    test_stage8_err_over_bound(key)


@pytest.mark.parametrize("key", sorted(CPU))
def test_cpu_pipeline_err_over_bound(key):
    """results/cpu/stage4.csv, stage6_best.csv: the reference's default scalar
    CPU pipeline (m-n-k loops, no FMA) and its reg-tile=6,16,4 AVX2 FMA kernel
    at ten shapes, ragged ones included; the oracle's scalar loop and its
    6x16x4 port give the same err/bound to the printed digits."""
    wl, m, n, k = shape_of(key)
    ins = o.make_inputs(wl, m, n, k)
    ref, bound = o.fp64_reference(wl, ins)
    mbr = wl == "mbr"
    outs = {"scalar": o.matmul_scalar_mnk(ins["a"], ins["b"]),
            "vec6x16": o.mbr_vec6x16(ins["a"], ins["b"], ins["bias"] if mbr else None, relu=mbr)}
    if mbr:
        outs["scalar"] = o.epilogue(outs["scalar"], ins["bias"], relu=True)
    for form, want in CPU[key].items():
        val = want["err_over_bound"]
        digits = len(val.replace(".", "").split("e")[0].lstrip("0"))
        got = o.e1_metrics(outs[form], ref, bound)["max_err_over_bound"]
        assert sig(got, digits) == float(val), (key, form, got, val)


@pytest.mark.parametrize("shape", [(256, 256, 256), (127, 129, 65), (777, 1111, 333), (6, 16, 4), (5, 15, 3)])
def test_vec6x16_port_is_bitwise_fma(shape):
    m, n, k = shape
    ins = o.make_inputs("mbr", m, n, k)
    want = o.mbr_fma(ins["a"], ins["b"], ins["bias"])
    got = o.mbr_vec6x16(ins["a"], ins["b"], ins["bias"])
    assert o.bitwise_diff(got, want) == 0
    got_mm = o.mbr_vec6x16(ins["a"], ins["b"], None, relu=False)
    assert o.bitwise_diff(got_mm, o.matmul_fma(ins["a"], ins["b"])) == 0


def test_thread_count_does_not_change_bits():
    ins = o.make_inputs("matmul", 200, 300, 100)
    assert o.bitwise_diff(o.matmul_fma(ins["a"], ins["b"], threads=1),
                          o.matmul_fma(ins["a"], ins["b"], threads=7)) == 0


def test_relu_is_ieee_maximum():
    x = np.array([[np.nan, -0.0, 0.0, -1.5, 2.5, -np.inf, np.inf]], np.float32)
    y = o.epilogue(x, relu=True)
    assert np.isnan(y[0, 0])
    assert y[0, 1] == 0 and not np.signbit(y[0, 1])  # -0 -> +0
    assert list(y[0, 2:]) == [0.0, 0.0, 2.5, 0.0, np.inf]


def test_small_brute_force():
    """Tiny case against an independent Python loop (exact products, one
    rounding per step emulated in float32)."""
    ins = o.make_inputs("mbr", 3, 5, 7)
    a, b, bias = ins["a"], ins["b"], ins["bias"]
    out = np.zeros((3, 5), np.float32)
    for i in range(3):
        for j in range(5):
            acc = np.float32(0)
            for kk in range(7):
                acc = np.float32(acc + np.float32(a[i, kk] * b[kk, j]))
            out[i, j] = max(np.float32(acc + bias[j]), np.float32(0))
    assert o.bitwise_diff(o.epilogue(o.matmul_nofma(a, b), bias, relu=True), out) == 0


def test_scalar_mnk_loop_is_the_nofma_form():
    """The timed scalar baseline (default pipeline loop order) is bitwise the
    no-FMA closed form that the E1 cpu-scalar rows pin, on a ragged shape."""
    ins = o.make_inputs("matmul", 37, 53, 129)
    assert o.bitwise_diff(o.matmul_scalar_mnk(ins["a"], ins["b"]), o.matmul_nofma(ins["a"], ins["b"])) == 0


# ---- planted mistakes: each must break a pin -------------------------------

def test_planted_wrong_order_fails_fma_pin():
    ins, fma, nofma, ref, bound = forms("mbr", 256, 256, 256)
    got = o.e1_metrics(nofma, ref, bound)
    assert sig(got["max_err_over_bound"], 3) != float(E1["mbr/256x256x256"]["fma"]["max_err_over_bound"])


def test_planted_dropped_bias_fails():
    ins, fma, nofma, ref, bound = forms("mbr", 256, 256, 256)
    wrong = o.epilogue(o.matmul_fma(ins["a"], ins["b"]), None, relu=True)
    assert o.e1_metrics(wrong, ref, bound)["max_err_over_bound"] > 1.0


def test_planted_transposed_operand_fails():
    ins = o.make_inputs("matmul", 256, 256, 256)
    ref, bound = o.fp64_reference("matmul", ins)
    wrong = o.matmul_fma(ins["a"], np.ascontiguousarray(ins["b"].T))
    assert o.e1_metrics(wrong, ref, bound)["max_err_over_bound"] > 1.0


def test_planted_wrong_gamma_fails_pin():
    ins, fma, nofma, ref, bound = forms("mbr", 256, 256, 256)
    # gamma_K instead of gamma_{K+1} for mbr changes the 4th digit of the
    # no-FMA row's err/bound (0.01381, printed to 4 digits)
    k = 256
    g_right = (k + 1) * o.F32_EPS / (1 - (k + 1) * o.F32_EPS)
    g_wrong = k * o.F32_EPS / (1 - k * o.F32_EPS)
    wrong_bound = (bound - o.FLT_MIN) / g_right * g_wrong + o.FLT_MIN
    got = o.e1_metrics(nofma, ref, wrong_bound)["max_err_over_bound"]
    assert sig(got, 4) != float(E1["mbr/256x256x256"]["nofma"]["max_err_over_bound"])


def test_planted_wrong_seed_fails_pin():
    ins = o.make_inputs("mbr", 256, 256, 256, seed=1235)
    out = o.mbr_fma(ins["a"], ins["b"], ins["bias"])
    ref, bound = o.fp64_reference("mbr", ins)
    assert sig(o.e1_metrics(out, ref, bound)["rms_err"]) != float(E1["mbr/256x256x256"]["fma"]["rms_err"])
