"""Pins the oracle functions that the reference's CSVs do not reach: the ReLU
mask gate every GPU parity test applies (mask_mismatches), the FP64
pre-activation it is given (preactivation64), and the element ops on their own
(add, relu, bias_add).  Each pin is chosen so that a plausible slip fails it:
a gate that always passes, a >= for the strict bound test, a dropped or
transposed term, a ReLU that drops NaN or keeps -0.0, a bias added along rows.
"""

import numpy as np
import pytest

from oracle import oracle as o


def _mbr(m=48, n=40, k=64, seed=1234):
    ins = o.make_inputs("mbr", m, n, k, seed)
    out = o.mbr_fma(ins["a"], ins["b"], ins["bias"])
    ref, bound = o.fp64_reference("mbr", ins)
    return ins, out, o.preactivation64(ins), bound


# ---- mask_mismatches -------------------------------------------------------

def test_mask_gate_accepts_both_closed_forms():
    ins, out, z, bound = _mbr()
    assert o.mask_mismatches(out, z, bound) == 0
    nofma = o.epilogue(o.matmul_nofma(ins["a"], ins["b"]), ins["bias"], relu=True)
    assert o.mask_mismatches(nofma, z, bound) == 0


def test_mask_gate_counts_a_decided_positive_reported_as_zero():
    _, out, z, bound = _mbr()
    pos = np.argwhere(z > bound)
    assert len(pos) > 100
    i, j = pos[len(pos) // 2]
    bad = out.copy()
    bad[i, j] = 0.0
    assert o.mask_mismatches(bad, z, bound) == 1


def test_mask_gate_counts_a_decided_negative_reported_positive():
    _, out, z, bound = _mbr()
    neg = np.argwhere(z < -bound)
    assert len(neg) > 100
    i, j = neg[len(neg) // 3]
    bad = out.copy()
    bad[i, j] = np.float32(0.25)
    assert o.mask_mismatches(bad, z, bound) == 1
    bad[i, j] = np.float32(-0.0)  # -0.0 == 0: still a zero, so no mismatch
    assert o.mask_mismatches(bad, z, bound) == 0


def test_mask_gate_ignores_undecided_elements_and_is_strict_at_the_bound():
    """Every element below has the 'wrong' mask; only |z| > bound counts, so
    |z| == bound (exactly representable here) and |z| < bound count nothing.
    A >= slip counts 4, a gate that always passes counts 0."""
    bound = np.full(6, 2.0 ** -10)
    z = np.array([2.0 ** -10, -2.0 ** -10, 2.0 ** -9, -2.0 ** -9, 2.0 ** -11, -2.0 ** -11])
    out = np.array([0.0, 1.0, 0.0, 1.0, 0.0, 1.0], np.float32)
    assert o.mask_mismatches(out, z, bound) == 2
    right = np.array([1.0, 0.0, 1.0, 0.0, 1.0, 0.0], np.float32)
    assert o.mask_mismatches(right, z, bound) == 0


def test_mask_gate_on_an_in_bound_perturbation_counts_nothing():
    """Outputs whose pre-activation lies within the bound may round either way:
    flipping every such element's mask changes no count."""
    ins, out, z, bound = _mbr()
    bound = bound * 4096.0  # widen so that a real sample of undecided elements exists
    undecided = np.abs(z) <= bound
    assert undecided.sum() > 5
    bad = out.copy()
    bad[undecided] = np.where(bad[undecided] == 0, np.float32(1e-6), np.float32(0.0))
    assert o.mask_mismatches(bad, z, bound) == 0
    decided_pos = np.argwhere(z > bound)[0]
    bad[tuple(decided_pos)] = 0.0
    assert o.mask_mismatches(bad, z, bound) == 1


# ---- preactivation64 -------------------------------------------------------

def test_preactivation_is_the_fp64_reference_before_relu():
    ins, _, z, _ = _mbr(64, 96, 80)
    ref, _ = o.fp64_reference("mbr", ins)
    assert np.array_equal(np.maximum(z, 0.0).view(np.uint64), ref.view(np.uint64))


def test_preactivation_equals_exact_integer_arithmetic():
    """Small multiples of 1/8 are exact in fp64, so z must equal the integer
    result computed with Python ints; a transposed B or a dropped (or
    row-wise) bias would not."""
    rng = np.random.default_rng(5)
    m, n, k = 5, 7, 9
    ai, bi, ci = (rng.integers(-8, 9, size=s) for s in ((m, k), (k, n), (n,)))
    ins = {"a": (ai / 8).astype(np.float32), "b": (bi / 8).astype(np.float32), "bias": (ci / 8).astype(np.float32)}
    z = o.preactivation64(ins)
    for i in range(m):
        for j in range(n):
            exact = sum(int(ai[i, t]) * int(bi[t, j]) for t in range(k)) + 8 * int(ci[j])  # 64 z
            assert z[i, j] * 64 == exact, (i, j)


# ---- add / relu / bias_add --------------------------------------------------

SPECIALS = np.array([np.nan, -0.0, 0.0, np.inf, -np.inf, 1e-45, -1e-45, 1.2e-38, -1.2e-38,
                     3.0e38, -3.0e38, 1.0, -1.0, 0.5, -2.5], np.float32)


def _pairs():
    x = np.repeat(SPECIALS, SPECIALS.size)
    y = np.tile(SPECIALS, SPECIALS.size)
    return x, y


def _bits_equal(got, want):
    nan = np.isnan(want)
    return bool((np.isnan(got) == nan).all() and np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32)))


def test_add_is_ieee_f32_add_on_special_pairs():
    x, y = _pairs()
    with np.errstate(invalid="ignore", over="ignore"):
        want = np.add(x, y, dtype=np.float32)
    got = o.add(x, y)
    assert _bits_equal(got, want)
    assert np.isinf(o.add(np.float32([3.0e38]), np.float32([3.0e38])))[0]     # overflow rounds to inf
    assert np.isnan(o.add(np.float32([np.inf]), np.float32([-np.inf])))[0]    # inf - inf
    r = o.add(np.float32([-0.0, -0.0]), np.float32([-0.0, 0.0]))
    assert np.signbit(r[0]) and not np.signbit(r[1])                           # -0 + -0 = -0, -0 + 0 = +0


def test_relu_is_maximum_with_positive_zero():
    got = o.relu(SPECIALS)
    assert np.isnan(got[0])
    rest = SPECIALS[1:]
    want = np.where(rest > 0, rest, np.float32(0.0)).astype(np.float32)
    assert np.array_equal(got[1:].view(np.uint32), want.view(np.uint32))
    assert not np.signbit(got[1:]).any()                       # -0.0, -denormal, -inf -> +0.0
    assert got[5] == SPECIALS[5] and got[7] == SPECIALS[7]     # positive denormal and normal kept
    # planted slips, each caught by the checks above: x > 0 ? x : 0 drops the
    # NaN, x >= 0 ? x : 0 keeps -0.0
    slip_nan = np.where(SPECIALS > 0, SPECIALS, np.float32(0)).astype(np.float32)
    slip_zero = np.where(SPECIALS >= 0, SPECIALS, np.float32(0)).astype(np.float32)
    assert not np.isnan(slip_nan[0]) and np.signbit(slip_zero[1])


def test_bias_add_runs_along_the_last_dimension():
    rng = np.random.default_rng(3)
    m, n = 7, 11
    x = rng.choice(SPECIALS, size=(m, n)).astype(np.float32)
    bias = rng.choice(SPECIALS, size=n).astype(np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        want = (x + bias[None, :]).astype(np.float32)
    got = o.bias_add(x, bias)
    assert _bits_equal(got, want)
    ramp = o.bias_add(np.zeros((3, 4), np.float32), np.arange(4, dtype=np.float32))
    assert (ramp == np.arange(4, dtype=np.float32)[None, :]).all()   # a row-wise bias would give a column ramp


@pytest.mark.parametrize("workload", ["add", "relu", "bias_add"])
def test_elementwise_dispatch(workload):
    ins = o.make_inputs(workload, 9, 13, None)
    want = {"add": lambda: ins["a"] + ins["b"], "relu": lambda: np.where(ins["a"] > 0, ins["a"], np.float32(0)),
            "bias_add": lambda: ins["a"] + ins["bias"]}[workload]().astype(np.float32)
    assert np.array_equal(o.elementwise(workload, ins).view(np.uint32), want.view(np.uint32))
