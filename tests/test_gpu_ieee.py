"""IEEE special values through every kernel family.

The reference's ops are IEEE-754 (docs/dialect.md:19-30; lib/Conversion/
TForgeToLinalg.cpp:31-35, 106): the product starts from +0.0, relu is
maximum(x, +0.0), so a NaN propagates and -0.0 / -inf map to +0.0.  What
follows from that does not depend on the summation order, so the direct
FMA kernel, the MFMA kernels (32x32 and 16x16 blocks, bias staged in LDS),
masked edge tiles, split-K and the wave-split kernel must all give exactly:

  * a NaN in row r of A makes row r of the output NaN;
  * +inf in row k1 of B makes column c of the product +inf or -inf (the sign
    of A[m, k1]); relu maps the -inf to +0.0 (positive zero);
  * a bias of -inf gives +0.0 after relu, a bias of +inf gives +inf;
  * a row of A that is -0.0 except one element 0.5 at k1 yields exactly
    0.5 * B[k1, n] (adding signed zeros to a nonzero value is exact);

and every other output keeps the usual bar (the FP64 bound, exact ReLU masks).
The element ops are compared with NumPy float32 results bit for bit, with NaN
compared as NaN.
"""

import numpy as np
import pytest

from oracle import oracle as o
from tensorforge_amd import _lib
from tensorforge_amd import tforge_cpu as tc

pytestmark = pytest.mark.gpu

STAGED = "block-tile={},{} thread-tile={},{} tile-k={} promote=1 vectorize=1"
R_NAN, R_ZERO, C_PINF, C_NINF, C_BPINF = 3, 11, 5, 7, 9


def _run(workload, m, n, k, options, arrays):
    kern = _lib.Kernel(tc.gen_mlir(workload, m, n, k), options, "t.mlir")
    out = np.full((m, n), 12345.0, np.float32)
    kern.run([np.ascontiguousarray(a) for a in arrays], out)
    return out


@pytest.mark.parametrize("workload", ["mbr", "matmul"])
@pytest.mark.parametrize("shape,options", [
    ((200, 140, 72), "block-tile=16,16 thread-tile=1,1"),                 # direct FMA chain
    ((256, 256, 128), STAGED.format(128, 128, 8, 4, 32)),                 # 32x32 blocks, bias in LDS
    ((256, 256, 128), STAGED.format(64, 64, 4, 4, 16)),                   # one 32x32 block per wave
    ((256, 256, 128), STAGED.format(64, 64, 2, 2, 64)),                   # 16x16 blocks
    ((200, 140, 72), STAGED.format(64, 64, 4, 4, 32) + " mask-edges=1"),  # edge tiles, K tail
    ((256, 256, 128), STAGED.format(64, 128, 4, 4, 32) + " split-k=4"),   # partial sums + reduction
    ((256, 256, 128), STAGED.format(32, 32, 1, 1, 32) + " wave-split-k=1"),  # waves split K, sum in LDS
    ((256, 256, 128), STAGED.format(16, 64, 1, 1, 16) + " wave-split-k=1"),  # 16x16 blocks, B staged
    ((256, 256, 128), STAGED.format(32, 32, 2, 1, 16) + " wave-split-k=1 split-k=2"),
])
def test_special_values_through_gemm(workload, shape, options):
    m, n, k = shape
    ins = o.make_inputs(workload, m, n, k)
    a, b = ins["a"].copy(), ins["b"].copy()
    k1, k2 = k // 3, k // 2
    a[R_NAN, k2] = np.nan
    b[k1, C_PINF] = np.inf
    a[R_ZERO, :] = -0.0
    a[R_ZERO, k1] = 0.5
    arrays = [a, b]
    if workload == "mbr":
        bias = ins["bias"].copy()
        bias[C_NINF] = -np.inf
        bias[C_BPINF] = np.inf
        arrays.append(bias)
    out = _run(workload, m, n, k, options, arrays)
    mbr = workload == "mbr"

    # NaN row
    assert np.isnan(out[R_NAN]).all()
    rows = np.array([r for r in range(m) if r != R_NAN])
    # +inf column: sign of A[m, k1]; relu maps -inf to +0.0
    col = out[rows, C_PINF]
    pos = a[rows, k1] > 0
    assert (col[pos] == np.inf).all()
    if mbr:
        assert (col[~pos] == 0.0).all() and not np.signbit(col[~pos]).any()
    else:
        assert (col[~pos] == -np.inf).all()
    if mbr:
        assert (out[rows, C_NINF] == 0.0).all() and not np.signbit(out[rows, C_NINF]).any()
        assert (out[rows, C_BPINF] == np.inf).all()
    # the -0.0 row with one 0.5: exactly one product
    cols = np.array([c for c in range(n) if c not in (C_PINF, C_NINF, C_BPINF)])
    want = (np.float32(0.5) * b[k1, cols]).astype(np.float32)
    if mbr:
        want = o.relu(o.add(want, arrays[2][cols]))
    got = out[R_ZERO, cols]
    assert o.bitwise_diff(got, want.astype(np.float32)) == 0

    # every other output: the usual bar against the unmodified inputs
    keep_r = np.array([r for r in range(m) if r not in (R_NAN, R_ZERO)])
    ref, bound = o.fp64_reference(workload, ins)
    sub = np.ix_(keep_r, cols)
    assert not np.isnan(out[sub]).any()
    eob = o.e1_metrics(out[sub], ref[sub], bound[sub])["max_err_over_bound"]
    assert eob <= 1.0, eob
    if mbr:
        z = o.preactivation64(ins)
        assert o.mask_mismatches(out[sub], z[sub], bound[sub]) == 0


SPECIALS = np.array([np.nan, -0.0, 0.0, np.inf, -np.inf, 1e-45, -1e-45, 3.0e38, -3.0e38, 1.0, -1.0],
                    np.float32)


def _same(got, want):
    nan = np.isnan(want)
    assert (np.isnan(got) == nan).all()
    assert o.bitwise_diff(got[~nan], want[~nan]) == 0


@pytest.mark.parametrize("options", ["block-tile=16,16 thread-tile=1,1", "block-tile=4,256 thread-tile=1,4"])
@pytest.mark.parametrize("workload", ["relu", "bias_add", "add"])
@pytest.mark.parametrize("n", [132, 130])   # 16-byte aligned rows (128-bit path) and unaligned ones
def test_special_values_through_element_ops(workload, options, n):
    m = 64
    rng = np.random.default_rng(7)
    x = rng.choice(SPECIALS, size=(m, n)).astype(np.float32)
    if workload == "relu":
        arrays, want = [x], o.relu(x)
    elif workload == "bias_add":
        bias = rng.choice(SPECIALS, size=n).astype(np.float32)
        arrays, want = [x, bias], o.bias_add(x, bias)
    else:
        y = rng.choice(SPECIALS, size=(m, n)).astype(np.float32)
        arrays, want = [x, y], o.add(x, y)
    out = _run(workload, m, n, None, options, arrays)
    _same(out, want)
    if workload == "relu":
        assert not np.signbit(out[x == 0]).any()   # -0.0 -> +0.0
