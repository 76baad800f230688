"""TEST INFRASTRUCTURE ONLY -- the CPU oracle for the TensorForge GPU hot path.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this module, and only as the checker (or the timed CPU baseline).  The product
(tensorforge_amd/) never imports it.

Contents, each a restatement of the reference (paths in the TensorForge tree):

  make_inputs(workload, m, n, k, seed)   python/tforge_cpu.py:89-100
      numpy default_rng(seed).uniform(-1, 1) drawn in the order a, b[, bias],
      each rounded to float32.  Pinned by the e1 known answers (a wrong seed,
      draw order or distribution changes every error statistic).
  fp64_reference(...)                    python/tforge_gpu.py:134-145,
                                         python/tforge_cpu.py:288-304
      ref = A64 @ B64 (+ bias64, max 0); mag = |A64| @ |B64| (+ |bias64|);
      gamma_j = j u / (1 - j u), u = 2^-24, j = K (+1 for mbr);
      bound = gamma * mag + FLT_MIN.  Pinned by the e1 known answers and by the
      stage8 correctness column.
  matmul_fma / matmul_nofma / epilogue   C closed forms in tforge_oracle.c;
      pinned bit-for-bit by the e1 bitwise-difference counts.
  e1_metrics(out, ref, bound)            bench/e1_numerics.py:93-104
  preactivation64(ins)                   z = A64 @ B64 + bias64, the value whose
      sign the ReLU decides (lib/Conversion/TForgeToLinalg.cpp:94-133); pinned
      bit for bit to fp64_reference (max(z, 0) is its ref) and to exact integer
      arithmetic on a small case.
  mask_mismatches(out, z, bound)         the north star's ReLU-mask gate: where
      |z| > bound, out == 0 must agree with z <= 0; pinned by planted flips
      (each counts exactly once), in-bound perturbations (count nothing) and
      |z| == bound exactly (undecided).
  add / relu / bias_add                  tforge.add / relu / bias_add on their
      own (docs/dialect.md:26-30; python/tforge_gpu.py:116-126): one IEEE f32
      op per element, relu = maximum(x, +0.0) with NaN kept and -0 -> +0;
      pinned against NumPy float32 on NaN, +-0, +-inf, denormals and overflow.
  mbr_vec6x16 / matmul_scalar_mnk / time_*   the CPU baseline port and the default
      scalar pipeline's loop (tforge_oracle.c); pinned by the err/bound the reference's
      CPU results hold for both (results/cpu/stage4.csv, stage6_best.csv).

Nothing here is "parity unpinned": every function above has a known-answer
test against files the reference itself holds or against what the
mathematics fixes (tests/test_oracle_golden.py, tests/test_oracle_pins.py).
"""

import ctypes
import pathlib
import subprocess

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
F32_EPS = 2.0 ** -24
FLT_MIN = float(np.finfo(np.float32).tiny)
BIAS, RELU, RESID = 1, 2, 4

_lib = None


def _cpu_has_avx2_fma():
    try:
        flags = pathlib.Path("/proc/cpuinfo").read_text()
    except OSError:
        return False
    return " avx2" in flags and " fma" in flags


def build():
    """Compile the C oracle in place (the GPU box uses the prebuilt files)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


def lib():
    global _lib
    if _lib is not None:
        return _lib
    name = "libtforge_oracle.so" if _cpu_has_avx2_fma() else "libtforge_oracle_generic.so"
    path = HERE / name
    if not path.exists():
        build()
    L = ctypes.CDLL(str(path))
    fp, i64, i32 = ctypes.c_void_p, ctypes.c_long, ctypes.c_int
    for fn in ("tfo_matmul_fma", "tfo_matmul_nofma"):
        getattr(L, fn).argtypes = [fp, fp, fp, i64, i64, i64, i32]
        getattr(L, fn).restype = None
    L.tfo_epilogue.argtypes = [fp, fp, fp, i64, i64, i32]
    L.tfo_matmul_scalar_mnk.argtypes = [fp, fp, fp, i64, i64, i64]
    L.tfo_epilogue.restype = None
    L.tfo_add.argtypes = [fp, fp, fp, i64]
    L.tfo_relu.argtypes = [fp, fp, i64]
    L.tfo_bias_add.argtypes = [fp, fp, fp, i64, i64]
    for fn in ("tfo_add", "tfo_relu", "tfo_bias_add"):
        getattr(L, fn).restype = None
    L.tfo_mbr_vec6x16.argtypes = [fp, fp, fp, fp, i64, i64, i64, i32, i32]
    L.tfo_mbr_vec6x16.restype = None
    for fn in ("tfo_time_mbr_vec6x16", "tfo_time_scalar"):
        getattr(L, fn).argtypes = [fp, fp, fp, fp, i64, i64, i64, i32, i32, i32]
        getattr(L, fn).restype = ctypes.c_double
    L.tfo_have_avx2.restype = i32
    _lib = L
    return L


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def make_inputs(workload, m, n, k, seed=1234):
    rng = np.random.default_rng(seed)
    u = lambda *s: rng.uniform(-1.0, 1.0, size=s).astype(np.float32)
    if workload == "add":
        return {"a": u(m, n), "b": u(m, n)}
    if workload == "relu":
        return {"a": u(m, n)}
    if workload == "bias_add":
        return {"a": u(m, n), "bias": u(n)}
    if workload == "matmul":
        return {"a": u(m, k), "b": u(k, n)}
    if workload == "mbr":
        return {"a": u(m, k), "b": u(k, n), "bias": u(n)}
    raise ValueError(workload)


def matmul_fma(a, b, threads=0):
    a, b = _f32(a), _f32(b)
    (m, k), (k2, n) = a.shape, b.shape
    assert k == k2
    c = np.empty((m, n), np.float32)
    lib().tfo_matmul_fma(_p(a), _p(b), _p(c), m, n, k, threads)
    return c


def matmul_nofma(a, b, threads=0):
    a, b = _f32(a), _f32(b)
    (m, k), (k2, n) = a.shape, b.shape
    assert k == k2
    c = np.empty((m, n), np.float32)
    lib().tfo_matmul_nofma(_p(a), _p(b), _p(c), m, n, k, threads)
    return c


def matmul_scalar_mnk(a, b):
    """tfo_matmul_scalar_mnk: the no-FMA form in the default CPU pipeline's loop order."""
    a, b = _f32(a), _f32(b)
    (m, k), (k2, n) = a.shape, b.shape
    assert k == k2
    c = np.empty((m, n), np.float32)
    lib().tfo_matmul_scalar_mnk(_p(a), _p(b), _p(c), m, n, k)
    return c


def epilogue(c, bias=None, relu=False, resid=None):
    """In-place on a copy: y = c (+ bias[n]) (relu) (+ resid), one f32 op each."""
    y = np.array(c, dtype=np.float32, copy=True, order="C")
    m, n = y.shape
    flags = (BIAS if bias is not None else 0) | (RELU if relu else 0) | (RESID if resid is not None else 0)
    bias = None if bias is None else _f32(bias)
    resid = None if resid is None else _f32(resid)
    lib().tfo_epilogue(_p(y), _p(bias), _p(resid), m, n, flags)
    return y


def add(x, y):
    """tforge.add: x + y, one f32 rounding per element (tfo_add)."""
    x, y = _f32(x), _f32(y)
    assert x.shape == y.shape
    out = np.empty_like(x)
    lib().tfo_add(_p(x), _p(y), _p(out), x.size)
    return out


def relu(x):
    """tforge.relu: maximum(x, +0.0) -- NaN stays NaN, -0.0 becomes +0.0 (tfo_relu)."""
    x = _f32(x)
    out = np.empty_like(x)
    lib().tfo_relu(_p(x), _p(out), x.size)
    return out


def bias_add(x, bias):
    """tforge.bias_add: x[m, n] + bias[n] along the last dimension (tfo_bias_add)."""
    x, bias = _f32(x), _f32(bias)
    m, n = x.shape
    assert bias.shape == (n,)
    out = np.empty_like(x)
    lib().tfo_bias_add(_p(x), _p(bias), _p(out), m, n)
    return out


def elementwise(workload, ins):
    """Expected output of an element-op workload on make_inputs-style arrays."""
    if workload == "add":
        return add(ins["a"], ins["b"])
    if workload == "relu":
        return relu(ins["a"])
    if workload == "bias_add":
        return bias_add(ins["a"], ins["bias"])
    raise ValueError(workload)


def mbr_fma(a, b, bias, threads=0):
    return epilogue(matmul_fma(a, b, threads), bias=bias, relu=True)


def mbr_vec6x16(a, b, bias=None, relu=True, threads=0):
    a, b = _f32(a), _f32(b)
    (m, k), (_, n) = a.shape, b.shape
    c = np.empty((m, n), np.float32)
    flags = (BIAS if bias is not None else 0) | (RELU if relu else 0)
    bias = None if bias is None else _f32(bias)
    lib().tfo_mbr_vec6x16(_p(a), _p(b), _p(bias), _p(c), m, n, k, flags, threads)
    return c


def aligned_empty(shape, align=64):
    """An uninitialised float32 array whose data starts on an `align`-byte
    boundary (the reference CPU runner's buffers are 64-byte aligned:
    runners/cpu/tforge-cpu-bench.cpp:65-77)."""
    size = int(np.prod(shape))
    raw = np.empty(size + align // 4, np.float32)
    off = (-raw.ctypes.data % align) // 4
    return raw[off:off + size].reshape(shape)


def aligned_copy(x, align=64):
    out = aligned_empty(np.shape(x), align)
    out[...] = x
    return out


def _timing_args(a, b, bias, relu):
    a, b = _f32(a), _f32(b)
    (m, k), (_, n) = a.shape, b.shape
    flags = (BIAS if bias is not None else 0) | (RELU if relu else 0)
    return a, b, (None if bias is None else _f32(bias)), aligned_empty((m, n)), m, n, k, flags


def time_vec6x16(a, b, bias, warmup, reps, relu=True):
    """Median ns per call of the 6x16x4 port, one thread, on the calling
    thread's CPU (the caller pins it); bias None and relu False time plain matmul."""
    a, b, bias, c, m, n, k, flags = _timing_args(a, b, bias, relu)
    return lib().tfo_time_mbr_vec6x16(_p(a), _p(b), _p(bias), _p(c), m, n, k, flags, warmup, reps)


def time_scalar(a, b, bias, warmup, reps, relu=True):
    """Median ns per call of the default pipeline's scalar loop + epilogue."""
    a, b, bias, c, m, n, k, flags = _timing_args(a, b, bias, relu)
    return lib().tfo_time_scalar(_p(a), _p(b), _p(bias), _p(c), m, n, k, flags, warmup, reps)


def fp64_reference(workload, ins):
    """(ref, bound) of the reference's check for matmul / mbr."""
    a64, b64 = ins["a"].astype(np.float64), ins["b"].astype(np.float64)
    k = a64.shape[1]
    ref, mag, steps = a64 @ b64, np.abs(a64) @ np.abs(b64), k
    if workload == "mbr":
        bias64 = ins["bias"].astype(np.float64)
        ref, mag, steps = np.maximum(ref + bias64, 0.0), mag + np.abs(bias64), k + 1
    gamma = steps * F32_EPS / (1 - steps * F32_EPS)
    return ref, gamma * mag + FLT_MIN


def preactivation64(ins):
    """FP64 pre-activation z = A@B + bias, for the ReLU mask rule."""
    a64, b64 = ins["a"].astype(np.float64), ins["b"].astype(np.float64)
    return a64 @ b64 + ins["bias"].astype(np.float64)


def e1_metrics(out, ref, bound):
    err = np.abs(out.astype(np.float64) - ref)
    return {"max_abs_err": float(err.max()), "rms_err": float(np.sqrt((err ** 2).mean())),
            "max_err_over_bound": float((err / bound).max())}


def bitwise_diff(x, y):
    return int(np.count_nonzero(np.asarray(x, np.float32).view(np.uint32) != np.asarray(y, np.float32).view(np.uint32)))


def mask_mismatches(out, z, bound):
    """Count elements where |z| > bound but (out == 0) disagrees with (z <= 0)."""
    decided = np.abs(z) > bound
    return int(np.count_nonzero(decided & ((out == 0) != (z <= 0))))
