"""Compile, check, and time TensorForge GPU kernels on MI355X (gfx950).

Same functions, arguments and returned dictionaries as the reference's
python/tforge_gpu.py (cited per function); the tool chain underneath is
replaced by libtforge_hip.so:

  reference: input.mlir --tensorforge-opt--> device.mlir --mlir-translate/opt/
             llc/ptxas--> k.cubin; tforge-gpu-bench subprocess per call
  here:      input.mlir --tf_compile (front end + choice of an
             ahead-of-time gfx950 instantiation)--> launch.json;
             tf_run / tf_bench / tf_kernel_info in this process

compile_kernel still writes input.mlir and launch.json into the artifact
directory, and check / bench / info take that directory, as before.
Errors surface as RuntimeError with the library's message, where the
reference raised RuntimeError for a failed tool.
"""

import json
import os
import pathlib

import numpy as np

from . import _lib
from . import tforge_cpu as tc

ROOT = tc.ROOT
ART = tc.ART / "gpu"
ARCH = os.environ.get("TF_GPU_ARCH", "gfx950")
if ARCH != "gfx950":  # keep other targets' artifacts apart from the default ones
    ART = ART / ARCH
# MI355X: 256 CUs; FP32 matrix cores: v_mfma_f32_32x32x2_f32 is 4096 FLOP in
# 64 cycles per SIMD, 4 SIMDs per CU -> 256 FLOP per clock per CU.
CUS = int(os.environ.get("TF_GPU_CUS", "256"))
FP32_MFMA_FLOP_PER_CLK_PER_CU = 256
PEAK_CLOCK_MHZ = 2400


def fp32_peak_gflops(clock_mhz):
    """FP32 matrix peak at a clock (python/tforge_gpu.py:34-35 for the NVIDIA form)."""
    return CUS * FP32_MFMA_FLOP_PER_CLK_PER_CU * clock_mhz * 1e6 / 1e9


FP32_PEAK_TFLOPS = fp32_peak_gflops(PEAK_CLOCK_MHZ) / 1e3  # 157.3 TFLOP/s, the published figure


def parse_launch(path):
    """launch.json of a compiled kernel (python/tforge_gpu.py:42-51 parsed the
    tforge.launch attribute of device.mlir; the backend writes it as JSON)."""
    p = pathlib.Path(path)
    if p.is_dir():
        p = p / "launch.json"
    return json.loads(p.read_text())


def padded_shape(m, n, k, options):
    """Staged kernels (tile-k set) need M, N, K to be multiples of the block and
    K tiles; returns the padded problem the kernel is compiled for
    (python/tforge_gpu.py:54-63)."""
    opts = dict(o.split("=", 1) if "=" in o else (o, "1") for o in options.strip("{} ").split())
    tk = int(opts.get("tile-k", "0"))
    if tk <= 0 or opts.get("mask-edges", "0").lower() in ("1", "true"):
        return m, n, k  # mask-edges (backend option): the kernel masks edge tiles itself
    bm, bn = (int(x) for x in opts.get("block-tile", "16,16").split(","))
    up = lambda x, t: -(-x // t) * t
    return up(m, bm), up(n, bn), up(k, tk)


def _program_shape(workload, m, n, k, options):
    if workload in ("matmul", "mbr"):
        return padded_shape(m, n, k, options)
    if workload == "resmlp":
        pm, pn, pk = padded_shape(m, n, k, options)
        if (pm, pn, pk) != (m, n, k) or padded_shape(m, k, n, options) != (m, k, n):
            raise RuntimeError("resmlp: shapes must already be multiples of the block and K tiles")
        return m, n, k
    return m, n, k


def compile_kernel(workload, m, n, k, options="", tag="default"):
    """Compile one GPU kernel (python/tforge_gpu.py:66-91).  For elementwise
    workloads k is ignored.  Returns (artifact dir, launch dict)."""
    d = ART / tag / f"{workload}_{m}x{n}x{k}"
    d.mkdir(parents=True, exist_ok=True)
    pm, pn, pk = _program_shape(workload, m, n, k, options)
    text = tc.gen_mlir(workload, pm, pn, pk if workload in ("matmul", "mbr", "resmlp") else None)
    (d / "input.mlir").write_text(text)
    kern = _lib.Kernel(text, options, source_name=str(d / "input.mlir"))
    launches = kern.launches()
    first = launches[0]
    launch = {"kernel": first["kernel"], "grid": first["grid"], "block": first["block"],
              "args": first["args"], "padded": [pm, pn, pk], "options": options,
              "family": first["family"], "launches": launches}
    (d / "launch.json").write_text(json.dumps(launch))
    return d, launch


def _kernel(kdir, launch):
    kdir = pathlib.Path(kdir)
    text = (kdir / "input.mlir").read_text()
    return _lib.Kernel(text, launch.get("options", ""), source_name=str(kdir / "input.mlir"))


def _blas_kernel(workload, m, n, k):
    if workload not in ("matmul", "mbr"):
        raise RuntimeError("blas mode needs matmul or mbr")
    return _lib.Kernel(tc.gen_mlir(workload, m, n, k), "", source_name="blas.mlir")


def _mode(mode):
    if mode == "kernel":
        return _lib.TF_MODE_KERNEL
    if mode in ("rocblas", "cublas", "blas"):
        return _lib.TF_MODE_BLAS
    raise ValueError(mode)


def _logical(workload, m, n, k, launch):
    if workload not in ("matmul", "mbr") or launch is None:
        return None
    pm, pn, pk = launch.get("padded", [m, n, k])
    return None if (pm, pn, pk) == (m, n, k) else (m, n, k)


def info(workload, m, n, k, kdir, launch):
    """Registers, LDS, and occupancy from the HIP occupancy API
    (python/tforge_gpu.py:107-109; --info-only)."""
    return _kernel(kdir, launch).resources(0)


def reference64(workload, ins):
    """FP64 reference of a matmul or mbr on its inputs (python/tforge_gpu.py:134-145):
    (ref, bound, z) with ref = A64 @ B64 (+ bias64, max 0), bound =
    gamma_j * (|A64| @ |B64| (+ |bias64|)) + FLT_MIN, gamma_j = j u / (1 - j u),
    u = 2^-24, j = K (+1 for mbr), and z the FP64 pre-activation whose sign
    the ReLU decides (None for matmul)."""
    a64, b64 = ins["a"].astype(np.float64), ins["b"].astype(np.float64)
    acc, mag, steps = a64 @ b64, np.abs(a64) @ np.abs(b64), a64.shape[1]
    z = None
    if workload == "mbr":
        bias64 = ins["bias"].astype(np.float64)
        z = acc + bias64
        acc, mag, steps = np.maximum(z, 0.0), mag + np.abs(bias64), steps + 1
    gamma = steps * tc.F32_EPS / (1 - steps * tc.F32_EPS)
    return acc, gamma * mag + np.finfo(np.float32).tiny, z


def bound_verdict(out, ref, bound, z=None):
    """The reference's pass rule on an output: no NaN (outputs are
    NaN-prefilled) and err/bound <= 1; plus, where z is given, the ReLU mask
    rule: where |z| > bound, out == 0 exactly when z <= 0."""
    err = np.abs(out.astype(np.float64) - ref)
    res = {"nan_count": int(np.isnan(out).sum()),
           "max_abs_err": float(np.nanmax(err)) if err.size else 0.0,
           "err_over_bound": float(np.nanmax(err / bound)) if err.size else 0.0}
    if z is not None:
        decided = np.abs(z) > bound
        res["mask_mismatches"] = int(np.count_nonzero(decided & ((out == 0) != (z <= 0))))
    res["pass"] = res["nan_count"] == 0 and res["err_over_bound"] <= 1.0 and res.get("mask_mismatches", 0) == 0
    return res


def elementwise_verdict(workload, ins, out):
    """Element ops must equal NumPy float32 bit for bit (python/tforge_gpu.py:116-126)."""
    with np.errstate(invalid="ignore", over="ignore"):
        want = {"bias_add": lambda: ins["a"] + ins["bias"], "add": lambda: ins["a"] + ins["b"],
                "relu": lambda: np.maximum(ins["a"], np.float32(0))}[workload]()
    want = np.ascontiguousarray(want, np.float32)
    exact = bool(np.array_equal(out.view(np.uint32), want.view(np.uint32)))
    return {"pass": exact, "nan_count": int(np.isnan(out).sum()), "err_over_bound": 0.0 if exact else float("inf"),
            "max_abs_err": float(np.max(np.abs(out.astype(np.float64) - want))) if out.size else 0.0}


def _bound_check(workload, ins, out, k):
    """reference64 + bound_verdict for a matmul or mbr output."""
    return bound_verdict(out, *reference64(workload, ins))


def _resmlp_check(ins, out):
    """Bound for relu(relu(x@w1+b1)@w2+b2)+x, composed from the reference
    bound per layer.  With E1 = gamma_{n+1}(|x||w1| + |b1|) (layer 1, relu is
    1-Lipschitz), the computed h~ satisfies |h~ - h| <= E1, so the layer-2
    pre-activation error is at most
      Ez = gamma_{k+1}((|h| + E1)|w2| + |b2|) + E1 |w2|
    and the final f32 add contributes u |y~| <= u (|y| + Ez)."""
    x, w1, b1, w2, b2 = (ins[s].astype(np.float64) for s in ("x", "w1", "b1", "w2", "b2"))
    n, k = w1.shape
    g = lambda j: j * tc.F32_EPS / (1 - j * tc.F32_EPS)
    z1 = x @ w1 + b1
    h = np.maximum(z1, 0.0)
    e1 = g(n + 1) * (np.abs(x) @ np.abs(w1) + np.abs(b1))
    z2 = h @ w2 + b2
    ez = g(k + 1) * ((np.abs(h) + e1) @ np.abs(w2) + np.abs(b2)) + e1 @ np.abs(w2)
    y = np.maximum(z2, 0.0) + x
    bound = ez + tc.F32_EPS * (np.abs(y) + ez) + np.finfo(np.float32).tiny
    err = np.abs(out.astype(np.float64) - y)
    res = {"nan_count": int(np.isnan(out).sum()), "max_abs_err": float(np.nanmax(err)) if err.size else 0.0,
           "err_over_bound": float(np.nanmax(err / bound)) if err.size else 0.0}
    res["pass"] = res["nan_count"] == 0 and res["err_over_bound"] <= 1.0
    return res


def execute(workload, m, n, k, arrays, kdir=None, launch=None, mode="kernel"):
    """One correctness run (NaN-prefilled output) of a compiled kernel, or of
    the vendor-library mode, on host arrays in entry-argument order."""
    out = np.empty((m, n), dtype=np.float32)
    if mode == "kernel":
        _kernel(kdir, launch).run(arrays, out, _lib.TF_MODE_KERNEL, _logical(workload, m, n, k, launch))
    else:
        _blas_kernel(workload, m, n, k).run(arrays, out, _mode(mode))
    return out


def verdict(workload, ins, out):
    """Pass/fail of an output for its workload: bit-exact element ops, the
    FP64 bound for matmul / mbr, its two-layer composition for resmlp."""
    if workload in ("bias_add", "relu", "add"):
        return elementwise_verdict(workload, ins, out)
    if workload == "resmlp":
        return _resmlp_check(ins, out)
    return bound_verdict(out, *reference64(workload, ins))


def check(workload, m, n, k, kdir=None, launch=None, mode="kernel", seed=1234):
    """Run once on seeded inputs and check (python/tforge_gpu.py:112-145).
    Returns (result dict, output)."""
    ins = tc.make_inputs(workload, m, n, k, seed)
    out = execute(workload, m, n, k, [np.ascontiguousarray(v) for v in ins.values()], kdir, launch, mode)
    return verdict(workload, ins, out), out


def bench(workload, m, n, k, kdir=None, launch=None, mode="kernel", warmup=10, reps=100, flush=False):
    """Timed runs; the same keys as the reference runner's JSON line
    (runners/gpu/tforge-gpu-bench.cu:370-381, python/tforge_gpu.py:148-152).
    GPU clock and power come from amdsmi (-1 when unavailable)."""
    if mode == "kernel":
        kern = _kernel(kdir, launch)
        logical = _logical(workload, m, n, k, launch)
        res = kern.resources(0)
        geo = kern.launches()[0]
    else:
        kern = _blas_kernel(workload, m, n, k)
        logical = None
        res = {"regs": -1, "local_bytes": -1, "static_smem": -1, "blocks_per_sm": -1, "theo_occupancy": -1.0}
        geo = {"grid": [1, 1, 1], "block": [1, 1, 1]}
    r = kern.bench(None, _mode(mode), logical, seed=1234, warmup=warmup, reps=reps, flush=flush)
    dev = _lib.device_info()
    pm, pn, pk = (int(x) for x in r.padded)
    return {"gpu": dev["name"] or dev["arch"], "mode": "kernel" if mode == "kernel" else "rocblas",
            "workload": workload, "m": m, "n": n, "k": k, "padded": f"{pm}x{pn}x{pk}",
            "grid": "x".join(str(x) for x in geo["grid"]), "block": "x".join(str(x) for x in geo["block"]),
            "regs": res["regs"], "local_bytes": res["local_bytes"], "static_smem": res["static_smem"],
            "blocks_per_sm": res["blocks_per_sm"], "theo_occupancy": res["theo_occupancy"],
            "warmup": r.warmup, "reps": r.reps, "l2_flush": r.l2_flush, "median_ms": r.median_ms,
            "min_ms": r.min_ms, "std_ms": r.std_ms, "sm_clock_median_mhz": r.clock_median_mhz,
            "sm_clock_min_mhz": r.clock_min_mhz, "sm_clock_max_mhz": r.clock_max_mhz,
            "power_median_w": r.power_median_w, "hip_driver": dev["driver_version"],
            # key kept for drop-in readers of the reference's JSON; holds the HIP driver version
            "cuda_driver": dev["driver_version"], "samples_ms": kern.samples()}


def ptxas_resources(kdir):
    """Registers, spills and LDS of the selected instantiation from the
    compiler's resource remarks (python/tforge_gpu.py:155-160 read ptxas -v)."""
    launch = parse_launch(kdir)
    table = json.loads((pathlib.Path(__file__).resolve().parent / "kernel_resources.json").read_text())
    rec = table.get(launch["kernel"], {})
    return {"regs": rec.get("vgprs", 0), "agprs": rec.get("agprs", 0), "sgprs": rec.get("sgprs", 0),
            "spill_stores": rec.get("vgpr_spill", 0), "spill_loads": rec.get("vgpr_spill", 0),
            "smem": rec.get("lds_bytes", 0), "scratch": rec.get("scratch_bytes", 0),
            "occupancy_waves_per_simd": rec.get("occupancy_waves_per_simd", -1)}
