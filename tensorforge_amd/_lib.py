"""ctypes bindings of libtforge_hip.so (declared in include/tforge_hip.h).

The library must have been built (python -m tensorforge_amd.build); there is
no fallback: every call on the hot path goes through the gfx950 kernels.
"""

import ctypes
import pathlib

import numpy as np

PKG = pathlib.Path(__file__).resolve().parent
LIB_PATH = PKG / "libtforge_hip.so"

TF_MODE_KERNEL, TF_MODE_BLAS = 0, 1
FAMILY_NAMES = {0: "direct", 1: "staged", 2: "elementwise", 4: "wavek"}


class DeviceInfo(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 256), ("arch", ctypes.c_char * 64), ("compute_units", ctypes.c_int),
                ("max_clock_mhz", ctypes.c_int), ("lds_bytes_per_cu", ctypes.c_int),
                ("max_threads_per_cu", ctypes.c_int), ("l2_bytes", ctypes.c_longlong),
                ("global_mem_bytes", ctypes.c_longlong), ("driver_version", ctypes.c_int),
                ("runtime_version", ctypes.c_int)]


class LaunchInfo(ctypes.Structure):
    _fields_ = [("kernel", ctypes.c_char * 96), ("args", ctypes.c_char * 160), ("ops", ctypes.c_char * 96),
                ("family", ctypes.c_int), ("grid", ctypes.c_int * 3), ("block", ctypes.c_int * 3),
                ("m", ctypes.c_longlong), ("n", ctypes.c_longlong), ("k", ctypes.c_longlong),
                ("lds_bytes", ctypes.c_int)]


class KernelResources(ctypes.Structure):
    _fields_ = [("regs", ctypes.c_int), ("local_bytes", ctypes.c_int), ("static_smem", ctypes.c_int),
                ("blocks_per_cu", ctypes.c_int), ("theo_occupancy", ctypes.c_double), ("threads", ctypes.c_int)]


class BufferInfo(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 64), ("role", ctypes.c_int), ("rows", ctypes.c_longlong),
                ("cols", ctypes.c_longlong)]


class BenchResult(ctypes.Structure):
    _fields_ = [("median_ms", ctypes.c_double), ("min_ms", ctypes.c_double), ("mean_ms", ctypes.c_double),
                ("std_ms", ctypes.c_double), ("clock_median_mhz", ctypes.c_double),
                ("clock_min_mhz", ctypes.c_double), ("clock_max_mhz", ctypes.c_double),
                ("power_median_w", ctypes.c_double), ("warmup", ctypes.c_int), ("reps", ctypes.c_int),
                ("l2_flush", ctypes.c_int), ("padded", ctypes.c_longlong * 3)]


# (name, restype, argtypes) of every exported function, in header order.
P, I, LL, U = ctypes.c_void_p, ctypes.c_int, ctypes.c_longlong, ctypes.c_uint
SIGNATURES = [
    ("tf_last_error", ctypes.c_char_p, []),
    ("tf_device_info", I, [ctypes.POINTER(DeviceInfo)]),
    ("tf_compile", I, [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(P)]),
    ("tf_kernel_free", None, [P]),
    ("tf_kernel_num_launches", I, [P]),
    ("tf_kernel_launch_info", I, [P, I, ctypes.POINTER(LaunchInfo)]),
    ("tf_kernel_num_buffers", I, [P]),
    ("tf_kernel_buffer_info", I, [P, I, ctypes.POINTER(BufferInfo)]),
    ("tf_kernel_host_shape", I, [P, ctypes.POINTER(LL), I, ctypes.POINTER(LL), ctypes.POINTER(LL)]),
    ("tf_kernel_info", I, [P, I, ctypes.POINTER(KernelResources)]),
    ("tf_launch", I, [P, ctypes.POINTER(P), P]),
    ("tf_launch_noalloc", I, [P, ctypes.POINTER(P), P]),
    ("tf_run", I, [P, I, ctypes.POINTER(LL), ctypes.POINTER(ctypes.POINTER(ctypes.c_float)),
                   ctypes.POINTER(ctypes.c_float)]),
    ("tf_bench", I, [P, I, ctypes.POINTER(LL), ctypes.POINTER(ctypes.POINTER(ctypes.c_float)), U, I, I, I,
                     ctypes.POINTER(BenchResult)]),
    ("tf_clock_probe", I, [P, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double),
                           ctypes.POINTER(ctypes.c_double)]),
    ("tf_bench_samples", I, [P, ctypes.POINTER(ctypes.c_double), I]),
    ("tf_registry_size", I, []),
    ("tf_registry_entry", I, [I, ctypes.POINTER(I), ctypes.POINTER(I), ctypes.c_char_p, I]),
]

_lib = None


def lib():
    """The loaded library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m tensorforge_amd.build` "
                               "(the gfx950 kernels are the only execution path)")
        # One HIP runtime per process: PyTorch wheels ship their own
        # libamdhip64.so.7 / libhsa-runtime64.so.1.  Loading torch first makes
        # this library bind to that already-loaded runtime (same sonames);
        # loading this library first would leave torch with a second runtime
        # that cannot open the GPU.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        L = ctypes.CDLL(str(LIB_PATH))
        for name, res, args in SIGNATURES:
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc):
    if rc < 0:
        raise RuntimeError(lib().tf_last_error().decode())
    return rc


class Kernel:
    """A compiled tforge program (owns the tf_kernel_t handle)."""

    def __init__(self, program, options="", source_name="input.mlir"):
        L = lib()
        self.h = P()
        check(L.tf_compile(source_name.encode(), program.encode(), options.encode(), ctypes.byref(self.h)))
        self.program, self.options = program, options
        # The buffer list is fixed at compile time; launch() validates against
        # this copy instead of asking the library on every call (a launch of a
        # small problem is otherwise bound by those calls, not by the GPU).
        self._bufs = self.buffers()
        self._sizes = [b["shape"][0] * b["shape"][1] for b in self._bufs]
        self._launch_fn = L.tf_launch

    def __del__(self):
        h = getattr(self, "h", None)
        if h and _lib is not None:
            _lib.tf_kernel_free(h)
            self.h = None

    def launches(self):
        L, out = lib(), []
        for i in range(check(L.tf_kernel_num_launches(self.h))):
            li = LaunchInfo()
            check(L.tf_kernel_launch_info(self.h, i, ctypes.byref(li)))
            out.append({"kernel": li.kernel.decode(), "grid": list(li.grid), "block": list(li.block),
                        "args": li.args.decode().split(","), "ops": li.ops.decode(),
                        "family": FAMILY_NAMES[li.family], "m": li.m, "n": li.n, "k": li.k,
                        "lds_bytes": li.lds_bytes})
        return out

    def buffers(self):
        L, out = lib(), []
        for i in range(check(L.tf_kernel_num_buffers(self.h))):
            bi = BufferInfo()
            check(L.tf_kernel_buffer_info(self.h, i, ctypes.byref(bi)))
            out.append({"name": bi.name.decode(), "role": "output" if bi.role == 1 else "input",
                        "shape": (bi.rows, bi.cols)})
        return out

    def resources(self, launch=0):
        r = KernelResources()
        check(lib().tf_kernel_info(self.h, launch, ctypes.byref(r)))
        return {"regs": r.regs, "local_bytes": r.local_bytes, "static_smem": r.static_smem,
                "blocks_per_sm": r.blocks_per_cu, "theo_occupancy": round(r.theo_occupancy, 3),
                "threads": r.threads}

    def host_shapes(self, logical=None):
        """(rows, cols) of each buffer (inputs, then the output) as tf_run and
        tf_bench copy it: the library's own answer, so the check below and the
        copies agree (a buffer in two roles, reordered arguments).  Raises the
        library's error where it would refuse `logical`."""
        L, out = lib(), []
        r, c = LL(), LL()
        for i in range(check(L.tf_kernel_num_buffers(self.h))):
            check(L.tf_kernel_host_shape(self.h, self._logical(logical), i, ctypes.byref(r), ctypes.byref(c)))
            out.append((r.value, c.value))
        return out

    def _check_host(self, arrays, out, logical):
        # tf_run copies whole buffers from and to these pointers: a short,
        # strided or non-float32 array would be read or written out of bounds.
        nargs = len(self._bufs) - 1
        if len(arrays) != nargs:
            raise ValueError(f"this program takes {nargs} input arrays, got {len(arrays)}")
        want = [r * c for r, c in self.host_shapes(logical)]
        named = [(f"input {i}", a, want[i]) for i, a in enumerate(arrays)]
        if out is not None:
            named.append(("output", out, want[-1]))
        for what, a, size in named:
            if not isinstance(a, np.ndarray) or a.dtype != np.float32 or not a.flags.c_contiguous:
                raise TypeError(f"{what} must be a C-contiguous float32 numpy array")
            if a.size != size:
                raise ValueError(f"{what} has {a.size} elements, the program needs {size}")

    def launch(self, device_ptrs, stream=0):
        n = len(self._sizes)
        if len(device_ptrs) != n:
            raise ValueError(f"this program takes {n} device buffers (inputs, then the output), "
                             f"got {len(device_ptrs)}")
        ptrs = [int(p) for p in device_ptrs]
        if not all(ptrs):
            for i, p in enumerate(ptrs):
                if not p and self._sizes[i] > 0:
                    raise ValueError(f"device buffer {i} ({self._bufs[i]['name']}) is a null pointer")
        rc = self._launch_fn(self.h, (P * n)(*ptrs), int(stream) or None)
        if rc < 0:
            check(rc)

    def launch_noalloc(self, device_ptrs, stream=0):
        """tf_launch_noalloc: the same launches with the library's fixed
        per-GPU scratch array; calls that overlap on one GPU race."""
        if len(device_ptrs) != len(self._sizes):
            raise ValueError(f"this program takes {len(self._sizes)} device buffers, got {len(device_ptrs)}")
        arr = (P * len(device_ptrs))(*[P(int(p)) for p in device_ptrs])
        check(lib().tf_launch_noalloc(self.h, arr, P(int(stream)) if stream else None))

    @staticmethod
    def _host_ptrs(arrays):
        arr = (ctypes.POINTER(ctypes.c_float) * len(arrays))()
        for i, a in enumerate(arrays):
            arr[i] = a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))
        return arr

    @staticmethod
    def _logical(mnk):
        return None if mnk is None else (LL * 3)(*[int(x) for x in mnk])

    def run(self, inputs, out, mode=TF_MODE_KERNEL, logical=None):
        self._check_host(inputs, out, logical)
        check(lib().tf_run(self.h, mode, self._logical(logical), self._host_ptrs(inputs),
                           out.ctypes.data_as(ctypes.POINTER(ctypes.c_float))))
        return out

    def bench(self, inputs=None, mode=TF_MODE_KERNEL, logical=None, seed=1234, warmup=10, reps=100, flush=False):
        r = BenchResult()
        if inputs is not None:
            self._check_host(inputs, None, logical)
        ptrs = self._host_ptrs(inputs) if inputs is not None else None
        check(lib().tf_bench(self.h, mode, self._logical(logical), ptrs, seed, warmup, reps, int(flush),
                             ctypes.byref(r)))
        return r

    def samples(self, cap=100000):
        buf = (ctypes.c_double * cap)()
        n = check(lib().tf_bench_samples(self.h, buf, cap))
        return list(buf[:n])


def device_info():
    d = DeviceInfo()
    check(lib().tf_device_info(ctypes.byref(d)))
    return {"name": d.name.decode(), "arch": d.arch.decode(), "compute_units": d.compute_units,
            "max_clock_mhz": d.max_clock_mhz, "lds_bytes_per_cu": d.lds_bytes_per_cu,
            "max_threads_per_cu": d.max_threads_per_cu, "l2_bytes": d.l2_bytes,
            "global_mem_bytes": d.global_mem_bytes, "driver_version": d.driver_version,
            "runtime_version": d.runtime_version}


def clock_probe(stream=0):
    """Shader clock in MHz (mean, min, max over the XCDs), measured on the
    device after the work queued on `stream`; synchronises that stream."""
    v = [ctypes.c_double() for _ in range(3)]
    check(lib().tf_clock_probe(P(int(stream)) if stream else None, *(ctypes.byref(x) for x in v)))
    return tuple(x.value for x in v)


def registry():
    L, out = lib(), []
    fam, cfg, name = I(), (I * 7)(), ctypes.create_string_buffer(96)
    for i in range(L.tf_registry_size()):
        check(L.tf_registry_entry(i, ctypes.byref(fam), cfg, name, 96))
        out.append({"family": FAMILY_NAMES[fam.value], "cfg": tuple(cfg), "name": name.value.decode()})
    return out
