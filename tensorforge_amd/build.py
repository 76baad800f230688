"""Build libtforge_hip.so in place for gfx950.

Steps: generate the staged-kernel instantiation shards (csrc/gen_instances.py),
compile every translation unit in parallel (hipcc for HIP, g++ for the host
front end), link the shared library next to this file, and record each
kernel's register / LDS / scratch usage from the compiler's resource remarks
in kernel_resources.json (the counterpart of the reference's ptxas -v report,
python/tforge_gpu.py:155-160), and the commit the library was built from in
BUILD_INFO.json (results rows name it; the GPU machine gets no .git).

    python -m tensorforge_amd.build [--no-force] [-j N]
"""

import argparse
import concurrent.futures as cf
import json
import os
import pathlib
import re
import shutil
import subprocess
import sys

PKG = pathlib.Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OUT = CSRC / "_build"
LIB = PKG / "libtforge_hip.so"
RESOURCES = PKG / "kernel_resources.json"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
# Packed FP32 (v_pk_*_f32) is disabled for all device code.  Kernel-argument
# preloading: a kernel's leading scalar arguments (up to 16 SGPRs) arrive in
# SGPRs at wave launch instead of through loads from the argument segment
# (the staged GEMM kernels lead with the fields their prologue needs).
HIP_FLAGS = ["--offload-arch=" + ARCH, "-O3", "-std=c++17", "-fPIC", "-Wall",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-mllvm", "-amdgpu-kernarg-preload-count=16",
             "-I", str(ROOT / "include"), "-I", str(CSRC),
             "-Rpass-analysis=kernel-resource-usage"]
CXX_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wextra", "-I", str(ROOT / "include"), "-I", str(CSRC),
             "-I", "/opt/rocm/include", "-D__HIP_PLATFORM_AMD__"]


def _units():
    sys.path.insert(0, str(CSRC))
    import gen_instances  # noqa: E402
    gen_instances.main()
    units = [CSRC / "runtime.hip", CSRC / "direct_kernels.hip", CSRC / "_gen" / "registry.hip",
             CSRC / "_gen" / "wavek.hip"]
    units += sorted((CSRC / "_gen").glob("staged_*.hip"))
    return units


def _includes(src, seen=None):
    """src and the project headers it includes, transitively."""
    seen = set() if seen is None else seen
    if src in seen or not src.exists():
        return seen
    seen.add(src)
    for name in re.findall(r'^#include\s+"([^"]+)"', src.read_text(), re.M):
        for base in (src.parent, CSRC, ROOT / "include"):
            if (base / name).exists():
                _includes((base / name).resolve(), seen)
                break
    return seen


def _compile(src, force):
    obj = OUT / (src.parent.name + "_" + src.stem + ".o")
    log = obj.with_suffix(".log")
    deps = sorted(_includes(src.resolve()))
    if not force and obj.exists() and log.exists() and all(obj.stat().st_mtime >= d.stat().st_mtime for d in deps):
        return obj, log.read_text()
    if src.suffix == ".hip":
        cmd = [HIPCC] + HIP_FLAGS + ["-c", str(src), "-o", str(obj)]
    else:
        cmd = [os.environ.get("CXX", "g++")] + CXX_FLAGS + ["-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    text = r.stdout + r.stderr
    if r.returncode != 0:
        errs = "\n".join(l for l in text.splitlines() if "packed-fp32-ops" not in l and "remark" not in l)
        raise RuntimeError(f"compile failed: {src.name}\n{' '.join(cmd)}\n{errs}")
    log.write_text(text)
    return obj, text


def _demangle(names):
    if not names or not shutil.which("c++filt"):
        return {n: n for n in names}
    r = subprocess.run(["c++filt"], input="\n".join(names), capture_output=True, text=True)
    return dict(zip(names, r.stdout.splitlines()))


def _entry_name(demangled):
    m = re.search(r"staged_gemm_kernel<(\d+), (\d+), (\d+), (\d+), (\d+), (\d+), (\d+), (\d+)>", demangled)
    if m:
        bm, bn, tm, tn, bk, p, v, mk = m.groups()
        return (f"tf_staged_b{bm}x{bn}_t{tm}x{tn}_k{bk}" + ("" if p == "1" else "_noprom") +
                ("" if v == "1" else "_novec") + ("_masked" if mk == "1" else ""))
    m = re.search(r"wavek_gemm_kernel<(\d+), (\d+), (\d+), (\d+)(?:, \d+)?>", demangled)
    if m:
        # One kernel serves every thread tile with its thread count.
        import gen_instances  # noqa: E402  (csrc is on sys.path after _units)
        bm, bn, nt, bk = (int(x) for x in m.groups())
        return [gen_instances.wavek_name(bm, bn, tm, tn, bk) for tm, tn in gen_instances.wavek_thread_tiles(bm, bn, nt)]
    m = re.search(r"(direct_gemm|elementwise)_kernel<(\d+), (\d+)>", demangled)
    if m:
        fam = "direct" if m.group(1) == "direct_gemm" else "elementwise"
        return f"tf_{fam}_t{m.group(2)}x{m.group(3)}"
    return None


def _resources(logs):
    """Parse -Rpass-analysis=kernel-resource-usage remarks per kernel."""
    recs, cur = {}, None
    for text in logs:
        for line in text.splitlines():
            m = re.search(r"remark:\s+Function Name: (\S+)", line)
            if m:
                cur = recs.setdefault(m.group(1), {})
                continue
            m = re.search(r"remark:\s+([A-Za-z /\[\]]+?): (\d+)", line)
            if m and cur is not None:
                key = m.group(1).strip()
                cur[key] = int(m.group(2))
    dem = _demangle(list(recs))
    out = {}
    for mangled, rec in recs.items():
        names = _entry_name(dem[mangled])
        if names is None:
            continue
        for name in names if isinstance(names, list) else [names]:
            out[name] = {"vgprs": rec.get("VGPRs", -1), "agprs": rec.get("AGPRs", -1), "sgprs": rec.get("TotalSGPRs", -1),
                         "scratch_bytes": rec.get("ScratchSize [bytes/lane]", 0),
                         "lds_bytes": rec.get("LDS Size [bytes/block]", 0),
                         "occupancy_waves_per_simd": rec.get("Occupancy [waves/SIMD]", -1),
                         "vgpr_spill": rec.get("VGPRs Spill", 0), "sgpr_spill": rec.get("SGPRs Spill", 0),
                         "symbol": mangled}
    return out


def build(force=True, jobs=None):
    OUT.mkdir(exist_ok=True)
    units = _units() + [CSRC / "frontend.cpp"]
    jobs = jobs or min(16, os.cpu_count() or 4)
    with cf.ThreadPoolExecutor(jobs) as ex:
        results = list(ex.map(lambda u: _compile(u, force), units))
    objs = [o for o, _ in results]
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, "--offload-arch=" + ARCH, "-shared", "-fPIC", "-o", str(tmp)] + [str(o) for o in objs] + ["-ldl"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stdout + r.stderr)
    os.replace(tmp, LIB)
    RESOURCES.write_text(json.dumps(_resources([t for _, t in results]), indent=1, sort_keys=True) + "\n")
    sys.path.insert(0, str(ROOT))
    from tensorforge_amd import provenance
    provenance.write_build_info()
    return LIB


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--no-force", action="store_true", help="reuse up-to-date object files")
    ap.add_argument("-j", type=int, default=None)
    a = ap.parse_args()
    print(build(force=not a.no_force, jobs=a.j))


if __name__ == "__main__":
    main()
