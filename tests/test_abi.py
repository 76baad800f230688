"""The C-ABI library loads and exports exactly what include/tforge_hip.h
declares; the ctypes structs have the C layout; the registry is complete.
No compute calls (runs without a GPU)."""

import json
import pathlib
import re
import subprocess

import pytest

from tensorforge_amd import _lib
from tensorforge_amd import costmodel as cm

ROOT = pathlib.Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "tforge_hip.h"


def declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^(?:int|void|const char \*)\s*(tf_\w+)\(", text, re.M)))


def test_every_declared_symbol_is_exported():
    lib = _lib.lib()
    names = declared_functions()
    assert len(names) >= 15
    for n in names:
        assert hasattr(lib, n), n
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True, text=True).stdout
    exported = set(re.findall(r" T (tf_\w+)$", out, re.M))
    assert exported == set(names), exported ^ set(names)


def test_ctypes_signatures_cover_header():
    assert sorted(n for n, _, _ in _lib.SIGNATURES) == declared_functions()


STRUCTS = {"tf_device_info_t": _lib.DeviceInfo, "tf_launch_info_t": _lib.LaunchInfo,
           "tf_kernel_resources_t": _lib.KernelResources, "tf_buffer_info_t": _lib.BufferInfo,
           "tf_bench_result_t": _lib.BenchResult}


def test_struct_layouts_match_c(tmp_path):
    src = tmp_path / "sizes.c"
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', "int main(void) {"]
    for cname, py in STRUCTS.items():
        lines.append(f'  printf("{cname} %zu\\n", sizeof({cname}));')
        for f, _ in py._fields_:
            lines.append(f'  printf("{cname}.{f} %zu\\n", offsetof({cname}, {f}));')
    lines += ["  return 0;", "}"]
    src.write_text("\n".join(lines))
    exe = tmp_path / "sizes"
    subprocess.run(["gcc", str(src), "-o", str(exe)], check=True)
    got = dict(l.split() for l in subprocess.run([str(exe)], capture_output=True, text=True).stdout.splitlines())
    import ctypes
    for cname, py in STRUCTS.items():
        assert int(got[cname]) == ctypes.sizeof(py), cname
        for f, _ in py._fields_:
            assert int(got[f"{cname}.{f}"]) == getattr(py, f).offset, (cname, f)


def test_error_codes_and_messages():
    lib = _lib.lib()
    import ctypes
    h = ctypes.c_void_p()
    assert lib.tf_compile(b"x.mlir", b"not a program", b"", ctypes.byref(h)) == -1  # TF_E_PARSE
    assert b"x.mlir:1:1: error" in lib.tf_last_error()
    prog = b"func.func @entry(%a: tensor<4xf32>) -> tensor<4xf32> {\n  %0 = tforge.relu %a : tensor<4xf32> -> tensor<4xf32>\n  return %0 : tensor<4xf32>\n}\n"
    assert lib.tf_compile(b"x.mlir", prog, b"bogus=1", ctypes.byref(h)) == -2  # TF_E_OPTIONS
    assert lib.tf_compile(b"x.mlir", prog, b"tile-k=8", ctypes.byref(h)) == -3  # TF_E_PLAN
    assert lib.tf_compile(b"x.mlir", None, b"", ctypes.byref(h)) == -4  # TF_E_ARG
    assert lib.tf_compile(b"x.mlir", prog, b"", ctypes.byref(h)) == 0
    assert lib.tf_kernel_launch_info(h, 5, None) == -4
    lib.tf_kernel_free(h)


def test_registry_covers_config_space_and_resources():
    reg = _lib.registry()
    staged = {e["cfg"][:5] for e in reg if e["family"] == "staged" and e["cfg"][5:] == (1, 1)}
    assert set(cm.config_space()) <= staged
    ablation = {e["cfg"] for e in reg if e["family"] == "staged" and e["cfg"][5:] != (1, 1)}
    assert (128, 64, 8, 4, 16, 0, 1) in ablation and (128, 64, 8, 4, 16, 1, 0) in ablation
    # every LDS-staged configuration whose threads stage <= 16 vectors per slab
    # has a masked twin (mask-edges)
    import importlib.util
    spec = importlib.util.spec_from_file_location("gen_instances", _lib.PKG / "csrc" / "gen_instances.py")
    gi = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(gi)
    plain = {e["cfg"] for e in reg if e["family"] == "staged" and not e["name"].endswith("_masked")}
    masked = {e["cfg"] for e in reg if e["family"] == "staged" and e["name"].endswith("_masked")}
    assert masked == {c for c in plain if c[5] == 1 and gi.staging_vectors(*c[:5], c[6]) <= 16}
    assert (128, 128, 4, 4, 32, 1, 1) in masked and (64, 64, 2, 2, 64, 1, 1) in masked
    res = json.loads((_lib.PKG / "kernel_resources.json").read_text())
    for e in reg:
        assert e["name"] in res, e["name"]
        assert res[e["name"]]["scratch_bytes"] == 0 and res[e["name"]]["vgpr_spill"] == 0, e["name"]
    for tm in (1, 2, 4, 8):
        for tn in (1, 2, 4, 8):
            assert any(e["family"] == "direct" and e["cfg"][2:4] == (tm, tn) for e in reg)


def _oracle_imports(tree):
    """(function name or None, node) of every import that names the oracle."""
    import ast
    found = []

    def visit(node, func):
        for child in ast.iter_child_nodes(node):
            f = child.name if isinstance(child, (ast.FunctionDef, ast.AsyncFunctionDef)) else func
            if isinstance(child, ast.Import) and any(a.name.split(".")[0] == "oracle" for a in child.names):
                found.append((func, child))
            elif isinstance(child, ast.ImportFrom) and (child.module or "").split(".")[0] == "oracle":
                found.append((func, child))
            visit(child, f)
    visit(tree, None)
    return found


def test_product_does_not_import_the_oracle():
    """Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline may
    import the oracle; nothing in the package does."""
    import ast
    for path in sorted((ROOT / "tensorforge_amd").rglob("*.py")):
        assert not _oracle_imports(ast.parse(path.read_text())), path
    bench = _oracle_imports(ast.parse((ROOT / "bench.py").read_text()))
    assert bench and all(f == "cpu_baseline" for f, _ in bench)
    entry = _oracle_imports(ast.parse((ROOT / "__graft_entry__.py").read_text()))
    assert entry and all(f == "smoke" for f, _ in entry)
