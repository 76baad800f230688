"""The staged kernel's A staging order (StagedGemm::a_item), checked on the
host: tests/staging_order_driver.cpp is compiled for the host only against
the real header and checks, per configuration, that every (row, column
vector) of the slab is staged exactly once, that every 8-lane pass of a
128-bit LDS write covers 8 distinct 4-bank groups of the padded tile, and
that one wave's 64 items are whole rows of the slab (whole-row-segment
global loads).  No GPU needed."""

import pathlib
import shutil
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"


def test_a_staging_order_is_a_conflict_free_bijection(tmp_path):
    if not pathlib.Path(HIPCC).exists():
        pytest.skip("needs hipcc")
    exe = tmp_path / "staging_order"
    subprocess.run([HIPCC, "-x", "hip", "--cuda-host-only", "-std=c++17", "-O1", "-I", str(ROOT / "include"),
                    "-I", str(ROOT / "tensorforge_amd" / "csrc"), str(ROOT / "tests" / "staging_order_driver.cpp"),
                    "-o", str(exe)], check=True, capture_output=True, timeout=300)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stdout + r.stderr
    lines = r.stdout.strip().splitlines()
    assert lines[-1] == "ok"
    assert len(lines) == 16 and all("0 bank-group collisions" in ln for ln in lines[:-1])
