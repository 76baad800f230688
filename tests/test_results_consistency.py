"""The committed MI355X result tables agree with the reference's own numbers
where the arithmetic is the same (CPU only: reads committed CSVs).

results/numerics/e1_mi355x.csv is written on the GPU by
tensorforge_amd/bench/e1_numerics.py; its gpu-naive rows (the direct kernel:
one FMA per k in k order) and cpu-scalar rows must equal the reference's E1
rows (results/numerics/e1.csv, kept in tests/golden/e1_known_answers.json)
in every printed statistic and bitwise-difference count."""

import csv
import json
import pathlib

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
E1 = json.loads((ROOT / "tests" / "golden" / "e1_known_answers.json").read_text())
OURS = ROOT / "results" / "numerics" / "e1_mi355x.csv"


def _rows():
    if not OURS.exists():
        pytest.skip("no MI355X E1 table committed")
    return {(r["workload"], r["shape"], r["variant"]): r for r in csv.DictReader(OURS.open())}


@pytest.mark.parametrize("key", sorted(E1))
@pytest.mark.parametrize("variant,form", [("gpu-naive", "fma"), ("cpu-scalar", "nofma")])
def test_e1_rows_equal_reference(key, variant, form):
    workload, shape = key.split("/")
    row = _rows()[(workload, shape, variant)]
    want = E1[key][form]
    for col in ("max_abs_err", "rms_err", "max_err_over_bound"):
        assert row[col] == want[col], (col, row[col], want[col])
    assert int(row["bitwise_diff_vs_cpu_scalar"]) == want["bitwise_diff_vs_nofma"]


def test_e1_every_variant_within_bound():
    for (wl, shape, variant), r in _rows().items():
        assert float(r["max_err_over_bound"]) <= 1.0, (wl, shape, variant)
