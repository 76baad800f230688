"""bench.py's JSON line on the GPU: the driver's contract (metric and unit from
BASELINE.json, one GPU, steps and warm-up as asked, roofline and parity
objects), run in this process with few steps and without the CPU baseline
and the autotune comparison.  --gpus 2 is refused without touching the GPU."""

import json
import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]


def _line(capsys, monkeypatch, *argv):
    import bench
    monkeypatch.setattr(sys, "argv", ["bench.py", *argv])
    rc = bench.main()
    out = [ln for ln in capsys.readouterr().out.splitlines() if ln.startswith("{")]
    return rc, json.loads(out[-1])


def test_more_than_one_gpu_is_refused(capsys, monkeypatch):
    rc, line = _line(capsys, monkeypatch, "--gpus", "2")
    assert rc == 2 and line["n_gpus"] == 2 and "one GPU" in line["error"]


@pytest.mark.gpu
def test_bench_line_contract(capsys, monkeypatch):
    rc, line = _line(capsys, monkeypatch, "--steps", "5", "--warmup", "2", "--no-cpu-baseline",
                     "--no-autotune-compare")
    baseline = json.loads((ROOT / "BASELINE.json").read_text())
    assert rc == 0
    assert line["metric"] == baseline["metric"] and line["unit"] == "TFLOP/s"
    assert (line["n_gpus"], line["steps"], line["warmup"]) == (1, 5, 2)
    assert line["higher_is_better"] is True and line["dtype"] == "f32" and line["vs_baseline"] is None
    assert 0.0 < line["value"] < 157.3
    assert line["value"] == pytest.approx(2.0 * 2048 ** 3 / (line["ms_per_step"] * 1e-3) / 1e12, rel=1e-3)
    roof = line["roofline"]
    assert roof["bound"] == "mfma" and roof["peak"] == 157.3 and roof["unit"] == "TFLOP/s"
    assert roof["frac"] == pytest.approx(roof["achieved"] / roof["peak"], abs=1e-4)
    parity = line["parity"]
    assert parity["pass"] and parity["rows_checked"] == 2048 and parity["mask_mismatches"] == 0
    assert parity["err_over_bound"] <= 1.0
    assert line["config"]["kernel"].startswith("tf_staged_") and line["cpu_baseline"] is None
