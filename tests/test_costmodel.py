"""The cost model: the reference formula restated exactly (pinned by the
reference's own Stage 9 result rows), and the CDNA4 retarget's invariants."""

import csv
import json
import pathlib

import pytest

from tensorforge_amd import costmodel as cm

GOLDEN = json.loads((pathlib.Path(__file__).resolve().parent / "golden" / "stage9_costmodel.json").read_text())
ROWS = [dict(zip(GOLDEN["columns"], r)) for r in GOLDEN["rows"]]
RESULTS = pathlib.Path(__file__).resolve().parents[1] / "results" / "gpu"


def test_reference_formula_reproduces_stage9_rows():
    """Every 4th row of results/gpu/stage9_autotune.csv (RTX PRO 6000, 188
    SMs) and e2_a6000_autotune.csv (A6000, 84 SMs, 768 GB/s): pred_ms to the
    printed 4 decimals and every printed model term."""
    assert len(ROWS) == 420
    for r in ROWS:
        t = cm.Target("ref", "simt", r["sms"], 2280.0, r["dram_bw"])
        p = cm.predict(tuple(r["cfg"]), r["padded"], {"blocks_per_sm": r["blocks_per_sm"]}, target=t)
        assert f"{p['pred_ms']:.4f}" == f"{r['pred_ms']:.4f}", r
        assert (p["waves"], p["resident"], p["bound"]) == (r["waves"], r["resident"], r["bound"]), r
        assert f"{p['fma_step']:.0f}" == f"{r['fma_step']:.0f}" and f"{p['lds_step']:.0f}" == f"{r['lds_step']:.0f}"
        assert int(p["latency_exposed"]) == r["latency_exposed"]


def test_planted_wrong_latency_breaks_pin():
    t = cm.Target("ref", "simt", 188, 2280.0, 1530e9, latency=500.0)
    bad = sum(f"{cm.predict(tuple(r['cfg']), r['padded'], {'blocks_per_sm': r['blocks_per_sm']}, target=t)['pred_ms']:.4f}"
              != f"{r['pred_ms']:.4f}" for r in ROWS if r["sms"] == 188)
    assert bad > 0


def test_reference_space_has_105_configs():
    assert len(cm.reference_space()) == 105


def test_cdna4_space_is_whole_mfma_waves():
    space = cm.config_space()
    assert len(space) > 100
    for bm, bn, tm, tn, bk in space:
        threads = (bm // tm) * (bn // tn)
        assert threads % 64 == 0 and threads <= 1024
        assert bm % (8 * tm) == 0 and bn % (8 * tn) == 0
        mb = 32 if (8 * tm) % 32 == 0 and (8 * tn) % 32 == 0 else 16
        assert (8 * tm) % mb == 0 and (8 * tn) % mb == 0 and bk % (256 // mb) == 0
        assert 2 * (bm * (bk + 4) + bk * (bn + (8 if mb == 32 else 4))) * 4 <= 160 * 1024
    assert (64, 64, 2, 2, 16) in space  # 16x16 blocks: 16 waves on a 64x64 tile


@pytest.mark.parametrize("shape", [(2048, 2048, 2048), (8192, 1024, 4096), (64, 4096, 4096), (4096, 4096, 256)])
def test_cdna4_model_picks_a_valid_config(shape):
    cfg = cm.default_config(*shape)
    assert cfg[:5] in cm.config_space() and cfg in cm.with_splits(cm.config_space(), *shape)
    p = cm.predict(cfg, cm.padded(cfg, *shape), cm.estimate_info(cfg))
    m, n, k = shape
    # never faster than the FP32 matrix peak
    assert p["pred_ms"] * 1e-3 >= 2.0 * m * n * k / (256 * 256 * 2.4e9) * 0.999


def test_cdna4_model_monotonic_in_k():
    cfg = (128, 128, 4, 4, 64)
    inf = {"blocks_per_sm": 1}
    ts = [cm.predict(cfg, (2048, 2048, k), inf)["pred_ms"] for k in (512, 1024, 2048, 4096)]
    assert ts == sorted(ts)


def test_more_waves_per_simd_hide_the_barrier():
    # same tile, 16 waves (4 per SIMD) vs 4 waves (1 per SIMD): the barrier term shrinks
    a = cm.predict((128, 128, 4, 4, 32), (2048, 2048, 2048), {"blocks_per_sm": 1})
    b = cm.predict((128, 128, 8, 8, 32), (2048, 2048, 2048), {"blocks_per_sm": 1})
    assert a["waves_per_simd"] == 4 and b["waves_per_simd"] == 1


def test_split_k_configurations():
    cfg = (64, 128, 4, 4, 32)
    assert cm.options(cfg + (8,)) == cm.options(cfg) + " split-k=8"
    assert cm.name(cfg + (8,)) == "b64x128-t4x4-k32-s8" and cm.kernel_name(cfg + (8,)) == cm.kernel_name(cfg)
    assert cm.options(cfg + (1,)) == cm.options(cfg)
    # 64 K slabs of 32 at K = 2048: every factor up to 64 fits, 128 does not
    sp = cm.with_splits([cfg], 64, 4096, 2048, (1, 2, 64, 128))
    assert sp == [cfg, cfg + (2,), cfg + (64,)]


def test_split_k_model_terms():
    """Splitting K multiplies the workgroups, divides the K steps, and pays
    the reduction's HBM traffic plus one launch."""
    cfg, shape = (64, 64, 4, 4, 32), (64, 4096, 4096)
    inf = {"blocks_per_sm": 4}
    one = cm.predict(cfg, shape, inf)
    four = cm.predict(cfg + (4,), shape, inf)
    assert four["blocks"] == 4 * one["blocks"] and four["pred_ms"] < one["pred_ms"]
    # a shape that already fills the GPU gains nothing from splitting
    big = (2048, 2048, 2048)
    c = (128, 128, 4, 4, 32)
    assert cm.predict(c + (2,), big, inf)["pred_ms"] > cm.predict(c, big, inf)["pred_ms"]
    assert len(cm.default_config(2048, 2048, 2048)) == 5
    assert cm.splits_of(cm.default_config(64, 4096, 4096)) > 1


def test_config_of_inverts_options():
    from tensorforge_amd.bench import stage9_costmodel as s9
    for cfg in cm.config_space()[::7] + cm.wave_split_space()[::5]:
        for c in {tuple(cfg[:5]), tuple(cfg[:5]) + (4,)} if not cm.wave_split_of(cfg) else {cfg, cfg[:5] + (4, 1)}:
            assert s9.config_of("tforge-gpu-pipeline{" + cm.options(c) + "}") == c
            assert s9.config_of(cm.options(c) + " mask-edges=1") == c


def _summaries():
    rows = []
    for name in ("stage9_summary.csv", "stage9_summary_matmul.csv", "stage9_summary_reference_space.csv"):
        with open(RESULTS / name, newline="") as fh:
            rows += [dict(r, workload="matmul" if "matmul" in name else "mbr") for r in csv.DictReader(fh)]
    return rows


def test_rescore_reproduces_the_recorded_studies():
    """Rescoring the committed per-configuration rows finds, for every study
    in the summaries, the same configurations, the same measured best and
    its time: the rows and the summaries describe the same runs."""
    from tensorforge_amd.bench import stage9_costmodel as s9
    got = {(r[0], r[2], r[3], r[4]): r for r in s9.rescore(RESULTS / "stage9_autotune.csv")}
    for s in _summaries():
        r = got[(s["commit"], s["workload"], s["shape"], int(s["configs_compiled"]))]
        assert (r[7], r[8]) == (s["best"], s["best_ms"]), s


def test_rescore_file_is_the_current_model():
    """results/gpu/stage9_rescore.csv is what the current model scores on the
    committed rows, and the quality the cost model's docstring states holds:
    every pick within 0.90 of the measured best, mean Spearman above 0.8."""
    from tensorforge_amd.bench import stage9_costmodel as s9
    rows = s9.rescore(RESULTS / "stage9_autotune.csv")
    with open(RESULTS / "stage9_rescore.csv", newline="") as fh:
        committed = list(csv.reader(fh))
    assert committed[0] == s9.RESCORE_COLUMNS
    assert committed[1:] == [[str(v) for v in r] for r in rows]
    assert min(float(r[9]) for r in rows) >= 0.90
    assert sum(float(r[12]) for r in rows) / len(rows) > 0.80


def test_rescore_sees_a_planted_inversion(monkeypatch):
    """A model whose prediction is inverted ranks the measurements backwards."""
    from tensorforge_amd.bench import stage9_costmodel as s9
    real = cm.predict
    monkeypatch.setattr(cm, "predict", lambda *a, **k: {"pred_ms": 1.0 / real(*a, **k)["pred_ms"]})
    rows = s9.rescore(RESULTS / "stage9_autotune.csv")
    assert all(float(r[12]) < 0 for r in rows)
