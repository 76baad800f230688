"""Extract known-answer fixtures from the TensorForge reference's own result files.

Reads only data files the reference ships (CSV), never its code, and writes
small JSON fixtures next to this script:

  e1_known_answers.json   results/numerics/e1.csv: per workload x shape, the
                          error statistics of the no-FMA closed form
                          (variant cpu-scalar) and of the sequential-FMA closed
                          form (variant gpu-naive), and the count of outputs on
                          which the two differ bitwise.
  stage8_err_bound.json   the err/bound of the TensorForge kernels in
                          results/gpu/stage8.csv and stage7.csv (identical for
                          every TF variant of a shape, since they are bitwise
                          equal), per workload x shape.
  cpu_err_bound.json      the err/bound of the reference's CPU pipelines in
                          results/cpu/stage4.csv and stage6_best.csv per
                          workload x shape: the default scalar pipeline
                          (params baseline / scalar-baseline, no FMA, m-n-k
                          loops) and the reg-tile=6,16,4 AVX2 FMA kernel
                          (params vec-r6x16x4).
  stage9_costmodel.json   every 4th row of results/gpu/stage9_autotune.csv and
                          e2_a6000_autotune.csv reduced to the cost model's
                          inputs (config, padded shape, blocks/SM) and outputs
                          (pred_ms, waves, resident, bound, fma_step, lds_step,
                          latency_exposed).

Usage: python tests/golden/make_golden.py [/root/reference]
"""

import csv
import json
import pathlib
import re
import sys

HERE = pathlib.Path(__file__).resolve().parent


def e1(ref):
    rows = list(csv.DictReader(open(ref / "results/numerics/e1.csv")))
    out = {}
    for r in rows:
        if r["variant"] not in ("cpu-scalar", "gpu-naive"):
            continue
        key = f"{r['workload']}/{r['shape']}"
        form = "nofma" if r["variant"] == "cpu-scalar" else "fma"
        out.setdefault(key, {})[form] = {
            "max_abs_err": r["max_abs_err"], "rms_err": r["rms_err"],
            "max_err_over_bound": r["max_err_over_bound"],
            "bitwise_diff_vs_nofma": int(r["bitwise_diff_vs_cpu_scalar"]),
            "source": f"results/numerics/e1.csv variant={r['variant']}"}
    return out


def err_bound(ref):
    out = {}
    for name in ("stage7.csv", "stage8.csv"):
        for r in csv.DictReader(open(ref / "results/gpu" / name)):
            if not r["pipeline"].startswith("tforge-gpu-pipeline"):
                continue
            m = re.search(r"err/bound=([0-9.e+-]+)", r["correctness"])
            key = f"{r['workload']}/{r['shape']}"
            val = m.group(1)
            prev = out.get(key)
            if prev is not None and prev["err_over_bound"] != val:
                raise SystemExit(f"TF variants disagree at {key}: {prev} vs {val}")
            out[key] = {"err_over_bound": val, "source": f"results/gpu/{name}"}
    return out


def cpu_err_bound(ref):
    out = {}
    forms = {"baseline": "scalar", "scalar-baseline": "scalar", "vec-r6x16x4": "vec6x16"}
    for name in ("stage4.csv", "stage6_best.csv"):
        for r in csv.DictReader(open(ref / "results/cpu" / name)):
            form = forms.get(r["params"])
            if r["workload"] not in ("matmul", "mbr") or form is None:
                continue
            val = re.search(r"err/bound=([0-9.e+-]+)", r["correctness"]).group(1)
            entry = out.setdefault(f"{r['workload']}/{r['shape']}", {})
            if form in entry and entry[form]["err_over_bound"] != val:
                raise SystemExit(f"CPU rows disagree at {r['workload']}/{r['shape']} {form}")
            entry[form] = {"err_over_bound": val, "source": f"results/cpu/{name} params={r['params']}"}
    return out


def costmodel(ref):
    rows = []
    for name, sms, bw in (("stage9_autotune.csv", 188, 1530e9), ("e2_a6000_autotune.csv", 84, 768e9)):
        for r in csv.DictReader(open(ref / "results/gpu" / name)):
            cfg = re.match(r"b(\d+)x(\d+)-t(\d+)x(\d+)-k(\d+);", r["params"])
            padded = re.search(r"padded=(\d+)x(\d+)x(\d+)", r["params"])
            bps = re.search(r"blocks/SM=(\d+)", r["params"])
            notes = dict(kv.split("=") for kv in r["notes"].replace("model: ", "").split())
            rows.append({
                "file": name, "sms": sms, "dram_bw": bw,
                "cfg": [int(x) for x in cfg.groups()],
                "padded": [int(x) for x in padded.groups()],
                "blocks_per_sm": int(bps.group(1)),
                "pred_ms": float(notes["pred_ms"]), "waves": int(notes["waves"]),
                "resident": int(notes["resident"]), "bound": notes["bound"],
                "fma_step": float(notes["fma_step"]), "lds_step": float(notes["lds_step"]),
                "latency_exposed": int(notes["latency_exposed"])})
    return rows


def main():
    ref = pathlib.Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
    (HERE / "e1_known_answers.json").write_text(json.dumps(e1(ref), indent=1, sort_keys=True) + "\n")
    (HERE / "stage8_err_bound.json").write_text(json.dumps(err_bound(ref), indent=1, sort_keys=True) + "\n")
    (HERE / "cpu_err_bound.json").write_text(json.dumps(cpu_err_bound(ref), indent=1, sort_keys=True) + "\n")
    rows = costmodel(ref)[::4]  # every 4th row keeps the fixture small; all shapes stay covered
    keys = list(rows[0])
    (HERE / "stage9_costmodel.json").write_text(
        json.dumps({"columns": keys, "rows": [[r[k] for k in keys] for r in rows]}, separators=(",", ":")) + "\n")
    print("wrote", sorted(p.name for p in HERE.glob("*.json")))


if __name__ == "__main__":
    main()
