#!/usr/bin/env python3
"""Stage 9 on MI355X: the CDNA4 cost model versus empirical autotuning, fused mbr.

Same procedure, CSV rows and summary columns as the reference's
bench/stage9_costmodel.py:1-155.  For each shape:
  1. compile every configuration of costmodel.config_space(); configurations
     that fail to compile are recorded and excluded,
  2. cost model: read VGPRs / LDS / occupancy (HIP occupancy API) and predict
     the time of each configuration; the model's pick is the minimum,
  3. autotuner: check (one FP64 reference per shape) and time every
     configuration; the autotuner's pick is the fastest measured,
  4. report the model pick relative to the best, raw and clock-adjusted, the
     Spearman rank correlation (with --split-k, every configuration is also
     tried with each split-K factor, a backend option), and record the best configuration in
     tensorforge_amd/tuned_configs.json (read by bench.py and tuned_options()).

  python -m tensorforge_amd.bench.stage9_costmodel --shapes 2048x2048x2048 \\
      --csv results/gpu/stage9_autotune.csv --summary results/gpu/stage9_summary.csv
"""

import argparse
import csv
import json
import pathlib
import sys
import time

import numpy as np

from tensorforge_amd import _lib
from tensorforge_amd import costmodel as cm
from tensorforge_amd import provenance
from tensorforge_amd import tforge_cpu as tc
from tensorforge_amd import tforge_gpu as tg

SHAPES = [(1024, 1024, 1024), (2048, 2048, 2048), (4096, 4096, 4096), (1536, 1536, 1536),
          (2560, 2560, 2560), (1000, 1000, 1000), (777, 1111, 333), (3000, 2000, 1000)]
TUNED = pathlib.Path(tg.__file__).resolve().parent / "tuned_configs.json"


def spearman(x, y):
    rx = np.argsort(np.argsort(x))
    ry = np.argsort(np.argsort(y))
    return float(np.corrcoef(rx, ry)[0, 1])


def record_tuned(path, workload, m, n, k, cfg, ms, extra, suffix=""):
    path = pathlib.Path(path)
    table = json.loads(path.read_text()) if path.exists() else {}
    table[f"{workload}/{m}x{n}x{k}"] = {"options": cm.options(cfg) + suffix, "config": cm.name(cfg), "median_ms": ms,
                                         "tflops": 2.0 * m * n * k / (ms * 1e-3) / 1e12, **extra}
    path.write_text(json.dumps(table, indent=1, sort_keys=True) + "\n")


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--csv", default="results/gpu/stage9_autotune.csv")
    ap.add_argument("--summary", default="results/gpu/stage9_summary.csv")
    ap.add_argument("--shapes", default="")
    ap.add_argument("--workload", default="mbr", choices=("mbr", "matmul"))
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--reps", type=int, default=100)
    ap.add_argument("--space", choices=("cdna4", "reference"), default="cdna4")
    ap.add_argument("--top", type=int, default=0, help="time only the N best-predicted configurations")
    ap.add_argument("--split-k", default="1",
                    help="split-K factors to cross with the configuration grid, e.g. 1,2,4,8 (backend option)")
    ap.add_argument("--tuned", default=str(TUNED), help="JSON table the best configuration is recorded in")
    ap.add_argument("--no-record", action="store_true", help="do not record the best configuration")
    ap.add_argument("--mask-edges", action="store_true",
                    help="run every configuration on the true shape with mask-edges (no pad copies)")
    ap.add_argument("--prewarm", type=int, default=500,
                    help="untimed launches of the first configuration per shape before timing (GPU clock settles)")
    args = ap.parse_args(argv)
    shapes = SHAPES
    if args.shapes:
        shapes = [tuple(int(v) for v in s.split("x")) for s in args.shapes.split(",")]
    base = provenance.common()
    out = provenance.CsvWriter(args.csv)
    summ_path = pathlib.Path(args.summary)
    summ_path.parent.mkdir(parents=True, exist_ok=True)
    new = not summ_path.exists()
    summ = open(summ_path, "a", newline="")
    sw = csv.writer(summ)
    if new:
        sw.writerow(["commit", "job_id", "date", "shape", "configs_total", "configs_compiled",
                     "model_pick", "model_pick_ms", "model_pick_pct", "best", "best_ms", "best_pct",
                     "ratio_raw", "ratio_clock_adjusted", "model_rank_of_best", "measured_rank_of_model_pick",
                     "spearman_pred_vs_measured", "model_cost_s", "autotune_cost_s"])
    base_space = cm.config_space() if args.space == "cdna4" else cm.reference_space()
    split_factors = tuple(int(v) for v in args.split_k.split(","))
    wl = args.workload
    suffix = " mask-edges=1" if args.mask_edges else ""
    for m, n, k in shapes:
        space = cm.with_splits(base_space, m, n, k, split_factors)
        tag = f"stage9/{m}x{n}x{k}"
        t0 = time.time()
        compiled, failed = [], []
        for cfg in space:
            try:
                d, launch = tg.compile_kernel(wl, m, n, k, cm.options(cfg) + suffix, tag=f"{tag}/{cm.name(cfg)}")
                compiled.append((cfg, d, launch))
            except RuntimeError as e:  # recorded, config excluded
                failed.append((cfg, str(e).splitlines()[0][:200]))
        t_compile = time.time() - t0
        for c, err in failed:
            print(f"  compile failed {cm.name(c)}: {err}", flush=True)

        t1 = time.time()
        preds = {}
        for c, d, l in compiled:
            inf = tg.info(wl, m, n, k, d, l)
            preds[c] = (cm.predict(c, cm.padded(c, m, n, k), inf), inf)  # a masked kernel runs the padded tiles
        t_model = time.time() - t1
        pick = min(preds, key=lambda c: preds[c][0]["pred_ms"])
        if args.top:
            # Model-guided autotuning: time only the best-predicted configurations.
            keep = set(sorted(preds, key=lambda c: preds[c][0]["pred_ms"])[:args.top])
            compiled = [(c, d, l) for c, d, l in compiled if c in keep]

        ins = tc.make_inputs(wl, m, n, k)
        arrays = [np.ascontiguousarray(v) for v in ins.values()]
        a64, b64 = ins["a"].astype(np.float64), ins["b"].astype(np.float64)
        ref, mag, steps = a64 @ b64, np.abs(a64) @ np.abs(b64), k
        if wl == "mbr":
            bias64 = ins["bias"].astype(np.float64)
            ref, mag, steps = np.maximum(ref + bias64, 0.0), mag + np.abs(bias64), k + 1
        gamma = steps * tc.F32_EPS / (1 - steps * tc.F32_EPS)
        bound = gamma * mag + np.finfo(np.float32).tiny
        del a64, b64, mag
        t2 = time.time()
        meas = {}
        got = np.empty((m, n), np.float32)
        if args.prewarm and compiled:
            c0, d0, l0 = compiled[0]
            tg.bench(wl, m, n, k, d0, l0, warmup=args.prewarm, reps=1)
        for c, d, l in compiled:
            kern = _lib.Kernel((d / "input.mlir").read_text(), l["options"], str(d / "input.mlir"))
            logical = None if tuple(l["padded"]) == (m, n, k) else (m, n, k)
            kern.run(arrays, got, logical=logical)
            eob = float(np.nanmax(np.abs(got.astype(np.float64) - ref) / bound))
            ok = not np.isnan(got).any() and eob <= 1.0
            if not ok:
                print(f"  [FAIL] {cm.name(c)} err/bound={eob}", flush=True)
                continue
            r = tg.bench(wl, m, n, k, d, l, warmup=args.warmup, reps=args.reps)
            gf = 2.0 * m * n * k / (r["median_ms"] * 1e-3) / 1e9
            clk = r["sm_clock_median_mhz"]
            pct = 100.0 * gf / tg.fp32_peak_gflops(clk if clk > 0 else tg.PEAK_CLOCK_MHZ)
            meas[c] = (r, gf, pct, eob)
            p, inf = preds[c]
            out.row(**base, device=r["gpu"], workload=wl, shape=f"{m}x{n}x{k}", dtype="f32",
                    pipeline=f"tforge-gpu-pipeline{{{cm.options(c) + suffix}}}",
                    params=(f"{cm.name(c)}; grid={r['grid']} block={r['block']} padded={r['padded']}; "
                            f"regs={inf['regs']} smem={inf['static_smem']} blocks/SM={inf['blocks_per_sm']} "
                            f"occ={inf['theo_occupancy']}"),
                    threads="", warmup=r["warmup"], reps=r["reps"], median_ms=r["median_ms"],
                    min_ms=r["min_ms"], std_ms=r["std_ms"], metric="GFLOP/s", metric_value=gf,
                    sm_clock_median_mhz=clk, clock_adjusted_metric=f"{pct:.2f}% of FP32 matrix peak at median clock",
                    alloc_bytes_per_call="", correctness=f"err/bound={eob:.3g}",
                    notes=(f"model: pred_ms={p['pred_ms']:.4f} waves={p['waves']} resident={p['resident']} "
                           f"bound={p['bound']} fma_step={p['fma_step']:.0f} lds_step={p['lds_step']:.0f} "
                           f"latency_exposed={int(p['latency_exposed'])}"))
            print(f"  {cm.name(c):>18} {r['median_ms']:.4f} ms {gf / 1e3:7.2f} TFLOP/s  pred {p['pred_ms']:.4f} ms",
                  flush=True)
        t_tune = time.time() - t2
        best = min(meas, key=lambda c: meas[c][0]["median_ms"])
        ok_cfgs = list(meas)
        pred_ms = [preds[c][0]["pred_ms"] for c in ok_cfgs]
        meas_ms = [meas[c][0]["median_ms"] for c in ok_cfgs]
        rho = spearman(pred_ms, meas_ms)
        order_pred = sorted(ok_cfgs, key=lambda c: preds[c][0]["pred_ms"])
        order_meas = sorted(ok_cfgs, key=lambda c: meas[c][0]["median_ms"])
        if pick not in meas:
            print(f"  model pick {cm.name(pick)} failed correctness; using next prediction", flush=True)
            pick = order_pred[0]
        rp, gp, pp, _ = meas[pick]
        rb, gb, pb, _ = meas[best]
        sw.writerow([base["commit"], base["job_id"], base["date"], f"{m}x{n}x{k}", len(space), len(preds),
                     cm.name(pick), f"{rp['median_ms']:.6f}", f"{pp:.2f}", cm.name(best), f"{rb['median_ms']:.6f}",
                     f"{pb:.2f}", f"{rb['median_ms'] / rp['median_ms']:.3f}", f"{pp / pb:.3f}",
                     order_pred.index(best) + 1, order_meas.index(pick) + 1, f"{rho:.3f}",
                     f"{t_compile + t_model:.1f}", f"{t_compile + t_tune:.1f}"])
        summ.flush()
        if not args.no_record:
            record_tuned(args.tuned, wl, m, n, k, best, rb["median_ms"],
                         {"model_pick": cm.name(pick), "model_pick_ms": rp["median_ms"],
                          "speedup_over_model_pick": rp["median_ms"] / rb["median_ms"], "spearman": rho}, suffix)
        print(f"{m}x{n}x{k}: model {cm.name(pick)} {rp['median_ms']:.4f} ms ({pp:.1f}%), "
              f"best {cm.name(best)} {rb['median_ms']:.4f} ms ({pb:.1f}%), ratio raw "
              f"{rb['median_ms'] / rp['median_ms']:.3f} clock-adj {pp / pb:.3f}, spearman {rho:.3f}, "
              f"compiled {len(compiled)}/{len(space)}, model {t_compile + t_model:.0f} s, "
              f"autotune {t_compile + t_tune:.0f} s", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
