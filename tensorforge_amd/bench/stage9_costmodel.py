#!/usr/bin/env python3
"""How well the CDNA4 cost model picks a configuration, against measuring them
all: model-predicted versus measured time of every configuration of the fused
mbr (or matmul) kernel, per shape, and the autotuner's record of the best.

Per shape the study builds one `Candidate` per configuration (x split-K
factor with --split-k; the wave-split configurations too with --wave-split)
and fills it in three passes:

  compile   tf_compile; a configuration without an instantiation is recorded
            with the compiler's reason and drops out
  predict   costmodel.predict on the kernel's resources (HIP occupancy API)
  measure   one checked run on the seeded inputs against a single FP64
            reference of the shape (err/bound <= 1, exact ReLU masks), then
            tf_bench; with --top N only the N best-predicted are measured

  throughput  (--objective throughput) every timed configuration's rate with
            launches issued back to back, as bench.py measures its value:
            one window of 50 launches after 10 untimed ones, then the six
            best alternate in ten rounds of ~25 ms windows (20-200 launches)
            and their median windows decide

and then compares: the model's pick (least predicted time, passing) against
the measured best, raw and clock-adjusted; each one's rank in the other's
order; and the Spearman rank correlation of predicted and measured times
(average ranks for ties, scipy.stats.spearmanr).  The per-configuration rows
and the summary columns are the reference's Stage 9 tables
(bench/stage9_costmodel.py), so both read the same way.  Unless --no-record,
the best configuration goes into tensorforge_amd/tuned_configs.json, which
bench.py and costmodel.tuned_options read: the least per-launch median
(tf_bench: one event pair per rep, the GPU idle between reps), or with
--objective throughput the least back-to-back time.  The two orders differ
where a configuration's ramp at the start and end of a launch, which back to
back launches overlap, sets it apart: at 2048^3 the 4-wave 64x128 tiles lead
per launch and the 128x128 thread-tile 8,8 tile back to back.

  python -m tensorforge_amd.bench.stage9_costmodel --shapes 2048x2048x2048 \\
      --csv results/gpu/stage9_autotune.csv --summary results/gpu/stage9_summary.csv
"""

import argparse
import csv
import dataclasses
import json
import pathlib
import sys
import time

from scipy import stats

from tensorforge_amd import costmodel as cm
from tensorforge_amd import provenance
from tensorforge_amd import tforge_gpu as tg
from tensorforge_amd.bench import harness

DEFAULT_SHAPES = [(1024, 1024, 1024), (2048, 2048, 2048), (4096, 4096, 4096), (1536, 1536, 1536),
                  (2560, 2560, 2560), (1000, 1000, 1000), (777, 1111, 333), (3000, 2000, 1000)]
TUNED = pathlib.Path(tg.__file__).resolve().parent / "tuned_configs.json"
SUMMARY_COLUMNS = ["commit", "job_id", "date", "shape", "configs_total", "configs_compiled",
                   "model_pick", "model_pick_ms", "model_pick_pct", "best", "best_ms", "best_pct",
                   "ratio_raw", "ratio_clock_adjusted", "model_rank_of_best", "measured_rank_of_model_pick",
                   "spearman_pred_vs_measured", "model_cost_s", "autotune_cost_s"]


@dataclasses.dataclass
class Candidate:
    cfg: tuple
    options: str
    kdir: pathlib.Path = None
    launch: dict = None
    rejected: str = ""
    info: dict = None        # resources from the occupancy API
    pred: dict = None        # costmodel.predict
    result: "harness.Result" = None
    window_ms: float = None  # back-to-back ms per launch (throughput objective)

    @property
    def name(self):
        return cm.name(self.cfg)

    @property
    def measured_ms(self):
        return self.result.timing["median_ms"] if self.result and self.result.timing else None

    def pct_at_clock(self):
        return self.result.shares()[1]


class ShapeStudy:
    def __init__(self, args, workload, m, n, k):
        self.args, self.workload, self.shape = args, workload, (m, n, k)
        space = cm.config_space() if args.space == "cdna4" else cm.reference_space()
        if args.wave_split:
            space = space + cm.wave_split_space()
        factors = tuple(int(v) for v in args.split_k.split(","))
        suffix = " mask-edges=1" if args.mask_edges else ""
        self.candidates = [Candidate(cfg, cm.options(cfg) + suffix) for cfg in cm.with_splits(space, m, n, k, factors)]
        self.seconds = {}

    def _timed(self, phase, fn):
        t0 = time.time()
        fn()
        self.seconds[phase] = time.time() - t0

    def compile(self):
        m, n, k = self.shape
        for c in self.candidates:
            try:
                c.kdir, c.launch = tg.compile_kernel(self.workload, m, n, k, c.options,
                                                     tag=f"stage9/{m}x{n}x{k}/{c.name}")
            except RuntimeError as e:
                c.rejected = str(e).splitlines()[0][:200]
                print(f"  compile failed {c.name}: {c.rejected}", flush=True)

    def predict(self):
        m, n, k = self.shape
        for c in self.compiled():
            c.info = tg.info(self.workload, m, n, k, c.kdir, c.launch)
            # a masked kernel still runs whole tiles, so the model sees the padded problem
            c.pred = cm.predict(c.cfg, cm.padded(c.cfg, m, n, k), c.info)

    def measure(self):
        m, n, k = self.shape
        pool = sorted(self.compiled(), key=lambda c: c.pred["pred_ms"])
        if self.args.top:
            pool = pool[:self.args.top]
        problem = harness.Problem(self.workload, m, n, k)
        if self.args.prewarm and pool:  # bring the GPU to its working clock before the first timing
            tg.bench(self.workload, m, n, k, pool[0].kdir, pool[0].launch, warmup=self.args.prewarm, reps=1)
        for c in pool:
            job = harness.Job(self.workload, m, n, k, c.name, c.options)
            c.result = harness.measure(job, problem, self.args.warmup, self.args.reps, tag=f"stage9/{m}x{n}x{k}")
            if not c.result.passed:
                print(f"  [FAIL] {c.name} err/bound={c.result.verdict['err_over_bound']}", flush=True)
                continue
            print(f"  {c.name:>18} {c.measured_ms:.4f} ms {c.result.rate()[1] / 1e3:7.2f} TFLOP/s  "
                  f"pred {c.pred['pred_ms']:.4f} ms", flush=True)

    def throughput(self, warm=10, steps=50, finalists=6, rounds=10, final_window_s=0.025):
        """Back-to-back ms per launch of every timed candidate (one window of
        `steps` launches after `warm` untimed ones), then of the `finalists`
        best again over `rounds` alternating rounds (first to last, then last
        to first), each candidate's median window; a final window spans about
        `final_window_s` of launches (20 to 200), since finalists lie within
        a percent of each other.  Inputs are uniform [-1, 1]
        device buffers of the shapes the kernel takes; launches go straight to
        tf_launch, so the host issues them faster than the shortest kernel
        here runs."""
        import statistics
        import torch
        from tensorforge_amd import _lib
        dev = torch.device("cuda:0")
        gen = torch.Generator(device=dev)
        gen.manual_seed(1234)
        stream = torch.cuda.current_stream()
        pool, bufs, launchers = self.timed(), {}, {}

        def launcher(c):
            kern = tg._kernel(c.kdir, c.launch)
            shapes = tuple(tuple(b["shape"]) for b in kern.buffers())
            if shapes not in bufs:
                bufs[shapes] = [torch.empty(s, device=dev).uniform_(-1, 1, generator=gen) for s in shapes]
            arr = (_lib.P * len(shapes))(*[_lib.P(t.data_ptr()) for t in bufs[shapes]])
            fn, h, st = _lib.lib().tf_launch, kern.h, _lib.P(stream.cuda_stream)

            def window(count):
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record(stream)
                bad = sum(fn(h, arr, st) < 0 for _ in range(count))
                b.record(stream)
                b.synchronize()
                if bad:
                    raise RuntimeError(f"tf_launch failed for {c.name}: {_lib.lib().tf_last_error().decode()}")
                return a.elapsed_time(b) / count
            return kern, window

        for c in pool:
            launchers[c.name] = launcher(c)
            _, window = launchers[c.name]
            window(warm)
            c.window_ms = window(steps)
        final = sorted(pool, key=lambda c: c.window_ms)[:finalists]
        times = {c.name: [] for c in final}
        long_steps = max(20, min(200, int(final_window_s / (final[0].window_ms * 1e-3))))
        for r in range(rounds):
            for c in (final if r % 2 == 0 else final[::-1]):
                _, window = launchers[c.name]
                window(warm)
                times[c.name].append(window(long_steps))
        for c in final:
            c.window_ms = statistics.median(times[c.name])
            print(f"  {c.name:>18} back to back {c.window_ms * 1e3:.1f} us/launch "
                  f"(rounds {', '.join(f'{t * 1e3:.1f}' for t in times[c.name])})", flush=True)
        self.finalists = final

    def compiled(self):
        return [c for c in self.candidates if not c.rejected]

    def timed(self):
        return [c for c in self.candidates if c.measured_ms is not None]

    def run(self):
        self._timed("compile", self.compile)
        self._timed("predict", self.predict)
        self._timed("measure", self.measure)
        if self.args.objective == "throughput" and self.timed():
            self._timed("throughput", self.throughput)
        return self

    def chosen(self, best):
        """The configuration the tuned table records: `best` (least per-launch
        median) or, with the throughput objective, the least back-to-back time
        among the finalists."""
        if self.args.objective != "throughput":
            return best
        return min(self.finalists, key=lambda c: c.window_ms)

    def row_of(self, c):
        p, inf = c.pred, c.info
        return c.result.row(params=(f"{c.name}; grid={c.result.timing['grid']} block={c.result.timing['block']} "
                                    f"padded={c.result.timing['padded']}; regs={inf['regs']} "
                                    f"smem={inf['static_smem']} blocks/SM={inf['blocks_per_sm']} "
                                    f"occ={inf['theo_occupancy']}"),
                            notes=(f"model: pred_ms={p['pred_ms']:.4f} waves={p['waves']} resident={p['resident']} "
                                   f"bound={p['bound']} fma_step={p['fma_step']:.0f} lds_step={p['lds_step']:.0f} "
                                   f"latency_exposed={int(p['latency_exposed'])}"
                                   + (f"; back_to_back_ms={c.window_ms:.6f}" if c.window_ms is not None else "")))

    def summary(self, base):
        """The summary row (SUMMARY_COLUMNS) and the (pick, best) candidates."""
        timed = self.timed()
        by_pred = sorted(timed, key=lambda c: c.pred["pred_ms"])
        by_meas = sorted(timed, key=lambda c: c.measured_ms)
        pick = min(self.compiled(), key=lambda c: c.pred["pred_ms"])
        if pick not in timed:  # the model's first choice failed its check (or was not measured)
            print(f"  model pick {pick.name} has no measurement; using the best-predicted measured one", flush=True)
            pick = by_pred[0]
        best = by_meas[0]
        rho = stats.spearmanr([c.pred["pred_ms"] for c in timed], [c.measured_ms for c in timed]).statistic \
            if len(timed) > 1 else float("nan")
        m, n, k = self.shape
        row = [base["commit"], base["job_id"], base["date"], f"{m}x{n}x{k}", len(self.candidates),
               len(self.compiled()), pick.name, f"{pick.measured_ms:.6f}", f"{pick.pct_at_clock():.2f}", best.name,
               f"{best.measured_ms:.6f}", f"{best.pct_at_clock():.2f}", f"{best.measured_ms / pick.measured_ms:.3f}",
               f"{pick.pct_at_clock() / best.pct_at_clock():.3f}", by_pred.index(best) + 1,
               by_meas.index(pick) + 1, f"{float(rho):.3f}",
               f"{self.seconds['compile'] + self.seconds['predict']:.1f}",
               f"{self.seconds['compile'] + self.seconds['measure']:.1f}"]
        return row, pick, best, float(rho)


def record_best(path, workload, shape, best, pick, rho, objective="latency", source=None):
    """Records `best` for (workload, shape).  "tflops" is at the objective's
    time: the per-launch median, or the back-to-back time (window_ms).
    `source` names the run behind the entry -- the commit the library was
    built from, the date and the summary file whose row (commit, date, shape)
    this study wrote -- so every recorded configuration traces to a row."""
    path = pathlib.Path(path)
    table = json.loads(path.read_text()) if path.exists() else {}
    m, n, k = shape
    ms = best.window_ms if objective == "throughput" else best.measured_ms
    entry = {
        "options": best.options, "config": best.name, "median_ms": best.measured_ms,
        "tflops": 2.0 * m * n * k / (ms * 1e-3) / 1e12, "model_pick": pick.name,
        "model_pick_ms": pick.measured_ms, "speedup_over_model_pick": pick.measured_ms / best.measured_ms,
        "spearman": rho, "objective": objective}
    if source:
        entry.update(source)
    if objective == "throughput":
        entry["back_to_back_ms"] = best.window_ms
    table[f"{workload}/{m}x{n}x{k}"] = entry
    path.write_text(json.dumps(table, indent=1, sort_keys=True) + "\n")


def config_of(pipeline):
    """(BM, BN, TM, TN, BK[, S[, 1]]) of a table row's pipeline text
    (`tforge-gpu-pipeline{...}`, or the bare option string): the inverse of
    costmodel.options."""
    text = pipeline[pipeline.find("{") + 1:pipeline.rfind("}")] if "{" in pipeline else pipeline
    kv = dict(tok.split("=", 1) for tok in text.split() if "=" in tok)
    bm, bn = (int(v) for v in kv["block-tile"].split(","))
    tm, tn = (int(v) for v in kv["thread-tile"].split(","))
    cfg = (bm, bn, tm, tn, int(kv["tile-k"]))
    s = int(kv.get("split-k", "1"))
    if kv.get("wave-split-k") == "1":
        return cfg + (s, 1)
    return cfg + (s,) if s > 1 else cfg


RESCORE_COLUMNS = ["commit", "date", "workload", "shape", "configs", "model_pick", "model_pick_ms", "best", "best_ms",
                   "ratio_raw", "model_rank_of_best", "measured_rank_of_model_pick", "spearman_pred_vs_measured"]


def rescore(csv_path, out_path=None):
    """Scores the current cost model on measured studies, without a GPU: the
    rows of `csv_path` grouped by study (workload, shape, commit, date), each
    configuration predicted from its measured blocks per CU (the `params`
    column), then the model's pick among the measured configurations against
    the measured best and the Spearman correlation of predicted and measured
    times, as a study's summary row computes them.  Returns the rows
    (RESCORE_COLUMNS) and writes them to `out_path` if given."""
    studies = {}
    with open(csv_path, newline="") as fh:
        for r in csv.DictReader(fh):
            key = (r["commit"], r["date"], r["workload"], r["shape"])
            bps = int(r["params"].split("blocks/SM=")[1].split()[0])
            studies.setdefault(key, []).append((config_of(r["pipeline"]), bps, float(r["median_ms"])))
    out = []
    for (commit, date, workload, shape), rows in sorted(studies.items(), key=lambda kv: kv[0][1]):
        m, n, k = (int(v) for v in shape.split("x"))
        pred = [cm.predict(c, cm.padded(c, m, n, k), {"blocks_per_sm": b})["pred_ms"] for c, b, _ in rows]
        meas = [ms for _, _, ms in rows]
        by_pred = sorted(range(len(rows)), key=lambda i: pred[i])
        by_meas = sorted(range(len(rows)), key=lambda i: meas[i])
        pick, best = by_pred[0], by_meas[0]
        rho = stats.spearmanr(pred, meas).statistic if len(rows) > 1 else float("nan")
        out.append([commit, date, workload, shape, len(rows), cm.name(rows[pick][0]), f"{meas[pick]:.6f}",
                    cm.name(rows[best][0]), f"{meas[best]:.6f}", f"{meas[best] / meas[pick]:.3f}",
                    by_pred.index(best) + 1, by_meas.index(pick) + 1, f"{float(rho):.3f}"])
    if out_path:
        with open(out_path, "w", newline="") as fh:
            w = csv.writer(fh)
            w.writerow(RESCORE_COLUMNS)
            w.writerows(out)
    return out


def default_summary(workload, space):
    """One summary file per workload and space, each with the reference's
    columns (bench/stage9_costmodel.py:58-61), so rows of different studies
    of one shape are never mixed."""
    name = "stage9_summary" + ("" if workload == "mbr" else f"_{workload}") + \
        ("" if space == "cdna4" else "_reference_space")
    return f"results/gpu/{name}.csv"


def cli():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--csv", default="results/gpu/stage9_autotune.csv")
    ap.add_argument("--summary", default=None,
                    help="summary CSV (the reference's columns); default results/gpu/stage9_summary.csv for mbr "
                         "over the CDNA4 space, with _matmul and/or _reference_space before .csv otherwise")
    ap.add_argument("--shapes", default="")
    ap.add_argument("--workload", default="mbr", choices=harness.GEMM_WORKLOADS)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--reps", type=int, default=100)
    ap.add_argument("--space", choices=("cdna4", "reference"), default="cdna4")
    ap.add_argument("--top", type=int, default=0, help="measure only the N best-predicted configurations")
    ap.add_argument("--split-k", default="1", help="split-K factors crossed with the configurations, e.g. 1,2,4,8")
    ap.add_argument("--tuned", default=str(TUNED), help="JSON table the best configuration is recorded in")
    ap.add_argument("--no-record", action="store_true")
    ap.add_argument("--mask-edges", action="store_true", help="every configuration on the true shape, masked edges")
    ap.add_argument("--wave-split", action="store_true",
                    help="add the wave-split configurations (wave-split-k=1) to the space")
    ap.add_argument("--prewarm", type=int, default=500, help="untimed launches before the first timing of a shape")
    ap.add_argument("--rescore", metavar="OUT", default=None,
                    help="no GPU: score the current cost model on the studies already in --csv and write one row "
                         "per study to OUT")
    ap.add_argument("--objective", choices=("latency", "throughput"), default="latency",
                    help="what the recorded configuration minimises: the per-launch median (tf_bench), or the "
                         "time per launch with launches back to back (bench.py's measure)")
    return ap


def main(argv=None):
    args = cli().parse_args(argv)
    if args.rescore:
        for row in rescore(args.csv, args.rescore):
            print(f"{row[2]:6s} {row[3]:16s} {row[0][:12]} n={row[4]:4d} pick {row[5]:22s} best {row[7]:22s} "
                  f"ratio {row[9]} rank_best {row[10]:3d} spearman {row[12]}")
        return 0
    table = provenance.ResultsTable(args.csv)
    base = table.base
    summary_path = pathlib.Path(args.summary or default_summary(args.workload, args.space))
    summary_path.parent.mkdir(parents=True, exist_ok=True)
    fresh = not summary_path.exists() or summary_path.stat().st_size == 0
    with open(summary_path, "a", newline="") as fh:
        writer = csv.writer(fh)
        if fresh:
            writer.writerow(SUMMARY_COLUMNS)
        for shape in harness.parse_shapes(args.shapes, DEFAULT_SHAPES):
            study = ShapeStudy(args, args.workload, *shape).run()
            for c in study.timed():
                table.add(**study.row_of(c))
            if not study.timed():
                print(f"{shape}: nothing passed", flush=True)
                continue
            row, pick, best, rho = study.summary(base)
            writer.writerow(row)
            fh.flush()
            chosen = study.chosen(best)
            if not args.no_record:
                source = {"commit": base["commit"], "date": base["date"], "summary": summary_path.name,
                          "summary_row": f"{base['commit']},{base['job_id']},{base['date']},{'x'.join(map(str, shape))}"}
                record_best(args.tuned, args.workload, shape, chosen, pick, rho, args.objective, source)
            print(f"{'x'.join(map(str, shape))}: model {pick.name} {pick.measured_ms:.4f} ms, best {best.name} "
                  f"{best.measured_ms:.4f} ms, ratio {best.measured_ms / pick.measured_ms:.3f}, spearman {rho:.3f}, "
                  f"{len(study.compiled())}/{len(study.candidates)} compiled", flush=True)
            if args.objective == "throughput":
                print(f"{'x'.join(map(str, shape))}: back to back {chosen.name} {chosen.window_ms:.4f} ms/launch "
                      f"(per-launch median {chosen.measured_ms:.4f} ms)", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
