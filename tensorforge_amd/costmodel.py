"""Analytical cost model of the staged GEMM kernel, retargeted to CDNA4 (MI355X).

The reference's Stage 9 model (python/costmodel.py:1-97) predicts the time of
its SIMT staged kernel from the tile sizes, the padded problem and the blocks
per SM reported by the occupancy API.  Its skeleton is kept:

  blocks   = (Mp / BM) * (Np / BN)
  waves    = ceil(blocks / (UNITS * blocks_per_unit))      rounds of resident blocks
  resident = min(blocks_per_unit, ceil(blocks / UNITS))
  cycles   = waves * (Kp / BK) * step
  time     = max(cycles / clock, compulsory_bytes / DRAM_BW)

and `predict(..., target=SM120)` restates the reference formula exactly (the
test suite checks it against every 4th row of the reference's own
stage9_autotune.csv and e2_a6000_autotune.csv notes).  The MI355X target
replaces the per-step terms with what bounds the gfx950 MFMA kernel:

  mfma_step  FP32 MFMA issue on the busiest SIMD: the resident waves share 4
             SIMDs (q = ceil(resident * W / 4) waves per SIMD), and a wave's
             slab is FM*FN*(BK/2) v_mfma_f32_32x32x2 of 64 cycles each,
             divided by the kernel structure's efficiency (below).
  lds_step   LDS bytes per slab over 128 B/clk: per wave (BK/8)*1 KiB per
             32-row A block (b128 reads) and per 32-column B block (b32
             reads), plus the block's (BM+BN)*BK*4 B of stores.
  l2_step    global -> LDS bytes per slab, (BM+BN)*BK*4 per block, over the
             rate one CU streams from L2: ~22 B/clk, set by the L2 requests a
             CU keeps in flight (~60 at ~340 cycles, measured), not by the
             64 B/clk fill bandwidth -- small tiles at one or two workgroups
             per CU are bound by it.
  exposed    the loads of a slab are issued DEPTH slabs before its LDS write
             (two register staging sets where a thread stages at most 8
             vectors per slab, else one set), so max(0, LATENCY - DEPTH *
             compute) is exposed per slab (DEPTH 2 or 1).
  serial     with one wave per SIMD and the slab staged in one burst (not
             spread over the MFMAs) nothing overlaps a wave's fragment reads
             with its MFMAs: the step is at least mfma_step + lds_step.
  sync       one barrier per slab; measured to cost nothing visible in the
             launch time (the waves' MFMAs cover it), so 0.
  efficiency of the kernel structure (calibrated on the Stage 9 measurements):
             16x16 MFMA blocks (v_mfma_f32_16x16x4_f32: twice the
             instructions and fragment reads per FLOP) run at 1/1.05 of the
             MFMA rate, block-staged kernels (the staging burst between two
             chunks of MFMAs, rather than one staging operation after each
             MFMA) at 1/1.10.

Split-K (a backend option, a sixth configuration entry S): S workgroups per
output tile, each over Kp/S; the tile count is multiplied by S and the K
steps divided by S, and the reduction launch adds its HBM traffic (S partial
slices written and read, C written; at least the shortest measured
reduction kernel) plus a fixed launch cost.

Wave-split (the wave-split-k backend option, a seventh configuration entry
1): the waves of a workgroup split its K range and add their partial tiles in
LDS, each wave loading its own operands (no sharing), so a workgroup pulls
(BM+BN)*K*4/S bytes from L2 into one CU.  That stream is bounded by the L2
requests one CU keeps in flight, not by the L2's bandwidth: a loads-only copy
of the kernel at 64 x 4096 x 4096 moves 1 MiB per CU in ~20 us, about 22 B/clk
per CU (l2_stream_bytes_per_cycle), against 64 B/clk of fill bandwidth.  The
model takes the larger of that stream and the MFMA time per CU, plus the LDS
round trip of the staged A (and B) slabs and the final partial-tile sum.

Constants are AMD's published MI355X figures (256 CUs, 2.4 GHz, FP32 matrix
256 FLOP/clk/CU, 160 KiB LDS, 8 TB/s HBM) and measured ones (the per-CU L2
stream, the shortest reduction kernel); LATENCY, the structure divisor 1.05
and the wave-split big-tile efficiency 0.55 (from the 64 x 4096 x 4096
measurements, where the wave-split family is the one that matters) are
calibrated on the Stage 9 measurements, and the model only ranks
configurations.  Over the 27 measured studies (results/gpu/stage9_autotune.csv,
rescored by bench/stage9_costmodel.py --rescore) its pick reaches 0.90-1.00
of the measured best (mean 0.983) and its Spearman rank correlation with the
measured times 0.48-0.98 (mean 0.82); the terms that moved the pick there
from 0.82-1.00 are the L2 stream rate for small tiles, the staging depth in
the exposed latency, the first-slab prologue and the structure divisors, and
the serial term lifted the mean correlation from 0.76.
"""

import dataclasses
import json
import math
import os
import pathlib

PKG = pathlib.Path(__file__).resolve().parent


@dataclasses.dataclass(frozen=True)
class Target:
    name: str
    kind: str               # "simt" (reference formula) or "mfma" (CDNA4)
    units: int              # SMs or CUs
    clock_mhz: float
    dram_bw: float          # bytes/s
    fma_per_cycle: float = 128.0        # simt: FP32 FMA lanes per SM
    smem_words_per_cycle: float = 32.0  # simt
    latency: float = 600.0              # cycles, global load missing L1
    lds_bytes_per_cycle: float = 128.0  # mfma
    l2_bytes_per_cycle: float = 64.0    # mfma, per CU
    sync: float = 0.0                   # mfma, barrier bubble per slab
    simds: int = 4
    mfma_cycles: float = 64.0           # v_mfma_f32_32x32x2_f32 per wave
    lds_per_cu: int = 160 * 1024
    max_waves_per_simd: int = 8
    launch_s: float = 3e-6              # mfma: one more dependent kernel launch (split-K reduction)
    reduce_min_s: float = 2.5e-6        # mfma: shortest reduction kernel (measured 3.3-4.0 us at 64 x 4096)
    l2_stream_bytes_per_cycle: float = 22.0  # mfma: measured per-CU L2 -> CU stream (L2 requests in flight)
    slow_structure: float = 1.05        # mfma: MFMA-rate divisor for 16x16 blocks
    slow_block_staging: float = 1.10    # mfma: MFMA-rate divisor for block staging (not spread over the MFMAs)
    wave_split_big_tile: float = 0.55   # mfma: MFMA efficiency of wave-split tiles of >= 4 32x32 blocks


# The reference's model (python/costmodel.py:41-46); TF_GPU_SMS / TF_GPU_DRAM_BW as there.
SM120 = Target("sm_120", "simt", int(os.environ.get("TF_GPU_SMS", "188")), 2280.0,
               float(os.environ.get("TF_GPU_DRAM_BW", "1530e9")))
MI355X = Target("gfx950", "mfma", int(os.environ.get("TF_GPU_CUS", "256")), 2400.0,
                float(os.environ.get("TF_GPU_HBM_BW", "8e12")), latency=900.0)

SMS = MI355X.units
CLOCK_MHZ = MI355X.clock_mhz


def _valid_staged(bm, bn, tm, tn, bk):
    if bm % tm or bn % tn:
        return False
    threads = (bm // tm) * (bn // tn)
    if threads % 64 or threads > 1024 or threads * tm * tn > 32768:
        return False
    wtm, wtn = 8 * tm, 8 * tn
    if wtm % 16 or wtn % 16 or bm % wtm or bn % wtn:
        return False
    if bk % (256 // _block(tm, tn)):
        return False
    return _lds_bytes(bm, bn, tm, tn, bk) <= 160 * 1024


def _block(tm, tn):
    """MFMA block edge: 32 when the wave tile (8*TM x 8*TN) is made of 32x32 blocks, else 16."""
    return 32 if (8 * tm) % 32 == 0 and (8 * tn) % 32 == 0 else 16


def _wave_lds_bytes(bm, bn, w, bk):
    # per-wave staging tiles (A, and B for 16-wide blocks) or the W partial tiles, whichever is larger
    mb = 32 if bm % 32 == 0 and bn % 32 == 0 else 16
    stage = bm * (bk + (4 if mb == 32 else 8)) + (0 if mb == 32 else bk * (bn + 4))
    return w * max(stage, bm * (bn + 4)) * 4


def _staging(bm, bn, tm, tn, bk):
    """(DEPTH, spread) of the staged kernel (csrc/staged_gemm.hpp): two register
    staging sets (loads two slabs ahead) where a thread stages at most 8
    vectors per slab, else one; the staging spread over the MFMAs for
    workgroups of at most 256 threads with two sets and at least two
    k-chunks per slab that have room for it."""
    mb = _block(tm, tn)
    nt = (bm // tm) * (bn // tn)
    fm, fn = 8 * tm // mb, 8 * tn // mb
    vec = -(-(bm * bk // 4) // nt) + -(-(bk * bn // 4) // nt)
    depth = 2 if vec <= 8 else 1
    chunks = bk // (256 // mb)
    spread = nt <= 256 and depth == 2 and chunks >= 2 and 2 * vec <= 4 * fm * fn * (chunks - 1)
    return depth, spread


def _lds_bytes(bm, bn, tm, tn, bk):
    # two A and B tile buffers plus the tile's bias values
    mb = _block(tm, tn)
    return (2 * (bm * (bk + (4 if mb == 32 else 8)) + bk * (bn + (8 if mb == 32 else 4))) + bn) * 4


def reference_space():
    """The reference's Stage 9 grid (python/costmodel.py:49-60)."""
    out = []
    for bm in (32, 64, 128):
        for bn in (32, 64, 128):
            for tm, tn in ((4, 4), (8, 4), (4, 8), (8, 8)):
                for bk in (8, 16, 32):
                    threads = (bm // tm) * (bn // tn)
                    if bm % tm or bn % tn or not 32 <= threads <= 1024:
                        continue
                    out.append((bm, bn, tm, tn, bk))
    return out


def config_space():
    """The CDNA4 grid: BM, BN in {32..256}, TM x TN in {4x4, 8x4, 4x8, 8x8},
    BK in {8..64} (32x32 MFMA blocks), and BM, BN in {32..128}, TM x TN in
    {2x2, 2x4, 4x2}, BK in {16..64} (16x16 blocks): every configuration that
    has a gfx950 instantiation (whole waves of MFMA blocks, LDS within 160 KiB,
    the register file)."""
    out = []
    for bm in (32, 64, 128, 256):
        for bn in (32, 64, 128, 256):
            for tm, tn in ((4, 4), (8, 4), (4, 8), (8, 8)):
                for bk in (8, 16, 32, 64):
                    if _valid_staged(bm, bn, tm, tn, bk):
                        out.append((bm, bn, tm, tn, bk))
    for bm in (32, 64, 128):
        for bn in (32, 64, 128):
            for tm, tn in ((2, 2), (2, 4), (4, 2)):
                for bk in (16, 32, 64):
                    if _valid_staged(bm, bn, tm, tn, bk):
                        out.append((bm, bn, tm, tn, bk))
    return out


def splits_of(cfg):
    """Split-K factor of a configuration: (BM, BN, TM, TN, BK[, S[, WAVE]])."""
    return cfg[5] if len(cfg) > 5 else 1


def wave_split_of(cfg):
    """1 for a wave-split configuration (seventh entry), else 0."""
    return cfg[6] if len(cfg) > 6 else 0


def options(cfg):
    bm, bn, tm, tn, bk = cfg[:5]
    s = splits_of(cfg)
    return (f"block-tile={bm},{bn} thread-tile={tm},{tn} tile-k={bk} promote=1 vectorize=1"
            + (" wave-split-k=1" if wave_split_of(cfg) else "") + (f" split-k={s}" if s > 1 else ""))


def name(cfg):
    bm, bn, tm, tn, bk = cfg[:5]
    s = splits_of(cfg)
    return f"b{bm}x{bn}-t{tm}x{tn}-k{bk}" + ("-w" if wave_split_of(cfg) else "") + (f"-s{s}" if s > 1 else "")


def kernel_tile(cfg):
    """(TM, TN) of the instantiation that runs cfg: the option's thread tile,
    or for a staged configuration whose (8 TM) x (8 TN) wave tile cannot tile
    the block, the wave layout that stands in for it (csrc/gen_instances.py
    wave_layout; the library reports that launch geometry)."""
    bm, bn, tm, tn = cfg[:4]
    if wave_split_of(cfg):
        return tm, tn
    return _gen_instances().wave_layout(bm, bn, tm, tn)


def kernel_name(cfg):
    bm, bn, _, _, bk = cfg[:5]
    tm, tn = kernel_tile(cfg)
    return f"tf_{'wavek' if wave_split_of(cfg) else 'staged'}_b{bm}x{bn}_t{tm}x{tn}_k{bk}"


_GEN = []


def _gen_instances():
    if not _GEN:
        import importlib.util
        spec = importlib.util.spec_from_file_location("tf_gen_instances", PKG / "csrc" / "gen_instances.py")
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        _GEN.append(mod)
    return _GEN[0]


def wave_split_space():
    """Every wave-split instantiation as (BM, BN, TM, TN, BK, 1, 1): the
    configurations csrc/gen_instances.py builds."""
    g = _gen_instances()
    return [(bm, bn, tm, tn, bk, 1, 1) for bm, bn, nt, bk in g.wavek_configs()
            for tm, tn in g.wavek_thread_tiles(bm, bn, nt)]


def with_splits(space, m, n, k, splits=(1, 2, 4, 8, 16)):
    """Each configuration once per split-K factor that leaves every split at
    least one K slab (S = 1 keeps the 5-entry form of a staged configuration)."""
    out = []
    for cfg in space:
        nk = padded(cfg, m, n, k)[2] // cfg[4]
        for s in splits:
            if s <= nk:
                if wave_split_of(cfg):
                    out.append(tuple(cfg[:5]) + (s, 1))
                else:
                    out.append(tuple(cfg[:5]) if s == 1 else tuple(cfg[:5]) + (s,))
    return out


def _resources():
    p = PKG / "kernel_resources.json"
    return json.loads(p.read_text()) if p.exists() else {}


def estimate_info(cfg, target=MI355X, resources=None):
    """Blocks per CU without a GPU: the smaller of the register-limited waves
    per SIMD (compiler resource remarks) and the LDS limit; the occupancy API
    (tforge_gpu.info) gives the same number on the device."""
    bm, bn, _, _, bk = cfg[:5]
    tm, tn = kernel_tile(cfg)
    threads = (bm // tm) * (bn // tn)
    w = threads // 64
    rec = (resources if resources is not None else _resources()).get(kernel_name(cfg), {})
    occ = rec.get("occupancy_waves_per_simd", target.max_waves_per_simd)
    if occ is None or occ <= 0:
        occ = target.max_waves_per_simd
    lds = rec.get("lds_bytes", _wave_lds_bytes(bm, bn, w, bk) if wave_split_of(cfg) else _lds_bytes(bm, bn, tm, tn, bk))
    by_regs = (occ * target.simds) // w
    by_lds = target.lds_per_cu // lds if lds else by_regs
    return {"blocks_per_sm": max(1, min(by_regs, by_lds, 2048 // threads)), "threads": threads}


def predict(cfg, padded, info, clock_mhz=None, target=MI355X):
    """Predicted time in ms and the terms that produced it."""
    bm, bn, tm, tn, bk = cfg[:5]
    splits = splits_of(cfg)
    mp, np_, kp = padded
    clock = clock_mhz or target.clock_mhz
    bps = max(1, info["blocks_per_sm"])
    threads = (bm // tm) * (bn // tn)
    blocks = (mp // bm) * (np_ // bn) * splits
    waves = math.ceil(blocks / (target.units * bps))
    resident = min(bps, math.ceil(blocks / target.units))
    if target.kind == "simt":
        # python/costmodel.py:74-97, unchanged.
        fma_step = bm * bn * bk / target.fma_per_cycle
        lds_step = threads * bk * (tm + tn) / target.smem_words_per_cycle
        compute_step = max(fma_step, lds_step)
        exposed = max(0.0, target.latency - (resident - 1) * compute_step)
        step = resident * compute_step + exposed
        cycles = waves * (kp // bk) * step
        t_compute = cycles / (clock * 1e6)
        t_dram = 4.0 * (mp * kp + kp * np_ + mp * np_) / target.dram_bw
        t = max(t_compute, t_dram)
        return {"pred_ms": t * 1e3, "waves": waves, "resident": resident, "blocks": blocks,
                "fma_step": fma_step, "lds_step": lds_step,
                "bound": "dram" if t_dram > t_compute else ("smem" if lds_step > fma_step else "fma"),
                "latency_exposed": exposed > 0, "intensity": 2.0 * bm * bn / (4.0 * (bm + bn))}
    if wave_split_of(cfg):
        return _predict_wave_split(cfg, padded, bps, blocks, waves, resident, clock, target)
    tm, tn = kernel_tile(cfg)  # the launch geometry that runs cfg
    w = (bm // tm) * (bn // tn) // 64
    mb = _block(tm, tn)
    fm, fn = 8 * tm // mb, 8 * tn // mb
    depth, spread = _staging(bm, bn, tm, tn, bk)
    q = math.ceil(resident * w / target.simds)
    # FP32 MFMA: 64 FLOP per SIMD clock for both block sizes (4096 FLOP in 64
    # cycles, or 2048 in 32); a wave's slab is 2 * (8 TM)(8 TN) BK FLOP.
    slow = (target.slow_structure if mb == 16 else 1.0) * (1.0 if spread else target.slow_block_staging)
    mfma_step = q * 2 * (8 * tm) * (8 * tn) * bk / 64.0 * (target.mfma_cycles / 64.0) * slow
    # per chunk of 256 / mb k values, 1 KiB per A block-row and per B block-column
    lds_bytes = resident * (w * (bk / (256 // mb)) * 1024 * (fm + fn) + (bm + bn) * bk * 4)
    lds_step = lds_bytes / target.lds_bytes_per_cycle
    l2_step = resident * (bm + bn) * bk * 4 / target.l2_stream_bytes_per_cycle
    compute = max(mfma_step, lds_step, l2_step)
    if q == 1 and not spread:
        # one wave per SIMD and the slab staged in one burst: no other wave
        # issues MFMAs while this one reads its fragments from LDS
        compute = max(compute, mfma_step + lds_step)
    exposed = max(0.0, target.latency - (2.0 if depth == 2 else 1.0) * compute)
    step = compute + exposed + target.sync / q
    epilogue = target.latency + resident * bm * bn * 4 / target.l2_bytes_per_cycle
    # the first slab of every resident workgroup arrives before any MFMA
    prologue = target.latency + resident * (bm + bn) * bk * 4 / target.l2_stream_bytes_per_cycle
    ksteps = -(-(kp // bk) // splits)
    cycles = waves * (ksteps * step + prologue + epilogue)
    t_compute = cycles / (clock * 1e6)
    t_dram = 4.0 * (mp * kp + kp * np_ + mp * np_ + np_) / target.dram_bw
    t = max(t_compute, t_dram)
    if splits > 1:
        t += max((2 * splits + 1) * 4.0 * mp * np_ / target.dram_bw, target.reduce_min_s) + target.launch_s
    terms = {"mfma": mfma_step, "lds": lds_step, "l2": l2_step}
    bound = "dram" if t_dram > t_compute else max(terms, key=terms.get)
    return {"pred_ms": t * 1e3, "waves": waves, "resident": resident, "blocks": blocks,
            "fma_step": mfma_step, "lds_step": lds_step, "l2_step": l2_step, "bound": bound,
            "latency_exposed": exposed > 0, "waves_per_simd": q,
            "intensity": 2.0 * bm * bn / (4.0 * (bm + bn))}


def _predict_wave_split(cfg, padded, bps, blocks, waves, resident, clock, target):
    """Wave-split kernel: per round of resident workgroups on a CU, the
    larger of its MFMA time and its L2 operand stream, plus the staged slabs'
    LDS round trip, the first slab's latency and the partial-tile sum."""
    bm, bn, tm, tn, bk = cfg[:5]
    splits = splits_of(cfg)
    mp, np_, kp = padded
    w = (bm // tm) * (bn // tn) // 64
    kz = kp / splits
    mfma = resident * 2.0 * bm * bn * kz / (target.simds * 64.0)
    if (bm // 32) * (bn // 32) >= 4:  # a 64x64 tile per wave: measured at about half the MFMA rate
        mfma /= target.wave_split_big_tile
    l2 = resident * (bm + bn) * kz * 4 / target.l2_stream_bytes_per_cycle
    mb = 32 if bm % 32 == 0 and bn % 32 == 0 else 16
    staged = bm + (0 if mb == 32 else bn)
    lds = resident * (2 * staged * kz * 4 + 2 * w * bm * bn * 4) / target.lds_bytes_per_cycle
    compute = max(mfma, l2, lds)
    cycles = waves * (compute + target.latency + resident * bm * bn * 4 / target.l2_bytes_per_cycle)
    t_compute = cycles / (clock * 1e6)
    t_dram = 4.0 * (mp * kp + kp * np_ + mp * np_ + np_) / target.dram_bw
    t = max(t_compute, t_dram)
    if splits > 1:
        t += max((2 * splits + 1) * 4.0 * mp * np_ / target.dram_bw, target.reduce_min_s) + target.launch_s
    terms = {"mfma": mfma, "lds": lds, "l2": l2}
    bound = "dram" if t_dram > t_compute else max(terms, key=terms.get)
    return {"pred_ms": t * 1e3, "waves": waves, "resident": resident, "blocks": blocks,
            "fma_step": mfma, "lds_step": lds, "l2_step": l2, "bound": bound,
            "latency_exposed": False, "waves_per_simd": math.ceil(resident * w / target.simds),
            "intensity": 2.0 * bm * bn / (4.0 * (bm + bn))}


def padded(cfg, m, n, k):
    bm, bn, _, _, bk = cfg[:5]
    up = lambda x, t: -(-x // t) * t
    return up(m, bm), up(n, bn), up(k, bk)


def rank(m, n, k, space=None, target=MI355X, infos=None):
    """Configurations sorted by predicted time (model pick first)."""
    res = _resources()
    space = space or config_space()
    scored = []
    for cfg in space:
        inf = (infos or {}).get(cfg) or estimate_info(cfg, target, res)
        scored.append((predict(cfg, padded(cfg, m, n, k), inf, target=target)["pred_ms"], cfg))
    scored.sort()
    return [c for _, c in scored]


def default_config(m, n, k):
    """The cost model's pick for a shape, split-K factors included: what the
    backend uses when no autotuned configuration is recorded."""
    return rank(m, n, k, space=with_splits(config_space(), m, n, k))[0]


def tuned_options(workload, m, n, k):
    """Options for a shape: the autotuner's recorded best
    (tuned_configs.json, written by bench/stage9_costmodel.py) if there is
    one, else the cost model's pick."""
    p = PKG / "tuned_configs.json"
    if p.exists():
        rec = json.loads(p.read_text()).get(f"{workload}/{m}x{n}x{k}")
        if rec:
            return rec["options"]
    return options(default_config(m, n, k))
