"""Generate the ahead-of-time instantiation list of the staged gfx950 GEMM kernel.

Every staged configuration a pipeline option string can select must exist as a
template instantiation in libtforge_hip.so.  This script writes
_gen/staged_XX.hip (one shard per parallel compile job) and _gen/registry.hip,
which tf_compile searches at run time.

The configuration space is the reference's Stage 9 grid (python/costmodel.py:49-60:
BM, BN in {32, 64, 128}, TM x TN in {4x4, 8x4, 4x8, 8x8}, BK in {8, 16, 32}),
widened for CDNA4 (BM, BN up to 256, BK up to 64), restricted to the
configurations that map onto whole waves of 32x32 MFMA blocks, thread tiles
2x2 / 2x4 / 4x2 on 16x16 MFMA blocks for small block tiles, the wave layouts
that run the reference grid's configurations whose own wave tile does not fit
the block (wave_layout: 32x128 as 4x16, 128x32 as 16x4), plus the
promote/vectorize ablation variants of the reference's Stage 8/9 ladders
(bench/stage8_gpu.sh:7-14, bench/stage9_ablation.py:23-28), and a masked
twin (any M, N, K; the mask-edges option) of every LDS-staged configuration.
"""

import pathlib
import sys

HERE = pathlib.Path(__file__).resolve().parent
LDS_LIMIT = 160 * 1024


def staged_valid(bm, bn, tm, tn, bk, promote=1):
    """Why a staged config cannot be instantiated, or None if it can."""
    if bm % tm or bn % tn:
        return "block tile must be a multiple of the thread tile"
    threads = (bm // tm) * (bn // tn)
    if threads % 64:
        return f"{threads} threads per block is not a whole number of 64-lane waves"
    if threads > 1024:
        return f"{threads} threads per block exceeds 1024"
    if threads * tm * tn > 32768:
        return (f"{threads} threads x {tm * tn} accumulators per lane exceed the register file "
                "(512 VGPRs per SIMD lane shared by the block's waves)")
    wtm, wtn = 8 * tm, 8 * tn
    if wtm % 16 or wtn % 16:
        return f"wave tile {wtm}x{wtn} (8*TM x 8*TN) is not made of 16x16 or 32x32 MFMA blocks"
    if bm % wtm or bn % wtn:
        return f"block tile {bm}x{bn} is not a multiple of the wave tile {wtm}x{wtn} (8*TM x 8*TN)"
    mb = 32 if wtm % 32 == 0 and wtn % 32 == 0 else 16
    if bk % (256 // mb):
        return f"tile-k must be a multiple of {256 // mb} for {mb}x{mb} MFMA blocks"
    lds = (2 * (bm * (bk + (4 if mb == 32 else 8)) + bk * (bn + (8 if mb == 32 else 4))) + bn) * 4 if promote else 0
    if lds > LDS_LIMIT:
        return f"LDS {lds} B exceeds 160 KiB"
    return None


def wave_layout(bm, bn, tm, tn):
    """The thread tile of the instantiation that runs block-tile=BM,BN
    thread-tile=TM,TN (mirrors staged_wave_layout in runtime.hip): the
    option's own, unless its (8*TM) x (8*TN) wave tile cannot tile the block
    -- fewer than 64 threads: one wave owns the block (BM/8 x BN/8); a wave
    tile taller or wider than the block: the same threads and accumulators
    per lane with the long side shortened to fit."""
    if bm % tm or bn % tn or bm % 8 or bn % 8:
        return tm, tn
    threads = (bm // tm) * (bn // tn)
    ktm, ktn = tm, tn
    if threads < 64:
        ktm, ktn = bm // 8, bn // 8
    elif 8 * tm > bm and (tm * tn) % (bm // 8) == 0:
        ktm = bm // 8
        ktn = tm * tn // ktm
    elif 8 * tn > bn and (tm * tn) % (bn // 8) == 0:
        ktn = bn // 8
        ktm = tm * tn // ktn
    if 8 * ktm > bm or 8 * ktn > bn or bm % ktm or bn % ktn:
        return tm, tn
    return ktm, ktn


def reference_grid():
    """The reference's Stage 9 grid (python/costmodel.py:49-60): 105 configurations."""
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


def configs():
    out = []
    for bm in (32, 64, 128, 256):
        for bn in (32, 64, 128, 256):
            for tm, tn in ((4, 4), (8, 4), (4, 8), (8, 8)):
                for bk in (8, 16, 32, 64):
                    if staged_valid(bm, bn, tm, tn, bk) is None:
                        out.append((bm, bn, tm, tn, bk, 1, 1))
    # 16x16 MFMA blocks: small block tiles with 4x the waves.
    for bm in (32, 64, 128):
        for bn in (32, 64, 128):
            for tm, tn in ((2, 2), (2, 4), (4, 2)):
                for bk in (16, 32, 64):
                    if staged_valid(bm, bn, tm, tn, bk) is None:
                        out.append((bm, bn, tm, tn, bk, 1, 1))
    # The wave layouts that stand in for the reference grid's configurations
    # whose own wave tile cannot tile the block (wave_layout).
    for bm, bn, tm, tn, bk in reference_grid():
        c = (bm, bn) + wave_layout(bm, bn, tm, tn) + (bk, 1, 1)
        if staged_valid(*c[:5]) is None and c not in out:
            out.append(c)
    for bm, bn, tm, tn, bk in ((128, 64, 8, 4, 16), (64, 64, 4, 4, 16), (64, 64, 4, 4, 32),
                               (128, 128, 8, 8, 16), (128, 128, 8, 8, 8)):
        for promote, vec in ((0, 1), (1, 0), (0, 0)):
            out.append((bm, bn, tm, tn, bk, promote, vec))
    # Masked twins (mask-edges) of the LDS-staged configurations whose threads
    # stage at most MASK_MAX_VECTORS vectors per slab (more does not fit the
    # register file next to the masked loads).
    out = [c + (0,) for c in out]
    out += [c[:7] + (1,) for c in out if c[5] == 1 and staging_vectors(*c[:5], c[6]) <= MASK_MAX_VECTORS]
    return out


MASK_MAX_VECTORS = 16

# Wave-split instantiations (the wave-split-k option): workgroup tiles with
# few outputs, whose waves split K.  Keyed by (BM, BN, threads, BK); each
# thread tile that gives that many threads gets a registry entry.
WAVEK_TILES = [(16, 16), (16, 32), (32, 16), (32, 32), (16, 64), (64, 16), (32, 64), (64, 32), (64, 64)]
WAVEK_THREADS = (256, 512, 1024)
WAVEK_BK = (16, 32, 64)


def wavek_valid(bm, bn, nt, bk):
    """Why a wave-split config cannot be instantiated, or None (mirrors wavek_gemm.hpp)."""
    w = nt // 64
    mb = 32 if bm % 32 == 0 and bn % 32 == 0 else 16
    kc = 256 // mb
    if bk % kc:
        return f"tile-k must be a multiple of {kc} for {mb}x{mb} MFMA blocks"
    fm, fn = bm // mb, bn // mb
    acc = fm * fn * mb * mb // 64
    c = bk // kc
    sb = 0 if mb == 32 else 1  # B staged through LDS for 16-wide MFMA blocks
    lpr, lprb = bk // 4, bn // 4
    if 64 % lpr or bm % (64 // lpr):
        return f"a {bm}x{bk} A slab does not split into whole rows per 128-bit load"
    if sb and (64 % lprb or bk % (64 // lprb)):
        return f"a {bk}x{bn} B slab does not split into whole rows per 128-bit load"
    regs = bm * bk // 64 + (bk * bn // 64 if sb else c * 4 * fn)
    frag = 2 * (fm * 4 + (fn * 4 if sb else 0))
    budget = (min(512 // (w // 4), 256) if w >= 4 else 256) - 24
    if (budget - acc - frag) // regs < 2:
        return (f"two register sets of a {bk}-deep slab ({regs} VGPRs each), {frag} fragment and {acc} "
                f"accumulator VGPRs exceed the {budget + 24} VGPRs per wave at {w} waves")
    stage = bm * (bk + (4 if mb == 32 else 8)) + (bk * (bn + (8 if mb == 32 else 4)) if sb else 0)
    lds = w * max(stage, bm * (bn + 4)) * 4
    if lds > LDS_LIMIT:
        return f"{w} staging / partial tiles of {bm}x{bn} ({lds} B) exceed 160 KiB of LDS"
    return None


def wavek_configs():
    out = []
    for bm, bn in WAVEK_TILES:
        for nt in WAVEK_THREADS:
            for bk in WAVEK_BK:
                if wavek_valid(bm, bn, nt, bk) is None:
                    out.append((bm, bn, nt, bk))
    return out


def wavek_thread_tiles(bm, bn, nt):
    """(TM, TN) pairs with (BM/TM)*(BN/TN) = nt."""
    per = bm * bn // nt
    return [(tm, tn) for tm in (1, 2, 4, 8) for tn in (1, 2, 4, 8)
            if tm * tn == per and bm % tm == 0 and bn % tn == 0]


def wavek_name(bm, bn, tm, tn, bk):
    return f"tf_wavek_b{bm}x{bn}_t{tm}x{tn}_k{bk}"


def staging_vectors(bm, bn, tm, tn, bk, vec=1):
    """Global-load vectors (128-bit, or 32-bit without vectorize) a thread stages per slab."""
    threads = (bm // tm) * (bn // tn)
    vw = 4 if vec else 1
    return -(-(bm * bk // vw) // threads) + -(-(bk * bn // vw) // threads)


def name(c):
    bm, bn, tm, tn, bk, p, v, mk = c
    return (f"tf_staged_b{bm}x{bn}_t{tm}x{tn}_k{bk}" + ("" if p else "_noprom") + ("" if v else "_novec")
            + ("_masked" if mk else ""))


def main(shards=16):
    gen = HERE / "_gen"
    gen.mkdir(exist_ok=True)
    cfgs = configs()
    parts = [cfgs[i::shards] for i in range(shards)]
    for i, part in enumerate(parts):
        lines = ['#include "../staged_gemm.hpp"', "", "namespace tfk {", "",
                 "#ifndef __HIP_DEVICE_COMPILE__  // host registry data", f"extern const KernelEntry kStaged{i}[] = {{"]
        for c in part:
            t = ", ".join(str(x) for x in c)
            lines.append(f"    KernelEntry{{FAM_STAGED, {t}, \"{name(c)}\",")
            lines.append(f"                reinterpret_cast<const void *>(&staged_gemm_kernel<{t}>),")
            t7 = ", ".join(str(x) for x in c[:7])
            lines.append(f"                &launch_staged<{t}>, nullptr, StagedGemm<{t7}>::LDS_BYTES}},")
        lines += ["};", f"extern const int kStagedCount{i} = {len(part)};", "#else",
                  "// Device pass: instantiate the kernels the host table names."]
        for c in part:
            t = ", ".join(str(x) for x in c)
            lines.append(f"template __global__ void staged_gemm_kernel<{t}>(const float *, const float *, long, long, int, "
                         "int, int, int, int, int, GemmParams);")
        lines += ["#endif", "", "}  // namespace tfk", ""]
        text = "\n".join(lines)
        p = gen / f"staged_{i:02d}.hip"
        if not p.exists() or p.read_text() != text:
            p.write_text(text)
    lines = ['#include "../wavek_gemm.hpp"', "", "namespace tfk {", "",
             "#ifndef __HIP_DEVICE_COMPILE__  // host registry data", "extern const KernelEntry kWaveK[] = {"]
    wk = wavek_configs()
    n_entries = 0
    for bm, bn, nt, bk in wk:
        t = f"{bm}, {bn}, {nt}, {bk}"
        for tm, tn in wavek_thread_tiles(bm, bn, nt):
            lines.append(f"    KernelEntry{{FAM_WAVEK, {bm}, {bn}, {tm}, {tn}, {bk}, 1, 1, 0, \"{wavek_name(bm, bn, tm, tn, bk)}\",")
            lines.append(f"                reinterpret_cast<const void *>(&wavek_gemm_kernel<{t}>),")
            lines.append(f"                &launch_wavek<{t}>, nullptr, WaveKGemm<{t}>::LDS_BYTES}},")
            n_entries += 1
    lines += ["};", f"extern const int kWaveKCount = {n_entries};", "#else",
              "// Device pass: instantiate the kernels the host table names."]
    for bm, bn, nt, bk in wk:
        lines.append(f"template __global__ void wavek_gemm_kernel<{bm}, {bn}, {nt}, {bk}>(const float *, const float *, long, "
                     "long, int, int, int, int, GemmParams);")
    lines += ["#endif", "", "}  // namespace tfk", ""]
    text = "\n".join(lines)
    p = gen / "wavek.hip"
    if not p.exists() or p.read_text() != text:
        p.write_text(text)
    reg = ['#include <vector>', '', '#include "../tf_kernels.h"', '', 'namespace tfk {', '',
           'extern const KernelEntry kDirectEntries[];', 'extern const int kDirectCount;',
           'extern const KernelEntry kWaveK[];', 'extern const int kWaveKCount;']
    for i in range(shards):
        reg += [f"extern const KernelEntry kStaged{i}[];", f"extern const int kStagedCount{i};"]
    reg += ["", "static const std::vector<KernelEntry> &all_entries() {",
            "  static const std::vector<KernelEntry> v = [] {",
            "    std::vector<KernelEntry> r(kDirectEntries, kDirectEntries + kDirectCount);"]
    for i in range(shards):
        reg.append(f"    r.insert(r.end(), kStaged{i}, kStaged{i} + kStagedCount{i});")
    reg += ["    r.insert(r.end(), kWaveK, kWaveK + kWaveKCount);",
            "    return r;", "  }();", "  return v;", "}", "",
            "const KernelEntry *registry_begin() { return all_entries().data(); }",
            "const KernelEntry *registry_end() { return all_entries().data() + all_entries().size(); }",
            "", "}  // namespace tfk", ""]
    text = "\n".join(reg)
    p = gen / "registry.hip"
    if not p.exists() or p.read_text() != text:
        p.write_text(text)
    print(f"{len(cfgs)} staged instantiations in {shards} shards, "
          f"{len(wk)} wave-split ({n_entries} entries)")


if __name__ == "__main__":
    main(int(sys.argv[1]) if len(sys.argv) > 1 else 16)
