// The wave-split FP32 GEMM for gfx950: C = epi(A @ B) where the waves of a
// workgroup split the K loop of the workgroup's output tile among themselves
// (the `wave-split-k` option).  For problems with few output tiles and a long
// K -- the skinny layer 64 x 4096 x 4096 has 64 tiles of 64 x 64 -- this fills
// the chip in ONE launch with no workspace: split-K across workgroups needs a
// second, reduction launch and writes every partial tile to HBM.
//
//  * Option mapping.  block-tile=BM,BN is the workgroup's output tile and the
//    workgroup has (BM/TM)*(BN/TN) threads as in the reference, i.e. W =
//    that many / 64 waves.  Every wave computes the WHOLE BM x BN tile over its
//    own contiguous range of K slabs (tile-k=BK k values each): wave w takes
//    slabs [nk*w/W, nk*(w+1)/W) of the nk = K/BK.  thread-tile=TM,TN is each
//    thread's share of the final reduction: the W partial tiles are summed
//    through LDS and each thread finishes TM*TN outputs (in 4-column groups).
//  * Math.  The staged kernel's MFMA blocks and lane layouts (staged_gemm.hpp):
//    MB x MB blocks, MB = 32 (v_mfma_f32_32x32x2_f32) when BM and BN are
//    multiples of 32, else 16 (v_mfma_f32_16x16x4_f32); operands swapped so a
//    lane's accumulators are runs of 4 consecutive columns of one row; k
//    chunk KC = 256 / MB with lane group g and step s taking k = 4g + s.
//  * Loads.  No wave shares an operand with another (their K ranges differ),
//    so nothing is staged for sharing.  A: a slab is BM rows x BK floats,
//    loaded row-contiguously (BK / 4 lanes per row, whole 128-byte lines per
//    load), written to the wave's own LDS tile and read back as fragments
//    (ds_read_b128): loading A fragments directly, one 4-k piece per row and
//    lane group, touches BM cache lines per instruction and measured twice as
//    slow, bound by the L1's tag lookups.  B: fragments straight from global
//    memory, 32-bit loads of MB consecutive columns of one row.  Raw buffer
//    loads: the per-lane offset is fixed, the slab / row / step offset is a
//    scalar, so the loop has almost no address arithmetic.
//  * Register pipeline.  NBUF register sets of one slab each; slab t + NBUF-1
//    is requested while slab t computes, so DEPTH = NBUF - 1 slabs of loads are
//    in flight per wave.  Every slab issues its loads unconditionally: a slab
//    past the wave's range is loaded through a buffer resource with zero
//    records, which returns zeros without touching memory, so the compiler's
//    wait counts stay exact (a conditional load makes it wait for every
//    outstanding load).
//  * Reduction and epilogue.  Each wave writes its partial tile to LDS
//    ([W][BM][BN + 4] floats); after one barrier every thread adds the W
//    partials of its 4-column groups in wave order 0..W-1 (a fixed order:
//    deterministic), applies the fused epilogue (bias, IEEE relu, residual
//    add) and stores 128 bits.
//  * Tile order.  The staged kernel's XCD-aware order: the workgroups one XCD
//    receives share B panels (and A) in its L2.
//  * With split-k=S, workgroup z of a tile takes the z-th of S contiguous
//    slab ranges and writes its summed partial tile to workspace slice z; the
//    staged family's reduction launch adds the slices in order and runs the
//    epilogue.  A bigger tile per compute unit halves the operand traffic
//    each unit pulls from L2 (64 x 64 over K/4 against 32 x 32 over K).
//
// Shapes: M, N, K multiples of BM, BN, BK (the host pads as for the staged
// kernels); A's BM-row panel and B below 2^31 bytes from the tile's origin
// (32-bit buffer offsets; the host checks).  The sum order differs from the
// reference's sequential k; parity is the reference's FP64 error bound, which
// holds for any order (python/tforge_cpu.py:263-271).
#pragma once

#include "staged_gemm.hpp"

namespace tfk {

// Buffer resource word 3 for gfx9-family raw buffers (32-bit data format,
// bounds-checked by byte offset).
constexpr int kBufferWord3 = 0x00020000;

// B through the wave's LDS tile too (SB = 1) where the MFMA block is 16
// wide: direct B fragment loads would then cover half cache lines (16
// columns); 32-wide blocks load whole 128-byte lines directly (measured 4%
// faster than staging B at 64 x 4096 x 4096).
template <int BM, int BN>
constexpr int wavek_stage_b() {
  return (BM % 32 == 0 && BN % 32 == 0) ? 0 : 1;
}

template <int BM, int BN, int NT, int BK, int SB = wavek_stage_b<BM, BN>()>
struct WaveKGemm {
  static constexpr int W = NT / 64;                                     // waves = K ranges
  static constexpr int MB = (BM % 32 == 0 && BN % 32 == 0) ? 32 : 16;  // MFMA block
  static constexpr int KC = 256 / MB;                                   // k per chunk
  static constexpr int C = BK / KC;                                     // chunks per slab
  static constexpr int FM = BM / MB, FN = BN / MB;
  static constexpr int ACC = FM * FN * MB * MB / 64;                    // accumulators per lane
  // A slab: BM rows x BK floats loaded row-contiguously, LPR lanes per row,
  // RPI rows per 128-bit load instruction, A_INSTR instructions.
  static constexpr int LPR = BK / 4, RPI = 64 / LPR, A_INSTR = BM / RPI;
  // B slab (SB = 1): BK rows x BN floats, LPRB lanes per row, RPIB rows per
  // instruction, B_INSTR instructions.
  static constexpr int LPRB = BN / 4, RPIB = 64 / LPRB, B_INSTR = SB ? BK / RPIB : 0;
  static constexpr int SET = 4 * A_INSTR + (SB ? 4 * B_INSTR : C * 4 * FN);  // VGPRs per slab
  static constexpr int FRAG = 2 * (FM * 4 + (SB ? FN * 4 : 0));        // fragments of two chunks
  // VGPRs per wave: 512 per SIMD lane shared by the workgroup's waves on that
  // SIMD (W / 4 of them), at most 256 architectural.  Leave 24 for offsets,
  // loop state and the epilogue.
  static constexpr int BUDGET = (W >= 4 ? (512 / (W / 4) < 256 ? 512 / (W / 4) : 256) : 256) - 24;
  static constexpr int NBUF_FIT = (BUDGET - ACC - FRAG) / SET;
  static constexpr int NBUF = NBUF_FIT > 4 ? 4 : NBUF_FIT;  // register sets (slabs in flight + 1)
  // Per-wave A staging tile [BM][LDA]: the row stride makes the fragment
  // reads (ds_read_b128) conflict-free, as in the staged kernel.
  static constexpr int LDA = BK + (MB == 32 ? 4 : 8);
  // Per-wave B staging tile [BK][LDB]: lane groups read rows 4 apart, the
  // padding puts them in disjoint banks (the staged kernel's B stride).
  static constexpr int LDB = BN + (MB == 32 ? 8 : 4);
  static constexpr int LDP = BN + 4;  // partial-tile row stride (floats)
  static constexpr int WAVE_STAGE = BM * LDA + (SB ? BK * LDB : 0);
  static constexpr int STAGE_FLOATS = W * WAVE_STAGE, PART_FLOATS = W * BM * LDP;
  static constexpr int LDS_BYTES = 4 * (STAGE_FLOATS > PART_FLOATS ? STAGE_FLOATS : PART_FLOATS);
  static constexpr int G4 = BM * BN / 4;  // 4-column output groups of the tile

  static_assert(NT % 64 == 0 && NT <= 1024, "whole waves, at most 1024 threads");
  static_assert(BM % MB == 0 && BN % MB == 0, "tile made of MFMA blocks");
  static_assert(BK % KC == 0, "tile-k must be a multiple of the k-chunk (8 for 32x32 blocks, 16 for 16x16)");
  static_assert(64 % LPR == 0 && BM % RPI == 0, "A slab rows split evenly over the load instructions");
  static_assert(!SB || (64 % LPRB == 0 && BK % RPIB == 0), "B slab rows split evenly over the load instructions");
  static_assert(NBUF >= 2, "registers for at least two slab sets");
  static_assert(LDS_BYTES <= 160 * 1024, "partial tiles exceed 160 KB of LDS");
};

// The first eight arguments repeat the fields of `p` the prologue needs, as
// scalars the hardware preloads into SGPRs (as for the staged kernels: the
// library is built with kernel-argument preloading); gx, gy = gridDim.x, .y;
// flags = swizzle | splits << 8 | blockDim.x << 16: one instantiation serves
// every thread tile with NT threads, so the block's width is an argument (a
// preloaded one: blockDim.x from the dispatch packet made every wave wait for
// that load, ~1.3k cycles, before its first global loads).
template <int BM, int BN, int NT, int BK, int SB = wavek_stage_b<BM, BN>()>
__global__ void __launch_bounds__(NT) wavek_gemm_kernel(const float *pA, const float *pB, long plda, long pldb, int pK,
                                                        int gx, int gy, int flags, GemmParams p) {
  p.A = pA;
  p.B = pB;
  p.lda = plda;
  p.ldb = pldb;
  p.K = pK;
  p.swizzle = flags & 255;
  p.splits = (flags >> 8) & 255;
  const int bx = flags >> 16;
  using G = WaveKGemm<BM, BN, NT, BK, SB>;
  constexpr int W = G::W, MB = G::MB, KC = G::KC, C = G::C, FM = G::FM, FN = G::FN, NBUF = G::NBUF;
  constexpr int LDP = G::LDP, LDA = G::LDA, LPR = G::LPR, RPI = G::RPI, A_INSTR = G::A_INSTR;
  constexpr int LDB = G::LDB, LPRB = G::LPRB, RPIB = G::RPIB, B_INSTR = G::B_INSTR;
  using AccT = AccOf<MB>;
  // Per-wave A staging tiles during the K loop, then the W partial tiles.
  __shared__ __attribute__((aligned(16))) float lds[G::LDS_BYTES / 4];

  const int tid = threadIdx.y * bx + threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane % MB, lg = lane / MB;

  int tile_m, tile_n;
  staged_tile_coords(gx, gy, p.swizzle, tile_m, tile_n);
  const long m0 = (long)tile_m * BM, n0 = (long)tile_n * BN;
  const int lda = (int)p.lda, ldb = (int)p.ldb;

  // This wave's slabs [kb, ke) of the nk = K / BK.
  // With split-K (gridDim.z = splits), workgroup z first takes the slab range
  // [nk*z/S, nk*(z+1)/S); its waves split that range.
  const int nk_all = p.K / BK;
  const int splits = p.splits > 1 ? p.splits : 1, split = blockIdx.z;
  const int zb = splits == 1 ? 0 : (int)((long)nk_all * split / splits);
  const int nkz = splits == 1 ? nk_all : (int)((long)nk_all * (split + 1) / splits) - zb;
  const int kb = zb + nkz * wave / W, ke = zb + nkz * (wave + 1) / W, nk = ke - kb;

  // Buffer resources over the tile's A panel and B columns; zero records for
  // the loads past the wave's range.
  const float *a_tile = p.A + m0 * p.lda;
  const float *b_tile = p.B + n0;
  const int a_bytes = p.K > 0 ? (int)(((long)(BM - 1) * lda + p.K) * 4) : 0;
  const int b_bytes = p.K > 0 ? (int)(((long)(p.K - 1) * ldb + BN) * 4) : 0;
  const __amdgpu_buffer_rsrc_t ra_live = __builtin_amdgcn_make_buffer_rsrc((void *)a_tile, 0, a_bytes, kBufferWord3);
  const __amdgpu_buffer_rsrc_t rb_live = __builtin_amdgcn_make_buffer_rsrc((void *)b_tile, 0, b_bytes, kBufferWord3);
  const __amdgpu_buffer_rsrc_t ra_none = __builtin_amdgcn_make_buffer_rsrc((void *)a_tile, 0, 0, kBufferWord3);
  const __amdgpu_buffer_rsrc_t rb_none = __builtin_amdgcn_make_buffer_rsrc((void *)b_tile, 0, 0, kBufferWord3);
  // Per-lane byte offsets.  A (row-contiguous slab loads): row lane / LPR,
  // k 4 * (lane % LPR); B (MFMA layout): row 4 * lg, column lr.
  const int a_row = lane / LPR, a_col = 4 * (lane % LPR);
  const int va = (a_row * lda + a_col) * 4;
  const int b_row = lane / LPRB, b_col = 4 * (lane % LPRB);
  const int vb = SB ? (b_row * ldb + b_col) * 4 : (4 * lg * ldb + lr) * 4;
  float *const stage = lds + wave * G::WAVE_STAGE;
  float *const stage_b = stage + BM * LDA;

  AccT acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < MB * MB / 64; ++r) acc[i][j][r] = 0.0f;

  f32x4 ar[NBUF][A_INSTR];  // A slab as loaded (rows a_row + RPI * i)
  float bf[NBUF][SB ? 1 : C][SB ? 1 : FN][4];  // B fragments (SB = 0)
  f32x4 br[NBUF][SB ? B_INSTR : 1];             // B slab as loaded (SB = 1)

  // The wave runs `rounds` rounds of NBUF slabs: its nk slabs preceded by
  // `lead` = rounds * NBUF - nk zero slabs (fewer than NBUF), so there is no
  // tail to handle.  A zero slab loads through the zero-record resources
  // (zeros, no memory access) and adds exact +0.0 products to the +0.0
  // accumulators: the result is the same bits, and its MFMAs run while the
  // first real slab's loads are in flight.
  const int rounds = (nk + NBUF - 1) / NBUF, lead = rounds * NBUF - nk;

  // Request virtual slab v (real slab v - lead of the wave) into register set `set`.
  auto load = [&](auto sc, int v) __attribute__((always_inline)) {
    constexpr int set = decltype(sc)::value;
    const bool live = v >= lead && v < lead + nk;
    const __amdgpu_buffer_rsrc_t ra = live ? ra_live : ra_none;
    const __amdgpu_buffer_rsrc_t rb = live ? rb_live : rb_none;
    const int k0 = (kb + v - lead) * BK;
#pragma unroll
    for (int i = 0; i < A_INSTR; ++i)
      ar[set][i] =
          __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(ra, va, (k0 + i * RPI * lda) * 4, 0));
    if constexpr (SB) {
#pragma unroll
      for (int i = 0; i < B_INSTR; ++i)
        br[set][i] =
            __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rb, vb, (k0 + i * RPIB) * ldb * 4, 0));
    } else {
#pragma unroll
      for (int c = 0; c < C; ++c)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int s = 0; s < 4; ++s)
            bf[set][c][j][s] = __builtin_bit_cast(
                float, __builtin_amdgcn_raw_buffer_load_b32(rb, vb, ((k0 + c * KC + s) * ldb + j * MB) * 4, 0));
    }
  };
  // A slab -> this wave's LDS tile -> fragments (lane (lr, lg) of block i,
  // chunk c: row i * MB + lr, k c * KC + 4 * lg .. +3), then the MFMAs.  Only
  // this wave touches its tile and a wave's LDS accesses complete in order,
  // so no barrier is needed between the writes, the reads and the next
  // slab's writes.
  auto compute = [&](auto sc) __attribute__((always_inline)) {
    constexpr int set = decltype(sc)::value;
#pragma unroll
    for (int i = 0; i < A_INSTR; ++i)
      *reinterpret_cast<f32x4 *>(stage + (i * RPI + a_row) * LDA + a_col) = ar[set][i];
    if constexpr (SB) {
#pragma unroll
      for (int i = 0; i < B_INSTR; ++i)
        *reinterpret_cast<f32x4 *>(stage_b + (i * RPIB + b_row) * LDB + b_col) = br[set][i];
    }
#pragma unroll
    for (int c = 0; c < C; ++c) {
      f32x4 af[FM];
      float bs[FN][4];
#pragma unroll
      for (int i = 0; i < FM; ++i)
        af[i] = *reinterpret_cast<const f32x4 *>(stage + (i * MB + lr) * LDA + c * KC + 4 * lg);
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          if constexpr (SB) bs[j][s] = stage_b[(c * KC + 4 * lg + s) * LDB + j * MB + lr];
          else bs[j][s] = bf[set][c][j][s];
        }
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j) acc[i][j] = mfma_block<MB>(bs[j][s], af[i][s], acc[i][j]);
    }
  };

  // Prologue: virtual slabs 0 .. NBUF-2 into sets 0 .. NBUF-2.
  static_for<NBUF - 1>([&](auto d) __attribute__((always_inline)) { load(d, decltype(d)::value); });
  // Steady state, unrolled by NBUF so the sets are compile-time: virtual
  // slab t computes from set t % NBUF after requesting slab t + NBUF - 1 into
  // the set slab t - 1 left.
  for (int r = 0; r < rounds; ++r) {
    const int t = r * NBUF;
    static_for<NBUF>([&](auto u) __attribute__((always_inline)) {
      constexpr int U = decltype(u)::value;
      load(std::integral_constant<int, (U + NBUF - 1) % NBUF>{}, t + U + NBUF - 1);
      // Keep the requests ahead of this slab's MFMAs: the scheduler would
      // otherwise sink them to their use in the next round.
      __builtin_amdgcn_sched_barrier(0);
      compute(u);
      __builtin_amdgcn_sched_barrier(0);
    });
  }

  // Partial tile of this wave -> LDS.  Lane (lr, lg) holds, per block and
  // group g < NG, row lr and columns 8g + 4lg .. +3 (MB = 32) or 4lg .. +3
  // (MB = 16) of the block.
  constexpr int NG = MB == 32 ? 4 : 1;
  float *const part = lds;
  __syncthreads();  // every wave is done with its staging tile
  float *own = part + wave * BM * LDP;
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        f32x4 v;
        v.x = acc[i][j][4 * g + 0];
        v.y = acc[i][j][4 * g + 1];
        v.z = acc[i][j][4 * g + 2];
        v.w = acc[i][j][4 * g + 3];
        *reinterpret_cast<f32x4 *>(own + (i * MB + lr) * LDP + j * MB + 8 * g + 4 * lg) = v;
      }
  __syncthreads();

  // Sum the W partials of each 4-column group in wave order, then the epilogue.
  for (int q = tid; q < G::G4; q += NT) {
    const int r = q / (BN / 4), c = (q - r * (BN / 4)) * 4;
    f32x4 v = *reinterpret_cast<const f32x4 *>(part + r * LDP + c);
#pragma unroll
    for (int w = 1; w < W; ++w) v += *reinterpret_cast<const f32x4 *>(part + (w * BM + r) * LDP + c);
    const long m = m0 + r;
    const int n = (int)n0 + c;
    if (splits > 1)  // partial sum of this K range -> workspace slice; the reduction launch runs the epilogue
      *reinterpret_cast<f32x4 *>(p.ws + split * p.ws_slice + m * p.ws_ld + n) = v;
    else
      *reinterpret_cast<f32x4 *>(p.C + m * p.ldc + n) = apply_epi4(v, p.epi, m, n);
  }
}

template <int BM, int BN, int NT, int BK, int SB = wavek_stage_b<BM, BN>()>
hipError_t launch_wavek(const GemmParams &p, dim3 grid, dim3 block, hipStream_t stream) {
  if (block.x * block.y != NT || block.z != 1 || p.splits > 255) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL((wavek_gemm_kernel<BM, BN, NT, BK, SB>), grid, block, 0, stream, p.A, p.B, p.lda, p.ldb, p.K,
                     (int)grid.x, (int)grid.y, p.swizzle | (p.splits << 8) | (int)(block.x << 16), p);
  return hipGetLastError();
}

}  // namespace tfk
