// The streamed (persistent) FP32 GEMM for gfx950: the staged kernel's tile
// math (staged_gemm.hpp: MFMA blocks, k order, LDS layout, schedule), run by
// one workgroup per CU over a sequence of output tiles, for problems with more
// tiles than the chip holds at once (the `persistent` option).
//
// Why: when several rounds of workgroups run, every workgroup of a round ends
// at the same moment and writes its whole C tile at once; under that burst the
// stores back up (4096 x 4096 x 256: ~11 us of each ~33 us round spent
// issuing them) and the CU's matrix cores idle until the next round starts.
// Here a workgroup keeps its LDS and streams K slabs continuously from one
// tile into the next:
//
//  * Slab stream.  Workgroup b owns tiles b, b + G, b + 2G, ... (G = grid
//    size); slab s of its stream is slab s % nk of its tile s / nk.  The
//    global loads for slab s + 1 + DEPTH are issued while slab s computes,
//    across tile boundaries, so a new tile starts with its first slabs
//    already staged (no per-tile prologue).
//  * C through LDS.  At the end of a tile the finished accumulators (epilogue
//    applied) go to an LDS tile Cs; during the next tile's slabs, right after
//    each slab barrier, every thread copies a share of Cs to global memory with
//    coalesced 128-bit stores, so the tile's stores spread over the next
//    tile's matrix work.  The last tile is written after the stream ends.
//  * Tile order.  Tile w is mapped with the XCD-aware order of the staged
//    kernel; workgroup b runs on XCD b % 8, so the tiles one XCD holds at any
//    time share A and B panels in its L2.
//  * Barriers.  One per slab as in the staged kernel, plus three per tile
//    around the end-of-tile drain and the Cs writes (see tile_end), so Cs is
//    never read before it is written or rewritten before it is read.  The
//    bias of a chain that starts with bias_add is loaded into a register as
//    the tile starts and written to LDS between those barriers, so the
//    epilogue reads it from LDS.
//
// Shapes: M, N, K multiples of BM, BN, BK with K an even number of at least 4
// slabs (the host pads or refuses); no split-K.  C must not overlap an input
// (the ABI's noalias pointers): a workgroup's first tile receives throwaway
// stores before its real values.  Same arithmetic per output as the staged
// kernel with the same configuration: the results are bit-identical to it.
#pragma once

#include "staged_gemm.hpp"

namespace tfk {

template <int BM, int BN, int TM, int TN, int BK>
struct StreamedGemm {
  using G = StagedGemm<BM, BN, TM, TN, BK, 1, 1>;
  static constexpr int LDC = BN + 4;  // Cs row stride: 16-lane groups of b128 accesses hit distinct banks
  static constexpr int C_ELEMS = BM * LDC;
  static constexpr int LDS_BYTES = 2 * (G::A_ELEMS + G::B_ELEMS) * 4 + BN * 4 + C_ELEMS * 4;
  static constexpr int C_VECS = BM * BN / 4;                  // float4s per tile
  static constexpr int C_PER = (C_VECS + G::NT - 1) / G::NT;  // per thread
  static_assert(LDS_BYTES <= 160 * 1024, "LDS per workgroup exceeds 160 KB");
  static_assert(C_VECS % G::NT == 0, "the threads must split the tile's float4s evenly");
};

template <int BM, int BN, int TM, int TN, int BK>
__global__ void __launch_bounds__((BM / TM) * (BN / TN))
streamed_gemm_kernel(GemmParams p) {
  using G = StagedGemm<BM, BN, TM, TN, BK, 1, 1>;
  using S = StreamedGemm<BM, BN, TM, TN, BK>;
  constexpr int NT = G::NT, WTM = G::WTM, WTN = G::WTN, NWN = G::NWN, FM = G::FM, FN = G::FN;
  constexpr int LDA = G::LDA, LDB = G::LDB, MB = G::MB, KC = G::KC, LDC = S::LDC;
  using AccT = AccOf<MB>;

  const int tid = threadIdx.y * (BN / TN) + threadIdx.x;  // launch_streamed checks the block
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / NWN, wn = wave - wm * NWN;
  const int lr = lane % MB, lg = lane / MB;

  const int gx = p.N / BN, gy = p.M / BM;
  const int tiles = gx * gy;
  const int nk = p.K / BK;
  // Tiles of this workgroup: blockIdx.x + j * gridDim.x for j < ntiles.
  const int ntiles = (tiles - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x;
  const int total = ntiles * nk;  // slabs in this workgroup's stream
  const long lda = p.lda, ldb = p.ldb;
  const bool bias_lds = p.epi.nops > 0 && p.epi.kind[0] == EPI_BIAS;

  auto tile_origin = [&](int j, long &m0, long &n0) __attribute__((always_inline)) {
    int tm, tn;
    tile_coords(blockIdx.x + j * gridDim.x, gx, gy, p.swizzle, tm, tn);
    m0 = (long)tm * BM;
    n0 = (long)tn * BN;
  };

  __shared__ __attribute__((aligned(16))) float As[2][G::A_ELEMS];
  __shared__ __attribute__((aligned(16))) float Bs[2][G::B_ELEMS];
  __shared__ __attribute__((aligned(16))) float Cs[S::C_ELEMS];
  __shared__ __attribute__((aligned(16))) float bias_s[BN];

  constexpr int DEPTH = (G::A_PER + G::B_PER) <= 8 ? 2 : 1;
  f32x4 ra[DEPTH][G::A_PER], rb[DEPTH][G::B_PER];
  // Per-thread parts of the staging addresses (the tile and slab add a
  // uniform base).
  int a_off[G::A_PER], b_off[G::B_PER], a_lds[G::A_PER], b_lds[G::B_PER];
#pragma unroll
  for (int it = 0; it < G::A_PER; ++it) {
    int r, c;
    G::a_item(tid + it * NT, r, c);  // bank-conflict-free LDS writes
    a_off[it] = r * (int)lda + c;
    a_lds[it] = r * LDA + c;
  }
#pragma unroll
  for (int it = 0; it < G::B_PER; ++it) {
    const int q = tid + it * NT;
    const int r = q / (BN / 4), c = (q - r * (BN / 4)) * 4;
    b_off[it] = r * (int)ldb + c;
    b_lds[it] = r * LDB + c;
  }
  // The next slab to load, tracked incrementally (loads are issued in stream
  // order): slab ld_kt of the tile whose A and B slabs start at ld_a, ld_b.
  // Loads run at most DEPTH + 1 <= 3 slabs ahead of the slab being computed
  // and a tile has at least 4 slabs (the host checks), so the loads enter
  // tile j + 1 only after tile j has started; the origin of tile j + 1
  // (nx_a, nx_b) is computed then, on the rare tile-boundary path, and the
  // loads switch to it with scalar selects -- no branch in the slab loop,
  // where one would cost conservative memory waits at its edges.
  // Loads are unconditional: past the end of the stream the position stays on
  // the last slab (in bounds; those registers are never stored), so every
  // load is issued in every slab and the compiler can wait for exactly the
  // older staging set before the LDS stores (a conditional load makes it
  // wait for all loads in flight, which would cut the prefetch to < 1 slab).
  int ld_kt = 0, ld_left = total;
  const float *ld_a, *ld_b, *nx_a, *nx_b;
  auto origin_ptrs = [&](int j, const float *&a, const float *&b) __attribute__((always_inline)) {
    long m0, n0;
    tile_origin(j < ntiles ? j : ntiles - 1, m0, n0);
    a = p.A + m0 * lda;
    b = p.B + n0;
  };
  origin_ptrs(0, ld_a, ld_b);
  origin_ptrs(1, nx_a, nx_b);
  auto load_slab = [&](auto sc) __attribute__((always_inline)) {
    constexpr int set = decltype(sc)::value;
#pragma unroll
    for (int it = 0; it < G::A_PER; ++it)
      if (G::A_VECS % NT == 0 || tid + it * NT < G::A_VECS) ra[set][it] = *reinterpret_cast<const f32x4 *>(ld_a + a_off[it]);
#pragma unroll
    for (int it = 0; it < G::B_PER; ++it)
      if (G::B_VECS % NT == 0 || tid + it * NT < G::B_VECS) rb[set][it] = *reinterpret_cast<const f32x4 *>(ld_b + b_off[it]);
    const bool adv = --ld_left > 0;
    const bool wrap = ld_kt + 1 == nk;
    const int kt_next = wrap ? 0 : ld_kt + 1;
    const float *a_next = wrap ? nx_a : ld_a + BK;
    const float *b_next = wrap ? nx_b : ld_b + BK * ldb;
    ld_kt = adv ? kt_next : ld_kt;
    ld_a = adv ? a_next : ld_a;
    ld_b = adv ? b_next : ld_b;
  };
  auto store_slab = [&](auto sc, int buf) __attribute__((always_inline)) {
    constexpr int set = decltype(sc)::value;
#pragma unroll
    for (int it = 0; it < G::A_PER; ++it)
      if (G::A_VECS % NT == 0 || tid + it * NT < G::A_VECS) *reinterpret_cast<f32x4 *>(&As[buf][a_lds[it]]) = ra[set][it];
#pragma unroll
    for (int it = 0; it < G::B_PER; ++it)
      if (G::B_VECS % NT == 0 || tid + it * NT < G::B_VECS) *reinterpret_cast<f32x4 *>(&Bs[buf][b_lds[it]]) = rb[set][it];
  };

  constexpr int C = BK / KC, MID = C >= 2 ? C / 2 - 1 : 0;
  f32x4 af[2][FM];
  float bf[2][FN][4];
  auto load_frags = [&](int buf, int kc, int slot) __attribute__((always_inline)) {
    const float *as = As[buf] + (wm * WTM + lr) * LDA + 4 * lg + kc * KC;
    const float *bs = Bs[buf] + (4 * lg + kc * KC) * LDB + wn * WTN + lr;
#pragma unroll
    for (int i = 0; i < FM; ++i) af[slot][i] = *reinterpret_cast<const f32x4 *>(as + i * MB * LDA);
#pragma unroll
    for (int jj = 0; jj < FN; ++jj)
#pragma unroll
      for (int s = 0; s < 4; ++s) bf[slot][jj][s] = bs[s * LDB + jj * MB];
  };

  AccT acc[FM][FN];
  auto zero_acc = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int jj = 0; jj < FN; ++jj)
#pragma unroll
        for (int r = 0; r < MB * MB / 64; ++r) acc[i][jj][r] = 0.0f;
  };

  // Draining Cs: thread tid's share of the finished tile at (cm0, cn0) is
  // the float4s tid + d * NT, d < C_PER; `drained` counts those written.
  long cm0 = 0, cn0 = 0;
  tile_origin(0, cm0, cn0);
  int drained = 0;
  auto drain_one = [&]() __attribute__((always_inline)) {
    const int q = tid + drained * NT;
    const int r = q / (BN / 4), c = (q - r * (BN / 4)) * 4;
    const f32x4 v = *reinterpret_cast<const f32x4 *>(&Cs[r * LDC + c]);
    *reinterpret_cast<f32x4 *>(p.C + (cm0 + r) * p.ldc + cn0 + c) = v;
    ++drained;
  };
  // A tile's C_PER float4s go out over the next tile's first slabs, DR per
  // slab, with no condition: stores count in the same wait counter as the
  // staging loads, and a store the compiler cannot count makes it wait for
  // every load in flight.  Once a tile is drained the index stays on its last
  // float4 and rewrites the same value; during a workgroup's first tile the
  // "previous" tile is that first tile itself, so those stores put
  // not-yet-computed values into its own C region, which its real values
  // overwrite after the tile-end barriers.  With at least 4 slabs per tile,
  // DR = C_PER / 4 drains a tile in time.
  constexpr int DR = (S::C_PER + 3) / 4;
  auto drain_some = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int e = 0; e < DR; ++e) {
      const int d = min(drained, S::C_PER - 1);
      const int q = tid + d * NT;
      const int r = q / (BN / 4), c = (q - r * (BN / 4)) * 4;
      const f32x4 v = *reinterpret_cast<const f32x4 *>(&Cs[r * LDC + c]);
      *reinterpret_cast<f32x4 *>(p.C + (cm0 + r) * p.ldc + cn0 + c) = v;
      drained = min(drained + 1, S::C_PER);
    }
  };

  f32x4 bias_reg = {0.0f, 0.0f, 0.0f, 0.0f};
  auto tile_start = [&](int j) __attribute__((always_inline)) {
    origin_ptrs(j + 1, nx_a, nx_b);
    if (bias_lds && tid < BN / 4) {
      long m0, n0;
      tile_origin(j, m0, n0);
      bias_reg = *reinterpret_cast<const f32x4 *>(p.epi.ptr[0] + n0 + 4 * tid);
    }
  };

  // Epilogue of tile j.  Barrier 1: the previous tile's Cs writes (and
  // bias_s reads) are done in every thread, whether or not a slab barrier
  // came since; then this thread drains the rest of that tile and writes the
  // new bias.  Barrier 2: every drain read is done; Cs can be rewritten.
  // Barrier 3: the new Cs is complete before any thread drains it.
  constexpr int NG = MB == 32 ? 4 : 1;
  auto tile_end = [&](int j) __attribute__((always_inline)) {
    __syncthreads();
    while (drained < S::C_PER) drain_one();
    if (bias_lds && tid < BN / 4) *reinterpret_cast<f32x4 *>(&bias_s[4 * tid]) = bias_reg;
    __syncthreads();
    long m0, n0;
    tile_origin(j, m0, n0);
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int r = wm * WTM + i * MB + lr;
#pragma unroll
      for (int jj = 0; jj < FN; ++jj)
#pragma unroll
        for (int g = 0; g < NG; ++g) {
          const int c = wn * WTN + jj * MB + 8 * g + 4 * lg;
          f32x4 v;
          v.x = acc[i][jj][4 * g + 0];
          v.y = acc[i][jj][4 * g + 1];
          v.z = acc[i][jj][4 * g + 2];
          v.w = acc[i][jj][4 * g + 3];
          v = bias_lds ? apply_epi4(v + *reinterpret_cast<const f32x4 *>(&bias_s[c]), p.epi, m0 + r, (int)n0 + c, 1)
                       : apply_epi4(v, p.epi, m0 + r, (int)n0 + c);
          *reinterpret_cast<f32x4 *>(&Cs[r * LDC + c]) = v;
        }
    }
    cm0 = m0;
    cn0 = n0;
    drained = 0;
    zero_acc();
    __syncthreads();
  };

  // The grid has at most one workgroup per tile and a tile at least 4 slabs
  // (the host checks both), so every stream holds at least 4 slabs and the
  // prologue's loads need no condition -- a skipped load on one path would
  // make the compiler wait for the newest staging set on every slab.
  zero_acc();
  tile_start(0);
  load_slab(std::integral_constant<int, 0>{});
  store_slab(std::integral_constant<int, 0>{}, 0);
  load_slab(std::integral_constant<int, DEPTH - 1>{});
  if constexpr (DEPTH == 2) load_slab(std::integral_constant<int, 0>{});
  __syncthreads();
  load_frags(0, 0, 0);

  // Stream slab s (buffer P = s & 1): the staged kernel's slab schedule, with
  // a share of the previous tile's C written where the slab stages the next.
  // `more` (a slab follows in the stream) is compile-time: false only for the
  // stream's last slab, peeled below, so the steady state has no condition
  // around its stores and loads.
  auto slab = [&](auto par, auto more_c) __attribute__((always_inline)) {
    constexpr int P = decltype(par)::value;
    constexpr bool more = decltype(more_c)::value;
#pragma unroll
    for (int kc = 0; kc < C; ++kc) {
      const int fs = kc & 1;
      if (C == 1 && more) {
        store_slab(std::integral_constant<int, DEPTH == 2 ? (P ^ 1) : 0>{}, P ^ 1);
        load_slab(std::integral_constant<int, DEPTH == 2 ? (P ^ 1) : 0>{});
        drain_some();
      }
      if (kc + 1 < C) {
        load_frags(P, kc + 1, fs ^ 1);
      } else if (more) {
        __syncthreads();
        load_frags(P ^ 1, 0, fs ^ 1);
      }
#pragma unroll
      for (int k4 = 0; k4 < 4; ++k4)
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int jj = 0; jj < FN; ++jj) acc[i][jj] = mfma_block<MB>(bf[fs][jj][k4], af[fs][i][k4], acc[i][jj]);
      constexpr int NM = 4 * FM * FN;
      if constexpr (FM * FN == 1 && MB == 32) {
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
      } else if constexpr (FM * FN == 1) {
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
          __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        }
      } else if constexpr (NT <= 512) {
        __builtin_amdgcn_sched_group_barrier(0x008, NM - 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, FM + 4 * FN, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
      } else {
#pragma unroll
        for (int q = 0; q < NM; ++q) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      if (C >= 2 && kc == MID && more) {
        store_slab(std::integral_constant<int, DEPTH == 2 ? (P ^ 1) : 0>{}, P ^ 1);
        load_slab(std::integral_constant<int, DEPTH == 2 ? (P ^ 1) : 0>{});
        drain_some();
      }
    }
    if constexpr (C % 2 == 1) {
#pragma unroll
      for (int i = 0; i < FM; ++i) af[0][i] = af[1][i];
#pragma unroll
      for (int jj = 0; jj < FN; ++jj)
#pragma unroll
        for (int k4 = 0; k4 < 4; ++k4) bf[0][jj][k4] = bf[1][jj][k4];
    }
  };
  // Tiles outside, slabs inside: a tile has an even number of slabs (the host
  // checks), so every tile starts on buffer 0 and the inner loop is the staged
  // kernel's unrolled slab pair.  At a tile's end its accumulators are final;
  // they go to Cs while the next tile's first slab is already in LDS and its
  // fragments in registers.  The last tile, whose last slab loads nothing,
  // has its own loop after this one: on a path back into the slab loop after
  // it, fewer loads would be in flight, and the compiler would wait for the
  // younger staging set on every slab.
  using B0 = std::integral_constant<int, 0>;
  using B1 = std::integral_constant<int, 1>;
  using More = std::integral_constant<bool, true>;
  using Last = std::integral_constant<bool, false>;
  for (int j = 0; j + 1 < ntiles; ++j) {
    for (int kt = 0; kt < nk; kt += 2) {
      slab(B0{}, More{});
      slab(B1{}, More{});
    }
    tile_end(j);
    tile_start(j + 1);
  }
  for (int kt = 2; kt < nk; kt += 2) {
    slab(B0{}, More{});
    slab(B1{}, More{});
  }
  slab(B0{}, More{});
  slab(B1{}, Last{});
  tile_end(ntiles - 1);

  // The last tile's C.
  __syncthreads();
  while (drained < S::C_PER) drain_one();
}

template <int BM, int BN, int TM, int TN, int BK>
hipError_t launch_streamed(const GemmParams &p, dim3 grid, dim3 block, hipStream_t stream) {
  if (block.x != BN / TN || block.y != BM / TM || block.z != 1) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL((streamed_gemm_kernel<BM, BN, TM, TN, BK>), grid, block, 0, stream, p);
  return hipGetLastError();
}

}  // namespace tfk
