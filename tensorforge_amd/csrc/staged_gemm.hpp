// The staged FP32 GEMM family for gfx950 (CDNA4): C = epi(A @ B) on wave64
// MFMA tiles.  This is the kernel the reference pipeline generates for
// "tile-k=BK" options (docs/stage8.md:9-30; lib/Transforms/Gpu.cpp:229-316),
// redesigned for the matrix cores instead of translated:
//
//  * Option mapping.  block-tile=BM,BN is the workgroup tile; the workgroup has
//    (BM/TM)*(BN/TN) threads as in the reference, i.e. that many / 64 waves.
//    thread-tile=TM,TN gives each lane TM*TN accumulators, so a wave owns an
//    (8*TM) x (8*TN) output tile built from MB x MB MFMA blocks: MB = 32 when
//    both sides are multiples of 32 (v_mfma_f32_32x32x2_f32), else MB = 16
//    (v_mfma_f32_16x16x4_f32, the same FP32 rate), which lets small block
//    tiles (thread-tile 2,2 / 2,4 / 4,2) run 4x as many waves.
//  * Math.  The MFMA with the operands swapped (the B tile feeds src0, the A
//    tile src1), so each lane's accumulators are runs of 4 consecutive columns
//    of one output row: the epilogue reads bias with one 128-bit load and
//    writes C with 128-bit stores.
//  * K order.  A k-chunk holds KC = 256 / MB k values; lane group g = lane / MB
//    and MFMA step s take k = KC*kc + 4*g + s, so every lane's A fragment is 4
//    consecutive k of one row (one ds_read_b128) and its B fragment 4 rows of
//    one column.  The sum order differs from the reference's sequential k;
//    parity is the reference's own FP64 error bound, which holds for any
//    order (python/tforge_cpu.py:263-271).
//  * Staging (promote=1).  A tile [BM][BK+4 or +8] and B tile [BK][BN+8 or +4] in LDS,
//    double-buffered, one barrier per slab.  Two register staging sets where
//    a thread stages few vectors: the global loads of slab t+3 are issued in
//    the middle of slab t, two slabs before they are written to LDS (in the
//    middle of slab t+2), so the LDS writes do not wait on HBM latency under
//    full-chip load (one set, 1.5 slabs ahead, for the register-heavy
//    configurations); the slab loop is unrolled by two so buffer and set
//    indices are compile-time.  (The loads are conditional near the end of
//    K, so the compiler's wait before every other slab's stores covers both
//    sets; loads issued a slab earlier have landed by then, and clamped
//    unconditional loads with exact waits measured no faster.)  The barrier sits before the slab's last
//    chunk so those MFMAs hide the next slab's first LDS reads.  Each
//    chunk's MFMAs are scheduled around the next chunk's fragment reads in a
//    measured order.  Row padding makes the b128 fragment reads and the b32
//    B reads bank-conflict-free.
//  * Epilogue in registers: bias (staged in LDS during the prologue when the
//    chain starts with bias_add), IEEE relu, residual add; 128-bit stores.
//  * vectorize=1: 128-bit global loads and LDS accesses; vectorize=0: 32-bit.
//  * promote=0: no LDS; each wave streams its fragments from global memory
//    (through L2), the reference's "+tiling" rung (bench/stage9_ablation.py:23-28).
//  * Tile order.  Workgroups are dealt round-robin to the 8 XCDs; with
//    swizzle=1 the workgroups one XCD receives own a compact block of tiles
//    (grouped by 4 tile rows), so they share A and B panels in that XCD's L2.
//  * Split-K (an option the reference does not have): gridDim.z workgroups
//    per output tile, each over a contiguous range of K slabs, so shapes with
//    few output tiles (64 x 4096 x 4096) still fill 256 CUs.  Partial sums go
//    to a workspace with ordinary cached stores; a second, HBM-bound kernel
//    adds them in a fixed order (deterministic) and applies the epilogue.
//  * Shapes: multiples of (BM, BN, BK), padded by the host as the reference
//    runner does (runners/gpu/tforge-gpu-bench.cu:214-232); or, with
//    masked=1 (the mask-edges option), any shape: edge tiles and the K tail
//    load zeros outside the matrices and store only inside, so the result is
//    bit-identical to the padded problem's without the pad copies.
#pragma once

#include <type_traits>

#include "epilogue.hpp"

namespace tfk {

typedef float f32x16 __attribute__((ext_vector_type(16)));

// One MFMA on an MB x MB block: acc += src0 (4 x MB, from B) ^T-contracted with
// src1 (from A); see the lane layouts in the header comment.
template <int MB>
using AccOf = typename std::conditional<MB == 32, f32x16, f32x4>::type;
template <int MB>
__device__ __forceinline__ AccOf<MB> mfma_block(float b, float a, AccOf<MB> c) {
  if constexpr (MB == 32) return __builtin_amdgcn_mfma_f32_32x32x2f32(b, a, c, 0, 0, 0);
  else return __builtin_amdgcn_mfma_f32_16x16x4f32(b, a, c, 0, 0, 0);
}

// Output tile (tm, tn) of linear tile index w on a gx x gy tile grid.  With
// swizzle, consecutive w are dealt to the 8 XCDs round-robin (as the hardware
// deals workgroups), so the indices one XCD receives are remapped to a
// compact block of tiles, grouped by 4 tile rows.
__device__ __forceinline__ void tile_coords(int w, int gx, int gy, int swizzle, int &tm, int &tn) {
  const int total = gx * gy;
  if (!swizzle) {
    tm = w / gx;
    tn = w - tm * gx;
    return;
  }
  constexpr int kXcds = 8;
  if (total % kXcds == 0) w = (w % kXcds) * (total / kXcds) + w / kXcds;
  constexpr int kGroup = 4;
  const int group = w / (kGroup * gx);
  const int first = group * kGroup;
  const int rows = min(gy - first, kGroup);
  const int r = w - group * kGroup * gx;
  tm = first + r % rows;
  tn = r / rows;
}

__device__ __forceinline__ void staged_tile_coords(int gx, int gy, int swizzle, int &tm, int &tn) {
  tile_coords(blockIdx.y * gx + blockIdx.x, gx, gy, swizzle, tm, tn);
}

// Calls f(integral_constant<0>), ..., f(integral_constant<N-1>) in order.
template <int N, typename F>
__device__ __forceinline__ void static_for(F &&f) {
  if constexpr (N > 0) {
    static_for<N - 1>(f);
    f(std::integral_constant<int, N - 1>{});
  }
}

// One staging vector (a float or a 4-vector) by a raw buffer load at a byte
// offset from the resource's base.
template <typename VT>
__device__ __forceinline__ VT buffer_load_vt(__amdgpu_buffer_rsrc_t rs, int byte_off) {
  if constexpr (sizeof(VT) == 16) return __builtin_bit_cast(VT, __builtin_amdgcn_raw_buffer_load_b128(rs, byte_off, 0, 0));
  else return __builtin_bit_cast(VT, __builtin_amdgcn_raw_buffer_load_b32(rs, byte_off, 0, 0));
}

// Write element e of a staging register (a float or a 4-vector).
__device__ __forceinline__ void put(float &v, int, float x) { v = x; }
__device__ __forceinline__ void put(f32x4 &v, int e, float x) { v[e] = x; }

template <int BM, int BN, int TM, int TN, int BK, int PROMOTE, int VEC>
struct StagedGemm {
  static constexpr int NT = (BM / TM) * (BN / TN);
  static constexpr int WTM = 8 * TM, WTN = 8 * TN;
  static constexpr int NWM = BM / WTM, NWN = BN / WTN;
  static constexpr int MB = (WTM % 32 == 0 && WTN % 32 == 0) ? 32 : 16;  // MFMA block
  static constexpr int KC = 256 / MB;                                     // k per chunk
  static constexpr int FM = WTM / MB, FN = WTN / MB;
  // LDS A row stride (floats).  A fragment read (ds_read_b128) has lanes
  // (lr, lg) at lr * LDA + 4 * lg: conflict-free for MB = 32 with BK + 4, and
  // for MB = 16 (4 lane groups on one row) only with LDA = 8 mod 16, so BK + 8
  // (measured on gfx950: BK + 4 costs 4 bank-conflict cycles per read).
  static constexpr int LDA = BK + ((WTM % 32 == 0 && WTN % 32 == 0) ? 4 : 8);
  // LDS B row stride: the 64 / MB lane groups read rows 4 apart; +8 (MB = 32)
  // or +4 (MB = 16) puts them in disjoint banks.
  static constexpr int LDB = BN + (MB == 32 ? 8 : 4);
  static constexpr int A_ELEMS = BM * LDA, B_ELEMS = BK * LDB;
  // Two A and B tile buffers, plus the tile's BN bias values.
  static constexpr int LDS_BYTES = PROMOTE ? 2 * (A_ELEMS + B_ELEMS) * 4 + BN * 4 : 0;
  // Global -> register staging per thread and slab.
  static constexpr int VW = VEC ? 4 : 1;
  static constexpr int A_VECS = BM * BK / VW, B_VECS = BK * BN / VW;
  static constexpr int A_PER = (A_VECS + NT - 1) / NT, B_PER = (B_VECS + NT - 1) / NT;

  // A staging vector q -> (row r, column c) of the BM x BK slab; thread tid
  // stages q = tid + it * NT.  A 128-bit LDS write is served 8 lanes per
  // cycle over 32 banks, so the 8 lanes of a pass must cover 8 distinct
  // 4-bank groups; row r starts at group (r * LDA / 4) mod 8.  With BK >= 32
  // a pass stays in one row (8 consecutive groups).  With BK = 16 a pass
  // holds two whole rows, r and r + d with d * LDA / 4 = 4 mod 8 (d = 4 for
  // LDA = 20, d = 2 for LDA = 24; consecutive rows share a group: 8 conflict
  // cycles per write instruction, measured); with BK = 8 and LDA / 4 odd,
  // four rows r, r + 2, r + 4, r + 6.  The rows of one wave's loads are the
  // same 16 whole rows as with the row-major order, so global accesses
  // coalesce as before.
  static __host__ __device__ __forceinline__ void a_item(int q, int &r, int &c) {
    constexpr int CPR = BK / VW, L = LDA / 4;
    if constexpr (VEC && CPR == 4 && (L % 2 == 1 || L % 4 == 2)) {
      const int s = q & 31, pass = s >> 3, i = s & 7;
      const int base = L % 2 == 1 ? pass : (pass & 1) + 4 * (pass >> 1);
      r = 8 * (q >> 5) + base + (L % 2 == 1 ? 4 : 2) * (i >> 2);
      c = 4 * (i & 3);
    } else if constexpr (VEC && CPR == 2 && L % 2 == 1) {
      const int s = q & 15, i = s & 7;
      r = 8 * (q >> 4) + (s >> 3) + 2 * (i >> 1);
      c = 4 * (i & 1);
    } else {
      r = q / CPR;
      c = (q - r * CPR) * VW;
    }
  }

  static_assert(BM % TM == 0 && BN % TN == 0, "block tile must be a multiple of the thread tile");
  static_assert(NWM * NWN * 64 == NT, "waves must tile the block");
  static_assert(WTM % 16 == 0 && WTN % 16 == 0, "wave tile must be made of 16x16 or 32x32 MFMA blocks");
  static_assert(BK % KC == 0, "tile-k must be a multiple of the k-chunk (8 for 32x32 blocks, 16 for 16x16)");
  static_assert(NT <= 1024, "at most 1024 threads per workgroup");
  static_assert(LDS_BYTES <= 160 * 1024, "LDS per workgroup exceeds 160 KB");
};

// The kernel's first ten arguments repeat the fields of `p` that the prologue
// needs before its first global loads, as scalars: the library is built with
// kernel-argument preloading (-mllvm -amdgpu-kernarg-preload-count), so the
// hardware puts scalar leading arguments in SGPRs at wave launch, while the
// by-value struct is read from the kernel-argument segment (a ~1.5k-cycle
// round trip measured at the start of every wave).  gx, gy = gridDim.x, .y;
// flags = swizzle | splits << 8.
template <int BM, int BN, int TM, int TN, int BK, int PROMOTE, int VEC, int MASK>
__global__ void __launch_bounds__((BM / TM) * (BN / TN))
staged_gemm_kernel(const float *pA, const float *pB, long plda, long pldb, int pK, int gx, int gy, int flags, int pM,
                   int pN, GemmParams p) {
  p.A = pA;
  p.B = pB;
  p.lda = plda;
  p.ldb = pldb;
  p.K = pK;
  p.M = pM;
  p.N = pN;
  p.swizzle = flags & 255;
  p.splits = flags >> 8;
  using G = StagedGemm<BM, BN, TM, TN, BK, PROMOTE, VEC>;
  constexpr int NT = G::NT, WTM = G::WTM, WTN = G::WTN, NWN = G::NWN, FM = G::FM, FN = G::FN;
  constexpr int LDA = G::LDA, LDB = G::LDB, VW = G::VW, MB = G::MB, KC = G::KC;
  using AccT = AccOf<MB>;

  // The block is (BN / TN) x (BM / TM) threads (launch_staged checks): with
  // blockDim.x read from the dispatch packet instead, every wave waited for
  // that load (~1.3k cycles) before its first global loads.
  const int tid = threadIdx.y * (BN / TN) + threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / NWN, wn = wave - wm * NWN;
  const int lr = lane % MB, lg = lane / MB;  // row/column within a block, k group

  int tile_m, tile_n;
  staged_tile_coords(gx, gy, p.swizzle, tile_m, tile_n);
  const long m0 = (long)tile_m * BM, n0 = (long)tile_n * BN;
  const long lda = p.lda, ldb = p.ldb;
  // Split-K: workgroup z reduces K slabs [kb, ke).
  const int nk_all = (p.K + BK - 1) / BK;
  const int splits = p.splits > 1 ? p.splits : 1, split = blockIdx.z;
  // (No 64-bit division in the common single-split case.)
  const int kb = splits == 1 ? 0 : (int)((long)nk_all * split / splits);
  const int ke = splits == 1 ? nk_all : (int)((long)nk_all * (split + 1) / splits);
  const long kbase = (long)kb * BK;
  const float *__restrict__ A = p.A + m0 * lda + kbase;
  const float *__restrict__ B = p.B + n0 + kbase * ldb;
  // Masked shapes: tiles that cross M or N, slabs that cross K, and rows that
  // are not 16-byte aligned take the guarded paths; the rest run unguarded.
  static_assert(!MASK || PROMOTE, "masked instantiations stage through LDS");
  const bool edge = MASK && (m0 + BM > p.M || n0 + BN > p.N);

  AccT acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < MB * MB / 64; ++r) acc[i][j][r] = 0.0f;

  const int nk = ke - kb;

  // When the chain starts with bias_add (mbr, the residual block) the
  // tile's BN bias values are staged in LDS during the prologue, so the
  // epilogue reads them from LDS instead of starting on a cold global load.
  // Not for split-K (the reduction applies the epilogue) or edge tiles
  // (their columns may leave the matrix).
  __shared__ __attribute__((aligned(16))) float bias_s[BN];
  const bool bias_early = PROMOTE && splits == 1 && !edge && p.epi.nops > 0 && p.epi.kind[0] == EPI_BIAS;

  if constexpr (PROMOTE) {
    __shared__ __attribute__((aligned(16))) float As[2][G::A_ELEMS];
    __shared__ __attribute__((aligned(16))) float Bs[2][G::B_ELEMS];
    using VT = typename std::conditional<VEC, f32x4, float>::type;
    // Staging sets in registers: two (loads two slabs ahead) when a thread
    // stages few vectors per slab, else one (loads 1.5 slabs ahead).
    constexpr int DEPTH = (G::A_PER + G::B_PER) <= 8 ? 2 : 1;
    VT ra[DEPTH][G::A_PER], rb[DEPTH][G::B_PER];

    // Masked instantiations (MASK = 1).  Rows of A at or past M and columns of B at
    // or past N only reach outputs that are never stored, so a slab that does
    // not hold the last K row loads them from a nearby valid element (row
    // M-1, column N-4) with the same 128-bit loads as the unmasked path.
    // The slab holding row K-1 (and every slab when N < 4) is "guarded":
    // element by element, with zeros outside the matrices, so the K tail adds
    // exact zeros as the pad path's zero-padded copies do.  A and B rows that
    // are not 16-byte aligned (K or N not a multiple of 4) use unaligned
    // 128-bit loads, which gfx950 serves at 4-byte alignment.  Offsets are
    // 32-bit from the matrices' base pointers (the host bounds M*K and K*N).
    const int Mi = p.M, Ni = p.N, Ki = p.K, m0i = (int)m0, n0i = (int)n0, kbi = (int)kbase;
    auto guarded = [&](int k0) __attribute__((always_inline)) { return MASK && (kbi + k0 + BK >= Ki || Ni < 4); };
    auto a_in = [&](int q, int k0, int e) __attribute__((always_inline)) {
      int r, c;
      G::a_item(q, r, c);
      return m0i + r < Mi && kbi + k0 + c + e < Ki;
    };
    auto b_in = [&](int q, int k0, int e) __attribute__((always_inline)) {
      const int r = q / (BN / VW), c = (q - r * (BN / VW)) * VW;
      return kbi + k0 + r < Ki && n0i + c + e < Ni;
    };
    auto load16 = [](const float *src) {
      VT v;
      __builtin_memcpy(&v, src, sizeof(VT));
      return v;
    };
    // Per-thread part of each B staging address: a slab then adds only the
    // uniform k0 * ldb (one scalar product) instead of recomputing
    // (k0 + r) * ldb per thread in 64-bit vector arithmetic.
    // (The masked twins' clamped loads do the same with 32-bit offsets.)
    const float *b_src[G::B_PER];
    int b_off[G::B_PER];
#pragma unroll
    for (int it = 0; it < G::B_PER; ++it) {
      const int q = tid + it * NT;
      const int r = q / (BN / VW), c = (q - r * (BN / VW)) * VW;
      b_src[it] = B + r * ldb + c;
      b_off[it] = (kbi + r) * (int)ldb + (n0i + c < Ni ? n0i + c : Ni - VW);
    }
    // `sc` is std::integral_constant<int, set>: the staging set is compile-time
    // even where the lambda is not inlined, so the registers stay registers.
    // `gm` (std::integral_constant<int, 0 or 1>): 0 when the caller knows
    // the slab is not guarded (the masked kernels' steady state, see the slab
    // loop), so the guarded branch is not compiled in.
    // Buffer loads (`bc` = BufOn; unmasked staging, and the masked kernels'
    // unguarded slabs): the slab's base addresses go into two buffer
    // resources (scalar 64-bit arithmetic) and each thread keeps one 32-bit
    // byte offset per vector, so a global load carries no 64-bit vector
    // address add.  Between the MFMAs of one wave per
    // SIMD those adds cost 1.5 us at 1024^3 (64x64 t4x4 k16: 19.3 -> 17.75 us
    // back to back) and 6 us at 2048^3 (128x128 t8x8 k16: 126.4 -> 120.0 us).
    // Used only when every offset fits 31 bits (the caller checks BM * lda and
    // BK * ldb); otherwise the same loop runs with flat loads.  Masked
    // kernels: A rows clamped to M - 1 as in their flat loads, offsets from
    // the tile's first row; B columns are absolute (clamped to N - 4), so B's
    // base is the slab's first row of the matrix.
    using BufOn = std::integral_constant<int, 1>;
    using BufOff = std::integral_constant<int, 0>;
    auto buf_rsrc = [](const float *base) __attribute__((always_inline)) {
      return __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(base), 0, 0x7fffffff, 0x00020000);
    };
    auto a_byte = [&](int it) __attribute__((always_inline)) {
      int r, c;
      G::a_item(tid + it * NT, r, c);
      if constexpr (MASK) r = min(m0i + r, Mi - 1) - m0i;
      return (int)((r * lda + c) * 4);
    };
    auto b_byte = [&](int it) __attribute__((always_inline)) {
      if constexpr (MASK) return (b_off[it] - kbi * (int)ldb) * 4;
      const int q = tid + it * NT, r = q / (BN / VW), c = (q - r * (BN / VW)) * VW;
      return (int)((r * ldb + c) * 4);
    };
    auto b_base = [&](int k0) __attribute__((always_inline)) {
      return MASK ? p.B + (kbase + k0) * ldb : B + (long)k0 * ldb;
    };
    auto buf_slab = [&](auto sc, int k0) __attribute__((always_inline)) {
      constexpr int set = decltype(sc)::value;
      const __amdgpu_buffer_rsrc_t rsa = buf_rsrc(A + k0), rsb = buf_rsrc(b_base(k0));
#pragma unroll
      for (int it = 0; it < G::A_PER; ++it)
        if (G::A_VECS % NT == 0 || tid + it * NT < G::A_VECS) ra[set][it] = buffer_load_vt<VT>(rsa, a_byte(it));
#pragma unroll
      for (int it = 0; it < G::B_PER; ++it)
        if (G::B_VECS % NT == 0 || tid + it * NT < G::B_VECS) rb[set][it] = buffer_load_vt<VT>(rsb, b_byte(it));
    };
    auto load_slab = [&](auto sc, auto gm, int k0, auto bc) __attribute__((always_inline)) {
      constexpr int set = decltype(sc)::value;
      if constexpr (!MASK && decltype(bc)::value) {
        buf_slab(sc, k0);
      } else if constexpr (!MASK) {
#pragma unroll
        for (int it = 0; it < G::A_PER; ++it) {
          const int q = tid + it * NT;
          if (G::A_VECS % NT == 0 || q < G::A_VECS) {
            int r, c;
            G::a_item(q, r, c);
            ra[set][it] = *reinterpret_cast<const VT *>(A + r * lda + k0 + c);
          }
        }
#pragma unroll
        for (int it = 0; it < G::B_PER; ++it) {
          const int q = tid + it * NT;
          if (G::B_VECS % NT == 0 || q < G::B_VECS) rb[set][it] = *reinterpret_cast<const VT *>(b_src[it] + k0 * ldb);
        }
      } else if (decltype(gm)::value == 0 || !guarded(k0)) {
        if constexpr (decltype(bc)::value) {
          buf_slab(sc, k0);
          return;
        }
#pragma unroll
        for (int it = 0; it < G::A_PER; ++it) {
          const int q = tid + it * NT;
          if (G::A_VECS % NT == 0 || q < G::A_VECS) {
            int r, c;
            G::a_item(q, r, c);
            ra[set][it] = load16(p.A + (min(m0i + r, Mi - 1) * (int)lda + kbi + k0 + c));
          }
        }
#pragma unroll
        for (int it = 0; it < G::B_PER; ++it) {
          const int q = tid + it * NT;
          if (G::B_VECS % NT == 0 || q < G::B_VECS) {
            rb[set][it] = load16(p.B + (b_off[it] + k0 * (int)ldb));
          }
        }
      } else {
#pragma unroll
        for (int it = 0; it < G::A_PER; ++it) {
          const int q = tid + it * NT;
          if (G::A_VECS % NT == 0 || q < G::A_VECS) {
            int r, c;
            G::a_item(q, r, c);
            const int base = (m0i + r) * (int)lda + kbi + k0 + c;
#pragma unroll
            for (int e = 0; e < VW; ++e) put(ra[set][it], e, p.A[a_in(q, k0, e) ? base + e : 0]);
          }
        }
#pragma unroll
        for (int it = 0; it < G::B_PER; ++it) {
          const int q = tid + it * NT;
          if (G::B_VECS % NT == 0 || q < G::B_VECS) {
            const int r = q / (BN / VW), c = (q - r * (BN / VW)) * VW;
            const int base = (kbi + k0 + r) * (int)ldb + n0i + c;
#pragma unroll
            for (int e = 0; e < VW; ++e) put(rb[set][it], e, p.B[b_in(q, k0, e) ? base + e : 0]);
          }
        }
      }
    };
    auto store_slab = [&](auto sc, auto gm, int buf, int k0) __attribute__((always_inline)) {
      constexpr int set = decltype(sc)::value;
      if (MASK && decltype(gm)::value == 1 && guarded(k0)) {
#pragma unroll
        for (int it = 0; it < G::A_PER; ++it)
#pragma unroll
          for (int e = 0; e < VW; ++e)
            if (!a_in(tid + it * NT, k0, e)) put(ra[set][it], e, 0.0f);
#pragma unroll
        for (int it = 0; it < G::B_PER; ++it)
#pragma unroll
          for (int e = 0; e < VW; ++e)
            if (!b_in(tid + it * NT, k0, e)) put(rb[set][it], e, 0.0f);
      }
#pragma unroll
      for (int it = 0; it < G::A_PER; ++it) {
        const int q = tid + it * NT;
        if (G::A_VECS % NT == 0 || q < G::A_VECS) {
          int r, c;
          G::a_item(q, r, c);
          *reinterpret_cast<VT *>(&As[buf][r * LDA + c]) = ra[set][it];
        }
      }
#pragma unroll
      for (int it = 0; it < G::B_PER; ++it) {
        const int q = tid + it * NT;
        if (G::B_VECS % NT == 0 || q < G::B_VECS) {
          const int r = q / (BN / VW), c = (q - r * (BN / VW)) * VW;
          *reinterpret_cast<VT *>(&Bs[buf][r * LDB + c]) = rb[set][it];
        }
      }
    };

    // Schedule per slab t (slab t lives in buffer t & 1, C = BK / KC chunks):
    //   chunk kc:     read chunk kc+1's fragments, then chunk kc's MFMAs
    //   chunk C/2-1:  after its MFMAs, store slab t+1 (registers, loaded one
    //                 slab earlier) into the other buffer and issue the global
    //                 loads of slab t+2 -- the LDS writes overlap matrix work
    //   chunk C-1:    barrier first (every wave has its last fragments of
    //                 slab t in registers and its slab t+1 stores done), then
    //                 read slab t+1's first fragments while the last MFMAs of
    //                 slab t run.
    // Hazards: buffer (t+1)&1 held slab t-1, whose last reads precede the
    // barrier of slab t-1; slab t+1's stores precede the barrier of slab t,
    // which precedes every read of it.
    // MID < C - 1 whenever C >= 2, so slab t+1's stores always precede the
    // barrier at chunk C-1; with a single chunk they are issued before it.
    constexpr int C = BK / KC, MID = C >= 2 ? C / 2 - 1 : 0;
    // Staging spread over the MFMAs (steady-state slabs of kernels with one
    // wave per SIMD): after each of the first 2 * NSTG MFMAs of the
    // chunks before the barrier, one staging operation -- the LDS write of
    // vector i, then the global load that refills its registers -- so the
    // wave always has an MFMA to issue.  With one wave per SIMD nothing
    // else covers a burst of writes and loads (measured: 64x64 t4x4 k32 at
    // 1024^3 20.8 -> 19.3 us, 128x128 t8x8 k32 at 2048^3 138.8 -> 126.9 us);
    // with two or more waves per SIMD the burst is covered and the spread
    // form is no faster.
    constexpr int NSTG = G::A_PER + G::B_PER, NMC = 4 * FM * FN;
    // (Only with the two staging sets of a thread that stages at most 8
    // vectors: the one-wave 64x64 t8x8 k64 stages 32, and its second copy of
    // the loop would spill.)
    constexpr bool SPREAD = PROMOTE && VEC && NT <= 256 && DEPTH == 2 && C >= 2 && 2 * NSTG <= NMC * (C - 1);
    f32x4 af[2][FM];
    float bf[2][FN][4];
    // One staging vector (item q < A_PER: A, else B) of a slab that is not
    // guarded (the loads of load_slab's unmasked and unguarded paths).
    auto load_item = [&](auto sc, auto qc, int k0, auto bc) __attribute__((always_inline)) {
      constexpr int set = decltype(sc)::value, it = decltype(qc)::value;
      if constexpr (decltype(bc)::value) {
        if constexpr (it < G::A_PER) {
          if (G::A_VECS % NT == 0 || tid + it * NT < G::A_VECS)
            ra[set][it] = buffer_load_vt<VT>(buf_rsrc(A + k0), a_byte(it));
        } else {
          constexpr int ib = it - G::A_PER;
          if (G::B_VECS % NT == 0 || tid + ib * NT < G::B_VECS)
            rb[set][ib] = buffer_load_vt<VT>(buf_rsrc(b_base(k0)), b_byte(ib));
        }
      } else if constexpr (it < G::A_PER) {
        const int q = tid + it * NT;
        if (G::A_VECS % NT == 0 || q < G::A_VECS) {
          int r, c;
          G::a_item(q, r, c);
          if constexpr (!MASK) ra[set][it] = *reinterpret_cast<const VT *>(A + r * lda + k0 + c);
          else ra[set][it] = load16(p.A + (min(m0i + r, Mi - 1) * (int)lda + kbi + k0 + c));
        }
      } else {
        constexpr int ib = it - G::A_PER;
        const int q = tid + ib * NT;
        if (G::B_VECS % NT == 0 || q < G::B_VECS) {
          if constexpr (!MASK) rb[set][ib] = *reinterpret_cast<const VT *>(b_src[ib] + k0 * ldb);
          else rb[set][ib] = load16(p.B + (b_off[ib] + k0 * (int)ldb));
        }
      }
    };
    auto store_item = [&](auto sc, auto qc, int buf) __attribute__((always_inline)) {
      constexpr int set = decltype(sc)::value, it = decltype(qc)::value;
      if constexpr (it < G::A_PER) {
        const int q = tid + it * NT;
        if (G::A_VECS % NT == 0 || q < G::A_VECS) {
          int r, c;
          G::a_item(q, r, c);
          *reinterpret_cast<VT *>(&As[buf][r * LDA + c]) = ra[set][it];
        }
      } else {
        const int q = tid + (it - G::A_PER) * NT;
        if (G::B_VECS % NT == 0 || q < G::B_VECS) {
          const int r = q / (BN / VW), c = (q - r * (BN / VW)) * VW;
          *reinterpret_cast<VT *>(&Bs[buf][r * LDB + c]) = rb[set][it - G::A_PER];
        }
      }
    };
    auto load_frags = [&](int buf, int kc, int slot) __attribute__((always_inline)) {
      const float *as = As[buf] + (wm * WTM + lr) * LDA + 4 * lg + kc * KC;
      const float *bs = Bs[buf] + (4 * lg + kc * KC) * LDB + wn * WTN + lr;
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const float *src = as + i * MB * LDA;
        if constexpr (VEC) {
          af[slot][i] = *reinterpret_cast<const f32x4 *>(src);
        } else {
          af[slot][i].x = src[0];
          af[slot][i].y = src[1];
          af[slot][i].z = src[2];
          af[slot][i].w = src[3];
        }
      }
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int s = 0; s < 4; ++s) bf[slot][j][s] = bs[s * LDB + j * MB];
    };
    // Slab 0's loads go out first: the bias test reads the epilogue fields
    // from the kernel-argument segment, and its wait would delay them.
    if (nk > 0) load_slab(std::integral_constant<int, 0>{}, std::integral_constant<int, 1>{}, 0, BufOff{});
    if (bias_early && tid < BN / 4)
      *reinterpret_cast<f32x4 *>(&bias_s[4 * tid]) = *reinterpret_cast<const f32x4 *>(p.epi.ptr[0] + n0 + 4 * tid);
    if (nk > 0) {
      store_slab(std::integral_constant<int, 0>{}, std::integral_constant<int, 1>{}, 0, 0);
      if (nk > 1) load_slab(std::integral_constant<int, DEPTH - 1>{}, std::integral_constant<int, 1>{}, BK, BufOff{});
      if (DEPTH == 2 && nk > 2)
        load_slab(std::integral_constant<int, 0>{}, std::integral_constant<int, 1>{}, 2 * BK, BufOff{});
    }
    __syncthreads();
    if (nk > 0) load_frags(0, 0, 0);
    // One slab; P = kt & 1 names its LDS buffer; slab s is staged in set
    // s & 1 (two sets) or 0 (one set), and slab kt + 1 + DEPTH is loaded into
    // the set that slab kt + 1 leaves.
    // `gm` = 0: a masked kernel's steady state, where every slab this one
    // stores or loads is unguarded and a next slab exists (see the loop
    // below), so the loads are unconditional and the compiler's waits exact.
    auto slab = [&](auto par, auto gm, int kt, auto bc) __attribute__((always_inline)) {
      constexpr int P = decltype(par)::value;
      constexpr int cur = P;
      constexpr bool steady = decltype(gm)::value == 0;
      const bool more = steady || kt + 1 < nk;
#pragma unroll
      for (int kc = 0; kc < C; ++kc) {
        const int fs = kc & 1;
        if (C == 1 && more) {
          store_slab(std::integral_constant<int, DEPTH == 2 ? (P ^ 1) : 0>{}, gm, cur ^ 1, (kt + 1) * BK);
          if (steady || kt + 1 + DEPTH < nk)
            load_slab(std::integral_constant<int, DEPTH == 2 ? (P ^ 1) : 0>{}, gm, (kt + 1 + DEPTH) * BK, bc);
        }
        if (kc + 1 < C) {
          load_frags(cur, kc + 1, fs ^ 1);
        } else if (more) {
          __syncthreads();
          load_frags(cur ^ 1, 0, fs ^ 1);
        }
        constexpr bool spread = SPREAD && steady;
        if constexpr (spread) {
          constexpr int SET = DEPTH == 2 ? (P ^ 1) : 0;
          static_for<NMC>([&](auto xc) __attribute__((always_inline)) {
            constexpr int x = decltype(xc)::value;
            constexpr int s = x / (FM * FN), i = (x / FN) % FM, j = x % FN;
            acc[i][j] = mfma_block<MB>(bf[fs][j][s], af[fs][i][s], acc[i][j]);
            const int op = kc * NMC + x;  // constant once the chunk loop is unrolled
            if (kc < C - 1 && op < 2 * NSTG) {
              __builtin_amdgcn_sched_barrier(0);
              static_for<2 * NSTG>([&](auto oc) __attribute__((always_inline)) {
                constexpr int o = decltype(oc)::value;
                if (o == op) {
                  if constexpr (o % 2 == 0)
                    store_item(std::integral_constant<int, SET>{}, std::integral_constant<int, o / 2>{}, cur ^ 1);
                  else
                    load_item(std::integral_constant<int, SET>{}, std::integral_constant<int, o / 2>{},
                              (kt + 1 + DEPTH) * BK, bc);
                }
              });
              __builtin_amdgcn_sched_barrier(0);
            }
          });
        } else {
#pragma unroll
          for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
              for (int j = 0; j < FN; ++j)
                acc[i][j] = mfma_block<MB>(bf[fs][j][s], af[fs][i][s], acc[i][j]);
        }
        // Order of this chunk's MFMAs and the next chunk's fragment reads,
        // chosen by measurement on MI355X (main-loop shader cycles at 2048^3,
        // launch times at 1024^3 and 4096^3 over 10 configurations):
        //   one 32x32 block per wave:  2 MFMAs, all reads, 2 MFMAs;
        //   one 16x16 block per wave:  2 MFMAs, 2 reads, repeated;
        //   several blocks, <= 8 waves: all reads 2 MFMAs before the end;
        //   several blocks, 16 waves:  MFMA, read, repeated.
        constexpr int NM = 4 * FM * FN;  // MFMAs per chunk
        if constexpr (spread) {
          // (order fixed above)
        } else if constexpr (FM * FN == 1 && MB == 32) {
          __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // MFMA
          __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);  // DS read
          __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
        } else if constexpr (FM * FN == 1) {
#pragma unroll
          for (int s = 0; s < 2; ++s) {
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
          }
        } else if constexpr (NT <= 512) {
          __builtin_amdgcn_sched_group_barrier(0x008, NM - 2, 0);
          __builtin_amdgcn_sched_group_barrier(0x100, FM + 4 * FN, 0);
          __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
        } else {
#pragma unroll
          for (int s = 0; s < NM; ++s) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
          }
        }
        __builtin_amdgcn_sched_barrier(0);
        if (!spread && C >= 2 && kc == MID && more) {
          __builtin_amdgcn_sched_barrier(0);
          store_slab(std::integral_constant<int, DEPTH == 2 ? (P ^ 1) : 0>{}, gm, cur ^ 1, (kt + 1) * BK);
          if (steady || kt + 1 + DEPTH < nk)
            load_slab(std::integral_constant<int, DEPTH == 2 ? (P ^ 1) : 0>{}, gm, (kt + 1 + DEPTH) * BK, bc);
        }
      }
      // With an odd chunk count the next slab's first fragments landed in
      // slot 1; the loop expects them in slot 0.
      if constexpr (C % 2 == 1) {
#pragma unroll
        for (int i = 0; i < FM; ++i) af[0][i] = af[1][i];
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int s = 0; s < 4; ++s) bf[0][j][s] = bf[1][j][s];
      }
    };
    using Steady = std::integral_constant<int, 0>;
    using Any = std::integral_constant<int, 1>;
    auto k_loop = [&](auto bc) __attribute__((always_inline)) {
      int kt = 0;
      // (Not for the configurations whose accumulators fill the register file,
      // 32768 per workgroup: the second copy of the loop would spill.)
      if constexpr ((MASK || SPREAD) && NT * TM * TN < 32768) {
        // Masked kernels: only the slab holding row K-1 (the last) is guarded
        // (every slab when N < 4).  While slab kt's loads (slab kt + 1 + DEPTH)
        // stay before it, run a loop without the guarded branch: a branch
        // between element-wise and vector loads leaves the compiler unsure how
        // many loads are in flight, and it then waits for all of them
        // (vmcnt(0)) three times per slab pair.  Spread kernels: the same
        // straight-line loop carries the spread staging (its loads are
        // unconditional there, so each LDS write waits for exactly its load).
        const int steady = (MASK && Ni < 4) ? 0 : max(0, nk - 2 - DEPTH) & ~1;
        for (; kt < steady; kt += 2) {
          slab(std::integral_constant<int, 0>{}, Steady{}, kt, bc);
          slab(std::integral_constant<int, 1>{}, Steady{}, kt + 1, bc);
        }
      }
      for (; kt + 1 < nk; kt += 2) {
        slab(std::integral_constant<int, 0>{}, Any{}, kt, bc);
        slab(std::integral_constant<int, 1>{}, Any{}, kt + 1, bc);
      }
      if (kt < nk) slab(std::integral_constant<int, 0>{}, Any{}, kt, bc);
    };
    // Buffer loads where measured faster: the spread kernels, and the
    // block-staged ones with tiles of at least 128 x 128 (2048^3 t8x4 k32
    // 124.9 -> 123.6 us; the 8-wave 64x64 t4x2 k64 at 1024^3 was 2.4% slower
    // with them).  Not for 1024-thread workgroups (128 VGPRs per lane): the
    // flat-load copy of the loop beside the buffer one spills there; masked
    // kernels only where they spread their staging (the block-staged masked
    // ones with 512 threads and tile-k 32 or 64 spill with both loops).
    constexpr bool BUFCAP = VEC && NT < 1024 && (SPREAD || (!MASK && BM * BN >= 128 * 128));
    if constexpr (BUFCAP) {
      if ((long)BM * lda + BK < (1L << 29) && (long)BK * ldb + (MASK ? Ni : BN) < (1L << 29)) k_loop(BufOn{});
      else k_loop(BufOff{});
    } else {
      k_loop(BufOff{});
    }
  } else {
    // promote=0: fragments straight from global memory, no LDS, no barriers.
    const float *ag = A + (long)(wm * WTM + lr) * lda + 4 * lg;
    const float *bg = B + 4 * lg * ldb + wn * WTN + lr;
    for (int kt = 0; kt < nk; ++kt) {
      const int k0 = kt * BK;
#pragma unroll
      for (int kc = 0; kc < BK / KC; ++kc) {
        f32x4 af[FM];
        float bf[FN][4];
#pragma unroll
        for (int i = 0; i < FM; ++i) {
          const float *src = ag + (long)i * MB * lda + k0 + kc * KC;
          if constexpr (VEC) {
            af[i] = *reinterpret_cast<const f32x4 *>(src);
          } else {
            af[i].x = src[0];
            af[i].y = src[1];
            af[i].z = src[2];
            af[i].w = src[3];
          }
        }
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int s = 0; s < 4; ++s) bf[j][s] = bg[(long)(k0 + kc * KC + s) * ldb + j * MB];
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
          for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
              acc[i][j] = mfma_block<MB>(bf[j][s], af[i][s], acc[i][j]);
      }
    }
  }

  // Epilogue: lane (lr, lg) holds, per block and group g < NG, C[m, n..n+3]
  // with m = row lr of the block and n = 8*g + 4*lg (MB = 32, 4 groups) or
  // n = 4*lg (MB = 16, one group).
  constexpr int NG = MB == 32 ? 4 : 1;
  auto group = [&](int i, int j, int g) __attribute__((always_inline)) {
    f32x4 v;
    v.x = acc[i][j][4 * g + 0];
    v.y = acc[i][j][4 * g + 1];
    v.z = acc[i][j][4 * g + 2];
    v.w = acc[i][j][4 * g + 3];
    return v;
  };
  auto row_of = [&](int i) __attribute__((always_inline)) { return m0 + wm * WTM + i * MB + lr; };
  auto col_of = [&](int j, int g) __attribute__((always_inline)) { return (int)n0 + wn * WTN + j * MB + 8 * g + 4 * lg; };

  if (splits > 1) {
    // Split-K: this workgroup's partial sums go to slice `split` of the
    // workspace; splitk_reduce_kernel, launched next on the same stream, adds
    // the slices in order and runs the epilogue.
    // The workspace holds whole tiles (ws_ld is N rounded up to BN), so
    // these stores need no masks.
    float *own = p.ws + split * p.ws_slice;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int g = 0; g < NG; ++g)
          *reinterpret_cast<f32x4 *>(own + row_of(i) * p.ws_ld + col_of(j, g)) = group(i, j, g);
    return;
  }

  if (MASK && (edge || (p.ldc & 3) != 0)) {
    // Edge tile, or rows of C not 16-byte aligned: outputs outside C are
    // dropped.  A group of 4 wholly inside C is written with one 128-bit
    // store at 4-byte alignment (16-byte aligned when N % 4 == 0, where every
    // group is wholly inside or outside); only a group that crosses column N
    // is written element by element.
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const long m = row_of(i);
      if (m >= p.M) continue;
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int g = 0; g < NG; ++g) {
          const int n = col_of(j, g);
          if (n >= p.N) continue;
          if (n + 4 <= p.N) {
            *reinterpret_cast<f32x4_u *>(p.C + m * p.ldc + n) = apply_epi4_rows(group(i, j, g), p.epi, m, n);
          } else {
            const f32x4 v = apply_epi4_edge(group(i, j, g), p.epi, m, n, p.N);
            for (int e = 0; e < 4 && n + e < p.N; ++e) p.C[m * p.ldc + n + e] = v[e];
          }
        }
    }
    return;
  }

#pragma unroll
  for (int i = 0; i < FM; ++i) {
    const long m = row_of(i);
    float *crow = p.C + m * p.ldc;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        const int n = col_of(j, g);
        f32x4 v = bias_early
                      ? apply_epi4(group(i, j, g) + *reinterpret_cast<const f32x4 *>(&bias_s[n - (int)n0]), p.epi, m, n, 1)
                      : apply_epi4(group(i, j, g), p.epi, m, n);
        if constexpr (VEC) {
          *reinterpret_cast<f32x4 *>(crow + n) = v;
        } else {
          crow[n + 0] = v.x;
          crow[n + 1] = v.y;
          crow[n + 2] = v.z;
          crow[n + 3] = v.w;
        }
      }
    }
  }
}

template <int BM, int BN, int TM, int TN, int BK, int PROMOTE, int VEC, int MASK>
hipError_t launch_staged(const GemmParams &p, dim3 grid, dim3 block, hipStream_t stream) {
  if (block.x != BN / TN || block.y != BM / TM || block.z != 1) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL((staged_gemm_kernel<BM, BN, TM, TN, BK, PROMOTE, VEC, MASK>), grid, block, 0, stream, p.A, p.B,
                     p.lda, p.ldb, p.K, (int)grid.x, (int)grid.y, p.swizzle | (p.splits << 8), p.M, p.N, p);
  return hipGetLastError();
}

}  // namespace tfk
