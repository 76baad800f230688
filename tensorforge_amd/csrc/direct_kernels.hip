// Direct (no K staging) GEMM family and the element-op kernels.
//
// Direct GEMM: what the reference pipeline emits for "tile-k=0" options, its
// default (docs/stage7.md:9-20; lib/Transforms/Gpu.cpp:188-197): the launch is
// grid (ceil(N/BN), ceil(M/BM)) x block (BN/TN, BM/TM), each thread owns a
// TM x TN sub-tile of its block tile and runs the K loop from +0.0 with one
// fused multiply-add per k, in sequential k order, then the fused epilogue.
// That arithmetic is bit-identical to the reference's naive kernel
// (docs/numerics.md:53), any shape is accepted and edges are masked.
//
// Element-op kernels: programs with no matmul (tforge.bias_add / relu / add
// alone, or chains of them) run one thread per TM x TN elements with the same
// launch geometry, one IEEE operation per op, so results are bit-exact against
// NumPy float32 (python/tforge_gpu.py:116-126).
//
// Split-K reduction: the second launch of a staged matmul compiled with
// split-k=S (a backend option): C = epi(slice 0 + ... + slice S-1).
#include "epilogue.hpp"

namespace tfk {

template <int TM, int TN>
__global__ void direct_gemm_kernel(GemmParams p) {
  const long m_base = ((long)blockIdx.y * blockDim.y + threadIdx.y) * TM;
  const long n_base = ((long)blockIdx.x * blockDim.x + threadIdx.x) * TN;
  if (m_base >= p.M || n_base >= p.N) return;
  float acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = 0.0f;
  const bool full = m_base + TM <= p.M && n_base + TN <= p.N;
  for (int k = 0; k < p.K; ++k) {
    float a[TM], b[TN];
#pragma unroll
    for (int i = 0; i < TM; ++i) a[i] = (full || m_base + i < p.M) ? p.A[(m_base + i) * p.lda + k] : 0.0f;
#pragma unroll
    for (int j = 0; j < TN; ++j) b[j] = (full || n_base + j < p.N) ? p.B[(long)k * p.ldb + n_base + j] : 0.0f;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = __builtin_fmaf(a[i], b[j], acc[i][j]);
  }
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const long m = m_base + i, n = n_base + j;
      if (m < p.M && n < p.N) p.C[m * p.ldc + n] = apply_epi1(acc[i][j], p.epi, m, (int)n);
    }
}

template <int TM, int TN>
__global__ void elementwise_kernel(EltParams p) {
  const long m_base = ((long)blockIdx.y * blockDim.y + threadIdx.y) * TM;
  const long n_base = ((long)blockIdx.x * blockDim.x + threadIdx.x) * TN;
  if constexpr (TN % 4 == 0) {
    // Thread tiles 4k wide on aligned rows: 128-bit loads and stores, so a
    // wave moves 64 x TN x 4 contiguous bytes per row.  Same IEEE ops.  Every
    // byte is read or written once, so the accesses are non-temporal (MI355X:
    // 6.80 against 6.38 TB/s for relu at 16384^2 with cached accesses).
    if (p.vec_ok && n_base + TN <= p.N) {
      // All loads first (rows past M read row M-1 and are not stored), so
      // they are in flight together; then the ops and the stores.  A chain
      // that starts with bias_add loads its bias here too (cached: every row
      // reads it), rather than behind the epilogue's per-op branch, where
      // each thread would wait for X before asking for the bias.
      const bool pre_bias = p.epi.nops > 0 && p.epi.kind[0] == EPI_BIAS;
      f32x4 bv[TN / 4];
#pragma unroll
      for (int j = 0; j < TN / 4; ++j)
        bv[j] = pre_bias ? *reinterpret_cast<const f32x4 *>(p.epi.ptr[0] + n_base + 4 * j) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      f32x4 x[TM][TN / 4];
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const long m = min(m_base + i, (long)p.M - 1);
#pragma unroll
        for (int j = 0; j < TN / 4; ++j)
          x[i][j] = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(p.X + m * p.ldx + n_base + 4 * j));
      }
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const long m = m_base + i;
        if (m >= p.M) break;
#pragma unroll
        for (int j = 0; j < TN / 4; ++j) {
          const int n = (int)n_base + 4 * j;
          const f32x4 v = pre_bias ? apply_epi4<true>(x[i][j] + bv[j], p.epi, m, n, 1)
                                   : apply_epi4<true>(x[i][j], p.epi, m, n);
          __builtin_nontemporal_store(v, reinterpret_cast<f32x4 *>(p.Y + m * p.ldy + n));
        }
      }
      return;
    }
  }
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const long m = m_base + i, n = n_base + j;
      if (m < p.M && n < p.N) p.Y[m * p.ldy + n] = apply_epi1(p.X[m * p.ldx + n], p.epi, m, (int)n);
    }
}

template <int TM, int TN>
hipError_t launch_direct(const GemmParams &p, dim3 grid, dim3 block, hipStream_t stream) {
  hipLaunchKernelGGL((direct_gemm_kernel<TM, TN>), grid, block, 0, stream, p);
  return hipGetLastError();
}

template <int TM, int TN>
hipError_t launch_elementwise(const EltParams &p, dim3 grid, dim3 block, hipStream_t stream) {
  hipLaunchKernelGGL((elementwise_kernel<TM, TN>), grid, block, 0, stream, p);
  return hipGetLastError();
}

// Split-K reduction: one thread per 4 consecutive outputs; the partial-sum
// slices are read 4 at a time (independent loads in flight) and added in
// slice order, so the result does not depend on scheduling.
__global__ void __launch_bounds__(256) splitk_reduce_kernel(ReduceParams p) {
  const long q = (long)blockIdx.x * 256 + threadIdx.x;
  const long per_row = (p.N + 3) / 4;
  if (q >= (long)p.M * per_row) return;
  const long m = q / per_row;
  const int n = (int)(q - m * per_row) * 4;
  const float *src = p.ws + m * p.ws_ld + n;
  auto ld = [&](int s) { return *reinterpret_cast<const f32x4 *>(src + s * p.ws_slice); };
  f32x4 v = ld(0);
  int s = 1;
  for (; s + 4 <= p.splits; s += 4) {
    const f32x4 t0 = ld(s), t1 = ld(s + 1), t2 = ld(s + 2), t3 = ld(s + 3);
    v += t0;
    v += t1;
    v += t2;
    v += t3;
  }
  for (; s < p.splits; ++s) v += ld(s);
  if ((p.ldc & 3) == 0 && n + 4 <= p.N) {
    *reinterpret_cast<f32x4 *>(p.C + m * p.ldc + n) = apply_epi4(v, p.epi, m, n);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (n + e < p.N) p.C[m * p.ldc + n + e] = apply_epi1(v[e], p.epi, m, n + e);
  }
}

hipError_t launch_splitk_reduce(const ReduceParams &p, hipStream_t stream) {
  const long quads = (long)p.M * ((p.N + 3) / 4);
  hipLaunchKernelGGL(splitk_reduce_kernel, dim3((unsigned)((quads + 255) / 256)), dim3(256), 0, stream, p);
  return hipGetLastError();
}

// The registry tables are host data (they hold host launch stubs).
#ifndef __HIP_DEVICE_COMPILE__
#define TF_DIRECT(TM, TN)                                                                       \
  KernelEntry{FAM_DIRECT, 0, 0, TM, TN, 0, 0, 0, 0, "tf_direct_t" #TM "x" #TN,                \
              reinterpret_cast<const void *>(&direct_gemm_kernel<TM, TN>), &launch_direct<TM, TN>, \
              nullptr, 0}
#define TF_ELT(TM, TN)                                                                          \
  KernelEntry{FAM_ELEMENTWISE, 0, 0, TM, TN, 0, 0, 0, 0, "tf_elementwise_t" #TM "x" #TN,      \
              reinterpret_cast<const void *>(&elementwise_kernel<TM, TN>), nullptr,             \
              &launch_elementwise<TM, TN>, 0}
#define TF_BOTH(TM, TN) TF_DIRECT(TM, TN), TF_ELT(TM, TN)

// Thread tiles 1, 2, 4, 8 in each dimension.
extern const KernelEntry kDirectEntries[] = {
    TF_BOTH(1, 1), TF_BOTH(1, 2), TF_BOTH(1, 4), TF_BOTH(1, 8), TF_BOTH(2, 1), TF_BOTH(2, 2),
    TF_BOTH(2, 4), TF_BOTH(2, 8), TF_BOTH(4, 1), TF_BOTH(4, 2), TF_BOTH(4, 4), TF_BOTH(4, 8),
    TF_BOTH(8, 1), TF_BOTH(8, 2), TF_BOTH(8, 4), TF_BOTH(8, 8),
};
extern const int kDirectCount = sizeof(kDirectEntries) / sizeof(kDirectEntries[0]);
#else
// Device pass: instantiate the kernels the host table names.
#define TF_INST(TM, TN)                                                  \
  template __global__ void direct_gemm_kernel<TM, TN>(GemmParams);       \
  template __global__ void elementwise_kernel<TM, TN>(EltParams);
TF_INST(1, 1) TF_INST(1, 2) TF_INST(1, 4) TF_INST(1, 8)
TF_INST(2, 1) TF_INST(2, 2) TF_INST(2, 4) TF_INST(2, 8)
TF_INST(4, 1) TF_INST(4, 2) TF_INST(4, 4) TF_INST(4, 8)
TF_INST(8, 1) TF_INST(8, 2) TF_INST(8, 4) TF_INST(8, 8)
#endif  // __HIP_DEVICE_COMPILE__

}  // namespace tfk
