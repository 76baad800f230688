// Kernel-side interface of libtforge_hip: parameter blocks passed by value to
// the gfx950 kernels, the epilogue op encoding, and the registry of
// ahead-of-time template instantiations.  Shared by the host runtime
// (runtime.hip) and the kernel translation units.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace tfk {

// Epilogue ops applied in order to each output element after the K reduction.
// They restate the tforge element ops the reference fuses into the matmul's
// writeback (lib/Transforms/TileAndFuse.cpp:78-131, "EpilogueIntoProducerInit"):
//   BIAS      y = y + bias[n]          tforge.bias_add (TForgeToLinalg.cpp:113-133)
//   RELU      y = maximum(y, +0.0)     tforge.relu, IEEE-754-2019 maximum
//   ADD       y = y + R[m, n]          tforge.add with another buffer
//   ADD_SELF  y = y + y                tforge.add %v, %v
enum EpiKind : int { EPI_NONE = 0, EPI_BIAS = 1, EPI_RELU = 2, EPI_ADD = 3, EPI_ADD_SELF = 4 };
constexpr int kMaxEpi = 4;

struct EpiParams {
  int nops;
  int kind[kMaxEpi];
  const float *ptr[kMaxEpi];  // bias: length-N vector; add: M x N matrix with row stride ldr[i]
  long ldr[kMaxEpi];
};

// C[M x N] = epi(A[M x K] @ B[K x N]); row-major, leading dimensions in elements.
struct GemmParams {
  const float *A;
  const float *B;
  float *C;
  int M, N, K;
  long lda, ldb, ldc;
  EpiParams epi;
  int swizzle;  // 1: XCD-aware workgroup -> tile order (staged family only)
  // Split-K (staged family): gridDim.z = splits workgroups per output tile,
  // each reducing a contiguous range of K slabs into slice z of ws
  // (splits x M x ldc floats) instead of writing C; launch_splitk_reduce
  // then forms C = epi(sum of the slices in order 0..splits-1).
  int splits;
  float *ws;
  long ws_ld, ws_slice;  // partial-sum row stride and slice size (floats); whole tiles
};

// C[M x N] = epi(ws[0] + ws[1] + ... + ws[splits-1]); slice s starts at
// ws + s * ws_slice, rows ws_ld apart (ws_ld a multiple of 4, >= N).
struct ReduceParams {
  const float *ws;
  float *C;
  int M, N, splits;
  long ws_ld, ws_slice, ldc;
  EpiParams epi;
};

// Y[M x N] = epi(X[M x N]) for element-op-only programs.
struct EltParams {
  const float *X;
  float *Y;
  int M, N;
  long ldx, ldy;
  EpiParams epi;
  int vec_ok;  // 1: every operand 16-byte aligned with row strides a multiple of 4
};

enum Family : int { FAM_DIRECT = 0, FAM_STAGED = 1, FAM_ELEMENTWISE = 2, FAM_WAVEK = 4 };

using GemmLauncher = hipError_t (*)(const GemmParams &, dim3 grid, dim3 block, hipStream_t);
using EltLauncher = hipError_t (*)(const EltParams &, dim3 grid, dim3 block, hipStream_t);

// One ahead-of-time instantiation of a kernel template.
struct KernelEntry {
  int family;
  int bm, bn, tm, tn, bk;  // staged, wave-split: full config; direct/elementwise: tm, tn only
  int promote, vectorize;
  int masked;  // staged: 1 = any M, N, K (edges masked in-kernel); 0 = tile multiples only
  const char *name;
  const void *fn;  // the __global__ function, for hipFuncGetAttributes / occupancy
  GemmLauncher gemm;
  EltLauncher elt;
  int lds_bytes;   // static LDS of the instantiation
};

// The split-K reduction (direct_kernels.hip); ws and C 16-byte aligned.
hipError_t launch_splitk_reduce(const ReduceParams &p, hipStream_t stream);

// Registry (defined in the generated registry translation unit).
const KernelEntry *registry_begin();
const KernelEntry *registry_end();

}  // namespace tfk
