// Device-side epilogue: the fused tforge element ops applied to accumulators.
#pragma once

#include "tf_kernels.h"

namespace tfk {

typedef float f32x4 __attribute__((ext_vector_type(4)));
// The same vector at 4-byte alignment: one dword-aligned 128-bit access.
typedef float f32x4_u __attribute__((ext_vector_type(4), aligned(4)));

// IEEE-754-2019 maximum(x, +0.0), the semantics of tforge.relu
// (docs/dialect.md:26-30): NaN propagates and -0.0 maps to +0.0.  v_max_f32
// would return +0.0 for a NaN input, so the select is written out.
__device__ __forceinline__ float relu_ieee(float x) { return (x > 0.0f || x != x) ? x : 0.0f; }

// Applies the epilogue ops first.. to four consecutive outputs C[m, n..n+3]
// (first = 1 when the caller has already added a prefetched bias).  STREAM:
// the add operand is read once by this launch, so its load is non-temporal
// (the element-op kernels); the bias, reused by every row, stays cached.
template <bool STREAM = false>
__device__ __forceinline__ f32x4 apply_epi4(f32x4 v, const EpiParams &e, long m, int n, int first = 0) {
#pragma unroll
  for (int i = 0; i < kMaxEpi; ++i) {
    if (i < first) continue;
    if (i >= e.nops) break;
    const int kind = e.kind[i];
    if (kind == EPI_BIAS) {
      v += *reinterpret_cast<const f32x4 *>(e.ptr[i] + n);
    } else if (kind == EPI_RELU) {
      v.x = relu_ieee(v.x);
      v.y = relu_ieee(v.y);
      v.z = relu_ieee(v.z);
      v.w = relu_ieee(v.w);
    } else if (kind == EPI_ADD) {
      const f32x4 *r = reinterpret_cast<const f32x4 *>(e.ptr[i] + m * e.ldr[i] + n);
      v += STREAM ? __builtin_nontemporal_load(r) : *r;
    } else if (kind == EPI_ADD_SELF) {
      v = v + v;
    }
  }
  return v;
}

// apply_epi4 for four outputs inside a matrix whose rows are not 16-byte
// aligned (buffers are, and n is a multiple of 4, so only a row-indexed
// operand is misaligned): the add operand is read with one dword-aligned
// 128-bit load.  Same operations in the same order as apply_epi4.
__device__ __forceinline__ f32x4 apply_epi4_rows(f32x4 v, const EpiParams &e, long m, int n) {
#pragma unroll
  for (int i = 0; i < kMaxEpi; ++i) {
    if (i >= e.nops) break;
    const int kind = e.kind[i];
    if (kind == EPI_BIAS) {
      v += *reinterpret_cast<const f32x4 *>(e.ptr[i] + n);
    } else if (kind == EPI_RELU) {
      v.x = relu_ieee(v.x);
      v.y = relu_ieee(v.y);
      v.z = relu_ieee(v.z);
      v.w = relu_ieee(v.w);
    } else if (kind == EPI_ADD) {
      v += *reinterpret_cast<const f32x4_u *>(e.ptr[i] + m * e.ldr[i] + n);
    } else if (kind == EPI_ADD_SELF) {
      v = v + v;
    }
  }
  return v;
}

// The same for C[m, n..n+3] at the right edge of a matrix whose rows are not
// 16-byte aligned: operands are read element by element, columns >= N are
// not read (their results are discarded).
__device__ __forceinline__ f32x4 apply_epi4_edge(f32x4 v, const EpiParams &e, long m, int n, int N) {
  auto ld4 = [&](const float *row) {
    f32x4 t = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int c = 0; c < 4; ++c)
      if (n + c < N) t[c] = row[n + c];
    return t;
  };
#pragma unroll
  for (int i = 0; i < kMaxEpi; ++i) {
    if (i >= e.nops) break;
    const int kind = e.kind[i];
    if (kind == EPI_BIAS) {
      v += ld4(e.ptr[i]);
    } else if (kind == EPI_RELU) {
      v.x = relu_ieee(v.x);
      v.y = relu_ieee(v.y);
      v.z = relu_ieee(v.z);
      v.w = relu_ieee(v.w);
    } else if (kind == EPI_ADD) {
      v += ld4(e.ptr[i] + m * e.ldr[i]);
    } else if (kind == EPI_ADD_SELF) {
      v = v + v;
    }
  }
  return v;
}

// Scalar form for the direct / elementwise kernels.
__device__ __forceinline__ float apply_epi1(float v, const EpiParams &e, long m, int n) {
#pragma unroll
  for (int i = 0; i < kMaxEpi; ++i) {
    if (i >= e.nops) break;
    const int kind = e.kind[i];
    if (kind == EPI_BIAS) v = v + e.ptr[i][n];
    else if (kind == EPI_RELU) v = relu_ieee(v);
    else if (kind == EPI_ADD) v = v + e.ptr[i][m * e.ldr[i] + n];
    else if (kind == EPI_ADD_SELF) v = v + v;
  }
  return v;
}

}  // namespace tfk
