// Block-mean pooling of the queries, fused with the selection's query scaling.
//
// Follows spattn/src/utils.py:340-351 (average_vector: fp32 mean over qps rows,
// the last block divided by its real row count, result cast back to the input
// dtype) and spattn/src/kernels/vecattention_kernels.py:94,244-245 (the
// selection multiplies the pooled rows by fp32(1/sqrt(D)) and rounds back to
// the input dtype before the score product).
//
// Canonical arithmetic: rows are summed sequentially in fp64, the sum is
// rounded to fp32, divided in fp32 by the real row count, and rounded to the
// element type.  The divide runs in fp64 and is rounded once to fp32, which is
// the correctly rounded fp32 quotient of two fp32 operands.
//
// HBM-bound: each Q element is read once.  A thread owns VEC consecutive
// features of one pooled row, so 16-byte loads of a full Q row are coalesced
// across D/VEC neighbouring threads, and keeps 8 rows' loads in flight.
#include "common.h"

namespace va {

template <typename T, int VEC>
__global__ __launch_bounds__(256) void pool_scale_kernel(
    const T* __restrict__ q, int64_t H, int64_t S, int64_t D, int64_t sqb,
    int64_t sqh, int64_t sqs, int64_t qps, int64_t nqb, float sm,
    T* __restrict__ pooled, T* __restrict__ scaled) {
  const int64_t lanes_per_row = D / VEC;
  const int64_t rows_per_block = blockDim.x / lanes_per_row;
  const int64_t local = threadIdx.x / lanes_per_row;
  const int64_t dv = (threadIdx.x % lanes_per_row) * VEC;
  const int64_t J = int64_t(blockIdx.x) * rows_per_block + local;
  const int64_t bh = blockIdx.y;
  if (local >= rows_per_block || J >= nqb) return;
  const int64_t b = bh / H, h = bh % H;
  const int64_t r0 = J * qps;
  const int64_t rows = (S - r0 < qps) ? (S - r0) : qps;
  const T* src = q + b * sqb + h * sqh + r0 * sqs + dv;

  double acc[VEC];
#pragma unroll
  for (int e = 0; e < VEC; ++e) acc[e] = 0.0;

  auto load = [&](T (&v)[VEC], int64_t r) {
    if constexpr (VEC * sizeof(T) == 16) {
      *reinterpret_cast<uint4*>(v) = *reinterpret_cast<const uint4*>(src + r * sqs);
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) v[e] = src[r * sqs + e];
    }
  };
  // Rows are loaded U at a time (U loads in flight per thread) and added in
  // row order, so the sums are those of the sequential loop.
  constexpr int U = 8;
  int64_t r = 0;
  for (; r + U <= rows; r += U) {
    T v[U][VEC];
#pragma unroll
    for (int u = 0; u < U; ++u) load(v[u], r + u);
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int e = 0; e < VEC; ++e) acc[e] += double(to_f32(v[u][e]));
  }
  for (; r < rows; ++r) {
    T v[VEC];
    load(v, r);
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[e] += double(to_f32(v[e]));
  }

  const int64_t o = (bh * nqb + J) * D + dv;
#pragma unroll
  for (int e = 0; e < VEC; ++e) {
    const float sum32 = float(acc[e]);
    const float mean32 = float(double(sum32) / double(rows));
    const float p = Round<T>::rt(mean32);
    if (pooled) pooled[o + e] = Round<T>::store(p);
    if (scaled) scaled[o + e] = Round<T>::store(p * sm);
  }
}

template <typename T>
static hipError_t launch_pool_t(const void* q, int64_t B, int64_t H, int64_t S,
                                int64_t D, int64_t sqb, int64_t sqh, int64_t sqs,
                                int64_t qps, void* pooled, void* scaled,
                                hipStream_t stream) {
  const int64_t nqb = (S + qps - 1) / qps;
  const float sm = float(1.0 / __builtin_sqrt(double(D)));
  constexpr int V16 = int(16 / sizeof(T));
  const uintptr_t addr = reinterpret_cast<uintptr_t>(q);
  const bool vec_ok = (D % V16 == 0) && (addr % 16 == 0) && (sqb % V16 == 0) &&
                      (sqh % V16 == 0) && (sqs % V16 == 0);
  if (vec_ok) {  // D / V16 <= 64 lanes per row (D <= 256)
    // 128 threads per work-group measured 3-6% faster than 256 at B, C, D.
    const int threads = 128;
    const int64_t lanes = D / V16;
    const int64_t rows_per_block = threads / lanes;
    dim3 grid(unsigned((nqb + rows_per_block - 1) / rows_per_block), unsigned(B * H));
    hipLaunchKernelGGL((pool_scale_kernel<T, V16>), grid, dim3(threads), 0, stream,
                       static_cast<const T*>(q), H, S, D, sqb, sqh, sqs, qps, nqb, sm,
                       static_cast<T*>(pooled), static_cast<T*>(scaled));
  } else {
    const int threads = 256;  // one thread per feature, D <= 256
    const int64_t rows_per_block = threads / D;
    dim3 grid(unsigned((nqb + rows_per_block - 1) / rows_per_block), unsigned(B * H));
    hipLaunchKernelGGL((pool_scale_kernel<T, 1>), grid, dim3(threads), 0, stream,
                       static_cast<const T*>(q), H, S, D, sqb, sqh, sqs, qps, nqb, sm,
                       static_cast<T*>(pooled), static_cast<T*>(scaled));
  }
  return hipGetLastError();
}

hipError_t launch_pool(int dtype, const void* q, int64_t B, int64_t H, int64_t S,
                       int64_t D, int64_t sqb, int64_t sqh, int64_t sqs, int64_t qps,
                       void* pooled, void* scaled, hipStream_t stream) {
  switch (dtype) {
    case kF32: return launch_pool_t<float>(q, B, H, S, D, sqb, sqh, sqs, qps, pooled, scaled, stream);
    case kBF16: return launch_pool_t<bf16_t>(q, B, H, S, D, sqb, sqh, sqs, qps, pooled, scaled, stream);
    case kF16: return launch_pool_t<f16_t>(q, B, H, S, D, sqb, sqh, sqs, qps, pooled, scaled, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace va
