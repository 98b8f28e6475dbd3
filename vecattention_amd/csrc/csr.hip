// Row offsets of the compact (CSR) selection output.
//
// A counting run of the selection writes counts[(r * nseg) + s], the keys row
// r selects in key segment s (nseg = 1 when the keys are not split).  The
// offsets are the int64 exclusive prefix sums of the row totals:
// offsets[0] = 0, offsets[r + 1] = offsets[r] + sum_s counts[r * nseg + s]
// (int64: at 128K keys with every key selected a head's rows alone hold 2^33
// keys).  Two launches on the caller's stream, no host round trip: the row
// totals, then one work-group scanning them in place, 1024 rows per step.
#include "common.h"

namespace va {

__global__ __launch_bounds__(256) void csr_row_totals_kernel(const int32_t* __restrict__ counts,
                                                             int64_t rows, int nseg,
                                                             int64_t* __restrict__ offsets) {
  const int64_t r = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (r == 0) offsets[0] = 0;
  if (r >= rows) return;
  int64_t t = 0;
  for (int s = 0; s < nseg; ++s) t += counts[r * nseg + s];
  offsets[r + 1] = t;
}

// In-place inclusive scan of offsets[1 .. rows]: per step each of the 1024
// threads takes one row, the waves scan their 64 rows with lane shuffles, and
// the 16 wave sums are added in from LDS; `carry` holds the earlier steps'
// total.
__global__ __launch_bounds__(1024) void csr_scan_kernel(int64_t* __restrict__ offsets,
                                                        int64_t rows) {
  __shared__ int64_t wsum[16];
  const int t = threadIdx.x, lane = t % 64, w = t / 64;
  int64_t carry = 0;
  for (int64_t base = 1; base <= rows; base += 1024) {
    const int64_t i = base + t;
    int64_t v = i <= rows ? offsets[i] : 0;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int64_t u = __shfl_up(v, d);
      if (lane >= d) v += u;
    }
    if (lane == 63) wsum[w] = v;
    __syncthreads();
    int64_t before = 0, total = 0;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      before += j < w ? wsum[j] : 0;
      total += wsum[j];
    }
    if (i <= rows) offsets[i] = carry + before + v;
    carry += total;
    __syncthreads();  // wsum is rewritten by the next step
  }
}

hipError_t launch_csr_offsets(const int32_t* counts, int64_t rows, int nseg, int64_t* offsets,
                              hipStream_t stream) {
  if (rows <= 0 || nseg <= 0) return hipErrorInvalidValue;
  const int64_t blocks = (rows + 255) / 256;
  hipLaunchKernelGGL(csr_row_totals_kernel, dim3(unsigned(blocks)), dim3(256), 0, stream, counts,
                     rows, nseg, offsets);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(csr_scan_kernel, dim3(1), dim3(1024), 0, stream, offsets, rows);
  return hipGetLastError();
}

}  // namespace va
