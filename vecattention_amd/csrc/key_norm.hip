// Per-(batch, kv head) maximum key norm, rounded up: the K-side factor of the
// error bound the MFMA selection kernel certifies its decisions with
// (|s_mfma - s| <= gamma * ||q|| * max_c ||k_c||).
//
// Two launches, no atomics and no memset: partial maxima over kNormParts key
// ranges per head, then one reduction per head.  HBM-bound (reads K once);
// the squared norms are summed in fp64 (exact products of the 16-bit inputs)
// and the final square root is rounded up.
#include "common.h"

namespace va {

constexpr int kNormParts = 256;

// Rows of 16-byte vectors: lane l of a wave reads vector l % VPR of row
// l / VPR of each group of 64 / VPR rows (coalesced 1 KB per load
// instruction); the squared norm of a row is summed over its VPR lanes.
template <typename T, int VPR>
__global__ __launch_bounds__(256) void key_norm_partial_vec_kernel(
    const T* __restrict__ k, int64_t skb, int64_t skh, int64_t sks, int64_t Hk, int64_t Sk,
    float* __restrict__ partial) {
  constexpr int RPW = 64 / VPR;  // rows per wave load
  const int64_t bh = blockIdx.y;
  const int64_t b = bh / Hk, h = bh % Hk;
  const T* kh = k + b * skb + h * skh;
  const int64_t per = (Sk + kNormParts - 1) / kNormParts;
  const int64_t k0 = int64_t(blockIdx.x) * per;
  const int64_t k1 = (k0 + per < Sk) ? k0 + per : Sk;
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int r = lane / VPR, v = lane % VPR;
  double best = 0.0;
  // `base` is the same for every lane of the wave, so the shuffles below run
  // with the whole wave active.
  for (int64_t base = k0 + wave * RPW; base < k1; base += 4 * RPW) {
    const int64_t key = base + r;
    double ss = 0.0;
    if (key < k1) {
      const uint4 raw = *reinterpret_cast<const uint4*>(kh + key * sks + v * (16 / sizeof(T)));
      const T* e = reinterpret_cast<const T*>(&raw);
#pragma unroll
      for (int i = 0; i < int(16 / sizeof(T)); ++i) {
        const double x = double(to_f32(e[i]));
        ss = __builtin_fma(x, x, ss);
      }
    }
#pragma unroll
    for (int o = 1; o < VPR; o <<= 1) ss += __shfl_xor(ss, o);  // sum over the row's lanes
    best = ss > best ? ss : best;
  }
  __shared__ double red[256];
  red[threadIdx.x] = best;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (int(threadIdx.x) < s) {
      const double o = red[threadIdx.x + s];
      if (o > red[threadIdx.x]) red[threadIdx.x] = o;
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) partial[bh * kNormParts + blockIdx.x] = float(red[0]);
}

// Any layout: one row per thread, element by element.
template <typename T>
__global__ __launch_bounds__(256) void key_norm_partial_kernel(
    const T* __restrict__ k, int64_t skb, int64_t skh, int64_t sks, int64_t Hk, int64_t Sk,
    int64_t D, float* __restrict__ partial) {
  const int64_t bh = blockIdx.y;
  const int64_t b = bh / Hk, h = bh % Hk;
  const T* kh = k + b * skb + h * skh;
  const int64_t per = (Sk + kNormParts - 1) / kNormParts;
  const int64_t k0 = int64_t(blockIdx.x) * per;
  const int64_t k1 = (k0 + per < Sk) ? k0 + per : Sk;
  double best = 0.0;
  for (int64_t key = k0 + threadIdx.x; key < k1; key += blockDim.x) {
    const T* kr = kh + key * sks;
    double ss = 0.0;
    for (int64_t d = 0; d < D; ++d) {
      const double x = double(to_f32(kr[d]));
      ss = __builtin_fma(x, x, ss);
    }
    best = ss > best ? ss : best;
  }
  __shared__ double red[256];
  red[threadIdx.x] = best;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (int(threadIdx.x) < s) {
      const double o = red[threadIdx.x + s];
      if (o > red[threadIdx.x]) red[threadIdx.x] = o;
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) partial[bh * kNormParts + blockIdx.x] = float(red[0]);
}

__global__ __launch_bounds__(64) void key_norm_final_kernel(const float* __restrict__ partial,
                                                            int64_t n, float* __restrict__ out) {
  const int64_t bh = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (bh >= n) return;
  double best = 0.0;
  for (int p = 0; p < kNormParts; ++p) {
    const double v = double(partial[bh * kNormParts + p]);
    best = v > best ? v : best;
  }
  // sqrt of an upper bound of the squared norm, rounded up generously.
  out[bh] = float(__builtin_sqrt(best) * (1.0 + 0x1p-20));
}

template <typename T>
static hipError_t launch_key_norm_t(const void* k, int64_t skb, int64_t skh, int64_t sks,
                                    int64_t B, int64_t Hk, int64_t Sk, int64_t D, float* partial,
                                    float* out, hipStream_t stream) {
  const dim3 grid(kNormParts, unsigned(B * Hk));
  const T* kp = static_cast<const T*>(k);
  const int64_t row_bytes = D * int64_t(sizeof(T)), a = 16 / int64_t(sizeof(T));
  const bool vec = reinterpret_cast<uintptr_t>(k) % 16 == 0 && skb % a == 0 && skh % a == 0 &&
                   sks % a == 0 && row_bytes % 16 == 0;
  const int64_t vpr = row_bytes / 16;
  if (vec && vpr == 8)
    hipLaunchKernelGGL((key_norm_partial_vec_kernel<T, 8>), grid, dim3(256), 0, stream, kp, skb,
                       skh, sks, Hk, Sk, partial);
  else if (vec && vpr == 16)
    hipLaunchKernelGGL((key_norm_partial_vec_kernel<T, 16>), grid, dim3(256), 0, stream, kp, skb,
                       skh, sks, Hk, Sk, partial);
  else if (vec && vpr == 32)
    hipLaunchKernelGGL((key_norm_partial_vec_kernel<T, 32>), grid, dim3(256), 0, stream, kp, skb,
                       skh, sks, Hk, Sk, partial);
  else
    hipLaunchKernelGGL((key_norm_partial_kernel<T>), grid, dim3(256), 0, stream, kp, skb, skh,
                       sks, Hk, Sk, D, partial);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int64_t n = B * Hk;
  hipLaunchKernelGGL(key_norm_final_kernel, dim3(unsigned((n + 63) / 64)), dim3(64), 0, stream,
                     partial, n, out);
  return hipGetLastError();
}

int64_t key_norm_scratch_floats(int64_t B, int64_t Hk) { return B * Hk * (kNormParts + 1); }

// scratch: key_norm_scratch_floats(B, Hk) floats; result = first B*Hk floats.
hipError_t launch_key_norm(int dtype, const void* k, int64_t skb, int64_t skh, int64_t sks,
                           int64_t B, int64_t Hk, int64_t Sk, int64_t D, float* scratch,
                           hipStream_t stream) {
  float* out = scratch;
  float* partial = scratch + B * Hk;
  switch (dtype) {
    case kF32: return launch_key_norm_t<float>(k, skb, skh, sks, B, Hk, Sk, D, partial, out, stream);
    case kBF16: return launch_key_norm_t<bf16_t>(k, skb, skh, sks, B, Hk, Sk, D, partial, out, stream);
    case kF16: return launch_key_norm_t<f16_t>(k, skb, skh, sks, B, Hk, Sk, D, partial, out, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace va
