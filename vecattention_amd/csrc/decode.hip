// Decode attention, merge step: combines the split-key partials that the
// attention kernel's split form writes (one normalised fp32 output row and
// (m, l) per query row and key range) into the output rows.
//
//   out_r = sum_s w_s O_s / sum_s w_s,   w_s = l_s * 2^(m_s - M),  M = max_s m_s
//
// is the softmax over the union of the key ranges (flash-decoding's merge of
// partial softmax states).
#include "common.h"

namespace va {

// One work-group of 256 threads per (group g, row r), whose nsplit partial
// rows are contiguous: thread t takes features [4 (t % (D/4)), +4) of the
// splits s = t / (D/4) (mod P = 256 / (D/4)) and merges them online (running
// maximum, rescaled sums), with the loads of U splits in flight; the P
// partial merges of a feature are then combined through LDS.  One pass over
// memory, no dependent round trip.
template <typename T, int D>
__global__ __launch_bounds__(256) void decode_merge_kernel(const float* __restrict__ part,
                                                           int64_t G, int64_t Sq, int64_t nsplit,
                                                           T* __restrict__ out, int64_t sog,
                                                           int64_t sor) {
  constexpr int TPR = D / 4;    // threads per partial row
  constexpr int P = 256 / TPR;  // partial rows read side by side
  constexpr int U = 4;          // splits per thread in flight
  __shared__ float4 sacc[P][TPR];
  __shared__ float smax[P], sden[P];
  const int64_t item = blockIdx.x;  // g * Sq + r
  const int t = threadIdx.x, c = t % TPR, p = t / TPR;
  const int64_t g = item / Sq, r = item % Sq;
  const float2* ml = reinterpret_cast<const float2*>(part) + item * nsplit;  // (m, l) of split s
  const float4* po = reinterpret_cast<const float4*>(
                         part + (2 * G * nsplit * Sq + 3) / 4 * 4 + item * nsplit * D) + c;
  float mrun = -__builtin_inff(), den = 0.f;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int64_t s0 = p; s0 < nsplit; s0 += int64_t(P) * U) {
    float2 st[U];
    float4 x[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t s = s0 + int64_t(u) * P;
      st[u] = s < nsplit ? ml[s] : make_float2(-__builtin_inff(), 0.f);
      x[u] = s < nsplit ? po[s * (D / 4)] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (!(st[u].y > 0.f)) continue;  // an empty span contributes nothing
      const float mnew = __builtin_fmaxf(mrun, st[u].x);
      const float a = __builtin_amdgcn_exp2f(mrun - mnew);  // 0 while mrun is -inf
      const float w = st[u].y * __builtin_amdgcn_exp2f(st[u].x - mnew);
      den = den * a + w;
      acc.x = acc.x * a + w * x[u].x;
      acc.y = acc.y * a + w * x[u].y;
      acc.z = acc.z * a + w * x[u].z;
      acc.w = acc.w * a + w * x[u].w;
      mrun = mnew;
    }
  }
  sacc[p][c] = acc;
  if (c == 0) {
    smax[p] = mrun;
    sden[p] = den;
  }
  __syncthreads();
  if (p == 0) {
    float M = -__builtin_inff();
#pragma unroll
    for (int j = 0; j < P; ++j) M = __builtin_fmaxf(M, smax[j]);
    float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
    float dn = 0.f;
#pragma unroll
    for (int j = 0; j < P; ++j) {
      if (!(sden[j] > 0.f)) continue;
      const float f = __builtin_amdgcn_exp2f(smax[j] - M);
      const float4 xj = sacc[j][c];
      a.x += f * xj.x;
      a.y += f * xj.y;
      a.z += f * xj.z;
      a.w += f * xj.w;
      dn += f * sden[j];
    }
    const float inv = dn > 0.f ? 1.f / dn : 0.f;
    T* orow = out + g * sog + r * sor + 4 * c;
    orow[0] = Round<T>::store(a.x * inv);
    orow[1] = Round<T>::store(a.y * inv);
    orow[2] = Round<T>::store(a.z * inv);
    orow[3] = Round<T>::store(a.w * inv);
  }
}

template <typename T>
static hipError_t launch_decode_merge_t(int64_t D, const float* part, int64_t G, int64_t Sq,
                                        int64_t nsplit, void* out, int64_t sog, int64_t sor,
                                        hipStream_t stream) {
  const unsigned nblocks = unsigned(G * Sq);
  if (D == 64)
    hipLaunchKernelGGL((decode_merge_kernel<T, 64>), dim3(nblocks), dim3(256), 0, stream, part, G,
                       Sq, nsplit, static_cast<T*>(out), sog, sor);
  else if (D == 128)
    hipLaunchKernelGGL((decode_merge_kernel<T, 128>), dim3(nblocks), dim3(256), 0, stream, part,
                       G, Sq, nsplit, static_cast<T*>(out), sog, sor);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_decode_merge(int dtype, int64_t D, const float* part, int64_t G, int64_t Sq,
                               int64_t nsplit, void* out, int64_t sog, int64_t sor,
                               hipStream_t stream) {
  if (dtype == kBF16)
    return launch_decode_merge_t<bf16_t>(D, part, G, Sq, nsplit, out, sog, sor, stream);
  if (dtype == kF16)
    return launch_decode_merge_t<f16_t>(D, part, G, Sq, nsplit, out, sog, sor, stream);
  return hipErrorInvalidValue;
}

}  // namespace va
