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
// rows are contiguous: thread t reads features [4 (t % (D/4)), +4) of the
// splits s = t / (D/4) (mod 256 / (D/4)) with 16-byte loads, all independent.
template <typename T, int D>
__global__ __launch_bounds__(256) void decode_merge_kernel(const float* __restrict__ part,
                                                           int64_t G, int64_t Sq, int64_t nsplit,
                                                           T* __restrict__ out, int64_t sog,
                                                           int64_t sor) {
  constexpr int TPR = D / 4;    // threads per partial row
  constexpr int P = 256 / TPR;  // partial rows read side by side
  __shared__ float wmax[4];
  __shared__ float4 sacc[P][TPR];
  __shared__ float sden[P];
  const int64_t item = blockIdx.x;  // g * Sq + r
  const int t = threadIdx.x, c = t % TPR, p = t / TPR;
  const int64_t g = item / Sq, r = item % Sq;
  const float2* ml = reinterpret_cast<const float2*>(part) + item * nsplit;  // (m, l) of split s
  const float4* po = reinterpret_cast<const float4*>(
                         part + (2 * G * nsplit * Sq + 3) / 4 * 4 + item * nsplit * D) + c;
  float M = -__builtin_inff();
  for (int64_t s = t; s < nsplit; s += 256) M = __builtin_fmaxf(M, ml[s].x);
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) M = __builtin_fmaxf(M, __shfl_xor(M, o));
  if (t % 64 == 0) wmax[t / 64] = M;
  __syncthreads();
  M = __builtin_fmaxf(__builtin_fmaxf(wmax[0], wmax[1]), __builtin_fmaxf(wmax[2], wmax[3]));
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  float den = 0.f;
#pragma unroll 8
  for (int64_t s = p; s < nsplit; s += P) {
    const float2 st = ml[s];
    const float w = st.y > 0.f ? st.y * __builtin_amdgcn_exp2f(st.x - M) : 0.f;
    const float4 x = po[s * (D / 4)];
    den += w;
    acc.x += w * x.x;
    acc.y += w * x.y;
    acc.z += w * x.z;
    acc.w += w * x.w;
  }
  sacc[p][c] = acc;
  if (c == 0) sden[p] = den;
  __syncthreads();
  if (p == 0) {
    float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
    float dn = 0.f;
#pragma unroll
    for (int j = 0; j < P; ++j) {
      const float4 x = sacc[j][c];
      a.x += x.x;
      a.y += x.y;
      a.z += x.z;
      a.w += x.w;
      dn += sden[j];
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
