// Vector-sparse attention, one thread per query row (any element type).
//
// Semantics of the reference call vllm_flash_attn.sparse_attn_func at
// spattn/src/VecAttention.py:110-121 as restated by the dense-mask code of
// spattn/threshold/model_tuner.py:193-216: for query row i of q-block J,
// softmax(q_i . k_c / sqrt(D)) over the keys of KeyList(J) (local blocks +
// selected columns, causal mask on the diagonal block), times V.  A row with
// no key gets 0.
//
// This kernel serves fp32 inputs (which the MFMA kernel does not take) and is
// an independent GPU cross-check of the MFMA kernel.  Every key row is read
// by all threads of the work-group at once, so loads broadcast through L1.
//
// dense_qoff >= 0: every key instead (KeyList::dense, causal rows aligned at
// offset dense_qoff).  stats != nullptr: no V; row i of head bh writes
// stats[(bh * Sq + i) * 2 + {0, 1}] = (m, l), the row maximum of the scaled
// scores in log2 units and l = sum of 2^(s * scale_log2 - m) over its keys
// (m = -inf, l = 0 for a row without keys).
#include "keylist.h"

namespace va {

constexpr int kSimpleMaxD = 256;

template <typename T>
__global__ __launch_bounds__(128) void attn_simple_kernel(
    const T* __restrict__ q, int64_t sqb, int64_t sqh, int64_t sqs,
    const T* __restrict__ k, int64_t skb, int64_t skh, int64_t sks,
    const T* __restrict__ v, int64_t svb, int64_t svh, int64_t svs,
    T* __restrict__ out, int64_t sob, int64_t soh, int64_t sos, int64_t B,
    int64_t Hq, int64_t Hk, int64_t Sq, int64_t Sk, int64_t D, int64_t qps,
    int causal, float scale_log2, const int32_t* __restrict__ counts,
    const int32_t* __restrict__ indices, RowLayout lay, int64_t dense_qoff,
    float* __restrict__ stats) {
  const int64_t BH = B * Hq;
  const int64_t jr = lay.nc - 1 - int64_t(blockIdx.x) / BH;
  const int64_t bh = int64_t(blockIdx.x) % BH;
  const int64_t b = bh / Hq, h = bh % Hq, hk = h / (Hq / Hk);
  const int64_t J = lay.J0 + jr;
  const int64_t row = threadIdx.x;
  const int64_t qpos = J * qps + row;
  if (row >= qps || qpos >= Sq) return;

  int64_t cnt = counts ? counts[bh * lay.nc + jr] : 0;
  const int64_t cap = lay.capacity(J);
  if (cnt > cap) cnt = cap;
  const int32_t* cols = indices ? indices + lay.row_offset(bh, jr) : nullptr;
  const KeyList kl = dense_qoff >= 0 ? KeyList::dense(J, qps, Sk, causal, dense_qoff)
                                     : KeyList::make(J, qps, Sk, causal, cnt, cols);
  const int64_t qkey = qpos + (dense_qoff > 0 ? dense_qoff : 0);  // last visible diagonal key

  float qv[kSimpleMaxD];
  float acc[kSimpleMaxD];
  const T* qr = q + b * sqb + h * sqh + qpos * sqs;
  for (int64_t d = 0; d < D; ++d) {
    qv[d] = to_f32(qr[d]);
    acc[d] = 0.f;
  }
  const T* kh = k + b * skb + hk * skh;
  const T* vh = v + b * svb + hk * svh;
  float m = -__builtin_inff(), l = 0.f;
  const int64_t n = kl.total();
  for (int64_t p = 0; p < n; ++p) {
    const int64_t key = kl.key(p);
    if (key < 0 || key >= Sk) continue;  // never read outside K / V
    if (causal && kl.is_diag(p) && key > qkey) continue;
    const T* kr = kh + key * sks;
    float s = 0.f;
    for (int64_t d = 0; d < D; ++d) s += qv[d] * to_f32(kr[d]);
    s *= scale_log2;
    const float m_new = __builtin_fmaxf(m, s);
    const float alpha = __builtin_amdgcn_exp2f(m - m_new);
    const float pe = __builtin_amdgcn_exp2f(s - m_new);
    l = l * alpha + pe;
    m = m_new;
    if (stats) continue;
    const T* vr = vh + key * svs;
    for (int64_t d = 0; d < D; ++d) acc[d] = acc[d] * alpha + pe * to_f32(vr[d]);
  }
  if (stats) {
    *reinterpret_cast<float2*>(stats + (bh * Sq + qpos) * 2) = make_float2(m, l);
    return;
  }
  const float inv = l > 0.f ? 1.f / l : 0.f;
  T* orow = out + b * sob + h * soh + qpos * sos;
  for (int64_t d = 0; d < D; ++d) orow[d] = Round<T>::store(acc[d] * inv);
}

template <typename T>
static hipError_t launch_attn_simple_t(const void* q, const int64_t* sq, const void* k,
                                       const int64_t* sk, const void* v, const int64_t* sv,
                                       void* out, const int64_t* so, int64_t B, int64_t Hq,
                                       int64_t Hk, int64_t Sq, int64_t Sk, int64_t D,
                                       int64_t qps, int causal, float scale_log2,
                                       const int32_t* counts, const int32_t* indices,
                                       const RowLayout& lay, int64_t dense_qoff, float* stats,
                                       hipStream_t stream) {
  const int64_t nblocks = lay.nc * B * Hq;
  hipLaunchKernelGGL((attn_simple_kernel<T>), dim3(unsigned(nblocks)), dim3(unsigned(qps)), 0,
                     stream, static_cast<const T*>(q), sq[0], sq[1], sq[2],
                     static_cast<const T*>(k), sk[0], sk[1], sk[2], static_cast<const T*>(v),
                     sv[0], sv[1], sv[2], static_cast<T*>(out), so[0], so[1], so[2], B, Hq, Hk,
                     Sq, Sk, D, qps, causal, scale_log2, counts, indices, lay, dense_qoff, stats);
  return hipGetLastError();
}

hipError_t launch_attn_simple(int dtype, const void* q, const int64_t* sq, const void* k,
                              const int64_t* sk, const void* v, const int64_t* sv, void* out,
                              const int64_t* so, int64_t B, int64_t Hq, int64_t Hk, int64_t Sq,
                              int64_t Sk, int64_t D, int64_t qps, int causal, float scale_log2,
                              const int32_t* counts, const int32_t* indices,
                              const RowLayout& lay, int64_t dense_qoff, float* stats,
                              hipStream_t stream) {
  switch (dtype) {
    case kF32:
      return launch_attn_simple_t<float>(q, sq, k, sk, v, sv, out, so, B, Hq, Hk, Sq, Sk, D, qps,
                                         causal, scale_log2, counts, indices, lay, dense_qoff,
                                         stats, stream);
    case kBF16:
      return launch_attn_simple_t<bf16_t>(q, sq, k, sk, v, sv, out, so, B, Hq, Hk, Sq, Sk, D, qps,
                                          causal, scale_log2, counts, indices, lay, dense_qoff,
                                         stats, stream);
    case kF16:
      return launch_attn_simple_t<f16_t>(q, sq, k, sk, v, sv, out, so, B, Hq, Hk, Sq, Sk, D, qps,
                                         causal, scale_log2, counts, indices, lay, dense_qoff,
                                         stats, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace va
