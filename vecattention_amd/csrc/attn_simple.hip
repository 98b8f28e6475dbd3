// Vector-sparse attention, four lanes per query row (any element type).
//
// Semantics of the reference call vllm_flash_attn.sparse_attn_func at
// spattn/src/VecAttention.py:110-121 as restated by the dense-mask code of
// spattn/threshold/model_tuner.py:193-216: for query row i of q-block J,
// softmax(q_i . k_c / sqrt(D)) over the keys of KeyList(J) (local blocks +
// selected columns, causal mask on the diagonal block), times V.  A row with
// no key gets 0.
//
// This kernel serves fp32 inputs (which the MFMA kernel does not take) and is
// an independent GPU cross-check of the MFMA kernel.  Four lanes (a quad)
// serve one query row, lane j holding features [j*DQ, (j+1)*DQ) of the row and
// of its output accumulator in registers (DQ = ceil(D/4) rounded up to 16, 32
// or 64): each score is the quad's four partial dot products added with two
// lane swaps, so the four lanes hold the same score and run the same online
// softmax.  A work-group covers 64 rows of a q-block; every key row is read by
// all quads of the work-group at once, so loads broadcast through L1, and the
// keys are taken in batches whose loads are issued together.
//
// dense_qoff >= 0: every key instead (KeyList::dense, causal rows aligned at
// offset dense_qoff).  stats != nullptr: no V; row i of head bh writes
// stats[(bh * Sq + i) * 2 + {0, 1}] = (m, l), the row maximum of the scaled
// scores in log2 units and l = sum of 2^(s * scale_log2 - m) over its keys
// (m = -inf, l = 0 for a row without keys).
#include "keylist.h"

namespace va {

constexpr int kSimpleMaxD = 256;
constexpr int kSimpleRows = 64;  // query rows per work-group (4 lanes each)

// x summed over the four lanes of each quad (the same value in all four).
__device__ inline float quad_sum(float x) {
  const float a = x + __builtin_bit_cast(
                          float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0xb1, 0xf,
                                                          0xf, false));  // quad_perm [1,0,3,2]
  return a + __builtin_bit_cast(
                 float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, a), 0x4e, 0xf, 0xf,
                                                 false));  // quad_perm [2,3,0,1]
}

// kFull: D == 4 * DQ (every lane's features exist; no per-feature guards).
template <typename T, int DQ, bool kFull>
__global__ __launch_bounds__(4 * kSimpleRows) void attn_simple_kernel(
    const T* __restrict__ q, int64_t sqb, int64_t sqh, int64_t sqs,
    const T* __restrict__ k, int64_t skb, int64_t skh, int64_t sks,
    const T* __restrict__ v, int64_t svb, int64_t svh, int64_t svs,
    T* __restrict__ out, int64_t sob, int64_t soh, int64_t sos, int64_t B,
    int64_t Hq, int64_t Hk, int64_t Sq, int64_t Sk, int64_t D, int64_t qps,
    int causal, float scale_log2, const int32_t* __restrict__ counts,
    const int32_t* __restrict__ indices, RowLayout lay, int64_t dense_qoff,
    float* __restrict__ stats) {
  const int64_t BH = B * Hq;
  const int64_t parts = (qps + kSimpleRows - 1) / kSimpleRows;  // work-groups per q-block
  const int64_t item = int64_t(blockIdx.x) / parts, part = int64_t(blockIdx.x) % parts;
  const int64_t jr = lay.nc - 1 - item / BH;
  const int64_t bh = item % BH;
  const int64_t b = bh / Hq, h = bh % Hq, hk = h / (Hq / Hk);
  const int64_t J = lay.J0 + jr;
  const int64_t row = part * kSimpleRows + threadIdx.x / 4;
  const int qlane = threadIdx.x % 4;
  const int64_t qpos = J * qps + row;
  // Rows past the q-block or past Sq compute row 0 of the block (whole quads,
  // so that the lane swaps see live lanes) and write nothing.
  const bool live = row < qps && qpos < Sq;
  const int64_t qrow = live ? qpos : J * qps;

  int64_t cnt = counts ? counts[bh * lay.nc + jr] : 0;
  const int64_t cap = lay.capacity(J);
  if (cnt > cap) cnt = cap;
  const int32_t* cols = indices ? indices + lay.row_offset(bh, jr) : nullptr;
  const KeyList kl = dense_qoff >= 0 ? KeyList::dense(J, qps, Sk, causal, dense_qoff)
                                     : KeyList::make(J, qps, Sk, causal, cnt, cols);
  const int64_t qkey = qrow + (dense_qoff > 0 ? dense_qoff : 0);  // last visible diagonal key

  // this lane's features: d0 + i for i < DQ with d0 + i < D
  const int64_t d0 = int64_t(qlane) * DQ;
  float qv[DQ], acc[DQ];
  const T* qr = q + b * sqb + h * sqh + qrow * sqs;
#pragma unroll
  for (int i = 0; i < DQ; ++i) {
    qv[i] = (kFull || d0 + i < D) ? to_f32(qr[d0 + i]) : 0.f;
    acc[i] = 0.f;
  }
  const T* kh = k + b * skb + hk * skh;
  const T* vh = v + b * svb + hk * svh;
  float m = -__builtin_inff(), l = 0.f;
  const int64_t n = kl.total();
  // Keys in batches of NB: the batch's K rows are loaded together, the online
  // softmax rescales once per batch (by the batch maximum), then the V rows
  // are loaded together, so a batch waits on memory twice instead of each key
  // twice.  A masked slot (past the list, outside [0, Sk), or after the row on
  // the diagonal block) reads key row 0 and weighs 0.
  constexpr int NB = DQ <= 16 ? 8 : (DQ <= 32 ? 4 : 2);
  for (int64_t p0 = 0; p0 < n; p0 += NB) {
    int64_t key[NB];
    bool ok[NB];
    const int64_t c0 = kl.n_init + kl.n_diag;  // first position of the selected columns
    if (p0 >= c0 && p0 + NB <= n) {
      // a whole batch of selected columns (every batch of a non-causal row):
      // its ids in one block of consecutive (scalar) loads
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        const int64_t kk = kl.cols[p0 - c0 + j];
        ok[j] = kk >= 0 && kk < Sk;
        key[j] = ok[j] ? kk : 0;
      }
    } else {
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        const int64_t p = p0 + j;
        const int64_t kk = p < n ? kl.key(p) : -1;  // the same key in every lane of the work-group
        ok[j] = kk >= 0 && kk < Sk && !(causal && kl.is_diag(p) && kk > qkey);
        key[j] = ok[j] ? kk : 0;
      }
    }
    float s[NB];
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const T* kr = kh + key[j] * sks + d0;
      float a = 0.f;
#pragma unroll
      for (int i = 0; i < DQ; ++i) a += (kFull || d0 + i < D) ? qv[i] * to_f32(kr[i]) : 0.f;
      s[j] = a;
    }
    float mb = m;
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      s[j] = quad_sum(s[j]) * scale_log2;  // the quad's four lanes share the row: same ok[j]
      if (ok[j]) mb = __builtin_fmaxf(mb, s[j]);
    }
    // a batch with no key of the row so far leaves (m, l, acc) unchanged
    const bool any = mb != -__builtin_inff();
    const float alpha = any ? __builtin_amdgcn_exp2f(m - mb) : 1.f;
    float pe[NB], ps = 0.f;
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      pe[j] = ok[j] ? __builtin_amdgcn_exp2f(s[j] - mb) : 0.f;
      ps += pe[j];
    }
    l = l * alpha + ps;
    m = mb;
    if (stats) continue;
#pragma unroll
    for (int i = 0; i < DQ; ++i) acc[i] *= alpha;
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const T* vr = vh + key[j] * svs + d0;
#pragma unroll
      for (int i = 0; i < DQ; ++i)
        if (kFull || d0 + i < D) acc[i] += pe[j] * to_f32(vr[i]);
    }
  }
  if (!live) return;
  if (stats) {
    if (qlane == 0) *reinterpret_cast<float2*>(stats + (bh * Sq + qpos) * 2) = make_float2(m, l);
    return;
  }
  const float inv = l > 0.f ? 1.f / l : 0.f;
  T* orow = out + b * sob + h * soh + qpos * sos + d0;
#pragma unroll
  for (int i = 0; i < DQ; ++i)
    if (kFull || d0 + i < D) orow[i] = Round<T>::store(acc[i] * inv);
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
  const int64_t parts = (qps + kSimpleRows - 1) / kSimpleRows;
  const int64_t nblocks = lay.nc * B * Hq * parts;
  auto go = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, dim3(unsigned(nblocks)), dim3(4 * kSimpleRows), 0, stream,
                       static_cast<const T*>(q), sq[0], sq[1], sq[2], static_cast<const T*>(k),
                       sk[0], sk[1], sk[2], static_cast<const T*>(v), sv[0], sv[1], sv[2],
                       static_cast<T*>(out), so[0], so[1], so[2], B, Hq, Hk, Sq, Sk, D, qps,
                       causal, scale_log2, counts, indices, lay, dense_qoff, stats);
    return hipGetLastError();
  };
  if (D == 64) return go(attn_simple_kernel<T, 16, true>);
  if (D == 128) return go(attn_simple_kernel<T, 32, true>);
  if (D < 64) return go(attn_simple_kernel<T, 16, false>);
  if (D < 128) return go(attn_simple_kernel<T, 32, false>);
  if (D <= kSimpleMaxD) return go(attn_simple_kernel<T, 64, false>);
  return hipErrorInvalidValue;
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
