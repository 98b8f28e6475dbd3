// Vector-sparse flash-attention prefill on CDNA4 bf16/fp16 MFMA.
//
// Replaces vllm_flash_attn.sparse_attn_func as called at
// spattn/src/VecAttention.py:110-121 (semantics restated from
// spattn/threshold/model_tuner.py:193-216; see keylist.h).  One work-group
// owns one q-block (QPS rows) of one q head; it walks that block's key list in
// tiles of 64 keys, gathering the K and V rows of each tile into LDS, and runs
// an online softmax.  GQA is native: q head h reads kv head h / (Hq / Hk).
//
// Wave w owns query rows [32w, 32w+32) of the block and computes, per 32-key
// half of a tile, S^T = K Q^T with v_mfma_f32_32x32x16 (A = K rows from LDS,
// B = Q^T held in VGPRs for the whole kernel).  In the 32x32 accumulator a lane
// holds one query (column l%32) and 16 keys, so the row max / row sum of the
// softmax are in-lane reductions plus one exchange with lane l^32.  The
// probabilities then feed O^T += V^T P^T directly as the B operand: the k-slot
// order of the B operand is the accumulator's key order with bits 2 and 3 of
// the key index swapped, and V is written to LDS transposed (V^T[d][key]) in
// that permuted key order, so the A operand is one 16-byte LDS read.
//
// Algorithmic work per gathered key: 4*D FLOPs per query row (QK^T and PV).
#include "keylist.h"
#include "mfma.h"

namespace va {

constexpr int kTileKeys = 64;

// Swap bits 2 and 3 of a key index inside its 16-key group (an involution).
__device__ inline int perm_key(int kk) {
  return (kk & ~12) | ((kk & 4) << 1) | ((kk & 8) >> 1);
}

template <typename T, int D, int QPS>
__global__ __launch_bounds__(QPS * 2, 2) void attn_mfma_kernel(
    const T* __restrict__ q, int64_t sqb, int64_t sqh, int64_t sqs,
    const T* __restrict__ k, int64_t skb, int64_t skh, int64_t sks,
    const T* __restrict__ v, int64_t svb, int64_t svh, int64_t svs,
    T* __restrict__ out, int64_t sob, int64_t soh, int64_t sos, int64_t B,
    int64_t Hq, int64_t Hk, int64_t Sq, int64_t Sk, int causal, float scale_log2,
    const int32_t* __restrict__ counts, const int32_t* __restrict__ indices,
    RowLayout lay) {
  using M = Mfma<T>;
  using vec = typename M::vec;
  constexpr int NT = QPS * 2;              // threads
  constexpr int KS = D + 8;                // K tile row stride (elements)
  constexpr int VS = kTileKeys + 8;        // V^T row stride (elements)
  constexpr int DCH = D / 8;               // 16-byte chunks per row
  constexpr int KTOTAL = kTileKeys * DCH;          // 16-byte K chunks per tile
  constexpr int VTOTAL = (kTileKeys / 4) * DCH;    // (key quad, d chunk) units per tile
  constexpr int KLOADS = (KTOTAL + NT - 1) / NT;   // per thread
  constexpr int VUNITS = (VTOTAL + NT - 1) / NT;   // per thread

  __shared__ __attribute__((aligned(16))) uint16_t Ks[kTileKeys * KS];
  __shared__ __attribute__((aligned(16))) uint16_t Vt[D * VS];
  __shared__ int32_t kid[2][kTileKeys];  // key ids of tiles t (slot t & 1)

  const int tid = threadIdx.x;
  const int wave = tid / 64, lane = tid % 64;
  const int l32 = lane % 32, hh = lane / 32;

  const WorkOrder wo{lay.nc, B, Hq, Hk};
  int64_t jr, bh;
  if (!wo.map_item(blockIdx.x, jr, bh)) return;  // idle block (uniform)
  const int64_t b = bh / Hq, h = bh % Hq, hk = h / (Hq / Hk);
  const int64_t J = lay.J0 + jr;

  int64_t cnt = counts ? counts[bh * lay.nc + jr] : 0;
  const int64_t cap = lay.capacity(J);
  if (cnt > cap) cnt = cap;
  const int32_t* cols = indices ? indices + lay.row_offset(bh, jr) : nullptr;
  const KeyList kl = KeyList::make(J, QPS, Sk, causal, cnt, cols);
  const int64_t t_init = (kl.n_init + kTileKeys - 1) / kTileKeys;
  const int64_t t_diag = (kl.n_diag + kTileKeys - 1) / kTileKeys;
  const int64_t t_col = (kl.n_col + kTileKeys - 1) / kTileKeys;
  const int64_t ntiles = t_init + t_diag + t_col;

  // Q^T operand: lane holds row (32*wave + l32), features [16s + 8hh, +8).
  const int qrow_local = 32 * wave + l32;
  const int64_t qpos = J * QPS + qrow_local;
  vec qreg[D / 16];
  {
    const T* qr = q + b * sqb + h * sqh + qpos * sqs;
#pragma unroll
    for (int s = 0; s < D / 16; ++s) {
      uint4 raw = make_uint4(0, 0, 0, 0);
      if (qpos < Sq) raw = *reinterpret_cast<const uint4*>(qr + 16 * s + 8 * hh);
      qreg[s] = __builtin_bit_cast(vec, raw);
    }
  }

  const T* kh = k + b * skb + hk * skh;
  const T* vh = v + b * svb + hk * svh;

  // Key of tile-relative slot kk of tile t (-1 if the slot is empty).
  auto tile_key = [&](int64_t t, int kk) -> int64_t {
    if (t < t_init) {
      const int64_t p = t * kTileKeys + kk;
      return p < kl.n_init ? p : -1;
    }
    if (t < t_init + t_diag) {
      const int64_t p = (t - t_init) * kTileKeys + kk;
      return p < kl.n_diag ? kl.diag0 + p : -1;
    }
    const int64_t p = (t - t_init - t_diag) * kTileKeys + kk;
    if (p >= kl.n_col) return -1;
    const int64_t key = kl.cols[p];
    return (key >= 0 && key < Sk) ? key : -1;  // never read outside K / V
  };

  uint4 kbuf[KLOADS];
  uint4 vbuf[VUNITS][4];

  auto load_tile = [&](const int32_t* ids) {
#pragma unroll
    for (int x = 0; x < KLOADS; ++x) {
      const int c = tid + NT * x;
      if (KTOTAL % NT != 0 && c >= KTOTAL) break;
      const int kk = c / DCH, dc = c % DCH;
      const int64_t key = ids[kk];
      kbuf[x] = key >= 0 ? *reinterpret_cast<const uint4*>(kh + key * sks + dc * 8)
                         : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int x = 0; x < VUNITS; ++x) {
      const int u = tid + NT * x;
      if (VTOTAL % NT != 0 && u >= VTOTAL) break;
      const int kq = u % (kTileKeys / 4), dc = u / (kTileKeys / 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t key = ids[4 * kq + i];
        vbuf[x][i] = key >= 0 ? *reinterpret_cast<const uint4*>(vh + key * svs + dc * 8)
                              : make_uint4(0, 0, 0, 0);
      }
    }
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int x = 0; x < KLOADS; ++x) {
      const int c = tid + NT * x;
      if (KTOTAL % NT != 0 && c >= KTOTAL) break;
      const int kk = c / DCH, dc = c % DCH;
      *reinterpret_cast<uint4*>(&Ks[kk * KS + dc * 8]) = kbuf[x];
    }
#pragma unroll
    for (int x = 0; x < VUNITS; ++x) {
      const int u = tid + NT * x;
      if (VTOTAL % NT != 0 && u >= VTOTAL) break;
      const int kq = u % (kTileKeys / 4), dc = u / (kTileKeys / 4);
      const int pos = perm_key(4 * kq);  // quads stay contiguous under the swap
      const uint16_t* e0 = reinterpret_cast<const uint16_t*>(&vbuf[x][0]);
      const uint16_t* e1 = reinterpret_cast<const uint16_t*>(&vbuf[x][1]);
      const uint16_t* e2 = reinterpret_cast<const uint16_t*>(&vbuf[x][2]);
      const uint16_t* e3 = reinterpret_cast<const uint16_t*>(&vbuf[x][3]);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        uint2 w;
        w.x = uint32_t(e0[e]) | (uint32_t(e1[e]) << 16);
        w.y = uint32_t(e2[e]) | (uint32_t(e3[e]) << 16);
        *reinterpret_cast<uint2*>(&Vt[(dc * 8 + e) * VS + pos]) = w;
      }
    }
  };

  f32x16_t o[D / 32];
#pragma unroll
  for (int i = 0; i < D / 32; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[i][e] = 0.f;
  float m_run = -__builtin_inff(), l_run = 0.f;

  // Key ids run two tiles ahead of the K/V gathers: the id of tile t+2 is
  // read from the index list one iteration before it is needed.
  int32_t nid = -1;
  if (ntiles > 0) {
    if (tid < kTileKeys) {
      kid[0][tid] = int32_t(tile_key(0, tid));
      kid[1][tid] = ntiles > 1 ? int32_t(tile_key(1, tid)) : -1;
      nid = ntiles > 2 ? int32_t(tile_key(2, tid)) : -1;
    }
    lds_barrier();
    load_tile(kid[0]);
    store_tile();
    lds_barrier();
  }

  for (int64_t t = 0; t < ntiles; ++t) {
    const bool more = (t + 1) < ntiles;
    if (more) load_tile(kid[(t + 1) & 1]);  // in flight while this tile computes

    // ---- S^T = K Q^T for the two 32-key halves -----------------------------
    f32x16_t s[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int e = 0; e < 16; ++e) s[kb][e] = 0.f;
      const uint16_t* krow = &Ks[(kb * 32 + l32) * KS + 8 * hh];
#pragma unroll
      for (int st = 0; st < D / 16; ++st) {
        const vec a = __builtin_bit_cast(vec, *reinterpret_cast<const uint4*>(krow + 16 * st));
        s[kb] = M::run(a, qreg[st], s[kb]);
      }
    }

    // ---- masking: empty slots, causal diagonal ------------------------------
    int lim;      // valid slots in this tile
    int dshift;   // for diagonal tiles: key - diag0 = dshift + slot
    bool diag = false;
    if (t < t_init) {
      const int64_t l = kl.n_init - t * kTileKeys;
      lim = l > kTileKeys ? kTileKeys : int(l);
      dshift = 0;
    } else if (t < t_init + t_diag) {
      dshift = int(t - t_init) * kTileKeys;
      const int64_t l = kl.n_diag - dshift;
      lim = l > kTileKeys ? kTileKeys : int(l);
      diag = causal != 0;
    } else {
      const int64_t l = kl.n_col - (t - t_init - t_diag) * kTileKeys;
      lim = l > kTileKeys ? kTileKeys : int(l);
      dshift = 0;
    }
    float tmax = -__builtin_inff();
    if (!diag && lim == kTileKeys) {  // full tile, nothing masked
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const float x = s[kb][e] * scale_log2;
          s[kb][e] = x;
          tmax = __builtin_fmaxf(tmax, x);
        }
    } else {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int slot = kb * 32 + 8 * (e / 4) + 4 * hh + (e % 4);
          bool ok = slot < lim;
          if (diag) ok = ok && (dshift + slot <= qrow_local);
          const float x = ok ? s[kb][e] * scale_log2 : -__builtin_inff();
          s[kb][e] = x;
          tmax = __builtin_fmaxf(tmax, x);
        }
      }
    }
    tmax = __builtin_fmaxf(tmax, __shfl_xor(tmax, 32));
    const float m_new = __builtin_fmaxf(m_run, tmax);
    const float m_use = (m_new == -__builtin_inff()) ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
    float lsum = 0.f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float p = __builtin_amdgcn_exp2f(s[kb][e] - m_use);
        s[kb][e] = p;
        lsum += p;
      }
    }
    lsum += __shfl_xor(lsum, 32);
    l_run = l_run * alpha + lsum;
    m_run = m_new;
    if (__ballot(alpha != 1.f)) {  // some row's maximum moved
#pragma unroll
      for (int i = 0; i < D / 32; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[i][e] *= alpha;
    }

    // ---- O^T += V^T P^T ------------------------------------------------------
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const int kb = st / 2, sub = st % 2;
      float pv[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        pv[e] = s[kb][4 * (2 * sub) + e];
        pv[4 + e] = s[kb][4 * (2 * sub + 1) + e];
      }
      const vec bfrag = M::pack(pv);
#pragma unroll
      for (int i = 0; i < D / 32; ++i) {
        const uint16_t* vrow = &Vt[(i * 32 + l32) * VS + 16 * st + 8 * hh];
        const vec a = __builtin_bit_cast(vec, *reinterpret_cast<const uint4*>(vrow));
        o[i] = M::run(a, bfrag, o[i]);
      }
    }

    __syncthreads();  // K/V of tile t+1 have arrived; Ks/Vt of tile t are free
    if (tid < kTileKeys) {
      kid[t & 1][tid] = nid;  // ids of tile t+2 (slot t & 1 was consumed by load_tile(t))
      nid = (t + 3 < ntiles) ? int32_t(tile_key(t + 3, tid)) : -1;
    }
    if (more) store_tile();
    lds_barrier();
  }

  // ---- epilogue: O / l, four consecutive features per store ----------------
  if (qpos < Sq) {
    const float inv = l_run > 0.f ? 1.f / l_run : 0.f;
    T* orow = out + b * sob + h * soh + qpos * sos;
#pragma unroll
    for (int i = 0; i < D / 32; ++i) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d0 = i * 32 + 8 * g + 4 * hh;
        uint2 w;
        const T e0 = Round<T>::store(o[i][4 * g + 0] * inv);
        const T e1 = Round<T>::store(o[i][4 * g + 1] * inv);
        const T e2 = Round<T>::store(o[i][4 * g + 2] * inv);
        const T e3 = Round<T>::store(o[i][4 * g + 3] * inv);
        w.x = uint32_t(e0.bits) | (uint32_t(e1.bits) << 16);
        w.y = uint32_t(e2.bits) | (uint32_t(e3.bits) << 16);
        *reinterpret_cast<uint2*>(orow + d0) = w;
      }
    }
  }
}

template <typename T, int D, int QPS>
static hipError_t launch_attn_mfma_tdq(const void* q, const int64_t* sq, const void* k,
                                       const int64_t* sk, const void* v, const int64_t* sv,
                                       void* out, const int64_t* so, int64_t B, int64_t Hq,
                                       int64_t Hk, int64_t Sq, int64_t Sk, int causal,
                                       float scale_log2, const int32_t* counts,
                                       const int32_t* indices, const RowLayout& lay,
                                       hipStream_t stream) {
  const int64_t nblocks = WorkOrder{lay.nc, B, Hq, Hk}.grid_items();
  hipLaunchKernelGGL((attn_mfma_kernel<T, D, QPS>), dim3(unsigned(nblocks)), dim3(QPS * 2), 0,
                     stream, static_cast<const T*>(q), sq[0], sq[1], sq[2],
                     static_cast<const T*>(k), sk[0], sk[1], sk[2], static_cast<const T*>(v),
                     sv[0], sv[1], sv[2], static_cast<T*>(out), so[0], so[1], so[2], B, Hq, Hk,
                     Sq, Sk, causal, scale_log2, counts, indices, lay);
  return hipGetLastError();
}

template <typename T>
static hipError_t launch_attn_mfma_t(int64_t D, int64_t qps, const void* q, const int64_t* sq,
                                     const void* k, const int64_t* sk, const void* v,
                                     const int64_t* sv, void* out, const int64_t* so, int64_t B,
                                     int64_t Hq, int64_t Hk, int64_t Sq, int64_t Sk, int causal,
                                     float scale_log2, const int32_t* counts,
                                     const int32_t* indices, const RowLayout& lay,
                                     hipStream_t stream) {
#define VA_ATTN_CASE(DD, QQ)                                                                   \
  if (D == DD && qps == QQ)                                                                    \
    return launch_attn_mfma_tdq<T, DD, QQ>(q, sq, k, sk, v, sv, out, so, B, Hq, Hk, Sq, Sk,   \
                                           causal, scale_log2, counts, indices, lay, stream);
  VA_ATTN_CASE(64, 64)
  VA_ATTN_CASE(128, 64)
  VA_ATTN_CASE(64, 128)
  VA_ATTN_CASE(128, 128)
#undef VA_ATTN_CASE
  return hipErrorInvalidValue;
}

bool attn_mfma_supported(int dtype, int64_t D, int64_t qps) {
  return (dtype == kBF16 || dtype == kF16) && (D == 64 || D == 128) && (qps == 64 || qps == 128);
}

hipError_t launch_attn_mfma(int dtype, int64_t D, int64_t qps, const void* q, const int64_t* sq,
                            const void* k, const int64_t* sk, const void* v, const int64_t* sv,
                            void* out, const int64_t* so, int64_t B, int64_t Hq, int64_t Hk,
                            int64_t Sq, int64_t Sk, int causal, float scale_log2,
                            const int32_t* counts, const int32_t* indices, const RowLayout& lay,
                            hipStream_t stream) {
  if (dtype == kBF16)
    return launch_attn_mfma_t<bf16_t>(D, qps, q, sq, k, sk, v, sv, out, so, B, Hq, Hk, Sq, Sk,
                                      causal, scale_log2, counts, indices, lay, stream);
  if (dtype == kF16)
    return launch_attn_mfma_t<f16_t>(D, qps, q, sq, k, sk, v, sv, out, so, B, Hq, Hk, Sq, Sk,
                                     causal, scale_log2, counts, indices, lay, stream);
  return hipErrorInvalidValue;
}

}  // namespace va
