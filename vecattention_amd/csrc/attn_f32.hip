// Vector-sparse attention for fp32 inputs on the fp32 matrix cores.
//
// Same semantics as attn_mfma.hip / attn_simple.hip (the reference call
// vllm_flash_attn.sparse_attn_func at spattn/src/VecAttention.py:110-121 as
// restated by spattn/threshold/model_tuner.py:193-216): for query row i of
// q-block J, softmax(q_i . k_c * scale) over the keys of KeyList(J) (local
// blocks + selected columns, causal mask on the diagonal block), times V; a
// row with no key gets 0.  The reference's attention extension takes only
// fp16/bf16; fp32 inputs (the reference's CPU-sized configuration) run here
// in fp32 throughout: v_mfma_f32_32x32x2_f32 products and sums, fp32 online
// softmax.
//
// A work-group takes one q-block (QPS = 64 or 128 rows) of one q head with 8
// waves (two per SIMD: 8 waves measured 6-30% faster than 4 on gfx950):
// QPS/32 row blocks of 32 rows times 8/(QPS/32) key splits, each split
// walking every KS-th 32-key tile of the row's list; the splits' states are
// merged through LDS at the end.  Per tile a wave computes
// S^T (32 keys x 32 rows) = K Q^T in D/2 MFMAs, with A = K rows and B = Q^T
// straight from registers (lane l: key / row l % 32, features (l / 32)*D/2 + s
// for step s, so each lane loads D/2 consecutive floats of its row), and
// O^T += V^T P^T in 16*D/32 MFMAs, whose B operand is the lane's own
// probabilities (the accumulator's key order is a valid k order) and whose A
// operand is one float per lane of the V row of the step's key (ids shared
// through lane shuffles).  Every K and V row feeds all 32 rows of a block from
// registers, against one row per load in the per-row kernel.
//
// Segmented lists (nseg > 1, the split selection): segment s of the row holds
// counts[(bh*nc + jr)*nseg + s] keys from slot max(s*segk, smin) - smin of the
// row.  Lane s of every wave keeps the exclusive prefix sv[s] of the segment
// counts, and column p of the concatenated list is found by a binary search
// over the lanes for the last s with sv[s] <= p (segment counts are clamped
// to the slots left in the row, as the MFMA kernel does).
#include "keylist.h"
#include "lanes.h"
#include "mfma.h"

namespace va {

constexpr int kF32Tile = 32;  // keys per tile
constexpr int kF32Waves = 8;  // waves per work-group

__device__ inline f32x16_t mfma_f32(float a, float b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

template <int D, int QPS, int W>
__global__ __launch_bounds__(64 * W) void attn_f32_kernel(
    const float* __restrict__ q, int64_t sqb, int64_t sqh, int64_t sqs,
    const float* __restrict__ k, int64_t skb, int64_t skh, int64_t sks,
    const float* __restrict__ v, int64_t svb, int64_t svh, int64_t svs,
    float* __restrict__ out, int64_t sob, int64_t soh, int64_t sos, int64_t B, int64_t Hq,
    int64_t Hk, int64_t Sq, int64_t Sk, int causal, float scale_log2,
    const int32_t* __restrict__ counts, const int32_t* __restrict__ indices, RowLayout lay,
    int nseg, int segk, int64_t dense_qoff) {
  constexpr int RB = QPS / 32;  // row blocks
  constexpr int KS = W / RB;    // key splits
  constexpr int NS = D / 2;     // QK^T steps (two features each)
  constexpr int OB = D / 32;    // output blocks of 32 features
  static_assert(RB * KS == W, "W waves per work-group");
  // merge buffer of the key splits (a single float when there is one split)
  __shared__ float mst[KS > 1 ? KS - 1 : 1][KS > 1 ? RB : 1][KS > 1 ? 64 : 1]
                      [KS > 1 ? 2 + 16 * OB : 1];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid / 64), lane = tid % 64;
  const int l32 = lane % 32, hh = lane / 32;
  const int rb = wave % RB, ks = wave / RB;

  const int64_t BH = B * Hq;
  const int64_t item = blockIdx.x;
  const int64_t jr = lay.nc - 1 - item / BH;  // longest rows first
  const int64_t bh = item % BH;
  const int64_t b = bh / Hq, h = bh % Hq, hk = h / (Hq / Hk);
  const int64_t J = lay.J0 + jr;

  const int64_t cap = lay.capacity(J);
  const int smin = int(lay.smin());
  auto seg_slot = [&](int sg) { return (sg * segk > smin ? sg * segk : smin) - smin; };
  int64_t cnt = 0;
  int sv = 0x7fffffff;  // lane s < nseg: first list column of segment s
  if (counts && nseg <= 1) {
    cnt = counts[bh * lay.nc + jr];
  } else if (counts) {
    int c = 0;
    if (lane < nseg) {
      c = counts[(bh * lay.nc + jr) * nseg + lane];
      const int room = int(cap) - seg_slot(lane);
      c = c < 0 ? 0 : (c > room ? (room > 0 ? room : 0) : c);
    }
    const int incl = wave_inclusive_sum(c);
    if (lane < nseg) sv = incl - c;
    cnt = __builtin_amdgcn_readlane(incl, nseg - 1);
  }
  if (cnt > cap) cnt = cap;
  const int32_t* cols = indices ? indices + lay.row_offset(bh, jr) : nullptr;
  const KeyList kl = dense_qoff >= 0 ? KeyList::dense(J, QPS, Sk, causal, dense_qoff)
                                     : KeyList::make(J, QPS, Sk, causal, cnt, cols);

  // This lane's query row (rows past Sq compute row J*QPS and store nothing).
  const int64_t qpos = J * QPS + 32 * rb + l32;
  const bool live = qpos < Sq;
  const int64_t qrow = live ? qpos : J * QPS;
  const int64_t qkey = qrow + (dense_qoff > 0 ? dense_qoff : 0);  // last visible diagonal key
  float qv[NS];
  {
    const float4* qr =
        reinterpret_cast<const float4*>(q + b * sqb + h * sqh + qrow * sqs + hh * (D / 2));
#pragma unroll
    for (int c = 0; c < NS / 4; ++c) {
      const float4 x = qr[c];
      qv[4 * c] = x.x;
      qv[4 * c + 1] = x.y;
      qv[4 * c + 2] = x.z;
      qv[4 * c + 3] = x.w;
    }
  }
  const float* kh = k + b * skb + hk * skh;
  const float* vh = v + b * svb + hk * svh;

  // Tiles: the initial, diagonal and column sections, each cut into 32-key
  // tiles (every key of a tile from one section).
  const int64_t n_init = kl.n_init, n_diag = kl.n_diag, n_col = kl.n_col;
  const int64_t t_init = (n_init + kF32Tile - 1) / kF32Tile;
  const int64_t t_diag = (n_diag + kF32Tile - 1) / kF32Tile;
  const int64_t t_col = (n_col + kF32Tile - 1) / kF32Tile;
  const int64_t ntiles = t_init + t_diag + t_col;

  f32x16_t o[OB];
#pragma unroll
  for (int ob = 0; ob < OB; ++ob)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[ob][e] = 0.f;
  float m = -__builtin_inff();  // running maximum of the row (log2 units)
  float lpart = 0.f;            // this lane's share of the row sum

  for (int64_t t = ks; t < ntiles; t += KS) {
    int64_t p0, lim, dkey0 = 0;
    bool diag = false;
    int64_t slot_shift = 0;  // slot - list column of this lane's column
    if (t < t_init) {
      p0 = t * kF32Tile;
      lim = n_init - p0;
    } else if (t < t_init + t_diag) {
      const int64_t d = (t - t_init) * kF32Tile;
      p0 = n_init + d;
      lim = n_diag - d;
      diag = causal != 0;
      dkey0 = kl.diag0 + d;  // key of slot 0 of this diagonal tile
    } else {
      const int64_t c = (t - t_init - t_diag) * kF32Tile;
      p0 = n_init + n_diag + c;
      lim = n_col - c;
      if (nseg > 1) {  // every lane takes part: the search reads other lanes
        const int col = int(c) + l32;
        int sg = 0;
#pragma unroll
        for (int step = 32; step >= 1; step /= 2) {
          const int cand = sg + step;
          const int bound = __shfl(sv, cand < 64 ? cand : 63);
          if (cand < nseg && bound <= col) sg = cand;
        }
        slot_shift = seg_slot(sg) - __shfl(sv, sg);
      }
    }
    if (lim > kF32Tile) lim = kF32Tile;
    // key of slot l32 (row 0 for empty slots and keys outside [0, Sk): read, weighed 0)
    int64_t key = 0;
    if (l32 < lim) {
      const int64_t p = p0 + l32;
      key = p < n_init + n_diag ? kl.key(p) : kl.cols[p - n_init - n_diag + slot_shift];
    }
    if (key < 0 || key >= Sk) key = 0;
    const float4* kr = reinterpret_cast<const float4*>(kh + key * sks + hh * (D / 2));
    float kv[NS];
#pragma unroll
    for (int c = 0; c < NS / 4; ++c) {
      const float4 x = kr[c];
      kv[4 * c] = x.x;
      kv[4 * c + 1] = x.y;
      kv[4 * c + 2] = x.z;
      kv[4 * c + 3] = x.w;
    }
    // keys of the slots this lane holds scores for: slot 8(e/4) + 4hh + e%4
    int32_t ek[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) ek[e] = __shfl(int32_t(key), 8 * (e / 4) + 4 * hh + (e % 4));
    // V^T operands (feature 32ob + l32 of each step's key): loaded here, ahead
    // of the QK^T MFMAs that hide their latency, when the registers allow
    // (D = 64); for D = 128 right before each block's PV MFMAs.
    constexpr bool kVEarly = OB <= 2;
    float vv[kVEarly ? OB : 1][16];
    auto load_v = [&](int ob, float(&dst)[16]) {
#pragma unroll
      for (int e = 0; e < 16; ++e) dst[e] = vh[int64_t(ek[e]) * svs + 32 * ob + l32];
    };
    if constexpr (kVEarly) {
#pragma unroll
      for (int ob = 0; ob < OB; ++ob) load_v(ob, vv[ob]);
    }

    f32x16_t sc;
#pragma unroll
    for (int e = 0; e < 16; ++e) sc[e] = 0.f;
#pragma unroll
    for (int s = 0; s < NS; ++s) sc = mfma_f32(kv[s], qv[s], sc);

    float tmax = -__builtin_inff();
    float sv[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int slot = 8 * (e / 4) + 4 * hh + (e % 4);
      const bool ok = slot < lim && !(diag && dkey0 + slot > qkey);
      sv[e] = ok ? sc[e] * scale_log2 : -__builtin_inff();
      tmax = __builtin_fmaxf(tmax, sv[e]);
    }
    tmax = __builtin_fmaxf(tmax, other_half(tmax));
    const float mnew = __builtin_fmaxf(m, tmax);
    // no key of the row so far: (m, l, O) stay as they are
    const bool any = mnew != -__builtin_inff();
    const float alpha = any ? __builtin_amdgcn_exp2f(m - mnew) : 1.f;
    float pe[16];
#pragma unroll
    for (int e = 0; e < 16; ++e)
      pe[e] = sv[e] != -__builtin_inff() ? __builtin_amdgcn_exp2f(sv[e] - mnew) : 0.f;
    float ps = 0.f;
#pragma unroll
    for (int e = 0; e < 16; ++e) ps += pe[e];
    lpart = lpart * alpha + ps;
    m = mnew;
#pragma unroll
    for (int ob = 0; ob < OB; ++ob) {
      const int vb = kVEarly ? ob : 0;
      if constexpr (!kVEarly) load_v(ob, vv[0]);
#pragma unroll
      for (int e = 0; e < 16; ++e) o[ob][e] *= alpha;
#pragma unroll
      for (int e = 0; e < 16; ++e) o[ob] = mfma_f32(vv[vb][e], pe[e], o[ob]);
    }
  }

  // Merge the key splits into split 0: with M the largest m, the sums and
  // outputs scale by 2^(m_s - M) (a split without keys has m = -inf and
  // weighs 0).
  if constexpr (KS > 1) {
    if (ks > 0) {
      float* st = mst[ks - 1][rb][lane];
      st[0] = m;
      st[1] = lpart;
#pragma unroll
      for (int ob = 0; ob < OB; ++ob)
#pragma unroll
        for (int e = 0; e < 16; ++e) st[2 + 16 * ob + e] = o[ob][e];
    }
    __syncthreads();
    if (ks > 0) return;
    float mm = m;
#pragma unroll
    for (int s2 = 0; s2 < KS - 1; ++s2) mm = __builtin_fmaxf(mm, mst[s2][rb][lane][0]);
    if (mm != -__builtin_inff()) {
      const float a0 = __builtin_amdgcn_exp2f(m - mm);
      lpart *= a0;
#pragma unroll
      for (int ob = 0; ob < OB; ++ob)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[ob][e] *= a0;
#pragma unroll
      for (int s2 = 0; s2 < KS - 1; ++s2) {
        const float* st = mst[s2][rb][lane];
        const float as = __builtin_amdgcn_exp2f(st[0] - mm);
        lpart += st[1] * as;
#pragma unroll
        for (int ob = 0; ob < OB; ++ob)
#pragma unroll
          for (int e = 0; e < 16; ++e) o[ob][e] += st[2 + 16 * ob + e] * as;
      }
    }
  }
  // the row's sum: this lane's keys and the other half's (same row, same m)
  const float l = lpart + other_half(lpart);
  if (!live) return;
  const float inv = l > 0.f ? 1.f / l : 0.f;
  // O^T element e of block ob: feature 32ob + 8(e/4) + 4hh + e%4 of row qpos
  float* orow = out + b * sob + h * soh + qpos * sos;
#pragma unroll
  for (int ob = 0; ob < OB; ++ob)
#pragma unroll
    for (int g = 0; g < 4; ++g)
      *reinterpret_cast<float4*>(orow + 32 * ob + 8 * g + 4 * hh) =
          make_float4(o[ob][4 * g] * inv, o[ob][4 * g + 1] * inv, o[ob][4 * g + 2] * inv,
                      o[ob][4 * g + 3] * inv);
}

bool attn_f32_supported(int64_t D, int64_t qps) {
  return (D == 64 || D == 128) && (qps == 64 || qps == 128);
}

hipError_t launch_attn_f32(const void* q, const int64_t* sq, const void* k, const int64_t* sk,
                           const void* v, const int64_t* sv, void* out, const int64_t* so,
                           int64_t B, int64_t Hq, int64_t Hk, int64_t Sq, int64_t Sk, int64_t D,
                           int64_t qps, int causal, float scale_log2, const int32_t* counts,
                           const int32_t* indices, const RowLayout& lay, int nseg, int segk,
                           int64_t dense_qoff, hipStream_t stream) {
  const int64_t nblocks = lay.nc * B * Hq;
  auto go = [&](auto kernel, int waves) {
    hipLaunchKernelGGL(kernel, dim3(unsigned(nblocks)), dim3(64 * waves), 0, stream,
                       static_cast<const float*>(q), sq[0], sq[1], sq[2],
                       static_cast<const float*>(k), sk[0], sk[1], sk[2],
                       static_cast<const float*>(v), sv[0], sv[1], sv[2],
                       static_cast<float*>(out), so[0], so[1], so[2], B, Hq, Hk, Sq, Sk, causal,
                       scale_log2, counts, indices, lay, nseg, segk, dense_qoff);
    return hipGetLastError();
  };
  constexpr int W = kF32Waves;
  if (D == 64 && qps == 64) return go(attn_f32_kernel<64, 64, W>, W);
  if (D == 64 && qps == 128) return go(attn_f32_kernel<64, 128, W>, W);
  if (D == 128 && qps == 64) return go(attn_f32_kernel<128, 64, W>, W);
  if (D == 128 && qps == 128) return go(attn_f32_kernel<128, 128, W>, W);
  return hipErrorInvalidValue;
}

}  // namespace va
