// TilingSelect — important-vertical-vector selection, exact-arithmetic kernel.
//
// Restates the program body of spattn/src/kernels/vecattention_kernels.py:206-272
// (and the per-head-gap twin :275-345) for one work-group per (b, q head,
// set of R pooled rows):
//   * keys are visited in tiles of `bk` in ascending order; a group of `group`
//     tiles restarts the running maximum (:227,231-233,252);
//   * with wo_init the first qps keys are skipped (:231);
//   * the running maximum takes the whole tile's maximum BEFORE the compare
//     (:257), and key c is selected iff fp32(s_c + gap) >= m (:258);
//   * the causal tile mask is  r > trunc((k_off - off0) / qps)  with Triton's
//     truncating signed division (:238,259-260), which rejects the tiles in
//     (off0 - qps, off0) for the first row of every BLOCK_SIZE_Q program;
//   * keys past the end are never selected and never move the maximum (the
//     reference pads them with NaN, :117-127, and tl.max ignores NaN).
// Output rows are written in ascending key order (the reference appends tile
// runs in atomic order; the set is the same).
//
// Scores are canonical: a sequential fp64 sum over d of exact products
// (bf16*bf16, fp16*fp16 and fp32*fp32 products are exact in fp64), rounded
// once to fp32.  This makes every decision bit-identical to the CPU oracle.
// Its scoring loop (R*D fp64 FMAs per key per work-group) is bound by the LDS
// broadcast reads of the fp64 query values that feed those FMAs.
#include "common.h"

namespace va {

constexpr int kSelChunk = 256;   // keys per inner chunk (== blockDim.x)
constexpr int kSelMaxD = 256;

// kSelRows: pooled rows per work-group (16, 8, 4, 2 or 1: the host takes the
// most rows that still give at least 256 work-groups (1024 with key
// segments), since each work-group walks every key of its rows; small grids
// take one row per work-group).
// Key segments (nseg > 1): work-group (row set, segment) walks the keys
// [seg*segk, (seg+1)*segk) only and writes its keys from its own first slot
// of the row and its count to counts[(bh*nc + jr)*nseg + seg].  One pass when
// segments are multiples of the group span (each starts a group).
// Two passes when one group spans the row (segments then do not start
// groups): the maxima pass (mode kPassMax) stores each (row, segment)'s
// exact running maximum at the segment's end, carry[(bh*nc + jr)*nseg + seg],
// and selects nothing; the carry pass (kPassCarry) starts segment s from the
// maximum of the carried values of segments 0 .. s-1 (with one group per row
// the running maximum before the segment is exactly that), then selects as
// the one-pass form does.
template <typename T, int kSelRows, int kD>
__global__ __launch_bounds__(256) void select_exact_kernel(
    const T* __restrict__ qs, int64_t sqb, int64_t sqh, int64_t sqn, const T* __restrict__ k,
    int64_t skb, int64_t skh, int64_t sks, int64_t B, int64_t Hq, int64_t Hk,
    int64_t Sk, int64_t D, int64_t qps, int64_t bk, int64_t group, int causal,
    int64_t bsq, float gap_scalar, const float* __restrict__ gaps, RowLayout lay,
    int32_t* __restrict__ counts, int32_t* __restrict__ indices, int64_t nrowsets,
    int64_t segk, int nseg, float* __restrict__ carry, int mode) {
  __shared__ double qd[kSelMaxD * kSelRows];          // [d][row]
  __shared__ float sc[kSelRows * kSelChunk];          // [row][key]
  __shared__ float mt[kSelRows * (kSelChunk / 16)];   // [row][tile] running max
  __shared__ float m_run[kSelRows];
  __shared__ int32_t cnt[kSelRows];
  __shared__ int64_t klim[kSelRows];  // causal: keys < klim are allowed

  const int tid = threadIdx.x;
  const int64_t BH = B * Hq;
  const int64_t item = int64_t(blockIdx.x) / BH;
  const int64_t rs = nrowsets - 1 - item / nseg;  // heavy rows first
  const int seg = int(item % nseg);
  const int64_t seg_lo = nseg > 1 ? int64_t(seg) * segk : 0;
  const int64_t bh = int64_t(blockIdx.x) % BH;
  const int64_t b = bh / Hq, h = bh % Hq;
  const int64_t hk = h / (Hq / Hk);
  const int64_t jr0 = rs * kSelRows;
  const int64_t nc = lay.nc, J0 = lay.J0;
  const int64_t rows_here = (nc - jr0 < kSelRows) ? (nc - jr0) : kSelRows;
  const float gap = gaps ? gaps[bh] : gap_scalar;
  const int64_t smin = lay.smin();
  const int64_t gspan = bk * group;
  const int ntile = int(kSelChunk / bk);
  const int lbk = __builtin_ctzll(uint64_t(bk));  // bk is a power of two

  // Key range of this work-group: [kstart, kend).
  const int64_t kstart = seg_lo > smin ? seg_lo : smin;
  int64_t kend = Sk;
  if (causal) {
    const int64_t lim = (J0 + jr0 + rows_here - 1) * qps;  // keys < J*qps only
    if (lim < kend) kend = lim;
  }
  if (nseg > 1 && seg_lo + segk < kend) kend = seg_lo + segk;

  // Stage the R pooled rows in fp64, transposed for broadcast reads.
  for (int64_t e = tid; e < int64_t(kSelRows) * D; e += blockDim.x) {
    const int64_t i = e / D, d = e % D;
    double v = 0.0;
    if (i < rows_here) v = double(to_f32(qs[b * sqb + h * sqh + (jr0 + i) * sqn + d]));
    qd[d * kSelRows + i] = v;
  }
  if (tid < kSelRows) {
    float m0 = -__builtin_inff();
    if (mode == kPassCarry && tid < rows_here)
      for (int s2 = 0; s2 < seg; ++s2)
        m0 = __builtin_fmaxf(m0, carry[(bh * nc + jr0 + tid) * nseg + s2]);
    m_run[tid] = m0;
    cnt[tid] = 0;
    // The reference's causal tile test r > trunc((k_off - off0) / qps), with r
    // the row inside its BLOCK_SIZE_Q program and off0 = (J - r) * qps, is
    // k_off < J*qps for r >= 1 and k_off <= (J-1)*qps for r == 0.
    const int64_t jr = jr0 + tid;
    const int64_t r = jr % bsq;
    const int64_t J = J0 + jr;
    klim[tid] = causal ? ((r == 0) ? (J - 1) * qps + 1 : J * qps) : INT64_MAX;
  }
  __syncthreads();

  const T* kh = k + b * skb + hk * skh;
  constexpr int VEC = int(16 / sizeof(T));
  const bool vec_ok = (D % VEC == 0) && (reinterpret_cast<uintptr_t>(kh) % 16 == 0) &&
                      (sks % VEC == 0);
  // kD: the head dim as a compile-time constant (64 or 128; 0: runtime), so
  // that the scoring loop unrolls and its LDS reads are issued ahead of use.
  const int64_t Dk = kD ? int64_t(kD) : D;

  for (int64_t kbase = kstart; kbase < kend; kbase += kSelChunk) {
    // ---- Phase A: canonical scores for R rows x 256 keys -----------------
    bool scored = false;
    if constexpr (kD > 0 && kSelRows >= 16) {
      if (vec_ok) {
        // Two keys per thread (kk and kk + 128) for half of the rows (threads
        // [0, 128): rows [0, R/2), the others rows [R/2, R)): every fp64 query
        // value read from LDS feeds two FMAs.  With a key per thread the
        // scoring loop is bound by these broadcast LDS reads (one per FMA) at
        // 16 rows (pairs: 20-40% faster); at 8 and 4 rows the second read of
        // each K row costs more than the LDS reads it saves (15-65% slower).
        constexpr int RH = kSelRows / 2;
        const int half = tid / (kSelChunk / 2), kk = tid % (kSelChunk / 2);
        const int64_t key0 = kbase + kk, key1 = key0 + kSelChunk / 2;
        // keys past the range score a valid row (the first one of the range):
        // their scores are written as 0 and never read
        const T* kr0 = kh + (key0 < kend ? key0 : kstart) * sks;
        const T* kr1 = kh + (key1 < kend ? key1 : kstart) * sks;
        double a0[RH], a1[RH];
#pragma unroll
        for (int i = 0; i < RH; ++i) a0[i] = a1[i] = 0.0;
#pragma unroll
        for (int d0 = 0; d0 < kD; d0 += VEC) {
          T v0[VEC], v1[VEC];
          *reinterpret_cast<uint4*>(v0) = *reinterpret_cast<const uint4*>(kr0 + d0);
          *reinterpret_cast<uint4*>(v1) = *reinterpret_cast<const uint4*>(kr1 + d0);
#pragma unroll
          for (int e = 0; e < VEC; ++e) {
            const double kd0 = double(to_f32(v0[e])), kd1 = double(to_f32(v1[e]));
            const double* qrow = &qd[(d0 + e) * kSelRows + half * RH];
#pragma unroll
            for (int i = 0; i < RH; ++i) {
              const double qv = qrow[i];
              a0[i] = __builtin_fma(qv, kd0, a0[i]);
              a1[i] = __builtin_fma(qv, kd1, a1[i]);
            }
          }
        }
#pragma unroll
        for (int i = 0; i < RH; ++i) {
          sc[(half * RH + i) * kSelChunk + kk] = key0 < kend ? float(a0[i]) : 0.f;
          sc[(half * RH + i) * kSelChunk + kk + kSelChunk / 2] = key1 < kend ? float(a1[i]) : 0.f;
        }
        scored = true;
      }
    }
    if (!scored) {
      const int64_t key = kbase + tid;
      double acc[kSelRows];
#pragma unroll
      for (int i = 0; i < kSelRows; ++i) acc[i] = 0.0;
      if (key < kend) {
        const T* kr = kh + key * sks;
        if (vec_ok) {
#pragma unroll
          for (int64_t d0 = 0; d0 < Dk; d0 += VEC) {
            T v[VEC];
            *reinterpret_cast<uint4*>(v) = *reinterpret_cast<const uint4*>(kr + d0);
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
              const double kd = double(to_f32(v[e]));
              const double* qrow = &qd[(d0 + e) * kSelRows];
#pragma unroll
              for (int i = 0; i < kSelRows; ++i) acc[i] = __builtin_fma(qrow[i], kd, acc[i]);
            }
          }
        } else {
          for (int64_t d = 0; d < D; ++d) {
            const double kd = double(to_f32(kr[d]));
            const double* qrow = &qd[d * kSelRows];
#pragma unroll
            for (int i = 0; i < kSelRows; ++i) acc[i] = __builtin_fma(qrow[i], kd, acc[i]);
          }
        }
      }
#pragma unroll
      for (int i = 0; i < kSelRows; ++i) sc[i * kSelChunk + tid] = float(acc[i]);
    }
    __syncthreads();

    // ---- Phase B1: tile maxima over the valid keys of each tile ------------
    if (tid < kSelRows * ntile) {
      const int i = tid / ntile, tl = tid % ntile;
      const int64_t koff = kbase + int64_t(tl) * bk;
      float tmax = -__builtin_inff();
      for (int64_t c = 0; c < bk; ++c) {
        if (koff + c < kend) tmax = __builtin_fmaxf(tmax, sc[i * kSelChunk + tl * bk + c]);
      }
      mt[i * (kSelChunk / 16) + tl] = tmax;
    }
    __syncthreads();

    // ---- Phase B2: running maximum, restarted at every group start ---------
    if (tid < kSelRows) {
      float m = m_run[tid];
      int64_t next_g = kbase + (gspan - kbase % gspan) % gspan;  // first group start >= kbase
      for (int tl = 0; tl < ntile; ++tl) {
        const int64_t koff = kbase + int64_t(tl) * bk;
        if (koff >= kend) break;
        if (koff == next_g) {
          m = -__builtin_inff();
          next_g += gspan;
        }
        m = __builtin_fmaxf(m, mt[tid * (kSelChunk / 16) + tl]);
        mt[tid * (kSelChunk / 16) + tl] = m;
      }
      m_run[tid] = m;
    }
    __syncthreads();

    // ---- Phase B3: decisions and ordered compaction, one wave per row ------
    if (mode != kPassMax) {
      const int wave = tid / 64, lane = tid % 64;
      for (int i = wave; i < rows_here; i += int(blockDim.x / 64)) {
        const int64_t jr = jr0 + i;
        const int64_t J = J0 + jr;
        const int64_t lim = klim[i];
        int64_t row_off, cap;
        lay.segment_slots(bh, jr, seg, nseg, seg_lo, row_off, cap);
        int32_t c = cnt[i];
        for (int step = 0; step < kSelChunk / 64; ++step) {
          const int kk = step * 64 + lane;
          const int64_t key = kbase + kk;
          const int tl = kk >> lbk;
          const int64_t koff = kbase + (int64_t(tl) << lbk);
          bool sel = key < kend && koff < lim;
          if (sel) sel = (sc[i * kSelChunk + kk] + gap) >= mt[i * (kSelChunk / 16) + tl];
          const uint64_t ballot = __ballot(sel);
          const uint32_t below = __builtin_amdgcn_mbcnt_hi(
              uint32_t(ballot >> 32), __builtin_amdgcn_mbcnt_lo(uint32_t(ballot), 0u));
          const int64_t pos = int64_t(c) + below;
          if (sel && pos < cap && indices) indices[row_off + pos] = int32_t(key);
          c += __builtin_popcountll(ballot);
        }
        if (lane == 0) cnt[i] = c;
      }
    }
    __syncthreads();
  }

  if (mode == kPassMax) {
    if (tid < rows_here) carry[(bh * nc + jr0 + tid) * nseg + seg] = m_run[tid];
    return;
  }
  if (tid < rows_here && counts) {
    int64_t start, cap;
    lay.segment_slots(bh, jr0 + tid, seg, nseg, seg_lo, start, cap);
    const int32_t c = cnt[tid];
    counts[(bh * nc + jr0 + tid) * nseg + seg] = (c < cap) ? c : int32_t(cap);
  }
}

template <typename T>
static hipError_t launch_select_exact_t(
    const void* qs, int64_t sqb, int64_t sqh, int64_t sqn, const void* k, int64_t skb, int64_t skh,
    int64_t sks, int64_t B, int64_t Hq, int64_t Hk, int64_t Sk, int64_t D,
    int64_t qps, int64_t bk, int64_t group, int causal, int64_t bsq,
    float gap_scalar, const float* gaps, const RowLayout& lay, int32_t* counts,
    int32_t* indices, int64_t segk, float* carry, int mode, hipStream_t stream) {
  const int64_t nseg = segk > 0 ? (Sk + segk - 1) / segk : 1;
  auto launch = [&](auto rows_tag) {
    constexpr int R = decltype(rows_tag)::value;
    const int64_t nrowsets = (lay.nc + R - 1) / R;
    const int64_t nblocks = nrowsets * nseg * B * Hq;
    auto go = [&](auto kernel) {
      hipLaunchKernelGGL(kernel, dim3(unsigned(nblocks)), dim3(kSelChunk), 0, stream,
                         static_cast<const T*>(qs), sqb, sqh, sqn, static_cast<const T*>(k), skb,
                         skh, sks, B, Hq, Hk, Sk, D, qps, bk, group, causal, bsq, gap_scalar,
                         gaps, lay, counts, indices, nrowsets, segk > 0 ? segk : Sk, int(nseg),
                         carry, mode);
    };
    if (D == 128)
      go(select_exact_kernel<T, R, 128>);
    else if (D == 64)
      go(select_exact_kernel<T, R, 64>);
    else
      go(select_exact_kernel<T, R, 0>);
    return hipGetLastError();
  };
  // Work-groups wanted: 256 for whole rows (more rows per work-group share
  // each K load: 1-row work-groups made the tuner's 8192-row chunks 15-50%
  // slower), 1024 for key segments, whose work-groups each score one or a
  // few 256-key chunks and are bound by latency (A: 27.5 -> 18.9 us).
  const int64_t kMinGroups = nseg > 1 ? 1024 : 256;
  const int64_t items = nseg * B * Hq;  // work-groups per row set
  if ((lay.nc + 15) / 16 * items >= kMinGroups) return launch(std::integral_constant<int, 16>{});
  if ((lay.nc + 7) / 8 * items >= kMinGroups) return launch(std::integral_constant<int, 8>{});
  if ((lay.nc + 3) / 4 * items >= kMinGroups) return launch(std::integral_constant<int, 4>{});
  if ((lay.nc + 1) / 2 * items >= kMinGroups) return launch(std::integral_constant<int, 2>{});
  return launch(std::integral_constant<int, 1>{});
}

// Key segments of the exact kernel's split: at least Sk / 64 keys (at most
// 64 segments) and otherwise as short as one 256-key chunk, so that a
// work-group scores its rows' keys in one or a few chunks instead of walking
// the row, and row sets take 16 rows each sooner (more rows per K load).
// Multiples of 256 keys and of the group span (each segment starts a group:
// one pass), or, when one group spans the row, any whole chunks (maxima pass,
// then carry pass).  0 when nothing is split.
int64_t select_exact_segment_keys(int64_t Sk, int64_t bk, int64_t group) {
  constexpr int64_t kMaxSeg = 64;
  const int64_t gs = bk * group;
  if (gs <= 0) return 0;
  int64_t a = kSelChunk, b = gs < Sk ? gs : kSelChunk;  // lcm(kSelChunk, gs) for short groups
  while (b) {
    const int64_t t = a % b;
    a = b;
    b = t;
  }
  const int64_t unit = gs < Sk ? kSelChunk / a * gs : kSelChunk;
  const int64_t want = (Sk + kMaxSeg - 1) / kMaxSeg;
  const int64_t segk = (want + unit - 1) / unit * unit;
  return segk < Sk ? segk : 0;
}

hipError_t launch_select_exact(int dtype, const void* qs, int64_t sqb, int64_t sqh,
                               int64_t sqn, const void* k, int64_t skb, int64_t skh, int64_t sks,
                               int64_t B, int64_t Hq, int64_t Hk, int64_t Sk, int64_t D,
                               int64_t qps, int64_t bk, int64_t group, int causal,
                               int64_t bsq, float gap_scalar, const float* gaps,
                               const RowLayout& lay, int32_t* counts, int32_t* indices,
                               int64_t segk, float* carry, int mode, hipStream_t stream) {
  switch (dtype) {
    case kF32:
      return launch_select_exact_t<float>(qs, sqb, sqh, sqn, k, skb, skh, sks, B, Hq, Hk, Sk, D, qps, bk,
                                          group, causal, bsq, gap_scalar, gaps, lay, counts,
                                          indices, segk, carry, mode, stream);
    case kBF16:
      return launch_select_exact_t<bf16_t>(qs, sqb, sqh, sqn, k, skb, skh, sks, B, Hq, Hk, Sk, D, qps,
                                           bk, group, causal, bsq, gap_scalar, gaps, lay, counts,
                                           indices, segk, carry, mode, stream);
    case kF16:
      return launch_select_exact_t<f16_t>(qs, sqb, sqh, sqn, k, skb, skh, sks, B, Hq, Hk, Sk, D, qps, bk,
                                          group, causal, bsq, gap_scalar, gaps, lay, counts,
                                          indices, segk, carry, mode, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace va
