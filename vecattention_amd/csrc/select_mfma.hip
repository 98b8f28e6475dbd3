// TilingSelect on bf16/fp16 MFMA with certified decisions.
//
// Same rule and output as select_exact.hip (spattn/src/kernels/
// vecattention_kernels.py:206-272 / :275-345): per pooled row, keys visited in
// tiles of BK, a running maximum restarted every G tiles and updated with the
// whole tile's maximum before the compare, key c selected iff
// fp32(s_c + gap) >= m, the truncating causal tile mask, keys past the end
// neither selected nor counted.  The selected sets are bit-identical to the
// canonical rule (sequential fp64 dot products rounded once to fp32).
//
// Scores are computed with v_mfma_f32_32x32x16 (fp32 accumulation).  For a row
// q and key k the MFMA score ŝ satisfies |ŝ - s| <= delta with
//   delta = (2*(D/16 + 2) + 1) * 2^-23 * ||q|| * Kmax
// (Kmax = max key norm of the head; ||q||, Kmax rounded up).  The MFMA term
// 2*(D/16 + 2) * 2^-23 * sum|q_d k_d| is calibrated on gfx950: products are
// exact, the 16 products of one instruction are summed wider than fp32 and the
// result is rounded to nearest-even once per instruction; the worst error
// observed on adversarial inputs (wide exponent spreads, large accumulators,
// cancellation) is 5.2 * 2^-24 * sum|q_d k_d| at D = 128, eight times below
// the term used (tests/test_gpu_mfma_numerics.py re-checks it on the GPU).  The
// extra 2^-23 covers the rounding of the canonical score, and
// sum|q_d k_d| <= ||q|| ||k||.  A decision is taken on the MFMA scores when
// |ŝ + gap - M̂| exceeds a band of 2*delta plus rounding slack; otherwise the
// pair is "ambiguous" and is recomputed exactly: the exact score of the key
// and the exact running maximum, which can only be attained by keys whose
// MFMA score is within 2*delta of the running maximum at their own tile
// ("candidates"; every other key is provably below the maximum).  Across chunk
// boundaries inside a group the running maximum is carried as an exact value.
// All exact work of a chunk is batched over its rows into one parallel pass.
//
// Work-group: 64 pooled rows of one q head (4 waves), keys in chunks of 256.
// Each chunk of K is loaded with coalesced 16-byte loads one chunk ahead (in
// flight while the previous chunk is processed) and stored to LDS in MFMA
// operand order; every K element is read from HBM/L2 once per work-group.
//   A  wave w scores keys [64w, 64w+64) of the chunk against all 64 rows; the
//      scores stay in VGPRs; the K operand rows are permuted so that a lane
//      holds one whole 16-key segment of one row; segment maxima -> LDS.
//   B  per row, prefix of tile maxima with group restarts (4 threads per row,
//      segmented scan) -> M̂ per tile.
//   C  decisions from the VGPR scores -> selected / ambiguous bit masks.
//   D  exact fp64 recomputation for ambiguous pairs and candidate maxima of
//      the rows that need it, as one batch over the work-group.
//   E  per-row exclusive scan of selected counts -> output offsets.
//   G  ordered stores of the selected key ids (ascending).
// Algorithmic work per (row, key): 2*D MFMA FLOPs; K is read once per 64 rows.
#include "mfma.h"

namespace va {

constexpr int kMR = 64;     // pooled rows per work-group
constexpr int kMKC = 256;   // keys per chunk
constexpr int kMSeg = 16;   // 16-key segments per chunk

// MFMA row m of the K operand -> key offset inside the 32-key block, such that
// accumulator element e of lane l holds key 16*(l/32) + e.
__device__ inline int kperm(int m) { return 16 * ((m >> 2) & 1) + 4 * (m >> 3) + (m & 3); }
// Inverse of kperm: key offset k (0..31) -> MFMA row.
__device__ inline int kinv(int k) { return 8 * ((k >> 2) & 3) + 4 * (k >> 4) + (k & 3); }

// Canonical score: sequential fp64 FMAs over d (exact products), one rounding
// to fp32.  All loads are issued before the dependent FMA chain.
template <typename T, int D>
__device__ inline float exact_dot(const T* __restrict__ q, const T* __restrict__ k) {
  uint4 qr[D / 8], kr[D / 8];
#pragma unroll
  for (int c = 0; c < D / 8; ++c) {
    qr[c] = *reinterpret_cast<const uint4*>(q + 8 * c);
    kr[c] = *reinterpret_cast<const uint4*>(k + 8 * c);
  }
  double acc = 0.0;
#pragma unroll
  for (int c = 0; c < D / 8; ++c) {
    const T* qv = reinterpret_cast<const T*>(&qr[c]);
    const T* kv = reinterpret_cast<const T*>(&kr[c]);
#pragma unroll
    for (int e = 0; e < 8; ++e)
      acc = __builtin_fma(double(to_f32(qv[e])), double(to_f32(kv[e])), acc);
  }
  return float(acc);
}

constexpr int kMJobs = 512;  // exact (row, key) jobs per batch

template <typename T, int D>
__global__ __launch_bounds__(256) void select_mfma_kernel(
    const T* __restrict__ qs, int64_t sqb, int64_t sqh, int64_t sqn, const T* __restrict__ k,
    int64_t skb, int64_t skh, int64_t sks, int64_t B, int64_t Hq, int64_t Hk, int64_t Sk,
    int64_t qps, int bk, uint32_t gspan, int causal, int64_t bsq, float gap_scalar,
    const float* __restrict__ gaps, const float* __restrict__ kmax, RowLayout lay,
    int32_t* __restrict__ counts, int32_t* __restrict__ indices, int64_t nrowsets, int segk,
    int nseg) {
  using M = Mfma<T>;
  using vec = typename M::vec;
  constexpr int NS = D / 16;        // MFMA steps over the features
  constexpr int STR = D + 8;        // LDS row stride (elements): 16-byte aligned rows
  constexpr int CPR = D / 8;        // 16-byte chunks per row
  constexpr int KLD = kMKC * CPR / 256;  // K chunks per thread per chunk of keys

  // K chunk, rows stored in MFMA operand order: LDS row 32*blk + m holds key
  // 32*blk + kperm(m), so the operand reads of a wave hit consecutive rows.
  __shared__ __attribute__((aligned(16))) uint16_t Ks[kMKC * STR];
  __shared__ __attribute__((aligned(16))) uint16_t Qs[kMR * STR];   // pooled rows
  __shared__ float tm[kMR][kMSeg + 1];        // segment maxima of MFMA scores
  __shared__ float mh[kMR][kMSeg + 1];        // running maximum at the segment's tile
  __shared__ uint32_t msk[kMR][kMSeg + 1];    // selected (low 16) / ambiguous (high 16)
  __shared__ uint32_t cmk[kMR][kMSeg + 1];    // running-maximum candidates (16 bits)
  __shared__ int32_t off[kMR][kMSeg + 1];     // output offset of the segment's first key
  __shared__ float rband[kMR], rwin[kMR], ecar[kMR];
  __shared__ int32_t rcnt[kMR], rwork[kMR];
  __shared__ uint32_t jobs[kMJobs];           // (row << 8) | key offset in chunk
  __shared__ float exv[kMJobs];               // exact scores of the jobs
  __shared__ int32_t jbeg[kMR], jcnt[kMR];
  __shared__ int32_t njobs, pending;
  __shared__ int32_t klim[kMR];               // causal: keys < klim are allowed
  __shared__ int64_t rowoff[kMR], rowcap[kMR];

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int l32 = lane & 31, hh = lane >> 5;

  const WorkOrder wo{nrowsets * nseg, B, Hq, Hk, causal == 0};
  int64_t item, bh;
  if (!wo.map_item(blockIdx.x, item, bh)) return;  // idle block (uniform)
  // Key segment [seg*segk, (seg+1)*segk) of the split selection (one segment
  // covering every key when nseg == 1); segments are multiples of the group
  // span and of the 256-key chunk, so each starts a group and a chunk.
  const int64_t rs = item / nseg;
  const int seg = int(item % nseg);
  const int64_t seg_lo = nseg > 1 ? int64_t(seg) * segk : 0;
  const int64_t b = bh / Hq, h = bh % Hq, hk = h / (Hq / Hk);
  const int64_t jr0 = rs * kMR;
  const int64_t nc = lay.nc, J0 = lay.J0;
  const int rows_here = int((nc - jr0 < kMR) ? (nc - jr0) : kMR);
  const float gap = gaps ? gaps[bh] : gap_scalar;
  const float kn = kmax[b * Hk + hk];
  const int64_t smin = lay.smin();
  const int lbk = __builtin_ctz(uint32_t(bk));  // bk is a power of two
  const int64_t kstart = seg_lo > smin ? seg_lo : smin;
  int64_t kend = Sk;
  if (causal) {
    const int64_t lim = (J0 + jr0 + rows_here - 1) * qps;
    if (lim < kend) kend = lim;
  }
  if (nseg > 1 && seg_lo + segk < kend) kend = seg_lo + segk;
  const T* qbase = qs + b * sqb + h * sqh;
  const T* kbh = k + b * skb + hk * skh;

  // ---- pooled rows -> LDS; per-row norms, bounds, state ---------------------
  for (int c = tid; c < kMR * CPR; c += 256) {
    const int row = c / CPR, ch = c % CPR;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (row < rows_here) v = *reinterpret_cast<const uint4*>(qbase + (jr0 + row) * sqn + 8 * ch);
    *reinterpret_cast<uint4*>(&Qs[row * STR + 8 * ch]) = v;
  }
  lds_barrier();
  if (tid < kMR) {
    float band = 0.f, win = 0.f;
    if (tid < rows_here) {
      const T* qr = reinterpret_cast<const T*>(&Qs[tid * STR]);
      double ss = 0.0;
      for (int d = 0; d < D; ++d) {
        const double x = double(to_f32(qr[d]));
        ss = __builtin_fma(x, x, ss);
      }
      const double A = __builtin_sqrt(ss) * (1.0 + 0x1p-20) * double(kn) * (1.0 + 0x1p-20);
      const double delta = double(2 * (D / 16 + 2) + 1) * 0x1p-23 * A;
      const double ag = __builtin_fabs(double(gap));
      band = float(1.25 * (2.0 * delta + 6.0 * 0x1p-24 * (A + ag)) + 1e-28);
      win = float(1.25 * (2.0 * delta + 4.0 * 0x1p-24 * A) + 1e-28);
    }
    rband[tid] = band;
    rwin[tid] = win;
    ecar[tid] = -__builtin_inff();
    rcnt[tid] = 0;
    rwork[tid] = 0;
    // The reference's causal tile test r > trunc((k_off - off0) / qps), with
    // r the row inside its BLOCK_SIZE_Q program and off0 = (J - r) * qps, is
    // k_off < J*qps for r >= 1 and k_off <= (J-1)*qps for r == 0 (C++ '/'
    // truncates like Triton's signed division).
    const int64_t jr = jr0 + tid;
    const int64_t J = J0 + jr;
    const int64_t r = jr % bsq;
    int64_t lim = 0x7fffffff;
    if (causal) lim = (r == 0) ? (J - 1) * qps + 1 : J * qps;
    klim[tid] = int32_t(lim < 0 ? 0 : (lim > 0x7fffffff ? 0x7fffffff : lim));
    // the segment's slots of the row (segments never overlap)
    int64_t start = 0, capr = 0;
    if (tid < rows_here) lay.segment_slots(bh, jr, seg, nseg, seg_lo, start, capr);
    rowoff[tid] = start;
    rowcap[tid] = capr;
  }
  // Q^T operands of all 64 rows: row 32*rb + l32, features (D/2)*hh + 8*s.
  vec qop[2][NS];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int s = 0; s < NS; ++s)
      qop[rb][s] = __builtin_bit_cast(
          vec, *reinterpret_cast<const uint4*>(&Qs[(rb * 32 + l32) * STR + (D / 2) * hh + 8 * s]));

  const int nseg_tile = bk / 16;           // segments per tile
  const int ntile = kMKC / bk;             // tiles per chunk (1 .. 16)
  // Tiles per thread in phase B (4 threads per row); with fewer than 4 tiles
  // (bk >= 128) the first ntile threads take one each and the rest idle.
  const int tpt = ntile >= 4 ? ntile / 4 : 1;
  const int last_part = (ntile - 1) / tpt;  // the thread that holds the last tile
  const int64_t kfirst = kstart / kMKC * kMKC;
  // Does the last group of the chunk at kb0 continue into the next chunk?
  // (key offsets < 2^31; 32-bit arithmetic)
  auto cont_chunk = [&](int64_t kb0) {
    return (uint32_t(kb0 + kMKC) % gspan != 0u) && (kb0 + kMKC < kend);
  };
  // Bit t set: tile t of the chunk at kb0 starts a group.
  auto group_starts = [&](int64_t kb0) {
    const uint32_t base = uint32_t(kb0);
    const uint32_t rem = base % gspan;
    uint32_t b0 = rem ? base + (gspan - rem) : base;
    uint32_t m = 0;
    for (; b0 < base + kMKC; b0 += gspan) {
      m |= 1u << ((b0 - base) >> lbk);
      if (b0 + gspan < b0) break;  // no wrap-around
    }
    return m;
  };
  // Coalesced K loads of one chunk: thread t takes 16-byte chunk t + 256*i.
  uint4 kpre[KLD];
  auto load_chunk = [&](int64_t kb0) {
#pragma unroll
    for (int i = 0; i < KLD; ++i) {
      const int c = tid + 256 * i;
      const int64_t key = kb0 + c / CPR;
      kpre[i] = key < Sk ? *reinterpret_cast<const uint4*>(kbh + key * sks + 8 * (c % CPR))
                         : make_uint4(0, 0, 0, 0);
    }
  };
  auto store_chunk = [&]() {
#pragma unroll
    for (int i = 0; i < KLD; ++i) {
      const int c = tid + 256 * i;
      const int kk = c / CPR;                    // key offset in the chunk
      const int lrow = (kk & ~31) | kinv(kk & 31);
      *reinterpret_cast<uint4*>(&Ks[lrow * STR + 8 * (c % CPR)]) = kpre[i];
    }
  };
  if (kfirst < kend) load_chunk(kfirst);

  for (int64_t kbase = kfirst; kbase < kend; kbase += kMKC) {
    lds_barrier();  // previous chunk's readers of Ks are done
    store_chunk();
    lds_barrier();
    if (kbase + kMKC < kend) load_chunk(kbase + kMKC);  // in flight until the next chunk

    // ================= A: MFMA scores, segment maxima =======================
    // wave w: keys [64w, 64w+64) of the chunk, all 64 rows.
    f32x16_t sc[2][2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const int blk = 2 * wave + kb;
      vec kop[NS];
      const uint16_t* kr = &Ks[(blk * 32 + l32) * STR + (D / 2) * hh];
#pragma unroll
      for (int s = 0; s < NS; ++s)
        kop[s] = __builtin_bit_cast(vec, *reinterpret_cast<const uint4*>(kr + 8 * s));
      const int64_t sbase = kbase + blk * 32 + 16 * hh;
      const bool edge = !(kbase + blk * 32 >= kstart && kbase + blk * 32 + 32 <= kend);
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) {
        f32x16_t acc;
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[e] = 0.f;
#pragma unroll
        for (int s = 0; s < NS; ++s) acc = M::run(kop[s], qop[rb][s], acc);
        if (edge) {
#pragma unroll
          for (int e = 0; e < 16; ++e)
            if (sbase + e < kstart || sbase + e >= kend) acc[e] = -__builtin_inff();
        }
        float m = acc[0];
#pragma unroll
        for (int e = 1; e < 16; ++e) m = __builtin_fmaxf(m, acc[e]);
        tm[rb * 32 + l32][blk * 2 + hh] = m;
        sc[rb][kb] = acc;
      }
    }
    lds_barrier();

    // ================= B: running maximum per tile ==========================
    const uint32_t gmask = group_starts(kbase);
    const bool cont = cont_chunk(kbase);
    {
      const int row = tid >> 2, part = tid & 3;
      float lp[4];
      bool lf[4];
      float v = -__builtin_inff();
      bool f = false;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        lp[i] = v;
        lf[i] = f;
        if (i < tpt && part * tpt + i < ntile) {
          const int t = part * tpt + i;
          float tv = -__builtin_inff();
          for (int j = 0; j < nseg_tile; ++j) tv = __builtin_fmaxf(tv, tm[row][t * nseg_tile + j]);
          if ((gmask >> t) & 1u) {
            v = tv;
            f = true;
          } else {
            v = __builtin_fmaxf(v, tv);
          }
          lp[i] = v;
          lf[i] = f;
        }
      }
      // exclusive combine of the aggregates of the row's earlier parts
      const int base_lane = lane & ~3;
      float in_v = ecar[row];
      for (int p = 0; p < 4; ++p) {
        const float pv = __shfl(v, base_lane + p);
        const bool pf = __shfl(int(f), base_lane + p) != 0;
        if (p < part) in_v = pf ? pv : __builtin_fmaxf(in_v, pv);
      }
      float mlast = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (i < tpt && part * tpt + i < ntile) {
          const int t = part * tpt + i;
          const float mt = lf[i] ? lp[i] : __builtin_fmaxf(in_v, lp[i]);
          for (int j = 0; j < nseg_tile; ++j) mh[row][t * nseg_tile + j] = mt;
          mlast = mt;
        }
      }
      // A group continuing into the next chunk needs its maximum carried
      // exactly: flag the row when a tile of that group can hold it.
      if (part == last_part && row < rows_here && cont) {
        const float win = rwin[row];
        for (int t = ntile - 1; t >= 0; --t) {
          float tv = -__builtin_inff();
          for (int j = 0; j < nseg_tile; ++j) tv = __builtin_fmaxf(tv, tm[row][t * nseg_tile + j]);
          if (tv >= mlast - win) { atomicOr(&rwork[row], 2); break; }
          if ((gmask >> t) & 1u) break;
        }
      }
    }
    lds_barrier();

    // ================= C: decisions from the VGPR scores ====================
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      const int row = rb * 32 + l32;
      const int64_t lim = klim[row];
      const float band = rband[row];
      const float win = rwin[row];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const int seg = (2 * wave + kb) * 2 + hh;
        const int64_t sbase = kbase + seg * 16;
        const int64_t koff = sbase & ~int64_t(bk - 1);  // tile start (tiles are bk-aligned)
        uint32_t sel = 0, amb = 0, cand = 0;
        const bool live = row < rows_here && sbase < kend && sbase + 16 > kstart;
        const bool ok = live && koff < lim;
        if (live) {
          const float mrun = mh[row][seg];
          // keys that may hold the exact running maximum of their tile prefix
          // (masked keys hold -inf and are never candidates)
          const float cthr = mrun - win;
#pragma unroll
          for (int e = 0; e < 16; ++e)
            cand |= uint32_t(sc[rb][kb][e] >= cthr && sc[rb][kb][e] > -__builtin_inff()) << e;
          if (ok) {
            const float thr = mrun - gap;
            float mind = __builtin_inff();
#pragma unroll
            for (int e = 0; e < 16; ++e) {
              const float d = sc[rb][kb][e] - thr;
              sel |= uint32_t(d > band) << e;
              mind = __builtin_fminf(mind, __builtin_fabsf(d));
            }
            if (mind <= band) {
#pragma unroll
              for (int e = 0; e < 16; ++e) {
                const float d = sc[rb][kb][e] - thr;
                amb |= uint32_t(__builtin_fabsf(d) <= band) << e;
              }
              sel &= ~amb;
              atomicOr(&rwork[row], 1);
            }
          }
        }
        cmk[row][seg] = cand;
        msk[row][seg] = sel | (amb << 16);
      }
    }
    lds_barrier();

    // ================= D: exact resolution (rare) ===========================
    // Rows flagged in B (carried maximum) or C (ambiguous pairs) enqueue their
    // candidate and ambiguous keys; the whole work-group computes the exact
    // scores from the LDS copies of K and Q; each row then resolves its
    // decisions and carried maximum.
    if (tid == 0) pending = 0;
    lds_barrier();
    if (tid < kMR && tid < rows_here && rwork[tid] != 0) atomicAdd(&pending, 1);
    lds_barrier();
    while (pending > 0) {
      if (tid == 0) njobs = 0;
      lds_barrier();
      // D1: enqueue.  Wave 0 (one lane per row) scans the rows' job counts;
      // the rows whose jobs fit are served this round, each in a contiguous
      // slot range, so slots [0, njobs) are all written.
      if (tid < kMR) {
        int n = 0;
        const bool work = tid < rows_here && rwork[tid] != 0;
        if (work)
          for (int seg = 0; seg < kMSeg; ++seg)
            n += __builtin_popcount((msk[tid][seg] >> 16) | cmk[tid][seg]);
        int incl = n;
        for (int o = 1; o < 64; o <<= 1) {
          const int y = __shfl_up(incl, o);
          if (lane >= o) incl += y;
        }
        const bool served = work && incl <= kMJobs;
        jbeg[tid] = incl - n;
        jcnt[tid] = served ? n : -1;
        if (served) {
          atomicMax(&njobs, incl);
          int w = incl - n;
          for (int seg = 0; seg < kMSeg; ++seg) {
            uint32_t bits = (msk[tid][seg] >> 16) | cmk[tid][seg];
            while (bits) {
              const int e = __builtin_ctz(bits);
              bits &= bits - 1;
              jobs[w++] = (uint32_t(tid) << 8) | uint32_t(seg * 16 + e);
            }
          }
        }
      }
      lds_barrier();
      // D2: exact scores, all threads, operands from LDS
      const int nj = njobs;
      for (int j = tid; j < nj; j += 256) {
        const int row = int(jobs[j] >> 8), kk = int(jobs[j] & 255u);
        const int64_t key = kbase + kk;
        const int lrow = (kk & ~31) | kinv(kk & 31);
        exv[j] = (row < rows_here && key >= kstart && key < kend)
                     ? exact_dot<T, D>(reinterpret_cast<const T*>(&Qs[row * STR]),
                                       reinterpret_cast<const T*>(&Ks[lrow * STR]))
                     : -__builtin_inff();
      }
      lds_barrier();
      // D3: per row resolution
      if (tid < kMR && jcnt[tid] >= 0) {
        const int row = tid;
        const int jb = jbeg[row], jn = jcnt[row];
        const bool first_open = (gmask & 1u) == 0;  // group began in an earlier chunk
        const float e_in = ecar[row];
        auto group_start_tile = [&](int t) {  // highest group start <= t, else 0
          const uint32_t m = gmask & ((2u << t) - 1u);
          return m ? 31 - __builtin_clz(m) : 0;
        };
        // running maximum of tiles [g0, t] from exact candidate scores
        auto exact_max = [&](int g0, int t) {
          float m = (g0 == 0 && first_open) ? e_in : -__builtin_inff();
          for (int j = jb; j < jb + jn; ++j) {
            const int kk = int(jobs[j] & 255u);
            const int seg = kk >> 4, e = kk & 15;
            const int tt = kk >> lbk;
            if (tt >= g0 && tt <= t && ((cmk[row][seg] >> e) & 1u)) m = __builtin_fmaxf(m, exv[j]);
          }
          return m;
        };
        for (int t = 0; t < ntile; ++t) {
          uint32_t any = 0;
          for (int jj = 0; jj < nseg_tile; ++jj) any |= msk[row][t * nseg_tile + jj] >> 16;
          if (!any) continue;
          const float mt = exact_max(group_start_tile(t), t);
          for (int j = jb; j < jb + jn; ++j) {
            const int kk = int(jobs[j] & 255u);
            if ((kk >> lbk) != t) continue;
            const int seg = kk >> 4, e = kk & 15;
            const uint32_t w = msk[row][seg];
            if ((w >> (16 + e)) & 1u) {
              const uint32_t take = uint32_t((exv[j] + gap) >= mt);
              msk[row][seg] = (w & ~(1u << (16 + e))) | (take << e);
            }
          }
        }
        if (cont) ecar[row] = exact_max(group_start_tile(ntile - 1), ntile - 1);
        rwork[row] = 0;
      }
      lds_barrier();
      if (tid == 0) {
        int left = 0;
        for (int r = 0; r < rows_here; ++r) left += rwork[r] != 0;
        pending = left;
      }
      lds_barrier();
    }
    // A group that does not continue hands no maximum to the next chunk.
    if (tid < kMR && !cont) ecar[tid] = -__builtin_inff();
    lds_barrier();

    // ================= E: output offsets per segment ========================
    {
      const int row = tid >> 2, part = tid & 3;
      int c4[4];
      int tot = 0;
      for (int i = 0; i < 4; ++i) {
        c4[i] = __builtin_popcount(msk[row][part * 4 + i] & 0xffffu);
        tot += c4[i];
      }
      const int base_lane = lane & ~3;
      int before = 0, all = 0;
      for (int p = 0; p < 4; ++p) {
        const int pt = __shfl(tot, base_lane + p);
        if (p < part) before += pt;
        all += pt;
      }
      const int rc = rcnt[row];
      int o = rc + before;
      for (int i = 0; i < 4; ++i) {
        off[row][part * 4 + i] = o;
        o += c4[i];
      }
      if (part == 3) rcnt[row] = rc + all;
    }
    lds_barrier();

    // ================= G: ordered stores (none when only counting) ===========
#pragma unroll
    for (int rb = 0; rb < 2 && indices; ++rb) {
      const int row = rb * 32 + l32;
      if (row < rows_here) {
        const int64_t row_off = rowoff[row];
        const int64_t cap = rowcap[row];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          const int seg = (2 * wave + kb) * 2 + hh;
          uint32_t bits = msk[row][seg] & 0xffffu;
          int64_t pos = off[row][seg];
          const int64_t sbase = kbase + seg * 16;
          while (bits) {
            const int e = __builtin_ctz(bits);
            bits &= bits - 1;
            if (pos < cap) indices[row_off + pos] = int32_t(sbase + e);
            ++pos;
          }
        }
      }
    }
  }
  lds_barrier();
  if (tid < rows_here && counts) {
    const int64_t cap = rowcap[tid];
    const int32_t c = rcnt[tid];
    counts[(bh * nc + jr0 + tid) * nseg + seg] = (c < cap) ? c : int32_t(cap);
  }
}

// Key segments of this kernel's split selection: whole 256-key chunks that
// each start a group, i.e. a multiple of lcm(256, group span), about Sk / 16
// keys within [2048, 4096] and at most 64 segments (the wave kernel's rule);
// 0 when one group covers a row (this kernel has no carry pass) or nothing is
// left to split.  Groups shorter than 64 keys (the reference models' default
// group_k_block of 1 with k_local_size 16) run on this kernel, and unsplit
// their long causal rows each take one work-group through every key.
int64_t select_mfma_segment_keys(int64_t Sk, int64_t bk, int64_t group) {
  constexpr int64_t kMaxSeg = 64, kChunk = 256;
  const int64_t gs = bk * group;
  if (gs <= 0 || gs >= Sk) return 0;
  int64_t a = kChunk, b = gs;  // lcm(kChunk, gs)
  while (b) {
    const int64_t t = a % b;
    a = b;
    b = t;
  }
  const int64_t unit = kChunk / a * gs;
  const int64_t target = Sk / 16 < 2048 ? 2048 : (Sk / 16 > 4096 ? 4096 : Sk / 16);
  int64_t want = (Sk + kMaxSeg - 1) / kMaxSeg;
  if (want < target) want = target;
  const int64_t segk = (want + unit - 1) / unit * unit;
  return segk < Sk ? segk : 0;
}

bool select_mfma_supported(int dtype, int64_t D, int64_t bk) {
  return (dtype == kBF16 || dtype == kF16) && (D == 64 || D == 128) &&
         (bk == 16 || bk == 32 || bk == 64 || bk == 128 || bk == 256);
}

template <typename T, int D>
static hipError_t launch_select_mfma_td(const void* qs, int64_t sqb, int64_t sqh, int64_t sqn,
                                        const void* k, int64_t skb, int64_t skh, int64_t sks,
                                        int64_t B, int64_t Hq, int64_t Hk, int64_t Sk, int64_t qps,
                                        int64_t bk, int64_t group, int causal, int64_t bsq,
                                        float gap, const float* gaps, const float* kmax,
                                        const RowLayout& lay, int32_t* counts, int32_t* indices,
                                        int64_t segk, hipStream_t stream) {
  const int64_t nrowsets = (lay.nc + kMR - 1) / kMR;
  const int64_t nseg = segk > 0 ? (Sk + segk - 1) / segk : 1;
  // Group span in keys, capped at 2^31 (key offsets are below 2^31, so a span
  // that large has its only boundary at 0 either way).
  const int64_t gs = (group > (int64_t(1) << 31) / bk) ? (int64_t(1) << 31) : bk * group;
  const uint32_t gspan32 = uint32_t(gs);
  const int64_t nblocks = WorkOrder{nrowsets * nseg, B, Hq, Hk, causal == 0}.grid_items();
  hipLaunchKernelGGL((select_mfma_kernel<T, D>), dim3(unsigned(nblocks)), dim3(256), 0,
                     stream, static_cast<const T*>(qs), sqb, sqh, sqn, static_cast<const T*>(k),
                     skb, skh, sks, B, Hq, Hk, Sk, qps, int(bk), gspan32, causal, bsq, gap, gaps,
                     kmax, lay, counts, indices, nrowsets, int(segk), int(nseg));
  return hipGetLastError();
}

hipError_t launch_select_mfma(int dtype, const void* qs, int64_t sqb, int64_t sqh, int64_t sqn,
                              const void* k, int64_t skb, int64_t skh, int64_t sks, int64_t B,
                              int64_t Hq, int64_t Hk, int64_t Sk, int64_t D, int64_t qps,
                              int64_t bk, int64_t group, int causal, int64_t bsq, float gap,
                              const float* gaps, const float* kmax, const RowLayout& lay,
                              int32_t* counts, int32_t* indices, int64_t segk,
                              hipStream_t stream) {
#define VA_SEL_CASE(TT, DD)                                                                     \
  return launch_select_mfma_td<TT, DD>(qs, sqb, sqh, sqn, k, skb, skh, sks, B, Hq, Hk, Sk, qps, \
                                       bk, group, causal, bsq, gap, gaps, kmax, lay, counts,    \
                                       indices, segk, stream);
  if (dtype == kBF16 && D == 128) { VA_SEL_CASE(bf16_t, 128) }
  if (dtype == kBF16 && D == 64) { VA_SEL_CASE(bf16_t, 64) }
  if (dtype == kF16 && D == 128) { VA_SEL_CASE(f16_t, 128) }
  if (dtype == kF16 && D == 64) { VA_SEL_CASE(f16_t, 64) }
#undef VA_SEL_CASE
  return hipErrorInvalidValue;
}

}  // namespace va
