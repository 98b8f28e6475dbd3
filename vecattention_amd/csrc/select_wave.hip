// TilingSelect on bf16/fp16 MFMA, one wave per 32 pooled rows, certified
// decisions.
//
// Same rule and output as select_exact.hip (spattn/src/kernels/
// vecattention_kernels.py:206-272 / :275-345): per pooled row, keys visited in
// tiles of BK, a running maximum restarted every G tiles and updated with the
// whole tile's maximum before the compare, key c selected iff
// fp32(s_c + gap) >= m, the truncating causal tile mask, keys past the end
// neither selected nor counted.  The selected sets are bit-identical to the
// canonical rule (sequential fp64 dot products rounded once to fp32).
//
// Organisation.  A work-group holds 4 waves and 128 consecutive pooled rows of
// one q head; wave w owns rows [32w, 32w+32).  The keys are walked in chunks
// of 64 (two 32-key blocks); each chunk of K is copied into LDS once for the
// work-group (buffer_load ... lds, two stages, the next chunk in flight while
// the current one is scored) and read by all four waves.  Within a wave the
// keys are visited in order, so each row's running maximum is a register:
// there is no cross-wave exchange at all.
//
// Scores.  S^T = K Q^T with v_mfma_f32_32x32x16: A = 32 key rows from LDS,
// B = the wave's 32 pooled rows held in VGPRs for the whole kernel.  The key
// rows of a block are stored in LDS permuted (row m holds key kperm(m)) so
// that the accumulator of lane l holds row l % 32 and the 16 consecutive keys
// 16 * (l / 32) + e: for BK = 16 a lane holds exactly one tile.
//
// Certified decisions.  For a row q and key k the MFMA score s^ satisfies
// |s^ - s| <= delta with delta = (2*(D/16 + 2) + 1) * 2^-23 * ||q|| * Kmax
// (see select_mfma.hip for the derivation and the calibration on gfx950).
// A key is selected outright when s^ exceeds m^ - gap by more than a band of
// 2*delta plus rounding slack, rejected when it is below by more, and is
// "ambiguous" otherwise.  The exact decision needs the exact score (fp64
// recomputation) and the exact running maximum M.  M can only be attained by
// keys whose s^ is within `win` (>= 2*delta) of m^ at their own tile, so each
// row keeps a short list of the tiles that contained such keys ("near-max
// tiles"); when a row meets an ambiguous key, the exact scores of its listed
// tiles are computed once and folded into an exact running maximum for the
// rest of the group, and the list is cleared.  Everything exact runs on the
// rare path of the wave that needs it.
//
// Groups shorter than a chunk.  A group span of 16 or 32 keys (k_local_size
// 16 or 32 with group_k_block 1 or 2) divides the 64-key chunk: every chunk
// starts a group and the running maximum also restarts at the group starts
// inside the chunk.  A row's exact maximum at a key then depends only on the
// key's own group, which lies in the chunk, so nothing is listed: the rare
// path takes, for each ambiguous key, the tiles of its group up to its own.
//
// Output.  Each lane writes its selected keys straight to the row's index
// list (ascending: the low half's tile before the high half's).
#include "lanes.h"
#include "mfma.h"

namespace va {

constexpr int kWRows = 32;         // pooled rows per wave
constexpr int kWWaves = 4;         // waves per work-group
constexpr int kWChunk = 64;        // keys per chunk
constexpr int kWList = 16;         // near-max tiles per row
constexpr int kCarryTiles = 4;     // near-max tiles a segment passes on

// What the maxima pass records per (row, segment) of a two-pass selection:
// the segment's MFMA maximum, the exact maximum of the tiles it folded (on
// list overflow), and its remaining near-max tiles (tile maximum within `win`
// of the segment maximum; the only tiles that can hold the exact maximum),
// whose exact scores are left to the carry pass's rare path.
struct SegCarry {
  float m, ex;
  int32_t n, pad;
  int32_t tile[kCarryTiles];
};
static_assert(sizeof(SegCarry) == 32, "the host sizes carry buffers at 32 bytes per record");


// MFMA row m of the K operand -> key offset inside the 32-key block, such that
// accumulator element e of lane l holds key 16*(l/32) + e.
__device__ inline int wkperm(int m) { return 16 * ((m >> 2) & 1) + 4 * (m >> 3) + (m & 3); }

// Canonical score from global memory: sequential fp64 FMAs over d (exact
// products), one rounding to fp32.
template <typename T, int D>
__device__ inline float exact_dot_global(const T* __restrict__ q, const T* __restrict__ k) {
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
    for (int e = 0; e < 8; ++e) acc = __builtin_fma(double(to_f32(qv[e])), double(to_f32(kv[e])), acc);
  }
  return float(acc);
}

// Maximum of the 16 scores of a lane: a depth-3 tree of plain v_max3_f32
// (scores are MFMA results or -inf, never signaling NaNs, so the quieting
// that fmaxf puts in front of each operand is not needed; on quiet NaNs
// v_max3_f32 returns the maximum of the other operands, as fmaxf does).
__device__ inline float max16(const f32x16_t& a) {
  const float t0 = max3_plain(a[0], a[1], a[2]), t1 = max3_plain(a[3], a[4], a[5]);
  const float t2 = max3_plain(a[6], a[7], a[8]), t3 = max3_plain(a[9], a[10], a[11]);
  const float t4 = max3_plain(a[12], a[13], a[14]);
  return max_plain(max3_plain(t0, t1, t2), max3_plain(t3, t4, a[15]));
}

template <typename T, int D, int BK>
__global__ __launch_bounds__(256, 2) void select_wave_kernel(
    const T* __restrict__ qs, int64_t sqb, int64_t sqh, int64_t sqn, const T* __restrict__ k,
    int64_t skb, int64_t skh, int64_t sks, int64_t B, int64_t Hq, int64_t Hk, int64_t Sk,
    int64_t qps, uint32_t gspan, int causal, int64_t bsq, float gap_scalar,
    const float* __restrict__ gaps, const float* __restrict__ kmax, RowLayout lay,
    int32_t* __restrict__ counts, int32_t* __restrict__ indices, int64_t nrowsets, int segk,
    int nseg, SegCarry* __restrict__ carry, int mode) {
  using M = Mfma<T>;
  using vec = typename M::vec;
  constexpr int NS = D / 16;                    // MFMA steps over the features
  constexpr int ROWB = 2 * D;                   // bytes per key row
  constexpr int NCH = D / 8;                    // 16-byte chunks per row
  constexpr int STAGE = kWChunk * ROWB;         // bytes of one chunk of K
  constexpr int RPC = 1024 / ROWB;              // rows per 1 KB copy
  constexpr int H = STAGE / 1024 / kWWaves;     // copies per wave per chunk
  static_assert(H >= 1 && H * kWWaves * RPC == kWChunk, "chunk copies must split over the waves");
  static_assert(BK == 16 || BK == 32 || BK == 64, "tile size");

  __shared__ __attribute__((aligned(1024))) unsigned char kst[2 * STAGE];
  __shared__ int32_t nml[kWWaves][kWRows][kWList];        // near-max tiles per row
  __shared__ float nmx[kWWaves][kWRows][kWList];          // their MFMA tile maxima
  __shared__ float exr[kWWaves][kWRows];                  // exact max of folded tiles
  __shared__ float tmx[kWWaves][kWList];                  // rare path: exact tile maxima
  __shared__ uint32_t ambm[kWWaves][kWRows][4];           // rare path: ambiguous keys
  __shared__ int32_t ambk[kWWaves][128];                  // rare path: keys [0,64), flags [64,128)

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid / 64), lane = tid % 64;
  const int l32 = lane % 32, hh = lane / 32;

  const WorkOrder wo{nrowsets * nseg, B, Hq, Hk, causal == 0};
  int64_t item, bh;
  if (!wo.map_item(blockIdx.x, item, bh)) return;  // idle block (uniform)
  const int64_t rs = item / nseg;    // row set
  const int seg = int(item % nseg);  // key segment [seg*segk, (seg+1)*segk)
  const int64_t b = bh / Hq, h = bh % Hq, hk = h / (Hq / Hk);
  const int64_t nc = lay.nc, J0 = lay.J0;
  const int64_t jr_wave = rs * (kWWaves * kWRows) + kWRows * wave;  // first row of this wave
  const int64_t jr = jr_wave + l32;
  const bool valid = jr < nc;
  const float gap = gaps ? gaps[bh] : gap_scalar;
  const float kn = kmax[b * Hk + hk];
  const int smin = int(lay.smin());
  const int sk = int(Sk);  // < 2^24 (host check)
  // Groups of 16 or 32 keys (the span then divides the chunk): the running
  // maximum restarts inside chunks and no near-max tiles are listed.
  const bool short_groups = BK < kWChunk && gspan < uint32_t(kWChunk);

  // Causal tile limit of a row: tiles with start < lim are selectable.  The
  // reference's test r > trunc((k_off - off0) / qps), r the row inside its
  // BLOCK_SIZE_Q program and off0 = (J - r) * qps, is k_off < J*qps for
  // r >= 1 and k_off <= (J-1)*qps for r == 0.
  auto row_lim = [&](int64_t row) -> int {
    if (!causal) return 0x7fffffff;
    const int64_t J = J0 + row, r = row % bsq;
    const int64_t lim = (r == 0) ? (J - 1) * qps + 1 : J * qps;
    return int(lim < 0 ? 0 : (lim > 0x7fffffff ? 0x7fffffff : lim));
  };
  // Key range a row set needs: up to the end of its last selectable tile.
  auto range_end = [&](int64_t last_row) -> int {
    if (!causal) return sk;
    const int64_t lim = row_lim(last_row);
    const int64_t e = (lim + BK - 1) / BK * BK;
    return int(e < Sk ? e : Sk);
  };
  const int64_t nvalid_wave = nc - jr_wave < kWRows ? nc - jr_wave : kWRows;
  const int64_t nvalid_wg = nc - rs * (kWWaves * kWRows) < kWWaves * kWRows
                                ? nc - rs * (kWWaves * kWRows)
                                : kWWaves * kWRows;
  // Keys of this work item: the row set's range clipped to the segment.
  const int seg_lo = seg * segk;
  const int seg_hi = nseg > 1 ? seg_lo + segk : 0x7fffffff;
  int wave_end = nvalid_wave > 0 ? range_end(jr_wave + nvalid_wave - 1) : 0;
  int wg_end = range_end(rs * (kWWaves * kWRows) + nvalid_wg - 1);
  if (wave_end > seg_hi) wave_end = seg_hi;
  if (wg_end > seg_hi) wg_end = seg_hi;
  const int lim = valid ? row_lim(jr) : 0;

  // ---- pooled rows: B operand (row l32, features [16s + 8hh, +8)) ---------
  const T* qrow = qs + b * sqb + h * sqh + jr * sqn;
  vec qreg[NS];
  double ss = 0.0;
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    uint4 raw = make_uint4(0, 0, 0, 0);
    if (valid) raw = *reinterpret_cast<const uint4*>(qrow + 16 * s + 8 * hh);
    qreg[s] = __builtin_bit_cast(vec, raw);
    const T* e8 = reinterpret_cast<const T*>(&raw);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const double x = double(to_f32(e8[e]));
      ss = __builtin_fma(x, x, ss);
    }
  }
  // Norm bound of the row (both halves of the features), rounded up.
  {
    const uint64_t u = __builtin_bit_cast(uint64_t, ss);
    const uint32_t lo = other_half(uint32_t(u)), hi = other_half(uint32_t(u >> 32));
    ss += __builtin_bit_cast(double, (uint64_t(hi) << 32) | lo);
  }
  float band, win;
  {
    const double A = __builtin_sqrt(ss) * (1.0 + 0x1p-20) * double(kn) * (1.0 + 0x1p-20);
    const double delta = double(2 * (D / 16 + 2) + 1) * 0x1p-23 * A;
    const double ag = __builtin_fabs(double(gap));
    band = float(1.25 * (2.0 * delta + 6.0 * 0x1p-24 * (A + ag)) + 1e-28);
    win = float(1.25 * (2.0 * delta + 4.0 * 0x1p-24 * A) + 1e-28);
  }

  // ---- output of this lane's row ------------------------------------------
  // Segment seg writes its keys from its first slot of the row (segments
  // never overlap); no keys are stored when only counting (indices null).
  int64_t ostart = 0, ocap = 0;
  if (valid) lay.segment_slots(bh, jr, seg, nseg, seg_lo, ostart, ocap);
  const int cap = int(ocap);
  // The keys are stored through a buffer resource over this wave's rows (the
  // rows of one (b, h) are contiguous, at most 32 * 2^24 slots: the byte
  // offsets fit 32 bits).  A lane's offset starts at its row's first slot of
  // the segment and is clamped to the row's last slot, so that no store
  // leaves its row and the loop needs no bounds branch.
  const int64_t wrow0 = nvalid_wave > 0 ? lay.row_start(bh, jr_wave) : 0;
  const int64_t wrow_end = nvalid_wave > 0 ? lay.row_start(bh, jr_wave + nvalid_wave) : 0;
  const __amdgpu_buffer_rsrc_t ors = make_rsrc(
      indices ? indices + wrow0 : indices, uint32_t(indices ? (wrow_end - wrow0) * 4 : 0));
  const uint32_t ofirst = valid ? uint32_t(ostart - wrow0) * 4u : 0xfffffff0u;
  const uint32_t olast = valid && cap > 0 ? ofirst + uint32_t(cap - 1) * 4u : 0xfffffff0u;
  int rowcnt = 0;   // keys selected so far for this row
  int listcnt = 0;  // near-max tiles listed for this row
  float m = -__builtin_inff();  // MFMA running maximum of the row

  // ---- K copies --------------------------------------------------------------
  const T* kh = k + b * skb + hk * skh;
  const uint32_t krb = uint32_t(sks * 2);
  const __amdgpu_buffer_rsrc_t krs = make_rsrc(kh, uint32_t(((Sk - 1) * sks + D) * 2));
  const uint32_t kst_lds = lds_addr(kst);
  // Copy x of this wave fills LDS rows [(wave*H + x)*RPC, +RPC) of a stage;
  // LDS row R of block R/32 holds key 32*(R/32) + wkperm(R % 32); this lane
  // fetches physical chunk p of row R, i.e. logical chunk p ^ (R % NCH).
  uint32_t coff[H];
#pragma unroll
  for (int x = 0; x < H; ++x) {
    const int R = (wave * H + x) * RPC + lane / NCH;
    const int key = 32 * (R / 32) + wkperm(R % 32);
    coff[x] = uint32_t(key) * krb + uint32_t(16 * ((lane % NCH) ^ (R % NCH)));
  }
  auto issue_chunk = [&](int kb0, int st) {
    const uint32_t base = uint32_t(kb0) * krb;
#pragma unroll
    for (int x = 0; x < H; ++x)
      copy16_to_lds(krs, kst_lds + uint32_t(st * STAGE + (wave * H + x) * 1024), base + coff[x]);
  };
  // A operand of step s for block b: LDS row 32b + l32, chunk 2s + hh.
  uint32_t aoff[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s)
    aoff[s] = uint32_t(l32 * ROWB + 16 * ((2 * s + hh) ^ (l32 % NCH)));
  auto score = [&](int st, f32x16_t* out) {
    const unsigned char* stage = kst + st * STAGE;
#pragma unroll
    for (int bb = 0; bb < 2; ++bb) {
      f32x16_t a2;
#pragma unroll
      for (int e = 0; e < 16; ++e) a2[e] = 0.f;
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const vec a = __builtin_bit_cast(
            vec, *reinterpret_cast<const uint4*>(stage + bb * 32 * ROWB + aoff[s]));
        a2 = M::run(a, qreg[s], a2);
      }
      out[bb] = a2;
    }
  };

  // The first visited chunk need not start a group: start with no folded tiles
  // (or, in the carry pass, with the maxima of the group's earlier segments).
  const int64_t crow = (bh * nc + jr) * nseg;  // this row's carry records
  const int s_first = int((int64_t(seg_lo) / int64_t(gspan)) * int64_t(gspan) / segk);  // group's first segment
  float cm_in = -__builtin_inff();  // carry pass: MFMA maximum of the earlier segments
  if (mode == kPassCarry) {
    float ce = -__builtin_inff();
    if (valid)
      for (int s2 = s_first; s2 < seg; ++s2) {
        cm_in = __builtin_fmaxf(cm_in, carry[crow + s2].m);
        ce = __builtin_fmaxf(ce, carry[crow + s2].ex);
      }
    m = cm_in;
    if (hh == 0) exr[wave][l32] = ce;
  } else if (hh == 0) {
    exr[wave][l32] = -__builtin_inff();
  }
  ambk[wave][64 + lane] = 0;  // resolved flags start cleared

  // Counts block bb's selections of the row and, unless only counting
  // (indices null), stores them.
  auto append = [&](int kb0, int bb, uint32_t bt) {
    const int cnt = __builtin_popcount(bt);
    const int ocnt = int(other_half(uint32_t(cnt)));
    if (indices) {
      uint32_t off = ofirst + uint32_t(rowcnt + (hh ? ocnt : 0)) * 4u;
      const int key0 = kb0 + 32 * bb + 16 * hh;
      while (bt) {
        const int e = __builtin_ctz(bt);
        bt &= bt - 1;
        __builtin_amdgcn_raw_buffer_store_b32(key0 + e, ors, off < olast ? off : olast, 0, 0);
        off += 4u;
      }
    }
    rowcnt += cnt + ocnt;
  };

  // Exact resolution of the rows in `need` (bit r for row r), one row at a
  // time: row r's jobs are every key of its listed tiles, then its ambiguous
  // keys (ambm, as chunk offsets from kb0); the exact tile maxima give the
  // exact running maximum at each ambiguous key's tile.  Resolved selections
  // go to ovr, the listed tiles are folded into the row's exact maximum and
  // the list is cleared.  With short groups the row's list is instead made
  // here: the tiles of the chunk from each ambiguous key's group start up to
  // the key's own tile.
  auto resolve = [&](uint64_t need, int kb0, uint32_t (&ovr)[2]) {
    while (need) {
      const int r = __builtin_ctzll(need);
      need &= need - 1;
      int n = __builtin_amdgcn_readlane(listcnt, r);
      const T* qr = qs + b * sqb + h * sqh + (jr_wave + r) * sqn;
      // Ambiguous keys of row r, as chunk offsets 32b + 16hh + e (64 bits).
      const uint64_t a64 = uint64_t(ambm[wave][r][0]) | (uint64_t(ambm[wave][r][1]) << 16) |
                           (uint64_t(ambm[wave][r][2]) << 32) |
                           (uint64_t(ambm[wave][r][3]) << 48);
      if constexpr (BK < kWChunk) {
        if (short_groups) {
          constexpr int NT = kWChunk / BK;  // tiles per chunk
          const int tpg = int(gspan) / BK;  // tiles per group
          uint32_t tneed = 0;
#pragma unroll
          for (int t = 0; t < NT; ++t)
            if ((a64 >> (t * BK)) & ((uint64_t(1) << BK) - 1u))
              tneed |= ((2u << t) - 1u) & ~((1u << (t / tpg * tpg)) - 1u);
          tneed = __builtin_amdgcn_readfirstlane(tneed);
          n = __builtin_popcount(tneed);
          if (lane < NT && ((tneed >> lane) & 1u))
            nml[wave][r][__builtin_popcount(tneed & ((1u << lane) - 1u))] = kb0 / BK + lane;
        }
      }
      if ((a64 >> lane) & 1u)
        ambk[wave][__builtin_amdgcn_mbcnt_hi(uint32_t(a64 >> 32),
                                             __builtin_amdgcn_mbcnt_lo(uint32_t(a64), 0))] =
            kb0 + lane;
      const int ntile = n * BK, njobs = ntile + __builtin_popcountll(a64);
      float E0 = exr[wave][r];
      uint64_t take = 0;
      for (int p = 0; p < njobs; p += 64) {
        const int j = p + lane;
        int key = -1;
        if (j < ntile) key = nml[wave][r][j / BK] * BK + j % BK;
        else if (j < njobs) key = ambk[wave][j - ntile];
        float ex = -__builtin_inff();
        if (key >= smin && key < sk) ex = exact_dot_global<T, D>(qr, kh + int64_t(key) * sks);
        // exact maxima of the listed tiles (groups of BK lanes)
        float tx = j < ntile ? ex : -__builtin_inff();
#pragma unroll
        for (int o = 1; o < BK; o <<= 1) tx = __builtin_fmaxf(tx, __shfl_xor(tx, o));
        if (j < ntile && j % BK == 0) tmx[wave][j / BK] = tx;
        // decisions of the ambiguous keys of this pass (all tile maxima
        // come from this or earlier passes)
        bool tk = false;
        if (j >= ntile && j < njobs) {
          // listed tiles of the key's group up to its own tile (with long
          // groups every listed tile is of the current group: tg = 0)
          const int t = key / BK;
          const int tg = short_groups ? int(uint32_t(key) & ~(gspan - 1u)) / BK : 0;
          float E = E0;
          for (int i = 0; i < n; ++i) {
            const int u = nml[wave][r][i];
            if (u <= t && u >= tg) E = __builtin_fmaxf(E, tmx[wave][i]);
          }
          tk = (ex + gap) >= E;
        }
        // Fold: bit (key - kb0) of the row's resolved selections.
        if (tk) ambk[wave][64 + key - kb0] = 1;
      }
      // Gather the resolved bits: lane l reads the flag of chunk offset l.
      const int fl = (a64 >> lane) & 1u ? ambk[wave][64 + lane] : 0;
      take = __builtin_amdgcn_ballot_w64(fl == 1);
      if ((a64 >> lane) & 1u) ambk[wave][64 + lane] = 0;
      // This lane's quarter (2*bb + hh) of row r.
      if (l32 == r) {
        ovr[0] |= uint32_t(take >> (16 * hh)) & 0xffffu;
        ovr[1] |= uint32_t(take >> (32 + 16 * hh)) & 0xffffu;
      }
      // Fold the listed tiles into the row's exact maximum (short groups end
      // with the chunk: nothing to fold).
      float E = E0;
      for (int i = 0; i < n; ++i) E = __builtin_fmaxf(E, tmx[wave][i]);
      if (lane == 0 && !short_groups) exr[wave][r] = E;
      if (l32 == r) listcnt = 0;
    }
  };

  // Carry pass: the near-max tiles of the earlier segments whose maximum is
  // within `win` of the carried maximum (only those can hold the exact
  // maximum) start the row's list; rows with more candidates than the list
  // holds fold a full list exactly and continue.
  if (mode == kPassCarry) {
    int ps = s_first, pi = 0;  // next candidate: segment ps, tile pi
    ambm[wave][l32][hh] = 0u;
    ambm[wave][l32][2 + hh] = 0u;
    while (true) {
      if (hh == 0 && valid) {
        while (listcnt < kWList - 4 && ps < seg) {
          const SegCarry& cr = carry[crow + ps];
          if (cr.m >= cm_in - win && pi < cr.n) {
            nml[wave][l32][listcnt] = cr.tile[pi++];
            nmx[wave][l32][listcnt] = cr.m;
            ++listcnt;
          } else {
            ++ps;
            pi = 0;
          }
        }
      }
      const uint64_t more = __builtin_amdgcn_ballot_w64(hh == 0 && valid && ps < seg);
      if (more == 0) break;
      uint32_t ovr[2] = {0u, 0u};
      resolve(more, 0, ovr);
    }
    const uint32_t lc = other_half(uint32_t(listcnt));  // the high half mirrors the count
    if (hh) listcnt = int(lc);
  }

  // ---- chunk loop -------------------------------------------------------------
  // Software pipeline: in iteration c the MFMA scores of chunk c+1 are computed
  // (stage (c+1)&1) while the decisions of chunk c run on the VALU, and the
  // copy of chunk c+2 is in flight into stage c&1.  The 2*NS MFMAs of chunk
  // c+1 are issued one per slot, the slots spread through chunk c's VALU work
  // (sched_barrier keeps the order): a wave's MFMA then executes while the
  // same wave issues the VALU instructions that follow it, instead of the wave
  // stalling on a burst of MFMA issues and then running its VALU work alone.
  const int kfirst = (smin > seg_lo ? smin : seg_lo) / kWChunk * kWChunk;
  const int nchunks = wg_end > kfirst ? (wg_end - kfirst + kWChunk - 1) / kWChunk : 0;
  f32x16_t acc_even[2], acc_odd[2];  // scores of the even / odd chunks
  if (nchunks > 0) {
    issue_chunk(kfirst, 0);
    if (nchunks > 1) issue_chunk(kfirst + kWChunk, 1);
    vm_lds_barrier();
    if (kfirst < wave_end) score(0, acc_even);
  }
  // One chunk; the parity P = c & 1 is a compile-time constant so that the
  // stage addresses fold into the instructions and the scores of chunk c
  // (acc) and c+1 (nxt) alternate between two register sets with no copy.
  auto chunk = [&](int c, auto parity_tag, f32x16_t (&acc)[2], f32x16_t (&nxt)[2]) {
    constexpr int st = decltype(parity_tag)::value;
    const int kb0 = kfirst + c * kWChunk;
    vm_lds_barrier();  // chunk c+1 landed; every wave has scored chunk c (stage st is free)
    if (c + 2 < nchunks) issue_chunk(kb0 + 2 * kWChunk, st);
    if (kb0 < wave_end) {  // this wave's rows still need keys (uniform)
      // MFMA slot i of chunk c+1: block i / NS, feature step i % NS; the A
      // operand is read from LDS two slots ahead of its MFMA.  Past the
      // wave's last chunk the slots score stale LDS contents, which the next
      // iteration does not use (kb0 >= wave_end there).
      const unsigned char* nstage = kst + (st ^ 1) * STAGE;
      auto aload = [&](int i) {
        return __builtin_bit_cast(vec, *reinterpret_cast<const uint4*>(
                                           nstage + (i / NS) * 32 * ROWB + aoff[i % NS]));
      };
      vec aring[3];
      aring[0] = aload(0);
      aring[1] = aload(1);
      auto slot = [&](int i) {
        __builtin_amdgcn_sched_barrier(0);
        if (i + 2 < 2 * NS) aring[(i + 2) % 3] = aload(i + 2);
        const int bb = i / NS, s = i % NS;
        if (s == 0) {
#pragma unroll
          for (int e = 0; e < 16; ++e) nxt[bb][e] = 0.f;
        }
        nxt[bb] = M::run(aring[i % 3], qreg[s], nxt[bb]);
        __builtin_amdgcn_sched_barrier(0);
      };
      // Slots are placed after MFMA-free stretches of roughly equal VALU work.
      constexpr int NSL = 2 * NS;
      auto slots = [&](int from, int to) {
#pragma unroll
        for (int i = from; i < to; ++i) slot(i);
      };

      if (kb0 < smin || kb0 + kWChunk > sk) {  // keys outside [smin, Sk) are not visited
#pragma unroll
        for (int bb = 0; bb < 2; ++bb)
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int key = kb0 + 32 * bb + 16 * hh + e;
            if (key < smin || key >= sk) acc[bb][e] = -__builtin_inff();
          }
      }
      if (uint32_t(kb0) % gspan == 0u) {  // a group starts with this chunk
        m = -__builtin_inff();
        listcnt = 0;
        if (hh == 0) exr[wave][l32] = -__builtin_inff();
      }
      slots(0, NSL / 8);

      // ---- running maximum per tile -------------------------------------------
      // A tile is worth listing only for a valid row, before the row's causal
      // limit (later tiles select nothing), and when it holds a visited key;
      // short groups list nothing.  Groups of 16 keys restart the running
      // maximum at every tile, groups of 32 at chunk offset 32 (rs1, rs2).
      bool live[2];
#pragma unroll
      for (int bb = 0; bb < 2; ++bb) {
        const int koff = BK == 16 ? kb0 + 32 * bb + 16 * hh : (BK == 32 ? kb0 + 32 * bb : kb0);
        live[bb] = !short_groups && valid && koff < lim && koff + BK > smin && koff < sk;
      }
      const bool rs1 = short_groups && gspan <= 16u, rs2 = short_groups;
      const float tm0 = max16(acc[0]), tm1 = max16(acc[1]);
      const float om0 = other_half(tm0), om1 = other_half(tm1);
      const float m_prev = m;  // running maximum before this chunk's tiles
      float mt[2];  // running max at this lane's tile of each block
      int rec[2];   // this lane lists the tile as near-max
      int nrec;     // tiles the row lists in this chunk
      int rpos[2];  // list positions of this lane's tiles
      float rmax[2];  // MFMA maxima of this lane's listed tiles
      {
        const float t00 = hh ? om0 : tm0, t01 = hh ? tm0 : om0;
        const float t10 = hh ? om1 : tm1, t11 = hh ? tm1 : om1;
        if (BK == 16) {
          const float r00 = max_plain(m, t00);
          const float r01 = rs1 ? t01 : max_plain(r00, t01);
          const float r10 = rs2 ? t10 : max_plain(r01, t10);
          const float r11 = rs1 ? t11 : max_plain(r10, t11);
          mt[0] = hh ? r01 : r00;
          mt[1] = hh ? r11 : r10;
          m = r11;
          rec[0] = (live[0] && tm0 >= mt[0] - win) ? 1 : 0;
          rec[1] = (live[1] && tm1 >= mt[1] - win) ? 1 : 0;
          const uint32_t orc = other_half(uint32_t(rec[0] | (rec[1] << 1)));
          const int f00 = hh ? int(orc & 1u) : rec[0], f01 = hh ? rec[0] : int(orc & 1u);
          const int f10 = hh ? int(orc >> 1) : rec[1], f11 = hh ? rec[1] : int(orc >> 1);
          rpos[0] = listcnt + (hh ? f00 : 0);
          rpos[1] = listcnt + f00 + f01 + (hh ? f10 : 0);
          nrec = f00 + f01 + f10 + f11;
          rmax[0] = tm0;
          rmax[1] = tm1;
        } else if (BK == 32) {
          const float bm0 = max_plain(t00, t01), bm1 = max_plain(t10, t11);
          const float r0 = max_plain(m, bm0), r1 = rs2 ? bm1 : max_plain(r0, bm1);
          mt[0] = r0;
          mt[1] = r1;
          m = r1;
          const int g0 = (live[0] && bm0 >= r0 - win) ? 1 : 0;
          const int g1 = (live[1] && bm1 >= r1 - win) ? 1 : 0;
          rec[0] = hh == 0 ? g0 : 0;
          rec[1] = hh == 0 ? g1 : 0;
          rpos[0] = listcnt;
          rpos[1] = listcnt + g0;
          nrec = g0 + g1;
          rmax[0] = bm0;
          rmax[1] = bm1;
        } else {
          const float cm = max_plain(max_plain(t00, t01), max_plain(t10, t11));
          const float r = max_plain(m, cm);
          mt[0] = mt[1] = r;
          m = r;
          const int g = (live[0] && cm >= r - win) ? 1 : 0;
          rec[0] = hh == 0 ? g : 0;
          rec[1] = 0;
          rpos[0] = rpos[1] = listcnt;
          nrec = g;
          rmax[0] = rmax[1] = cm;
        }
      }
      slots(NSL / 8, NSL / 4);
#pragma unroll
      for (int bb = 0; bb < 2; ++bb)
        if (rec[bb]) {
          const int tk = BK == 16 ? kb0 + 32 * bb + 16 * hh : (BK == 32 ? kb0 + 32 * bb : kb0);
          nml[wave][l32][rpos[bb]] = tk / BK;
          nmx[wave][l32][rpos[bb]] = rmax[bb];
        }
      listcnt += nrec;
      slots(NSL / 4, 3 * NSL / 8);

      // ---- decisions ------------------------------------------------------------
      // With hi = (m^ - gap) + band and x = hi - s^: selected outright when
      // x < 0 (the sign of a difference is exact, and hi is never -0: a sum of
      // opposite equal values rounds to +0), ambiguous when 0 <= x <= 2*band,
      // rejected above.  The sign bits are shifted into the lane's mask
      // (v_alignbit), and as unsigned integers the smallest non-negative x is
      // the smallest bit pattern (negative x sort above 2*band), so one
      // unsigned minimum tests ambiguity.  Tiles past the causal limit or
      // starting at or past Sk select nothing (hi = +inf).  x is never NaN:
      // s^ is -inf only for keys past Sk, and any other tile holds a key below
      // Sk, so its running maximum is finite, since the host runs this kernel
      // only when the first selectable key starts a 64-key chunk (keys below
      // it are never visited).
      uint32_t bits[2];
      float hi[2];
      uint32_t xmin = 0xffffffffu;
#pragma unroll
      for (int bb = 0; bb < 2; ++bb) {
        const int koff = BK == 16 ? kb0 + 32 * bb + 16 * hh : (BK == 32 ? kb0 + 32 * bb : kb0);
        const bool ok = valid && koff < lim && koff < sk && mode != kPassMax;  // maxima pass: none
        hi[bb] = ok ? (mt[bb] - gap) + band : __builtin_inff();
        uint32_t bt = 0;
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          if (mode != kPassMax) {
#pragma unroll
            for (int e = 15 - 8 * half; e >= 8 - 8 * half; --e) {
              const uint32_t x = __builtin_bit_cast(uint32_t, hi[bb] - acc[bb][e]);
              bt = __builtin_amdgcn_alignbit(bt, x, 31u);  // (bt << 1) | sign(x)
              xmin = x < xmin ? x : xmin;
            }
          }
          const int sl = 3 * NSL / 8 + (2 * bb + half) * NSL / 8;
          slots(sl, sl + NSL / 8);
        }
        bits[bb] = bt;
      }
      const uint32_t band2 = __builtin_bit_cast(uint32_t, 2.f * band);
      const bool amb_lane = xmin <= band2;
      if (__builtin_amdgcn_ballot_w64(amb_lane || listcnt > kWList - 4) != 0) {
        // ---- rare path: exact resolution, one row at a time ----------------------
        // Row r's jobs: every key of its listed tiles, then its ambiguous keys;
        // the exact tile maxima give the exact running maximum at each
        // ambiguous key's tile.
#pragma unroll
        for (int bb = 0; bb < 2; ++bb) {
          uint32_t x = 0;
#pragma unroll
          for (int e = 0; e < 16; ++e)
            x |= uint32_t(__builtin_bit_cast(uint32_t, hi[bb] - acc[bb][e]) <= band2) << e;
          ambm[wave][l32][2 * bb + hh] = x;
        }
        // (no short-circuit: the lane exchange must run with the whole wave active)
        const bool row_amb = (uint32_t(amb_lane) | other_half(uint32_t(amb_lane))) != 0u;
        uint64_t need = __builtin_amdgcn_ballot_w64(hh == 0 && (row_amb || listcnt > kWList - 4));
        // The rows found here first drop the listed tiles that cannot hold the
        // exact running maximum: a tile whose MFMA maximum is below
        // m_prev - win, m_prev the running maximum before this chunk's tiles,
        // since the tile that set m_prev (listed, or folded into exr) is
        // exactly above it (win >= 2*delta plus rounding).  Rows whose list is
        // then short enough and that hold no ambiguous key need no exact work.
        if ((need >> lane) & 1u) {
          const float cut = m_prev - win;
          int keep = 0;
          for (int i = 0; i < listcnt; ++i) {
            const float x = nmx[wave][l32][i];
            if (x >= cut) {
              nml[wave][l32][keep] = nml[wave][l32][i];
              nmx[wave][l32][keep] = x;
              ++keep;
            }
          }
          listcnt = keep;
        }
        {
          const uint32_t lc = other_half(uint32_t(listcnt));  // the high half mirrors the count
          if (hh) listcnt = int(lc);
        }
        need = __builtin_amdgcn_ballot_w64(hh == 0 && (row_amb || listcnt > kWList - 4));
        uint32_t ovr[2] = {0u, 0u};
        resolve(need, kb0, ovr);
        bits[0] |= ovr[0];
        bits[1] |= ovr[1];
      }
      if (mode != kPassMax) append(kb0, 0, bits[0]);
      slots(7 * NSL / 8, NSL);
      if (mode != kPassMax) append(kb0, 1, bits[1]);
    }
  };
  for (int c = 0; c < nchunks; c += 2) {
    chunk(c, std::integral_constant<int, 0>{}, acc_even, acc_odd);
    if (c + 1 < nchunks) chunk(c + 1, std::integral_constant<int, 1>{}, acc_odd, acc_even);
  }

  if (mode == kPassMax) {
    // Keep the listed tiles within `win` of the segment maximum; rows with
    // more than kCarryTiles of them fold them exactly now (rare).
    int keep = 0;
    if (hh == 0 && valid) {
      for (int i = 0; i < listcnt; ++i)
        if (nmx[wave][l32][i] >= m - win) nml[wave][l32][keep++] = nml[wave][l32][i];
      listcnt = keep;
    }
    ambm[wave][l32][hh] = 0u;
    ambm[wave][l32][2 + hh] = 0u;
    uint32_t ovr[2] = {0u, 0u};
    resolve(__builtin_amdgcn_ballot_w64(hh == 0 && valid && listcnt > kCarryTiles), 0, ovr);
    if (valid && hh == 0) {
      SegCarry cr;
      cr.m = m;
      cr.ex = exr[wave][l32];
      cr.n = listcnt;
      cr.pad = 0;
#pragma unroll
      for (int i = 0; i < kCarryTiles; ++i) cr.tile[i] = i < listcnt ? nml[wave][l32][i] : -1;
      carry[crow + seg] = cr;
    }
    return;
  }

  if (valid && hh == 0 && counts) counts[(bh * nc + jr) * nseg + seg] = rowcnt < cap ? rowcnt : cap;
}

// Segment length the splits aim for: Sk / 16 keys, within [2048, 4096].  Short
// key ranges get shorter segments so that a launch has enough work-groups
// (32K keys: 16 segments of 2048 instead of 8 of 4096, 1792 work-groups per
// 512-row chunk at 28 q heads instead of 896); long ones keep 4096, where a
// segment's fixed costs weigh more than the extra parallelism.  Measured per
// prefill step on MI355X: 32K causal GQA -4%, 32760 non-causal -2%, 128K
// causal best at 4096, 119056 non-causal within 0.3% of its best.
static int64_t segment_target(int64_t Sk) {
  const int64_t t = Sk / 16;
  return t < 2048 ? 2048 : (t > 4096 ? 4096 : t);
}

// Key segments of the split selection: a length that is a multiple of the
// group span (so every segment starts a group and carries no state in) and of
// the 64-key chunk; 0 when the groups are too long to split.
int64_t select_wave_segment_keys(int64_t Sk, int64_t bk, int64_t group) {
  constexpr int64_t kMaxSeg = 64;
  const int64_t gs = bk * group;
  if ((gs % kWChunk != 0 && kWChunk % gs != 0) || gs >= Sk) return 0;
  const int64_t unit = gs > kWChunk ? gs : kWChunk;  // groups of 16 or 32 keys: whole chunks
  int64_t want = (Sk + kMaxSeg - 1) / kMaxSeg;  // at most 64 segments
  if (want < segment_target(Sk)) want = segment_target(Sk);
  const int64_t segk = (want + unit - 1) / unit * unit;
  return segk < Sk ? segk : 0;
}

// Key segments of the two-pass split (maxima pass, then carry pass), for rows
// that are one group long (group span >= Sk): a multiple of the 64-key chunk,
// about segment_target(Sk) keys, at most 64 segments; 0 when there is nothing
// to split.
int64_t select_wave_carry_segment_keys(int64_t Sk, int64_t bk, int64_t group) {
  constexpr int64_t kMaxSeg = 64;
  if (bk * group < Sk) return 0;
  int64_t want = (Sk + kMaxSeg - 1) / kMaxSeg;
  if (want < segment_target(Sk)) want = segment_target(Sk);
  const int64_t segk = (want + kWChunk - 1) / kWChunk * kWChunk;
  return segk < Sk ? segk : 0;
}

// Group spans: multiples of the 64-key chunk, or 16 and 32 keys (spans that
// divide the chunk).
bool select_wave_supported(int dtype, int64_t D, int64_t bk, int64_t group) {
  const int64_t gs = bk * group;
  return (dtype == kBF16 || dtype == kF16) && (D == 64 || D == 128) &&
         (bk == 16 || bk == 32 || bk == 64) && gs > 0 &&
         (gs % kWChunk == 0 || kWChunk % gs == 0);
}

template <typename T, int D, int BK>
static hipError_t launch_select_wave_tdb(const void* qs, int64_t sqb, int64_t sqh, int64_t sqn,
                                         const void* k, int64_t skb, int64_t skh, int64_t sks,
                                         int64_t B, int64_t Hq, int64_t Hk, int64_t Sk,
                                         int64_t qps, int64_t group, int causal, int64_t bsq,
                                         float gap, const float* gaps, const float* kmax,
                                         const RowLayout& lay, int32_t* counts, int32_t* indices,
                                         int64_t segk, SegCarry* carry, int mode,
                                         hipStream_t stream) {
  const int64_t nrowsets = (lay.nc + kWWaves * kWRows - 1) / (kWWaves * kWRows);
  const int64_t nseg = segk > 0 ? (Sk + segk - 1) / segk : 1;
  // Group span in keys, capped at 2^31 (key offsets are below 2^24, so a span
  // that large has its only boundary at 0 either way).
  const int64_t gs = (group > (int64_t(1) << 31) / BK) ? (int64_t(1) << 31) : BK * group;
  const int64_t nblocks = WorkOrder{nrowsets * nseg, B, Hq, Hk, causal == 0}.grid_items();
  hipLaunchKernelGGL((select_wave_kernel<T, D, BK>), dim3(unsigned(nblocks)), dim3(256), 0,
                     stream, static_cast<const T*>(qs), sqb, sqh, sqn, static_cast<const T*>(k),
                     skb, skh, sks, B, Hq, Hk, Sk, qps, uint32_t(gs), causal, bsq, gap, gaps, kmax,
                     lay, counts, indices, nrowsets, int(segk > 0 ? segk : 0), int(nseg), carry,
                     mode);
  return hipGetLastError();
}

template <typename T, int D>
static hipError_t launch_select_wave_td(int64_t bk, const void* qs, int64_t sqb, int64_t sqh,
                                        int64_t sqn, const void* k, int64_t skb, int64_t skh,
                                        int64_t sks, int64_t B, int64_t Hq, int64_t Hk, int64_t Sk,
                                        int64_t qps, int64_t group, int causal, int64_t bsq,
                                        float gap, const float* gaps, const float* kmax,
                                        const RowLayout& lay, int32_t* counts, int32_t* indices,
                                        int64_t segk, SegCarry* carry, int mode,
                                        hipStream_t stream) {
#define VA_SELW_BK(BB)                                                                          \
  if (bk == BB)                                                                                 \
    return launch_select_wave_tdb<T, D, BB>(qs, sqb, sqh, sqn, k, skb, skh, sks, B, Hq, Hk, Sk, \
                                            qps, group, causal, bsq, gap, gaps, kmax, lay,      \
                                            counts, indices, segk, carry, mode, stream);
  VA_SELW_BK(16)
  VA_SELW_BK(32)
  VA_SELW_BK(64)
#undef VA_SELW_BK
  return hipErrorInvalidValue;
}

hipError_t launch_select_wave(int dtype, const void* qs, int64_t sqb, int64_t sqh, int64_t sqn,
                              const void* k, int64_t skb, int64_t skh, int64_t sks, int64_t B,
                              int64_t Hq, int64_t Hk, int64_t Sk, int64_t D, int64_t qps,
                              int64_t bk, int64_t group, int causal, int64_t bsq, float gap,
                              const float* gaps, const float* kmax, const RowLayout& lay,
                              int32_t* counts, int32_t* indices, int64_t segk, void* carry,
                              int mode, hipStream_t stream) {
#define VA_SELW_CASE(TT, DD)                                                                 \
  return launch_select_wave_td<TT, DD>(bk, qs, sqb, sqh, sqn, k, skb, skh, sks, B, Hq, Hk, \
                                       Sk, qps, group, causal, bsq, gap, gaps, kmax, lay,    \
                                       counts, indices, segk, static_cast<SegCarry*>(carry), mode, stream);
  if (dtype == kBF16 && D == 128) { VA_SELW_CASE(bf16_t, 128) }
  if (dtype == kBF16 && D == 64) { VA_SELW_CASE(bf16_t, 64) }
  if (dtype == kF16 && D == 128) { VA_SELW_CASE(f16_t, 128) }
  if (dtype == kF16 && D == 64) { VA_SELW_CASE(f16_t, 64) }
#undef VA_SELW_CASE
  return hipErrorInvalidValue;
}

}  // namespace va
