// Vector-sparse flash-attention prefill, pair form (gfx950, bf16/fp16 MFMA,
// head_dim 128, 64-row q-blocks).
//
// Same result as attn_mfma.hip (vllm_flash_attn.sparse_attn_func as called at
// spattn/src/VecAttention.py:110-121; key sets restated from
// spattn/threshold/model_tuner.py:193-216, see keylist.h), organised so that
// a key two adjacent q-blocks both attend to is gathered once for both.
//
// The kernel's bound is the L2 -> LDS gather path: at 64 query rows per
// gathered K/V row, the copy path and the matrix cores are matched, and the
// copies are what the single-q-block kernel waits on.  Adjacent q-blocks'
// selected lists share about half of their keys at 32K-128K causal and about
// four fifths at 32760 non-causal, so one work-group per pair of q-blocks
// (A = chunk row 2i, B = 2i+1 of the launch) walks
//   - the local blocks: [0, 64) (A's diagonal when A is the first q-block),
//     A's diagonal block, B's diagonal block (causal only);
//   - the keys both rows selected ("common"), each gathered once;
//   - the keys only A selected and the keys only B selected, one tile of
//     each in turn,
// which the wave selection kernel's pair mode writes as separate runs (see
// select_wave.hip).  Waves are (row, row half): wave w serves rows
// [32(w & 1), +32) of q-block A (w < 2) or B, and computes every tile that
// holds keys of its row's list, as two 32-key halves; a wave skips the
// compute of tiles that are not its row's (it still issues its share of the
// copies and passes the barriers).  So the matrix work is exactly the
// single-q-block kernel's, and the gathered bytes drop by the shared keys.
//
// Data movement and pipeline are the ring form of attn_mfma.hip: three 16 KB
// LDS slots hold the operand stream K(0), V(0), K(1), V(1), ...; each step
// waits for its operand, passes one barrier and refills the slot freed with
// the operand two ahead, so each copy has one tile to land.  Key ids are
// staged in LDS ahead of their copies, all waves together once every four
// tiles.  Each list run is rotated by the row's position in its XCD's
// dispatch sequence, so that the work-groups running together on an XCD
// gather about the same keys (see attn_mfma.hip).
//
// Algorithmic work per gathered key of a row's list: 4*D FLOPs per query row.
#include "attn_tile.h"
#include "keylist.h"

namespace va {

namespace {

constexpr int kPD = 128;                              // head_dim
constexpr int kPQ = 64;                               // rows per q-block
constexpr int kPWaves = 4;
constexpr int kPRowBytes = 2 * kPD;                   // one K or V row
constexpr int kPTileBytes = kTileKeys * kPRowBytes;   // one K or V tile, 16 KB
constexpr int kPRowsPerCopy = 1024 / kPRowBytes;      // 4 rows per 1 KB copy
constexpr int kPCopies = kPTileBytes / 1024 / kPWaves;  // 4 copies per wave per operand
constexpr int kPIdSlots = 2 * kPWaves;                // ring of key-id tile slots
// three operand slots, the key-id ring, the run starts of the segments
constexpr int kPLdsBytes = 3 * kPTileBytes + kPIdSlots * kTileKeys * 4 + 3 * 64 * 4;
constexpr uint32_t kPRotPeriod = 96;  // work-groups an XCD holds at once (32 CUs x 3)

enum Run : int { kRunLocal = 0, kRunCommon = 1, kRunA = 2, kRunB = 3, kRunNone = 4 };

// The walk of a pair's key list, as plain scalars (helpers take them as
// arguments: a selection between captured variables of a closure becomes a
// variable-offset load from the closure, which keeps it and everything it
// refers to in scratch memory).
struct PairWalk {
  int ntiles, t_loc, t_c, t_a, t_b, r_c, r_a, r_b;  // tiles, and run rotations
  int n_c, n_a, n_b;                                // keys per run
  int JA, has_b, Sk;                                // local blocks (causal)
};
struct Step {
  int run, ti;  // run and tile of the run
};
// Tile facts: first key (local tiles), valid slots, whether rows A / B attend
// to it and whether it is their diagonal block (causal mask inside).
struct Tile {
  int key0, lim;
  bool in_a, in_b, diag_a, diag_b;
};

__device__ __forceinline__ int wrap(int x, int t) { return x < t ? x : x - t; }

// Walk step u -> (run, tile of the run): local tiles, the common run, then
// the private runs alternating A, B while both last (so that the waves of
// both rows get work in turn), each run rotated by its r_*.
__device__ __forceinline__ Step pair_step(int u, int ntiles, int t_loc, int t_c, int t_a, int t_b,
                                          int r_c, int r_a, int r_b) {
  if (u >= ntiles) return Step{kRunNone, 0};
  if (u < t_loc) return Step{kRunLocal, u};
  u -= t_loc;
  if (u < t_c) return Step{kRunCommon, wrap(u + r_c, t_c)};
  u -= t_c;
  const int t_ab = t_a < t_b ? t_a : t_b;
  if (u < 2 * t_ab) {
    const int x = u >> 1;
    if (u & 1) return Step{kRunB, wrap(x + r_b, t_b)};
    return Step{kRunA, wrap(x + r_a, t_a)};
  }
  const int x = u - t_ab;
  if (t_a > t_b) return Step{kRunA, wrap(x + r_a, t_a)};
  return Step{kRunB, wrap(x + r_b, t_b)};
}

// Local tile ti (causal): L0 = [0, min(64, Sk)) for both rows (A's diagonal
// when JA == 0, B's initial block), then A's diagonal block (JA >= 1), then
// B's diagonal block (when B exists).
__device__ __forceinline__ Tile pair_local_tile(int ti, int JA, int has_b, int Sk) {
  Tile tl;
  if (ti == 0) {
    tl.key0 = 0;
    tl.in_a = true;
    tl.in_b = has_b != 0;
    tl.diag_a = JA == 0;
    tl.diag_b = false;
  } else if (ti == 1 && JA >= 1) {
    tl.key0 = JA * kTileKeys;
    tl.in_a = true;
    tl.in_b = false;
    tl.diag_a = true;
    tl.diag_b = false;
  } else {
    tl.key0 = (JA + 1) * kTileKeys;
    tl.in_a = false;
    tl.in_b = true;
    tl.diag_a = false;
    tl.diag_b = true;
  }
  const int rem = Sk - tl.key0;
  tl.lim = rem < kTileKeys ? (rem > 0 ? rem : 0) : kTileKeys;
  return tl;
}

// The tile of walk step u.
__device__ __forceinline__ Tile pair_tile(int u, int ntiles, int t_loc, int t_c, int t_a, int t_b,
                                          int r_c, int r_a, int r_b, int n_c, int n_a, int n_b,
                                          int JA, int has_b, int Sk) {
  const Step sp = pair_step(u, ntiles, t_loc, t_c, t_a, t_b, r_c, r_a, r_b);
  if (sp.run == kRunLocal) return pair_local_tile(sp.ti, JA, has_b, Sk);
  Tile tl;
  tl.key0 = 0;
  tl.diag_a = tl.diag_b = false;
  int n = 0;
  if (sp.run == kRunCommon) n = n_c;
  if (sp.run == kRunA) n = n_a;
  if (sp.run == kRunB) n = n_b;
  const int rem = n - sp.ti * kTileKeys;
  tl.lim = rem < kTileKeys ? (rem > 0 ? rem : 0) : kTileKeys;
  tl.in_a = sp.run == kRunCommon || sp.run == kRunA;
  tl.in_b = sp.run == kRunCommon || sp.run == kRunB;
  return tl;
}

}  // namespace

template <typename T>
__global__ __launch_bounds__(64 * kPWaves, 3) void attn_pair_kernel(
    const T* __restrict__ q, int64_t sqb, int64_t sqh, int64_t sqs,
    const T* __restrict__ k, int64_t skb, int64_t skh, int64_t sks,
    const T* __restrict__ v, int64_t svb, int64_t svh, int64_t svs,
    T* __restrict__ out, int64_t sob, int64_t soh, int64_t sos, int64_t B,
    int64_t Hq, int64_t Hk, int64_t Sq, int64_t Sk, int causal, float scale_log2,
    const int32_t* __restrict__ counts, const int32_t* __restrict__ pcommon,
    const int32_t* __restrict__ indices, RowLayout lay, int nseg, int segk) {
  constexpr int D = kPD, NCH = D / 8, RPC = kPRowsPerCopy, H = kPCopies, W = kPWaves;
  constexpr uint32_t TB = uint32_t(kPTileBytes);
  constexpr int NQK = D / 16, NPV = D / 16;  // MFMAs per 32-key half
  using M = Mfma<T>;
  using vec = typename M::vec;

  __shared__ __attribute__((aligned(1024))) unsigned char smem[kPLdsBytes];
  int32_t* const ids = reinterpret_cast<int32_t*>(smem + 3 * TB);  // [kPIdSlots][64]
  int32_t* const run_sv = ids + kPIdSlots * kTileKeys;              // [3][64]

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid / 64), lane = tid % 64;
  const int l32 = lane % 32, hh = lane / 32;
  const int lst = wave >> 1, rh = wave & 1;  // row of the pair (0: A, 1: B), row half

  const int npairs = int((lay.nc + 1) / 2);
  const WorkOrder wo{npairs, B, Hq, Hk, causal == 0};
  int pr32, bh32;
  if (!wo.map_item32(blockIdx.x, pr32, bh32)) return;  // idle block (uniform)
  const int jra = 2 * pr32;
  const bool has_b = jra + 1 < int(lay.nc);
  const uint32_t hq32 = uint32_t(Hq);  // 32-bit: every index is below 2^31
  const int64_t bh = bh32;
  const int64_t b = uint32_t(bh32) / hq32, h = uint32_t(bh32) % hq32;
  const int64_t hk = uint32_t(h) / (hq32 / uint32_t(Hk));
  const int JA = int(lay.J0) + jra;  // q-block of row A (< 2^24)
  const int Jw = JA + lst;           // q-block of this wave's rows
  const bool wave_rows = lst == 0 || has_b;
  const int ns = nseg;  // >= 1

  // Per-segment counts (lane s: segment s) of rows A and B and of the keys
  // they share, as buffer loads without a branch (lanes past nseg, and row B
  // of an unpaired row A, read past the range and get 0), issued before Q so
  // that the scan below waits for them alone.
  const int64_t nc = lay.nc;
  const int ca_in = int(__builtin_amdgcn_raw_buffer_load_b32(
      make_rsrc(counts + (bh * nc + jra) * ns, uint32_t(ns) * 4u), lane * 4, 0, 0));
  const int cb_in = int(__builtin_amdgcn_raw_buffer_load_b32(
      make_rsrc(counts + (bh * nc + jra + 1) * ns, has_b ? uint32_t(ns) * 4u : 0u), lane * 4,
      0, 0));
  const int cc_in = int(__builtin_amdgcn_raw_buffer_load_b32(
      make_rsrc(pcommon + (bh * npairs + pr32) * ns, uint32_t(ns) * 4u), lane * 4, 0, 0));

  // ---- Q^T operand: lane holds row 32rh + l32, features [16s + 8hh, +8) ----
  const int qrow_local = 32 * rh + l32;
  const int64_t qpos = int64_t(Jw) * kPQ + qrow_local;
  vec qreg[D / 16];
  {
    // Rows past Sq load row Sq - 1 (never stored).
    const T* qr_ptr = q + b * sqb + h * sqh + (qpos < Sq ? qpos : Sq - 1) * sqs;
#pragma unroll
    for (int s = 0; s < D / 16; ++s)
      qreg[s] = __builtin_bit_cast(vec, *reinterpret_cast<const uint4*>(qr_ptr + 16 * s + 8 * hh));
  }

  // ---- the three runs of selected keys ---------------------------------------
  // Segment s of row A holds its common keys ascending from slot seg_slot(s)
  // and its own keys descending from the segment's last slot end_a(s) - 1;
  // segment s of row B its own keys ascending from seg_slot(s).  Row B's
  // slots follow row A's in the capacity layout.  run_sv[run - 1][s] holds
  // the run position where segment s starts (exclusive prefix sums of the
  // segment counts; kNone past nseg), in LDS rather than in registers.
  constexpr int kNone = 0x7fffffff;
  const int smin = int(lay.smin());
  const int cap_a = int(lay.capacity(JA));
  const int cap_b = has_b ? int(lay.capacity(JA + 1)) : 0;
  auto seg_slot = [=](int sg) __attribute__((always_inline)) {
    return ns > 1 ? (sg * segk > smin ? sg * segk : smin) - smin : 0;
  };
  auto seg_end = [=](int sg, int cap) __attribute__((always_inline)) {  // end of segment sg's slots in a row of `cap` slots
    const int nxt = sg + 1 < ns ? seg_slot(sg + 1) : kNone;
    return nxt < cap ? nxt : cap;
  };
  int c_n = 0, a_n = 0, b_n = 0;
  if (lane < ns) {  // clamp to what the segment's slots can hold
    const int s0 = seg_slot(lane), end_a = seg_end(lane, cap_a), end_b = seg_end(lane, cap_b);
    const int room_a = end_a > s0 ? end_a - s0 : 0, room_b = end_b > s0 ? end_b - s0 : 0;
    const int xa = ca_in < 0 ? 0 : (ca_in > room_a ? room_a : ca_in);
    const int xb = cb_in < 0 ? 0 : (cb_in > room_b ? room_b : cb_in);
    const int xm = xa < xb ? xa : xb;
    c_n = cc_in < 0 ? 0 : (cc_in > xm ? xm : cc_in);
    a_n = xa - c_n;
    b_n = xb - c_n;
  }
  const int inc_c = wave_inclusive_sum(c_n), inc_a = wave_inclusive_sum(a_n),
            inc_b = wave_inclusive_sum(b_n);
  if (wave == 0) {
    run_sv[lane] = lane < ns ? inc_c - c_n : kNone;
    run_sv[64 + lane] = lane < ns ? inc_a - a_n : kNone;
    run_sv[128 + lane] = lane < ns ? inc_b - b_n : kNone;
  }
  // (readfirstlane: the compiler's divergence analysis then treats the run
  // sizes, and the tile loop bounded by them, as uniform)
  const int n_c = __builtin_amdgcn_readfirstlane(__builtin_amdgcn_readlane(inc_c, ns - 1));
  const int n_a = __builtin_amdgcn_readfirstlane(__builtin_amdgcn_readlane(inc_a, ns - 1));
  const int n_b = __builtin_amdgcn_readfirstlane(__builtin_amdgcn_readlane(inc_b, ns - 1));
  // Slot of position p of a run in segment sg (uniform), from the segment's
  // start position st: common st -> seg_slot, A st -> end_a - 1 (descending),
  // B st -> cap_a + seg_slot.  As base + p (common, B) or base - p (A).
  auto run_base = [=](int run, int sg, int st) __attribute__((always_inline)) {
    if (run == kRunCommon) return seg_slot(sg) - st;
    if (run == kRunA) return seg_end(sg, cap_a) - 1 + st;
    return cap_a + seg_slot(sg) - st;
  };

  // ---- walk ------------------------------------------------------------------
  // Local tiles (causal): L0 = [0, min(64, Sk)) for both rows (A's diagonal
  // when JA == 0, B's initial block), then A's diagonal block (JA >= 1), then
  // B's diagonal block (when B exists).
  const int t_loc = causal ? 1 + (JA >= 1 ? 1 : 0) + (has_b ? 1 : 0) : 0;
  const int t_c = (n_c + kTileKeys - 1) / kTileKeys;
  const int t_a = (n_a + kTileKeys - 1) / kTileKeys;
  const int t_b = (n_b + kTileKeys - 1) / kTileKeys;
  const int t_ab = t_a < t_b ? t_a : t_b;
  const int ntiles = __builtin_amdgcn_readfirstlane(t_loc + t_c + t_a + t_b);
  const uint32_t rank = wo.xcd_rank(uint32_t(JA) >> 1, uint32_t(bh32), kPRotPeriod);
  auto rot = [=](int t) __attribute__((always_inline)) { return t >= 2 ? int(rank * uint32_t(t) / kPRotPeriod) : 0; };
  const int r_c = rot(t_c), r_a = rot(t_a), r_b = rot(t_b);
#define VA_PAIR_WALK ntiles, t_loc, t_c, t_a, t_b, r_c, r_a, r_b
  auto tile_of = [=](int u) __attribute__((always_inline)) {
    return pair_tile(u, VA_PAIR_WALK, n_c, n_a, n_b, JA, has_b ? 1 : 0, int(Sk));
  };

  // ---- buffers -------------------------------------------------------------
  const T* kh = k + b * skb + hk * skh;
  const T* vh = v + b * svb + hk * svh;
  // K and V as Sk records of their row stride: a key outside [0, Sk) reads zeros.
  const __amdgpu_buffer_rsrc_t krs = make_rsrc_rows(kh, uint32_t(sks * 2), uint32_t(Sk));
  const __amdgpu_buffer_rsrc_t vrs = make_rsrc_rows(vh, uint32_t(svs * 2), uint32_t(Sk));
  // The index slots of rows A and B (the resource is rebuilt where it is used:
  // held across the loop, the compiler keeps it in VGPRs, which a buffer
  // instruction cannot take).
  const int32_t* const pair_idx = indices + lay.row_offset(bh, jra);
  const uint32_t pair_idx_bytes = uint32_t(cap_a + cap_b) * 4u;

  // Copy geometry (as the ring form of attn_mfma.hip): copy x of this wave
  // fills tile rows [(wave*H + x)*RPC, +RPC); this lane fetches physical chunk
  // pc of row (wave*H + x)*RPC + qr, whose key id sits at ids position
  // id_pos + x.  At D = 128 the swizzle of those rows is 4qr + x, so the
  // chunk offset of copy x is c0 ^ 16x.
  const int qr = lane / NCH, pc = lane % NCH;
  const uint32_t c0 = uint32_t(16 * (pc ^ chunk_swizzle<D>((wave * H) * RPC + qr)));
  const int id_pos = (wave * RPC + qr) * H;
  const int w_slot = [&]() __attribute__((always_inline)) {  // tile slot whose id this lane stages
    const int w = lane / (RPC * H), r = (lane / H) % RPC, x = lane % H;
    return (w * H + x) * RPC + r;
  }();

  // Stage the key ids of walk step u into ids slot `slot` (one wave).  Run
  // position p of the tile lies in the segment whose start is the last one
  // <= p: a ballot finds the tile's first segment, and the (rare) segment
  // starts inside the tile are stepped over in a uniform loop.  Positions past
  // the run's end read past the index range (0); copy_pairs masks them.
  auto stage_ids = [=](int u, int slot) __attribute__((always_inline)) {
    int32_t* dst = ids + slot * kTileKeys;
    const Step sp = pair_step(u, VA_PAIR_WALK);
    const int run = sp.run, ti = sp.ti;
    if (run == kRunNone) {
      dst[lane] = -1;
    } else if (run == kRunLocal) {
      const Tile tl = pair_local_tile(ti, JA, has_b ? 1 : 0, int(Sk));
      dst[lane] = w_slot < tl.lim ? tl.key0 + w_slot : -1;
    } else {
      const int* const svr = run_sv + (run - kRunCommon) * 64;
      const int sv = svr[lane];
      // (a sum of masked terms: a selection between captured values would be
      // folded into a load through a selected closure field)
      const int n = n_c * int(run == kRunCommon) + n_a * int(run == kRunA) + n_b * int(run == kRunB);
      const int p0 = ti * kTileKeys, p = p0 + w_slot;
      const int sg = int(__builtin_popcountll(__builtin_amdgcn_ballot_w64(sv <= p0))) - 1;
      int base = run_base(run, sg, __builtin_amdgcn_readlane(sv, sg));
      const int pend = (p0 + kTileKeys < n ? p0 + kTileKeys : n) - 1;
      for (int s2 = sg + 1; s2 < ns; ++s2) {
        const int bnd = __builtin_amdgcn_readlane(sv, s2);
        if (bnd > pend) break;
        const int b2 = run_base(run, s2, bnd);
        if (p >= bnd) base = b2;
      }
      const int sl = run == kRunA ? base - p : base + p;
      copy4_to_lds(make_rsrc(pair_idx, pair_idx_bytes), lds_addr(dst),
                   p < n ? uint32_t(sl) * 4u : kOutOfRange);
    }
  };
  // Copy pairs of walk step u (ids in slot idslot): (key, chunk offset) per
  // copy; rows at or past the tile's valid slots get key 2^32 - 1 (zeros).
  auto copy_pairs = [=](int idslot, int lim, uint64_t (&pr)[H]) {
#pragma unroll
    for (int x = 0; x < H; ++x) {
      uint32_t key = uint32_t(ids[idslot * kTileKeys + id_pos + x]);
      if (lim < kTileKeys && qr >= lim - (wave * H + x) * RPC) key = 0xffffffffu;
      pr[x] = uint64_t(key) | (uint64_t(c0 ^ (16u * uint32_t(x))) << 32);
    }
  };
  const uint32_t lds_copy_base =
      uint32_t(__builtin_amdgcn_readfirstlane(int(lds_addr(smem) + uint32_t(wave * H * 1024))));
  auto copy_op = [=](auto base_tag, auto x_tag, bool is_v, uint64_t pr) __attribute__((always_inline)) {
    constexpr uint32_t off = decltype(base_tag)::value + decltype(x_tag)::value * 1024u;
    if (is_v)
      copy16_row_to_lds_at<off>(vrs, lds_copy_base, pr);
    else
      copy16_row_to_lds_at<off>(krs, lds_copy_base, pr);
  };

  // Wait for Q here, not inside the loop (where the wait would also cover the
  // copies in flight).
#pragma unroll
  for (int s = 0; s < D / 16; ++s) asm volatile("" ::"v"(qreg[s]));

  // LDS read offsets (D = 128): K rows 32hf + l32 (hf: key half), chunk
  // 2s + hh, at k0 ^ 32s (+ 8 KB for hf = 1); V^T rows 32hf + 16sub + 8r +
  // 4hh + j, features 32i + 16((lane/16) % 2) + 4(lane % 4), at v0[r] ^ 64i.
  const uint32_t k0 = uint32_t(l32 * kPRowBytes + 16 * (hh ^ chunk_swizzle<D>(l32)));
  uint32_t v0[2];
  {
    const int j = (lane % 16) / 4, g2 = 2 * ((lane / 16) % 2) + (lane % 4) / 2;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int R = 8 * r + 4 * hh + j;
      v0[r] = uint32_t(R * kPRowBytes + 16 * (g2 ^ chunk_swizzle<D>(R)) + 8 * (lane % 2));
    }
  }

  f32x16_t o[D / 32];
#pragma unroll
  for (int i = 0; i < D / 32; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[i][e] = 0.f;
  // Online softmax of this lane's row (as attn_mfma.hip): running maximum mc
  // in log2 units, -mc as the exponent offset, the raw-score level above
  // which a tile moves the maximum, and the partial row sum of this lane's
  // keys (lanes l and l ^ 32 hold the two halves of row l % 32).
  float mc = -__builtin_inff(), mneg = 0.f, thr = -__builtin_inff();
  const float inv_scale = 1.f / scale_log2;  // the host passes scale_log2 > 0
  float lsum = 0.f;
  // Returns the factor applied to O and the row sum (1 when the maximum stays).
  auto rescale = [&](float tmax) __attribute__((always_inline)) {
    float alpha = 1.f;
    if (__builtin_amdgcn_ballot_w64(tmax > thr)) {
      tmax = max_halves(tmax);
      const float mnew = __builtin_fmaxf(mc, tmax * scale_log2);
      alpha = (mnew == mc) ? 1.f : __builtin_amdgcn_exp2f(mc - mnew);
#pragma unroll
      for (int i = 0; i < D / 32; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[i][e] *= alpha;
      lsum *= alpha;
      mc = mnew;
      const bool none = mnew == -__builtin_inff();
      mneg = none ? 0.f : -mnew;
      thr = none ? -__builtin_inff() : (mnew + kRescaleSlack) * inv_scale;
    }
    return alpha;
  };
  // V^T operand of PV MFMA f of key half hf (as attn_mfma.hip's read_v).
  auto read_v = [=](const unsigned char* vbuf, uint32_t va, uint32_t vb1, int f) __attribute__((always_inline)) {
    const int sub = f / (D / 32), i = f % (D / 32);
    const unsigned char* p0 = vbuf + (va ^ uint32_t(64 * i)) + sub * 16 * kPRowBytes;
    const unsigned char* p1 = vbuf + (vb1 ^ uint32_t(64 * i)) + sub * 16 * kPRowBytes;
    const s16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) s16x4_t*)(p0));
    const s16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) s16x4_t*)(p1));
    const s16x4_t both[2] = {lo, hi};
    return __builtin_bit_cast(vec, both);
  };

  // ---- pipeline ------------------------------------------------------------
  // Operand i of the stream (o_2t = K(t), o_2t+1 = V(t)) sits in slot i % 3.
  // Step i waits until o_i has landed (the H copies of o_i+1 stay in
  // flight), passes a barrier (every wave is done with o_i-1), issues the
  // copies of o_i+2 into o_i-1's slot and computes on o_i.  Ids: every W
  // tiles each wave stages one of tiles t+W .. t+2W-1; the ids of tile u are
  // first read at step K(u-1).
  lds_barrier();  // run_sv written
  if (ntiles > 0) {
    stage_ids(wave, wave);  // tiles 0 .. W-1
    vm_lds_barrier();
    uint64_t pr[H];
    copy_pairs(0, tile_of(0).lim, pr);
    static_for<H>([&](auto x) __attribute__((always_inline)) { copy_op(lds_off<0>{}, x, false, pr[x]); });
    static_for<H>([&](auto x) __attribute__((always_inline)) { copy_op(lds_off<TB>{}, x, true, pr[x]); });
  }
  auto step = [&](int t, auto r_tag) __attribute__((always_inline)) {
    constexpr int r = decltype(r_tag)::value;
    constexpr uint32_t k_this = uint32_t((2 * r) % 3) * TB;
    constexpr uint32_t v_this = uint32_t((2 * r + 1) % 3) * TB;
    constexpr uint32_t k_next = uint32_t((2 * r + 2) % 3) * TB;
    constexpr uint32_t v_next = k_this;
    // ---- K(t): S(t) = QK(t) over both key halves and its softmax; copies of K(t+1)
    vm_lds_barrier_keep<H>();  // K(t) landed; every wave is done with V(t-1)
    if (t % W == 0) {
      const int u = t + W + wave;
      stage_ids(u, u % kPIdSlots);
    }
    const Tile tl = tile_of(t);
    const bool mine = wave_rows && (lst == 0 ? tl.in_a : tl.in_b);
    const bool diag = lst == 0 ? tl.diag_a : tl.diag_b;
    const int lim_next = tile_of(t + 1).lim;
    const int slot_next = (t + 1) % kPIdSlots;
    vec bfrag[2][2];  // probabilities of key half hf, keys 16sub .. 16sub+15
    {  // copies of K(t+1), issued before the MFMAs (their pairs then hold no registers there)
      uint64_t cpr[H];
      copy_pairs(slot_next, lim_next, cpr);
      static_for<H>([&](auto c) __attribute__((always_inline)) { copy_op(lds_off<k_next>{}, c, false, cpr[c]); });
    }
    if (mine) {
      uint32_t kx = k0;
      asm volatile("" : "+v"(kx));
      const unsigned char* kb = smem + k_this;
      auto kread = [=](int hf, int st) __attribute__((always_inline)) {  // K operand of QK MFMA (half hf, feature step st)
        return __builtin_bit_cast(vec, *reinterpret_cast<const uint4*>(
                                           kb + hf * (32 * kPRowBytes) + (kx ^ uint32_t(32 * st))));
      };
      // One 32-key half at a time: S = QK, mask, maximum, probabilities.  A
      // half that moves the running maximum rescales the probabilities the
      // first half already holds (rare).
      auto half = [&](auto hf_tag) __attribute__((always_inline)) {
        constexpr int hf = decltype(hf_tag)::value;
        f32x16_t sc;
#pragma unroll
        for (int e = 0; e < 16; ++e) sc[e] = 0.f;
        vec a0 = kread(hf, 0), a1;
        __builtin_amdgcn_s_setprio(2);
#pragma unroll
        for (int st = 0; st < NQK; ++st) {
          __builtin_amdgcn_sched_barrier(0);
          if (st + 1 < NQK) a1 = kread(hf, st + 1);
          sc = M::run(a0, qreg[st], sc);
          a0 = a1;
        }
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(0);
        if (tl.lim < kTileKeys || diag) {  // slots past the valid ones, the causal diagonal
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int slot = 32 * hf + 8 * (e / 4) + 4 * hh + (e % 4);
            const bool ok = (slot < tl.lim) & (!diag | (slot <= qrow_local));
            sc[e] = ok ? sc[e] : -__builtin_inff();
          }
        }
        float tmax = -__builtin_inff();
#pragma unroll
        for (int e = 0; e < 16; e += 2) tmax = max3_plain(tmax, sc[e], sc[e + 1]);
        const float alpha = rescale(tmax);
        if constexpr (hf == 1) {
          if (__builtin_amdgcn_ballot_w64(alpha != 1.f)) {  // rare: rescale half 0
#pragma unroll
            for (int sub = 0; sub < 2; ++sub) {
              float x[8];
#pragma unroll
              for (int e = 0; e < 8; ++e) x[e] = float(bfrag[0][sub][e]) * alpha;
              bfrag[0][sub] = M::pack(x);
            }
          }
        }
        float pr[16];
#pragma unroll
        for (int e = 0; e < 16; ++e)
          pr[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[e], scale_log2, mneg));
        bfrag[hf][0] = M::pack(pr);
        bfrag[hf][1] = M::pack(pr + 8);
      };
      half(std::integral_constant<int, 0>{});
      half(std::integral_constant<int, 1>{});
    }
    // ---- V(t): PV(t) and the row sums of P(t); copies of V(t+1)
    vm_lds_barrier_keep<H>();  // V(t) landed; every wave is done with K(t)
    {
      uint64_t cpr[H];
      copy_pairs(slot_next, lim_next, cpr);
      static_for<H>([&](auto c) __attribute__((always_inline)) { copy_op(lds_off<v_next>{}, c, true, cpr[c]); });
    }
    if (mine) {
      uint32_t va = v0[0], vb1 = v0[1];
      asm volatile("" : "+v"(va), "+v"(vb1));
      const unsigned char* vb = smem + v_this;
      auto vread = [=](int f) __attribute__((always_inline)) {  // V^T operand of PV MFMA f (half f / NPV)
        return read_v(vb + (f / NPV) * (32 * kPRowBytes), va, vb1, f % NPV);
      };
      vec f0 = vread(0), f1;
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int f = 0; f < 2 * NPV; ++f) {
        __builtin_amdgcn_sched_barrier(0);
        if (f + 1 < 2 * NPV) f1 = vread(f + 1);
        const int hf = f / NPV, fl = f % NPV;
        const int sub = fl / (D / 32), i = fl % (D / 32);
        o[i] = M::run(f0, bfrag[hf][sub], o[i]);
        f0 = f1;
#pragma unroll
        for (int j = fl * 8 / NPV; j < (fl + 1) * 8 / NPV; ++j)
          lsum = M::add_pair(bfrag[hf][j / 4], j % 4, lsum);
      }
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_setprio(0);
    }
  };
  for (int t = 0; t < ntiles; t += 3) {
    step(t, std::integral_constant<int, 0>{});
    if (t + 1 < ntiles) step(t + 1, std::integral_constant<int, 1>{});
    if (t + 2 < ntiles) step(t + 2, std::integral_constant<int, 2>{});
  }
  vm_lds_barrier();  // the last copies have landed before the work-group ends

#undef VA_PAIR_WALK

  // ---- normalise and store (each wave owns whole rows) ----------------------
  const float l = sum_halves(lsum);
  const float inv = l > 0.f ? 1.f / l : 0.f;
  if (!wave_rows || qpos >= Sq) return;
  T* orow = out + b * sob + h * soh + qpos * sos;
#pragma unroll
  for (int i = 0; i < D / 32; ++i)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d0 = i * 32 + 8 * g + 4 * hh;
      const T e0 = Round<T>::store(o[i][4 * g + 0] * inv);
      const T e1 = Round<T>::store(o[i][4 * g + 1] * inv);
      const T e2 = Round<T>::store(o[i][4 * g + 2] * inv);
      const T e3 = Round<T>::store(o[i][4 * g + 3] * inv);
      uint2 w;
      w.x = uint32_t(e0.bits) | (uint32_t(e1.bits) << 16);
      w.y = uint32_t(e2.bits) | (uint32_t(e3.bits) << 16);
      *reinterpret_cast<uint2*>(orow + d0) = w;
    }
}

bool attn_pair_supported(int dtype, int64_t D, int64_t qps) {
  return (dtype == kBF16 || dtype == kF16) && D == kPD && qps == kPQ;
}

template <typename T>
static hipError_t launch_attn_pair_t(const void* q, const int64_t* sq, const void* k,
                                     const int64_t* sk, const void* v, const int64_t* sv,
                                     void* out, const int64_t* so, int64_t B, int64_t Hq,
                                     int64_t Hk, int64_t Sq, int64_t Sk, int causal,
                                     float scale_log2, const int32_t* counts,
                                     const int32_t* pcommon, const int32_t* indices,
                                     const RowLayout& lay, int nseg, int segk,
                                     hipStream_t stream) {
  const int64_t npairs = (lay.nc + 1) / 2;
  const int64_t nblocks = WorkOrder{npairs, B, Hq, Hk, causal == 0}.grid_items();
  hipLaunchKernelGGL(attn_pair_kernel<T>, dim3(unsigned(nblocks)), dim3(64 * kPWaves), 0, stream,
                     static_cast<const T*>(q), sq[0], sq[1], sq[2], static_cast<const T*>(k),
                     sk[0], sk[1], sk[2], static_cast<const T*>(v), sv[0], sv[1], sv[2],
                     static_cast<T*>(out), so[0], so[1], so[2], B, Hq, Hk, Sq, Sk, causal,
                     scale_log2, counts, pcommon, indices, lay, nseg, segk);
  return hipGetLastError();
}

hipError_t launch_attn_pair(int dtype, const void* q, const int64_t* sq, const void* k,
                            const int64_t* sk, const void* v, const int64_t* sv, void* out,
                            const int64_t* so, int64_t B, int64_t Hq, int64_t Hk, int64_t Sq,
                            int64_t Sk, int causal, float scale_log2, const int32_t* counts,
                            const int32_t* pcommon, const int32_t* indices, const RowLayout& lay,
                            int nseg, int segk, hipStream_t stream) {
  if (dtype == kBF16)
    return launch_attn_pair_t<bf16_t>(q, sq, k, sk, v, sv, out, so, B, Hq, Hk, Sq, Sk, causal,
                                      scale_log2, counts, pcommon, indices, lay, nseg, segk,
                                      stream);
  if (dtype == kF16)
    return launch_attn_pair_t<f16_t>(q, sq, k, sk, v, sv, out, so, B, Hq, Hk, Sq, Sk, causal,
                                     scale_log2, counts, pcommon, indices, lay, nseg, segk,
                                     stream);
  return hipErrorInvalidValue;
}

}  // namespace va
