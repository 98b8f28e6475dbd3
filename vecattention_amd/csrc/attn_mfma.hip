// Vector-sparse flash-attention prefill on CDNA4 (gfx950) bf16/fp16 MFMA.
//
// Replaces vllm_flash_attn.sparse_attn_func as called at
// spattn/src/VecAttention.py:110-121 (semantics restated from
// spattn/threshold/model_tuner.py:193-216; see keylist.h).  One work-group
// owns one q-block (QPS rows) of one q head and walks that block's key list in
// tiles of 64 keys.  GQA is native: q head h reads kv head h / (Hq / Hk).
//
// Data movement.  The K and V rows of a tile are gathered straight into LDS
// with buffer_load_dwordx4 ... lds (no register staging, no LDS stores): each
// copy instruction fills 1 KB of LDS, lane i writing bytes [16i, 16i+16), and
// each lane chooses which 16-byte chunk of which key row it fetches.  Empty
// slots of a tile and keys outside [0, Sk) use an offset past the buffer's
// range, which the hardware returns as zeros.  Rows are stored with an XOR
// swizzle of their 16-byte chunks (chunk c of row R sits at c ^ swizzle(R))
// so that the MFMA operand reads below are free of bank conflicts.  Two LDS
// stages: the copies of tile t+1 are in flight while tile t is computed, and a
// single barrier per tile separates them.  Key ids are staged in LDS ahead of
// their copies (copied from the index list, or generated for the local
// blocks), all waves together once every kWaves tiles, one tile per wave, so
// that no wave carries the staging work alone into every barrier.
//
// Compute.  Waves form a (row half, key half) grid: wave (rh, kc) owns query
// rows [32rh, 32rh+32) and keys [32kc, 32kc+32) of every tile, with its own
// online-softmax state; the two key halves are merged once at the end.
// S^T = K Q^T uses v_mfma_f32_32x32x16 with A = K rows from LDS and B = Q^T
// held in VGPRs, so a lane holds one query and 16 keys: the row maximum is an
// in-lane reduction plus one v_permlane32_swap.  The probabilities feed
// O^T += V^T P^T directly as the B operand (the accumulator's key order is a
// valid k-slot order), and the V^T operand is read from the row-major V tile
// with ds_read_b64_tr_b16, which transposes 16-bit elements across each group
// of 16 lanes.  The running maximum is only moved when a tile's maximum
// exceeds it by more than 2^8 in probability, so the O rescale (D/2 multiplies
// per lane) is rare; probabilities stay below 2^8, far inside fp32 and
// bf16/fp16 range, and O / l is unchanged by the choice of reference maximum.
//
// Algorithmic work per gathered key: 4*D FLOPs per query row (QK^T and PV).
#include <type_traits>
#include <utility>

#include "keylist.h"
#include "lanes.h"
#include "mfma.h"

namespace va {

constexpr int kTileKeys = 64;
constexpr int kMaxSegments = 64;  // key segments of a split selection (a wave's lanes)
constexpr uint32_t kOutOfRange = 0xfffffff0u;  // voffset past every buffer's range
constexpr float kRescaleSlack = 8.f;           // log2 of the largest kept probability

typedef short s16x4_t __attribute__((ext_vector_type(4)));

// f(std::integral_constant<int, i>) for i = 0 .. N-1, in order.
template <typename F, int... I>
__device__ inline void static_for_impl(F& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ inline void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}
template <uint32_t V>
using lds_off = std::integral_constant<uint32_t, V>;

template <int D, int QPS, bool kRing3 = false, bool kStats = false>
struct AttnShape {
  static constexpr int kRowHalves = QPS / 32;
  static constexpr int kWaves = 2 * kRowHalves;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int kRowBytes = 2 * D;
  static constexpr int kChunks = D / 8;                      // 16-byte chunks per row
  static constexpr int kTileBytes = kTileKeys * kRowBytes;   // one K (or V) tile
  // K tile, then V tile (the statistics form reads no V: K tile only)
  static constexpr int kStageBytes = (kStats ? 1 : 2) * kTileBytes;
  static constexpr int kRowsPerCopy = 1024 / kRowBytes;      // rows per 1 KB copy
  static constexpr int kCopiesPerWave = kTileBytes / 1024 / kWaves;  // per operand
  // Epilogue: half of each row half's partial output and its (m, l) per
  // wave, or (statistics form) the (m, l) of each row half only.
  static constexpr int kMergeBytes =
      kStats ? kRowHalves * 128 * 4 : kRowHalves * 64 * (D / 2 + 4) * 4;
  // Two stages of a K and a V tile, or (kRing3) a ring of three tile slots.
  static constexpr int kRingBytes = kRing3 ? 3 * kTileBytes : 2 * kStageBytes;
  static constexpr int kDataBytes = kRingBytes > kMergeBytes ? kRingBytes : kMergeBytes;
  // Key ids: a ring of 2 * kWaves tile slots; every kWaves tiles each wave
  // stages the ids of one tile kWaves to 2 * kWaves - 1 tiles ahead.
  static constexpr int kIdSlots = 2 * kWaves;
  static constexpr int kLdsBytes = kDataBytes + kIdSlots * kTileKeys * 4;
  static_assert(kCopiesPerWave >= 1 && kRowsPerCopy * kCopiesPerWave * kWaves == kTileKeys,
                "tile copies must split evenly over the waves");
};

// XOR swizzle of the 16-byte chunks of tile row R.  The LDS serves 256 bytes
// per clock from 64 four-byte banks: a ds_read_b128 is served 16 lanes at a
// time, a ds_read_b64_tr_b16 32 lanes at a time.  Rows R and R + 256 / (2D)
// start on the same bank, so m = (R * 2D / 256) mod NCH numbers the rows of a
// 256-byte bank period, and the swizzle is m with its bits rotated right by
// log2(NCH) - 2:
//  - the K reads (16 consecutive rows, one logical chunk) need m -> swizzle
//    to be a bijection, which any rotation is;
//  - the V^T reads (rows R0 + j, j < 4, R0 % 4 == 0, logical chunks 4i + g,
//    g < 4) need the four rows to differ in swizzle bits 2.., which the
//    rotation gives by moving the low bits of m there.
template <int D>
__device__ inline int chunk_swizzle(int R) {
  constexpr int NCH = D / 8;
  if constexpr (NCH == 16) {
    const int m = R % 16;
    return ((m & 3) << 2) | (m >> 2);
  } else {
    static_assert(NCH == 8, "D must be 64 or 128");
    const int m = (R / 2) % 8;
    return ((m & 1) << 2) | (m >> 1);
  }
}

// Per-tile facts shared by the copy and the compute of a tile: number of
// valid slots, and for diagonal tiles the offset of slot 0 from the first
// diagonal key.
struct TileInfo {
  int lim;
  int dshift;
  bool diag;
};

// kDense: every key of the block's rows (dense attention, causal offset
// dense_qoff) instead of the local blocks and the selected columns; a
// separate instantiation, so that the sparse kernel's code does not carry
// the general key-span arithmetic.
// kStats: the row's softmax statistics instead of the attention output: no
// V copies and no PV products; the row sums add the fp32 probabilities (not
// their bf16/fp16 roundings), and row i of head bh gets
// stats[(bh * Sq + i) * 2 + {0, 1}] = (m, l) with l = sum over its keys of
// 2^(s * scale_log2 - m), s the raw score (m = -inf, l = 0 without keys).
// kSplit: split key ranges (decode): block row J holds keys [J*span,
// (J+1)*span) of the K/V rows, span passed in dense_qoff, for the same query
// rows [0, Sq) in every J (no causal mask); each (bh, J) writes its rows'
// normalised partial output and (m, l) in fp32 to stats, row-major over
// (bh, i, J) so that the partials of one row are contiguous: (m, l) of row i
// at stats[((bh * Sq + i) * nc + J) * 2], the output after all of them (from
// the next multiple of 4 floats, P = ceil(2 * B * Hq * nc * Sq / 4) * 4), at
// stats + P + ((bh * Sq + i) * nc + J) * D.
// QPS * 4 threads (kThreads); three waves per SIMD for the ring form and at
// D = 64, two otherwise.
template <typename T, int D, int QPS, bool kDense, bool kStats, bool kSplit, bool kRing3>
__global__ __launch_bounds__(QPS * 4, (kRing3 || D == 64) ? 3 : 2) void attn_mfma_kernel(
    const T* __restrict__ q, int64_t sqb, int64_t sqh, int64_t sqs,
    const T* __restrict__ k, int64_t skb, int64_t skh, int64_t sks,
    const T* __restrict__ v, int64_t svb, int64_t svh, int64_t svs,
    T* __restrict__ out, int64_t sob, int64_t soh, int64_t sos, int64_t B,
    int64_t Hq, int64_t Hk, int64_t Sq, int64_t Sk, int causal, float scale_log2,
    const int32_t* __restrict__ counts, const int32_t* __restrict__ indices,
    RowLayout lay, int nseg, int segk, int64_t dense_qoff, float* __restrict__ stats) {
  using S = AttnShape<D, QPS, kRing3, kStats>;
  static_assert(!kRing3 || (!kDense && !kStats && !kSplit), "the ring form is the sparse kernel's");
  using M = Mfma<T>;
  using vec = typename M::vec;
  constexpr int NCH = S::kChunks;
  constexpr int RPC = S::kRowsPerCopy;
  constexpr int H = S::kCopiesPerWave;

  __shared__ __attribute__((aligned(1024))) unsigned char smem[S::kLdsBytes];
  int32_t* const ids = reinterpret_cast<int32_t*>(smem + S::kDataBytes);  // [kIdSlots][64]

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid / 64), lane = tid % 64;
  const int l32 = lane % 32, hh = lane / 32;
  const int rh = wave % S::kRowHalves, kc = wave / S::kRowHalves;

  const WorkOrder wo{lay.nc, B, Hq, Hk, causal == 0};
  int jr32, bh32;
  if (!wo.map_item32(blockIdx.x, jr32, bh32)) return;  // idle block (uniform)
  const int64_t jr = jr32, bh = bh32;
  const uint32_t hq32 = uint32_t(Hq);  // 32-bit: every index is below 2^31
  const int64_t b = uint32_t(bh32) / hq32, h = uint32_t(bh32) % hq32;
  const int64_t hk = uint32_t(h) / (hq32 / uint32_t(Hk));
  const int64_t J = lay.J0 + jr;

  // Segment counts of the row (lane s: segment s), loaded ahead of Q: the
  // wait counter retires loads in issue order, so the scan below then waits
  // for these alone and not for the Q rows too.
  // A buffer load without a branch (lanes past nseg, and every lane when the
  // row has a single count, read past the range and get 0), so that the wait
  // counter's bookkeeping sees it issued before the Q rows on every path.
  const bool seg_counts = counts != nullptr && nseg > 1;
  const int c_seg = int(__builtin_amdgcn_raw_buffer_load_b32(
      make_rsrc(seg_counts ? counts + (bh * lay.nc + jr) * nseg : counts,
                seg_counts ? uint32_t(nseg) * 4u : 0u),
      lane * 4, 0, 0));

  // ---- Q^T operand: lane holds row 32rh + l32, features [16s + 8hh, +8) ----
  // (loads issued early; their latency overlaps the list bookkeeping below)
  const int qrow_local = 32 * rh + l32;
  const int64_t qpos = (kSplit ? 0 : J * QPS) + qrow_local;
  vec qreg[D / 16];
  {
    // Rows past Sq load row Sq - 1: no branch around the loads and nothing
    // consumes them before the first QK^T.  Those rows' results are never
    // written (every epilogue form skips qpos >= Sq).
    const T* qr_ptr = q + b * sqb + h * sqh + (qpos < Sq ? qpos : Sq - 1) * sqs;
#pragma unroll
    for (int s = 0; s < D / 16; ++s)
      qreg[s] = __builtin_bit_cast(vec, *reinterpret_cast<const uint4*>(qr_ptr + 16 * s + 8 * hh));
  }

  // Selected columns.  With nseg > 1 the row's list comes in key segments:
  // segment s holds counts[.., s] keys from slot max(s*segk, smin) - smin of
  // the row (see select_wave.hip).  Lane s of every wave keeps sv = the
  // exclusive prefix of the segment counts (the column where segment s
  // starts), so column p of the concatenated list is slot seg_slot(s) + p -
  // sv[s] for the last s with sv[s] <= p.
  int sv = 0x7fffffff;
  const int64_t cap = lay.capacity(J);
  const int smin = int(lay.smin());
  auto seg_slot = [&](int sg) { return (sg * segk > smin ? sg * segk : smin) - smin; };
  int64_t cnt = 0;
  if (counts && nseg <= 1) {
    cnt = counts[bh * lay.nc + jr];
  } else if (counts) {  // whole wave: the scan exchanges lanes
    int c = 0;
    if (lane < nseg) {
      c = c_seg;
      const int room = int(cap) - seg_slot(lane);
      c = c < 0 ? 0 : (c > room ? (room > 0 ? room : 0) : c);
    }
    const int incl = wave_inclusive_sum(c);
    if (lane < nseg) sv = incl - c;
    cnt = __builtin_amdgcn_readlane(incl, nseg - 1);
  }
  if (cnt > cap) cnt = cap;
  const int32_t* cols = indices ? indices + lay.row_offset(bh, jr) : nullptr;
  KeyList kl;
  if constexpr (kSplit)
    kl = KeyList::split(J, dense_qoff, Sk);
  else if constexpr (kDense)
    kl = KeyList::dense(J, QPS, Sk, causal, dense_qoff);
  else
    kl = KeyList::make(J, QPS, Sk, causal, cnt, cols);
  // Every count below fits in 32 bits (the host checks Sk < 2^24).
  const int n_init = int(kl.n_init), n_diag = int(kl.n_diag), n_col = int(kl.n_col);
  const int diag0 = int(kl.diag0);
  const int t_init = (n_init + kTileKeys - 1) / kTileKeys;
  const int t_diag = (n_diag + kTileKeys - 1) / kTileKeys;
  const int t_col = (n_col + kTileKeys - 1) / kTileKeys;
  const int ntiles = t_init + t_diag + t_col;
  // The column tiles are walked from a row-dependent tile c_rot on, wrapping
  // around (walk step u visits list tile list_tile(u)): a row dispatched later
  // on an XCD starts further into its list, kRotPeriod rows (about the
  // work-groups an XCD holds at once) spanning the whole list, so that the
  // work-groups running together sit at about the same keys and rows that
  // share keys find them in L2 (128K causal GQA -5%, 119056 non-causal -3% of
  // a chunk's attention).  The rank comes from the absolute row, so every
  // launch and both loop forms walk a row the same way.
  constexpr uint32_t kRotPeriod = 96;
  const int tc0 = t_init + t_diag;
  const int c_rot =
      (kDense || kStats || kSplit || t_col < 2)
          ? 0
          : int(wo.xcd_rank(uint32_t(J), uint32_t(bh32), kRotPeriod) * uint32_t(t_col) /
                kRotPeriod);
  auto list_tile = [&](int u) {
    if (u < tc0) return u;
    const int x = u - tc0 + c_rot;
    return tc0 + (x >= t_col ? x - t_col : x);
  };

  auto tile_info = [&](int t) -> TileInfo {
    TileInfo ti;
    ti.dshift = 0;
    ti.diag = false;
    int l;
    if (t < t_init) {
      l = n_init - t * kTileKeys;
    } else if (t < t_init + t_diag) {
      ti.dshift = (t - t_init) * kTileKeys;
      l = n_diag - ti.dshift;
      ti.diag = causal != 0;
    } else {
      l = n_col - (t - t_init - t_diag) * kTileKeys;
    }
    ti.lim = l > kTileKeys ? kTileKeys : l;
    return ti;
  };

  // ---- buffers -------------------------------------------------------------
  const T* kh = k + b * skb + hk * skh;
  const T* vh = v + b * svb + hk * svh;
  // K and V as Sk records of their row stride: a copy addresses row `key`,
  // and any key outside [0, Sk) reads zeros (the host checks that the
  // strides fit the resource's 14-bit field).
  const __amdgpu_buffer_rsrc_t krs = make_rsrc_rows(kh, uint32_t(sks * 2), uint32_t(Sk));
  const __amdgpu_buffer_rsrc_t vrs = make_rsrc_rows(vh, uint32_t(svs * 2), uint32_t(Sk));
  const __amdgpu_buffer_rsrc_t irs =
      make_rsrc(cols, uint32_t(nseg > 1 ? (cap > 0 ? cap : 0) : n_col) * 4u);

  // Copy geometry.  Copy x of this wave fills rows [(wave*H + x)*RPC, +RPC) of
  // a tile; this lane fetches physical chunk p of row R_x, i.e. logical chunk
  // p ^ chunk_swizzle(R_x).  The H key ids a lane needs sit contiguously in `ids` at
  // position (wave*RPC + qr)*H + x, where qr = lane / NCH.
  const int qr = lane / NCH, pc = lane % NCH;
  uint32_t cchunk[H];
#pragma unroll
  for (int x = 0; x < H; ++x)
    cchunk[x] = uint32_t(16 * (pc ^ chunk_swizzle<D>((wave * H + x) * RPC + qr)));
  const int id_pos = (wave * RPC + qr) * H;
  // Inverse map for the lanes of wave 0 that write ids: position -> slot.
  const int w_slot = [&] {
    const int w = lane / (RPC * H), r = (lane / H) % RPC, x = lane % H;
    return (w * H + x) * RPC + r;
  }();

  // Stage the key ids of tile u into ids[slot] (one wave; each wave stages
  // its tiles in increasing order).  Column positions of the selected list
  // map to index slots through a scalar segment cursor: segment sc holds positions
  // [sv[sc], sc_next) at slots position + sc_base.  Positions only grow from
  // tile to tile, so the cursor moves forward once per segment (empty
  // segments are stepped over), and a tile with no segment boundary inside
  // it costs one add per lane.  Every slot past the key count of a tile, and
  // every slot of a tile past the end of the list, gets key 2^32 - 1: its
  // copies read zeros and move no data.  The slots of the selected columns
  // are copied from the index list, where positions past its end read as 0;
  // copy_pairs replaces those keys in the one partial column tile.
  const int kNoBoundary = 0x7fffffff;
  auto boundary = [&](int sg) {  // start of segment sg, or none
    return sg < nseg ? __builtin_amdgcn_readlane(sv, sg) : kNoBoundary;
  };
  int sc = 0, sc_base = 0, sc_next = nseg > 1 ? boundary(1) : kNoBoundary;
  int sc_last = -1;  // list position of the last column tile this wave staged
  auto stage_ids = [&](int u, int slot) {
    int32_t* dst = ids + slot * kTileKeys;
    if (u >= ntiles) {
      dst[lane] = -1;
    } else if (u < t_init) {
      const int key = u * kTileKeys + w_slot;
      dst[lane] = key < n_init ? key : -1;
    } else if (u < t_init + t_diag) {
      const int d = (u - t_init) * kTileKeys + w_slot;
      dst[lane] = d < n_diag ? diag0 + d : -1;
    } else {
      const int p0 = (list_tile(u) - tc0) * kTileKeys, p = p0 + w_slot;
      if (p0 < sc_last) {  // the walk wrapped to the list's start
        sc = 0;
        sc_base = 0;
        sc_next = nseg > 1 ? boundary(1) : kNoBoundary;
      }
      sc_last = p0;
      while (sc_next <= p0) {  // the tile starts past segment sc
        ++sc;
        sc_base = seg_slot(sc) - sc_next;
        sc_next = boundary(sc + 1);
      }
      int base = sc_base;
      const int pend = (p0 + kTileKeys < n_col ? p0 + kTileKeys : n_col) - 1;  // last position
      if (sc_next <= pend) {  // boundaries inside the tile
        int sg = sc, b = sc_next;
        while (b <= pend) {
          ++sg;
          if (p >= b) base = seg_slot(sg) - b;
          b = boundary(sg + 1);
        }
      }
      const uint32_t off = p < n_col ? uint32_t(p + base) * 4u : kOutOfRange;
      copy4_to_lds(irs, lds_addr(dst), off);
    }
  };

  // Copy addresses of tile u: for each of this lane's H copies, the (row,
  // byte offset) pair of its 16-byte chunk, the row being the key id in ids
  // slot idslot; K and V copies of a tile use the same pairs.  Keys outside
  // [0, Sk) read zeros.  In the partial column tile (one per list, a uniform
  // test), rows past the list's end get key 2^32 - 1.
  const int p_col = n_col % kTileKeys != 0 ? ntiles - 1 : -1;
  // Walk step of the partial column tile (-1: none) and its key count, so
  // that the per-tile tests compare walk steps without mapping them.
  const int u_pcol = __builtin_amdgcn_readfirstlane(p_col < 0 ? -1 : ntiles - 1 - c_rot);
  const int lim_pcol = __builtin_amdgcn_readfirstlane(n_col - (t_col - 1) * kTileKeys);
  auto copy_pairs = [&](int u, int idslot, uint64_t (&pr)[H]) {
    uint32_t key[H];
#pragma unroll
    for (int x = 0; x < H; ++x) key[x] = uint32_t(ids[idslot * kTileKeys + id_pos + x]);
    if (u == u_pcol) {
      const int lim = lim_pcol;
#pragma unroll
      for (int x = 0; x < H; ++x)  // row (wave*H + x)*RPC + qr holds a key below lim
        if (qr >= lim - (wave * H + x) * RPC) key[x] = 0xffffffffu;
    }
#pragma unroll
    for (int x = 0; x < H; ++x) pr[x] = uint64_t(key[x]) | (uint64_t(cchunk[x]) << 32);
  };
  // Copy x of this wave into the K or V tile at LDS offset kBase of the
  // stages (a compile-time constant): M0 = this wave's copy base + offset.
  const uint32_t lds_copy_base =
      uint32_t(__builtin_amdgcn_readfirstlane(int(lds_addr(smem) + uint32_t(wave * H * 1024))));
  auto copy_k = [&](auto base_tag, auto x_tag, uint64_t pr) {
    copy16_row_to_lds_at<decltype(base_tag)::value + decltype(x_tag)::value * 1024u>(
        krs, lds_copy_base, pr);
  };
  auto copy_v = [&](auto base_tag, auto x_tag, uint64_t pr) {
    copy16_row_to_lds_at<decltype(base_tag)::value + decltype(x_tag)::value * 1024u>(
        vrs, lds_copy_base, pr);
  };

  // Wait for Q here: otherwise the compiler places the wait at the first MFMA
  // inside the tile loop, where it would also wait for the K/V copies in flight.
#pragma unroll
  for (int s = 0; s < D / 16; ++s) asm volatile("" ::"v"(qreg[s]));

  // LDS read offsets inside a K or V tile.  K (A operand of S^T): row 32kc + l32,
  // chunk 2s + hh.  V^T (A operand of O^T) via the transposing read: lane
  // group g16 = lane / 16 reads rows 32kc + 16sub + 8r + 4hh + j with
  // j = (lane % 16) / 4, features 32i + 16(g16 % 2) + 4(lane % 4).
  uint32_t koff[D / 16];
#pragma unroll
  for (int s = 0; s < D / 16; ++s) {
    const int R = 32 * kc + l32;
    koff[s] = uint32_t(R * S::kRowBytes + 16 * ((2 * s + hh) ^ chunk_swizzle<D>(R)));
  }
  uint32_t voff[D / 32][2];
  {
    const int j = (lane % 16) / 4, g2 = 2 * ((lane / 16) % 2) + (lane % 4) / 2;
#pragma unroll
    for (int i = 0; i < D / 32; ++i)
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int R = 32 * kc + 8 * r + 4 * hh + j;  // + 16 sub (same swizzle)
        const int c = 4 * i + g2;
        voff[i][r] = uint32_t(R * S::kRowBytes + 16 * (c ^ chunk_swizzle<D>(R)) +
                              8 * (lane % 2));
      }
  }

  f32x16_t o[D / 32];
#pragma unroll
  for (int i = 0; i < D / 32; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[i][e] = 0.f;
  // Online-softmax state of this lane's row: running maximum mc (scaled, log2
  // units), -mc as the exponent offset (0 while no key has been seen), and
  // the raw-score level above which a tile moves the maximum.
  float mc = -__builtin_inff(), mneg = 0.f, thr = -__builtin_inff();
  const float inv_scale = 1.f / scale_log2;  // the host passes scale_log2 > 0
  // Partial row sum of the probabilities of this lane's keys (lanes l and
  // l ^ 32 hold the two halves of row l % 32): dot products of the packed
  // bf16/fp16 probabilities with (1, 1), i.e. the rounded values that also
  // weight V.
  float lsum = 0.f;

  // S^T of one tile: 8 (D/16) MFMAs with K rows from the K slot at kbuf.
  auto qk = [&](const unsigned char* kbuf) {
    f32x16_t s;
#pragma unroll
    for (int e = 0; e < 16; ++e) s[e] = 0.f;
#pragma unroll
    for (int st = 0; st < D / 16; ++st) {
      const vec a = __builtin_bit_cast(vec, *reinterpret_cast<const uint4*>(kbuf + koff[st]));
      s = M::run(a, qreg[st], s);
    }
    return s;
  };
  // Mask the scores of walk step u: empty slots, the causal diagonal, every
  // slot of a step past the end of the list.  Slot of s[e]: 32kc + 8(e/4) +
  // 4hh + e%4.  Steps that may need masking, found with three comparisons:
  // [m_lo, m_lo + m_span) holds the partial last tile of the initial blocks
  // and the diagonal tiles, u_pcol is the partial column tile, and steps from
  // ntiles on lie past the end of the list.
  const int m_lo = __builtin_amdgcn_readfirstlane(t_init - (n_init % kTileKeys != 0 ? 1 : 0));
  const uint32_t m_span = uint32_t(__builtin_amdgcn_readfirstlane(t_init + t_diag - m_lo));
  auto mask = [&](int u, f32x16_t& s) {
    // uniform: a full column tile (the staged pipeline also scores the step
    // past the last tile, whose slots are all masked)
    if (uint32_t(u - m_lo) >= m_span && u != u_pcol && u < ntiles) return;
    const TileInfo ti = tile_info(u < ntiles ? list_tile(u) : u);
    if (ti.diag || ti.lim < kTileKeys) {  // rare: partial, diagonal or empty tiles
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int slot = 32 * kc + 8 * (e / 4) + 4 * hh + (e % 4);
        const bool ok = (slot < ti.lim) & (!ti.diag | (ti.dshift + slot <= qrow_local));
        s[e] = ok ? s[e] : -__builtin_inff();
      }
    }
  };
  // Move the running maximum when some row's tile maximum exceeds it by more
  // than the slack (rare): rescale O and the row sums.  The test compares raw
  // scores with thr = (mc + slack) / scale; its rounding only moves the
  // bound on the kept probabilities by a few ulps of 2^8.
  // tmax is this lane's maximum over its 16 keys: a row moves when either of
  // its two lanes exceeds thr, and only then is the row's maximum formed.
  auto rescale = [&](float tmax) {
    if (__builtin_amdgcn_ballot_w64(tmax > thr)) {
      tmax = max_halves(tmax);
      const float mnew = __builtin_fmaxf(mc, tmax * scale_log2);
      const float alpha = (mnew == mc) ? 1.f : __builtin_amdgcn_exp2f(mc - mnew);
#pragma unroll
      for (int i = 0; i < D / 32; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[i][e] *= alpha;  // dead code under kStats
      lsum *= alpha;
      mc = mnew;
      const bool none = mnew == -__builtin_inff();
      mneg = none ? 0.f : -mnew;
      thr = none ? -__builtin_inff() : (mnew + kRescaleSlack) * inv_scale;
    }
  };
  // O^T += V^T P^T in NPV MFMAs, 16 keys each: MFMA f = sub * (D/32) + i
  // adds keys 32kc + 16sub + .. into output block i; k-slot 8hh + e of step
  // sub is key 32kc + 16sub + 8(e/4) + 4hh + e%4, i.e. accumulator entries
  // 8sub .. 8sub+7.  read_v fetches MFMA f's V^T operand from the V tile at
  // vbuf (issued ahead of its use), pv_mfma runs it.
  constexpr int NPV = D / 16;
  auto read_v = [&](const unsigned char* vbuf, int f) {
    const int sub = f / (D / 32), i = f % (D / 32);
    const unsigned char* p0 = vbuf + voff[i][0] + sub * 16 * S::kRowBytes;
    const unsigned char* p1 = vbuf + voff[i][1] + sub * 16 * S::kRowBytes;
    const s16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) s16x4_t*)(p0));
    const s16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) s16x4_t*)(p1));
    const s16x4_t both[2] = {lo, hi};
    return __builtin_bit_cast(vec, both);
  };
  auto pv_mfma = [&](int f, const vec& vf, const vec (&bfrag)[2]) {
    const int sub = f / (D / 32), i = f % (D / 32);
    o[i] = M::run(vf, bfrag[sub], o[i]);
  };

  // ---- pipeline ------------------------------------------------------------
  // LDS slots: K(u) in K slot u&1, V(u) in V slot u&1 (slot p of K at
  // p * kStageBytes, of V kTileBytes after it), key ids of tile u in ids slot
  // u % kIdSlots.  Iteration t has two halves, each opened by a barrier:
  //  - first half (K(t+1) landed): S(t+1) = QK(t+1) next to the softmax of
  //    S(t); the copies of V(t+1) go out between the QK MFMAs;
  //  - second half (V(t) landed; every wave is done with K(t+1)): PV(t) next
  //    to the masking and maximum of S(t+1); the copies of K(t+3) go into the
  //    K slot QK(t+1) just read.
  // Each copy thus has one and a half tiles to land, and a barrier leaves
  // the 2H most recent copies of the wave in flight.  Iterations t = 0 mod W
  // stage the ids of tiles t+W .. t+2W-1, first read (for the copies of
  // K(t+W)) at iteration t+W-3 > t, and written over 2W tiles later, after
  // their last read.  Copies are spread over the MFMAs (one DMA instruction
  // after an MFMA), so that a copy that waits for room in the memory pipeline
  // overlaps the matrix work already issued.
  constexpr int NQK = D / 16;  // QK MFMAs per tile
  f32x16_t s_cur;              // masked scores of tile t
  constexpr int W = S::kWaves;
  // Copies a wave may leave in flight at a barrier: the K and V copies of the
  // tiles ahead (K only under kStats, where the copies of tile t+1 are
  // K(t+1) and K(t+2)).
  constexpr int kKeep = kStats ? H : 2 * H;
  if constexpr (kRing3) {
    // Ring of three tile slots (three work-groups fit a CU's LDS): operand
    // o_i (o_2t = K(t), o_2t+1 = V(t)) sits in slot i % 3.  Step i waits until
    // o_i has landed (the H copies of o_i+1 stay in flight), passes a barrier
    // (every wave is done with o_i-1), issues the copies of o_i+2 into the
    // slot of o_i-1 and computes on o_i, so each copy has one tile to land.
    // A wave runs QK(t), the softmax of S(t) and PV(t) in order, without the
    // two score sets of the staged pipeline: the other waves of its SIMD fill
    // its waits.  Iteration t % 3 fixes the slots, so the loop runs three
    // tiles per trip with compile-time LDS offsets.  Ids: as the staged
    // pipeline (every W tiles each wave stages one of tiles t+W .. t+2W-1);
    // the ids of tile u are first read at step K(u-1), at least W-1 tiles
    // after they were staged.
    // Registers (three waves per SIMD allow 168): the operand offsets are
    // rebuilt from one base per operand each step instead of being kept.  At
    // D = 128 the swizzle only flips offset bits that the feature step owns:
    // koff[s] = koff[0] ^ 32s, voff[i][r] = voff[0][r] ^ 64i, and the chunk
    // offset of copy x is cchunk[0] ^ 16x (rows (4 wave + x) * 4 + qr have
    // swizzle 4qr + x).  Each base passes through an empty asm per step so
    // that the compiler does not hoist the eight offsets out of the loop.
    static_assert(D == 128 && S::kRowsPerCopy == 4 && H == 4, "offset identities assume D = 128");
    constexpr uint32_t TB = uint32_t(S::kTileBytes);
    const uint32_t k0 = koff[0], v00 = voff[0][0], v01 = voff[0][1], c0 = cchunk[0];
    auto copy_pairs3 = [&](int u, int idslot, uint32_t cbase, uint64_t (&pr)[H]) {
      uint32_t key[H];
#pragma unroll
      for (int x = 0; x < H; ++x) key[x] = uint32_t(ids[idslot * kTileKeys + id_pos + x]);
      if (u == u_pcol) {
        const int lim = lim_pcol;
#pragma unroll
        for (int x = 0; x < H; ++x)
          if (qr >= lim - (wave * H + x) * RPC) key[x] = 0xffffffffu;
      }
#pragma unroll
      for (int x = 0; x < H; ++x) pr[x] = uint64_t(key[x]) | (uint64_t(cbase ^ (16u * x)) << 32);
    };
    auto read_v3 = [&](const unsigned char* vbuf, uint32_t va, uint32_t vb1, int f) {
      const int sub = f / (D / 32), i = f % (D / 32);
      const unsigned char* p0 = vbuf + (va ^ uint32_t(64 * i)) + sub * 16 * S::kRowBytes;
      const unsigned char* p1 = vbuf + (vb1 ^ uint32_t(64 * i)) + sub * 16 * S::kRowBytes;
      const s16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) s16x4_t*)(p0));
      const s16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) s16x4_t*)(p1));
      const s16x4_t both[2] = {lo, hi};
      return __builtin_bit_cast(vec, both);
    };
    if (ntiles > 0) {
      stage_ids(wave, wave);  // tiles 0 .. W-1
      // Tile 0's ids are LDS writes when it is a local block; column-id
      // copies of later tiles are covered by the waits of the first steps.
      if (t_init + t_diag >= 1)
        lds_barrier();
      else
        vm_lds_barrier();
      uint64_t pr[H];
      copy_pairs(0, 0, pr);
      static_for<H>([&](auto x) { copy_k(lds_off<0>{}, x, pr[x]); });
      static_for<H>([&](auto x) { copy_v(lds_off<TB>{}, x, pr[x]); });
    }
    auto step = [&](int t, auto r_tag) {
      constexpr int r = decltype(r_tag)::value;
      constexpr uint32_t k_this = uint32_t((2 * r) % 3) * TB;
      constexpr uint32_t v_this = uint32_t((2 * r + 1) % 3) * TB;
      constexpr uint32_t k_next = uint32_t((2 * r + 2) % 3) * TB;
      constexpr uint32_t v_next = k_this;
      // ---- K(t): S(t) = QK(t), its softmax; copies of K(t+1)
      vm_lds_barrier_keep<H>();  // K(t) landed; every wave is done with V(t-1)
      if (t % W == 0) {
        const int u = t + W + wave;
        stage_ids(u, u % S::kIdSlots);
      }
      uint32_t kx = k0, cx = c0;
      asm volatile("" : "+v"(kx), "+v"(cx));
      uint64_t cpr[H];  // tile t+1's copy pairs: K(t+1) here, V(t+1) at the V step
      copy_pairs3(t + 1, (t + 1) % S::kIdSlots, cx, cpr);
      const unsigned char* kb = smem + k_this;
      constexpr int kAhead = 2, kVAhead = 2;
      vec a[NQK];
#pragma unroll
      for (int st = 0; st < kAhead; ++st)
        a[st] = __builtin_bit_cast(vec,
                                   *reinterpret_cast<const uint4*>(kb + (kx ^ uint32_t(32 * st))));
      f32x16_t sc;
#pragma unroll
      for (int e = 0; e < 16; ++e) sc[e] = 0.f;
      // Issue priority by phase (s_setprio, per wave): the QK(t) chain
      // highest, then PV(t), the softmax lowest, so that a SIMD's three waves
      // hand the matrix pipe to whichever wave has MFMAs ready and fill the
      // gaps with softmax work (same-box A/B: 32K -3 to -5%, 128K -1.5%).
      __builtin_amdgcn_s_setprio(2);
#pragma unroll
      for (int st = 0; st < NQK; ++st) {
        __builtin_amdgcn_sched_barrier(0);
        if (st + kAhead < NQK)
          a[st + kAhead] = __builtin_bit_cast(
              vec, *reinterpret_cast<const uint4*>(kb + (kx ^ uint32_t(32 * (st + kAhead)))));
        sc = M::run(a[st], qreg[st], sc);
        static_for<H>([&](auto c) {  // copy c goes out after MFMA c * NQK / H
          if (c * NQK / H == st) copy_k(lds_off<k_next>{}, c, cpr[c]);
        });
      }
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_setprio(0);
      mask(t, sc);
      float tmax = -__builtin_inff();
#pragma unroll
      for (int e = 0; e < 16; e += 2) tmax = max3_plain(tmax, sc[e], sc[e + 1]);
      rescale(tmax);
      float pr[16];
#pragma unroll
      for (int e = 0; e < 16; ++e)
        pr[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[e], scale_log2, mneg));
      const vec bfrag[2] = {M::pack(pr), M::pack(pr + 8)};
      // ---- V(t): PV(t) with the row sums of P(t); copies of V(t+1)
      vm_lds_barrier_keep<H>();  // V(t) landed; every wave is done with K(t)
      uint32_t va = v00, vb1 = v01;
      asm volatile("" : "+v"(va), "+v"(vb1));
      const unsigned char* vb = smem + v_this;
      vec vf[NPV];
#pragma unroll
      for (int f = 0; f < kVAhead; ++f) vf[f] = read_v3(vb, va, vb1, f);
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int f = 0; f < NPV; ++f) {
        __builtin_amdgcn_sched_barrier(0);
        if (f + kVAhead < NPV) vf[f + kVAhead] = read_v3(vb, va, vb1, f + kVAhead);
        pv_mfma(f, vf[f], bfrag);
        static_for<H>([&](auto c) {  // copy c goes out after MFMA c * NPV / H
          if (c * NPV / H == f) copy_v(lds_off<v_next>{}, c, cpr[c]);
        });
#pragma unroll
        for (int j = f * 8 / NPV; j < (f + 1) * 8 / NPV; ++j)
          lsum = M::add_pair(bfrag[j / 4], j % 4, lsum);
      }
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_setprio(0);
    };
    for (int t = 0; t < ntiles; t += 3) {
      step(t, std::integral_constant<int, 0>{});
      if (t + 1 < ntiles) step(t + 1, std::integral_constant<int, 1>{});
      if (t + 2 < ntiles) step(t + 2, std::integral_constant<int, 2>{});
    }
  } else {
    if (ntiles > 0) {
      stage_ids(wave, wave);  // tiles 0 .. W-1
      // When tiles 0 and 1 are local blocks (their ids are LDS writes), their
      // copies need no column ids: the barrier waits for LDS only and the
      // column-id copies stay in flight next to K(0), K(1), V(0); the barrier
      // after them (K(0) landed) also covers the older column-id copies, which
      // copy_pairs(2) reads next.
      if (t_init + t_diag >= 2)
        lds_barrier();
      else
        vm_lds_barrier();
      // K(0), K(1), V(0); after QK(0), K(2) into K(0)'s slot.  The loop's
      // barriers leave the kKeep most recent copies of the wave in flight.
      uint64_t pr[H], pr1[H];
      copy_pairs(0, 0, pr);
      copy_pairs(1, 1, pr1);
      static_for<H>([&](auto x) { copy_k(lds_off<0>{}, x, pr[x]); });
      static_for<H>([&](auto x) { copy_k(lds_off<S::kStageBytes>{}, x, pr1[x]); });
      if constexpr (!kStats)
        static_for<H>([&](auto x) { copy_v(lds_off<S::kTileBytes>{}, x, pr[x]); });
      vm_lds_barrier_keep<kKeep>();  // K(0) landed
      s_cur = qk(smem);
      mask(0, s_cur);
      float tmax = -__builtin_inff();
#pragma unroll
      for (int e = 0; e < 16; e += 2) tmax = max3_plain(tmax, s_cur[e], s_cur[e + 1]);
      rescale(tmax);
      lds_barrier();  // every wave is done with K(0)
      copy_pairs(2, 2, pr);
      static_for<H>([&](auto x) { copy_k(lds_off<0>{}, x, pr[x]); });
    }
    // One iteration; the parity P = t & 1 is a compile-time constant so that
    // the LDS slot addresses fold into the instructions' offsets and S(t),
    // S(t+1) alternate between two register sets.
    auto iteration = [&](int t, auto parity_tag, const f32x16_t& s_cur, f32x16_t& s_next) {
      constexpr int P = decltype(parity_tag)::value;
      constexpr uint32_t k_next = uint32_t((P ^ 1) * S::kStageBytes);    // K slot of t+1 and t+3
      constexpr uint32_t v_this = uint32_t(P * S::kStageBytes + S::kTileBytes);  // V slot of t
      constexpr uint32_t v_next = k_next + uint32_t(S::kTileBytes);      // V slot of t+1
      // ---- first half: QK(t+1) next to the softmax of S(t); copies of V(t+1)
      vm_lds_barrier_keep<kKeep>();  // K(t+1) landed; every wave is done with PV(t-1)
      if (P == 0 && t % W == 0) {  // every wave stages one of tiles t+W .. t+2W-1
        const int u = t + W + wave;
        stage_ids(u, u % S::kIdSlots);
      }
      const unsigned char* kb = smem + k_next;
#pragma unroll
      for (int e = 0; e < 16; ++e) s_next[e] = 0.f;
      float pr[16];
      uint64_t cpr[H];
      // K operands are read kAhead MFMAs ahead of their use (LDS latency), the
      // V^T operands of PV(t) kVAhead MFMAs ahead.
      constexpr int kAhead = 3, kVAhead = 3;
      const unsigned char* vb = smem + v_this;
      vec a[NQK], vf[NPV];
#pragma unroll
      for (int st = 0; st < kAhead; ++st)
        a[st] = __builtin_bit_cast(vec, *reinterpret_cast<const uint4*>(kb + koff[st]));
#pragma unroll
      for (int st = 0; st < NQK; ++st) {
        __builtin_amdgcn_sched_barrier(0);
        if (st + kAhead < NQK)
          a[st + kAhead] =
              __builtin_bit_cast(vec, *reinterpret_cast<const uint4*>(kb + koff[st + kAhead]));
        s_next = M::run(a[st], qreg[st], s_next);  // past the last tile: masked away below
        if (st == 0) copy_pairs(t + 1, (t + 1) % S::kIdSlots, cpr);
        static_for<H>([&](auto c) {  // copy c goes out after MFMA c * NQK / H
          if (!kStats && c * NQK / H == st) copy_v(lds_off<v_next>{}, c, cpr[c]);
        });
        // this step's share of the softmax of S(t)
#pragma unroll
        for (int e = st * 16 / NQK; e < (st + 1) * 16 / NQK; ++e) {
          pr[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(s_cur[e], scale_log2, mneg));
          asm volatile("" : "+v"(pr[e]));  // keeps the exp in this step (not sunk past mask)
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      mask(t + 1, s_next);
      if constexpr (kStats) {  // row sums of P(t), maximum of S(t+1), copies of K(t+3)
        vm_lds_barrier_keep<kKeep>();  // every wave is done with K(t+1)
        copy_pairs(t + 3, (t + 3) % S::kIdSlots, cpr);
        static_for<H>([&](auto c) { copy_k(lds_off<k_next>{}, c, cpr[c]); });
        float ps[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) ps[e] = pr[e] + pr[e + 8];
#pragma unroll
        for (int e = 0; e < 4; ++e) ps[e] += ps[e + 4];
        lsum += (ps[0] + ps[2]) + (ps[1] + ps[3]);
        float tmax = -__builtin_inff();
#pragma unroll
        for (int e = 0; e < 16; e += 2) tmax = max3_plain(tmax, s_next[e], s_next[e + 1]);
        rescale(tmax);
        return;
      }
      const vec bfrag[2] = {M::pack(pr), M::pack(pr + 8)};
      // ---- second half: PV(t), with the row sums of P(t) and the maximum of
      // S(t+1) spread over its MFMAs (in-order issue: VALU work placed between
      // the MFMAs runs while they execute); copies of K(t+3) into the slot QK
      // just read
      vm_lds_barrier_keep<kKeep>();  // V(t) landed; every wave is done with K(t+1)
#pragma unroll
      for (int f = 0; f < kVAhead; ++f) vf[f] = read_v(vb, f);
      copy_pairs(t + 3, (t + 3) % S::kIdSlots, cpr);
      float tmax = -__builtin_inff();
#pragma unroll
      for (int f = 0; f < NPV; ++f) {
        __builtin_amdgcn_sched_barrier(0);
        if (f + kVAhead < NPV) vf[f + kVAhead] = read_v(vb, f + kVAhead);
        pv_mfma(f, vf[f], bfrag);
        static_for<H>([&](auto c) {  // copy c goes out after MFMA c * NPV / H
          if (c * NPV / H == f) copy_k(lds_off<k_next>{}, c, cpr[c]);
        });
#pragma unroll
        for (int j = f * 8 / NPV; j < (f + 1) * 8 / NPV; ++j)
          lsum = M::add_pair(bfrag[j / 4], j % 4, lsum);
#pragma unroll
        for (int e = f * 16 / NPV; e < (f + 1) * 16 / NPV; e += 2)
          tmax = max3_plain(tmax, s_next[e], s_next[e + 1]);
      }
      __builtin_amdgcn_sched_barrier(0);
      rescale(tmax);
    };
    f32x16_t s_alt;  // scores of the odd tiles (s_cur holds the even ones)
    for (int t = 0; t < ntiles; t += 2) {
      iteration(t, std::integral_constant<int, 0>{}, s_cur, s_alt);
      if (t + 1 < ntiles) iteration(t + 1, std::integral_constant<int, 1>{}, s_alt, s_cur);
    }
  }

  // ---- merge the two key halves, normalise, store --------------------------
  vm_lds_barrier();  // every wave is done with the stages, the last copies have landed
  float* mo = reinterpret_cast<float*>(smem) + rh * (kStats ? 128 : 64 * (D / 2 + 4));
  if constexpr (kStats) {
    const float lrow = sum_halves(lsum);
    if (kc == 1) {
      mo[lane] = mc;
      mo[64 + lane] = lrow;
    }
    lds_barrier();
    if (kc == 0 && hh == 0 && qpos < Sq) {
      const float m1 = mo[lane], l1 = mo[64 + lane];
      const float m = __builtin_fmaxf(mc, m1);
      const float a0 = (mc == m) ? 1.f : __builtin_amdgcn_exp2f(mc - m);
      const float a1 = (m1 == m) ? 1.f : __builtin_amdgcn_exp2f(m1 - m);
      *reinterpret_cast<float2*>(stats + (bh * Sq + qpos) * 2) =
          make_float2(m, lrow * a0 + l1 * a1);
    }
    return;
  }
  // Each wave of a row half finishes half of the features (kc 0: blocks
  // [0, HB), kc 1: [HB, NB) of 32 features): it leaves the other half of its
  // partial output and its (m, l) in LDS and combines its own half with the
  // other wave's.  Per row half: two 64 x D/4 float regions (written by kc 0,
  // kc 1), then (m, l) of both waves.
  constexpr int NB = D / 32, HB = NB / 2;
  float* xw = mo + kc * 64 * (D / 4);
  const float* xr = mo + (kc ^ 1) * 64 * (D / 4);
  float* mlx = mo + 64 * (D / 2);
  const float lrow = sum_halves(lsum);  // row sum of this wave's key half, both halves
  auto finish = [&](auto keep_tag) {
    constexpr int K0 = decltype(keep_tag)::value * HB;  // first block kept here
    constexpr int O0 = HB - K0;                          // first block the other wave keeps
#pragma unroll
    for (int ii = 0; ii < HB; ++ii)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *reinterpret_cast<float4*>(xw + ((4 * ii + g) * 64 + lane) * 4) =
            make_float4(o[O0 + ii][4 * g], o[O0 + ii][4 * g + 1], o[O0 + ii][4 * g + 2],
                        o[O0 + ii][4 * g + 3]);
    mlx[kc * 128 + lane] = mc;
    mlx[kc * 128 + 64 + lane] = lrow;
    lds_barrier();
    const float m1 = mlx[(kc ^ 1) * 128 + lane], l1 = mlx[(kc ^ 1) * 128 + 64 + lane];
    const float m = __builtin_fmaxf(mc, m1);
    const float a0 = (mc == m) ? 1.f : __builtin_amdgcn_exp2f(mc - m);
    const float a1 = (m1 == m) ? 1.f : __builtin_amdgcn_exp2f(m1 - m);
    const float l = lrow * a0 + l1 * a1;
    const float inv = l > 0.f ? 1.f / l : 0.f;
    const float c0 = a0 * inv, c1 = a1 * inv;
    if (qpos >= Sq) return;
    if constexpr (kSplit) {  // fp32 partial output and (m, l) of this key range
      const int64_t item = (bh * Sq + qpos) * lay.nc + jr;
      float* po = stats + (2 * B * Hq * lay.nc * Sq + 3) / 4 * 4 + item * D;
#pragma unroll
      for (int ii = 0; ii < HB; ++ii) {
        const int i = K0 + ii;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const float4 x1 = *reinterpret_cast<const float4*>(xr + ((4 * ii + g) * 64 + lane) * 4);
          const int d0 = i * 32 + 8 * g + 4 * hh;
          *reinterpret_cast<float4*>(po + d0) = make_float4(
              o[i][4 * g + 0] * c0 + x1.x * c1, o[i][4 * g + 1] * c0 + x1.y * c1,
              o[i][4 * g + 2] * c0 + x1.z * c1, o[i][4 * g + 3] * c0 + x1.w * c1);
        }
      }
      if (kc == 0 && hh == 0) *reinterpret_cast<float2*>(stats + item * 2) = make_float2(m, l);
    } else {
      T* orow = out + b * sob + h * soh + qpos * sos;
#pragma unroll
      for (int ii = 0; ii < HB; ++ii) {
        const int i = K0 + ii;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const float4 x1 = *reinterpret_cast<const float4*>(xr + ((4 * ii + g) * 64 + lane) * 4);
          const int d0 = i * 32 + 8 * g + 4 * hh;
          const T e0 = Round<T>::store(o[i][4 * g + 0] * c0 + x1.x * c1);
          const T e1 = Round<T>::store(o[i][4 * g + 1] * c0 + x1.y * c1);
          const T e2 = Round<T>::store(o[i][4 * g + 2] * c0 + x1.z * c1);
          const T e3 = Round<T>::store(o[i][4 * g + 3] * c0 + x1.w * c1);
          uint2 w;
          w.x = uint32_t(e0.bits) | (uint32_t(e1.bits) << 16);
          w.y = uint32_t(e2.bits) | (uint32_t(e3.bits) << 16);
          *reinterpret_cast<uint2*>(orow + d0) = w;
        }
      }
    }
  };
  if (kc == 0)
    finish(std::integral_constant<int, 0>{});
  else
    finish(std::integral_constant<int, 1>{});
}

// Form of the sparse loop at D = 128 with 64-row blocks when the caller
// leaves it open: the staged pipeline where the kv heads are not shared and
// one head's K and V exceed 32 MiB (their gathers mostly miss L2, and the
// fabric's latency wants the staged form's longer copy lead: 119056 keys,
// 24 heads, +2.5% on the ring), the ring form otherwise (32K and 128K causal
// GQA, 32760 non-causal: -1.5 to -2.7% of a prefill, same-box A/B).
bool ring_form_preferred(int64_t Hq, int64_t Hk, int64_t Sk, int64_t D) {
  return !(Hq == Hk && Sk * D * 2 * 2 > (int64_t(32) << 20));
}

template <typename T, int D, int QPS, bool kDense, bool kStats, bool kSplit = false>
static hipError_t launch_attn_mfma_k(const void* q, const int64_t* sq, const void* k,
                                     const int64_t* sk, const void* v, const int64_t* sv,
                                     void* out, const int64_t* so, int64_t B, int64_t Hq,
                                     int64_t Hk, int64_t Sq, int64_t Sk, int causal,
                                     float scale_log2, const int32_t* counts,
                                     const int32_t* indices, const RowLayout& lay, int nseg,
                                     int segk, int64_t dense_qoff, float* stats, int form,
                                     hipStream_t stream) {
  static const int64_t zero[3] = {0, 0, 0};
  if (kStats) sv = so = zero;  // no V, no output
  const int64_t nblocks = WorkOrder{lay.nc, B, Hq, Hk, causal == 0}.grid_items();
  constexpr bool kRingOk = !kDense && !kStats && !kSplit && QPS == 64 && D == 128;
  bool ring = false;
  if constexpr (kRingOk)
    ring = form == kAttnFormRing || (form == kAttnFormAuto && ring_form_preferred(Hq, Hk, Sk, D));
  else if (form == kAttnFormRing)
    return hipErrorInvalidValue;
  auto go = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, dim3(unsigned(nblocks)), dim3(AttnShape<D, QPS>::kThreads), 0,
                       stream, static_cast<const T*>(q), sq[0], sq[1], sq[2],
                       static_cast<const T*>(k), sk[0], sk[1], sk[2], static_cast<const T*>(v),
                       sv[0], sv[1], sv[2], static_cast<T*>(out), so[0], so[1], so[2], B, Hq, Hk,
                       Sq, Sk, causal, scale_log2, counts, indices, lay, nseg, segk,
                       (kDense || kSplit) ? dense_qoff : 0, stats);
    return hipGetLastError();
  };
  if constexpr (kRingOk)
    if (ring) return go(attn_mfma_kernel<T, D, QPS, kDense, kStats, kSplit, true>);
  return go(attn_mfma_kernel<T, D, QPS, kDense, kStats, kSplit, false>);
}

// dense_qoff >= 0: dense key lists (64-row blocks only); stats != nullptr: the
// row statistics instead of the output.
template <typename T, int D, int QPS>
static hipError_t launch_attn_mfma_tdq(const void* q, const int64_t* sq, const void* k,
                                       const int64_t* sk, const void* v, const int64_t* sv,
                                       void* out, const int64_t* so, int64_t B, int64_t Hq,
                                       int64_t Hk, int64_t Sq, int64_t Sk, int causal,
                                       float scale_log2, const int32_t* counts,
                                       const int32_t* indices, const RowLayout& lay, int nseg,
                                       int segk, int64_t dense_qoff, float* stats, int form,
                                       hipStream_t stream) {
#define VA_ATTN_LAUNCH(DENSE, STATS)                                                           \
  return launch_attn_mfma_k<T, D, QPS, DENSE, STATS>(q, sq, k, sk, v, sv, out, so, B, Hq, Hk,  \
                                                     Sq, Sk, causal, scale_log2, counts,      \
                                                     indices, lay, nseg, segk, dense_qoff,    \
                                                     stats, form, stream)
  if (dense_qoff >= 0) {
    if constexpr (QPS == 64) {
      if (stats) VA_ATTN_LAUNCH(true, true);
      VA_ATTN_LAUNCH(true, false);
    }
    return hipErrorInvalidValue;
  }
  if (stats) VA_ATTN_LAUNCH(false, true);
  VA_ATTN_LAUNCH(false, false);
#undef VA_ATTN_LAUNCH
}

template <typename T>
static hipError_t launch_attn_mfma_t(int64_t D, int64_t qps, const void* q, const int64_t* sq,
                                     const void* k, const int64_t* sk, const void* v,
                                     const int64_t* sv, void* out, const int64_t* so, int64_t B,
                                     int64_t Hq, int64_t Hk, int64_t Sq, int64_t Sk, int causal,
                                     float scale_log2, const int32_t* counts,
                                     const int32_t* indices, const RowLayout& lay, int nseg,
                                     int segk, int64_t dense_qoff, float* stats, int form,
                                     hipStream_t stream) {
#define VA_ATTN_CASE(DD, QQ)                                                                   \
  if (D == DD && qps == QQ)                                                                    \
    return launch_attn_mfma_tdq<T, DD, QQ>(q, sq, k, sk, v, sv, out, so, B, Hq, Hk, Sq, Sk,   \
                                           causal, scale_log2, counts, indices, lay, nseg,    \
                                           segk, dense_qoff, stats, form, stream);
  VA_ATTN_CASE(64, 64)
  VA_ATTN_CASE(128, 64)
  VA_ATTN_CASE(64, 128)
  VA_ATTN_CASE(128, 128)
#undef VA_ATTN_CASE
  return hipErrorInvalidValue;
}

// Split-key partials for decode: q rows [0, Sq) of each of the B*H row groups
// (the query heads sharing kv head h of batch b) against keys
// [J*span, (J+1)*span), J < nsplit; results in `part` as described at the
// kernel.
template <typename T>
static hipError_t launch_attn_split_t(int64_t D, const void* q, const int64_t* sq, const void* k,
                                      const int64_t* sk, const void* v, const int64_t* sv,
                                      int64_t B, int64_t H, int64_t Sq, int64_t Sk,
                                      float scale_log2, int64_t nsplit, int64_t span,
                                      float* part, hipStream_t stream) {
  RowLayout lay;
  lay.J0 = 0;
  lay.nc = nsplit;
  lay.qps = 64;
  lay.Sk = Sk;
  lay.dense_stride = 0;
  lay.causal = 0;
  lay.wo_init = 0;
  static const int64_t zero[3] = {0, 0, 0};
  if (D == 64)
    return launch_attn_mfma_k<T, 64, 64, true, false, true>(
        q, sq, k, sk, v, sv, nullptr, zero, B, H, H, Sq, Sk, 0, scale_log2, nullptr, nullptr, lay,
        1, 0, span, part, kAttnFormAuto, stream);
  if (D == 128)
    return launch_attn_mfma_k<T, 128, 64, true, false, true>(
        q, sq, k, sk, v, sv, nullptr, zero, B, H, H, Sq, Sk, 0, scale_log2, nullptr, nullptr, lay,
        1, 0, span, part, kAttnFormAuto, stream);
  return hipErrorInvalidValue;
}

hipError_t launch_attn_split(int dtype, int64_t D, const void* q, const int64_t* sq,
                             const void* k, const int64_t* sk, const void* v, const int64_t* sv,
                             int64_t B, int64_t H, int64_t Sq, int64_t Sk, float scale_log2,
                             int64_t nsplit, int64_t span, float* part, hipStream_t stream) {
  if (dtype == kBF16)
    return launch_attn_split_t<bf16_t>(D, q, sq, k, sk, v, sv, B, H, Sq, Sk, scale_log2, nsplit,
                                       span, part, stream);
  if (dtype == kF16)
    return launch_attn_split_t<f16_t>(D, q, sq, k, sk, v, sv, B, H, Sq, Sk, scale_log2, nsplit,
                                      span, part, stream);
  return hipErrorInvalidValue;
}

bool attn_mfma_supported(int dtype, int64_t D, int64_t qps) {
  return (dtype == kBF16 || dtype == kF16) && (D == 64 || D == 128) && (qps == 64 || qps == 128);
}

bool attn_mfma_ring_supported(int dtype, int64_t D, int64_t qps) {
  return (dtype == kBF16 || dtype == kF16) && D == 128 && qps == 64;
}

hipError_t launch_attn_mfma(int dtype, int64_t D, int64_t qps, const void* q, const int64_t* sq,
                            const void* k, const int64_t* sk, const void* v, const int64_t* sv,
                            void* out, const int64_t* so, int64_t B, int64_t Hq, int64_t Hk,
                            int64_t Sq, int64_t Sk, int causal, float scale_log2,
                            const int32_t* counts, const int32_t* indices, const RowLayout& lay,
                            int nseg, int segk, int64_t dense_qoff, float* stats, int form,
                            hipStream_t stream) {
  if (dtype == kBF16)
    return launch_attn_mfma_t<bf16_t>(D, qps, q, sq, k, sk, v, sv, out, so, B, Hq, Hk, Sq, Sk,
                                      causal, scale_log2, counts, indices, lay, nseg, segk,
                                      dense_qoff, stats, form, stream);
  if (dtype == kF16)
    return launch_attn_mfma_t<f16_t>(D, qps, q, sq, k, sk, v, sv, out, so, B, Hq, Hk, Sq, Sk,
                                     causal, scale_log2, counts, indices, lay, nseg, segk,
                                     dense_qoff, stats, form, stream);
  return hipErrorInvalidValue;
}

}  // namespace va
