// Shared device/host helpers for the VecAttention prefill kernels (gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace va {

enum DType : int { kF32 = 0, kBF16 = 1, kF16 = 2 };

// Passes of the wave selection kernel.  A selection whose groups are longer
// than a key segment runs twice: the maxima pass scores every segment and
// records, per row, the segment's MFMA maximum and its exact maximum; the
// carry pass then selects each segment starting from the maxima of the
// earlier segments of the same group, which are exactly the running maxima a
// sequential walk would hold there.  Plain: one pass, no carried state.
enum SelectPass : int { kPassPlain = 0, kPassMax = 1, kPassCarry = 2 };

// Forms of the MFMA attention kernel's sparse loop (D = 128, 64-row blocks):
// staged (two stages of a K and a V tile, two work-groups per CU) or ring
// (three tile slots, three work-groups per CU); auto picks by shape.
enum AttnForm : int { kAttnFormAuto = 0, kAttnFormStaged = 1, kAttnFormRing = 2 };

// Raw 16-bit storage types; arithmetic goes through explicit conversions so
// that every rounding step is visible.
struct bf16_t { uint16_t bits; };
struct f16_t { uint16_t bits; };

__host__ __device__ inline float bits_to_float(uint32_t u) {
  return __builtin_bit_cast(float, u);
}
__host__ __device__ inline uint32_t float_to_bits(float f) {
  return __builtin_bit_cast(uint32_t, f);
}

// bf16 -> fp32 is exact (bf16 is the upper half of an fp32 pattern).
__device__ inline float to_f32(bf16_t x) { return bits_to_float(uint32_t(x.bits) << 16); }
__device__ inline float to_f32(f16_t x) { return float(__builtin_bit_cast(_Float16, x.bits)); }
__device__ inline float to_f32(float x) { return x; }

// Round-to-nearest-even fp32 -> bf16, NaN kept quiet.
__device__ inline uint16_t rne_bf16_bits(float f) {
  uint32_t u = float_to_bits(f);
  if ((u & 0x7f800000u) == 0x7f800000u) {
    if (u & 0x007fffffu) u |= 0x00400000u;
    return uint16_t(u >> 16);
  }
  u += 0x7fffu + ((u >> 16) & 1u);
  return uint16_t(u >> 16);
}

// fp32 -> fp16 with the hardware conversion (round-to-nearest-even mode).
__device__ inline uint16_t rne_f16_bits(float f) {
  return __builtin_bit_cast(uint16_t, _Float16(f));
}

template <typename T> struct Round;
template <> struct Round<float> {
  __device__ static float rt(float x) { return x; }
  __device__ static float store(float x) { return x; }
};
template <> struct Round<bf16_t> {
  __device__ static float rt(float x) { return bits_to_float(uint32_t(rne_bf16_bits(x)) << 16); }
  __device__ static bf16_t store(float x) { return bf16_t{rne_bf16_bits(x)}; }
};
template <> struct Round<f16_t> {
  __device__ static float rt(float x) { return float(__builtin_bit_cast(_Float16, rne_f16_bits(x))); }
  __device__ static f16_t store(float x) { return f16_t{rne_f16_bits(x)}; }
};

// Work-group barrier for LDS traffic only.  __syncthreads() also orders global
// memory, which makes every wave wait for all of its outstanding global loads
// and stores (prefetches included); this barrier waits for LDS operations only,
// so prefetched global loads stay in flight across it.
__device__ inline void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Work-group barrier after this wave's global loads into LDS
// (buffer_load ... lds) and its LDS operations have completed: afterwards the
// LDS data written by every wave's copies is visible to all waves.
__device__ inline void vm_lds_barrier() {
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
}
// The same, leaving this wave's N most recent global loads in flight (loads
// complete in issue order, so every older one has landed).
template <int N>
__device__ inline void vm_lds_barrier_keep() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

// ---------------------------------------------------------------------------
// Work order.  Work-groups are dispatched round-robin over the 8 XCDs of the
// chip (block i runs on XCD i % 8), each with its own L2.  A work item is
// (row block jr in [0, nrows), q head bh in [0, B*Hq)); items of one kv head
// (b, hk) read the same K/V rows, so they are kept on the same XCDs:
//  - fewer kv groups than XCDs: each group gets 8/g XCDs, which walk its
//    items longest-first (descending jr);
//  - otherwise, the XCDs work in pairs (kTeam), each pair walking a
//    contiguous share of the items in group-major order and its two XCDs
//    taking alternate items, i.e. about one group per pair at a time: the
//    rows an L2 holds are those of one kv head, and the kv heads in use at
//    once are four, whose K/V fit the chip's 256 MB Infinity Cache at the
//    DiT shapes (61 MB per head at 119056 keys); one group per XCD kept eight
//    heads live and measured 1.8% slower at 119056 keys, one group per four
//    XCDs 0.5% (the share is whole groups when g % 8 == 0; for other g only
//    when every row costs the same, `equal_rows`, else the items are dealt
//    round-robin, longest-first, to keep the XCDs balanced).
// grid_items() is the launch size; map_item() returns false for the few idle
// blocks of a launch whose items do not split evenly over the XCDs.
// ---------------------------------------------------------------------------
struct WorkOrder {
  int64_t nrows, B, Hq, Hk;
  bool equal_rows;  // every row block costs the same (non-causal)
  static constexpr int kXcd = 8;
  static constexpr int kTeam = 2;  // XCDs sharing a contiguous share (see above)

  __host__ __device__ int64_t nkv() const { return B * Hk; }
  __host__ __device__ int64_t rep() const { return Hq / Hk; }
  __host__ __device__ int64_t grid_items() const {
    const int64_t g = nkv();
    if (kXcd % g == 0) {
      const int64_t copies = kXcd / g;
      const int64_t per = (rep() * nrows + copies - 1) / copies;
      return kXcd * per;
    }
    if (g % kXcd == 0 || equal_rows) {
      const int64_t n = g * rep() * nrows, teams = kXcd / kTeam, per = (n + teams - 1) / teams;
      return kXcd * ((per + kTeam - 1) / kTeam);
    }
    return nrows * B * Hq;
  }
  __host__ __device__ bool map_item(int64_t i, int64_t& jr, int64_t& bh) const {
    const int64_t g = nkv(), r = rep();
    if (kXcd % g == 0) {  // several XCDs per kv group
      const int64_t copies = kXcd / g;
      const int64_t x = i % kXcd, s = i / kXcd;
      const int64_t grp = x % g, c = x / g;
      const int64_t j = s * copies + c;
      if (j >= r * nrows) return false;
      jr = nrows - 1 - j / r;
      const int64_t b = grp / Hk, hk = grp % Hk;
      bh = b * Hq + hk * r + j % r;
      return true;
    }
    if (g % kXcd == 0 || equal_rows) {  // contiguous shares per XCD pair, group-major
      const int64_t n = g * r * nrows, teams = kXcd / kTeam, per = (n + teams - 1) / teams;
      const int64_t x = i % kXcd, k = (i / kXcd) * kTeam + x % kTeam;
      const int64_t L = (x / kTeam) * per + k;
      if (k >= per || L >= n) return false;
      const int64_t grp = L / (r * nrows), rem = L % (r * nrows);
      jr = nrows - 1 - rem / r;
      const int64_t b = grp / Hk, hk = grp % Hk;
      bh = b * Hq + hk * r + rem % r;
      return true;
    }
    const int64_t BH = B * Hq;  // plain longest-first order
    jr = nrows - 1 - i / BH;
    bh = i % BH;
    return true;
  }
  // Position of item (J, bh) in its XCD's dispatch sequence, modulo `period`
  // and up to a constant, from the absolute q-block J (items are walked in
  // descending J), so that every launch holding the row gives it the same
  // value.  Only (back mod period * span) matters for the result, which keeps
  // every product in 32 bits.
  __device__ uint32_t xcd_rank(uint32_t J, uint32_t bh, uint32_t period) const {
    const uint32_t hq = uint32_t(Hq), g = uint32_t(B) * uint32_t(Hk), r = hq / uint32_t(Hk);
    const uint32_t back = (1u << 24) - J;  // J < 2^24 (the host bounds Sk, hence Sq / qps)
    uint32_t rank;
    if (kXcd % g == 0) {
      const uint32_t copies = kXcd / g, bk = back % (period * copies);
      rank = (bk * r + bh % r) / copies;
    } else if (g % kXcd == 0 || equal_rows) {
      rank = (back % (period * kTeam)) / kTeam;
    } else {
      rank = ((back % (period * kXcd)) * (uint32_t(B) * hq) + bh) / kXcd;
    }
    return rank % period;
  }
  // map_item in 32-bit arithmetic, for kernels: every quantity is below 2^31
  // (the host bounds nrows * B * Hq by the grid limit), and a 64-bit division
  // costs a few hundred dependent scalar instructions at every work-group start.
  __device__ bool map_item32(uint32_t i, int& jr, int& bh) const {
    const uint32_t n_rows = uint32_t(nrows), hq = uint32_t(Hq), hkv = uint32_t(Hk);
    const uint32_t g = uint32_t(B) * hkv, r = hq / hkv;
    if (kXcd % g == 0) {
      const uint32_t copies = kXcd / g;
      const uint32_t x = i % kXcd, s = i / kXcd;
      const uint32_t grp = x % g, c = x / g;
      const uint32_t j = s * copies + c;
      if (j >= r * n_rows) return false;
      jr = int(n_rows - 1 - j / r);
      bh = int((grp / hkv) * hq + (grp % hkv) * r + j % r);
      return true;
    }
    if (g % kXcd == 0 || equal_rows) {
      const uint32_t rn = r * n_rows, n = g * rn, teams = kXcd / kTeam, per = (n + teams - 1) / teams;
      const uint32_t x = i % kXcd, k = (i / kXcd) * kTeam + x % kTeam;
      const uint32_t L = (x / kTeam) * per + k;
      if (k >= per || L >= n) return false;
      const uint32_t grp = L / rn, rem = L % rn;
      jr = int(n_rows - 1 - rem / r);
      bh = int((grp / hkv) * hq + (grp % hkv) * r + rem % r);
      return true;
    }
    const uint32_t BH = uint32_t(B) * hq;
    jr = int(n_rows - 1 - i / BH);
    bh = int(i % BH);
    return true;
  }
};

// ---------------------------------------------------------------------------
// Per-row index lists of the selection ("capacity layout").
//
// Row J of a chunk [J0, J0+nc) owns `row_capacity(J)` int32 slots: the number
// of keys the selection rule can ever pick for it.  The rows of one (b, h) are
// packed back to back, and the (b, h) blocks follow each other, so the offset
// of every row is a closed form and selection needs no host round trip to size
// its output.  A non-zero `dense_stride` instead gives every row that stride
// (the reference's dense (B, H, nqb, padded_k) layout).
//   causal:     keys [smin, J*qps) with smin = wo_init ? qps : 0
//   non-causal: keys [smin, Sk)    with smin = wo_init ? min(qps, Sk) : 0
// A non-null `csr` selects the compact layout instead: row r = bh*nc + jr
// holds exactly its selected keys from slot csr[r] on (csr[r+1] - csr[r] of
// them), as counted by an earlier run of the same selection; with key
// segments, segment s of the row follows the keys of its earlier segments and
// holds seg_counts[r*nseg + s] of them.
// ---------------------------------------------------------------------------
struct RowLayout {
  int64_t J0, nc, qps, Sk;
  int64_t dense_stride;  // > 0: dense rows
  int causal, wo_init;
  const int64_t* csr = nullptr;         // compact layout: row offsets (B*Hq*nc + 1)
  const int32_t* seg_counts = nullptr;  // compact layout: keys per (row, segment)

  __host__ __device__ int64_t smin() const {
    if (!wo_init) return 0;
    if (causal) return qps;
    return qps < Sk ? qps : Sk;
  }
  // T(n) = n(n-1)/2 for n >= 1, else 0.
  __host__ __device__ static int64_t tri(int64_t n) { return n >= 1 ? n * (n - 1) / 2 : 0; }
  // Sum over j in [0, J) of max(0, j - a).
  __host__ __device__ int64_t prefix_causal(int64_t J) const {
    const int64_t a = wo_init ? 1 : 0;  // smin / qps for causal rows
    return tri(J - a);
  }
  __host__ __device__ int64_t capacity(int64_t J) const {
    if (dense_stride > 0) return dense_stride;
    if (causal) {
      int64_t c = J * qps - smin();
      return c > 0 ? c : 0;
    }
    return Sk - smin();
  }
  // Offset of chunk row jr (J = J0 + jr) inside one (b, h) block.
  __host__ __device__ int64_t row_in_block(int64_t jr) const {
    if (dense_stride > 0) return jr * dense_stride;
    if (causal) return qps * (prefix_causal(J0 + jr) - prefix_causal(J0));
    return jr * (Sk - smin());
  }
  __host__ __device__ int64_t block_size() const { return row_in_block(nc); }
  __host__ __device__ int64_t row_offset(int64_t bh, int64_t jr) const {
    return bh * block_size() + row_in_block(jr);
  }
  // First slot of row jr of (b, h) (jr == nc: the end of the (b, h) block).
  __device__ int64_t row_start(int64_t bh, int64_t jr) const {
    return csr ? csr[bh * nc + jr] : row_offset(bh, jr);
  }
  // First slot and number of slots of key segment `seg` (of nseg, keys from
  // seg_lo on) of row jr: in the capacity layout slot k - smin holds key k;
  // in the compact layout the segment holds exactly its counted keys.
  __device__ void segment_slots(int64_t bh, int64_t jr, int seg, int nseg, int64_t seg_lo,
                                int64_t& start, int64_t& cap) const {
    if (csr) {
      const int64_t r = bh * nc + jr;
      start = csr[r];
      if (nseg > 1) {
        for (int s = 0; s < seg; ++s) start += seg_counts[r * nseg + s];
        cap = seg_counts[r * nseg + seg];
      } else {
        cap = csr[r + 1] - csr[r];
      }
      return;
    }
    const int64_t sm = smin();
    const int64_t slot = (seg_lo > sm ? seg_lo : sm) - sm;
    start = row_offset(bh, jr) + slot;
    const int64_t c = capacity(J0 + jr) - slot;
    cap = c > 0 ? c : 0;
  }
};

}  // namespace va
