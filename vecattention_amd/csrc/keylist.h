// The key set of one q-block in the vector-sparse attention.
//
// The reference passes (blk_count, blk_idx) local blocks of 64 keys plus the
// selected columns (spattn/src/VecAttention.py:63-92,110-121); the masked-dense
// restatement in spattn/threshold/model_tuner.py:202-216 fixes the meaning:
// the union of the blocks [blk_idx, blk_idx + 64) clipped to [0, S_k) and the
// columns, intersected with the causal mask.  The local blocks are closed
// forms of the q-block index J, so they are generated here instead of being
// read from memory:
//   causal, J >= 1 : init  = [0, qps)
//                    diag  = [J*qps, min((J+1)*qps, S_k))   (causal mask applies)
//   causal, J == 0 : diag  = [0, min(qps, S_k))             (causal mask applies)
//   non-causal     : no local blocks
// followed by the selected columns, which always lie in [qps, J*qps) under the
// causal rule, so the three segments never overlap.
#pragma once
#include "common.h"

namespace va {

struct KeyList {
  int64_t n_init;   // keys 0 .. n_init-1
  int64_t diag0;    // first diagonal key
  int64_t n_diag;   // keys diag0 .. diag0+n_diag-1
  int64_t n_col;    // selected columns
  const int32_t* cols;

  __device__ static KeyList make(int64_t J, int64_t qps, int64_t Sk, int causal,
                                 int64_t count, const int32_t* cols) {
    KeyList kl;
    kl.cols = cols;
    kl.n_col = count;
    if (causal) {
      kl.n_init = (J >= 1) ? qps : 0;
      kl.diag0 = J * qps;
      const int64_t rem = Sk - kl.diag0;
      kl.n_diag = rem < qps ? (rem > 0 ? rem : 0) : qps;
    } else {
      kl.n_init = 0;
      kl.diag0 = 0;
      kl.n_diag = 0;
    }
    return kl;
  }
  // Every key, for dense attention (the reference's Full_prefill).  A causal
  // row at absolute position qoff + J*qps + r sees keys up to that position
  // (qoff = Sk - Sq aligns the last query with the last key): the span
  // [0, a0) whole and the diagonal span [a0, a0 + qps) under the causal mask,
  // a0 = qoff + J*qps.  A non-causal row sees all Sk keys.
  __device__ static KeyList dense(int64_t J, int64_t qps, int64_t Sk, int causal, int64_t qoff) {
    KeyList kl;
    kl.cols = nullptr;
    kl.n_col = 0;
    if (causal) {
      const int64_t a0 = qoff + J * qps;
      kl.n_init = a0 < Sk ? a0 : Sk;
      kl.diag0 = a0;
      const int64_t rem = Sk - a0;
      kl.n_diag = rem < qps ? (rem > 0 ? rem : 0) : qps;
    } else {
      kl.n_init = Sk;
      kl.diag0 = 0;
      kl.n_diag = 0;
    }
    return kl;
  }
  // Keys [J*span, min((J+1)*span, Sk)) of a split key range (decode: the
  // work-group's share of the KV cache), held as the "diagonal" span of the
  // list; the kernel applies no causal mask to it (causal = 0).
  __device__ static KeyList split(int64_t J, int64_t span, int64_t Sk) {
    KeyList kl;
    kl.cols = nullptr;
    kl.n_col = 0;
    kl.n_init = 0;
    kl.diag0 = J * span;
    const int64_t rem = Sk - kl.diag0;
    kl.n_diag = rem < span ? (rem > 0 ? rem : 0) : span;
    return kl;
  }
  __device__ int64_t total() const { return n_init + n_diag + n_col; }
  __device__ int64_t key(int64_t p) const {
    if (p < n_init) return p;
    p -= n_init;
    if (p < n_diag) return diag0 + p;
    return cols[p - n_diag];
  }
  __device__ bool is_diag(int64_t p) const { return p >= n_init && p < n_init + n_diag; }
};

}  // namespace va
