/*
 * C ABI of the MI355X-native VecAttention prefill hot path (libvecattn.so).
 *
 * Plain pointers and sizes only.  All device pointers are HIP device memory on
 * the current device; `stream` is a hipStream_t (NULL = default stream).
 * Every entry point is stream-ordered, allocates nothing, and returns VA_OK or
 * a negative error code; va_last_error() returns the message of the last
 * failure on the calling thread.  Strides are in elements; the feature
 * dimension D must be contiguous (stride 1).
 *
 * Element types: VA_F32 (float), VA_BF16 (bfloat16), VA_F16 (IEEE half).
 * Tensor shapes use the reference's BHSD convention:
 *   q (B, Hq, Sq, D), k and v (B, Hk, Sk, D), out (B, Hq, Sq, D).
 *
 * Selected key lists ("index layout"): row J of a chunk [J0, J0+nc) of q-block
 * rows owns capacity(J) int32 slots, written in ascending key order from its
 * row offset; counts[(b*Hq + h)*nc + (J - J0)] holds the number written.
 *   dense_stride > 0 : every row has `dense_stride` slots (the reference's
 *                      dense (B, H, nqb, padded_k) column_index layout);
 *   dense_stride == 0: packed capacities; a causal row holds max(0, J*qps - smin)
 *                      slots (keys [smin, J*qps), smin = wo_init ? qps : 0), a
 *                      non-causal row Sk - smin slots (smin = wo_init ?
 *                      min(qps, Sk) : 0).  va_select_index_capacity() gives
 *                      the total, va_select_row_offset() the offset of a row.
 */
#ifndef VECATTN_H_
#define VECATTN_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { VA_F32 = 0, VA_BF16 = 1, VA_F16 = 2 };

enum {
  VA_OK = 0,
  VA_ERR_ARG = -1,          /* invalid argument (mirrors the reference's asserts) */
  VA_ERR_UNSUPPORTED = -2,  /* valid for the reference, not handled by this build */
  VA_ERR_HIP = -3,          /* a HIP runtime call failed (no device, launch error) */
  VA_ERR_WORKSPACE = -4     /* workspace smaller than its *_workspace_size() query */
};

enum {
  VA_ATTN_AUTO = 0,
  VA_ATTN_MFMA = 1,
  VA_ATTN_SIMPLE = 2,
  VA_ATTN_MFMA_STAGED = 3,
  VA_ATTN_MFMA_RING = 4
};
enum { VA_SEL_AUTO = 0, VA_SEL_EXACT = 1, VA_SEL_MFMA = 2, VA_SEL_WAVE = 3 };

/* Library version (major*10000 + minor*100 + patch). */
int va_version(void);

/* Message of the last failing call on this thread ("" if none). */
const char* va_last_error(void);

/* Number of HIP devices visible, or a negative code (no GPU is an error). */
int va_device_count(void);

/*
 * Query pooling: block means over q_pooling_size rows, fused with the
 * selection's query scaling.
 * Replaces spattn/src/utils.py:340-360 (average_vector -> triton_bnhd_pool
 * :86-137 -> bnhd_pool_kernel :8-83) and the pooled-query scaling of
 * spattn/src/kernels/vecattention_kernels.py:94,244-245.
 *   pooled[b,h,J,:] = T(fp32 mean of rows J*qps .. min(S,(J+1)*qps)-1)
 *   scaled[b,h,J,:] = T(fp32(pooled * fp32(1/sqrt(D))))
 * pooled / scaled: contiguous (B, H, ceil(S/qps), D); either may be NULL.
 */
int va_pool(int dtype, const void* q, int64_t B, int64_t H, int64_t S, int64_t D,
            int64_t sqb, int64_t sqh, int64_t sqs, int64_t q_pooling_size,
            void* pooled, void* scaled, void* stream);

/*
 * TilingSelect: important-vertical-vector selection for q-block rows
 * [J0, J0+nc) of every (b, h).
 * Replaces spattn/src/kernels/vecattention_kernels.py:59-181
 * (fuse_qk_softmax_minp_wo_causal) and its kernels :206-272 / :275-345.
 *   qs     : scaled pooled queries of the chunk: row jr of (b, h) at
 *            qs + b*sqb + h*sqh + jr*sqn (element strides, features contiguous)
 *   k      : keys (B, Hk, Sk, D) with strides; q head h reads kv head h/(Hq/Hk)
 *   gap    : fp32 gap (= -ln(threshold + 1e-9)) used when gaps == NULL
 *   gaps   : device fp32 array of B*Hq gaps (per-head thresholds), or NULL
 *   bsq    : BLOCK_SIZE_Q of the reference launch (64 for the shipped VLM
 *            configs); it places the reference's causal first-row tile quirk
 * Output: see "index layout" above.  Decisions follow canonical arithmetic
 * (a sequential fp64 dot product rounded once to fp32), so the selected sets
 * match the CPU restatement of the rule bit for bit, whichever kernel runs:
 *   VA_SEL_EXACT : fp64 scores for every pair (any dtype, any k_local_size);
 *   VA_SEL_MFMA  : bf16/fp16 MFMA scores with a certified error band and exact
 *                  fp64 recomputation inside the band (D in {64,128},
 *                  k_local_size in {16,32,64}); needs `scratch`;
 *   VA_SEL_WAVE  : the same certified scheme organised one wave per 32 rows
 *                  (additionally k_local_size * group_k_block 16, 32 or a
 *                  multiple of 64, Sk < 2^24, < 2 GiB of key rows per kv
 *                  head); needs `scratch`;
 *   VA_SEL_AUTO  : WAVE, else MFMA, when supported and scratch is given, else
 *                  exact.
 * scratch: device fp32 buffer of va_select_scratch_floats(B, Hk) floats (key
 * norms), or NULL.
 */
int va_select(int dtype, const void* qs, int64_t sqb, int64_t sqh, int64_t sqn,
              const void* k, int64_t skb, int64_t skh, int64_t sks, int64_t B, int64_t Hq,
              int64_t Hk, int64_t Sk, int64_t D, int64_t q_pooling_size, int64_t k_local_size,
              int64_t group_k_block, int causal, int wo_init, int64_t J0, int64_t nc,
              int64_t bsq, float gap, const float* gaps, int64_t dense_stride,
              int32_t* counts, int32_t* indices, int kernel, float* scratch,
              int64_t scratch_floats, void* stream);

/*
 * Split selection ("key segments"), the form va_prefill uses internally: the
 * keys are cut into segments of segment_keys keys (a multiple of 64, at most
 * 64 segments) that are selected in parallel.  When segment_keys is also a
 * multiple of the group span k_local_size*group_k_block, every segment starts
 * a group and one pass suffices.  When one group covers a whole row (group
 * span >= Sk; the DiT configurations), a first pass records each segment's
 * maxima and a second pass selects every segment from the maxima of the
 * segments before it, in scratch (va_select_segments_scratch_floats).
 * Segment s of row J writes its keys in ascending order from slot
 * max(s*segment_keys, smin) - smin of the row's index layout and its count to
 * counts[((b*Hq + h)*nc + (J - J0))*nseg + s], nseg = ceil(Sk / segment_keys);
 * a row's list is the concatenation of its segments.  Runs on the VA_SEL_WAVE
 * kernel where its conditions hold, else on the 64-row MFMA kernel (VA_SEL_MFMA
 * conditions, one pass, segment_keys a multiple of 256), else (fp32 inputs,
 * other head dims) on the exact kernel, in one or two passes.  No counterpart in the
 * reference (its single launch writes dense rows); the selected sets are the
 * reference rule's, as for va_select.
 * va_select_segment_keys returns the segment length va_prefill uses for
 * bf16/fp16 inputs with head_dim 64 or 128: the wave kernel's (tiles of 16 to
 * 64 keys, group span of 16 or 32 keys or a multiple of 64), else the 64-row
 * MFMA kernel's (whole 256-key chunks that each start a group, e.g.
 * k_local_size 128 or a group span of 48 keys); 0 when the keys are not split,
 * or -1 on invalid sizes.
 */
int64_t va_select_segment_keys(int64_t Sk, int64_t k_local_size, int64_t group_k_block);
/* The segment length va_prefill uses for fp32 inputs that run on the fp32
 * matrix-core attention (VA_KERNELS_ATTN_F32 with VA_KERNELS_SELECT_EXACT):
 * the exact kernel's split, at least Sk/64 keys, multiples of 256 keys and of
 * the group span (one pass), or of 256 keys when one group spans the row
 * (maxima pass, then carry pass); 0 when the keys are not split, -1 on
 * invalid sizes.  No counterpart in the reference. */
int64_t va_select_exact_segment_keys(int64_t Sk, int64_t k_local_size, int64_t group_k_block);
/* fp32 scratch floats va_select_segments needs: the key norms, plus two floats
 * per (row, segment) in the two-pass form.  -1 on invalid sizes. */
int64_t va_select_segments_scratch_floats(int64_t B, int64_t Hq, int64_t Hk, int64_t Sk,
                                          int64_t nc, int64_t segment_keys,
                                          int64_t k_local_size, int64_t group_k_block);
int va_select_segments(int dtype, const void* qs, int64_t sqb, int64_t sqh, int64_t sqn,
                       const void* k, int64_t skb, int64_t skh, int64_t sks, int64_t B,
                       int64_t Hq, int64_t Hk, int64_t Sk, int64_t D, int64_t q_pooling_size,
                       int64_t k_local_size, int64_t group_k_block, int causal, int wo_init,
                       int64_t J0, int64_t nc, int64_t bsq, float gap, const float* gaps,
                       int64_t dense_stride, int64_t segment_keys, int32_t* counts,
                       int32_t* indices, float* scratch, int64_t scratch_floats, void* stream);

/*
 * Compact (CSR) selection: the same selected sets as va_select, stored with
 * no padding, in two calls on one stream and with the same arguments.
 *   Counting call (indices == NULL): counts[(b*Hq + h)*nc + jr] (times nseg,
 *   plus the segment, when split) and the int64 row offsets
 *   offsets[0 .. B*Hq*nc]: offsets[0] = 0, row r = (b*Hq + h)*nc + jr holds
 *   offsets[r+1] - offsets[r] keys.  No keys are stored; the offsets are
 *   computed on the device (no host round trip).
 *   Writing call (indices != NULL, room for offsets[B*Hq*nc] int32): row r's
 *   keys in ascending order at indices[offsets[r] ..]; counts and offsets
 *   must hold the counting call's results and are left unchanged.
 * segment_keys: 0 selects each row in one pass (kernel as VA_SEL_AUTO;
 * scratch of va_select_scratch_floats, or NULL for the exact kernel), > 0
 * splits the keys as va_select_segments does (its conditions and scratch),
 * nseg = ceil(Sk / segment_keys).  The writing call runs the selection again
 * (bit-identical), so a compact list costs two selections and
 * 4*offsets[B*Hq*nc] bytes instead of the capacity layout's slots.
 * Replaces the output of fuse_qk_softmax_minp_wo_causal
 * (spattn/src/kernels/vecattention_kernels.py:131-136,178-180: a zeroed dense
 * B*H*nqb*padded_Sk int32 buffer, then trimmed to the longest row) with the
 * count / scan / write form of the same sets; the reference itself has no
 * compact output.
 */
int va_select_csr(int dtype, const void* qs, int64_t sqb, int64_t sqh, int64_t sqn,
                  const void* k, int64_t skb, int64_t skh, int64_t sks, int64_t B, int64_t Hq,
                  int64_t Hk, int64_t Sk, int64_t D, int64_t q_pooling_size, int64_t k_local_size,
                  int64_t group_k_block, int causal, int wo_init, int64_t J0, int64_t nc,
                  int64_t bsq, float gap, const float* gaps, int64_t segment_keys,
                  int32_t* counts, int64_t* offsets, int32_t* indices, float* scratch,
                  int64_t scratch_floats, void* stream);

/* fp32 scratch floats va_select's MFMA kernel needs (B*Hk key-norm slots). */
int64_t va_select_scratch_floats(int64_t B, int64_t Hk);

/* Total int32 slots of the index layout for B*Hq rows sets [J0, J0+nc). */
int64_t va_select_index_capacity(int64_t B, int64_t Hq, int64_t Sk, int64_t q_pooling_size,
                                 int causal, int wo_init, int64_t J0, int64_t nc,
                                 int64_t dense_stride);

/* Offset of row (bh = b*Hq + h, jr = J - J0) in the index layout. */
int64_t va_select_row_offset(int64_t Sk, int64_t q_pooling_size, int causal, int wo_init,
                             int64_t J0, int64_t nc, int64_t dense_stride, int64_t bh,
                             int64_t jr);

/*
 * Vector-sparse attention for q-block rows [J0, J0+nc): query row i of block J
 * attends to the local blocks of J (causal: [0,qps) and the diagonal block) and
 * the selected columns of J, with softmax scale `softmax_scale`.
 * Replaces vllm_flash_attn.sparse_attn_func as called at
 * spattn/src/VecAttention.py:104-121 (vertical + local-block semantics of
 * spattn/threshold/model_tuner.py:193-216).  Rows with no key are 0.
 * `kernel`: VA_ATTN_AUTO (MFMA for bf16/fp16, D in {64,128}, qps in {64,128};
 * for fp32 with the same D and qps and 16-byte aligned rows the fp32
 * matrix-core kernel (v_mfma_f32_32x32x2_f32, fp32 throughout); otherwise the
 * per-row kernel), VA_ATTN_MFMA (either matrix-core kernel, by dtype) or
 * VA_ATTN_SIMPLE (the per-row kernel).  The bf16/fp16 MFMA
 * kernel's loop has two forms at D = 128, qps = 64, which VA_ATTN_AUTO and
 * VA_ATTN_MFMA pick by shape: staged (two stages of a K and a V tile, two
 * work-groups per CU) and ring (three tile slots, three work-groups per CU);
 * VA_ATTN_MFMA_STAGED and VA_ATTN_MFMA_RING force one (the ring form only at
 * D = 128, qps = 64, bf16/fp16; VA_ERR_UNSUPPORTED otherwise).  Both run the
 * same arithmetic in the same order, so their outputs are bit-identical.
 */
int va_sparse_attn(int dtype, const void* q, int64_t sqb, int64_t sqh, int64_t sqs,
                   const void* k, int64_t skb, int64_t skh, int64_t sks, const void* v,
                   int64_t svb, int64_t svh, int64_t svs, void* out, int64_t sob,
                   int64_t soh, int64_t sos, int64_t B, int64_t Hq, int64_t Hk, int64_t Sq,
                   int64_t Sk, int64_t D, int64_t q_pooling_size, int causal, int wo_init,
                   int64_t J0, int64_t nc, int64_t dense_stride, const int32_t* counts,
                   const int32_t* indices, float softmax_scale, int kernel, void* stream);

/*
 * Dense attention over all keys (every key visible; causal: query row i sees
 * keys [0, i + Sk - Sq], the last query aligned with the last key, so
 * Sq <= Sk), on the same MFMA kernel as va_sparse_attn.  Replaces
 * spattn/src/Fullprefill.py:4-16 (Full_prefill, flashinfer
 * single_prefill_with_kv_cache), which the dispatcher at
 * spattn/src/models/utils.py:99-128 calls on the text tokens around a vision
 * span.  bf16/fp16, or fp32 on the fp32 matrix-core kernel (16-byte aligned
 * rows); D in {64, 128}; GQA as in va_sparse_attn.
 */
int va_dense_attn(int dtype, const void* q, int64_t sqb, int64_t sqh, int64_t sqs,
                  const void* k, int64_t skb, int64_t skh, int64_t sks, const void* v,
                  int64_t svb, int64_t svh, int64_t svs, void* out, int64_t sob, int64_t soh,
                  int64_t sos, int64_t B, int64_t Hq, int64_t Hk, int64_t Sq, int64_t Sk,
                  int64_t D, int causal, float softmax_scale, void* stream);

/*
 * Per-row softmax statistics for the threshold tuner's recall evaluation
 * (seg_pr_perHead, spattn/threshold/model_tuner.py:118-226): for each query
 * row i of head bh, stats[(bh*Sq + i)*2 + 0] = m and [+1] = l with
 * l = sum over the row's keys j of 2^(s_ij - m), s_ij = q_i.k_j *
 * softmax_scale * log2(e) (m = -inf, l = 0 for a row without keys).  m is a
 * reference level within 8 of the row maximum, not necessarily the maximum.
 *
 * va_sparse_row_stats: the keys of va_sparse_attn (local blocks + selected
 * columns, causal mask on the diagonal), rows of q-blocks [J0, J0+nc), same
 * arguments minus V and the output.  va_dense_row_stats: every key (causal:
 * j <= i + Sk - Sq), every row.  The row's attention mass on its selected
 * keys, the tuner's per-row recall (model_tuner.py:202-219), is
 * l_sparse * 2^(m_sparse - m_dense) / l_dense.  `kernel` as in
 * va_sparse_attn: MFMA for bf16/fp16 (D in {64, 128}), the per-row kernel
 * for fp32.
 */
int va_sparse_row_stats(int dtype, const void* q, int64_t sqb, int64_t sqh, int64_t sqs,
                        const void* k, int64_t skb, int64_t skh, int64_t sks, int64_t B,
                        int64_t Hq, int64_t Hk, int64_t Sq, int64_t Sk, int64_t D,
                        int64_t q_pooling_size, int causal, int wo_init, int64_t J0, int64_t nc,
                        int64_t dense_stride, const int32_t* counts, const int32_t* indices,
                        float softmax_scale, int kernel, float* stats, void* stream);
/* va_sparse_row_stats on the segmented lists of va_select_segments (counts of
 * shape (B, Hq, nc, ceil(Sk/segment_keys))), on the MFMA kernel (bf16/fp16, D
 * in {64, 128}); the statistics equal those of the concatenated lists.  No
 * counterpart in the reference: it lets the tuner's fp32 selection run split
 * on the exact kernel. */
int va_sparse_row_stats_segments(int dtype, const void* q, int64_t sqb, int64_t sqh,
                                 int64_t sqs, const void* k, int64_t skb, int64_t skh,
                                 int64_t sks, int64_t B, int64_t Hq, int64_t Hk, int64_t Sq,
                                 int64_t Sk, int64_t D, int64_t q_pooling_size, int causal,
                                 int wo_init, int64_t J0, int64_t nc, int64_t dense_stride,
                                 int64_t segment_keys, const int32_t* counts,
                                 const int32_t* indices, float softmax_scale, float* stats,
                                 void* stream);
int va_dense_row_stats(int dtype, const void* q, int64_t sqb, int64_t sqh, int64_t sqs,
                       const void* k, int64_t skb, int64_t skh, int64_t sks, int64_t B,
                       int64_t Hq, int64_t Hk, int64_t Sq, int64_t Sk, int64_t D, int causal,
                       float softmax_scale, int kernel, float* stats, void* stream);

/*
 * Decode attention: one query row per q head over the whole KV cache of its kv
 * head, no mask.  Replaces flashinfer.single_decode_with_kv_cache as called at
 * spattn/src/models/load_qwen2p5_vl.py:61-66 (kv_layout "NHD") and
 * spattn/src/models/load_llama.py:183-188 (kv_layout "HND"): out[h] =
 * softmax(q[h] . K[:, h / (Hq/Hk)]^T * softmax_scale) V[:, h / (Hq/Hk)].
 * q: (Hq, D) with head stride sqh; K/V element (n, h, d) at base + h*skh +
 * n*sks + d (NHD: skh = D, sks = Hk*D; HND: skh = L*D, sks = D); out: (Hq, D)
 * with head stride soh, q's dtype.  The MFMA path (bf16/fp16, D in {64, 128},
 * Hq/Hk <= 64) splits each kv head's L keys over work-groups and merges their
 * partial softmax states; it needs `workspace` of va_decode_workspace_size()
 * bytes (16-byte aligned).  VA_ATTN_SIMPLE (any dtype) needs none.
 */
int64_t va_decode_workspace_size(int64_t Hq, int64_t Hk, int64_t L, int64_t D);
int va_decode_attn(int dtype, const void* q, int64_t sqh, const void* k, int64_t skh,
                   int64_t sks, const void* v, int64_t svh, int64_t svs, void* out, int64_t soh,
                   int64_t Hq, int64_t Hk, int64_t L, int64_t D, float softmax_scale, int kernel,
                   void* workspace, int64_t workspace_bytes, void* stream);

/*
 * va_decode_attn without a workspace: no counterpart in the reference.  For
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  Same arguments,
 * kernels and results as va_decode_attn; the partial softmax states live in a
 * device array inside the library, one per GPU, of
 * va_decode_noalloc_scratch_bytes() bytes (8 MiB), held until the process
 * ends.  Sizes whose va_decode_workspace_size() exceeds it return
 * VA_ERR_UNSUPPORTED.  The entry point calls no allocator.  Calls on one GPU
 * share the array: calls ordered on one stream are safe, calls that overlap
 * on one GPU (unordered streams) race.
 */
int64_t va_decode_noalloc_scratch_bytes(void);
int va_decode_attn_noalloc(int dtype, const void* q, int64_t sqh, const void* k, int64_t skh,
                           int64_t sks, const void* v, int64_t svh, int64_t svs, void* out,
                           int64_t soh, int64_t Hq, int64_t Hk, int64_t L, int64_t D,
                           float softmax_scale, int kernel, void* stream);

/*
 * va_sparse_attn on the segmented lists of va_select_segments (counts of shape
 * (B, Hq, nc, ceil(Sk/segment_keys))); the bf16/fp16 MFMA kernel or the fp32
 * matrix-core kernel only.  No counterpart in the reference: it is the second
 * half of va_prefill's chunk step.
 */
int va_sparse_attn_segments(int dtype, const void* q, int64_t sqb, int64_t sqh, int64_t sqs,
                            const void* k, int64_t skb, int64_t skh, int64_t sks, const void* v,
                            int64_t svb, int64_t svh, int64_t svs, void* out, int64_t sob,
                            int64_t soh, int64_t sos, int64_t B, int64_t Hq, int64_t Hk,
                            int64_t Sq, int64_t Sk, int64_t D, int64_t q_pooling_size,
                            int causal, int wo_init, int64_t J0, int64_t nc,
                            int64_t dense_stride, int64_t segment_keys, const int32_t* counts,
                            const int32_t* indices, float softmax_scale, void* stream);

/*
 * Bytes of device workspace va_prefill needs for the same sizes and bsq
 * (256-byte aligned segments; -1 on invalid sizes).  bsq matters for causal
 * prefills only: their row groups start at multiples of bsq rows.
 */
int64_t va_prefill_workspace_size(int dtype, int64_t B, int64_t Hq, int64_t Sq, int64_t Sk,
                                  int64_t D, int64_t q_pooling_size, int causal,
                                  int64_t chunk_size, int64_t bsq);

/*
 * Kernels va_prefill runs for these tensors and parameters, as a bit set
 * (negative on invalid sizes): the selection on the certified MFMA wave kernel
 * (VA_KERNELS_SELECT_WAVE), the 64-row MFMA kernel (VA_KERNELS_SELECT_MFMA) or
 * the exact fp64 kernel (VA_KERNELS_SELECT_EXACT: fp32 inputs, D outside
 * {64, 128}, k_local_size outside {16, 32, 64, 128, 256}, unaligned K; the
 * wave kernel takes tiles of 16 to 64 keys, the 64-row MFMA kernel 128 and
 * 256); the attention on
 * the MFMA kernel (VA_KERNELS_ATTN_MFMA), for fp32 inputs the fp32 matrix-core
 * kernel (VA_KERNELS_ATTN_F32: D and q_pooling_size 64 or 128, 16-byte
 * aligned rows), or the per-row kernel (VA_KERNELS_ATTN_ROW: D or
 * q_pooling_size outside {64, 128}, K/V row strides of 16 KiB or more,
 * unaligned tensors), with VA_KERNELS_ATTN_RING
 * when that kernel runs its ring form (see va_sparse_attn); VA_KERNELS_SPLIT
 * when the selection runs in key segments (va_select_segment_keys, or
 * va_select_exact_segment_keys with VA_KERNELS_SELECT_EXACT, which splits only
 * for the fp32 matrix-core attention).  The exact selection and the per-row
 * attention are several times slower than the MFMA kernels.  No counterpart
 * in the reference: it lets callers see which path a configuration takes.
 */
#define VA_KERNELS_SELECT_WAVE 1
#define VA_KERNELS_SELECT_MFMA 2
#define VA_KERNELS_SELECT_EXACT 4
#define VA_KERNELS_ATTN_MFMA 16
#define VA_KERNELS_ATTN_ROW 32
#define VA_KERNELS_SPLIT 64
#define VA_KERNELS_ATTN_RING 128
#define VA_KERNELS_ATTN_F32 256
int va_prefill_kernels(int dtype, const void* q, int64_t sqb, int64_t sqh, int64_t sqs,
                       const void* k, int64_t skb, int64_t skh, int64_t sks, const void* v,
                       int64_t svb, int64_t svh, int64_t svs, const void* out, int64_t sob,
                       int64_t soh, int64_t sos, int64_t Hq, int64_t Hk, int64_t Sk, int64_t D,
                       int64_t q_pooling_size, int64_t k_local_size, int64_t group_k_block);

/*
 * The whole VecAttention prefill: pooling, then per query chunk selection and
 * vector-sparse attention, all on `stream` with no host synchronisation.
 * Replaces spattn/src/VecAttention.py:10-123 (VecAttention_prefill).
 * `gap`/`gaps` as in va_select.  out: (B, Hq, Sq, D) with strides.
 */
int va_prefill(int dtype, const void* q, int64_t sqb, int64_t sqh, int64_t sqs,
               const void* k, int64_t skb, int64_t skh, int64_t sks, const void* v,
               int64_t svb, int64_t svh, int64_t svs, void* out, int64_t sob, int64_t soh,
               int64_t sos, int64_t B, int64_t Hq, int64_t Hk, int64_t Sq, int64_t Sk,
               int64_t D, float gap, const float* gaps, int64_t q_pooling_size,
               int64_t k_local_size, int64_t group_k_block, int causal, int64_t chunk_size,
               int64_t bsq, void* workspace, int64_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* VECATTN_H_ */
