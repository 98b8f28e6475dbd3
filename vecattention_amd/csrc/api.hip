// C ABI of libvecattn.so: argument validation, dispatch and the fused prefill.
// Declarations and their reference counterparts: include/vecattn.h.
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <string>

#include "../../include/vecattn.h"
#include "common.h"

namespace va {
hipError_t launch_pool(int dtype, const void* q, int64_t B, int64_t H, int64_t S, int64_t D,
                       int64_t sqb, int64_t sqh, int64_t sqs, int64_t qps, void* pooled,
                       void* scaled, hipStream_t stream);
hipError_t launch_select_exact(int dtype, const void* qs, int64_t sqb, int64_t sqh,
                               int64_t sqn, const void* k,
                               int64_t skb, int64_t skh, int64_t sks, int64_t B, int64_t Hq,
                               int64_t Hk, int64_t Sk, int64_t D, int64_t qps, int64_t bk,
                               int64_t group, int causal, int64_t bsq, float gap_scalar,
                               const float* gaps, const RowLayout& lay, int32_t* counts,
                               int32_t* indices, int64_t segk, float* carry, int mode,
                               hipStream_t stream);
hipError_t launch_attn_simple(int dtype, const void* q, const int64_t* sq, const void* k,
                              const int64_t* sk, const void* v, const int64_t* sv, void* out,
                              const int64_t* so, int64_t B, int64_t Hq, int64_t Hk, int64_t Sq,
                              int64_t Sk, int64_t D, int64_t qps, int causal, float scale_log2,
                              const int32_t* counts, const int32_t* indices,
                              const RowLayout& lay, int64_t dense_qoff, float* stats,
                              hipStream_t stream);
bool attn_mfma_supported(int dtype, int64_t D, int64_t qps);
bool select_mfma_supported(int dtype, int64_t D, int64_t bk);
hipError_t launch_select_mfma(int dtype, const void* qs, int64_t sqb, int64_t sqh, int64_t sqn,
                              const void* k, int64_t skb, int64_t skh, int64_t sks, int64_t B,
                              int64_t Hq, int64_t Hk, int64_t Sk, int64_t D, int64_t qps,
                              int64_t bk, int64_t group, int causal, int64_t bsq, float gap,
                              const float* gaps, const float* kmax, const RowLayout& lay,
                              int32_t* counts, int32_t* indices, int64_t segk, hipStream_t stream);
bool select_wave_supported(int dtype, int64_t D, int64_t bk, int64_t group);
hipError_t launch_select_wave(int dtype, const void* qs, int64_t sqb, int64_t sqh, int64_t sqn,
                              const void* k, int64_t skb, int64_t skh, int64_t sks, int64_t B,
                              int64_t Hq, int64_t Hk, int64_t Sk, int64_t D, int64_t qps,
                              int64_t bk, int64_t group, int causal, int64_t bsq, float gap,
                              const float* gaps, const float* kmax, const RowLayout& lay,
                              int32_t* counts, int32_t* indices, int64_t segk, void* carry,
                              int mode, hipStream_t stream);
constexpr int64_t kSegCarryBytes = 32;  // per (row, segment) record of the two-pass selection
int64_t select_wave_segment_keys(int64_t Sk, int64_t bk, int64_t group);
int64_t select_mfma_segment_keys(int64_t Sk, int64_t bk, int64_t group);
int64_t select_wave_carry_segment_keys(int64_t Sk, int64_t bk, int64_t group);
int64_t select_exact_segment_keys(int64_t Sk, int64_t bk, int64_t group);
int64_t key_norm_scratch_floats(int64_t B, int64_t Hk);
hipError_t launch_csr_offsets(const int32_t* counts, int64_t rows, int nseg, int64_t* offsets,
                              hipStream_t stream);
hipError_t launch_key_norm(int dtype, const void* k, int64_t skb, int64_t skh, int64_t sks,
                           int64_t B, int64_t Hk, int64_t Sk, int64_t D, float* scratch,
                           hipStream_t stream);
hipError_t launch_attn_mfma(int dtype, int64_t D, int64_t qps, const void* q, const int64_t* sq,
                            const void* k, const int64_t* sk, const void* v, const int64_t* sv,
                            void* out, const int64_t* so, int64_t B, int64_t Hq, int64_t Hk,
                            int64_t Sq, int64_t Sk, int causal, float scale_log2,
                            const int32_t* counts, const int32_t* indices, const RowLayout& lay,
                            int nseg, int segk, int64_t dense_qoff, float* stats, int form,
                            hipStream_t stream);
bool attn_mfma_ring_supported(int dtype, int64_t D, int64_t qps);
bool attn_f32_supported(int64_t D, int64_t qps);
hipError_t launch_attn_f32(const void* q, const int64_t* sq, const void* k, const int64_t* sk,
                           const void* v, const int64_t* sv, void* out, const int64_t* so,
                           int64_t B, int64_t Hq, int64_t Hk, int64_t Sq, int64_t Sk, int64_t D,
                           int64_t qps, int causal, float scale_log2, const int32_t* counts,
                           const int32_t* indices, const RowLayout& lay, int nseg, int segk,
                           int64_t dense_qoff, hipStream_t stream);
bool ring_form_preferred(int64_t Hq, int64_t Hk, int64_t Sk, int64_t D);
hipError_t launch_attn_split(int dtype, int64_t D, const void* q, const int64_t* sq,
                             const void* k, const int64_t* sk, const void* v, const int64_t* sv,
                             int64_t B, int64_t H, int64_t Sq, int64_t Sk, float scale_log2,
                             int64_t nsplit, int64_t span, float* part, hipStream_t stream);
hipError_t launch_decode_merge(int dtype, int64_t D, const float* part, int64_t G, int64_t Sq,
                               int64_t nsplit, void* out, int64_t sog, int64_t sor,
                               hipStream_t stream);
}  // namespace va

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int ok() {
  g_err.clear();
  return VA_OK;
}

int hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(VA_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return VA_OK;
}

int64_t esize(int dtype) { return dtype == VA_F32 ? 4 : 2; }
bool dtype_ok(int dtype) { return dtype == VA_F32 || dtype == VA_BF16 || dtype == VA_F16; }
bool pow2(int64_t x) { return x > 0 && (x & (x - 1)) == 0; }
int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
int64_t align256(int64_t x) { return (x + 255) / 256 * 256; }
constexpr int64_t kMaxSegments = 64;  // key segments of a split selection

va::RowLayout make_layout(int64_t J0, int64_t nc, int64_t qps, int64_t Sk, int causal,
                          int wo_init, int64_t dense_stride) {
  va::RowLayout lay;
  lay.J0 = J0;
  lay.nc = nc;
  lay.qps = qps;
  lay.Sk = Sk;
  lay.dense_stride = dense_stride;
  lay.causal = causal ? 1 : 0;
  lay.wo_init = wo_init ? 1 : 0;
  return lay;
}

constexpr int64_t kMaxGrid = (int64_t(1) << 31) - 1;

int check_select_args(int dtype, const void* qs, const void* k, int64_t B, int64_t Hq,
                      int64_t Hk, int64_t Sk, int64_t D, int64_t qps, int64_t bk,
                      int64_t group, int causal, int wo_init, int64_t J0, int64_t nc,
                      int64_t bsq) {
  if (!dtype_ok(dtype)) return fail(VA_ERR_ARG, "unknown dtype %d", dtype);
  if (!qs || !k) return fail(VA_ERR_ARG, "null tensor pointer");
  if (B <= 0 || Hq <= 0 || Hk <= 0 || Sk <= 0 || D <= 0 || nc <= 0 || J0 < 0)
    return fail(VA_ERR_ARG, "non-positive size");
  if (Hq % Hk) return fail(VA_ERR_ARG, "num q heads %lld not a multiple of kv heads %lld",
                           (long long)Hq, (long long)Hk);
  if (D > 256) return fail(VA_ERR_UNSUPPORTED, "head_dim %lld > 256", (long long)D);
  if (qps <= 0) return fail(VA_ERR_ARG, "q_pooling_size must be positive");
  if (!pow2(bk) || bk < 16 || bk > 256)
    return fail(VA_ERR_UNSUPPORTED, "k_local_size %lld must be a power of two in [16, 256]",
                (long long)bk);
  if (group <= 0) return fail(VA_ERR_ARG, "group_k_block must be positive");
  if (bsq <= 0) return fail(VA_ERR_ARG, "bsq must be positive");
  if (causal && qps % bk) return fail(VA_ERR_ARG, "causal requires q_pooling_size %% k_local_size == 0");
  if (wo_init && qps % bk)
    return fail(VA_ERR_UNSUPPORTED, "wo_initial requires q_pooling_size %% k_local_size == 0");
  if (Sk >= (int64_t(1) << 31)) return fail(VA_ERR_UNSUPPORTED, "Sk does not fit int32 indices");
  if (cdiv(nc, 16) * B * Hq > kMaxGrid) return fail(VA_ERR_UNSUPPORTED, "grid too large");
  return VA_OK;
}

}  // namespace

extern "C" {

int va_version(void) { return 100; }

const char* va_last_error(void) { return g_err.c_str(); }

int va_device_count(void) {
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess) return fail(VA_ERR_HIP, "hipGetDeviceCount: %s", hipGetErrorString(e));
  if (n <= 0) return fail(VA_ERR_HIP, "no HIP device");
  ok();
  return n;
}

int va_pool(int dtype, const void* q, int64_t B, int64_t H, int64_t S, int64_t D, int64_t sqb,
            int64_t sqh, int64_t sqs, int64_t qps, void* pooled, void* scaled, void* stream) {
  if (!dtype_ok(dtype)) return fail(VA_ERR_ARG, "unknown dtype %d", dtype);
  if (!q) return fail(VA_ERR_ARG, "null q");
  if (B <= 0 || H <= 0 || S <= 0 || D <= 0 || qps <= 0) return fail(VA_ERR_ARG, "non-positive size");
  if (D > 256) return fail(VA_ERR_UNSUPPORTED, "head_dim %lld > 256", (long long)D);
  if (B * H > 65535) return fail(VA_ERR_UNSUPPORTED, "B*H > 65535");
  if (!pooled && !scaled) return ok();
  int rc = hip_check(va::launch_pool(dtype, q, B, H, S, D, sqb, sqh, sqs, qps, pooled, scaled,
                                     static_cast<hipStream_t>(stream)),
                     "pool launch");
  return rc ? rc : ok();
}

int64_t va_select_index_capacity(int64_t B, int64_t Hq, int64_t Sk, int64_t qps, int causal,
                                 int wo_init, int64_t J0, int64_t nc, int64_t dense_stride) {
  if (B <= 0 || Hq <= 0 || Sk <= 0 || qps <= 0 || nc <= 0 || J0 < 0) return -1;
  return B * Hq * make_layout(J0, nc, qps, Sk, causal, wo_init, dense_stride).block_size();
}

int64_t va_select_row_offset(int64_t Sk, int64_t qps, int causal, int wo_init, int64_t J0,
                             int64_t nc, int64_t dense_stride, int64_t bh, int64_t jr) {
  if (Sk <= 0 || qps <= 0 || nc <= 0 || J0 < 0 || jr < 0 || jr > nc || bh < 0) return -1;
  return make_layout(J0, nc, qps, Sk, causal, wo_init, dense_stride).row_offset(bh, jr);
}

int64_t va_select_scratch_floats(int64_t B, int64_t Hk) {
  if (B <= 0 || Hk <= 0) return -1;
  return va::key_norm_scratch_floats(B, Hk);
}

// A group longer than the key range is a single group: any value covering
// every tile gives the same selection.  Capped so that bk * group stays small,
// and to a multiple of 4 tiles so that a capped span is a multiple of 64 keys
// (the wave kernel takes spans of 16 or 32 keys or multiples of 64).
static int64_t effective_group(int64_t group, int64_t Sk, int64_t bk) {
  const int64_t gmax = (cdiv(Sk, bk) + 1 + 3) / 4 * 4;
  return group > gmax ? gmax : group;
}

enum SelKernel { kSelExact = VA_SEL_EXACT, kSelMfma = VA_SEL_MFMA, kSelWave = VA_SEL_WAVE };

// Selection with the key norms (MFMA paths) already in kmax[0 .. B*Hk).
static int select_impl(int dtype, const void* qs, int64_t sqb, int64_t sqh, int64_t sqn,
                       const void* k, int64_t skb, int64_t skh, int64_t sks, int64_t B,
                       int64_t Hq, int64_t Hk, int64_t Sk, int64_t D, int64_t qps, int64_t bk,
                       int64_t group, int causal, int wo_init, int64_t J0, int64_t nc,
                       int64_t bsq, float gap, const float* gaps, int64_t dense_stride,
                       int32_t* counts, int32_t* indices, SelKernel which, const float* kmax,
                       int64_t segk, hipStream_t stream, void* carry = nullptr,
                       int mode = 0, const int64_t* csr = nullptr,
                       const int32_t* seg_counts = nullptr) {
  va::RowLayout lay = make_layout(J0, nc, qps, Sk, causal, wo_init, dense_stride);
  lay.csr = csr;  // compact output (non-null) instead of the capacity layout
  lay.seg_counts = seg_counts;
  group = effective_group(group, Sk, bk);
  hipError_t e;
  if (which == kSelWave)
    e = va::launch_select_wave(dtype, qs, sqb, sqh, sqn, k, skb, skh, sks, B, Hq, Hk, Sk, D, qps,
                               bk, group, causal, bsq, gap, gaps, kmax, lay, counts, indices,
                               segk, carry, mode, stream);
  else if (which == kSelMfma)
    e = va::launch_select_mfma(dtype, qs, sqb, sqh, sqn, k, skb, skh, sks, B, Hq, Hk, Sk, D, qps,
                               bk, group, causal, bsq, gap, gaps, kmax, lay, counts, indices,
                               segk, stream);
  else
    e = va::launch_select_exact(dtype, qs, sqb, sqh, sqn, k, skb, skh, sks, B, Hq, Hk, Sk, D,
                                qps, bk, group, causal, bsq, gap, gaps, lay, counts, indices,
                                segk, static_cast<float*>(carry), mode, stream);
  return hip_check(e, "select launch");
}

static bool select_mfma_ok(int dtype, const void* qs, int64_t sqb, int64_t sqh, int64_t sqn,
                           const void* k, int64_t skb, int64_t skh, int64_t sks, int64_t D,
                           int64_t bk) {
  const int64_t a = 16 / esize(dtype);
  return va::select_mfma_supported(dtype, D, bk) && reinterpret_cast<uintptr_t>(qs) % 16 == 0 &&
         reinterpret_cast<uintptr_t>(k) % 16 == 0 && sqb % a == 0 && sqh % a == 0 &&
         sqn % a == 0 && skb % a == 0 && skh % a == 0 && sks % a == 0;
}

// The wave kernel copies K rows into LDS with 32-bit buffer offsets computed
// from keys up to Sk + 64: each kv head's rows (and one chunk past the end)
// must span < 2 GiB, and rows must not overlap (sks >= D).
static bool select_wave_ok(int dtype, const void* qs, int64_t sqb, int64_t sqh, int64_t sqn,
                           const void* k, int64_t skb, int64_t skh, int64_t sks, int64_t Sk,
                           int64_t D, int64_t bk, int64_t group) {
  return select_mfma_ok(dtype, qs, sqb, sqh, sqn, k, skb, skh, sks, D, bk) &&
         va::select_wave_supported(dtype, D, bk, effective_group(group, Sk, bk)) && sks >= D &&
         Sk < (int64_t(1) << 24) && (Sk + 64) * sks * esize(dtype) < (int64_t(1) << 31);
}

// The wave kernel starts a row's scan at the 64-key chunk holding its first
// selectable key (smin) and keeps the running maximum of the keys below smin at
// -inf; its sign-bit decisions assume that no visited chunk starts with such
// keys, i.e. smin is a multiple of 64 (always so for q_pooling_size 64 or 128).
static bool first_key_aligned(int64_t qps, int64_t Sk, int causal, int wo_init) {
  const int64_t smin = !wo_init ? 0 : (causal ? qps : (qps < Sk ? qps : Sk));
  return smin % 64 == 0;
}

int va_select(int dtype, const void* qs, int64_t sqb, int64_t sqh, int64_t sqn,
              const void* k, int64_t skb, int64_t skh, int64_t sks, int64_t B, int64_t Hq,
              int64_t Hk, int64_t Sk, int64_t D, int64_t qps, int64_t bk, int64_t group,
              int causal, int wo_init, int64_t J0, int64_t nc, int64_t bsq, float gap,
              const float* gaps, int64_t dense_stride, int32_t* counts, int32_t* indices,
              int kernel, float* scratch, int64_t scratch_floats, void* stream) {
  int rc = check_select_args(dtype, qs, k, B, Hq, Hk, Sk, D, qps, bk, group, causal, wo_init, J0,
                             nc, bsq);
  if (rc) return rc;
  if (!counts || !indices) return fail(VA_ERR_ARG, "null output pointer");
  if (dense_stride < 0) return fail(VA_ERR_ARG, "negative dense_stride");
  if (dense_stride > 0 && dense_stride < Sk)
    return fail(VA_ERR_ARG, "dense_stride %lld < Sk %lld", (long long)dense_stride, (long long)Sk);
  const bool have_scratch = scratch != nullptr &&
                            scratch_floats >= va::key_norm_scratch_floats(B, Hk);
  const bool mfma_ok = select_mfma_ok(dtype, qs, sqb, sqh, sqn, k, skb, skh, sks, D, bk);
  const bool wave_ok =
      select_wave_ok(dtype, qs, sqb, sqh, sqn, k, skb, skh, sks, Sk, D, bk, group) &&
      first_key_aligned(qps, Sk, causal, wo_init);
  SelKernel which;
  if (kernel == VA_SEL_EXACT) {
    which = kSelExact;
  } else if (kernel == VA_SEL_MFMA || kernel == VA_SEL_WAVE) {
    if (kernel == VA_SEL_MFMA && !mfma_ok)
      return fail(VA_ERR_UNSUPPORTED,
                  "MFMA selection needs bf16/fp16, D in {64,128}, k_local_size in {16,32,64} "
                  "and 16-byte aligned rows");
    if (kernel == VA_SEL_WAVE && !wave_ok)
      return fail(VA_ERR_UNSUPPORTED,
                  "wave selection needs bf16/fp16, D in {64,128}, k_local_size in {16,32,64}, "
                  "k_local_size * group_k_block 16, 32 or a multiple of 64, 16-byte aligned "
                  "rows, "
                  "Sk < 2^24, < 2 GiB of key rows per kv head and a first selectable key "
                  "at a multiple of 64");
    if (!have_scratch) return fail(VA_ERR_ARG, "MFMA selection needs scratch");
    which = kernel == VA_SEL_WAVE ? kSelWave : kSelMfma;
  } else if (kernel == VA_SEL_AUTO) {
    which = (wave_ok && have_scratch) ? kSelWave : (mfma_ok && have_scratch) ? kSelMfma : kSelExact;
  } else {
    return fail(VA_ERR_ARG, "unknown selection kernel %d", kernel);
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (which != kSelExact) {
    rc = hip_check(va::launch_key_norm(dtype, k, skb, skh, sks, B, Hk, Sk, D, scratch, st),
                   "key norm launch");
    if (rc) return rc;
  }
  rc = select_impl(dtype, qs, sqb, sqh, sqn, k, skb, skh, sks, B, Hq, Hk, Sk, D, qps, bk, group,
                   causal, wo_init, J0, nc, bsq, gap, gaps, dense_stride, counts, indices, which,
                   scratch, 0, st);
  return rc ? rc : ok();
}

// Segments of the split selection.  The segment length must be a multiple of
// the 64-key chunk and of the group span (one pass), or the groups must cover
// every key of a row (two passes, carried maxima), with at most 64 segments.
int64_t va_select_segment_keys(int64_t Sk, int64_t k_local_size, int64_t group_k_block) {
  if (Sk <= 0 || k_local_size <= 0 || group_k_block <= 0) return -1;
  const int64_t g = effective_group(group_k_block, Sk, k_local_size);
  const int64_t segk = va::select_wave_segment_keys(Sk, k_local_size, g);
  if (segk > 0) return segk;
  // tiles and groups the wave kernel takes (bf16/fp16, D 64 or 128): its
  // two-pass split; others run on the 64-row MFMA kernel's split
  if (va::select_wave_supported(VA_BF16, 128, k_local_size, g))
    return va::select_wave_carry_segment_keys(Sk, k_local_size, g);
  return va::select_mfma_segment_keys(Sk, k_local_size, g);
}

int64_t va_select_exact_segment_keys(int64_t Sk, int64_t k_local_size, int64_t group_k_block) {
  if (Sk <= 0 || k_local_size <= 0 || group_k_block <= 0) return -1;
  return va::select_exact_segment_keys(Sk, k_local_size,
                                       effective_group(group_k_block, Sk, k_local_size));
}

// The two-pass form: the groups cover every key of a row and the segments do
// not start groups.
static bool segments_two_pass(int64_t Sk, int64_t bk, int64_t group, int64_t segment_keys) {
  const int64_t gs = bk * effective_group(group, Sk, bk);
  return segment_keys % gs != 0 && gs >= Sk;
}

int64_t va_select_segments_scratch_floats(int64_t B, int64_t Hq, int64_t Hk, int64_t Sk,
                                          int64_t nc, int64_t segment_keys,
                                          int64_t k_local_size, int64_t group_k_block) {
  if (B <= 0 || Hq <= 0 || Hk <= 0 || Sk <= 0 || nc <= 0 || segment_keys <= 0 ||
      k_local_size <= 0 || group_k_block <= 0)
    return -1;
  const int64_t kn = (va::key_norm_scratch_floats(B, Hk) + 7) / 8 * 8;  // 32-byte aligned
  if (!segments_two_pass(Sk, k_local_size, group_k_block, segment_keys)) return kn;
  return kn + va::kSegCarryBytes / 4 * B * Hq * nc * cdiv(Sk, segment_keys);  // carry records
}

// Kernel and passes of a split selection: segment lengths that are multiples
// of 64 and of the group span (one pass), or any multiple of 64 when one
// group covers the row (maxima pass, then carry pass), at most 64 segments.
// The wave kernel takes every split; the 64-row MFMA kernel (tiles of 128 and
// 256 keys) takes segments of whole 256-key chunks that start groups; the
// exact kernel (other inputs, fp32 among them) takes every split.
static int plan_segments(int dtype, const void* qs, int64_t sqb, int64_t sqh, int64_t sqn,
                         const void* k, int64_t skb, int64_t skh, int64_t sks, int64_t B,
                         int64_t Hq, int64_t Hk, int64_t Sk, int64_t D, int64_t qps, int64_t bk,
                         int64_t group, int causal, int wo_init, int64_t nc,
                         int64_t segment_keys, const float* scratch, int64_t scratch_floats,
                         SelKernel& which, bool& two_pass) {
  const int64_t gs = bk * effective_group(group, Sk, bk);
  if (segment_keys <= 0 || segment_keys % 64 || cdiv(Sk, segment_keys) > 64 ||
      (segment_keys % gs != 0 && gs < Sk))
    return fail(VA_ERR_ARG, "segment_keys %lld: need a multiple of 64 and of the group span "
                            "(%lld keys) unless one group covers the row, at most 64 segments",
                (long long)segment_keys, (long long)gs);
  two_pass = segments_two_pass(Sk, bk, group, segment_keys);
  which = (select_wave_ok(dtype, qs, sqb, sqh, sqn, k, skb, skh, sks, Sk, D, bk, group) &&
           first_key_aligned(qps, Sk, causal, wo_init))
              ? kSelWave
          : (!two_pass && segment_keys % 256 == 0 &&
             select_mfma_ok(dtype, qs, sqb, sqh, sqn, k, skb, skh, sks, D, bk))
              ? kSelMfma
              : kSelExact;
  // exact kernel: up to 16 rows per work-group, one work-group per (rows, segment)
  if (which == kSelExact && cdiv(nc, 16) * cdiv(Sk, segment_keys) * B * Hq > (int64_t(1) << 24))
    return fail(VA_ERR_UNSUPPORTED, "grid too large");
  const int64_t need = va_select_segments_scratch_floats(B, Hq, Hk, Sk, nc, segment_keys, bk, group);
  if (!scratch || scratch_floats < need)
    return fail(VA_ERR_ARG, "segmented selection needs %lld scratch floats", (long long)need);
  return VA_OK;
}

int va_select_segments(int dtype, const void* qs, int64_t sqb, int64_t sqh, int64_t sqn,
                       const void* k, int64_t skb, int64_t skh, int64_t sks, int64_t B,
                       int64_t Hq, int64_t Hk, int64_t Sk, int64_t D, int64_t qps, int64_t bk,
                       int64_t group, int causal, int wo_init, int64_t J0, int64_t nc, int64_t bsq,
                       float gap, const float* gaps, int64_t dense_stride, int64_t segment_keys,
                       int32_t* counts, int32_t* indices, float* scratch, int64_t scratch_floats,
                       void* stream) {
  int rc = check_select_args(dtype, qs, k, B, Hq, Hk, Sk, D, qps, bk, group, causal, wo_init, J0,
                             nc, bsq);
  if (rc) return rc;
  if (!counts || !indices) return fail(VA_ERR_ARG, "null output pointer");
  if (dense_stride < 0 || (dense_stride > 0 && dense_stride < Sk))
    return fail(VA_ERR_ARG, "invalid dense_stride");
  SelKernel which;
  bool two_pass;
  rc = plan_segments(dtype, qs, sqb, sqh, sqn, k, skb, skh, sks, B, Hq, Hk, Sk, D, qps, bk, group,
                     causal, wo_init, nc, segment_keys, scratch, scratch_floats, which, two_pass);
  if (rc) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (which != kSelExact) {
    rc = hip_check(va::launch_key_norm(dtype, k, skb, skh, sks, B, Hk, Sk, D, scratch, st),
                   "key norm launch");
    if (rc) return rc;
  }
  void* carry = scratch + (va::key_norm_scratch_floats(B, Hk) + 7) / 8 * 8;
  if (two_pass) {
    rc = select_impl(dtype, qs, sqb, sqh, sqn, k, skb, skh, sks, B, Hq, Hk, Sk, D, qps, bk, group,
                     causal, wo_init, J0, nc, bsq, gap, gaps, dense_stride, counts, indices,
                     which, scratch, segment_keys, st, carry, va::kPassMax);
    if (rc) return rc;
  }
  rc = select_impl(dtype, qs, sqb, sqh, sqn, k, skb, skh, sks, B, Hq, Hk, Sk, D, qps, bk, group,
                   causal, wo_init, J0, nc, bsq, gap, gaps, dense_stride, counts, indices,
                   which, scratch, segment_keys, st, carry,
                   two_pass ? va::kPassCarry : va::kPassPlain);
  return rc ? rc : ok();
}

int va_select_csr(int dtype, const void* qs, int64_t sqb, int64_t sqh, int64_t sqn,
                  const void* k, int64_t skb, int64_t skh, int64_t sks, int64_t B, int64_t Hq,
                  int64_t Hk, int64_t Sk, int64_t D, int64_t qps, int64_t bk, int64_t group,
                  int causal, int wo_init, int64_t J0, int64_t nc, int64_t bsq, float gap,
                  const float* gaps, int64_t segment_keys, int32_t* counts, int64_t* offsets,
                  int32_t* indices, float* scratch, int64_t scratch_floats, void* stream) {
  int rc = check_select_args(dtype, qs, k, B, Hq, Hk, Sk, D, qps, bk, group, causal, wo_init, J0,
                             nc, bsq);
  if (rc) return rc;
  if (!counts || !offsets) return fail(VA_ERR_ARG, "null counts or offsets");
  if (segment_keys < 0) return fail(VA_ERR_ARG, "negative segment_keys");
  SelKernel which;
  bool two_pass = false;
  int64_t nseg = 1;
  if (segment_keys > 0) {
    rc = plan_segments(dtype, qs, sqb, sqh, sqn, k, skb, skh, sks, B, Hq, Hk, Sk, D, qps, bk,
                       group, causal, wo_init, nc, segment_keys, scratch, scratch_floats, which,
                       two_pass);
    if (rc) return rc;
    nseg = cdiv(Sk, segment_keys);
  } else {
    // every kernel selects the same keys: the counting and the writing call
    // agree even when only one of them is given scratch
    const bool have_scratch = scratch != nullptr &&
                              scratch_floats >= va::key_norm_scratch_floats(B, Hk);
    const bool wave = select_wave_ok(dtype, qs, sqb, sqh, sqn, k, skb, skh, sks, Sk, D, bk,
                                     group) &&
                      first_key_aligned(qps, Sk, causal, wo_init);
    which = (wave && have_scratch) ? kSelWave
            : (select_mfma_ok(dtype, qs, sqb, sqh, sqn, k, skb, skh, sks, D, bk) && have_scratch)
                ? kSelMfma
                : kSelExact;
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (which != kSelExact) {
    rc = hip_check(va::launch_key_norm(dtype, k, skb, skh, sks, B, Hk, Sk, D, scratch, st),
                   "key norm launch");
    if (rc) return rc;
  }
  void* carry = scratch ? scratch + (va::key_norm_scratch_floats(B, Hk) + 7) / 8 * 8 : nullptr;
  const bool write = indices != nullptr;
  if (two_pass) {  // the maxima pass stores neither counts nor keys
    rc = select_impl(dtype, qs, sqb, sqh, sqn, k, skb, skh, sks, B, Hq, Hk, Sk, D, qps, bk, group,
                     causal, wo_init, J0, nc, bsq, gap, gaps, 0, nullptr, nullptr, which,
                     scratch, segment_keys, st, carry, va::kPassMax);
    if (rc) return rc;
  }
  // Counting call: counts only (no keys stored), then the offsets.  Writing
  // call: the keys, at the offsets and segment counts of the counting call.
  rc = select_impl(dtype, qs, sqb, sqh, sqn, k, skb, skh, sks, B, Hq, Hk, Sk, D, qps, bk, group,
                   causal, wo_init, J0, nc, bsq, gap, gaps, 0, write ? nullptr : counts, indices,
                   which, scratch, segment_keys, st, carry,
                   two_pass ? va::kPassCarry : va::kPassPlain, write ? offsets : nullptr,
                   write ? counts : nullptr);
  if (rc) return rc;
  if (!write) {
    rc = hip_check(va::launch_csr_offsets(counts, B * Hq * nc, int(nseg), offsets, st),
                   "offsets launch");
    if (rc) return rc;
  }
  return ok();
}

// Whether the MFMA attention kernel can run these operands: bf16/fp16, D in
// {64,128}, qps in {64,128}, 16-byte aligned rows, and K/V rows it can gather
// with 32-bit buffer offsets computed by 24-bit multiplies (each kv head's
// rows span < 2 GiB, keys and row strides in bytes below 2^24).
struct AttnMfmaCheck {
  bool shape, align, span;
  bool ok() const { return shape && align && span; }
};
static AttnMfmaCheck attn_mfma_check(int dtype, const void* q, const int64_t* sq, const void* k,
                                     const int64_t* sk, const void* v, const int64_t* sv,
                                     const void* out, const int64_t* so, int64_t Sk, int64_t D,
                                     int64_t qps) {
  const int64_t es = esize(dtype);
  auto aligned = [&](const void* p, const int64_t* s, int64_t a) {
    return reinterpret_cast<uintptr_t>(p) % 16 == 0 && s[0] % a == 0 && s[1] % a == 0 &&
           s[2] % a == 0;
  };
  // The kernel addresses K and V rows through buffer resources whose record
  // stride (the row stride in bytes) is a 14-bit field.
  auto span_ok = [&](const int64_t* s) {
    return Sk < (int64_t(1) << 24) && s[2] >= 0 && s[2] * es < (int64_t(1) << 14) &&
           ((Sk - 1) * s[2] + D) * es < (int64_t(1) << 31);
  };
  AttnMfmaCheck c;
  c.shape = va::attn_mfma_supported(dtype, D, qps);
  c.align = aligned(q, sq, 16 / es) && aligned(k, sk, 16 / es) && aligned(v, sv, 16 / es) &&
            aligned(out, so, 8 / es);
  c.span = span_ok(sk) && span_ok(sv);
  return c;
}

// Whether the fp32 matrix-core attention takes these operands: fp32, D in
// {64, 128}, qps in {64, 128}, rows 16-byte aligned (it loads float4 runs of
// Q, K and V rows and stores float4 runs of output rows).
static bool attn_f32_ok(int dtype, const void* q, const int64_t* sq, const void* k,
                        const int64_t* sk, const void* v, const int64_t* sv, const void* out,
                        const int64_t* so, int64_t D, int64_t qps) {
  auto aligned = [](const void* p, const int64_t* st) {
    return reinterpret_cast<uintptr_t>(p) % 16 == 0 && st[0] % 4 == 0 && st[1] % 4 == 0 &&
           st[2] % 4 == 0;
  };
  return dtype == VA_F32 && va::attn_f32_supported(D, qps) && aligned(q, sq) && aligned(k, sk) &&
         aligned(v, sv) && aligned(out, so);
}

static int attn_dispatch(int dtype, const void* q, const int64_t* sq, const void* k,
                         const int64_t* sk, const void* v, const int64_t* sv, void* out,
                         const int64_t* so, int64_t B, int64_t Hq, int64_t Hk, int64_t Sq,
                         int64_t Sk, int64_t D, int64_t qps, int causal,
                         const va::RowLayout& lay, const int32_t* counts,
                         const int32_t* indices, float softmax_scale, int kernel, int nseg,
                         int64_t segk, hipStream_t stream, float* stats = nullptr) {
  const float scale_log2 = softmax_scale * 1.4426950408889634f;
  // Row statistics read no V and write no output: only q and k are checked.
  const AttnMfmaCheck chk = stats ? attn_mfma_check(dtype, q, sq, k, sk, k, sk, q, sq, Sk, D, qps)
                                  : attn_mfma_check(dtype, q, sq, k, sk, v, sv, out, so, Sk, D, qps);
  const bool mfma_shape = chk.shape, mfma_align = chk.align, mfma_span = chk.span;
  bool use_mfma = false;
  int form = va::kAttnFormAuto;
  if (kernel == VA_ATTN_MFMA_STAGED || kernel == VA_ATTN_MFMA_RING) {
    if (kernel == VA_ATTN_MFMA_RING && (stats || !va::attn_mfma_ring_supported(dtype, D, qps)))
      return fail(VA_ERR_UNSUPPORTED, "the ring form needs bf16/fp16, D = 128, qps = 64 and "
                                      "attention output (not row statistics)");
    form = kernel == VA_ATTN_MFMA_RING ? va::kAttnFormRing : va::kAttnFormStaged;
    kernel = VA_ATTN_MFMA;
  }
  // fp32 inputs: the fp32 matrix-core kernel (attention output), else the
  // per-row kernel
  const bool f32 = !stats && attn_f32_ok(dtype, q, sq, k, sk, v, sv, out, so, D, qps);
  bool use_f32 = false;
  if (form != va::kAttnFormAuto && dtype == VA_F32)
    return fail(VA_ERR_UNSUPPORTED, "the staged and ring forms are the bf16/fp16 MFMA kernel's");
  if (kernel == VA_ATTN_MFMA && dtype == VA_F32) {
    if (!f32)
      return fail(VA_ERR_UNSUPPORTED, "fp32 MFMA attention needs D in {64,128}, qps in {64,128}, "
                                      "16-byte aligned rows and attention output");
    use_f32 = true;
  } else if (kernel == VA_ATTN_MFMA) {
    if (!mfma_shape)
      return fail(VA_ERR_UNSUPPORTED, "MFMA attention needs bf16/fp16, D in {64,128}, qps in {64,128}");
    if (!mfma_align) return fail(VA_ERR_UNSUPPORTED, "MFMA attention needs 16-byte aligned rows");
    if (!mfma_span)
      return fail(VA_ERR_UNSUPPORTED, "MFMA attention needs Sk < 2^24, K/V row strides "
                                      "< 16 KiB and < 2 GiB of rows per kv head");
    if (!(softmax_scale > 0.f))
      return fail(VA_ERR_UNSUPPORTED, "MFMA attention needs a positive softmax scale");
    use_mfma = true;
  } else if (kernel == VA_ATTN_AUTO) {
    use_mfma = mfma_shape && mfma_align && mfma_span && softmax_scale > 0.f;
    use_f32 = !use_mfma && f32;
  } else if (kernel != VA_ATTN_SIMPLE) {
    return fail(VA_ERR_ARG, "unknown kernel selector %d", kernel);
  }
  if (!use_mfma && qps > 1024) return fail(VA_ERR_UNSUPPORTED, "q_pooling_size > 1024");
  if (!use_mfma && !use_f32 && nseg > 1)
    return fail(VA_ERR_UNSUPPORTED, "segmented key lists need a matrix-core attention kernel");
  if (use_f32)
    return hip_check(va::launch_attn_f32(q, sq, k, sk, v, sv, out, so, B, Hq, Hk, Sq, Sk, D, qps,
                                         causal, scale_log2, counts, indices, lay, nseg,
                                         int(segk), -1, stream),
                     "attention launch");
  hipError_t e = use_mfma
                     ? va::launch_attn_mfma(dtype, D, qps, q, sq, k, sk, v, sv, out, so, B, Hq,
                                            Hk, Sq, Sk, causal, scale_log2, counts, indices, lay,
                                            nseg, int(segk), -1, stats, form, stream)
                     : va::launch_attn_simple(dtype, q, sq, k, sk, v, sv, out, so, B, Hq, Hk, Sq,
                                              Sk, D, qps, causal, scale_log2, counts, indices,
                                              lay, -1, stats, stream);
  return hip_check(e, "attention launch");
}

static int sparse_attn_impl(int dtype, const void* q, int64_t sqb, int64_t sqh, int64_t sqs,
                            const void* k, int64_t skb, int64_t skh, int64_t sks, const void* v,
                            int64_t svb, int64_t svh, int64_t svs, void* out, int64_t sob,
                            int64_t soh, int64_t sos, int64_t B, int64_t Hq, int64_t Hk,
                            int64_t Sq, int64_t Sk, int64_t D, int64_t qps, int causal,
                            int wo_init, int64_t J0, int64_t nc, int64_t dense_stride,
                            const int32_t* counts, const int32_t* indices, float softmax_scale,
                            int kernel, int nseg, int64_t segk, void* stream,
                            float* stats = nullptr) {
  if (!dtype_ok(dtype)) return fail(VA_ERR_ARG, "unknown dtype %d", dtype);
  if (!q || !k || (!stats && (!v || !out))) return fail(VA_ERR_ARG, "null tensor pointer");
  if ((counts == nullptr) != (indices == nullptr))
    return fail(VA_ERR_ARG, "counts and indices must both be given or both be NULL");
  if (B <= 0 || Hq <= 0 || Hk <= 0 || Sq <= 0 || Sk <= 0 || D <= 0 || qps <= 0 || nc <= 0 || J0 < 0)
    return fail(VA_ERR_ARG, "non-positive size");
  if (Hq % Hk) return fail(VA_ERR_ARG, "num q heads not a multiple of kv heads");
  if (D > 256) return fail(VA_ERR_UNSUPPORTED, "head_dim %lld > 256", (long long)D);
  if (causal && Sq != Sk) return fail(VA_ERR_UNSUPPORTED, "causal attention needs Sq == Sk");
  if (J0 + nc > cdiv(Sq, qps)) return fail(VA_ERR_ARG, "rows [J0, J0+nc) exceed q blocks");
  if (nc * B * Hq > kMaxGrid) return fail(VA_ERR_UNSUPPORTED, "grid too large");
  const int64_t sq[3] = {sqb, sqh, sqs}, sk[3] = {skb, skh, sks}, sv[3] = {svb, svh, svs},
                so[3] = {sob, soh, sos};
  const va::RowLayout lay = make_layout(J0, nc, qps, Sk, causal, wo_init, dense_stride);
  int rc = attn_dispatch(dtype, q, sq, k, sk, v, sv, out, so, B, Hq, Hk, Sq, Sk, D, qps, causal,
                         lay, counts, indices, softmax_scale, kernel, nseg, segk,
                         static_cast<hipStream_t>(stream), stats);
  return rc ? rc : ok();
}

int va_sparse_attn(int dtype, const void* q, int64_t sqb, int64_t sqh, int64_t sqs,
                   const void* k, int64_t skb, int64_t skh, int64_t sks, const void* v,
                   int64_t svb, int64_t svh, int64_t svs, void* out, int64_t sob, int64_t soh,
                   int64_t sos, int64_t B, int64_t Hq, int64_t Hk, int64_t Sq, int64_t Sk,
                   int64_t D, int64_t qps, int causal, int wo_init, int64_t J0, int64_t nc,
                   int64_t dense_stride, const int32_t* counts, const int32_t* indices,
                   float softmax_scale, int kernel, void* stream) {
  return sparse_attn_impl(dtype, q, sqb, sqh, sqs, k, skb, skh, sks, v, svb, svh, svs, out, sob,
                          soh, sos, B, Hq, Hk, Sq, Sk, D, qps, causal, wo_init, J0, nc,
                          dense_stride, counts, indices, softmax_scale, kernel, 1, 0, stream);
}

int va_dense_attn(int dtype, const void* q, int64_t sqb, int64_t sqh, int64_t sqs,
                  const void* k, int64_t skb, int64_t skh, int64_t sks, const void* v,
                  int64_t svb, int64_t svh, int64_t svs, void* out, int64_t sob, int64_t soh,
                  int64_t sos, int64_t B, int64_t Hq, int64_t Hk, int64_t Sq, int64_t Sk,
                  int64_t D, int causal, float softmax_scale, void* stream) {
  if (!dtype_ok(dtype)) return fail(VA_ERR_ARG, "unknown dtype %d", dtype);
  if (!q || !k || !v || !out) return fail(VA_ERR_ARG, "null tensor pointer");
  if (B <= 0 || Hq <= 0 || Hk <= 0 || Sq <= 0 || Sk <= 0 || D <= 0)
    return fail(VA_ERR_ARG, "non-positive size");
  if (Hq % Hk) return fail(VA_ERR_ARG, "num q heads not a multiple of kv heads");
  if (causal && Sq > Sk) return fail(VA_ERR_ARG, "causal attention needs Sq <= Sk");
  constexpr int64_t qps = 64;
  const int64_t nc = cdiv(Sq, qps);
  if (nc * B * Hq > kMaxGrid) return fail(VA_ERR_UNSUPPORTED, "grid too large");
  const int64_t sq[3] = {sqb, sqh, sqs}, sk[3] = {skb, skh, sks}, sv[3] = {svb, svh, svs},
                so[3] = {sob, soh, sos};
  if (dtype == VA_F32) {  // the fp32 matrix-core kernel over every key
    if (!attn_f32_ok(dtype, q, sq, k, sk, v, sv, out, so, D, qps))
      return fail(VA_ERR_UNSUPPORTED, "fp32 dense attention needs D in {64, 128} and 16-byte "
                                      "aligned rows");
    const va::RowLayout lay = make_layout(0, nc, qps, Sk, causal, 0, 0);
    const int rc = hip_check(
        va::launch_attn_f32(q, sq, k, sk, v, sv, out, so, B, Hq, Hk, Sq, Sk, D, qps, causal,
                            softmax_scale * 1.4426950408889634f, nullptr, nullptr, lay, 1, 0,
                            causal ? Sk - Sq : 0, static_cast<hipStream_t>(stream)),
        "dense attention launch");
    return rc ? rc : ok();
  }
  const AttnMfmaCheck chk = attn_mfma_check(dtype, q, sq, k, sk, v, sv, out, so, Sk, D, qps);
  if (!chk.shape)
    return fail(VA_ERR_UNSUPPORTED, "dense attention needs bf16/fp16/fp32 and D in {64, 128}");
  if (!chk.align) return fail(VA_ERR_UNSUPPORTED, "dense attention needs 16-byte aligned rows");
  if (!chk.span)
    return fail(VA_ERR_UNSUPPORTED, "dense attention needs Sk < 2^24, K/V row strides < 16 KiB "
                                    "and < 2 GiB of rows per kv head");
  if (!(softmax_scale > 0.f)) return fail(VA_ERR_UNSUPPORTED, "softmax scale must be positive");
  const va::RowLayout lay = make_layout(0, nc, qps, Sk, causal, 0, 0);
  const hipError_t e = va::launch_attn_mfma(
      dtype, D, qps, q, sq, k, sk, v, sv, out, so, B, Hq, Hk, Sq, Sk, causal,
      softmax_scale * 1.4426950408889634f, nullptr, nullptr, lay, 1, 0,
      causal ? Sk - Sq : 0, nullptr, va::kAttnFormAuto, static_cast<hipStream_t>(stream));
  const int rc = hip_check(e, "dense attention launch");
  return rc ? rc : ok();
}

int va_sparse_row_stats(int dtype, const void* q, int64_t sqb, int64_t sqh, int64_t sqs,
                        const void* k, int64_t skb, int64_t skh, int64_t sks, int64_t B,
                        int64_t Hq, int64_t Hk, int64_t Sq, int64_t Sk, int64_t D, int64_t qps,
                        int causal, int wo_init, int64_t J0, int64_t nc, int64_t dense_stride,
                        const int32_t* counts, const int32_t* indices, float softmax_scale,
                        int kernel, float* stats, void* stream) {
  if (!stats) return fail(VA_ERR_ARG, "null stats");
  return sparse_attn_impl(dtype, q, sqb, sqh, sqs, k, skb, skh, sks, nullptr, 0, 0, 0, nullptr, 0,
                          0, 0, B, Hq, Hk, Sq, Sk, D, qps, causal, wo_init, J0, nc, dense_stride,
                          counts, indices, softmax_scale, kernel, 1, 0, stream, stats);
}

int va_sparse_row_stats_segments(int dtype, const void* q, int64_t sqb, int64_t sqh,
                                 int64_t sqs, const void* k, int64_t skb, int64_t skh,
                                 int64_t sks, int64_t B, int64_t Hq, int64_t Hk, int64_t Sq,
                                 int64_t Sk, int64_t D, int64_t qps, int causal, int wo_init,
                                 int64_t J0, int64_t nc, int64_t dense_stride,
                                 int64_t segment_keys, const int32_t* counts,
                                 const int32_t* indices, float softmax_scale, float* stats,
                                 void* stream) {
  if (!stats) return fail(VA_ERR_ARG, "null stats");
  if (!counts || !indices) return fail(VA_ERR_ARG, "null counts / indices");
  if (segment_keys <= 0 || segment_keys % 64 || cdiv(Sk, segment_keys) > kMaxSegments)
    return fail(VA_ERR_ARG, "segment_keys %lld: need a positive multiple of 64, at most %lld "
                            "segments", (long long)segment_keys, (long long)kMaxSegments);
  return sparse_attn_impl(dtype, q, sqb, sqh, sqs, k, skb, skh, sks, nullptr, 0, 0, 0, nullptr, 0,
                          0, 0, B, Hq, Hk, Sq, Sk, D, qps, causal, wo_init, J0, nc, dense_stride,
                          counts, indices, softmax_scale, VA_ATTN_MFMA,
                          int(cdiv(Sk, segment_keys)), segment_keys, stream, stats);
}

int va_dense_row_stats(int dtype, const void* q, int64_t sqb, int64_t sqh, int64_t sqs,
                       const void* k, int64_t skb, int64_t skh, int64_t sks, int64_t B,
                       int64_t Hq, int64_t Hk, int64_t Sq, int64_t Sk, int64_t D, int causal,
                       float softmax_scale, int kernel, float* stats, void* stream) {
  if (!dtype_ok(dtype)) return fail(VA_ERR_ARG, "unknown dtype %d", dtype);
  if (!q || !k || !stats) return fail(VA_ERR_ARG, "null pointer");
  if (B <= 0 || Hq <= 0 || Hk <= 0 || Sq <= 0 || Sk <= 0 || D <= 0)
    return fail(VA_ERR_ARG, "non-positive size");
  if (Hq % Hk) return fail(VA_ERR_ARG, "num q heads not a multiple of kv heads");
  if (D > 256) return fail(VA_ERR_UNSUPPORTED, "head_dim %lld > 256", (long long)D);
  if (causal && Sq > Sk) return fail(VA_ERR_ARG, "causal rows need Sq <= Sk");
  constexpr int64_t qps = 64;
  const int64_t nc = cdiv(Sq, qps);
  if (nc * B * Hq > kMaxGrid) return fail(VA_ERR_UNSUPPORTED, "grid too large");
  const int64_t sq[3] = {sqb, sqh, sqs}, sk[3] = {skb, skh, sks};
  const AttnMfmaCheck chk = attn_mfma_check(dtype, q, sq, k, sk, k, sk, q, sq, Sk, D, qps);
  const bool mfma_ok = chk.ok() && softmax_scale > 0.f;
  bool use_mfma;
  if (kernel == VA_ATTN_MFMA) {
    if (!mfma_ok)
      return fail(VA_ERR_UNSUPPORTED, "MFMA row statistics need bf16/fp16, D in {64, 128}, "
                                      "16-byte aligned rows, Sk < 2^24, K row stride < 16 KiB "
                                      "and a positive softmax scale");
    use_mfma = true;
  } else if (kernel == VA_ATTN_AUTO) {
    use_mfma = mfma_ok;
  } else if (kernel == VA_ATTN_SIMPLE) {
    use_mfma = false;
  } else {
    return fail(VA_ERR_ARG, "unknown kernel selector %d", kernel);
  }
  const va::RowLayout lay = make_layout(0, nc, qps, Sk, causal, 0, 0);
  const float scale_log2 = softmax_scale * 1.4426950408889634f;
  const int64_t qoff = causal ? Sk - Sq : 0;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const hipError_t e =
      use_mfma ? va::launch_attn_mfma(dtype, D, qps, q, sq, k, sk, nullptr, sk, nullptr, sq, B, Hq,
                                      Hk, Sq, Sk, causal, scale_log2, nullptr, nullptr, lay, 1, 0,
                                      qoff, stats, va::kAttnFormAuto, st)
               : va::launch_attn_simple(dtype, q, sq, k, sk, nullptr, sk, nullptr, sq, B, Hq, Hk,
                                        Sq, Sk, D, qps, causal, scale_log2, nullptr, nullptr, lay,
                                        qoff, stats, st);
  const int rc = hip_check(e, "row statistics launch");
  return rc ? rc : ok();
}

int va_sparse_attn_segments(int dtype, const void* q, int64_t sqb, int64_t sqh, int64_t sqs,
                            const void* k, int64_t skb, int64_t skh, int64_t sks, const void* v,
                            int64_t svb, int64_t svh, int64_t svs, void* out, int64_t sob,
                            int64_t soh, int64_t sos, int64_t B, int64_t Hq, int64_t Hk,
                            int64_t Sq, int64_t Sk, int64_t D, int64_t qps, int causal,
                            int wo_init, int64_t J0, int64_t nc, int64_t dense_stride,
                            int64_t segment_keys, const int32_t* counts, const int32_t* indices,
                            float softmax_scale, void* stream) {
  if (!counts || !indices) return fail(VA_ERR_ARG, "null counts / indices");
  if (segment_keys <= 0 || segment_keys % 64 || cdiv(Sk, segment_keys) > kMaxSegments)
    return fail(VA_ERR_ARG, "segment_keys %lld: need a positive multiple of 64, at most %lld "
                            "segments", (long long)segment_keys, (long long)kMaxSegments);
  return sparse_attn_impl(dtype, q, sqb, sqh, sqs, k, skb, skh, sks, v, svb, svh, svs, out, sob,
                          soh, sos, B, Hq, Hk, Sq, Sk, D, qps, causal, wo_init, J0, nc,
                          dense_stride, counts, indices, softmax_scale, VA_ATTN_MFMA,
                          int(cdiv(Sk, segment_keys)), segment_keys, stream);
}

// Decode: the kv cache of each kv head is cut into nsplit ranges of `span`
// keys (a multiple of the 64-key tile, at least 4 tiles), enough ranges for
// about one work-group per CU over all kv heads (measured on MI355X against
// 128 - 1024 work-groups: fewer, longer ranges amortise each work-group's
// first copies and halve the partials the merge reads).
static void decode_split(int64_t L, int64_t Hk, int64_t* nsplit, int64_t* span) {
  constexpr int64_t kTargetGroups = 256;
  const int64_t n = cdiv(kTargetGroups, Hk);
  int64_t sp = cdiv(cdiv(L, n), 64) * 64;
  if (sp < 256) sp = 256;
  *span = sp;
  *nsplit = cdiv(L, sp);
}

int64_t va_decode_workspace_size(int64_t Hq, int64_t Hk, int64_t L, int64_t D) {
  if (Hq <= 0 || Hk <= 0 || L <= 0 || D <= 0 || Hq % Hk) return -1;
  int64_t nsplit, span;
  decode_split(L, Hk, &nsplit, &span);
  return align256(((2 * Hq * nsplit + 3) / 4 * 4 + Hq * nsplit * D) * 4);
}

}  // extern "C"

namespace va {

int api_error(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

// Decode attention with the partial softmax states in `workspace`
// (va_decode_attn, and the allocation-free variant with its static array).
int decode_run(int dtype, const void* q, int64_t sqh, const void* k, int64_t skh, int64_t sks,
               const void* v, int64_t svh, int64_t svs, void* out, int64_t soh, int64_t Hq,
               int64_t Hk, int64_t L, int64_t D, float softmax_scale, int kernel,
               void* workspace, int64_t workspace_bytes, void* stream) {
  if (!dtype_ok(dtype)) return fail(VA_ERR_ARG, "unknown dtype %d", dtype);
  if (!q || !k || !v || !out) return fail(VA_ERR_ARG, "null tensor pointer");
  if (Hq <= 0 || Hk <= 0 || L <= 0 || D <= 0) return fail(VA_ERR_ARG, "non-positive size");
  if (Hq % Hk) return fail(VA_ERR_ARG, "num q heads not a multiple of kv heads");
  if (D > 256) return fail(VA_ERR_UNSUPPORTED, "head_dim %lld > 256", (long long)D);
  const int64_t rep = Hq / Hk;
  // The query heads of kv head h are the rows of one group: q row r of group h
  // is q head h*rep + r.
  const int64_t sq[3] = {0, rep * sqh, sqh}, sk[3] = {0, skh, sks}, sv[3] = {0, svh, svs},
                so[3] = {0, rep * soh, soh};
  const AttnMfmaCheck chk = attn_mfma_check(dtype, q, sq, k, sk, v, sv, out, so, L, D, 64);
  const bool mfma_ok = chk.ok() && rep <= 64 && softmax_scale > 0.f;
  bool use_mfma;
  if (kernel == VA_ATTN_MFMA) {
    if (!mfma_ok)
      return fail(VA_ERR_UNSUPPORTED, "MFMA decode needs bf16/fp16, D in {64, 128}, at most 64 "
                                      "q heads per kv head, 16-byte aligned rows, L < 2^24, "
                                      "K/V row strides < 16 KiB and a positive softmax scale");
    use_mfma = true;
  } else if (kernel == VA_ATTN_AUTO) {
    use_mfma = mfma_ok;
  } else if (kernel == VA_ATTN_SIMPLE) {
    use_mfma = false;
  } else {
    return fail(VA_ERR_ARG, "unknown kernel selector %d", kernel);
  }
  const float scale_log2 = softmax_scale * 1.4426950408889634f;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (!use_mfma) {
    if (rep > 1024) return fail(VA_ERR_UNSUPPORTED, "more than 1024 q heads per kv head");
    const va::RowLayout lay = make_layout(0, 1, rep, L, 0, 0, 0);
    const int rc = hip_check(va::launch_attn_simple(dtype, q, sq, k, sk, v, sv, out, so, 1, Hk, Hk,
                                                    rep, L, D, rep, 0, scale_log2, nullptr,
                                                    nullptr, lay, 0, nullptr, st),
                             "decode launch");
    return rc ? rc : ok();
  }
  int64_t nsplit, span;
  decode_split(L, Hk, &nsplit, &span);
  const int64_t need = va_decode_workspace_size(Hq, Hk, L, D);
  if (!workspace || workspace_bytes < need)
    return fail(VA_ERR_WORKSPACE, "decode needs %lld workspace bytes", (long long)need);
  if (reinterpret_cast<uintptr_t>(workspace) % 16)
    return fail(VA_ERR_ARG, "workspace must be 16-byte aligned");
  float* part = static_cast<float*>(workspace);
  int rc = hip_check(va::launch_attn_split(dtype, D, q, sq, k, sk, v, sv, 1, Hk, rep, L,
                                           scale_log2, nsplit, span, part, st),
                     "decode split launch");
  if (rc) return rc;
  rc = hip_check(va::launch_decode_merge(dtype, D, part, Hk, rep, nsplit, out, rep * soh, soh, st),
                 "decode merge launch");
  return rc ? rc : ok();
}

}  // namespace va

extern "C" {

int va_decode_attn(int dtype, const void* q, int64_t sqh, const void* k, int64_t skh,
                   int64_t sks, const void* v, int64_t svh, int64_t svs, void* out, int64_t soh,
                   int64_t Hq, int64_t Hk, int64_t L, int64_t D, float softmax_scale, int kernel,
                   void* workspace, int64_t workspace_bytes, void* stream) {
  return va::decode_run(dtype, q, sqh, k, skh, sks, v, svh, svs, out, soh, Hq, Hk, L, D,
                        softmax_scale, kernel, workspace, workspace_bytes, stream);
}

// Row groups of a causal prefill chunk.  The selected-key lists of a chunk
// are held for one row group at a time (selection, then attention), so the
// index buffer is sized by the largest group instead of the whole chunk (6.2
// GiB for the last 32K chunk at 128K keys, 28 heads; 2.0 GiB in groups).  A
// group is a run of whole units, a unit being the smallest multiple of bsq
// rows that is at least 128 rows (one selection row set): groups start at
// multiples of bsq rows from the chunk origin, so the programs of bsq rows the
// reference's causal rule is tied to are unchanged and the results are
// identical.  A group grows while its index capacity stays within
// kIndexBudget bytes (always at least one unit).  Non-causal chunks are not
// split: their rows all see every key, the row sets of one launch share the
// K reads in L2, and groups measured 8% (256-row groups) to 21% (128-row
// groups) slower on MI355X at 119056 keys.
constexpr int64_t kIndexBudget = int64_t(2) << 30;

static int64_t group_unit(int64_t bsq) { return cdiv(128, bsq) * bsq; }

// End (exclusive, chunk-relative) of the row group starting at chunk row a.
static int64_t group_end(int64_t B, int64_t Hq, int64_t Sk, int64_t qps, int causal, int64_t J0,
                         int64_t nc, int64_t a, int64_t unit) {
  if (!causal) return nc;
  int64_t b = a + unit < nc ? a + unit : nc;
  while (b < nc) {
    const int64_t nb = b + unit < nc ? b + unit : nc;
    const int64_t cap = B * Hq * make_layout(J0 + a, nb - a, qps, Sk, causal, causal, 0).block_size();
    if (cap * 4 > kIndexBudget) break;
    b = nb;
  }
  return b;
}

// Workspace of va_prefill: [scaled pooled q][counts][indices][key norms]
// [segment maxima], 256-byte aligned.
static void prefill_segments(int dtype, int64_t B, int64_t Hq, int64_t Sq, int64_t Sk, int64_t D,
                             int64_t qps, int causal, int64_t chunk, int64_t bsq,
                             int64_t* qs_bytes, int64_t* cnt_bytes, int64_t* idx_bytes,
                             int64_t* kn_bytes, int64_t* carry_bytes = nullptr) {
  *kn_bytes = align256(va::key_norm_scratch_floats(B, Hq) * 4);  // Hk <= Hq
  const int64_t nqb = cdiv(Sq, qps);
  *qs_bytes = align256(B * Hq * nqb * D * esize(dtype));
  const int64_t nc_max = cdiv(chunk < Sq ? chunk : Sq, qps);
  *cnt_bytes = align256(B * Hq * nc_max * 4 * kMaxSegments);  // per-segment counts
  if (carry_bytes) *carry_bytes = align256(B * Hq * nc_max * va::kSegCarryBytes * kMaxSegments);
  int64_t idx_max = 0;
  const int64_t unit = group_unit(bsq);
  for (int64_t i = 0; i < Sq; i += chunk) {
    const int64_t rows = (Sq - i < chunk) ? (Sq - i) : chunk;
    const int64_t nc = cdiv(rows, qps), J0 = i / qps;
    for (int64_t a = 0; a < nc;) {
      const int64_t b = group_end(B, Hq, Sk, qps, causal, J0, nc, a, unit);
      const int64_t cap = B * Hq * make_layout(J0 + a, b - a, qps, Sk, causal, causal, 0).block_size();
      if (cap > idx_max) idx_max = cap;
      a = b;
    }
  }
  *idx_bytes = align256((idx_max > 0 ? idx_max : 1) * 4);
}

int64_t va_prefill_workspace_size(int dtype, int64_t B, int64_t Hq, int64_t Sq, int64_t Sk,
                                  int64_t D, int64_t qps, int causal, int64_t chunk_size,
                                  int64_t bsq) {
  if (!dtype_ok(dtype) || B <= 0 || Hq <= 0 || Sq <= 0 || Sk <= 0 || D <= 0 || qps <= 0 ||
      chunk_size <= 0 || chunk_size % qps || bsq <= 0)
    return -1;
  int64_t a, b, c, d, e;
  prefill_segments(dtype, B, Hq, Sq, Sk, D, qps, causal, chunk_size, bsq, &a, &b, &c, &d, &e);
  return a + b + c + d + e;
}

int va_prefill_kernels(int dtype, const void* q, int64_t sqb, int64_t sqh, int64_t sqs,
                       const void* k, int64_t skb, int64_t skh, int64_t sks, const void* v,
                       int64_t svb, int64_t svh, int64_t svs, const void* out, int64_t sob,
                       int64_t soh, int64_t sos, int64_t Hq, int64_t Hk, int64_t Sk, int64_t D,
                       int64_t qps, int64_t bk, int64_t group) {
  if (!dtype_ok(dtype) || Hq <= 0 || Hk <= 0 || Hq % Hk != 0 || Sk <= 0 || D <= 0 || qps <= 0 ||
      bk <= 0 || group <= 0)
    return fail(VA_ERR_ARG, "invalid prefill sizes");
  // va_prefill's own precondition; with q_pooling_size 64 or 128 the first
  // selectable key (0, or q_pooling_size for causal rows) is 64-aligned, as
  // the wave selection kernel needs, so the plan below is the one it runs.
  if (qps != 64 && qps != 128) return fail(VA_ERR_ARG, "q_pooling_size must be 64 or 128");
  // The pooled queries live in the 256-byte aligned workspace with element
  // strides that are multiples of D: any aligned address and D strides stand
  // for them.
  const void* qs = reinterpret_cast<const void*>(uintptr_t(256));
  int flags = 0;
  const bool wave = select_wave_ok(dtype, qs, D, D, D, k, skb, skh, sks, Sk, D, bk, group);
  if (wave)
    flags |= VA_KERNELS_SELECT_WAVE;
  else if (select_mfma_ok(dtype, qs, D, D, D, k, skb, skh, sks, D, bk))
    flags |= VA_KERNELS_SELECT_MFMA;
  else
    flags |= VA_KERNELS_SELECT_EXACT;
  const int64_t sq[3] = {sqb, sqh, sqs}, sk[3] = {skb, skh, sks}, sv[3] = {svb, svh, svs},
                so[3] = {sob, soh, sos};
  const bool attn = attn_mfma_check(dtype, q, sq, k, sk, v, sv, out, so, Sk, D, qps).ok();
  flags |= attn ? VA_KERNELS_ATTN_MFMA
                : attn_f32_ok(dtype, q, sq, k, sk, v, sv, out, so, D, qps) ? VA_KERNELS_ATTN_F32
                                                                           : VA_KERNELS_ATTN_ROW;
  if (attn && va::attn_mfma_ring_supported(dtype, D, qps) && va::ring_form_preferred(Hq, Hk, Sk, D))
    flags |= VA_KERNELS_ATTN_RING;
  const int64_t g = effective_group(group, Sk, bk);
  if (attn && (flags & (VA_KERNELS_SELECT_WAVE | VA_KERNELS_SELECT_MFMA))) {
    if (wave ? (va::select_wave_segment_keys(Sk, bk, g) > 0 ||
                va::select_wave_carry_segment_keys(Sk, bk, g) > 0)
             : va::select_mfma_segment_keys(Sk, bk, g) > 0)
      flags |= VA_KERNELS_SPLIT;
  } else if ((flags & VA_KERNELS_ATTN_F32) && !(flags & (VA_KERNELS_SELECT_WAVE |
                                                          VA_KERNELS_SELECT_MFMA))) {
    if (va::select_exact_segment_keys(Sk, bk, g) > 0) flags |= VA_KERNELS_SPLIT;
  }
  ok();
  return flags;
}

int va_prefill(int dtype, const void* q, int64_t sqb, int64_t sqh, int64_t sqs, const void* k,
               int64_t skb, int64_t skh, int64_t sks, const void* v, int64_t svb, int64_t svh,
               int64_t svs, void* out, int64_t sob, int64_t soh, int64_t sos, int64_t B,
               int64_t Hq, int64_t Hk, int64_t Sq, int64_t Sk, int64_t D, float gap,
               const float* gaps, int64_t qps, int64_t bk, int64_t group, int causal,
               int64_t chunk_size, int64_t bsq, void* workspace, int64_t workspace_bytes,
               void* stream) {
  if (chunk_size <= 0 || chunk_size % qps)
    return fail(VA_ERR_ARG, "chunk_size must be a multiple of q_pooling_size");
  if (qps != 64 && qps != 128) return fail(VA_ERR_ARG, "q_pooling_size must be 64 or 128");
  if (!q || !k || !v || !out) return fail(VA_ERR_ARG, "null tensor pointer");
  if (causal && Sq != Sk) return fail(VA_ERR_UNSUPPORTED, "causal prefill needs Sq == Sk");
  if (bsq <= 0) return fail(VA_ERR_ARG, "bsq must be positive");
  const int64_t need =
      va_prefill_workspace_size(dtype, B, Hq, Sq, Sk, D, qps, causal, chunk_size, bsq);
  if (need < 0) return fail(VA_ERR_ARG, "invalid prefill sizes");
  if (!workspace || workspace_bytes < need)
    return fail(VA_ERR_WORKSPACE, "workspace %lld bytes < required %lld (bsq %lld)",
                (long long)workspace_bytes, (long long)need, (long long)bsq);
  const int64_t nqb = cdiv(Sq, qps);
  int64_t qs_bytes, cnt_bytes, idx_bytes, kn_bytes, carry_bytes;
  prefill_segments(dtype, B, Hq, Sq, Sk, D, qps, causal, chunk_size, bsq, &qs_bytes, &cnt_bytes,
                   &idx_bytes, &kn_bytes, &carry_bytes);
  char* ws = static_cast<char*>(workspace);
  void* qs = ws;
  int32_t* counts = reinterpret_cast<int32_t*>(ws + qs_bytes);
  int32_t* indices = reinterpret_cast<int32_t*>(ws + qs_bytes + cnt_bytes);
  float* knorm = reinterpret_cast<float*>(ws + qs_bytes + cnt_bytes + idx_bytes);
  void* carry = ws + qs_bytes + cnt_bytes + idx_bytes + kn_bytes;
  hipStream_t st = static_cast<hipStream_t>(stream);

  int rc = va_pool(dtype, q, B, Hq, Sq, D, sqb, sqh, sqs, qps, nullptr, qs, stream);
  if (rc) return rc;
  rc = check_select_args(dtype, qs, k, B, Hq, Hk, Sk, D, qps, bk, group, causal, causal, 0,
                         cdiv(Sq, qps), bsq);
  if (rc) return rc;
  const SelKernel which =
      select_wave_ok(dtype, qs, Hq * nqb * D, nqb * D, D, k, skb, skh, sks, Sk, D, bk, group)
          ? kSelWave
      : select_mfma_ok(dtype, qs, Hq * nqb * D, nqb * D, D, k, skb, skh, sks, D, bk)
          ? kSelMfma
          : kSelExact;
  if (which != kSelExact) {
    rc = hip_check(va::launch_key_norm(dtype, k, skb, skh, sks, B, Hk, Sk, D, knorm, st),
                   "key norm launch");
    if (rc) return rc;
  }
  // Split the selection into key segments when the wave kernel and the MFMA
  // attention (which reads the segmented lists) both run: segments that each
  // start a group when the groups are short, otherwise (one group per row) a
  // maxima pass followed by a carry pass.
  int64_t segk = 0;
  bool two_pass = false;
  {
    const int64_t sq[3] = {sqb, sqh, sqs}, sk[3] = {skb, skh, sks}, sv[3] = {svb, svh, svs},
                  so[3] = {sob, soh, sos};
    const bool attn = attn_mfma_check(dtype, q, sq, k, sk, v, sv, out, so, Sk, D, qps).ok();
    const int64_t g = effective_group(group, Sk, bk);
    if (which == kSelWave && attn) {
      segk = va::select_wave_segment_keys(Sk, bk, g);
      if (segk == 0) {
        segk = va::select_wave_carry_segment_keys(Sk, bk, g);
        two_pass = segk > 0;
      }
    } else if (which == kSelMfma && attn) {
      // the 64-row MFMA kernel splits at whole 256-key chunks (no carry pass)
      segk = va::select_mfma_segment_keys(Sk, bk, g);
    } else if (which == kSelExact && attn_f32_ok(dtype, q, sq, k, sk, v, sv, out, so, D, qps)) {
      // fp32: the exact kernel's split (two passes when a group spans the
      // row), read by the fp32 matrix-core attention
      segk = va::select_exact_segment_keys(Sk, bk, g);
      two_pass = segk > 0 && segments_two_pass(Sk, bk, group, segk);
      if (segk > 0 && cdiv(cdiv(chunk_size, qps), 16) * cdiv(Sk, segk) * B * Hq > (int64_t(1) << 24))
        segk = 0;  // grid of (16-row sets, segment) work-groups too large
    }
  }
  const float scale = float(1.0 / std::sqrt(double(D)));
  // Segment length of a row group: groups of few rows (the later groups of a
  // long causal prefill) halve the segments, down to 2048 keys and at most 64
  // segments, until the selection has kMinSelectBlocks work-groups (each
  // covers 128 rows of one segment); the attention of the group reads the
  // lists with the same length.
  const int64_t gspan = segk > 0 && !two_pass ? bk * effective_group(group, Sk, bk) : 0;
  const int64_t wg_rows = which == kSelWave ? 128 : 64;  // pooled rows per selection work-group
  auto group_segk = [&](int64_t nc) {
    constexpr int64_t kMinSelectBlocks = 1536, kMinSeg = 2048;
    int64_t sg = segk;
    if (gspan <= 0) return sg;
    while (sg / 2 >= kMinSeg && (sg / 2) % gspan == 0 && (sg / 2) % 256 == 0 &&
           cdiv(Sk, sg / 2) <= kMaxSegments &&
           cdiv(nc, wg_rows) * cdiv(Sk, sg) * B * Hq < kMinSelectBlocks)
      sg /= 2;
    return sg;
  };
  const int64_t unit = group_unit(bsq);
  for (int64_t i = 0; i < Sq; i += chunk_size) {
    const int64_t rows = (Sq - i < chunk_size) ? (Sq - i) : chunk_size;
    const int64_t Jc = i / qps, nrows = cdiv(rows, qps);
    // Row groups [Jc + a, Jc + b) of the chunk: start at multiples of bsq rows
    // from the chunk origin (the reference's program tiling), so the
    // selection of a group equals that of the whole chunk on its rows.
    for (int64_t a = 0; a < nrows;) {
      const int64_t b = group_end(B, Hq, Sk, qps, causal, Jc, nrows, a, unit);
      const int64_t J0 = Jc + a, nc = b - a;
      a = b;
      const int64_t segk_g = group_segk(nc);
      const int nseg = segk_g > 0 ? int(cdiv(Sk, segk_g)) : 1;
      const int64_t es = esize(dtype);
      const void* qs_chunk = static_cast<const char*>(qs) + J0 * D * es;
      if (two_pass) {
        rc = select_impl(dtype, qs_chunk, Hq * nqb * D, nqb * D, D, k, skb, skh, sks, B, Hq, Hk,
                         Sk, D, qps, bk, group, causal, causal, J0, nc, bsq, gap, gaps, 0, counts,
                         indices, which, knorm, segk_g, st, carry, va::kPassMax);
        if (rc) return rc;
      }
      rc = select_impl(dtype, qs_chunk, Hq * nqb * D, nqb * D, D, k, skb, skh, sks, B, Hq, Hk,
                       Sk, D, qps, bk, group, causal, causal, J0, nc, bsq, gap, gaps, 0, counts,
                       indices, which, knorm, segk_g, st, carry,
                       two_pass ? va::kPassCarry : va::kPassPlain);
      if (rc) return rc;
      rc = sparse_attn_impl(dtype, q, sqb, sqh, sqs, k, skb, skh, sks, v, svb, svh, svs, out, sob,
                            soh, sos, B, Hq, Hk, Sq, Sk, D, qps, causal, causal, J0, nc, 0, counts,
                            indices, scale, VA_ATTN_AUTO, nseg, segk_g, st);
      if (rc) return rc;
    }
  }
  return ok();
}

}  // extern "C"
