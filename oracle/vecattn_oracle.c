/*
 * CPU oracle for the VecAttention prefill hot path — TEST INFRASTRUCTURE ONLY.
 *
 * This file is a plain-C restatement of the reference selection rule.  It is
 * compiled into oracle/liboracle.so and loaded by tests/, by
 * __graft_entry__.smoke() and by bench.py's cpu_baseline leg, always as the
 * checker and never as the product path.  The product (vecattention_amd/)
 * never links or calls it.
 *
 * Canonical arithmetic (the contract the HIP kernels are bit-exact against):
 *   - data arrives as float32 arrays whose values are already representable in
 *     the element type T (bf16 / fp16 / fp32); `dtype` selects the rounding
 *     applied where the reference rounds back to T;
 *   - every dot product is a sequential fp64 sum over d = 0..D-1 of exact
 *     products (bf16*bf16 and fp32*fp32 products are exact in fp64), rounded
 *     once to fp32;
 *   - pooling sums rows sequentially in fp64, rounds to fp32, divides in fp32
 *     (IEEE) by the real row count, then rounds to T.
 *
 * Functions and the reference lines they follow:
 *   orc_pool    spattn/src/utils.py:48,63-64 (bnhd_pool_kernel: fp32 mean over
 *               the real rows of a block), :340-351 (average_vector: fp32
 *               upcast, result cast back to T); scaled copy as in
 *               spattn/src/kernels/vecattention_kernels.py:94,244-245.
 *   orc_select  spattn/src/kernels/vecattention_kernels.py:91-181 (host
 *               wrapper: padding, grid, trimming) and :206-272 / :275-345
 *               (program body: group start, causal end, prefix max updated
 *               before the compare, truncating causal tile mask, NaN tail).
 *
 * Parity status: pinned by the checks in tests/test_oracle.py (closed forms,
 * hand-derived known answers, a brute force written from the reference
 * kernel's program structure on small-integer inputs whose scores are exact,
 * and the invariants listed there).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

enum { ORC_F32 = 0, ORC_BF16 = 1, ORC_F16 = 2 };

/* Round-to-nearest-even of an fp32 value to bf16, returned as fp32. */
static float round_bf16(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7f800000u) == 0x7f800000u) { /* inf / nan */
        if (u & 0x007fffffu) u |= 0x00400000u;
        u &= 0xffff0000u;
    } else {
        uint32_t lsb = (u >> 16) & 1u;
        u += 0x7fffu + lsb;
        u &= 0xffff0000u;
    }
    float r;
    memcpy(&r, &u, 4);
    return r;
}

/* Round-to-nearest-even of an fp32 value to IEEE binary16, returned as fp32.
 * The quantum of the target binade (2^-24 for subnormals) is a power of two,
 * so x / quantum is exact in fp64 and nearbyint() performs the RNE step. */
static float round_f16(float x) {
    if (isnan(x) || isinf(x)) return x;
    const float ax = fabsf(x);
    if (ax >= 65520.0f) return copysignf(INFINITY, x);
    if (ax == 0.0f) return x;
    int e;
    frexpf(ax, &e);
    int lead = e - 1;
    if (lead < -14) lead = -14;
    const double quantum = ldexp(1.0, lead - 10);
    const double r = nearbyint((double)ax / quantum) * quantum;
    return copysignf((float)r, x);
}

static float round_t(float x, int dtype) {
    if (dtype == ORC_BF16) return round_bf16(x);
    if (dtype == ORC_F16) return round_f16(x);
    return x;
}

/* Sequential fp64 dot product rounded once to fp32 (the canonical score). */
static float dot_canonical(const float* a, const float* b, int64_t D) {
    double acc = 0.0;
    for (int64_t d = 0; d < D; ++d) acc += (double)a[d] * (double)b[d];
    return (float)acc;
}

/*
 * Block-mean pooling of q (contiguous [B,H,S,D]) over blocks of qps rows.
 * pooled / scaled: contiguous [B,H,nqb,D]; either may be NULL.
 *   pooled = T( fp32(sum_rows) / rows )
 *   scaled = T( fp32(pooled * fp32(1/sqrt(D))) )
 */
int orc_pool(const float* q, int64_t B, int64_t H, int64_t S, int64_t D,
             int64_t qps, int dtype, float* pooled, float* scaled) {
    if (qps <= 0 || D <= 0) return -1;
    const int64_t nqb = (S + qps - 1) / qps;
    const float sm = (float)(1.0 / sqrt((double)D));
    for (int64_t bh = 0; bh < B * H; ++bh) {
        const float* qb = q + bh * S * D;
        for (int64_t j = 0; j < nqb; ++j) {
            const int64_t r0 = j * qps;
            const int64_t rows = (S - r0 < qps) ? (S - r0) : qps;
            for (int64_t d = 0; d < D; ++d) {
                double acc = 0.0;
                for (int64_t r = 0; r < rows; ++r) acc += (double)qb[(r0 + r) * D + d];
                const float sum32 = (float)acc;
                const float mean32 = sum32 / (float)rows;
                const float p = round_t(mean32, dtype);
                const int64_t o = (bh * nqb + j) * D + d;
                if (pooled) pooled[o] = p;
                if (scaled) scaled[o] = round_t(p * sm, dtype);
            }
        }
    }
    return 0;
}

/* Truncating signed division, as Triton's integer `//` on int64 (sdiv). */
static int64_t div_trunc(int64_t a, int64_t b) { return a / b; }

/*
 * TilingSelect for the pooled rows J0+jr_begin .. J0+jr_end-1 of every (b, h),
 * where [J0, J0+nc) is the chunk the reference launch covers (its start fixes
 * the BLOCK_SIZE_Q program tiling); rows outside [jr_begin, jr_end) get count 0.
 *
 * qs      : scaled pooled queries, contiguous [B,Hq,nqb_total,D] (row J at
 *           index J, i.e. the whole sequence; only rows of the chunk are read)
 * k       : keys, contiguous [B,Hk,Sk,D]; q head h reads kv head h/(Hq/Hk)
 * gaps    : fp32 gap per (b,h), length B*Hq
 * bsq     : BLOCK_SIZE_Q of the reference launch (sets the causal row tiling)
 * counts  : out, [B,Hq,nc] int32
 * indices : out, row (b,h,J) written from row_base[(b*Hq+h)*nc + (J-J0)]
 *           (int64 element offsets) in ascending key order
 * Returns 0, or -1 on invalid arguments, or -2 if a row exceeds row_cap.
 */
int orc_select(const float* qs, int64_t nqb_total, const float* k, int64_t B,
               int64_t Hq, int64_t Hk, int64_t Sk, int64_t D, int64_t qps,
               int64_t bk, int64_t group, int causal, int wo_init, int64_t J0,
               int64_t nc, int64_t jr_begin, int64_t jr_end, int64_t bsq,
               const float* gaps, int32_t* counts, int32_t* indices,
               const int64_t* row_base, const int64_t* row_cap) {
    if (qps <= 0 || bk <= 0 || bk > 512 || group <= 0 || bsq <= 0 || Hk <= 0 || Hq % Hk) return -1;
    if (causal && qps % bk) return -1;
    const int64_t rep = Hq / Hk;
    const int64_t padded_k = (Sk + bk - 1) / bk * bk;
    const int64_t gspan = bk * group;
    const int64_t ngroups = (padded_k + gspan - 1) / gspan;
    for (int64_t b = 0; b < B; ++b) {
        for (int64_t h = 0; h < Hq; ++h) {
            const float* kh = k + (b * Hk + h / rep) * Sk * D;
            const float gap = gaps[b * Hq + h];
            for (int64_t jr = 0; jr < nc; ++jr) {
                if (jr < jr_begin || jr >= jr_end) {
                    counts[(b * Hq + h) * nc + jr] = 0;
                    continue;
                }
                const int64_t J = J0 + jr;
                const float* qrow = qs + ((b * Hq + h) * nqb_total + J) * D;
                const int64_t qtile = jr / bsq;          /* program_id(0) */
                const int64_t r = jr - qtile * bsq;      /* row inside the program */
                const int64_t off0 = (J0 + qtile * bsq) * qps;
                const int64_t rowid = (b * Hq + h) * nc + jr;
                int32_t* out = indices + row_base[rowid];
                int64_t cnt = 0;
                for (int64_t g = 0; g < ngroups; ++g) {
                    const int64_t kblock = g * group;
                    int64_t start = kblock * bk;
                    if (wo_init && start < qps) start = qps;
                    int64_t max_valid = Sk;
                    if (causal) {
                        const int64_t lim = (J0 + (qtile + 1) * bsq) * qps - qps;
                        if (lim < max_valid) max_valid = lim;
                    }
                    int64_t end = kblock * bk + gspan;
                    if (max_valid < end) end = max_valid;
                    if (end <= start) continue;
                    float m = -INFINITY;
                    for (int64_t koff = start; koff < end; koff += bk) {
                        float sc[512];
                        float tmax = -INFINITY;
                        const int64_t nvalid = (Sk - koff < bk) ? (Sk - koff) : bk;
                        for (int64_t c = 0; c < nvalid; ++c) {
                            sc[c] = dot_canonical(qrow, kh + (koff + c) * D, D);
                            if (sc[c] > tmax) tmax = sc[c];
                        }
                        if (tmax > m) m = tmax;
                        if (causal && !(r > div_trunc(koff - off0, qps))) continue;
                        for (int64_t c = 0; c < nvalid; ++c) {
                            const float t = sc[c] + gap;
                            if (t >= m) {
                                if (cnt >= row_cap[rowid]) return -2;
                                out[cnt++] = (int32_t)(koff + c);
                            }
                        }
                    }
                }
                counts[rowid] = (int32_t)cnt;
            }
        }
    }
    return 0;
}

/* Exposed for tests: canonical score of one pair and the T rounding. */
float orc_dot(const float* a, const float* b, int64_t D) { return dot_canonical(a, b, D); }
float orc_round(float x, int dtype) { return round_t(x, dtype); }
