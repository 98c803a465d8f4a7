/*
 * tq_cpu_baseline.c -- the reference's CPU decode path, restated (TEST INFRASTRUCTURE / BASELINE ONLY).
 *
 * The reference's CPU MUL_MAT_ID decode path is ggml-cpu plus patch 0002, which hooks an AVX-512 VNNI
 * one-column GEMV (KTransformers' iqk kernels) into ggml_compute_forward_mul_mat_id
 * (patches/0002-iqk-avx512-q4k-q6k-decode.patch:36-57). That code cannot be built here (it needs ggml's
 * headers, which are not in the reference checkout), so this file restates its algorithm in code of its
 * own, to be timed as the reported CPU baseline beside the GPU kernels:
 *
 *   - static split of the Nx rows over nth threads, ceil(Nx/nth) rows each (patches/0002:1205-1229,
 *     :139-150, and the early return for threads past the end, :139-150);
 *   - per super-block: u8 x s8 dot products of 4 (vpdpbusd), saturating pack to 16 bits, 16-bit scale
 *     products summed into 32 bits (vpdpwssd), one fp32 fused multiply-add by d_x*d_y per super-block
 *     (compute_block, :1713-1722);
 *   - the Q4_K mins and the Q6_K -32 offset folded in through the Q8_K bsums (:1296-1342, :1581-1598,
 *     :1638-1663);
 *   - two super-blocks in flight per row (mul_mat_qX_K_q8_K_AVX512_1, :1812-1849).
 *
 * The lane arrangement differs from iqk's: weights stay in natural nibble order and the activation
 * 64-byte groups are re-paired with one 128-bit-lane shuffle instead of permuting the weights.
 * Hosts without AVX-512 VNNI fall back to the scalar vec_dot of tq_oracle.c, and the report says so.
 */
#include "tq_oracle.h"

#include <immintrin.h>
#include <pthread.h>
#include <sched.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>

#define ORC_AVX512 __attribute__((target("avx2,fma,avx512f,avx512bw,avx512dq,avx512vl,avx512vnni")))

int orc_cpu_has_avx512_vnni(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
           __builtin_cpu_supports("avx512dq") && __builtin_cpu_supports("avx512vl") &&
           __builtin_cpu_supports("avx512vnni");
}

ORC_AVX512 static inline float orc_hsum512(__m512 v) { return _mm512_reduce_add_ps(v); }

ORC_AVX512 static inline float orc_hsum256(__m256 v) {
    __m128 s = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
    s = _mm_add_ps(s, _mm_movehl_ps(s, s));
    s = _mm_add_ss(s, _mm_movehdup_ps(s));
    return _mm_cvtss_f32(s);
}

/* Q4_K: the 8 scales and 8 mins of one block as bytes, sc[0..7] then m[0..7]. */
static inline void orc_q4_unpack(const uint8_t *s, uint8_t out[16]) {
    uint32_t a0, a1, a2;
    memcpy(&a0, s, 4), memcpy(&a1, s + 4, 4), memcpy(&a2, s + 8, 4);
    const uint32_t w[4] = {
        a0 & 0x3f3f3f3fu,                                        /* sc0..3 */
        (a2 & 0x0f0f0f0fu) | ((a0 >> 2) & 0x30303030u),          /* sc4..7 */
        a1 & 0x3f3f3f3fu,                                        /* m0..3  */
        ((a2 >> 4) & 0x0f0f0f0fu) | ((a1 >> 2) & 0x30303030u),   /* m4..7  */
    };
    memcpy(out, w, 16);
}

/* One Q4_K row against one Q8_K row. Registers of 64 weights: qs[0..63] low nibbles are elements
 * 0..31 | 64..95 (sub-blocks 0|2), high nibbles 32..63 | 96..127 (1|3); qs[64..127] likewise for
 * sub-blocks 4..7. The activation 32-byte halves are paired to match with _mm512_shuffle_i64x2. */
ORC_AVX512 static float orc_row_q4_K(const orc_block_q4_K *x, const orc_block_q8_K *y, int nb) {
    const __m512i m4 = _mm512_set1_epi8(0x0f);
    /* 16-bit scale positions after the 32->16 pack: 128-bit lane L holds 4 partials of operand a then
     * 4 of operand b, so lanes 0,1 take sub-blocks (0,1) and lanes 2,3 sub-blocks (2,3). */
    const __m512i idx_lo = _mm512_set_epi16(3, 3, 3, 3, 2, 2, 2, 2, 3, 3, 3, 3, 2, 2, 2, 2,
                                            1, 1, 1, 1, 0, 0, 0, 0, 1, 1, 1, 1, 0, 0, 0, 0);
    const __m512i idx_hi = _mm512_add_epi16(idx_lo, _mm512_set1_epi16(4));
    const __m256i idx_m = _mm256_set_epi16(7, 7, 6, 6, 5, 5, 4, 4, 3, 3, 2, 2, 1, 1, 0, 0);
    __m512 accd = _mm512_setzero_ps();
    __m256 accm = _mm256_setzero_ps();
    for (int i = 0; i < nb; ++i) {
        uint8_t sm[16];
        orc_q4_unpack(x[i].scales, sm);
        const __m512i sc16 = _mm512_cvtepu8_epi16(_mm256_castsi128_si256(_mm_loadu_si128((const __m128i *)sm)));
        const __m512i s_lo = _mm512_permutexvar_epi16(idx_lo, sc16);
        const __m512i s_hi = _mm512_permutexvar_epi16(idx_hi, sc16);
        const __m256i m16 = _mm256_permutexvar_epi16(idx_m, _mm256_cvtepu8_epi16(_mm_loadl_epi64((const __m128i *)(sm + 8))));

        const __m512i y0 = _mm512_loadu_si512(y[i].qs), y1 = _mm512_loadu_si512(y[i].qs + 64);
        const __m512i y2 = _mm512_loadu_si512(y[i].qs + 128), y3 = _mm512_loadu_si512(y[i].qs + 192);
        const __m512i q0 = _mm512_loadu_si512(x[i].qs), q1 = _mm512_loadu_si512(x[i].qs + 64);
        const __m512i p0 = _mm512_dpbusd_epi32(_mm512_setzero_si512(), _mm512_and_si512(q0, m4),
                                               _mm512_shuffle_i64x2(y0, y1, 0x44));
        const __m512i p1 = _mm512_dpbusd_epi32(_mm512_setzero_si512(), _mm512_and_si512(_mm512_srli_epi16(q0, 4), m4),
                                               _mm512_shuffle_i64x2(y0, y1, 0xee));
        const __m512i p2 = _mm512_dpbusd_epi32(_mm512_setzero_si512(), _mm512_and_si512(q1, m4),
                                               _mm512_shuffle_i64x2(y2, y3, 0x44));
        const __m512i p3 = _mm512_dpbusd_epi32(_mm512_setzero_si512(), _mm512_and_si512(_mm512_srli_epi16(q1, 4), m4),
                                               _mm512_shuffle_i64x2(y2, y3, 0xee));
        __m512i isum = _mm512_dpwssd_epi32(_mm512_setzero_si512(), _mm512_packs_epi32(p0, p1), s_lo);
        isum = _mm512_dpwssd_epi32(isum, _mm512_packs_epi32(p2, p3), s_hi);
        const __m256i msum = _mm256_madd_epi16(m16, _mm256_loadu_si256((const __m256i *)y[i].bsums));

        const float dy = y[i].d;
        accd = _mm512_fmadd_ps(_mm512_set1_ps(orc_fp16_to_fp32(x[i].d) * dy), _mm512_cvtepi32_ps(isum), accd);
        accm = _mm256_fmadd_ps(_mm256_set1_ps(-orc_fp16_to_fp32(x[i].dmin) * dy), _mm256_cvtepi32_ps(msum), accm);
    }
    return orc_hsum512(accd) + orc_hsum256(accm);
}

/* One Q6_K row against one Q8_K row. ql[0..63] low nibbles are elements 0..63 and high nibbles
 * 64..127 in natural order (ql[64..127]: 128..255); qh bits 2t..2t+1 of byte l add to quarter t. */
ORC_AVX512 static float orc_row_q6_K(const orc_block_q6_K *x, const orc_block_q8_K *y, int nb) {
    const __m512i m4 = _mm512_set1_epi8(0x0f), m2 = _mm512_set1_epi8(0x03);
    /* shift per 16-bit lane: bytes 0..31 take qh bits (0,1) or (4,5), bytes 32..63 bits (2,3) or (6,7) */
    const __m512i sh_a = _mm512_inserti64x4(_mm512_setzero_si512(), _mm256_set1_epi16(2), 1);
    const __m512i sh_b = _mm512_inserti64x4(_mm512_set1_epi16(4), _mm256_set1_epi16(6), 1);
    const __m512i idx_a = _mm512_set_epi16(7, 7, 7, 7, 3, 3, 3, 3, 6, 6, 6, 6, 2, 2, 2, 2,
                                           5, 5, 5, 5, 1, 1, 1, 1, 4, 4, 4, 4, 0, 0, 0, 0);
    const __m512i idx_b = _mm512_add_epi16(idx_a, _mm512_set1_epi16(8));
    __m512 accd = _mm512_setzero_ps();
    __m256 accm = _mm256_setzero_ps();
    for (int i = 0; i < nb; ++i) {
        const __m256i sc16 = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i *)x[i].scales));
        const __m512i s_a = _mm512_permutexvar_epi16(idx_a, _mm512_castsi256_si512(sc16));
        const __m512i s_b = _mm512_permutexvar_epi16(idx_b, _mm512_castsi256_si512(sc16));

        const __m512i l0 = _mm512_loadu_si512(x[i].ql), l1 = _mm512_loadu_si512(x[i].ql + 64);
        const __m512i h = _mm512_loadu_si512(x[i].qh);
        const __m512i h0 = _mm512_shuffle_i64x2(h, h, 0x44), h1 = _mm512_shuffle_i64x2(h, h, 0xee);
        const __m512i q0 = _mm512_or_si512(_mm512_and_si512(l0, m4),
                                           _mm512_slli_epi16(_mm512_and_si512(_mm512_srlv_epi16(h0, sh_a), m2), 4));
        const __m512i q1 = _mm512_or_si512(_mm512_and_si512(_mm512_srli_epi16(l0, 4), m4),
                                           _mm512_slli_epi16(_mm512_and_si512(_mm512_srlv_epi16(h0, sh_b), m2), 4));
        const __m512i q2 = _mm512_or_si512(_mm512_and_si512(l1, m4),
                                           _mm512_slli_epi16(_mm512_and_si512(_mm512_srlv_epi16(h1, sh_a), m2), 4));
        const __m512i q3 = _mm512_or_si512(_mm512_and_si512(_mm512_srli_epi16(l1, 4), m4),
                                           _mm512_slli_epi16(_mm512_and_si512(_mm512_srlv_epi16(h1, sh_b), m2), 4));
        const __m512i p0 = _mm512_dpbusd_epi32(_mm512_setzero_si512(), q0, _mm512_loadu_si512(y[i].qs));
        const __m512i p1 = _mm512_dpbusd_epi32(_mm512_setzero_si512(), q1, _mm512_loadu_si512(y[i].qs + 64));
        const __m512i p2 = _mm512_dpbusd_epi32(_mm512_setzero_si512(), q2, _mm512_loadu_si512(y[i].qs + 128));
        const __m512i p3 = _mm512_dpbusd_epi32(_mm512_setzero_si512(), q3, _mm512_loadu_si512(y[i].qs + 192));
        __m512i isum = _mm512_dpwssd_epi32(_mm512_setzero_si512(), _mm512_packs_epi32(p0, p1), s_a);
        isum = _mm512_dpwssd_epi32(isum, _mm512_packs_epi32(p2, p3), s_b);
        const __m256i msum = _mm256_madd_epi16(sc16, _mm256_loadu_si256((const __m256i *)y[i].bsums));

        const float dd = orc_fp16_to_fp32(x[i].d) * y[i].d;
        accd = _mm512_fmadd_ps(_mm512_set1_ps(dd), _mm512_cvtepi32_ps(isum), accd);
        accm = _mm256_fmadd_ps(_mm256_set1_ps(-32.f * dd), _mm256_cvtepi32_ps(msum), accm);
    }
    return orc_hsum512(accd) + orc_hsum256(accm);
}

int orc_iqk_mul_mat(long Nx, long Ny, long ne00, int typeA, const void *A, long strideA, int typeB,
                    const void *B, long strideB, float *C, long stride_C, int ith, int nth) {
    (void)strideB, (void)stride_C;
    if (Ny != 1 || typeB != ORC_TYPE_Q8_K || (typeA != ORC_TYPE_Q4_K && typeA != ORC_TYPE_Q6_K)) return 0;
    if (ne00 % ORC_QK_K || !orc_cpu_has_avx512_vnni()) return 0;
    const long per = (Nx + nth - 1) / nth;
    const long first = (long)ith * per;
    if (first >= Nx) return 1;
    const long last = first + per < Nx ? first + per : Nx;
    const int nb = (int)(ne00 / ORC_QK_K);
    const size_t row = (size_t)strideA * orc_type_size(typeA);
    const orc_block_q8_K *y = (const orc_block_q8_K *)B;
    for (long r = first; r < last; ++r) {
        const void *xr = (const char *)A + r * row;
        C[r] = typeA == ORC_TYPE_Q4_K ? orc_row_q4_K((const orc_block_q4_K *)xr, y, nb)
                                      : orc_row_q6_K((const orc_block_q6_K *)xr, y, nb);
    }
    return 1;
}

/* ---- a small spinning thread pool: the caller is thread 0, workers 1..nth-1 ---- */

typedef void (*orc_job_fn)(void *arg, int ith, int nth);

static struct {
    int nth;
    pthread_t *tid;
    _Atomic unsigned gen;
    _Atomic int done;
    _Atomic int quit;
    orc_job_fn fn;
    void *arg;
} orc_pool;

static void *orc_worker(void *p) {
    const int ith = (int)(intptr_t)p;
    unsigned seen = 0;
    for (;;) {
        unsigned g;
        while ((g = atomic_load_explicit(&orc_pool.gen, memory_order_acquire)) == seen) {
            if (atomic_load_explicit(&orc_pool.quit, memory_order_relaxed)) return NULL;
            _mm_pause();
        }
        seen = g;
        orc_pool.fn(orc_pool.arg, ith, orc_pool.nth);
        atomic_fetch_add_explicit(&orc_pool.done, 1, memory_order_acq_rel);
    }
}

int orc_pool_init(int nth) {
    orc_pool_free();
    if (nth < 1) nth = 1;
    orc_pool.nth = nth;
    atomic_store(&orc_pool.gen, 0);
    atomic_store(&orc_pool.quit, 0);
    orc_pool.tid = calloc((size_t)nth, sizeof(pthread_t));
    if (!orc_pool.tid) return -2;
    for (int i = 1; i < nth; ++i)
        if (pthread_create(&orc_pool.tid[i], NULL, orc_worker, (void *)(intptr_t)i)) return -1;
    return 0;
}

void orc_pool_free(void) {
    if (!orc_pool.tid) return;
    atomic_store(&orc_pool.quit, 1);
    for (int i = 1; i < orc_pool.nth; ++i) pthread_join(orc_pool.tid[i], NULL);
    free(orc_pool.tid);
    orc_pool.tid = NULL;
    orc_pool.nth = 0;
}

int orc_pool_threads(void) { return orc_pool.nth ? orc_pool.nth : 1; }

static void orc_pool_run(orc_job_fn fn, void *arg) {
    if (!orc_pool.tid || orc_pool.nth == 1) {
        fn(arg, 0, 1);
        return;
    }
    orc_pool.fn = fn;
    orc_pool.arg = arg;
    atomic_store_explicit(&orc_pool.done, 0, memory_order_relaxed);
    atomic_fetch_add_explicit(&orc_pool.gen, 1, memory_order_acq_rel);
    fn(arg, 0, orc_pool.nth);
    while (atomic_load_explicit(&orc_pool.done, memory_order_acquire) != orc_pool.nth - 1) _mm_pause();
}

/* ---- baseline jobs ---- */

typedef struct {
    int type, use_iqk;
    const void *w;
    size_t expert_bytes;
    int64_t n, k, ncols, ne11, n_used;
    const float *x;
    const int32_t *ids;
    void *q8;
    float *y;
} orc_job;

static void orc_job_quantize(void *p, int ith, int nth) {
    orc_job *j = (orc_job *)p;
    const size_t qrow = orc_row_size(ORC_TYPE_Q8_K, j->k);
    for (int64_t r = ith; r < j->ncols; r += nth) /* ggml splits the src1 conversion by rows */
        orc_quantize_row_q8_K(j->x + r * j->k, (char *)j->q8 + r * qrow, j->k);
}

static void orc_rows(orc_job *j, const void *w, const void *q8, float *y, int ith, int nth) {
    const size_t row = orc_row_size(j->type, j->k);
    if (j->use_iqk && orc_iqk_mul_mat((long)j->n, 1, (long)j->k, j->type, w, (long)(row / orc_type_size(j->type)),
                                      ORC_TYPE_Q8_K, q8, (long)(j->k / ORC_QK_K), y, (long)j->n, ith, nth))
        return;
    const int64_t per = (j->n + nth - 1) / nth, first = ith * per;
    const int64_t last = first + per < j->n ? first + per : j->n;
    for (int64_t r = first; r < last; ++r) {
        const void *xr = (const char *)w + r * row;
        y[r] = j->type == ORC_TYPE_Q4_K ? orc_vec_dot_q4_K_q8_K(j->k, xr, q8) : orc_vec_dot_q6_K_q8_K(j->k, xr, q8);
    }
}

static void orc_job_gemv(void *p, int ith, int nth) {
    orc_job *j = (orc_job *)p;
    const size_t qrow = orc_row_size(ORC_TYPE_Q8_K, j->k);
    for (int64_t c = 0; c < j->ncols; ++c) orc_rows(j, j->w, (const char *)j->q8 + c * qrow, j->y + c * j->n, ith, nth);
}

static void orc_job_gemv_id(void *p, int ith, int nth) {
    orc_job *j = (orc_job *)p;
    const size_t qrow = orc_row_size(ORC_TYPE_Q8_K, j->k);
    for (int64_t s = 0; s < j->n_used; ++s) {
        float *ys = j->y + s * j->n;
        const int32_t e = j->ids[s];
        if (e < 0) {
            const int64_t per = (j->n + nth - 1) / nth, first = ith * per;
            for (int64_t r = first; r < first + per && r < j->n; ++r) ys[r] = 0.f;
            continue;
        }
        orc_rows(j, (const char *)j->w + (size_t)e * j->expert_bytes, (const char *)j->q8 + (s % j->ne11) * qrow, ys, ith,
                 nth);
    }
}

int orc_baseline_mul_mat(int type, const void *w, int64_t n, int64_t k, const float *x, int64_t ncols, void *q8_scratch,
                         float *y, int use_iqk) {
    if ((type != ORC_TYPE_Q4_K && type != ORC_TYPE_Q6_K) || k % ORC_QK_K) return -1;
    orc_job j = {.type = type, .use_iqk = use_iqk, .w = w, .n = n, .k = k, .ncols = ncols, .x = x, .q8 = q8_scratch, .y = y};
    orc_pool_run(orc_job_quantize, &j);
    orc_pool_run(orc_job_gemv, &j);
    return 0;
}

int orc_baseline_mul_mat_id(int type, const void *w, size_t expert_bytes, int64_t n, int64_t k, const float *x,
                            int64_t ne11, const int32_t *ids, int64_t n_used, void *q8_scratch, float *y, int use_iqk) {
    if ((type != ORC_TYPE_Q4_K && type != ORC_TYPE_Q6_K) || k % ORC_QK_K || ne11 < 1 || n_used % ne11) return -1;
    orc_job j = {.type = type, .use_iqk = use_iqk, .w = w, .expert_bytes = expert_bytes, .n = n, .k = k,
                 .ncols = ne11, .ne11 = ne11, .n_used = n_used, .x = x, .ids = ids, .q8 = q8_scratch, .y = y};
    orc_pool_run(orc_job_quantize, &j);
    orc_pool_run(orc_job_gemv_id, &j);
    return 0;
}
