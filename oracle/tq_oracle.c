/*
 * tq_oracle.c -- CPU oracle for the Q4_K / Q6_K x Q8_K matmul path (TEST INFRASTRUCTURE ONLY).
 *
 * Plain C restatement of ggml b12426's scalar reference algorithms (ggml is an absent submodule of the
 * reference, vendor/PIN:1-2). Built with -ffp-contract=off so every float operation rounds as written.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this library.
 *
 * How each function is pinned (tests/test_oracle_*.py):
 *   orc_fp16_to_fp32          exhaustive over all 65536 halves against numpy's float16 conversion.
 *   orc_quantize_row_q8_K     hand known-answer blocks (exact scales, round-half-even ties, first-max
 *                             rule, all-zero block), invariants (bsums, |qs|<=127, d = 1/(-127/max)).
 *   orc_dequantize_row_q4_K   the iqk formulation of the scale unpack and nibble order
 *                             (patches/0002:371-380, :1430-1440) restated independently in numpy.
 *   orc_dequantize_row_q6_K   the iqk formulation prepare64 + add_high_bits (patches/0002:1638-1663)
 *                             restated independently in numpy.
 *   orc_vec_dot_*             f64 brute force over the dequantized rows with the bound of
 *                             crates/ggml-sys/tests/iqk_kernels.rs:127-148, and the AVX-512 iqk-style
 *                             baseline (a different summation route) within the same bound.
 *   orc_mul_mat(_id)          per-expert reassembly as crates/ggml-sys/tests/mul_mat_id_skip.rs:124-206,
 *                             -1 rows exactly zero, broadcast rules, F32 known answer of
 *                             crates/ggml-sys/tests/ggml.rs:13-30 through the Q8_K path.
 */
#include "tq_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

_Static_assert(sizeof(orc_block_q4_K) == 144, "block_q4_K is 144 bytes");
_Static_assert(sizeof(orc_block_q6_K) == 210, "block_q6_K is 210 bytes");
_Static_assert(sizeof(orc_block_q8_K) == 292, "block_q8_K is 292 bytes");

/* IEEE 754 binary16 -> binary32, exact (every half is representable as a float). */
float orc_fp16_to_fp32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    const uint32_t exp = (h >> 10) & 0x1f;
    const uint32_t man = h & 0x3ff;
    uint32_t bits;
    if (exp == 0) {
        /* zero or subnormal: man * 2^-24, exact in binary32 */
        float f = (float)man * 5.9604644775390625e-08f;
        memcpy(&bits, &f, 4);
        bits |= sign;
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp - 15 + 127) << 23) | (man << 13);
    }
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

size_t orc_type_size(int type) {
    switch (type) {
    case ORC_TYPE_F32: return 4;
    case ORC_TYPE_I32: return 4;
    case ORC_TYPE_Q4_K: return sizeof(orc_block_q4_K);
    case ORC_TYPE_Q6_K: return sizeof(orc_block_q6_K);
    case ORC_TYPE_Q8_K: return sizeof(orc_block_q8_K);
    default: return 0;
    }
}

int64_t orc_blck_size(int type) {
    switch (type) {
    case ORC_TYPE_Q4_K:
    case ORC_TYPE_Q6_K:
    case ORC_TYPE_Q8_K: return ORC_QK_K;
    case ORC_TYPE_F32:
    case ORC_TYPE_I32: return 1;
    default: return 0;
    }
}

size_t orc_row_size(int type, int64_t ne) {
    const int64_t b = orc_blck_size(type);
    if (b == 0 || ne % b) return 0;
    return orc_type_size(type) * (size_t)(ne / b);
}

/* ggml's nearest_int: add 1.5 * 2^23 so the float's low mantissa bits hold the integer rounded to
 * nearest, ties to even (valid for |v| <= 2^22). */
static int orc_nearest_int(float v) {
    float t = v + 12582912.f;
    int32_t i;
    memcpy(&i, &t, 4);
    return (i & 0x007fffff) - 0x00400000;
}

/* quantize_row_q8_K_ref (ggml-quants.c at b12426), per 256-element block:
 *   max = the first element with the largest |x| (strict >),
 *   all-zero block: d = 0, qs = 0 (ggml leaves bsums unwritten; this oracle writes 0),
 *   iscale = -127/max, qs = min(127, nearest_int(iscale * x)), bsums = sums of 16 qs, d = 1/iscale. */
void orc_quantize_row_q8_K(const float *x, void *vy, int64_t k) {
    orc_block_q8_K *y = (orc_block_q8_K *)vy;
    const int64_t nb = k / ORC_QK_K;
    for (int64_t i = 0; i < nb; ++i, x += ORC_QK_K) {
        float amax = 0.f, max = 0.f;
        for (int j = 0; j < ORC_QK_K; ++j) {
            const float ax = fabsf(x[j]);
            if (ax > amax) {
                amax = ax;
                max = x[j];
            }
        }
        if (amax == 0.f) {
            y[i].d = 0.f;
            memset(y[i].qs, 0, sizeof y[i].qs);
            memset(y[i].bsums, 0, sizeof y[i].bsums);
            continue;
        }
        const float iscale = -127.f / max;
        for (int j = 0; j < ORC_QK_K; ++j) {
            const int v = orc_nearest_int(iscale * x[j]);
            y[i].qs[j] = (int8_t)(v < 127 ? v : 127);
        }
        for (int g = 0; g < ORC_QK_K / 16; ++g) {
            int s = 0;
            for (int l = 0; l < 16; ++l) s += y[i].qs[16 * g + l];
            y[i].bsums[g] = (int16_t)s;
        }
        y[i].d = 1.f / iscale;
    }
}

void orc_dequantize_row_q8_K(const void *vx, float *y, int64_t k) {
    const orc_block_q8_K *x = (const orc_block_q8_K *)vx;
    const int64_t nb = k / ORC_QK_K;
    for (int64_t i = 0; i < nb; ++i)
        for (int j = 0; j < ORC_QK_K; ++j) *y++ = x[i].d * x[i].qs[j];
}

/* The 12-byte scale field of block_q4_K holds eight 6-bit scales and eight 6-bit mins. Sub-blocks
 * 0..3 keep scale and min in the low 6 bits of bytes j and j+4; sub-blocks 4..7 keep their low 4 bits
 * in the nibbles of byte j+4 and their top 2 bits in the top bits of bytes j-4 (scale) and j (min). */
static void orc_q4_K_scale_min(int j, const uint8_t *s, int *sc, int *m) {
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (s[j + 4] & 0x0f) | ((s[j - 4] >> 6) << 4);
        *m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

/* Element e of a Q4_K block: qs byte 32*(e/64) + e%32, low nibble when (e/32) is even. */
void orc_dequantize_row_q4_K(const void *vx, float *y, int64_t k) {
    const orc_block_q4_K *x = (const orc_block_q4_K *)vx;
    const int64_t nb = k / ORC_QK_K;
    for (int64_t i = 0; i < nb; ++i) {
        const float d = orc_fp16_to_fp32(x[i].d);
        const float dmin = orc_fp16_to_fp32(x[i].dmin);
        for (int c = 0; c < 4; ++c) {
            const uint8_t *q = x[i].qs + 32 * c;
            int sc, m;
            orc_q4_K_scale_min(2 * c, x[i].scales, &sc, &m);
            const float d1 = d * sc, m1 = dmin * m;
            orc_q4_K_scale_min(2 * c + 1, x[i].scales, &sc, &m);
            const float d2 = d * sc, m2 = dmin * m;
            for (int l = 0; l < 32; ++l) *y++ = d1 * (q[l] & 0x0f) - m1;
            for (int l = 0; l < 32; ++l) *y++ = d2 * (q[l] >> 4) - m2;
        }
    }
}

/* The 6-bit quant of element e of a Q6_K block (0..63, before the -32 offset). For half h = e/128 and
 * r = e%128, l = r%32, quarter t = r/32: low nibble of ql[64h + 32*(t&1) + l] (t<2) or its high
 * nibble (t>=2), with bits 2t..2t+1 of qh[32h + l] on top. The scale of element e is scales[e/16]. */
static int orc_q6_K_quant(const orc_block_q6_K *b, int e) {
    const int h = e / 128, r = e % 128, t = r / 32, l = r % 32;
    const uint8_t lq = b->ql[64 * h + 32 * (t & 1) + l];
    const int lo = t < 2 ? (lq & 0x0f) : (lq >> 4);
    const int hi = (b->qh[32 * h + l] >> (2 * t)) & 3;
    return lo | (hi << 4);
}

void orc_dequantize_row_q6_K(const void *vx, float *y, int64_t k) {
    const orc_block_q6_K *x = (const orc_block_q6_K *)vx;
    const int64_t nb = k / ORC_QK_K;
    for (int64_t i = 0; i < nb; ++i) {
        const float d = orc_fp16_to_fp32(x[i].d);
        for (int e = 0; e < ORC_QK_K; ++e)
            *y++ = d * x[i].scales[e / 16] * (orc_q6_K_quant(&x[i], e) - 32);
    }
}

/* ggml_vec_dot_q4_K_q8_K (generic scalar form): exact integer sums per super-block, split over eight
 * lanes (element index mod 8) like ggml's generic kernel; the mins enter through the Q8_K bsums:
 *   sum_i  d_x d_y * sum_lane sum_j sc_j q.y  -  dmin_x d_y * sum_j m_j (bsums[2j] + bsums[2j+1]). */
float orc_vec_dot_q4_K_q8_K(int64_t n, const void *vx, const void *vy) {
    const orc_block_q4_K *x = (const orc_block_q4_K *)vx;
    const orc_block_q8_K *y = (const orc_block_q8_K *)vy;
    const int64_t nb = n / ORC_QK_K;
    float lane_sums[8] = {0};
    float sumf = 0.f;
    for (int64_t i = 0; i < nb; ++i) {
        int32_t lane[8] = {0};
        int sc[8], m[8];
        for (int j = 0; j < 8; ++j) orc_q4_K_scale_min(j, x[i].scales, &sc[j], &m[j]);
        int32_t summ = 0;
        for (int j = 0; j < 8; ++j) summ += m[j] * (y[i].bsums[2 * j] + y[i].bsums[2 * j + 1]);
        for (int e = 0; e < ORC_QK_K; ++e) {
            const uint8_t byte = x[i].qs[32 * (e / 64) + e % 32];
            const int q = ((e / 32) & 1) ? (byte >> 4) : (byte & 0x0f);
            lane[e % 8] += sc[e / 32] * (q * y[i].qs[e]);
        }
        const float d = orc_fp16_to_fp32(x[i].d) * y[i].d;
        for (int l = 0; l < 8; ++l) lane_sums[l] += d * (float)lane[l];
        const float dmin = orc_fp16_to_fp32(x[i].dmin) * y[i].d;
        sumf -= dmin * (float)summ;
    }
    for (int l = 0; l < 8; ++l) sumf += lane_sums[l];
    return sumf;
}

/* ggml_vec_dot_q6_K_q8_K (generic scalar form): sum_i d_x d_y * sum_lane sum_g sc_g (q-32).y. */
float orc_vec_dot_q6_K_q8_K(int64_t n, const void *vx, const void *vy) {
    const orc_block_q6_K *x = (const orc_block_q6_K *)vx;
    const orc_block_q8_K *y = (const orc_block_q8_K *)vy;
    const int64_t nb = n / ORC_QK_K;
    float lane_sums[8] = {0};
    float sumf = 0.f;
    for (int64_t i = 0; i < nb; ++i) {
        int32_t lane[8] = {0};
        for (int e = 0; e < ORC_QK_K; ++e) {
            const int q = orc_q6_K_quant(&x[i], e) - 32;
            lane[e % 8] += x[i].scales[e / 16] * (q * y[i].qs[e]);
        }
        const float d = orc_fp16_to_fp32(x[i].d) * y[i].d;
        for (int l = 0; l < 8; ++l) lane_sums[l] += d * (float)lane[l];
    }
    for (int l = 0; l < 8; ++l) sumf += lane_sums[l];
    return sumf;
}

static float orc_vec_dot(int type, int64_t n, const void *x, const void *y) {
    return type == ORC_TYPE_Q4_K ? orc_vec_dot_q4_K_q8_K(n, x, y) : orc_vec_dot_q6_K_q8_K(n, x, y);
}

static int orc_is_weight_type(int type) { return type == ORC_TYPE_Q4_K || type == ORC_TYPE_Q6_K; }

/* ggml_compute_forward_mul_mat: src1 rows converted to Q8_K, then
 * dst[i01, i11, i12, i13] = vec_dot(a[:, i01, i12/r2, i13/r3], q8(b[:, i11, i12, i13])). */
int orc_mul_mat(const orc_tensor *a, const orc_tensor *b, orc_tensor *dst) {
    if (!orc_is_weight_type(a->type) || b->type != ORC_TYPE_F32 || dst->type != ORC_TYPE_F32) return -1;
    const int64_t K = a->ne[0];
    if (K % ORC_QK_K || b->ne[0] != K) return -1;
    if (b->ne[2] % a->ne[2] || b->ne[3] % a->ne[3]) return -1;
    if (dst->ne[0] != a->ne[1] || dst->ne[1] != b->ne[1] || dst->ne[2] != b->ne[2] || dst->ne[3] != b->ne[3])
        return -1;
    if (a->nb[0] != orc_type_size(a->type) || b->nb[0] != sizeof(float) || dst->nb[0] != sizeof(float)) return -1;
    const int64_t r2 = b->ne[2] / a->ne[2], r3 = b->ne[3] / a->ne[3];
    const size_t qrow = orc_row_size(ORC_TYPE_Q8_K, K);
    void *q = malloc(qrow);
    if (!q) return -2;
    for (int64_t i13 = 0; i13 < b->ne[3]; ++i13)
        for (int64_t i12 = 0; i12 < b->ne[2]; ++i12)
            for (int64_t i11 = 0; i11 < b->ne[1]; ++i11) {
                const float *brow =
                    (const float *)((const char *)b->data + i11 * b->nb[1] + i12 * b->nb[2] + i13 * b->nb[3]);
                orc_quantize_row_q8_K(brow, q, K);
                const char *abase = (const char *)a->data + (i12 / r2) * a->nb[2] + (i13 / r3) * a->nb[3];
                float *drow = (float *)((char *)dst->data + i11 * dst->nb[1] + i12 * dst->nb[2] + i13 * dst->nb[3]);
                for (int64_t i01 = 0; i01 < a->ne[1]; ++i01) drow[i01] = orc_vec_dot(a->type, K, abase + i01 * a->nb[1], q);
            }
    free(q);
    return 0;
}

/* ggml_compute_forward_mul_mat_id with patch 0004's rule: as [K, N, E], b [K, ne11, T], ids I32
 * [n_used, T], dst [N, n_used, T]; slot (j, t) reads src1 row b[:, j % ne11, t]; id < 0 -> zero row. */
int orc_mul_mat_id(const orc_tensor *as, const orc_tensor *b, const orc_tensor *ids, orc_tensor *dst) {
    if (!orc_is_weight_type(as->type) || b->type != ORC_TYPE_F32 || ids->type != ORC_TYPE_I32 ||
        dst->type != ORC_TYPE_F32)
        return -1;
    const int64_t K = as->ne[0], N = as->ne[1], E = as->ne[2];
    const int64_t n_used = ids->ne[0], T = ids->ne[1], ne11 = b->ne[1];
    if (K % ORC_QK_K || b->ne[0] != K || b->ne[2] != T || ne11 < 1 || n_used % ne11) return -1;
    if (dst->ne[0] != N || dst->ne[1] != n_used || dst->ne[2] != T) return -1;
    const size_t qrow = orc_row_size(ORC_TYPE_Q8_K, K);
    void *q = malloc(qrow);
    if (!q) return -2;
    for (int64_t t = 0; t < T; ++t)
        for (int64_t j = 0; j < n_used; ++j) {
            const int32_t e = *(const int32_t *)((const char *)ids->data + j * ids->nb[0] + t * ids->nb[1]);
            float *drow = (float *)((char *)dst->data + j * dst->nb[1] + t * dst->nb[2]);
            if (e < 0) {
                for (int64_t n = 0; n < N; ++n) drow[n] = 0.f;
                continue;
            }
            if (e >= E) {
                free(q);
                return -1;
            }
            const float *brow = (const float *)((const char *)b->data + (j % ne11) * b->nb[1] + t * b->nb[2]);
            orc_quantize_row_q8_K(brow, q, K);
            const char *abase = (const char *)as->data + e * as->nb[2];
            for (int64_t n = 0; n < N; ++n) drow[n] = orc_vec_dot(as->type, K, abase + n * as->nb[1], q);
        }
    free(q);
    return 0;
}

int orc_ref_f64_rows(int type, const void *w_rows, size_t row_bytes, int64_t n, int64_t k, const float *x,
                     double *out, double *bound) {
    if (!orc_is_weight_type(type) || k % ORC_QK_K) return -1;
    float *xq = malloc(sizeof(float) * k), *w = malloc(sizeof(float) * k);
    void *q = malloc(orc_row_size(ORC_TYPE_Q8_K, k));
    if (!xq || !w || !q) {
        free(xq), free(w), free(q);
        return -2;
    }
    orc_quantize_row_q8_K(x, q, k);
    orc_dequantize_row_q8_K(q, xq, k);
    for (int64_t r = 0; r < n; ++r) {
        const void *row = (const char *)w_rows + r * row_bytes;
        if (type == ORC_TYPE_Q4_K) orc_dequantize_row_q4_K(row, w, k);
        else orc_dequantize_row_q6_K(row, w, k);
        double s = 0, a = 0;
        for (int64_t i = 0; i < k; ++i) {
            const double p = (double)w[i] * (double)xq[i];
            s += p;
            a += fabs(p);
        }
        out[r] = s;
        bound[r] = 1e-5 * a + 1e-6;
    }
    free(xq), free(w), free(q);
    return 0;
}
