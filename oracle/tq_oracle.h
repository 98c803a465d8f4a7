/*
 * tq_oracle.h -- CPU oracle for the Q4_K / Q6_K x Q8_K matmul path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product library links, loads or calls this code; only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, as the checker and as the
 * reported CPU baseline. It is a plain-C restatement of ggml's (b12426) scalar algorithms for the
 * block formats, written from the format definitions and the reference's own evidence:
 *
 *   block_q4_K   reference: patches/0002-iqk-avx512-q4k-q6k-decode.patch:371-380 (scale unpack),
 *                :1430-1440 (nibble order), :1474-1487 (d, dmin, scales, qs)
 *   block_q6_K   reference: patches/0002:1638-1663 (ql, qh, scales, d; -32 offset via bsums)
 *   block_q8_K   reference: patches/0002:1277-1294 (d, qs, bsums); quantize_row_q8_K_ref is called at
 *                crates/ggml-sys/tests/iqk_kernels.rs:52,64 (ggml b12426, ggml-quants.c)
 *   MUL_MAT      reference: crates/ggml-sys/src/ggml/context.rs:294-299
 *   MUL_MAT_ID   reference: crates/ggml-sys/src/ggml/context.rs:320-336, patches/0004 (id < 0 -> zero row)
 *
 * Which checks pin each function is listed in tq_oracle.c next to the function.
 */
#ifndef TQ_ORACLE_H
#define TQ_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_QK_K 256

/* ggml_type ids (ggml.h enum ggml_type; also the GGUF tensor type ids). */
enum {
    ORC_TYPE_F32 = 0,
    ORC_TYPE_Q4_K = 12,
    ORC_TYPE_Q6_K = 14,
    ORC_TYPE_Q8_K = 15,
    ORC_TYPE_I32 = 26,
};

typedef struct {
    uint16_t d;          /* fp16 super-block scale for the 6-bit sub-block scales */
    uint16_t dmin;       /* fp16 super-block scale for the 6-bit sub-block mins   */
    uint8_t scales[12];  /* 8 scales + 8 mins, 6 bits each                         */
    uint8_t qs[128];     /* 4-bit quants                                           */
} orc_block_q4_K;        /* 144 bytes */

typedef struct {
    uint8_t ql[128];     /* low 4 bits of the 6-bit quants  */
    uint8_t qh[64];      /* high 2 bits of the 6-bit quants */
    int8_t scales[16];   /* 8-bit sub-block scales          */
    uint16_t d;          /* fp16 super-block scale          */
} orc_block_q6_K;        /* 210 bytes */

typedef struct {
    float d;             /* delta                              */
    int8_t qs[256];      /* quants                             */
    int16_t bsums[16];   /* sum of quants in groups of 16      */
} orc_block_q8_K;        /* 292 bytes */

/* A ggml tensor view: ne[] elements per dimension, nb[] byte strides (ggml.h struct ggml_tensor). */
typedef struct {
    int32_t type;
    int64_t ne[4];
    size_t nb[4];
    void *data;
} orc_tensor;

float orc_fp16_to_fp32(uint16_t h);
size_t orc_type_size(int type);   /* bytes per block (per element for F32/I32) */
int64_t orc_blck_size(int type);  /* elements per block                        */
size_t orc_row_size(int type, int64_t ne);

void orc_quantize_row_q8_K(const float *x, void *y, int64_t k);
void orc_dequantize_row_q8_K(const void *x, float *y, int64_t k);
void orc_dequantize_row_q4_K(const void *x, float *y, int64_t k);
void orc_dequantize_row_q6_K(const void *x, float *y, int64_t k);

float orc_vec_dot_q4_K_q8_K(int64_t n, const void *vx, const void *vy);
float orc_vec_dot_q6_K_q8_K(int64_t n, const void *vx, const void *vy);

/* dst = a . b with ggml MUL_MAT semantics (a quantized [K, N, ne2, ne3], b F32 [K, M, ne12, ne13],
 * dst F32 [N, M, ne12, ne13], broadcast of a over dims 2 and 3). Returns 0, or -1 on bad shapes. */
int orc_mul_mat(const orc_tensor *a, const orc_tensor *b, orc_tensor *dst);

/* dst[:, j, t] = as[:, :, ids[j, t]] . b[:, j % ne11, t]; ids < 0 give an exact zero row. */
int orc_mul_mat_id(const orc_tensor *as, const orc_tensor *b, const orc_tensor *ids, orc_tensor *dst);

/* f64 reference: dequantized weight rows against the Q8_K round trip of x, with the per-output bound
 * 1e-5 * sum|w*x| + 1e-6 of crates/ggml-sys/tests/iqk_kernels.rs:127-148. w_rows are n rows of
 * row_bytes each; x is one row of k floats; out and bound get n values. */
int orc_ref_f64_rows(int type, const void *w_rows, size_t row_bytes, int64_t n, int64_t k,
                     const float *x, double *out, double *bound);

/* ---- CPU baseline (tq_cpu_baseline.c): restatement of the iqk AVX-512 VNNI one-column GEMV. ---- */

/* The ABI of ggml_iqk_mul_mat (patches/0002:170-195): C[0..Nx) of this thread's static share of rows.
 * Ny must be 1. Returns 0 when not handled (types or ISA), 1 when done. */
int orc_iqk_mul_mat(long Nx, long Ny, long ne00, int typeA, const void *A, long strideA, int typeB,
                    const void *B, long strideB, float *C, long stride_C, int ith, int nth);

/* 1 when the host has AVX-512 F/BW/DQ/VL + VNNI, the iqk kernel's requirement. */
int orc_cpu_has_avx512_vnni(void);

/* Thread pool for the baseline: nth threads (including the caller). */
int orc_pool_init(int nth);
void orc_pool_free(void);
int orc_pool_threads(void);

/* One MUL_MAT decode step on the pool: quantize x (ncols rows of k floats) to Q8_K, then for each
 * column the static-split GEMV over n rows (iqk path when available, else the scalar vec_dot).
 * y is [ncols][n]. q8 scratch must hold ncols * k/256 Q8_K blocks. use_iqk=0 forces vec_dot. */
int orc_baseline_mul_mat(int type, const void *w, int64_t n, int64_t k, const float *x, int64_t ncols,
                         void *q8_scratch, float *y, int use_iqk);

/* One MUL_MAT_ID decode step (one token): quantize x (ne11 rows of k) to Q8_K, then one GEMV per
 * routed slot with id >= 0 (the hook at patches/0002:36-57), zero rows for id < 0. w is the stacked
 * [k, n, n_expert] tensor with expert stride expert_bytes. y is [n_used][n]. */
int orc_baseline_mul_mat_id(int type, const void *w, size_t expert_bytes, int64_t n, int64_t k,
                            const float *x, int64_t ne11, const int32_t *ids, int64_t n_used,
                            void *q8_scratch, float *y, int use_iqk);

#ifdef __cplusplus
}
#endif

#endif
