// tq_skinny.h -- one super-block step of the Q4_K and Q6_K int8-MFMA kernels for a few activation
// columns (the skinny MUL_MAT of tq_skinny.hip and the grouped MUL_MAT_ID of tq_mmid.hip); the Q6_K
// step is at the end.
//
// ggml's dot product per Q4_K super-block (vec_dot_q4_K_q8_K):
//   d_y * (d * sum_j sc_j * sum_{k in j} q_k y_k  -  dmin * sum_j m_j * S_j),  S_j = sum_{k in j} y_k
// with 6-bit sub-block scales sc_j and mins m_j (32 weights each). int8 MFMA needs int8 operands and sc*q
// does not fit a byte, so the weights enter as two digit planes (sc >> 3) q and (sc & 7) q (both <= 105):
// sum_j sc_j sum q y = 8 R0 + R1, each R one int32 MFMA accumulation over the super-block (exact). The
// min term is a 16x16x4 fp32 MFMA pair over (S_j, dmin m_j); it and the per-super-block combination
// round in fp32, in another order than ggml's (within fp32 accumulation error of it).
//
// Operands: A = activations (Q8_K qs straight from the quantized columns; lane l holds column l % 16 of
// a 16-column tile), B = weights (lane l holds weight row l % 16 of a 16-row tile; its header gives the
// row's scales in-lane), C = 16 columns x 16 rows, lane l holding columns 4 (l / 16) + i of row l % 16.
// A lane (column or row r, group g = l / 16) holds the k-slots 64 s + 16 g .. +15 of each 64-deep step
// s of a super-block; for Q4_K those are the low nibbles of qs[32 s + 16 g ..] (g < 2) or the high
// nibbles of qs[32 s + 16 (g - 2) ..] (g >= 2): one 16-byte load per step, one sub-block scale each.
#pragma once

#include "tq_device.h"

namespace tq {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef unsigned short v2u16 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ v4i ld16_a4(const uint8_t *p) {  // 16 bytes at a 4-byte aligned address
    const uint32_t *q = (const uint32_t *)p;
    return v4i{(int)q[0], (int)q[1], (int)q[2], (int)q[3]};
}

// The 4 bytes of q (each <= 15) times s (<= 7), bytewise: two 16-bit lanes, no carry between bytes.
__device__ __forceinline__ int mul_bytes(uint32_t q, uint32_t s) {
    const v2u16 p = __builtin_bit_cast(v2u16, q) * v2u16{(unsigned short)s, (unsigned short)s};
    return __builtin_bit_cast(int, p);
}

// The lane's weight words of one Q4_K block (the header and its four 16-byte qs pieces).
struct Q4kLaneBlock {
    uint4 hdr, qw[4];
    __device__ __forceinline__ void load(const uint8_t *__restrict__ wb) {
        const int g = (threadIdx.x & 63) >> 4;
        hdr = *(const uint4 *)wb;
#pragma unroll
        for (int s = 0; s < 4; ++s) qw[s] = *(const uint4 *)(wb + 16 + 32 * s + 16 * (g & 1));
    }
};

// The activation operands of one 16-column tile against one super-block: column n = lane % 16 of the
// tile (the A operand), its 32-sums S_g and S_{4+g} and d of the C layout's columns 4 g + i.
struct Q4kTileAct {
    v4i A[4];
    float s0, s1;
    v4f dy;
};

// S_j of a Q8_K block from its bsums word j (the two 16-sums of sub-block j).
__device__ __forceinline__ float bsums_pair(uint32_t w) {
    return (float)((int)(int16_t)(w & 0xffff) + (int)(int16_t)(w >> 16));
}

// The tile at column offset c0 of a chunk whose column k's Q8_K block is col_blk(k) (k < nvalid;
// col_blk(0) must be readable); columns k >= nvalid are zero.
template <class ColBlk>
__device__ __forceinline__ void load_tile_act(Q4kTileAct &t, int c0, int nvalid, ColBlk col_blk) {
    const int lane = threadIdx.x & 63, n = lane & 15, g = lane >> 4;
    const int k = c0 + n;
    const bool cv = k < nvalid;
    const uint8_t *qb = col_blk(cv ? k : 0);
#pragma unroll
    for (int s = 0; s < 4; ++s) t.A[s] = cv ? ld16_a4(qb + Q8K_QS + 64 * s + 16 * g) : v4i{0, 0, 0, 0};
    t.s0 = cv ? bsums_pair(*(const uint32_t *)(qb + Q8K_BSUMS + 4 * g)) : 0.f;
    t.s1 = cv ? bsums_pair(*(const uint32_t *)(qb + Q8K_BSUMS + 16 + 4 * g)) : 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int k2 = c0 + 4 * g + i;
        t.dy[i] = k2 < nvalid ? *(const float *)col_blk(k2) : 0.f;
    }
}

// A chunk's activation blocks staged in LDS (the grouped MUL_MAT_ID kernel), pair p = b * ncol + k for
// column k and super-block b: its qs at qs + 256 p with the 16-byte piece c at position c ^ (k % 16)
// (the 16 columns of a tile read one piece each from 16 different bank groups, with no padding), its
// eight 32-sums S_j as floats at S + 8 p and its d at D + p. Columns past the chunk's count hold
// anything: their products are computed and never stored.
__device__ __forceinline__ void load_tile_act_lds(Q4kTileAct &t, const uint8_t *qs, const float *S, const float *D,
                                                  int p0) {
    const int lane = threadIdx.x & 63, n = lane & 15, g = lane >> 4;
    const uint8_t *q = qs + 256 * (p0 + n);
#pragma unroll
    for (int s = 0; s < 4; ++s) t.A[s] = *(const v4i *)(q + 16 * ((4 * s + g) ^ n));
    t.s0 = S[8 * (p0 + n) + g];
    t.s1 = S[8 * (p0 + n) + 4 + g];
    t.dy = *(const v4f *)(D + p0 + 4 * g);
}

// The weight side of one super-block for the lane's row: the two digit planes of its codes, d, and
// dmin times the lane's two mins (rv false: a row past the end, contributing zero).
struct Q4kPlanes {
    v4i D0[4], D1[4];
    float d, mb0, mb1;
};

__device__ __forceinline__ void q4k_planes(const Q4kLaneBlock &w, bool rv, Q4kPlanes &P) {
    const int lane = threadIdx.x & 63, g = lane >> 4;
    const int nsh = 4 * (g >> 1);  // low nibbles for g < 2, high for g >= 2
    const uint4 hdr = w.hdr;
    // scales and mins (ggml's get_scale_min_k4)
    P.d = rv ? half_bits_to_float(hdr.x) : 0.f;
    const float dmin = rv ? half_bits_to_float(hdr.x >> 16) : 0.f;
    const uint32_t sc_lo = hdr.y & 0x3f3f3f3fu, m_lo = hdr.z & 0x3f3f3f3fu;
    const uint32_t sc_hi = (hdr.w & 0x0f0f0f0fu) | ((hdr.y >> 2) & 0x30303030u);
    const uint32_t m_hi = ((hdr.w >> 4) & 0x0f0f0f0fu) | ((hdr.z >> 2) & 0x30303030u);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const uint32_t sc = ((s < 2 ? sc_lo : sc_hi) >> (8 * (2 * (s & 1) + (g >> 1)))) & 0xffu;
        const uint32_t q[4] = {w.qw[s].x, w.qw[s].y, w.qw[s].z, w.qw[s].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t c = (q[i] >> nsh) & 0x0f0f0f0fu;
            P.D0[s][i] = mul_bytes(c, sc >> 3);
            P.D1[s][i] = mul_bytes(c, sc & 7u);
        }
    }
    // dmin * m is exact in fp32 (an 11-bit significand times a 6-bit integer)
    P.mb0 = dmin * (float)((m_lo >> (8 * g)) & 0xffu);
    P.mb1 = dmin * (float)((m_hi >> (8 * g)) & 0xffu);
}

// acc += the products of the lane's weight row (its planes P) with one 16-column tile (operands t)
// against that super-block.
__device__ __forceinline__ void q4k_tile_mma(const Q4kPlanes &P, const Q4kTileAct &t, v4f &acc) {
    v4i R0 = {0, 0, 0, 0}, R1 = {0, 0, 0, 0};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        R0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(t.A[s], P.D0[s], R0, 0, 0, 0);
        R1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(t.A[s], P.D1[s], R1, 0, 0, 0);
    }
    // dmin * sum_j m_j S_j
    v4f Rm = __builtin_amdgcn_mfma_f32_16x16x4f32(t.s0, P.mb0, v4f{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
    Rm = __builtin_amdgcn_mfma_f32_16x16x4f32(t.s1, P.mb1, Rm, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] = __builtin_fmaf(t.dy[i], __builtin_fmaf(P.d, (float)(8 * R0[i] + R1[i]), -Rm[i]), acc[i]);
}

// acc[ct] += the products of the weight block at wb (loaded here) with the MT 16-column tiles of a chunk
// (column k's Q8_K block at col_blk(k), k < nvalid).
template <int MT, class ColBlk>
__device__ __forceinline__ void q4k_skinny_step(const uint8_t *__restrict__ wb, bool rv, int nvalid, ColBlk col_blk,
                                                v4f (&acc)[MT]) {
    Q4kLaneBlock w;
    w.load(wb);
    Q4kTileAct t[MT];
#pragma unroll
    for (int ct = 0; ct < MT; ++ct) load_tile_act(t[ct], 16 * ct, nvalid, col_blk);
    Q4kPlanes P;
    q4k_planes(w, rv, P);
#pragma unroll
    for (int ct = 0; ct < MT; ++ct) q4k_tile_mma(P, t[ct], acc[ct]);
}

// ---- Q6_K: 4 activation columns x 4 scale groups per 16x16x64 step ----
// ggml's vec_dot_q6_K_q8_K per super-block: d * d_y * sum_G sc_G * sum_{k in G} (q_k - 32) y_k over 16
// groups of 16 weights with signed 8-bit scales. In step j (of 4) lane group g = 2h + v holds, for its
// weight row, the 16 codes of group G(j, g) = 8h + 2j + v; A-operand row 4c + i holds column c's Q8_K
// bytes of group G(j, i) in the k-slots of lane group i and zeros elsewhere; the accumulator starts
// from -32 times the column's bsums of those groups. Lane l of the result then holds the four group sums
// of step j for weight row l % 16 and column l / 16.

// The code planes of a Q6_K block for lane group g = 2h + v from 5 aligned dwords of each of its windows
// (ql at 64h + 16v and 64h + 32 + 16v, qh at 128 + 32h + 16v, the scales at 192), the block starting sh
// bytes into each window's first dword: P[j] = the 16 codes (0..63) of group 8h + 2j + v, T = the 16
// scale bytes. (6-bit codes: the low nibble from ql, bits 4-5 from the qh field of the quarter; a
// bit-field insert merges them without the neighbour byte's bits leaking in.)
__device__ __forceinline__ void q6k_planes(const uint32_t (&ra)[5], const uint32_t (&rb)[5], const uint32_t (&rh)[5],
                                           const uint32_t (&rt)[5], uint32_t sh, v4i (&P)[4], uint32_t (&T)[4]) {
    const uint32_t m4 = 0x0f0f0f0fu;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t A = align_bytes(ra[i + 1], ra[i], sh), B = align_bytes(rb[i + 1], rb[i], sh);
        const uint32_t H = align_bytes(rh[i + 1], rh[i], sh);
        T[i] = align_bytes(rt[i + 1], rt[i], sh);
        const uint32_t Hl = H & 0x33333333u, Hh = (H >> 2) & 0x33333333u;
        P[0][i] = (int)bfi(m4, A, Hl << 4);
        P[1][i] = (int)bfi(m4, B, Hh << 4);
        P[2][i] = (int)bfi(m4, A >> 4, Hl);
        P[3][i] = (int)bfi(m4, B >> 4, Hh);
    }
}

// sum_G sc_G * (the group sums of one set of 4 columns) over the 4 steps of a super-block: a_op(j) and
// c_op(j) give the A operand and the accumulator start of step j.
template <class AOp, class COp>
__device__ __forceinline__ int q6k_set_isum(const v4i (&P)[4], const uint32_t (&T)[4], AOp a_op, COp c_op) {
    int isum = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const v4i R = __builtin_amdgcn_mfma_i32_16x16x64_i8(a_op(j), P[j], c_op(j), 0, 0, 0);
        // scales of groups 2j, 2j + 1 (bytes of T[j / 2]) and 8 + 2j, 9 + 2j (of T[2 + j / 2])
        const int bp = 16 * (j & 1);
        isum = mad24(sext8(T[j >> 1], bp), R[0], isum);
        isum = mad24(sext8(T[j >> 1], bp + 8), R[1], isum);
        isum = mad24(sext8(T[2 + (j >> 1)], bp), R[2], isum);
        isum = mad24(sext8(T[2 + (j >> 1)], bp + 8), R[3], isum);
    }
    return isum;
}

// Stages super-block b of a column into the Q6_K operand layout (called by one wave; lane l has the
// column's packed qs bytes 4l .. 4l + 3 in pk, its quad's bsum (group l / 4) in bs and d in dq): qs at
// aq (256 bytes), -32 x bsum of group G at cin[j * 4 + i] for G = 8 (i >> 1) + 2 j + (i & 1), d at *dp.
__device__ __forceinline__ void q6k_stage_column(uint32_t pk, int bs, float dq, uint8_t *aq, int *cin, float *dp) {
    const int lane = (int)(threadIdx.x & 63);
    *(uint32_t *)(aq + 4 * lane) = pk;
    if ((lane & 3) == 0) {
        const int G = lane >> 2, j = (G >> 1) & 3, i = ((G >> 3) << 1) | (G & 1);
        cin[j * 4 + i] = -32 * bs;
    }
    if (lane == 0) *dp = dq;
}

}  // namespace tq
