// tq_skinny.hip -- MUL_MAT over Q4_K weights for a few activation columns (batched decode, 9..64
// columns) on int8 MFMA (v_mfma_i32_16x16x64_i8), every weight byte read once for all columns.
//
// ggml's dot product per Q4_K super-block (vec_dot_q4_K_q8_K):
//   d_y * (d * sum_j sc_j * sum_{k in j} q_k y_k  -  dmin * sum_j m_j * S_j),  S_j = sum_{k in j} y_k
// with 6-bit sub-block scales sc_j and mins m_j (32 weights each). int8 MFMA needs int8 operands and sc*q
// does not fit a byte, so the weights enter as two digit planes (sc >> 3) q and (sc & 7) q (both <= 105):
// sum_j sc_j sum q y = 8 R0 + R1, each R one int32 MFMA accumulation over the super-block. The min term
// is a 16x16x4 fp32 MFMA pair over (S_j, m_j) (exact: |m_j S_j| < 2^18). Only the per-super-block
// combination rounds, in fp32, as in ggml.
//
// Operands: A = activations (Q8_K qs straight from the quantized columns; lane l holds column l % 16 of
// a 16-column tile), B = weights (lane l holds weight row l % 16 of a 16-row tile; its header gives the
// row's scales in-lane), C = 16 columns x 16 rows, lane l holding columns 4 (l / 16) + i of row l % 16.
// A lane (column or row r, group g = l / 16) holds the k-slots 64 s + 16 g .. +15 of each 64-deep step
// s of a super-block; for Q4_K those are the low nibbles of qs[32 s + 16 g ..] (g < 2) or the high
// nibbles of qs[32 s + 16 (g - 2) ..] (g >= 2): one 16-byte load per step, one sub-block scale each.
// Grid: one workgroup of 4 waves per 16-row tile; the waves split the super-blocks and their partial
// sums meet in LDS.
#include "tq_device.h"
#include "tq_internal.h"

#include <algorithm>

namespace tq {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef unsigned short v2u16 __attribute__((ext_vector_type(2)));

#ifndef TQ_SK_WAVES
#define TQ_SK_WAVES 8
#endif
constexpr int SK_WAVES = TQ_SK_WAVES;

__device__ __forceinline__ v4i ld16_a4(const uint8_t *p) {  // 16 bytes at a 4-byte aligned address
    const uint32_t *q = (const uint32_t *)p;
    return v4i{(int)q[0], (int)q[1], (int)q[2], (int)q[3]};
}

// The 4 bytes of q (each <= 15) times s (<= 7), bytewise: two 16-bit lanes, no carry between bytes.
__device__ __forceinline__ int mul_bytes(uint32_t q, uint32_t s) {
    const v2u16 p = __builtin_bit_cast(v2u16, q) * v2u16{(unsigned short)s, (unsigned short)s};
    return __builtin_bit_cast(int, p);
}

template <int MT>
__global__ __launch_bounds__(SK_WAVES * 64) void k_skinny_q4k(SkinnyArgs a) {
    __shared__ v4f red[SK_WAVES - 1][MT][64];  // partial sums of waves 1 .. SK_WAVES-1
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n = lane & 15, g = lane >> 4;
    const int nb = a.nb;
    const int i2 = blockIdx.y % a.ne12, i3 = blockIdx.y / a.ne12;
    const uint8_t *w = a.w + (int64_t)(i2 / a.r2) * a.w_s2 + (int64_t)(i3 / a.r3) * a.w_s3;
    const uint8_t *q8 = a.q8 + (int64_t)blockIdx.y * a.ncols * nb * Q8K_BYTES;
    float *dst = a.dst + i2 * a.d_s2 + i3 * a.d_s3;
    const int64_t row = (int64_t)blockIdx.x * 16 + n;
    const bool rv = row < a.nrows;
    const uint8_t *wrow = w + (rv ? row : 0) * a.row_stride;
    const int nsh = 4 * (g >> 1);  // low nibbles for g < 2, high for g >= 2

    // column chunks of 16 MT: the row tile's weights come from HBM once and from L2 for later chunks
    for (int c0 = 0; c0 < a.ncols; c0 += 16 * MT) {
        v4f acc[MT];
#pragma unroll
        for (int ct = 0; ct < MT; ++ct) acc[ct] = v4f{0.f, 0.f, 0.f, 0.f};
        for (int b = wave; b < nb; b += SK_WAVES) {
            // weights of row `row`, super-block b: header and this lane's four 16-byte qs pieces
            const uint8_t *wb = wrow + (int64_t)b * Q4K_BYTES;
            const uint4 hdr = *(const uint4 *)wb;
            uint4 qw[4];
#pragma unroll
            for (int s = 0; s < 4; ++s) qw[s] = *(const uint4 *)(wb + 16 + 32 * s + 16 * (g & 1));
            // activations: column c0 + 16 ct + n (A), its 32-sums S_g and S_{4+g}, and d of the C layout's
            // columns c0 + 16 ct + 4 g + i
            v4i A[MT][4];
            float s0[MT], s1[MT];
            v4f dy[MT];
#pragma unroll
            for (int ct = 0; ct < MT; ++ct) {
                const int col = c0 + 16 * ct + n;
                const bool cv = col < a.ncols;
                const uint8_t *qb = q8 + ((int64_t)(cv ? col : 0) * nb + b) * Q8K_BYTES;
#pragma unroll
                for (int s = 0; s < 4; ++s) A[ct][s] = cv ? ld16_a4(qb + Q8K_QS + 64 * s + 16 * g) : v4i{0, 0, 0, 0};
                const uint32_t bs0 = *(const uint32_t *)(qb + Q8K_BSUMS + 4 * g);
                const uint32_t bs1 = *(const uint32_t *)(qb + Q8K_BSUMS + 16 + 4 * g);
                s0[ct] = cv ? (float)((int)(int16_t)(bs0 & 0xffff) + (int)(int16_t)(bs0 >> 16)) : 0.f;
                s1[ct] = cv ? (float)((int)(int16_t)(bs1 & 0xffff) + (int)(int16_t)(bs1 >> 16)) : 0.f;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int c2 = c0 + 16 * ct + 4 * g + i;
                    dy[ct][i] = c2 < a.ncols ? *(const float *)(q8 + ((int64_t)c2 * nb + b) * Q8K_BYTES) : 0.f;
                }
            }
            // scales and mins (ggml's get_scale_min_k4), the two digit planes of this lane's codes
            const float d = rv ? half_bits_to_float(hdr.x) : 0.f, dmin = rv ? half_bits_to_float(hdr.x >> 16) : 0.f;
            const uint32_t sc_lo = hdr.y & 0x3f3f3f3fu, m_lo = hdr.z & 0x3f3f3f3fu;
            const uint32_t sc_hi = (hdr.w & 0x0f0f0f0fu) | ((hdr.y >> 2) & 0x30303030u);
            const uint32_t m_hi = ((hdr.w >> 4) & 0x0f0f0f0fu) | ((hdr.z >> 2) & 0x30303030u);
            v4i D0[4], D1[4];
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const uint32_t sc = ((s < 2 ? sc_lo : sc_hi) >> (8 * (2 * (s & 1) + (g >> 1)))) & 0xffu;
                const uint32_t q[4] = {qw[s].x, qw[s].y, qw[s].z, qw[s].w};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t c = (q[i] >> nsh) & 0x0f0f0f0fu;
                    D0[s][i] = mul_bytes(c, sc >> 3);
                    D1[s][i] = mul_bytes(c, sc & 7u);
                }
            }
            const float mb0 = (float)((m_lo >> (8 * g)) & 0xffu), mb1 = (float)((m_hi >> (8 * g)) & 0xffu);
#pragma unroll
            for (int ct = 0; ct < MT; ++ct) {
                v4i R0 = {0, 0, 0, 0}, R1 = {0, 0, 0, 0};
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    R0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[ct][s], D0[s], R0, 0, 0, 0);
                    R1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[ct][s], D1[s], R1, 0, 0, 0);
                }
                v4f Rm = __builtin_amdgcn_mfma_f32_16x16x4f32(s0[ct], mb0, v4f{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                Rm = __builtin_amdgcn_mfma_f32_16x16x4f32(s1[ct], mb1, Rm, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    acc[ct][i] = __builtin_fmaf(dy[ct][i], d * (float)(8 * R0[i] + R1[i]) - dmin * Rm[i], acc[ct][i]);
            }
        }
        // the waves' super-block shares meet in LDS; wave 0 adds them up and stores the chunk
        if (wave > 0) {
#pragma unroll
            for (int ct = 0; ct < MT; ++ct) red[wave - 1][ct][lane] = acc[ct];
        }
        __syncthreads();
        if (wave == 0 && rv) {
#pragma unroll
            for (int ct = 0; ct < MT; ++ct) {
                v4f v = acc[ct];
#pragma unroll
                for (int k = 0; k < SK_WAVES - 1; ++k) v += red[k][ct][lane];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int col = c0 + 16 * ct + 4 * g + i;
                    if (col < a.ncols) dst[col * a.d_s1 + row] = v[i];
                }
            }
        }
        __syncthreads();  // red is rewritten by the next chunk
    }
}

bool skinny_supported(int type, int64_t ncols) { return type == FMT_Q4K && ncols >= 1 && ncols <= 0x7fffffff; }

hipError_t launch_skinny(int type, const SkinnyArgs &a, hipStream_t stream) {
    if (!skinny_supported(type, a.ncols)) return hipErrorNotSupported;
    const dim3 grid((unsigned)((a.nrows + 15) / 16), (unsigned)a.nbatch);
    const int mt = (a.ncols + 15) / 16;
    switch (mt) {
    case 1: k_skinny_q4k<1><<<grid, SK_WAVES * 64, 0, stream>>>(a); break;
    case 2: k_skinny_q4k<2><<<grid, SK_WAVES * 64, 0, stream>>>(a); break;
    case 3: k_skinny_q4k<3><<<grid, SK_WAVES * 64, 0, stream>>>(a); break;
    default: k_skinny_q4k<4><<<grid, SK_WAVES * 64, 0, stream>>>(a); break;
    }
    return hipGetLastError();
}

}  // namespace tq
