// tq_mmq.hip -- MUL_MAT with many activation columns (prefill and batched decode) on int8 MFMA
// (v_mfma_i32_32x32x32_i8), Q4_K / Q6_K weights against Q8_K activations.
//
// ggml's dot product per super-block (vec_dot_q4_K_q8_K / vec_dot_q6_K_q8_K) is
//   Q4_K: d_x * (d * sum_j sc_j * sum_{k in j} q_k x_k  -  dmin * sum_j m_j * sum_{k in j} x_k)
//   Q6_K: d_x * d * sum_j sc_j * sum_{k in j} (q_k - 32) x_k
// with 6-bit (Q4_K) or signed 8-bit (Q6_K) sub-block scales sc_j that change every 32 (Q4_K) or 16
// (Q6_K) k. int8 MFMA needs int8 operands, and sc_j * q does not fit in a byte, so each workgroup
// expands a super-block of its weight rows into three int8 "digit" planes in LDS whose weighted sum is
// the scaled weight:
//   Q4_K: D0 = (sc >> 3) * q, D1 = (sc & 7) * q      (<= 105)   -> sum sc*q*x = 8*R0 + R1
//         D2 = m (the sub-block min, on every k)                 -> sum_j m_j * sum x = R2
//   Q6_K: sc = e0 + 8 e1 + 64 e2 with balanced digits e in [-3, 4], Di = ei * (q - 32) in [-128, 124]
//                                                                  -> sum sc*(q-32)*x = R0 + 8 R1 + 64 R2
// where Ri = sum_k x_k Di_k is one int32 MFMA accumulation over the super-block's 256 k. The integer
// sums are exact (|R| < 2^23), so only the per-super-block fp32 combination rounds, as in ggml.
//
// Tiling: a workgroup of WM x WN waves owns TM = 32 FM WM activation rows (m) by TN = 32 FN WN weight
// rows (n) and walks k in chunks of 64: it copies the Q8_K activation bytes of the chunk into LDS,
// expands the weight chunk into the three digit planes, and every wave issues FM x FN x 3 MFMAs per
// 32 k. Rows are padded to 80 bytes in LDS so the 16-byte fragment reads of 8 lanes hit distinct
// banks. The MFMA output layout (32 x 32, lane l holds column l % 32 and rows
// 8 (v / 4) + 4 (l / 32) + v % 4 of its 16 values) puts one weight row per lane, so the per-row scales
// are one LDS read per lane and tile.
#include "tq_device.h"
#include "tq_internal.h"

#include <algorithm>

namespace tq {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int MMQ_KC = 64;    // k per LDS chunk
constexpr int MMQ_LROW = 80;  // LDS bytes per row of a chunk (64 + 16 padding)

template <int F> struct MmqDigits;

template <> struct MmqDigits<FMT_Q4K> {
    // Sub-block j = 2c + h (weights 64c + 32h .. +32 of the super-block at blk): three digit planes of 32
    // bytes each, and the super-block scales.
    static __device__ __forceinline__ void make(const uint8_t *blk, int c, int h, uint32_t (&D)[3][8], float &d,
                                                float &dmin) {
        const uint4 hdr = *(const uint4 *)blk;  // d, dmin, scales[0..11]
        const uint4 qa = *(const uint4 *)(blk + 16 + 32 * c);
        const uint4 qb = *(const uint4 *)(blk + 32 + 32 * c);
        const int j = 2 * c + h, sh = 8 * (j & 3);
        uint32_t sc, mn;
        if (j < 4) {
            sc = (hdr.y >> sh) & 63;
            mn = (hdr.z >> sh) & 63;
        } else {
            sc = ((hdr.w >> sh) & 15) | (((hdr.y >> sh) >> 6 & 3) << 4);
            mn = ((hdr.w >> sh) >> 4 & 15) | (((hdr.z >> sh) >> 6 & 3) << 4);
        }
        const uint32_t qw[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
        const uint32_t hi = sc >> 3, lo = sc & 7, mb = mn * 0x01010101u;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t q = (qw[i] >> (4 * h)) & 0x0F0F0F0Fu;  // bytes <= 15, products <= 105: no carries
            D[0][i] = q * hi;
            D[1][i] = q * lo;
            D[2][i] = mb;
        }
        d = half_bits_to_float(hdr.x);
        dmin = half_bits_to_float(hdr.x >> 16);
    }
};

template <> struct MmqDigits<FMT_Q6K> {
    // Weights 32r .. 32r + 32 of the super-block (r = 2c + h), sub-blocks 2r and 2r + 1. The block is
    // only 2-byte aligned: every load is an aligned dword holding at least one byte of the block.
    static __device__ __forceinline__ void make(const uint8_t *blk, int c, int h, uint32_t (&D)[3][8], float &d,
                                                float &dmin) {
        const int r = 2 * c + h, H = r >> 2, g = r & 3;
        const uint32_t a0 = (uint32_t)(uintptr_t)blk & 3;  // 0 or 2
        const uint32_t *p = (const uint32_t *)(blk - a0);
        const int ol = (64 * H + 32 * (g & 1)) >> 2, oh = (128 + 32 * H) >> 2;
        uint32_t L[9], Q[9];
#pragma unroll
        for (int i = 0; i < 9; ++i) {
            L[i] = p[ol + i];
            Q[i] = p[oh + i];
        }
        const int so = 2 * r + (int)a0;
        const uint32_t s16 = p[48 + (so >> 2)] >> (8 * (so & 3));
        const uint32_t dw = p[52];
        d = half_bits_to_float(a0 ? dw >> 16 : dw);
        dmin = 0.f;
        int e[2][3];
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const int v = sext8(s16, 8 * s);
            const int e0 = ((v + 3) & 7) - 3, t = (v - e0) >> 3;
            const int e1 = ((t + 3) & 7) - 3;
            e[s][0] = e0;
            e[s][1] = e1;
            e[s][2] = (t - e1) >> 3;
        }
        const int lsh = g >= 2 ? 4 : 0, hsh = 2 * g;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t l = align_bytes(L[i + 1], L[i], a0), hb = align_bytes(Q[i + 1], Q[i], a0);
            const uint32_t q = ((l >> lsh) & 0x0F0F0F0Fu) | (((hb >> hsh) & 0x03030303u) << 4);  // 6-bit codes
            const int qe = (int)(q & 0x00FF00FFu), qo = (int)((q >> 8) & 0x00FF00FFu);
#pragma unroll
            for (int k = 0; k < 3; ++k) {
                // per byte w = e*q + 128 - 32e = e*(q - 32) + 128 in [0, 252]: the two 16-bit lanes never
                // borrow or carry, and w ^ 0x80 is the signed byte e*(q - 32)
                const int ek = e[i >> 2][k];
                const int kk = (128 - 32 * ek) * 0x00010001;
                const uint32_t we = (uint32_t)(__mul24(qe, ek) + kk), wo = (uint32_t)(__mul24(qo, ek) + kk);
                D[k][i] = (we | (wo << 8)) ^ 0x80808080u;
            }
        }
    }
};

template <int F, int WM, int WN, int FM, int FN>
__global__ __launch_bounds__(64 * WM * WN) void k_mmq(MmqArgs a) {
    constexpr int NT = 64 * WM * WN;
    constexpr int TM = 32 * FM * WM, TN = 32 * FN * WN;
    __shared__ __align__(16) uint8_t sA[TM * MMQ_LROW];
    __shared__ __align__(16) uint8_t sB[3 * TN * MMQ_LROW];
    __shared__ __align__(16) float sdx[TM];
    __shared__ float sdw[TN], sdm[TN];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int wm = wave % WM, wn = wave / WM;

    // tile of this workgroup; consecutive ids on one XCD (ids are dealt round robin over 8) walk the n
    // tiles of one m tile, so that m tile's activations stay in that XCD's L2
    const int tiles_m = (a.ncols + TM - 1) / TM, tiles_n = (int)((a.nrows + TN - 1) / TN);
    const int ntiles = tiles_m * tiles_n;
    int id = blockIdx.x;
    if ((ntiles & 7) == 0) id = (id & 7) * (ntiles >> 3) + (id >> 3);
    const int nt = id % tiles_n, mt = id / tiles_n;
    const int m0 = mt * TM;
    const int64_t n0 = (int64_t)nt * TN;

    const int i2 = blockIdx.y % a.ne12, i3 = blockIdx.y / a.ne12;
    const uint8_t *w = a.w + (int64_t)(i2 / a.r2) * a.w_s2 + (int64_t)(i3 / a.r3) * a.w_s3;
    const int nb = a.nb;
    const uint8_t *q8 = a.q8 + (int64_t)blockIdx.y * a.ncols * nb * Q8K_BYTES;
    float *dst = a.dst + i2 * a.d_s2 + i3 * a.d_s3;

    v16i R[FM][FN][3];
    float acc[FM][FN][16];
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
        for (int fn = 0; fn < FN; ++fn) {
#pragma unroll
            for (int k = 0; k < 3; ++k) R[fm][fn][k] = v16i{};
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[fm][fn][v] = 0.f;
        }

    for (int b = 0; b < nb; ++b) {
        for (int c = 0; c < QK / MMQ_KC; ++c) {
            __syncthreads();  // the previous chunk's fragment reads are done
            // activations: TM rows x 64 bytes of Q8_K qs (4-byte aligned 16-byte loads)
            for (int idx = tid; idx < TM * 4; idx += NT) {
                const int m = idx >> 2, part = idx & 3;
                uint4 v = {0u, 0u, 0u, 0u};
                float dx = 0.f;
                if (m0 + m < a.ncols) {
                    const uint8_t *blk = q8 + ((int64_t)(m0 + m) * nb + b) * Q8K_BYTES;
                    v = *(const uint4 *)(blk + Q8K_QS + MMQ_KC * c + 16 * part);
                    dx = *(const float *)blk;
                }
                *(uint4 *)(sA + m * MMQ_LROW + 16 * part) = v;
                if (c == 0 && part == 0) sdx[m] = dx;
            }
            // weights: TN rows x 2 halves of 32 k, expanded into the digit planes
            for (int t = tid; t < TN * 2; t += NT) {
                const int n = t >> 1, h = t & 1;
                uint32_t D[3][8];
                float d = 0.f, dmin = 0.f;
                if (n0 + n < a.nrows) {
                    const uint8_t *blk = w + (n0 + n) * a.row_stride + (int64_t)b * FmtInfo<F>::bytes;
                    MmqDigits<F>::make(blk, c, h, D, d, dmin);
                } else {
#pragma unroll
                    for (int k = 0; k < 3; ++k)
#pragma unroll
                        for (int i = 0; i < 8; ++i) D[k][i] = 0u;
                }
#pragma unroll
                for (int k = 0; k < 3; ++k) {
                    uint8_t *o = sB + (k * TN + n) * MMQ_LROW + 32 * h;
                    *(uint4 *)o = uint4{D[k][0], D[k][1], D[k][2], D[k][3]};
                    *(uint4 *)(o + 16) = uint4{D[k][4], D[k][5], D[k][6], D[k][7]};
                }
                if (c == 0 && h == 0) {
                    sdw[n] = d;
                    sdm[n] = dmin;
                }
            }
            __syncthreads();
#pragma unroll
            for (int ks = 0; ks < MMQ_KC / 32; ++ks) {
                const int col = 32 * ks + 16 * (lane >> 5);
                v4i af[FM];
#pragma unroll
                for (int fm = 0; fm < FM; ++fm)
                    af[fm] = *(const v4i *)(sA + ((wm * FM + fm) * 32 + (lane & 31)) * MMQ_LROW + col);
#pragma unroll
                for (int fn = 0; fn < FN; ++fn)
#pragma unroll
                    for (int k = 0; k < 3; ++k) {
                        const v4i bf = *(const v4i *)(sB + (k * TN + (wn * FN + fn) * 32 + (lane & 31)) * MMQ_LROW + col);
#pragma unroll
                        for (int fm = 0; fm < FM; ++fm)
                            R[fm][fn][k] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[fm], bf, R[fm][fn][k], 0, 0, 0);
                    }
            }
        }
        // end of the super-block: combine the digits and apply the fp32 scales
#pragma unroll
        for (int fm = 0; fm < FM; ++fm) {
            float dx[16];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float4 v = *(const float4 *)(sdx + (wm * FM + fm) * 32 + 8 * q + 4 * (lane >> 5));
                dx[4 * q] = v.x;
                dx[4 * q + 1] = v.y;
                dx[4 * q + 2] = v.z;
                dx[4 * q + 3] = v.w;
            }
#pragma unroll
            for (int fn = 0; fn < FN; ++fn) {
                const int n = (wn * FN + fn) * 32 + (lane & 31);
                const float dw = sdw[n];
                if (F == FMT_Q4K) {
                    const float dm = sdm[n];
#pragma unroll
                    for (int v = 0; v < 16; ++v) {
                        const int i1 = (R[fm][fn][0][v] << 3) + R[fm][fn][1][v];
                        const float f = dw * (float)i1 - dm * (float)R[fm][fn][2][v];
                        acc[fm][fn][v] = __builtin_fmaf(dx[v], f, acc[fm][fn][v]);
                    }
                } else {
#pragma unroll
                    for (int v = 0; v < 16; ++v) {
                        const int i = R[fm][fn][0][v] + (R[fm][fn][1][v] << 3) + (R[fm][fn][2][v] << 6);
                        acc[fm][fn][v] = __builtin_fmaf(dx[v] * dw, (float)i, acc[fm][fn][v]);
                    }
                }
#pragma unroll
                for (int k = 0; k < 3; ++k) R[fm][fn][k] = v16i{};
            }
        }
    }

    const int64_t d_s1 = a.d_s1;
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
        for (int fn = 0; fn < FN; ++fn) {
            const int64_t n = n0 + (wn * FN + fn) * 32 + (lane & 31);
            if (n >= a.nrows) continue;
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int m = m0 + (wm * FM + fm) * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
                if (m < a.ncols) dst[m * d_s1 + n] = acc[fm][fn][v];
            }
        }
}

template <int F, int WM, int WN, int FM, int FN>
static hipError_t launch_cfg(const MmqArgs &a, hipStream_t stream) {
    constexpr int TM = 32 * FM * WM, TN = 32 * FN * WN;
    const int64_t tiles = (int64_t)((a.ncols + TM - 1) / TM) * ((a.nrows + TN - 1) / TN);
    if (tiles > 0x7fffffff) return hipErrorInvalidValue;
    k_mmq<F, WM, WN, FM, FN><<<dim3((unsigned)tiles, (unsigned)a.nbatch), 64 * WM * WN, 0, stream>>>(a);
    return hipGetLastError();
}

template <int F>
static hipError_t launch_fmt(const MmqArgs &a, hipStream_t stream) {
    if (a.ncols <= 32) return launch_cfg<F, 1, 4, 1, 1>(a, stream);  // 32 x 128 tiles
    if (a.ncols <= 64) return launch_cfg<F, 1, 4, 2, 1>(a, stream);  // 64 x 128
    return launch_cfg<F, 2, 2, 2, 1>(a, stream);                      // 128 x 64
}

hipError_t launch_mmq(int type, const MmqArgs &a, hipStream_t stream) {
    return type == FMT_Q4K ? launch_fmt<FMT_Q4K>(a, stream) : launch_fmt<FMT_Q6K>(a, stream);
}

}  // namespace tq
