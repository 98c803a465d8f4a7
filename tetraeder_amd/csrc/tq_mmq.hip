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
typedef short v2s __attribute__((ext_vector_type(2)));

constexpr int MMQ_KC = 64;    // k per LDS chunk
constexpr int MMQ_LROW = 80;  // LDS bytes per row of a chunk (64 + 16 padding)

// A staging task covers TW (8, 16 or 32) consecutive weights of one row inside a 64-k chunk: task part
// p, sub-block half h = p / (32 / TW), slice s = p % (32 / TW) of TW weights inside that half.
template <int F> struct MmqFmt;

template <> struct MmqFmt<FMT_Q4K> {
    template <int TW> struct Raw {
        uint4 hdr;             // d, dmin, scales[12]
        uint32_t qs[TW / 4];   // the qs bytes holding the task's nibbles

        __device__ __forceinline__ void load(const uint8_t *blk, int c, int p) {
            const int s = p % (32 / TW);
            hdr = *(const uint4 *)blk;
            const uint8_t *q = blk + 16 + 32 * c + TW * s;
            if (TW == 8) {
                const uint2 v = *(const uint2 *)q;
                qs[0] = v.x;
                qs[1] = v.y;
            } else {
#pragma unroll
                for (int i = 0; i < TW / 16; ++i) {
                    const uint4 v = *(const uint4 *)(q + 16 * i);
                    qs[4 * i] = v.x;
                    qs[4 * i + 1] = v.y;
                    qs[4 * i + 2] = v.z;
                    qs[4 * i + 3] = v.w;
                }
            }
        }

        // planes (sc >> 3) q and (sc & 7) q of sub-block j = 2c + h: sum sc q x = 8 R0 + R1
        __device__ __forceinline__ void expand(int c, int p, uint32_t (&D)[2][TW / 4]) const {
            const int h = p / (32 / TW);
            const int j = 2 * c + h, sh = 8 * (j & 3);
            const uint32_t sc = j < 4 ? (hdr.y >> sh) & 63 : ((hdr.w >> sh) & 15) | (((hdr.y >> sh) >> 6 & 3) << 4);
            const uint32_t hi = sc >> 3, lo = sc & 7;
#pragma unroll
            for (int i = 0; i < TW / 4; ++i) {
                const uint32_t q = (qs[i] >> (4 * h)) & 0x0F0F0F0Fu;  // bytes <= 15, products <= 105: no carries
                D[0][i] = q * hi;
                D[1][i] = q * lo;
            }
        }

        __device__ __forceinline__ float d() const { return half_bits_to_float(hdr.x); }
        __device__ __forceinline__ float dmin() const { return half_bits_to_float(hdr.x >> 16); }
        // the eight 6-bit sub-block mins as bytes
        __device__ __forceinline__ uint2 mins() const {
            const uint32_t lo4 = hdr.z & 0x3F3F3F3Fu;
            const uint32_t hi4 = ((hdr.w >> 4) & 0x0F0F0F0Fu) | (((hdr.z >> 6) & 0x03030303u) << 4);
            return uint2{lo4, hi4};
        }
    };
};

template <> struct MmqFmt<FMT_Q6K> {
    template <int TW> struct Raw {
        // the block is only 2-byte aligned: aligned dwords that each hold at least one byte of it
        uint32_t L[TW / 4 + 1], Q[TW / 4 + 1], s, dw, a0;

        __device__ __forceinline__ void load(const uint8_t *blk, int c, int p) {
            const int h = p / (32 / TW), sl = p % (32 / TW);
            const int r = 2 * c + h, H = r >> 2, g = r & 3;
            a0 = (uint32_t)(uintptr_t)blk & 3;  // 0 or 2
            const uint32_t *q = (const uint32_t *)(blk - a0);
            const int ol = (64 * H + 32 * (g & 1) + TW * sl) >> 2, oh = (128 + 32 * H + TW * sl) >> 2;
#pragma unroll
            for (int i = 0; i <= TW / 4; ++i) {
                L[i] = q[ol + i];
                Q[i] = q[oh + i];
            }
            const int so = 2 * r + (TW * sl) / 16 + (int)a0;  // the task's scale byte(s)
            s = q[48 + (so >> 2)] >> (8 * (so & 3));
            dw = q[52];
        }

        // bytes of P = sc (q - 32) in [-4096, 4064]: plane 0 = P >> 7 in [-32, 31], plane 1 = P & 127,
        // so sum sc (q - 32) x = 128 R0 + R1
        __device__ __forceinline__ void expand(int c, int p, uint32_t (&D)[2][TW / 4]) const {
            const int h = p / (32 / TW);
            const int g = (2 * c + h) & 3;
            const int lsh = g >= 2 ? 4 : 0, hsh = 2 * g;
            const short s0 = (short)sext8(s, 0), s1 = (short)sext8(s, 8);
#pragma unroll
            for (int i = 0; i < TW / 4; ++i) {
                const uint32_t l = align_bytes(L[i + 1], L[i], a0), hb = align_bytes(Q[i + 1], Q[i], a0);
                const uint32_t q = ((l >> lsh) & 0x0F0F0F0Fu) | (((hb >> hsh) & 0x03030303u) << 4);  // 6-bit codes
                const short sc = (TW == 32 && i >= 4) ? s1 : s0;
                const v2s scv = {sc, sc}, off = {32, 32};
                const v2s pe = (__builtin_bit_cast(v2s, q & 0x00FF00FFu) - off) * scv;
                const v2s po = (__builtin_bit_cast(v2s, (q >> 8) & 0x00FF00FFu) - off) * scv;
                const uint32_t he = __builtin_bit_cast(uint32_t, (v2s)(pe >> (short)7));
                const uint32_t ho = __builtin_bit_cast(uint32_t, (v2s)(po >> (short)7));
                D[0][i] = (he & 0x00FF00FFu) | ((ho & 0x00FF00FFu) << 8);
                D[1][i] = (__builtin_bit_cast(uint32_t, pe) & 0x007F007Fu) |
                          ((__builtin_bit_cast(uint32_t, po) & 0x007F007Fu) << 8);
            }
        }

        __device__ __forceinline__ float d() const { return half_bits_to_float(a0 ? dw >> 16 : dw); }
        __device__ __forceinline__ float dmin() const { return 0.f; }
        __device__ __forceinline__ uint2 mins() const { return uint2{0u, 0u}; }
    };
};

template <int F, int WM, int WN, int FM, int FN>
__global__ __launch_bounds__(64 * WM * WN, (WM * WN >= 8 ? 1 : 2)) void k_mmq(MmqArgs a) {
    constexpr bool Q4 = F == FMT_Q4K;
    constexpr int NT = 64 * WM * WN, TM = 32 * FM * WM, TN = 32 * FN * WN;
    constexpr int TW = TN * MMQ_KC / NT;  // weights per staging task: one task per thread
    static_assert(TW == 8 || TW == 16 || TW == 32, "staging task width");
    constexpr int PARTS = MMQ_KC / TW;
    constexpr int APIECES = TM * MMQ_KC / 16;  // 16-byte activation pieces per chunk
    constexpr int AP = (APIECES + NT - 1) / NT;
    constexpr int ST_A = TM * MMQ_LROW, ST = ST_A + 2 * TN * MMQ_LROW;
    __shared__ __align__(16) uint8_t lds[2 * ST];
    // per super-block values, double-buffered by super-block parity
    __shared__ __align__(16) float sdx[2][TM];
    __shared__ float sdw[2][TN], sdm[2][TN];
    __shared__ __align__(16) uint8_t sS[Q4 ? 2 : 1][Q4 ? TM : 1][16];  // Q4_K: bsum pairs as bytes (S >> 7, S & 127)
    __shared__ __align__(8) uint8_t sM[Q4 ? 2 : 1][Q4 ? TN : 1][8];    // Q4_K: the eight mins of each row

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

    // this thread's weight staging task
    const int n_t = tid / PARTS, p_t = tid % PARTS;
    const bool row_ok = n0 + n_t < a.nrows;
    const uint8_t *wrow = w + (row_ok ? (n0 + n_t) * a.row_stride : 0);

    uint4 ra[AP];
    float rdx[AP];
    typename MmqFmt<F>::template Raw<TW> rw;

    // global -> registers for super-block b, chunk c
    auto load = [&](int b, int c) {
#pragma unroll
        for (int s = 0; s < AP; ++s) {
            const int idx = tid + s * NT, m = idx >> 2, part = idx & 3;
            ra[s] = uint4{0u, 0u, 0u, 0u};
            if (c == 0) rdx[s] = 0.f;
            if (idx < APIECES && m0 + m < a.ncols) {
                const uint8_t *blk = q8 + ((int64_t)(m0 + m) * nb + b) * Q8K_BYTES;
                ra[s] = *(const uint4 *)(blk + Q8K_QS + MMQ_KC * c + 16 * part);
                if (c == 0 && part == 0) rdx[s] = *(const float *)blk;
            }
        }
        if (row_ok) rw.load(wrow + (int64_t)b * FmtInfo<F>::bytes, c, p_t);
    };
    // registers -> LDS stage `st` (the weights expanded into their two int8 planes); the per-super-block
    // values of super-block buffer sb are written unless `scalars` is false
    auto store = [&](int c, int st, int sb, bool scalars) {
        uint8_t *base = lds + st * ST;
#pragma unroll
        for (int s = 0; s < AP; ++s) {
            const int idx = tid + s * NT, m = idx >> 2, part = idx & 3;
            if (Q4) {
                // S_j, the sum of the 32 activation bytes of sub-block j = 2c + part / 2: each lane sums
                // its 16 bytes, the neighbouring lane (same row, other half of the sub-block) adds its
                // own; |S_j| <= 4064 is kept as the bytes S >> 7 and S & 127
                int ps = dot4(ra[s].x, 0x01010101u, 0);
                ps = dot4(ra[s].y, 0x01010101u, ps);
                ps = dot4(ra[s].z, 0x01010101u, ps);
                ps = dot4(ra[s].w, 0x01010101u, ps);
                ps += __builtin_amdgcn_mov_dpp(ps, 0xB1, 0xf, 0xf, false);  // quad_perm [1,0,3,2]
                if (idx < APIECES && (part & 1) == 0 && scalars) {
                    const int j = 2 * c + (part >> 1);
                    sS[sb][m][j] = (uint8_t)(ps >> 7);
                    sS[sb][m][8 + j] = (uint8_t)(ps & 127);
                }
            }
            if (idx < APIECES) {
                *(uint4 *)(base + m * MMQ_LROW + 16 * part) = ra[s];
                if (c == 0 && part == 0 && scalars) sdx[sb][m] = rdx[s];
            }
        }
        uint32_t D[2][TW / 4];
        if (row_ok) {
            rw.expand(c, p_t, D);
        } else {
#pragma unroll
            for (int k = 0; k < 2; ++k)
#pragma unroll
                for (int i4 = 0; i4 < TW / 4; ++i4) D[k][i4] = 0u;
        }
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            uint8_t *o = base + ST_A + (k * TN + n_t) * MMQ_LROW + TW * p_t;
            if (TW == 8) {
                *(uint2 *)o = uint2{D[k][0], D[k][1]};
            } else {
#pragma unroll
                for (int i4 = 0; i4 < TW / 16; ++i4)
                    *(uint4 *)(o + 16 * i4) = uint4{D[k][4 * i4], D[k][4 * i4 + 1], D[k][4 * i4 + 2], D[k][4 * i4 + 3]};
            }
        }
        if (c == 0 && p_t == 0 && scalars) {
            sdw[sb][n_t] = row_ok ? rw.d() : 0.f;
            if (Q4) {
                sdm[sb][n_t] = row_ok ? rw.dmin() : 0.f;
                *(uint2 *)(&sM[sb][n_t][0]) = row_ok ? rw.mins() : uint2{0u, 0u};
            }
        }
    };

    v16i R[FM][FN][2];
    float acc[FM][FN][16];
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
        for (int fn = 0; fn < FN; ++fn)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[fm][fn][v] = 0.f;

    load(0, 0);
    store(0, 0, 0, true);
    __syncthreads();
    for (int b = 0; b < nb; ++b) {
        const bool last = b + 1 == nb;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            // the next chunk (the last super-block's final step reloads its own chunk 0 into the idle
            // stage and skips the per-super-block values, so nothing reads past the end)
            const int bn = c == 3 ? (last ? b : b + 1) : b, cn = (c + 1) & 3;
            load(bn, cn);
            const uint8_t *base = lds + (c & 1) * ST;
#pragma unroll
            for (int ks = 0; ks < MMQ_KC / 32; ++ks) {
                const int col = 32 * ks + 16 * (lane >> 5);
                v4i af[FM];
#pragma unroll
                for (int fm = 0; fm < FM; ++fm)
                    af[fm] = *(const v4i *)(base + ((wm * FM + fm) * 32 + (lane & 31)) * MMQ_LROW + col);
#pragma unroll
                for (int fn = 0; fn < FN; ++fn)
#pragma unroll
                    for (int k = 0; k < 2; ++k) {
                        const v4i bf =
                            *(const v4i *)(base + ST_A + (k * TN + (wn * FN + fn) * 32 + (lane & 31)) * MMQ_LROW + col);
#pragma unroll
                        for (int fm = 0; fm < FM; ++fm)
                            R[fm][fn][k] = __builtin_amdgcn_mfma_i32_32x32x32_i8(
                                af[fm], bf, (c == 0 && ks == 0) ? v16i{} : R[fm][fn][k], 0, 0, 0);
                    }
            }
            if (c == 3) {
                // end of the super-block: combine the planes and apply the fp32 scales
                const int sb = b & 1;
#pragma unroll
                for (int fm = 0; fm < FM; ++fm) {
                    const int mrow = (wm * FM + fm) * 32;
                    float dx[16];
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const float4 v = *(const float4 *)(&sdx[sb][mrow + 8 * q + 4 * (lane >> 5)]);
                        dx[4 * q] = v.x;
                        dx[4 * q + 1] = v.y;
                        dx[4 * q + 2] = v.z;
                        dx[4 * q + 3] = v.w;
                    }
                    long sa = 0;
                    if (Q4) sa = *(const long *)(&sS[sb][mrow + (lane & 31)][8 * (lane >> 5)]);
#pragma unroll
                    for (int fn = 0; fn < FN; ++fn) {
                        const int n = (wn * FN + fn) * 32 + (lane & 31);
                        const float dw = sdw[sb][n];
                        if (Q4) {
                            // sum_j m_j S_j = 128 sum m_j (S_j >> 7) + sum m_j (S_j & 127): two 16-deep
                            // products, k 0..7 the high bytes, k 8..15 the low bytes
                            const long mv = *(const long *)(&sM[sb][n][0]);
                            const long b_hi = (lane >> 5) ? 0l : mv, b_lo = (lane >> 5) ? mv : 0l;
                            v16i t = __builtin_amdgcn_mfma_i32_32x32x16_i8(sa, b_hi, v16i{}, 0, 0, 0);
#pragma unroll
                            for (int v = 0; v < 16; ++v) t[v] <<= 7;
                            t = __builtin_amdgcn_mfma_i32_32x32x16_i8(sa, b_lo, t, 0, 0, 0);
                            const float dm = sdm[sb][n];
#pragma unroll
                            for (int v = 0; v < 16; ++v) {
                                const int i1 = (R[fm][fn][0][v] << 3) + R[fm][fn][1][v];
                                const int i2v = t[v];
                                const float f = dw * (float)i1 - dm * (float)i2v;
                                acc[fm][fn][v] = __builtin_fmaf(dx[v], f, acc[fm][fn][v]);
                            }
                        } else {
#pragma unroll
                            for (int v = 0; v < 16; ++v) {
                                const int iv = (R[fm][fn][0][v] << 7) + R[fm][fn][1][v];
                                acc[fm][fn][v] = __builtin_fmaf(dx[v] * dw, (float)iv, acc[fm][fn][v]);
                            }
                        }
                    }
                }
            }
            store(cn, (c + 1) & 1, bn & 1, !(c == 3 && last));
            __syncthreads();
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
    if (a.ncols <= 64) return launch_cfg<F, 1, 4, 2, 1>(a, stream);   // 64 x 128 tiles
    if (a.ncols <= 128) return launch_cfg<F, 2, 2, 2, 1>(a, stream);  // 128 x 64
    return launch_cfg<F, 4, 2, 2, 1>(a, stream);                       // 256 x 64, 8 waves
}

hipError_t launch_mmq(int type, const MmqArgs &a, hipStream_t stream) {
    if (mmq_tile_supported(type, a)) return launch_mmq_tile(type, a, stream);
    if (type == FMT_Q6K && mmq_tile_q6k_supported(a)) return launch_mmq_tile_q6k(a, stream);
    return type == FMT_Q4K ? launch_fmt<FMT_Q4K>(a, stream) : launch_fmt<FMT_Q6K>(a, stream);
}

}  // namespace tq
