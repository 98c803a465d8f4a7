// tq_skinny.hip -- MUL_MAT over Q4_K weights for a few activation columns (batched decode, 4..64
// columns) on int8 MFMA (v_mfma_i32_16x16x64_i8), every weight byte read once for all columns. The
// operand layout and the super-block step are in tq_skinny.h.
// Grid: one workgroup of SK_WAVES waves per 16-row tile; the waves split the super-blocks and their
// partial sums meet in LDS.
#include "tq_device.h"
#include "tq_internal.h"
#include "tq_skinny.h"

#include <algorithm>

namespace tq {

#ifndef TQ_SK_WAVES
#define TQ_SK_WAVES 8
#endif
constexpr int SK_WAVES = TQ_SK_WAVES;

// Weights of a workgroup's 16 rows staged in LDS: piece c (16 bytes) of row n at position
// rp n + (c + n) mod rp, rp = 9 nb pieces a row: rows rotated by n pieces, so the same piece of 16 rows
// lands on 16 different groups of 4 banks for the row lengths of interest. sk_rot(rp, n) = n mod rp
// (rp >= 9, n < 16).
__device__ __forceinline__ int sk_rot(int rp, int n) { return n >= rp ? n - rp : n; }
__device__ __forceinline__ int sk_pos(int rp, int n, int c) {
    const int r = c + sk_rot(rp, n);
    return rp * n + (r >= rp ? r - rp : r);
}

constexpr int SK_LDS_NB_MAX = 32;  // staged weights: up to K = 8192 (72 KB)

// One workgroup per 16-row tile (and batch matrix): the tile's weights come into LDS by wave-wide LDS
// DMAs of one kilobyte of consecutive bytes each (the tile's rows are contiguous in memory), the waves
// split the super-blocks and their partial sums meet in LDS.
template <int MT>
__global__ __launch_bounds__(SK_WAVES * 64) void k_skinny_q4k(SkinnyArgs a) {
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ v4f red[SK_WAVES - 1][MT][64];  // partial sums of waves 1 .. SK_WAVES-1
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n = lane & 15, g = lane >> 4;
    const int nb = a.nb, rp = 9 * nb;
    const int i2 = blockIdx.y % a.ne12, i3 = blockIdx.y / a.ne12;
    const uint8_t *w = a.w + (int64_t)(i2 / a.r2) * a.w_s2 + (int64_t)(i3 / a.r3) * a.w_s3;
    const uint8_t *q8 = a.q8 + (int64_t)blockIdx.y * a.ncols * nb * Q8K_BYTES;
    float *dst = a.dst + i2 * a.d_s2 + i3 * a.d_s3;
    const int64_t r0 = (int64_t)blockIdx.x * 16, row = r0 + n;
    const bool rv = row < a.nrows;
    uint8_t *wt = lds;  // the staged tile: 16 rows x nb blocks
    {
        // the tile's rows are the buffer resource (rows past the end read as zeros)
        const int64_t rows = min<int64_t>(16, a.nrows - r0);
        const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
            (void *)(w + r0 * a.row_stride), (short)0, (int)(rows * a.row_stride), BUFFER_FLAGS);
        const int pieces = 16 * rp;
        for (int q = wave; 64 * q < pieces; q += SK_WAVES) {
            const int p = 64 * q + lane;
            if (p < pieces) {
                const int rn = p / rp, pr = p - rn * rp, rot = sk_rot(rp, rn);
                const int c = pr >= rot ? pr - rot : pr - rot + rp;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void *)(wt + 1024 * q),
                                                         16, (uint32_t)(rn * a.row_stride + 16 * c), 0, 0, 0);
            }
        }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    // column chunks of 16 MT
    for (int c0 = 0; c0 < a.ncols; c0 += 16 * MT) {
        v4f acc[MT];
#pragma unroll
        for (int ct = 0; ct < MT; ++ct) acc[ct] = v4f{0.f, 0.f, 0.f, 0.f};
        const int nvalid = min(16 * MT, a.ncols - c0);
        const int ntile = (nvalid + 15) >> 4;
        for (int b = wave; b < nb; b += SK_WAVES) {
            Q4kLaneBlock wl;
            const int cb = 9 * b;
            wl.hdr = *(const uint4 *)(wt + 16 * sk_pos(rp, n, cb));
#pragma unroll
            for (int s4 = 0; s4 < 4; ++s4) wl.qw[s4] = *(const uint4 *)(wt + 16 * sk_pos(rp, n, cb + 1 + 2 * s4 + (g & 1)));
            Q4kPlanes P;
            q4k_planes(wl, rv, P);
#pragma unroll
            for (int ct = 0; ct < MT; ++ct) {
                if (ct < ntile) {
                    Q4kTileAct t;
                    load_tile_act(t, 16 * ct, nvalid, [&](int k) { return q8 + ((int64_t)(c0 + k) * nb + b) * Q8K_BYTES; });
                    q4k_tile_mma(P, t, acc[ct]);
                }
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

// K above the staged limit: the weights straight from memory.
template <int MT>
__global__ __launch_bounds__(SK_WAVES * 64) void k_skinny_q4k_direct(SkinnyArgs a) {
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

    // column chunks of 16 MT: the row tile's weights come from HBM once and from L2 for later chunks
    for (int c0 = 0; c0 < a.ncols; c0 += 16 * MT) {
        v4f acc[MT];
#pragma unroll
        for (int ct = 0; ct < MT; ++ct) acc[ct] = v4f{0.f, 0.f, 0.f, 0.f};
        const int nvalid = min(16 * MT, a.ncols - c0);
        for (int b = wave; b < nb; b += SK_WAVES)
            q4k_skinny_step<MT>(wrow + (int64_t)b * Q4K_BYTES, rv, nvalid,
                                [&](int k) { return q8 + ((int64_t)(c0 + k) * nb + b) * Q8K_BYTES; }, acc);
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
    if (a.nb <= SK_LDS_NB_MAX && (int64_t)16 * a.row_stride < (1ll << 31)) {
        const size_t lds = (size_t)a.nb * 16 * Q4K_BYTES;
        switch (mt) {
        case 1: k_skinny_q4k<1><<<grid, SK_WAVES * 64, lds, stream>>>(a); break;
        case 2: k_skinny_q4k<2><<<grid, SK_WAVES * 64, lds, stream>>>(a); break;
        case 3: k_skinny_q4k<3><<<grid, SK_WAVES * 64, lds, stream>>>(a); break;
        default: k_skinny_q4k<4><<<grid, SK_WAVES * 64, lds, stream>>>(a); break;
        }
        return hipGetLastError();
    }
    switch (mt) {
    case 1: k_skinny_q4k_direct<1><<<grid, SK_WAVES * 64, 0, stream>>>(a); break;
    case 2: k_skinny_q4k_direct<2><<<grid, SK_WAVES * 64, 0, stream>>>(a); break;
    case 3: k_skinny_q4k_direct<3><<<grid, SK_WAVES * 64, 0, stream>>>(a); break;
    default: k_skinny_q4k_direct<4><<<grid, SK_WAVES * 64, 0, stream>>>(a); break;
    }
    return hipGetLastError();
}

}  // namespace tq
